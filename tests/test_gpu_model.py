"""Model-level parity through the C ABI: the token loop on the GPU against the oracle
(the reference --stage v2 path restated; bit-identical to the compiled reference).

Bar: identical greedy token streams; logits, per-layer activations and KV cache within
normwise relative error 1e-3 (max|gpu - oracle| / max|oracle|).
"""
import numpy as np
import pytest

from conftest import rel_err
from gpu_util import REGRESS, model_parity

pytestmark = pytest.mark.gpu

SMALL = ["tiny_f32", "tiny_q8", "tiny_mixq4", "tiny_qwen", "tiny_hd128", "small_q8"]
GRAPH, STEP = 0, 1  # HipModel.PATH_GRAPH, PATH_STEP


@pytest.mark.parametrize("path", [GRAPH, STEP], ids=["graph", "step"])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("preset", SMALL)
def test_small_models(pkg, gguf, preset, layout, path):
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"], 6, info["n_vocab"])
    ids, worst, worst_tap, margin = model_parity(pkg, gguf(preset), prompt, 16, 64, layout, decode_path=path)
    print(f"{preset} layout {layout} path {path}: ids {ids} logits {worst:.2e} taps {worst_tap:.2e} "
          f"margin {margin:.3e}")


@pytest.mark.parametrize("preset,want", [("tiny_q8", STEP), ("tiny_f32", STEP), ("small_q8", STEP),
                                         ("tiny_mixq4", STEP), ("tiny_hd128", STEP)])
def test_decode_path_selection(pkg, gguf, preset, want):
    """The persistent step kernel runs models whose layer matrices share a compiled format
    (Q4_0 layers may have Q4_1 wo / ffn_down, as tiny_mixq4's first and last layer do),
    also with caches longer than 512 positions (attention split over workgroups);
    PATH_GRAPH forces the graph."""
    hip = pkg.HipModel(gguf(preset), max_seq=64)
    assert hip.decode_path() == want
    hip.set_decode_path(GRAPH)
    assert hip.decode_path() == GRAPH
    hip.close()
    big = pkg.HipModel(gguf(preset), max_seq=1024)
    assert big.decode_path() == want
    big.close()


@pytest.mark.parametrize("path", [GRAPH, STEP], ids=["graph", "step"])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("preset", ["tiny_q8", "tiny_f32", "tiny_qwen", "small_q8", "tiny_mixq4", "tiny_hd128"])
def test_long_cache_split_attention(pkg, gguf, preset, layout, path):
    """A 600-token prompt in a 1024-position cache: the step kernel's attention splits the
    positions over its trailing workgroups and merges the splits there, the graph path's
    over split workgroups and a combine launch; each against the oracle while decoding
    past it."""
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"] + 7, 600, info["n_vocab"])
    ids, worst, worst_tap, margin = model_parity(pkg, gguf(preset), prompt, 12, 1024, layout, decode_path=path)
    print(f"{preset} layout {layout} path {path}: logits {worst:.2e} taps {worst_tap:.2e} margin {margin:.3e}")


# (preset, prompt tokens, cache positions, switch span): the step kernel's splits move from
# its trailing workgroups to every workgroup once the span passes the switch
# (tf_hip_set_split_all_from). The prompts end a few positions short of it, so the
# per-token decodes and the one-launch greedy loop both cross it; with 1024 and 4096 the
# trailing splits hold 64 positions each at the switch (16 and 64 splits per kv head).
# tiny_hd128 runs the head_dim-128 build (6 query heads per kv head, as the Qwen2.5-1.5B
# shape) through both layouts past 1,800 positions.
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("preset,n_prompt,max_seq,switch", [("tiny_f32", 1018, 2048, 1024),
                                                            ("tiny_q8", 4090, 4200, 4096),
                                                            ("tiny_qwen", 700, 1024, 705),
                                                            ("tiny_hd128", 1800, 2048, 1805)])
def test_long_cache_split_layout_switch(pkg, gguf, preset, n_prompt, max_seq, switch, layout):
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"] + 11, n_prompt, info["n_vocab"])

    def setup(hip):
        hip.set_split_all_from(switch)
        cfg = hip.step_config()
        assert cfg["split"] > 0 and cfg["split_all"] > 0 and cfg["split_all_from"] == switch, cfg

    ids, worst, worst_tap, margin = model_parity(pkg, gguf(preset), prompt, 12, max_seq, layout, decode_path=STEP,
                                                 setup=setup)
    print(f"{preset} {n_prompt} layout {layout}: logits {worst:.2e} taps {worst_tap:.2e} margin {margin:.3e}")


# Caches of at most 512 positions: tokens attending up to 64 positions run attention on one
# workgroup per kv head, longer spans split it. Prompts of 60 tokens put the switch inside
# the per-token decodes and inside the one-launch greedy loop, whose later, split tokens
# read the rows the earlier ones stored from other workgroups. tiny_hd128 and the
# full-size Qwen2.5-1.5B shape run the head_dim-128 build on both sides of the switch.
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("preset", ["tiny_f32", "tiny_q8", "tiny_qwen", "tiny_hd128", "qwen15b_q8"])
def test_short_cache_split_switch(pkg, gguf, preset, layout):
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"] + 5, 60, info["n_vocab"])

    def setup(hip):
        assert hip.decode_path() == STEP
        cfg = hip.step_config()
        # the switch really happens inside the decode: a split layout exists and spans
        # 61..72 cross split_from
        assert cfg["split"] > 0 and cfg["split_from"] == 64, cfg

    ids, worst, worst_tap, margin = model_parity(pkg, gguf(preset), prompt, 12, 512, layout, decode_path=STEP,
                                                 setup=setup)
    print(f"{preset} layout {layout}: logits {worst:.2e} taps {worst_tap:.2e} margin {margin:.3e}")


@pytest.mark.parametrize("span", [0, 512])
def test_split_from_knob(pkg, gguf, span):
    """tf_hip_set_split_from: every token split (0) or none below 512 positions (512) gives
    the same function; values above 512 are rejected."""
    preset = "tiny_q8"
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"] + 3, 40, info["n_vocab"])

    def setup(hip):
        with pytest.raises(RuntimeError, match="above 512"):
            hip.set_split_from(513)
        hip.set_split_from(span)
        assert hip.step_config()["split_from"] == span

    ids, worst, _, _ = model_parity(pkg, gguf(preset), prompt, 12, 512, 0, decode_path=STEP, setup=setup)
    print(f"split_from {span}: logits {worst:.2e}")


def test_exchange_epoch_wrap(pkg, gguf):
    """A greedy launch that runs the step kernel's 32-bit exchange epoch past 2^32: the
    backend clears the exchange words and restarts the count, and the tokens and logits
    are those of a run far from the wrap."""
    path = gguf("small_q8")
    prompt = np.array([3, 99, 7, 1200, 5, 42, 8], np.int32)
    out = []
    for start in (None, 2**32 - 300):
        hip = pkg.HipModel(path, max_seq=64)
        hip.set_decode_path(STEP)
        hip.prefill(prompt)
        if start is not None:
            hip.set_exchange_epoch(start)  # a few tokens before the wrap (32 epochs per token)
        ids = hip.generate(24)
        ld, _ = hip.decode(int(ids[-1]))
        out.append((ids, ld))
        hip.close()
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][1], out[1][1])


@pytest.mark.parametrize("call", ["generate", "decode", "prefill"])
def test_cooperative_refusal_falls_back_to_graph(pkg, gguf, call):
    """A refused cooperative launch (another process holding the GPU's cooperative-launch
    resource, forced here through the test hook) runs the same tokens on the graph path,
    and the context stays there; the greedy stream equals the oracle's."""
    from oracle.bind import OracleModel, greedy_stream

    path = gguf("tiny_q8")
    info = pkg.synth_preset_info("tiny_q8")
    prompt = pkg.synth_prompt(info["seed"], 6, info["n_vocab"])
    ref_ids, _ = greedy_stream(OracleModel(path, max_seq=64, n_threads=4), prompt, 12)
    hip = pkg.HipModel(path, max_seq=64)
    try:
        assert hip.decode_path() == STEP
        if call == "prefill":
            hip.set_prefill_path(pkg.HipModel.PREFILL_TOKENS)  # the prompt runs on the decode path
            hip.test_refuse_cooperative(1)
        _, am = hip.prefill(prompt)
        assert am == ref_ids[0]
        if call == "decode":
            hip.test_refuse_cooperative(1)
            _, am2 = hip.decode(int(ref_ids[0]))
            assert am2 == ref_ids[1]
            assert np.array_equal(hip.generate(10), ref_ids[1:11])
        else:
            if call == "generate":
                hip.test_refuse_cooperative(1)
            ids = hip.generate(11)
            assert np.array_equal(ids, ref_ids[:11])
        assert hip.decode_path() == GRAPH
        hip.set_decode_path(STEP)  # the switch holds for the context's life
        assert hip.decode_path() == GRAPH
    finally:
        hip.close()


TOKENS, MFMA = 0, 1  # HipModel.PREFILL_TOKENS, HipModel.PREFILL_MFMA


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("preset", ["tiny_q8", "tiny_qwen", "small_q8"])
def test_small_models_token_prefill(pkg, gguf, preset, layout):
    """The per-token prefill path on the models whose prompts otherwise take the matrix cores."""
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"], 6, info["n_vocab"])
    ids, worst, worst_tap, margin = model_parity(pkg, gguf(preset), prompt, 8, 64, layout, prefill_path=TOKENS)
    print(f"{preset} layout {layout}: ids {ids} logits {worst:.2e} taps {worst_tap:.2e} margin {margin:.3e}")


@pytest.mark.parametrize("preset,want", [("tiny_q8", MFMA), ("tiny_qwen", MFMA), ("small_q8", MFMA),
                                         ("tiny_f32", TOKENS), ("tiny_mixq4", MFMA), ("tiny_mixfmt", MFMA)])
def test_prefill_path_selection(pkg, gguf, preset, want):
    """Prompts run on the matrix cores when every layer matrix is Q8_0, Q4_0, Q4_1, F16,
    F32 or Q6_K with rows of a multiple of 64 (256 for Q6_K; gate and up in one format);
    tiny_f32's rows of 32 keep the per-token path; PREFILL_TOKENS forces it."""
    hip = pkg.HipModel(gguf(preset), max_seq=64)
    assert hip.prefill_path() == want
    hip.set_prefill_path(TOKENS)
    assert hip.prefill_path() == TOKENS
    hip.close()


def test_prefill_paths_agree(pkg, gguf):
    """A 150-token prompt through the matrix cores and token by token: logits within 1e-4,
    same argmax, same per-layer activations and KV cache within 1e-4, same greedy stream."""
    path = gguf("small_q8")
    info = pkg.synth_preset_info("small_q8")
    prompt = pkg.synth_prompt(info["seed"] + 1, 150, info["n_vocab"])
    res = []
    for pf in (TOKENS, MFMA):
        hip = pkg.HipModel(path, max_seq=256)
        hip.set_prefill_path(pf)
        lg, am = hip.prefill(prompt)
        taps = [hip.layer_act(layer) for layer in range(5)]
        kv = [hip.read_kv(layer, w, 0, 150) for layer in (0, 3) for w in (0, 1)]
        ids = hip.generate(8)
        res.append((lg, am, taps, kv, ids))
        hip.close()
    (l0, a0, t0, k0, i0), (l1, a1, t1, k1, i1) = res
    assert a0 == a1 and np.array_equal(i0, i1)
    assert rel_err(l1, l0) <= 1e-4
    for a, b in zip(t1, t0):
        assert rel_err(a, b) <= 1e-4
    for a, b in zip(k1, k0):
        assert rel_err(a, b) <= 1e-4


@pytest.mark.parametrize("n_prompt", [2, 16, 17, 32, 33, 64, 65, 129, 257, 2700])
def test_prefill_prompt_lengths(pkg, gguf, n_prompt):
    """Prompt lengths on either side of every tile shape the matrix-core prefill picks by
    row count (16-, 32- and 64-row register-streamed tiles, chunks padded to 128-row tiles,
    K split or not; at 2700 rows gate/up's 264 large tiles run as 242 + 22 in two launches):
    logits, per-layer activations and the greedy stream against the oracle."""
    info = pkg.synth_preset_info("small_q8")
    prompt = pkg.synth_prompt(info["seed"] + n_prompt, n_prompt, info["n_vocab"])
    max_seq = max(512, n_prompt + 64)
    ids, worst, worst_tap, margin = model_parity(pkg, gguf("small_q8"), prompt, 2, max_seq, 0)
    print(f"small_q8 {n_prompt}-token prompt: ids {ids} logits {worst:.2e} taps {worst_tap:.2e}")


@pytest.mark.parametrize("n_prompt", [6, 150])
@pytest.mark.parametrize("preset", ["tiny_mixq4", "tiny_mixfmt"])
def test_mixed_format_prefill(pkg, gguf, preset, n_prompt):
    """Q4_0 / Q4_1 / F16 / F32 / Q6_K / Q8_0 layer matrices on the matrix cores against the
    oracle (tiny_mixfmt: q, k and v in different formats, one launch each; Q4_1 and F16
    gate / up; F32 q and ffn_down; a Q6_K attention output), and against the per-token
    prefill of the same prompt."""
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"] + 3, n_prompt, info["n_vocab"])
    hip = pkg.HipModel(gguf(preset), max_seq=256)
    assert hip.prefill_path() == MFMA
    hip.close()
    ids, worst, worst_tap, margin = model_parity(pkg, gguf(preset), prompt, 8, 256, 0)
    print(f"{preset} {n_prompt}-token prompt: ids {ids} logits {worst:.2e} taps {worst_tap:.2e} margin {margin:.3e}")
    res = []
    for pf in (TOKENS, MFMA):
        hip = pkg.HipModel(gguf(preset), max_seq=256)
        hip.set_prefill_path(pf)
        lg, am = hip.prefill(prompt)
        kv = [hip.read_kv(layer, w, 0, n_prompt) for layer in range(hip.n_layer) for w in (0, 1)]
        res.append((lg, am, kv))
        hip.close()
    (l0, a0, k0), (l1, a1, k1) = res
    assert a0 == a1 and rel_err(l1, l0) <= 1e-4
    for a, b in zip(k1, k0):
        assert rel_err(a, b) <= 1e-4


@pytest.mark.parametrize("n_prompt", [4200, 4097])
def test_long_prompt_runs_in_chunks(pkg, gguf, n_prompt):
    """A prompt longer than one prefill chunk (4096 rows): later chunks attend to the earlier
    ones through the cache, as one attn_prefill over the whole prompt does; 4097 tokens leave
    a last chunk of one row."""
    info = pkg.synth_preset_info("tiny_q8")
    prompt = pkg.synth_prompt(info["seed"] + 2, n_prompt, info["n_vocab"])
    ids, worst, worst_tap, margin = model_parity(pkg, gguf("tiny_q8"), prompt, 4, 4352, 1)
    print(f"tiny_q8 {n_prompt}-token prompt: ids {ids} logits {worst:.2e} taps {worst_tap:.2e}")


def test_step_and_graph_agree(pkg, gguf):
    """Both decode paths give the same greedy stream and logits within 1e-5 from the same state."""
    path = gguf("small_q8")
    prompt = np.array([3, 99, 7, 1200, 5, 42, 8], np.int32)
    out = []
    for p in (GRAPH, STEP):
        hip = pkg.HipModel(path, max_seq=64)
        hip.set_decode_path(p)
        lp, _ = hip.prefill(prompt)
        ids = hip.generate(12)
        ld, _ = hip.decode(int(ids[-1]))
        out.append((lp, ids, ld))
        hip.close()
    assert np.array_equal(out[0][1], out[1][1])
    assert rel_err(out[0][0], out[1][0]) <= 1e-5 and rel_err(out[0][2], out[1][2]) <= 1e-5


def test_reference_ci_prompts(pkg, gguf):
    """The reference's correctness gate corpus (test_correctness.cpp:102-109) on its model shape."""
    path = gguf("tiny_f32")
    for i in range(20):
        prompt = np.array([1, 3 + (i % 20), 5 + (i * 3) % 30, 7], np.int32)
        model_parity(pkg, path, prompt, 8, 64, 0, taps=False)


def test_second_prefill_attends_only_to_its_chunk(pkg, gguf):
    """attn_prefill covers only the current call's tokens (attention.cpp:82-111), also when
    n_pos > 0 at entry; the backend reproduces that."""
    from oracle.bind import OracleModel
    path = gguf("tiny_q8")
    orc = OracleModel(path, max_seq=64)
    hip = pkg.HipModel(path, max_seq=64)
    a = np.array([5, 9, 11], np.int32)
    b = np.array([300, 17, 2, 40], np.int32)
    orc.prefill(a)
    hip.prefill(a)
    lo = orc.prefill(b)
    lh, _ = hip.prefill(b)
    assert rel_err(lh, lo) <= 1e-3
    assert hip.n_pos == 7
    hip.close()


def test_errors_and_reset(pkg, gguf):
    path = gguf("tiny_q8")
    hip = pkg.HipModel(path, max_seq=8)
    with pytest.raises(RuntimeError, match="exceeds max_seq"):
        hip.prefill(np.arange(9, dtype=np.int32))
    with pytest.raises(RuntimeError, match="out of range"):
        hip.decode(hip.n_vocab)
    with pytest.raises(RuntimeError, match="out of range"):
        hip.decode(-1)
    with pytest.raises(RuntimeError):
        hip.generate(3)  # nothing decoded yet
    l1, _ = hip.prefill(np.array([1, 2, 3], np.int32))
    g1 = hip.generate(5)
    with pytest.raises(RuntimeError, match="exceeds max_seq"):
        hip.decode(1)  # position 8 == max_seq
    hip.reset()
    assert hip.n_pos == 0
    l2, _ = hip.prefill(np.array([1, 2, 3], np.int32))
    g2 = hip.generate(5)
    assert np.array_equal(l1, l2) and np.array_equal(g1, g2)  # deterministic replays
    hip.close()


@pytest.mark.parametrize("preset,n_prompt,n_gen,max_seq,layout", [
    ("llama1b_q8", 6, 32, 512, 0),      # Llama-3.2-1B shape, Q8_0: the headline workload
    ("qwen05b_q8", 16, 128, 512, 0),    # Qwen2.5-0.5B shape with QKV bias
    ("llama1b_mixq4", 6, 64, 512, 0),   # Q4_0 / Q4_1 / Q6_K mix
    ("qwen15b_q8", 64, 16, 8192, 1),    # Qwen2.5-1.5B shape, head-major cache (short prompt)
    ("llama1b_q8", 512, 16, 1024, 0),   # 512-token prompt on the matrix cores, then 16 decode tokens
    ("llama1b_q8", 513, 8, 1024, 0),    # 513 rows: gate/up's 320 large tiles run as 256 + 64 (K split)
    ("llama1b_mixq4", 512, 16, 1024, 0),  # the same on Q4_0 / Q4_1 layer matrices
])
def test_full_size(pkg, gguf, preset, n_prompt, n_gen, max_seq, layout):
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"], n_prompt, info["n_vocab"])
    ids, worst, worst_tap, margin = model_parity(pkg, gguf(preset), prompt, n_gen, max_seq, layout)
    print(f"{preset}: {len(ids)} tokens identical; logits {worst:.2e} taps {worst_tap:.2e} margin {margin:.3e}")


GOLDEN =__import__("pathlib").Path(__file__).resolve().parent / "golden"


def test_long_context_workload_vs_reference_fixture(pkg, gguf):
    """The Qwen2.5-1.5B-shape workload at full size: a 4096-token prompt (matrix-core
    prefill in one chunk), head-major cache of 8192 positions, then 256 greedy tokens,
    against the reference's own run (tests/golden/qwen15b_4096.npz, written by
    make_golden_long.py from the compiled reference; the taps from the oracle run whose
    logits equal the reference's bit for bit). Per step: the device argmax is the
    reference's token, and the device logits at the reference's top-8 tokens are within
    1e-3 of the largest of them; the last step's taps within 1e-3; the one-launch greedy
    loop from a reset gives the same 256 tokens."""
    fx = np.load(GOLDEN / "qwen15b_4096.npz")
    path = gguf("qwen15b_q8")
    import hashlib
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    assert h.digest() == fx["gguf_sha256"].tobytes(), "synthetic writer output changed"
    info = pkg.synth_preset_info("qwen15b_q8")
    prompt = pkg.synth_prompt(int(fx["prompt_seed"]), int(fx["n_prompt"]), info["n_vocab"])
    ids, top_i, top_v = fx["ids"], fx["top_idx"], fx["top_val"]
    hip = pkg.HipModel(path, max_seq=int(fx["max_seq"]), kv_layout=int(fx["layout"]))
    try:
        assert hip.decode_path() == STEP
        worst = 0.0

        def check(step, lg, am):
            nonlocal worst
            want = top_v[step].astype(np.float64)
            e = float(np.max(np.abs(lg[top_i[step]] - want)) / np.max(np.abs(want)))
            assert e <= 1e-3, f"step {step}: top-8 logits rel err {e:.3e}"
            assert am == int(top_i[step][0]), f"step {step}: argmax {am} != reference {top_i[step][0]}"
            worst = max(worst, e)

        lg, am = hip.prefill(prompt)
        check(0, lg, am)
        for i in range(len(ids)):
            lg, am = hip.decode(int(ids[i]))
            check(i + 1, lg, am)
        for layer, want in zip(fx["tap_layers"], fx["taps"]):
            e = rel_err(hip.layer_act(int(layer)), want)
            assert e <= 1e-3, f"tap {layer} rel err {e:.3e}"
            assert e <= REGRESS, f"tap {layer}: numerics regression {e:.2e}"
        hip.reset()
        _, am0 = hip.prefill(prompt, want_logits=False)
        assert am0 == ids[0]
        gen = hip.generate(len(ids))  # its first token is the prefill's argmax
        assert gen.tolist() == ids.tolist()
        assert worst <= REGRESS, f"numerics regression: top-8 logits {worst:.2e}"
        print(f"qwen15b 4096 + {len(ids)}: ids identical, top-8 logits rel err {worst:.2e}")
    finally:
        hip.close()


@pytest.mark.parametrize("preset,layout", [("tiny_q8", "seq"), ("tiny_qwen", "head"), ("tiny_mixq4", "seq")])
def test_reference_cli_with_gpu_backend(pkg, gguf, preset, layout):
    """The reference's own CLI and Model with the backend switch patched in
    (oracle/backend_patch.py): `--backend hip` prints the same greedy tokens as its CPU path.
    (This process holds the cooperative-launch resource, so the child runs the graph path.)"""
    import os
    import pathlib
    import subprocess

    exe = pathlib.Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "tinferno_backend"
    if not exe.exists():
        pytest.skip("oracle/_ref/tinferno_backend not built (needs the reference sources)")
    info = pkg.synth_preset_info(preset)
    toks = ",".join(str(t) for t in pkg.synth_prompt(info["seed"], 6, info["n_vocab"]))
    args = [str(exe), "--model", gguf(preset), "--tokens", toks, "--n-predict", "16", "--max-seq", "64",
            "--kv-layout", layout, "--threads", "4"]
    env = dict(os.environ, TF_HIP_DECODE_PATH="graph")
    cpu = subprocess.run(args, capture_output=True, text=True, timeout=300, env=env)
    gpu = subprocess.run(args + ["--backend", "hip"], capture_output=True, text=True, timeout=300, env=env)
    assert cpu.returncode == 0 and gpu.returncode == 0, cpu.stderr[-500:] + gpu.stderr[-500:]
    assert gpu.stdout == cpu.stdout and cpu.stdout.strip()
