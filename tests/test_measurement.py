"""What the roofline figures rest on, pinned on the CPU.

* Model::decode_bytes (the numerator of every achieved-GB/s figure) against the per-token
  byte formula written out from each workload's shape: every tensor once (the tied
  token_embd as the lm_head), one embedding row, fp32 K and V rows of every attended
  position plus the new row.
* The host RoPE tables the Model uploads against the reference's own rope_one
  (attention.cpp:31-41, compiled from its sources): rotating a vector whose pairs are
  (1, 0) yields exactly (cos, sin) of the reference's angle, since the rotation's products
  with 1 and 0 are exact.
"""
import ctypes as C

import numpy as np
import pytest

from oracle.bind import ref_available, ref_lib

needs_ref = pytest.mark.skipif(not ref_available(), reason="reference not built (oracle/_ref)")

BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 8: (32, 34), 14: (256, 210)}


def rb(t, k):
    """row_nbytes (tensor.cpp:66-70)."""
    e, b = BLOCK[t]
    return k // e * b


def formula_bytes(info, pos, layer_type, embd_type, bias=False, overrides=()):
    """Bytes one decode step reads at position pos, from the shape alone."""
    D, F, L, H, G, V = (info[k] for k in ("n_embd", "n_ff", "n_layer", "n_head", "n_kv_head", "n_vocab"))
    hd = D // H
    total = 0
    for layer in range(L):
        down_t = dict(overrides).get(layer, layer_type)
        total += rb(layer_type, D) * (H * hd + 2 * G * hd)  # wq, wk, wv
        total += rb(layer_type, H * hd) * D                 # wo
        total += 2 * rb(layer_type, D) * F                  # gate, up
        total += rb(down_t, F) * D                          # down
        total += 2 * D * 4                                  # attn_norm, ffn_norm (F32)
        if bias:
            total += (H * hd + 2 * G * hd) * 4              # bq, bk, bv (F32)
    total += D * 4                                          # output_norm
    total += rb(embd_type, D) * V                           # tied lm_head = token_embd
    total += rb(embd_type, D)                               # the embedding row
    total += L * G * hd * 4 * 2 * (pos + 2)                 # K, V rows at 0..pos and the new row
    return total


@pytest.mark.slow
@pytest.mark.parametrize("preset,layer_type,embd_type,bias,overrides", [
    ("llama1b_q8", 8, 8, False, ()),
    ("qwen05b_q8", 8, 8, True, ()),
    ("llama1b_mixq4", 2, 14, False, ((0, 3), (15, 3))),
])
def test_decode_bytes_formula(pkg, gguf, preset, layer_type, embd_type, bias, overrides):
    info = pkg.synth_preset_info(preset)
    path = gguf(preset)
    for pos in (0, 6, 25, 511):
        want = formula_bytes(info, pos, layer_type, embd_type, bias, overrides)
        assert pkg.file_decode_bytes(path, pos) == want, pos
    if preset == "llama1b_q8":
        # the headline workload: mean over the 32 greedy steps after the 6-token prompt
        mean = np.mean([pkg.file_decode_bytes(path, 6 + i) for i in range(32)])
        assert mean == formula_bytes(info, 6, 8, 8) + 15.5 * 16 * 8 * 64 * 8
        assert abs(mean / 1e9 - 1.3148) < 5e-5


def test_decode_bytes_small_presets(pkg, gguf):
    """Same formula on the small presets (untied tiny_f32: output.weight is the lm_head and
    token_embd contributes one row)."""
    for preset, lt, et, bias in (("tiny_q8", 8, 8, False), ("tiny_qwen", 8, 8, True), ("tiny_hd128", 8, 8, True),
                                 ("small_q8", 8, 8, False)):
        info = pkg.synth_preset_info(preset)
        assert pkg.file_decode_bytes(gguf(preset), 9) == formula_bytes(info, 9, lt, et, bias), preset
    info = pkg.synth_preset_info("tiny_f32")
    D, V = info["n_embd"], info["n_vocab"]
    untied = formula_bytes(info, 9, 0, 0)  # tied form: V rows of token_embd + one row
    assert pkg.file_decode_bytes(gguf("tiny_f32"), 9) == untied  # output.weight has token_embd's size
    assert V * D * 4 == rb(0, D) * V


def _ref_tables(freq, n_pos):
    """cos/sin of the reference's angles for every position: rope_one on pairs (1, 0)."""
    R = ref_lib()
    d2 = len(freq)
    fp = C.POINTER(C.c_float)
    f = np.ascontiguousarray(freq, np.float32)
    c = np.zeros((n_pos, d2), np.float32)
    s = np.zeros((n_pos, d2), np.float32)
    for p in range(n_pos):
        x = np.concatenate([np.ones(d2, np.float32), np.zeros(d2, np.float32)])
        R.ref_rope(x.ctypes.data_as(fp), 1, 2 * d2, p, f.ctypes.data_as(fp))
        c[p], s[p] = x[:d2], x[d2:]
    return c, s


def _ref_freqs(theta, n_rot):
    R = ref_lib()
    f = np.zeros(n_rot // 2, np.float32)
    R.ref_rope_freqs(f.ctypes.data_as(C.POINTER(C.c_float)), n_rot, theta, 0, 1.0, 1.0, 4.0, 8192.0)
    return f


@needs_ref
@pytest.mark.parametrize("theta,n_rot,n_pos", [(500000.0, 64, 512), (1000000.0, 128, 8192), (1000000.0, 64, 512),
                                               (10000.0, 32, 64)])
def test_rope_tables_bit_exact_vs_reference(pkg, theta, n_rot, n_pos):
    """The tables of the headline (theta 5e5, head_dim 64, 512 positions) and long-context
    (theta 1e6, head_dim 128, 8192 positions) workloads, bit for bit."""
    c, s = pkg.rope_tables(theta, n_rot, n_pos)
    rc, rs = _ref_tables(_ref_freqs(theta, n_rot), n_pos)
    assert np.array_equal(c.view(np.uint32), rc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("preset", ["tiny_q8", "tiny_qwen", "tiny_hd128"])
def test_model_rope_tables_from_file(pkg, gguf, preset):
    """The tables the Model derives from a GGUF's metadata (its theta and head_dim)."""
    info = pkg.synth_preset_info(preset)
    hd = info["n_embd"] // info["n_head"]
    c, s = pkg.file_rope_tables(gguf(preset), 256, hd // 2)
    theta = {"tiny_q8": 500000.0, "tiny_qwen": 1000000.0, "tiny_hd128": 1000000.0}[preset]
    rc, rs = _ref_tables(_ref_freqs(theta, hd), 256)
    assert np.array_equal(c.view(np.uint32), rc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_stream_checksum_closed_form(pkg):
    """The streams' expected checksum (word i = i * 0x9E3779B1, summed mod 2^32) against a
    brute-force sum, including sizes that are not a multiple of 16 bytes."""
    for nbytes in (16, 48, 4096, 1 << 20, (1 << 20) + 40):
        n = nbytes // 16 * 4
        words = (np.arange(n, dtype=np.uint64) * np.uint64(0x9E3779B1)) % np.uint64(1 << 32)
        assert pkg.stream_checksum(nbytes) == int(words.sum() % np.uint64(1 << 32)), nbytes


def _load(name, path):
    import importlib.util
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_traffic_summaries_are_of_these_sources(tmp_path, monkeypatch):
    """bench.py takes a config's roofline.traffic from its counter summary only while the
    summary's kernel-source digest is that of the sources it runs: the committed summaries
    carry profsum's digest of this tree, a summary with another digest gives no traffic, and
    the figure is the per-token bytes x tokens."""
    import pathlib
    import sys
    root = pathlib.Path(__file__).resolve().parents[1]
    monkeypatch.setattr(sys, "argv", ["bench.py"])
    bench = _load("bench_for_test", root / "bench.py")
    profsum = _load("profsum_for_test", root / "agent-serve_amd" / "profsum.py")
    digest = profsum.kernel_source_digest()
    assert bench.kernel_source_digest() == digest
    for key in ("cfg1", "cfg2", "cfg3", "cfg4", "cfg5"):
        traffic, src = bench.measured_traffic(key, 32, "k_step")
        assert src["current"], (key, src)
        assert src["csrc_sha256"] == digest and traffic > 0
    stale = tmp_path / "stale.txt"
    stale.write_text("traffic_bytes_per_token k_step 1000\ncommit abc\ncsrc_sha256 0000000000000000\n")
    monkeypatch.setitem(bench.TRAFFIC_SUMMARIES, "cfg1", stale)
    traffic, src = bench.measured_traffic("cfg1", 32, "k_step")
    assert traffic is None and src["current"] is False and src["commit"] == "abc"
    good = tmp_path / "good.txt"
    good.write_text(f"traffic_bytes_per_token k_step 1000\ncommit abc\ncsrc_sha256 {digest}\n")
    monkeypatch.setitem(bench.TRAFFIC_SUMMARIES, "cfg1", good)
    traffic, src = bench.measured_traffic("cfg1", 32, "k_step")
    assert traffic == 32000 and src["current"]
