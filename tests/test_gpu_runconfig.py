"""RunConfig stage presets and the timing entry points on the GPU.

Stage presets (common.hpp:289-322, main.cpp:79-91): `--stage v5` selects the head-major KV
cache (common.hpp:313-317), `--kv-layout` overrides a preset's layout. On the GPU that is the
device cache's layout, read back through tf_hip_get_hparams and the TF_HIP_LOG line of
tf_hip_create. The layout changes no result, so every variant must print the same tokens.

Timings (common.hpp:118-134, main.cpp:132-141): tf_hip_last_timing and tf_hip_profile_generate
against the host clock, the greedy loop and the decode byte formula.
"""
import os
import pathlib
import subprocess
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]
SEQ, HEAD = 0, 1  # TF_HIP_KV_SEQ_MAJOR, TF_HIP_KV_HEAD_MAJOR


@pytest.mark.parametrize("stage,kv_layout,want", [("v2", -1, SEQ), ("v5", -1, HEAD), ("v0", -1, SEQ),
                                                  ("v4", -1, SEQ), ("v5", SEQ, SEQ), ("v2", HEAD, HEAD)])
def test_stage_preset_selects_device_kv_layout(pkg, gguf, stage, kv_layout, want):
    """Model(path, RunConfig) through the host side: the preset's layout (or the override)
    is the device cache's, and the greedy stream is the same for every layout."""
    path = gguf("tiny_q8")
    info = pkg.synth_preset_info("tiny_q8")
    prompt = pkg.synth_prompt(info["seed"], 6, info["n_vocab"])
    streams = []
    for st, kv in ((stage, kv_layout), ("v2", SEQ)):
        m = pkg.HipModel(path, max_seq=64, kv_layout=kv, stage=st)
        try:
            if (st, kv) == (stage, kv_layout):
                assert m.kv_layout == want
                assert m.device_hparams()["kv_layout"] == want
            _, first = m.prefill(prompt)
            streams.append([first] + m.generate(12).tolist())
        finally:
            m.close()
    assert streams[0] == streams[1]


def _run(args, env):
    r = subprocess.run(args, capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr[-800:]
    return r


def _cli_case(pkg, gguf):
    info = pkg.synth_preset_info("tiny_qwen")
    toks = ",".join(str(t) for t in pkg.synth_prompt(info["seed"], 6, info["n_vocab"]))
    # no decode path is forced: a test process that launched the step kernel holds the
    # GPU's cooperative-launch resource, and the child's refused step launch then runs its
    # tokens on the graph path (the library's fallback)
    env = dict(os.environ, TF_HIP_LOG="1")
    return gguf("tiny_qwen"), toks, env


def test_cli_stage_v5_runs_head_major(pkg, gguf):
    """tinferno_hip --stage v5 creates a head-major device cache (its TF_HIP_LOG line and its
    describe() line say kv=head) and prints the tokens of --kv-layout head and of v2."""
    path, toks, env = _cli_case(pkg, gguf)
    exe = str(pkg.BIN_DIR / "tinferno_hip")
    base = [exe, "--model", path, "--tokens", toks, "--n-predict", "16", "--max-seq", "64"]
    v5 = _run(base + ["--stage", "v5"], env)
    head = _run(base + ["--kv-layout", "head"], env)
    v2 = _run(base + ["--stage", "v2"], env)
    describe = [ln for ln in v5.stderr.splitlines() if ln.startswith("arch=")]
    assert "tf_hip: device 0 kv=head" in v5.stderr and describe and " kv=head" in describe[0]
    assert "tf_hip: device 0 kv=head" in head.stderr
    assert "tf_hip: device 0 kv=seq" in v2.stderr
    assert v5.stdout.strip() and v5.stdout == head.stdout == v2.stdout


def test_cli_device_loop_prints_the_loop_tokens(pkg, gguf):
    """tinferno_hip --device-loop (the greedy tokens from one tf_hip_generate call, as bench.py
    runs them) prints the tokens of the reference's decode-per-token loop."""
    path, toks, env = _cli_case(pkg, gguf)
    exe = str(pkg.BIN_DIR / "tinferno_hip")
    base = [exe, "--model", path, "--tokens", toks, "--n-predict", "24", "--max-seq", "64"]
    loop = _run(base, env)
    dev = _run(base + ["--device-loop"], env)
    assert loop.stdout.strip() and dev.stdout == loop.stdout


def test_patched_reference_stage_v5_runs_head_major(pkg, gguf):
    """The reference's own CLI with the backend switch (oracle/backend_patch.py): with
    --backend hip, --stage v5 hands the head-major layout to tf_hip_create, and the tokens
    equal those of --kv-layout head and of its CPU v2 path."""
    exe = ROOT / "oracle" / "_ref" / "tinferno_backend"
    if not exe.exists():
        pytest.skip("oracle/_ref/tinferno_backend not built (needs the reference sources)")
    path, toks, env = _cli_case(pkg, gguf)
    base = [str(exe), "--model", path, "--tokens", toks, "--n-predict", "16", "--max-seq", "64", "--threads", "4"]
    v5 = _run(base + ["--stage", "v5", "--backend", "hip"], env)
    head = _run(base + ["--kv-layout", "head", "--backend", "hip"], env)
    cpu = _run(base + ["--stage", "v2"], env)  # the CPU path whose arithmetic the GPU follows
    assert "tf_hip: device 0 kv=head" in v5.stderr
    assert "tf_hip: device 0 kv=head" in head.stderr
    assert "tf_hip:" not in cpu.stderr  # the CPU path creates no device context
    assert v5.stdout.strip() and v5.stdout == head.stdout == cpu.stdout


@pytest.mark.parametrize("path_id", [0, 1], ids=["graph", "step"])
def test_last_timing_against_host_clock(pkg, gguf, path_id):
    """tf_hip_last_timing after tf_hip_generate: the step path is one launch named k_step,
    the graph path one replay per token; the kernel time is positive and no longer than the
    call's host wall time."""
    path = gguf("tiny_q8")
    info = pkg.synth_preset_info("tiny_q8")
    prompt = pkg.synth_prompt(info["seed"], 6, info["n_vocab"])
    m = pkg.HipModel(path, max_seq=64)
    try:
        m.set_decode_path(path_id)
        m.prefill(prompt)
        n = 16
        t0 = time.perf_counter()
        m.generate(n)
        wall_ms = (time.perf_counter() - t0) * 1e3
        total, kernel, launches, name = m.last_timing()
        if path_id == 1:
            assert (name, launches) == ("k_step", 1)
        else:
            assert (name, launches) == ("decode_graph", n)
        assert 0 < kernel <= total <= wall_ms, (kernel, total, wall_ms)
    finally:
        m.close()


@pytest.mark.parametrize("preset", ["tiny_q8", "tiny_qwen", "tiny_mixq4"])
def test_profile_generate_counts(pkg, gguf, preset):
    """tf_hip_profile_generate runs the greedy loop kernel by kernel: the same tokens as
    tf_hip_generate, one launch per class and layer (embedding and lm_head once per token),
    and its per-class bytes add up to the decode byte formula over the steps."""
    path = gguf(preset)
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"], 6, info["n_vocab"])
    n = 8
    m = pkg.HipModel(path, max_seq=64)
    try:
        m.prefill(prompt)
        pos0 = m.n_pos
        ids_p, by = m.profile_generate(n)
        m.reset()
        m.prefill(prompt)
        ids_g = m.generate(n)
        assert np.array_equal(ids_p, ids_g)
        L = m.n_layer
        want_launches = {"embed": n, "qkv_gemv": n * L, "attention": n * L, "wo_gemv": n * L,
                         "gateup_gemv": n * L, "down_gemv": n * L, "lmhead_gemv": n}
        for k, v in want_launches.items():
            assert by[k][1] == v, (k, by[k])
        assert all(ms > 0 for ms, _, _ in by.values())
        total = sum(b for _, _, b in by.values())
        want = sum(m.decode_bytes(pos0 + i) for i in range(n))
        assert total == want, (total, want)
    finally:
        m.close()
