"""Host side on the CPU: the seeded synthetic writer, its quantizers, the GGUF readers,
and the CLI harnesses' argument handling."""
import ctypes as C
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

from oracle.bind import OracleModel, oracle_lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SYNTH = os.path.join(ROOT, "agent-serve_amd", "bin", "tinferno_synth")
CLI = os.path.join(ROOT, "agent-serve_amd", "bin", "tinferno_hip")
fp = C.POINTER(C.c_float)


def dequant(t, blob, n):
    out = np.zeros(n, np.float32)
    assert oracle_lib().orc_dequant_row(t, blob.ctypes.data, n, out.ctypes.data_as(fp)) == 0
    return out


def test_quantizer_round_trips(pkg):
    """test_ops.cpp:68-97 bounds (Q8_0 < 0.05, Q4_0 < 0.6 on sin(0.3 i)), and the
    half-step bounds the Q4_1/Q6_K quantizers promise."""
    x = np.sin(0.3 * np.arange(256)).astype(np.float32)
    assert np.max(np.abs(dequant(8, pkg.quantize_row(8, x), 256) - x)) < 0.05
    assert np.max(np.abs(dequant(2, pkg.quantize_row(2, x), 256) - x)) < 0.6
    y = dequant(3, pkg.quantize_row(3, x), 256)
    for b in range(8):
        blk = x[32 * b:32 * b + 32]
        assert np.max(np.abs(y[32 * b:32 * b + 32] - blk)) <= (blk.max() - blk.min()) / 30 * 1.01 + 1e-3
    rng = np.random.default_rng(0)
    z = (rng.standard_normal(1024) * 0.02).astype(np.float32)
    w = dequant(14, pkg.quantize_row(14, z), 1024)
    assert np.max(np.abs(w - z)) < 0.02 * 0.2
    assert np.array_equal(dequant(0, pkg.quantize_row(0, z), 1024), z)
    assert np.array_equal(dequant(1, pkg.quantize_row(1, z), 1024), z.astype(np.float16).astype(np.float32))


def test_writer_is_deterministic_and_readable(pkg, tmp_path):
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    wa = pkg.synth_write("tiny_mixq4", str(a), threads=1)
    wb = pkg.synth_write("tiny_mixq4", str(b), threads=7)
    assert wa == wb
    assert hashlib.sha256(a.read_bytes()).digest() == hashlib.sha256(b.read_bytes()).digest()
    s = pkg.gguf_summary(str(a))
    assert s["weight_bytes"] == wa and s["arch"] == "llama" and s["n_tensors"] == 2 + 3 * 9
    m = OracleModel(str(a), 16)
    assert (m.n_vocab, m.n_embd, m.n_layer, m.n_head, m.n_kv_head, m.head_dim) == (512, 256, 3, 4, 2, 64)


def test_seed_changes_weights_and_prompt(pkg, tmp_path):
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    pkg.synth_write("tiny_q8", str(a), seed=1)
    pkg.synth_write("tiny_q8", str(b), seed=2)
    assert a.read_bytes() != b.read_bytes()
    p1, p2 = pkg.synth_prompt(1, 16, 512), pkg.synth_prompt(2, 16, 512)
    assert not np.array_equal(p1, p2) and p1.min() >= 0 and p1.max() < 512
    assert np.array_equal(p1, pkg.synth_prompt(1, 16, 512))


def test_full_size_byte_footprint(pkg):
    """The Llama presets reproduce the reference's published weight footprints less the
    128 B rope_freqs tensor of the real files (BASELINE: 1,313,251,456 and 765,194,368)."""
    info = pkg.synth_preset_info("llama1b_q8")
    D, F, L, V = info["n_embd"], info["n_ff"], info["n_layer"], info["n_vocab"]
    hd = D // info["n_head"]
    kv = info["n_kv_head"] * hd
    q8 = lambda k, n: k // 32 * 34 * n  # noqa: E731
    per_layer = q8(D, D) + 2 * q8(D, kv) + q8(D, D) + 2 * q8(D, F) + q8(F, D) + 2 * D * 4
    assert q8(D, V) + D * 4 + L * per_layer == 1313251456 - 128
    q4 = lambda k, n: k // 32 * 18 * n  # noqa: E731
    q41 = lambda k, n: k // 32 * 20 * n  # noqa: E731
    per_layer4 = q4(D, D) + 2 * q4(D, kv) + q4(D, D) + 2 * q4(D, F) + 2 * D * 4
    total = D // 256 * 210 * V + D * 4 + L * per_layer4 + (L - 2) * q4(F, D) + 2 * q41(F, D)
    assert total == 765194368 - 128


def test_host_reader_errors(pkg, tmp_path):
    good = tmp_path / "m.gguf"
    pkg.synth_write("tiny_q8", str(good))
    raw = good.read_bytes()
    bad = tmp_path / "bad.gguf"
    cases = [(b"XXXX" + raw[4:], "not a GGUF file"), (raw[:100], "truncated"), (raw[: len(raw) // 2], "out of range"),
             (raw[:4] + (9).to_bytes(4, "little") + raw[8:], "unsupported GGUF version")]
    for blob, msg in cases:
        bad.write_bytes(blob)
        with pytest.raises(RuntimeError, match=msg):
            pkg.gguf_summary(str(bad))


def test_synth_cli(tmp_path):
    out = subprocess.run([SYNTH, "--preset", "tiny_qwen", "--out", str(tmp_path / "q.gguf"), "--prompt", "4"],
                         check=True, capture_output=True, text=True)
    d = json.loads(out.stdout)
    assert d["preset"] == "tiny_qwen" and len(d["prompt"]) == 4 and d["weight_bytes"] > 0
    r = subprocess.run([SYNTH, "--preset", "nope", "--out", str(tmp_path / "x.gguf")], capture_output=True, text=True)
    assert r.returncode == 1 and "presets:" in r.stderr


def test_cli_argument_errors():
    r = subprocess.run([CLI], capture_output=True, text=True)
    assert r.returncode == 1 and "usage" in r.stderr
    r = subprocess.run([CLI, "--model", "/nonexistent.gguf", "--tokens", "1,2"], capture_output=True, text=True)
    assert r.returncode == 1 and "cannot open" in r.stderr
    r = subprocess.run([CLI, "--bogus"], capture_output=True, text=True)
    assert r.returncode == 1 and "unknown flag" in r.stderr
    r = subprocess.run([CLI, "--model", "x", "--stage", "v9", "--tokens", "1"], capture_output=True, text=True)
    assert r.returncode == 1 and "unknown stage" in r.stderr
