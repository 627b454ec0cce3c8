"""Op-level parity of the HIP kernels against the oracle, through the C ABI.

Dequantization and argmax are integer/index work: bit-exact. GEMV, RMSNorm and attention
are fp32 reductions in a different order than the AVX2 reference: bounded by a
per-element error budget stated in each test.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import rel_err
from gpu_util import oracle_dequant, oracle_matmul, random_rows
from oracle.bind import oracle_lib

pytestmark = pytest.mark.gpu

FORMATS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q8_0": 8, "Q6_K": 14}


@pytest.mark.parametrize("fmt", list(FORMATS))
def test_dequant_rows_bit_exact(pkg, fmt):
    t = FORMATS[fmt]
    rng = np.random.default_rng(7 + t)
    k = 512 if t != 0 else 96
    rows = random_rows(rng, t, k, 37)
    got = pkg.dequant_rows(t, rows, k, 37)
    want = oracle_dequant(t, rows, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a sub-range of rows, as the embedding lookup reads one row
    got = pkg.dequant_rows(t, rows, k, 37, row0=11, nrows=3)
    assert np.array_equal(got.view(np.uint32), want[11:14].view(np.uint32))


# (K, N) of the workloads' matrices (some N trimmed to keep the oracle fast)
GEMV_SHAPES = {
    8: [(2048, 512), (2048, 2048), (8192, 384), (896, 128), (896, 4864), (4864, 896), (1536, 256), (8960, 256),
        (2048, 8200)],
    2: [(2048, 512), (8192, 256), (256, 64)],
    3: [(8192, 256), (2048, 96)],
    14: [(2048, 1024), (1536, 128), (256, 40)],
    0: [(32, 64), (64, 32), (2048, 64)],
    1: [(256, 64), (2048, 33)],
}


@pytest.mark.parametrize("t,k,n", [(t, k, n) for t, shapes in GEMV_SHAPES.items() for (k, n) in shapes])
def test_gemv_matches_oracle(pkg, t, k, n):
    """y = W x: |y - y_oracle| <= 2e-5 * sum_k |x_k w_nk| per output (fp32 reassociation)."""
    rng = np.random.default_rng(1000 + k + n + t)
    rows = random_rows(rng, t, k, n)
    x = rng.standard_normal(k).astype(np.float32)
    got = pkg.matmul(t, rows, k, n, x)[0]
    want = oracle_matmul(t, rows, k, x)[0]
    budget = np.abs(oracle_dequant(t, rows, k)).astype(np.float64) @ np.abs(x).astype(np.float64)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 2e-5 * budget + 1e-30), f"max err/budget {np.max(err / (budget + 1e-30)):.3e}"


def outlier_rows(pkg, rng, t, k, n):
    """Rows whose every block is dominated by one outlier: one element of magnitude 1 per
    32-element block (per 16-element sub-block for Q6_K), the others N(0, 0.01), quantized
    by the synthetic writer's quantizer, so the outlier takes the largest quant and the
    rest quantize to |q| <= 4 (Q8_0), 0 (Q4_0) or a few steps of 32 (Q6_K)."""
    group = 16 if t == 14 else 32
    out = []
    for _ in range(n):
        x = (rng.standard_normal(k) * 0.01).astype(np.float32)
        pos = np.arange(0, k, group) + rng.integers(0, group, size=k // group)
        x[pos] = rng.choice([-1.0, 1.0], size=k // group)
        out.append(pkg.quantize_row(t, x))
    return np.stack(out)


@pytest.mark.parametrize("t,k,n", [(8, 2048, 256), (8, 8192, 64), (2, 2048, 256), (14, 2048, 128)])
def test_gemv_outlier_blocks(pkg, t, k, n):
    """Outlier-dominated blocks, as real checkpoints have: within the oracle's 2e-5 budget,
    and for Q8_0 (signed quants, no offset term) within the rounding bound of the kernel's
    summation against the exact fp64 dot: each product passes 16 FMAs, the scale multiply,
    K / 1024 step adds and 6 wave-reduction adds, so |err| <= (23 + K/1024 + 1) 2^-24
    sum_k |x_k w_nk|."""
    rng = np.random.default_rng(4000 + t + k)
    rows = outlier_rows(pkg, rng, t, k, n)
    deq = oracle_dequant(t, rows, k)
    if t == 8:
        q = np.rint(np.abs(deq) / np.max(np.abs(deq), axis=1, keepdims=True) * 127)
        assert np.median(q) <= 4  # the blocks really are outlier-dominated
    x = rng.standard_normal(k).astype(np.float32)
    got = pkg.matmul(t, rows, k, n, x)[0].astype(np.float64)
    want = oracle_matmul(t, rows, k, x)[0]
    budget = np.abs(deq).astype(np.float64) @ np.abs(x).astype(np.float64)
    err = np.abs(got - want)
    assert np.all(err <= 2e-5 * budget + 1e-30), f"max err/budget {np.max(err / (budget + 1e-30)):.3e}"
    if t == 8:
        exact = deq.astype(np.float64) @ x.astype(np.float64)
        bound = (23 + k // 1024 + 1) * 2.0**-24 * budget
        e = np.abs(got - exact)
        assert np.all(e <= bound), f"max err / rounding bound {np.max(e / bound):.3f}"
        # typical error well inside the bound: a CPU model of the kernel's summation order
        # on such rows gives a median of 0.002 of the bound for the signed dot and 0.04 for
        # the offset form sum x (q + 128) - 128 sum x, whose rounding scales with 128 sum |x|
        med = float(np.median(e / bound))
        assert med <= 0.01, f"median err / rounding bound {med:.4f}"
        print(f"Q8_0 K={k}: max |gpu - exact| / sum|x w| = {np.max(e / budget):.3e}, median / bound {med:.4f}")


def test_matmul_several_rows(pkg):
    rng = np.random.default_rng(3)
    k, n = 2048, 256
    rows = random_rows(rng, 8, k, n)
    x = rng.standard_normal((5, k)).astype(np.float32)
    got = pkg.matmul(8, rows, k, n, x)
    want = oracle_matmul(8, rows, k, x)
    assert rel_err(got, want) < 1e-5


# (M, K, N) of the prefill GEMM: row counts around the 64-row tile, the workloads' K
PF_GEMM_SHAPES = [(2, 64, 16), (37, 2048, 256), (64, 896, 1152), (100, 8192, 128), (130, 1536, 48),
                  (512, 2048, 64), (65, 8960, 32), (7, 192, 320), (24, 2048, 512), (11, 8192, 2048),
                  (500, 256, 16384),  # enough 128 x 256 tiles for every CU: the LDS-staged kernel
                  (512, 2048, 2048),  # 32 such tiles, K split in 8 slices and reduced
                  (512, 512, 12288)]  # 192 such tiles, unsplit (slices would not shorten the span)


# the other formats the matrix cores take, read in their own layout: the register-streamed
# tiles, the LDS-staged tiles (500 x 256 x 16384) and K split in slices (512 x 2048 x 2048);
# F32 (0) and Q6_K (14, rows of a multiple of 256) always on their register-streamed tiles
PF_GEMM_FMT_SHAPES = [(t, m, k, n) for t in (2, 3, 1, 0, 14)
                      for (m, k, n) in [(2, 64, 16), (37, 2048, 256), (130, 1536, 48), (7, 192, 320),
                                        (500, 256, 16384), (512, 2048, 2048)]
                      if t != 14 or k % 256 == 0]


@pytest.mark.parametrize("t,m,k,n", [(8, m, k, n) for (m, k, n) in PF_GEMM_SHAPES] + PF_GEMM_FMT_SHAPES)
def test_prefill_gemm_matches_oracle(pkg, t, m, k, n):
    """Q8_0, Q4_0, Q4_1, F16, F32 or Q6_K rows x M activation rows on the matrix cores: |y - y_oracle|
    <= 2e-5 * sum_k |x_k w_nk| per output. The fp16 pair of an activation keeps it to 2^-22
    of its row's largest element; the rest is fp32 reassociation, as for the GEMV."""
    rng = np.random.default_rng(2000 + m + k + n + t)
    rows = random_rows(rng, t, k, n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = pkg.matmul(t, rows, k, n, x)
    want = oracle_matmul(t, rows, k, x)
    budget = np.abs(x).astype(np.float64) @ np.abs(oracle_dequant(t, rows, k)).astype(np.float64).T
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 2e-5 * budget + 1e-30), f"max err/budget {np.max(err / (budget + 1e-30)):.3e}"


@pytest.mark.parametrize("t", [8, 2, 3, 1, 0, 14])
def test_prefill_gemm_single_element_rows(pkg, t):
    """A row with one non-zero x_j gives x_j * w[:, j] (one product per output; Q4_1's
    d n + m as d (x n) + m x, which the oracle's fp32 dequant rounds once: within 2 ulp;
    Q6_K's d (x sc q), where the dequant rounds d sc q: within 2 ulp)."""
    rng = np.random.default_rng(90 + t)
    k, n = 256, 4096  # 500 rows below: the LDS-staged kernel
    rows = random_rows(rng, t, k, n)
    deq = oracle_dequant(t, rows, k)
    x = np.zeros((500, k), np.float32)
    js = rng.integers(0, k, 500)
    x[np.arange(500), js] = rng.choice([-3.0, 0.5, 2.0, 7.0], 500).astype(np.float32)
    got = pkg.matmul(t, rows, k, n, x)
    want = (x[np.arange(500), js][:, None] * deq[:, js].T).astype(np.float32)
    if t == 3:
        # Q4_1 blocks are (d, m, 16 bytes): the two roundings of x (d n) + x m, against the
        # magnitudes of their terms
        m = rows.reshape(n, k // 32, 20)[:, :, 2:4].copy().view(np.float16).astype(np.float64)[:, :, 0]
        mj = m[:, js // 32].T
        xa = np.abs(x[np.arange(500), js].astype(np.float64))[:, None]
        bound = 2.0**-22 * xa * (np.abs(deq[:, js].T - mj) + np.abs(mj))
        assert np.all(np.abs(got.astype(np.float64) - want) <= bound + 1e-30)
    elif t == 14:
        assert np.all(np.abs(got.astype(np.float64) - want) <= 2.0**-22 * np.abs(want) + 1e-30)
    else:
        assert np.array_equal(got, want)


def test_prefill_gemm_seeded_shapes(pkg):
    """Twenty shapes drawn from a fixed seed (rows 1..700, K a multiple of 64 up to 10,240, N a
    multiple of 16 up to 4,096; Q8_0, Q4_0 and Q4_1): whatever tile kernel and K split the
    launch picks for them, each output within 2e-5 * sum_k |x_k w_nk| of the oracle."""
    rng = np.random.default_rng(4242)
    for _ in range(20):
        t = int(rng.choice([8, 2, 3]))
        m = int(rng.integers(1, 701))
        k = 64 * int(rng.integers(1, 161))
        n = 16 * int(rng.integers(1, 257))
        while m * k * n > 1.5e9:
            n = max(16, n // 32 * 16)
            m = max(1, m // 2)
        rows = random_rows(rng, t, k, n)
        x = rng.standard_normal((m, k)).astype(np.float32)
        got = pkg.matmul(t, rows, k, n, x)
        want = oracle_matmul(t, rows, k, x)
        budget = np.abs(x).astype(np.float64) @ np.abs(oracle_dequant(t, rows, k)).astype(np.float64).T
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= 2e-5 * budget + 1e-30), f"type {t} {m}x{k}x{n}: max err/budget {np.max(err / (budget + 1e-30)):.3e}"


def test_prefill_gemm_row_scales(pkg):
    """Rows of very different magnitude keep their relative precision (each row has its own
    power-of-two scale); a zero row gives zeros; a row with one non-zero x_j gives
    x_j * w[:, j] bit-exactly (one exact product per output)."""
    rng = np.random.default_rng(77)
    k, n = 512, 64
    rows = random_rows(rng, 8, k, n)
    deq = oracle_dequant(8, rows, k)
    x = rng.standard_normal((6, k)).astype(np.float32)
    x[1] = 0.0
    x[2] *= 1e4
    x[3] *= 1e-6
    x[4] = 0.0
    x[4, 7] = 3.0
    x[5, 100] = 6.0e4  # one outlier above fp16's largest finite value
    got = pkg.matmul(8, rows, k, n, x)
    want = oracle_matmul(8, rows, k, x)
    budget = np.abs(x).astype(np.float64) @ np.abs(deq).astype(np.float64).T
    assert np.all(np.abs(got.astype(np.float64) - want) <= 2e-5 * budget + 1e-30)
    assert np.all(got[1] == 0.0)
    assert np.array_equal(got[4], (np.float32(3.0) * deq[:, 7]).astype(np.float32))


PF_ATTN_CASES = [  # seq, heads, kv heads, head_dim
    (1, 4, 2, 64), (5, 4, 2, 32), (16, 32, 8, 64), (17, 14, 2, 64), (100, 12, 2, 128), (70, 6, 1, 32),
    (512, 32, 8, 64), (300, 9, 3, 64), (200, 8, 1, 128), (77, 10, 2, 32),
    # enough query blocks for two 16-query subtiles per wave
    (1024, 32, 8, 64), (1024, 48, 8, 128),
    # few query blocks of 8+ key tiles: 1, 2 and 4 query heads per kv head (4, 2 and 1
    # 16-query subtiles per workgroup), rows not a multiple of 16, head sizes 32 / 128
    (256, 4, 4, 32), (400, 4, 2, 128), (333, 8, 2, 64), (260, 2, 2, 64),
]


def oracle_attn_prefill(q, k, v):
    seq, h, hd = q.shape
    g = k.shape[1]
    want = np.zeros_like(q)
    fp = C.POINTER(C.c_float)
    scores = np.zeros(seq + 1, np.float32)
    oracle_lib().orc_attn_prefill(want.ctypes.data_as(fp), q.ctypes.data_as(fp), k.ctypes.data_as(fp),
                                  v.ctypes.data_as(fp), seq, h, g, hd, scores.ctypes.data_as(fp))
    return want


@pytest.mark.parametrize("seq,h,g,hd", PF_ATTN_CASES)
def test_attn_prefill_matches_oracle(pkg, seq, h, g, hd):
    """Causal attention of a chunk over its own rows (attention.cpp:82-111) on fp16 MFMA
    with every operand an fp16 pair (22 bits) and an online softmax: within 1e-5 normwise
    of the oracle."""
    rng = np.random.default_rng(seq * 100 + h + hd)
    q = rng.standard_normal((seq, h, hd)).astype(np.float32)
    k = rng.standard_normal((seq, g, hd)).astype(np.float32)
    v = rng.standard_normal((seq, g, hd)).astype(np.float32)
    got = pkg.attn_prefill(q, k, v)
    want = oracle_attn_prefill(q, k, v)
    for i in range(seq):
        assert rel_err(got[i], want[i]) <= 1e-5, f"row {i}: {rel_err(got[i], want[i]):.3e}"


def test_attn_prefill_wide_value_range(pkg):
    """Rows of q and k scaled by powers of two over 2^-6 .. 2^1, rows of v over 2^-12 ..
    2^12, and a zero value row: the per-row scaling of the fp16 pairs keeps every head of
    every row within 1e-5 normwise of the oracle."""
    rng = np.random.default_rng(21)
    seq, h, g, hd = 150, 8, 2, 64
    q = rng.standard_normal((seq, h, hd)).astype(np.float32)
    k = rng.standard_normal((seq, g, hd)).astype(np.float32)
    v = rng.standard_normal((seq, g, hd)).astype(np.float32)
    q *= np.exp2(rng.integers(-6, 2, (seq, h, 1))).astype(np.float32)
    k *= np.exp2(rng.integers(-6, 2, (seq, g, 1))).astype(np.float32)
    v *= np.exp2(rng.integers(-12, 13, (seq, g, 1))).astype(np.float32)
    v[7] = 0.0
    got = pkg.attn_prefill(q, k, v)
    want = oracle_attn_prefill(q, k, v)
    for i in range(seq):
        for j in range(h):
            assert rel_err(got[i, j], want[i, j]) <= 1e-5, f"row {i} head {j}: {rel_err(got[i, j], want[i, j]):.3e}"


def test_attn_prefill_closed_forms(pkg):
    """Row 0 attends to itself only: its heads are v[0] of their kv head, to the 22 bits of
    the fp16 operand pair (its probability is a power of two, exact in fp16). With q = 0
    every score is 0 and row i is the mean of v[0..i]."""
    rng = np.random.default_rng(8)
    seq, h, g, hd = 40, 8, 2, 64
    q = rng.standard_normal((seq, h, hd)).astype(np.float32)
    k = rng.standard_normal((seq, g, hd)).astype(np.float32)
    v = rng.standard_normal((seq, g, hd)).astype(np.float32)
    got = pkg.attn_prefill(q, k, v)
    v0 = np.repeat(v[0], h // g, axis=0)
    assert np.max(np.abs(got[0] - v0) / np.abs(v0)) <= 2.0**-21
    got = pkg.attn_prefill(np.zeros_like(q), k, v)
    mean = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, seq + 1)[:, None, None]
    want = np.repeat(mean, h // g, axis=1)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(v))


@pytest.mark.parametrize("n", [32, 896, 2048, 8960])
def test_rmsnorm(pkg, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((4, n)) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    got = pkg.rmsnorm(x, w, 1e-5)
    L = oracle_lib()
    fp = C.POINTER(C.c_float)
    for i in range(4):
        want = np.zeros(n, np.float32)
        xi = np.ascontiguousarray(x[i])
        L.orc_rmsnorm(want.ctypes.data_as(fp), xi.ctypes.data_as(fp), w.ctypes.data_as(fp), n, 1e-5)
        # fp64 sum of squares in another order: at most one ulp of the scale
        assert rel_err(got[i], want) <= 2.5e-7


ROPE_CASES = [  # theta, head_dim, heads, rows, first position
    (500000.0, 64, 32, 6, 0), (1e6, 64, 14, 37, 100), (1e6, 128, 12, 5, 4091), (10000.0, 8, 4, 9, 0),
]


@pytest.mark.parametrize("theta,hd,heads,seq,pos0", ROPE_CASES)
def test_rope_bit_exact(pkg, theta, hd, heads, seq, pos0):
    """tf_hip_rope against the oracle's rope_one, position by position, bit for bit (the host
    tables hold the reference's own cos/sin values)."""
    rng = np.random.default_rng(hd * 7 + seq)
    x = (rng.standard_normal((seq, heads, hd)) * 2).astype(np.float32)
    cos_t, sin_t = pkg.rope_tables(theta, hd, pos0 + seq)
    got = pkg.rope(x, pos0, cos_t, sin_t)
    L = oracle_lib()
    fp = C.POINTER(C.c_float)
    freq = np.zeros(hd // 2, np.float32)
    L.orc_rope_freqs(freq.ctypes.data_as(fp), hd, theta, 0, 1.0, 1.0, 4.0, 8192.0)
    want = x.copy()
    for i in range(seq):
        row = np.ascontiguousarray(want[i])
        L.orc_rope(row.ctypes.data_as(fp), heads, hd, pos0 + i, freq.ctypes.data_as(fp))
        want[i] = row
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if pos0 == 0:
        assert np.array_equal(got[0], x[0])  # position 0 is the identity


def test_rope_rejects_rows_past_the_tables(pkg):
    cos_t, sin_t = pkg.rope_tables(10000.0, 8, 4)
    with pytest.raises(RuntimeError):
        pkg.rope(np.zeros((3, 2, 8), np.float32), 2, cos_t, sin_t)


ATTN_CASES = [  # heads, kv heads, head_dim, n_pos, max_seq
    (32, 8, 64, 1, 64), (32, 8, 64, 7, 64), (32, 8, 64, 38, 512), (32, 8, 64, 300, 512),
    (14, 2, 64, 144, 256), (12, 2, 128, 1000, 2048), (12, 2, 128, 4352, 8192), (4, 2, 8, 9, 16),
]


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("h,g,hd,n_pos,max_seq", ATTN_CASES)
def test_attn_decode(pkg, layout, h, g, hd, n_pos, max_seq):
    rng = np.random.default_rng(h * 1000 + n_pos)
    q = rng.standard_normal((h, hd)).astype(np.float32)
    k = rng.standard_normal((n_pos, g, hd)).astype(np.float32)
    v = rng.standard_normal((n_pos, g, hd)).astype(np.float32)
    got = pkg.attn_decode(q, k, v, max_seq, layout)
    # oracle over the same cache layout
    cache_k = np.zeros(g * max_seq * hd, np.float32)
    cache_v = np.zeros_like(cache_k)
    for p in range(n_pos):
        for j in range(g):
            o = (j * max_seq + p) * hd if layout else (p * g + j) * hd
            cache_k[o:o + hd] = k[p, j]
            cache_v[o:o + hd] = v[p, j]
    want = np.zeros((h, hd), np.float32)
    scores = np.zeros(max_seq + 1, np.float32)
    fp = C.POINTER(C.c_float)
    oracle_lib().orc_attn_decode(want.ctypes.data_as(fp), q.ctypes.data_as(fp), cache_k.ctypes.data_as(fp),
                                 cache_v.ctypes.data_as(fp), layout, g, max_seq, h, hd, n_pos,
                                 scores.ctypes.data_as(fp))
    assert rel_err(got, want) <= 1e-5


def test_attn_decode_single_position_returns_v(pkg):
    """n_pos = 1: softmax weight 1, the output head is its kv head's v (attention.cpp:55-80)."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((8, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 64)).astype(np.float32)
    got = pkg.attn_decode(q, k, v, 16, 0)
    assert np.array_equal(got, np.repeat(v[0], 4, axis=0))


def test_attn_decode_zero_query_is_mean_of_v(pkg):
    rng = np.random.default_rng(6)
    n_pos = 50
    q = np.zeros((4, 64), np.float32)
    k = rng.standard_normal((n_pos, 1, 64)).astype(np.float32)
    v = rng.standard_normal((n_pos, 1, 64)).astype(np.float32)
    got = pkg.attn_decode(q, k, v, 64, 1)
    assert rel_err(got[0], v[:, 0].mean(axis=0)) < 1e-5


def test_argmax_first_maximum(pkg):
    rng = np.random.default_rng(8)
    x = rng.standard_normal(151936).astype(np.float32)
    assert pkg.argmax(x) == int(np.argmax(x))
    x[[17, 90000, 151935]] = 50.0  # ties: the lowest index wins (sampler.cpp:8-13)
    assert pkg.argmax(x) == 17
    y = -np.abs(rng.standard_normal(1000).astype(np.float32)) - 1
    y[999] = -0.5
    assert pkg.argmax(y) == 999
    z = np.full(64, -0.0, np.float32)
    z[10] = 0.0  # -0 and +0 compare equal: the first one wins
    assert pkg.argmax(z) == 0


# MI355X reads 6.4-6.6 TB/s and copies at about 5 TB/s (read + write) beyond its 256 MB
# last-level cache: floors well under that, which a stream that skipped or re-read part of
# its buffer, or fell back to host code, would still have to reach while also giving the
# exact checksum.
READ_FLOOR_GBS = 4500.0
COPY_FLOOR_GBS = 3000.0


@pytest.mark.parametrize("nbytes", [1 << 30, (1 << 30) + 48])
def test_read_stream_reads_every_byte(pkg, nbytes):
    best, med, cs = pkg.read_stream(nbytes, iters=3, with_checksum=True)
    assert cs == pkg.stream_checksum(nbytes)
    assert best >= READ_FLOOR_GBS and med > 0, (best, med)


def test_copy_stream_copies_every_byte(pkg):
    nbytes = 1 << 30
    best, med, cs = pkg.copy_stream(nbytes, iters=3, with_checksum=True)
    assert cs == pkg.stream_checksum(nbytes)
    assert best >= COPY_FLOOR_GBS and med > 0, (best, med)
