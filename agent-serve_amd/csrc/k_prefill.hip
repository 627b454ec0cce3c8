// Prefill of prompt tokens on the matrix cores: Model::prefill and layer_prefill
// (model.cpp:144-195) for a chunk of M tokens at once.
//
// k_pf_pack_q8   a Q8_0 matrix's integers as fp16 in MFMA fragment order, once per matrix
// k_pf_split     rmsnorm (layers.cpp:7-12) of each row, or the row as it is, scaled by
//                a power of two and written as fp16 hi + lo in fragment order (the A operand)
// k_pf_gemm_q8   matmul (matmul.cpp:64-73) of Q8_0 weights on v_mfma_f32_16x16x32_f16,
//                epilogues: store (+ F32 bias, model.cpp:85-89), residual add
//                (add_inplace, layers.cpp:21-23), silu(gate) * up (layers.cpp:14-19)
// k_pf_rope_store apply_rope_many of q and k (attention.cpp:48-53) and KVCache::store
//                (kvcache.cpp:31-36) of every row
// k_pf_attn      causal GQA attention of the chunk (attn_prefill, attention.cpp:82-111)
//                on v_mfma_f32_16x16x4_f32 with an online softmax
//
// Numerics. A Q8_0 weight q is an integer in [-128, 127] and exact in fp16; a
// 32-element block's products with the fp16 pair (hi, lo) of an activation are exact
// in the fp32 accumulator, and hi + lo carries 22 significant bits of the fp32
// activation (24). Each block's two MFMAs start from zero and the block sum is scaled
// by its fp16 d in fp32 (quant.cpp:266-321 scales block sums the same way), so the
// result differs from the fp32 reference by summation order and the 2^-22 split, both
// far inside the 1e-3 parity bound. Scaling rows by 2^e (max |x| in [2^14, 2^15))
// keeps hi and lo in fp16 range and off its subnormals; the epilogue multiplies the
// exact inverse back.
#include "dev_common.hpp"
#include "tf_internal.hpp"

namespace tfk {

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- operands in MFMA fragment order
//
// v_mfma_f32_16x16x32_f16 takes from lane l the 8 halves (row l % 16, k = 8 (l / 16) + j)
// of a 16 x 32 operand tile. Both operands are stored so that one tile is 64 lanes x 16
// bytes, contiguous: a wave fills a fragment with one coalesced 1 KiB load.
//   activations: xa[row tile][block][hi, lo][lane][8]   (k_pf_split)
//   weights:     wf[row tile][block][lane][8]            (k_pf_pack_q8, once per matrix)

// Eight int8 bytes q -> their fp16 values: with u = q + 128 (the byte with its top bit
// flipped), 0x64UU is the half 1024 + u, and 1024 + u - 1152 = q exactly.
__device__ __forceinline__ h8_t q8_to_h8(uint2 w) {
    w.x ^= 0x80808080u;
    w.y ^= 0x80808080u;
    const uint32_t p0 = (w.x & 0xFFu) | ((w.x & 0xFF00u) << 8) | 0x64006400u;
    const uint32_t p1 = ((w.x >> 16) & 0xFFu) | ((w.x >> 8) & 0xFF0000u) | 0x64006400u;
    const uint32_t p2 = (w.y & 0xFFu) | ((w.y & 0xFF00u) << 8) | 0x64006400u;
    const uint32_t p3 = ((w.y >> 16) & 0xFFu) | ((w.y >> 8) & 0xFF0000u) | 0x64006400u;
    const tf_u32x4 p = {p0, p1, p2, p3};
    const h8_t off = {1152, 1152, 1152, 1152, 1152, 1152, 1152, 1152};
    return __builtin_bit_cast(h8_t, p) - off;
}

// Q8_0 matrix (DevMat q stream, N x K) -> its integers q as fp16 in fragment order.
__global__ __launch_bounds__(kBlock) void k_pf_pack_q8(const uint8_t* q, int K, int64_t N, h8_t* wf) {
    const int nblk = K / 32;
    const int64_t total = N / 16 * nblk * 64;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
        const int l = (int)(i & 63);
        const int64_t tb = i >> 6;
        const int b = (int)(tb % nblk);
        const int64_t t = tb / nblk;
        wf[i] = q8_to_h8(*(const uint2*)(q + (16 * t + (l & 15)) * (int64_t)K + 32 * b + 8 * (l >> 4)));
    }
}

constexpr int kSplitGroups = 8;  // 8-element groups per thread: rows up to 256 * 8 * 8 = 16384

// One workgroup per row, the row held in registers (thread t owns the 8-element groups
// t, t + 256, ...): the rmsnorm scale inv (when w is given), a power of two sc putting
// max |row| in [2^14, 2^15) (rs = 1 / sc), then every element as hi + lo into the
// fragment layout (16 bytes of a hi and of a lo fragment per group). Rows M.. are zeros
// with rs = 0.
__global__ __launch_bounds__(kBlock) void k_pf_split(const float* x, int64_t ldx, const float* w, float eps, int K,
                                                     int M, h8_t* xa, float* rs) {
    __shared__ double red_d[kWavesPerBlock];
    __shared__ float red_f[kWavesPerBlock];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int ng = K / 8, nblk = K / 32;
    h8_t* tile = xa + (int64_t)(m / 16) * nblk * 128 + (m % 16);
    if (m >= M) {
        const h8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = tid; j < ng; j += kBlock) {
            h8_t* o = tile + (j / 4) * 128 + 16 * (j % 4);
            o[0] = z;
            o[64] = z;
        }
        if (tid == 0) rs[m] = 0.0f;
        return;
    }
    const float4* xr = (const float4*)(x + (int64_t)m * ldx);
    const float4* wr = (const float4*)w;
    float v[kSplitGroups][8];
#pragma unroll
    for (int i = 0; i < kSplitGroups; ++i) {
        const int j = tid + i * kBlock;
        const int jj = j < ng ? j : ng - 1;  // a clamped re-read, masked below
        const float4 a = xr[2 * jj], b = xr[2 * jj + 1];
        v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
        v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
    }
    float inv = 1.0f;
    if (w) {
        double ss = 0;
#pragma unroll
        for (int i = 0; i < kSplitGroups; ++i)
            if (tid + i * kBlock < ng)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += (double)v[i][e] * v[i][e];
        ss = wave_sum_d(ss);
        if ((tid & 63) == 0) red_d[tid >> 6] = ss;
        __syncthreads();
        ss = (red_d[0] + red_d[1]) + (red_d[2] + red_d[3]);
        inv = 1.0f / sqrtf((float)(ss / K) + eps);
#pragma unroll
        for (int i = 0; i < kSplitGroups; ++i) {
            int j = tid + i * kBlock;
            j = j < ng ? j : ng - 1;
            const float4 a = wr[2 * j], b = wr[2 * j + 1];
            const float g[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[i][e] = v[i][e] * inv * g[e];
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kSplitGroups; ++i)
        if (tid + i * kBlock < ng)
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
    amax = wave_max(amax);
    if ((tid & 63) == 0) red_f[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    int ex = 0;
    (void)frexpf(amax, &ex);  // amax = f 2^ex, f in [0.5, 1)
    int e2 = amax > 0.0f ? 15 - ex : 0;
    e2 = e2 < -100 ? -100 : (e2 > 100 ? 100 : e2);
    const float sc = ldexpf(1.0f, e2);
    if (tid == 0) rs[m] = ldexpf(1.0f, -e2);
#pragma unroll
    for (int i = 0; i < kSplitGroups; ++i) {
        const int j = tid + i * kBlock;
        if (j < ng) {
            h8_t hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float t = v[i][e] * sc;
                hi[e] = (_Float16)t;
                lo[e] = (_Float16)(t - (float)hi[e]);
            }
            h8_t* o = tile + (j / 4) * 128 + 16 * (j % 4);
            o[0] = hi;
            o[64] = lo;
        }
    }
}

// ---------------------------------------------------------------- Q8_0 GEMM

// Field of the segment holding output subtile u (uniform per wave: scalar selects).
#define PF_SEL(s, f) ((s) == 0 ? a.seg[0].f : ((s) == 1 ? a.seg[1].f : a.seg[2].f))

// Workgroup: 4 waves as 2 (rows) x 2 (columns); a wave owns 32 rows x NI column subtiles
// of 16 (GEMV_SILU: NI / 2 output subtiles, each a gate and an up subtile). Per 32-element
// block: for each (row subtile, column subtile) an MFMA of the hi part from zero, then
// one of the lo part on top (issued after all eight hi MFMAs, so no MFMA waits on the
// one before it), then acc += d * block sum. Fragments stream from L2 into registers,
// one stage of two blocks ahead; every load is unconditional (indices clamped) so the
// compiler waits only for the stage it consumes.
template <int MODE, int NI>
__global__ __launch_bounds__(256) void k_pf_gemm_q8(const PfGemmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // XCD-aware order: workgroup b runs on XCD b % 8; give each XCD a contiguous range
    // of tiles, rows fastest, so the row tiles that share a weight tile share an L2.
    int b = blockIdx.x;
    {
        const int q = (int)gridDim.x / 8;
        if (b < 8 * q) b = (b % 8) * q + b / 8;
    }
    const int MT = a.Mpad / kPfTileM;
    const int mt = b % MT, nt = b / MT;
    const int m0 = mt * kPfTileM + (wave & 1) * 32;
    const int wid = nt * 2 + (wave >> 1);
    const int K = a.K, nblk = K / 32;
    const int l16 = lane & 15;

    constexpr int NO = MODE == GEMV_SILU ? NI / 2 : NI;  // output subtiles per wave
    const TF_GLOBAL h8_t* bp[NI];
    const uint16_t* sp[NI];
    float* yp[NI];
    const float* bsp[NI];
    int64_t ldy[NI];
    int col[NI];
    bool ok[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
        int u = wid * NO + ni % NO;
        ok[ni] = u < a.n_sub;
        u = u < a.n_sub ? u : a.n_sub - 1;
        const int s = (a.n_seg > 2 && u >= a.seg[2].sub0) ? 2 : ((a.n_seg > 1 && u >= a.seg[1].sub0) ? 1 : 0);
        const int tile = u - PF_SEL(s, sub0);
        const int c = tile * 16 + l16;
        const bool up = MODE == GEMV_SILU && ni >= NO;
        const uint16_t* wf = up ? PF_SEL(s, wf2) : PF_SEL(s, wf);
        const uint8_t* ws = up ? PF_SEL(s, w2.s) : PF_SEL(s, w.s);
        bp[ni] = (const TF_GLOBAL h8_t*)wf + (int64_t)tile * nblk * 64 + lane;
        sp[ni] = (const uint16_t*)ws + (int64_t)c * nblk;
        yp[ni] = PF_SEL(s, y);
        bsp[ni] = PF_SEL(s, bias);
        ldy[ni] = PF_SEL(s, ldy);
        col[ni] = c;
    }
    const TF_GLOBAL h8_t* ap[2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) ap[mi] = (const TF_GLOBAL h8_t*)a.xa + (int64_t)(m0 / 16 + mi) * nblk * 128 + lane;

    f4_t acc[2][NI];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};

    struct Stage {
        h8_t ah[2][2], al[2][2];  // [row subtile][block]
        h8_t bh[NI][2];           // [column subtile][block]
        uint32_t d[NI];           // the two blocks' fp16 scales
    };
    const int S = K / 64;
    auto load = [&](int s, Stage& g) {
        s = s < S ? s : S - 1;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int blk = 2 * s + j;
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                g.ah[mi][j] = ap[mi][blk * 128];
                g.al[mi][j] = ap[mi][blk * 128 + 64];
            }
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) g.bh[ni][j] = bp[ni][blk * 64];
        }
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) g.d[ni] = *(const TF_GLOBAL uint32_t*)(sp[ni] + 2 * s);
    };
    auto compute = [&](const Stage& g) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f4_t t[2][NI];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
                    t[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(g.ah[mi][j], g.bh[ni][j],
                                                                      (f4_t){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
                    t[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(g.al[mi][j], g.bh[ni][j], t[mi][ni], 0, 0, 0);
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) {
                const float dv = h2f(g.d[ni] >> (16 * j));
#pragma unroll
                for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[mi][ni][r] = fmaf(dv, t[mi][ni][r], acc[mi][ni][r]);
            }
        }
    };
    Stage s0, s1;
    load(0, s0);
    int s = 0;
    for (; s + 2 <= S; s += 2) {
        load(s + 1, s1);
        compute(s0);
        load(s + 2, s0);
        compute(s1);
    }
    if (s < S) compute(s0);

    // epilogue: lane holds rows m0 + 16 mi + 4 (lane / 16) + r of column col[ni]
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
        const int r0 = m0 + 16 * mi + 4 * (lane >> 4);
        const float4 rsv = *(const float4*)(a.rs + r0);
        const float rsa[4] = {rsv.x, rsv.y, rsv.z, rsv.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = r0 + r;
            if (row >= a.M) continue;
            if (MODE == GEMV_SILU) {
#pragma unroll
                for (int j = 0; j < NO; ++j) {
                    if (!ok[j]) continue;
                    const float gv = acc[mi][j][r] * rsa[r];
                    const float uv = acc[mi][j + NO][r] * rsa[r];
                    yp[j][(int64_t)row * ldy[j] + col[j]] = (gv / (1.0f + expf(-gv))) * uv;
                }
            } else {
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) {
                    if (!ok[ni]) continue;
                    const float v = acc[mi][ni][r] * rsa[r];
                    float* p = yp[ni] + (int64_t)row * ldy[ni] + col[ni];
                    if (MODE == GEMV_STORE) {
                        *p = bsp[ni] ? v + bsp[ni][col[ni]] : v;
                    } else {
                        const float nv = *p + v;
                        *p = nv;
                        if (row == a.tap_row && a.tap) a.tap[col[ni]] = nv;
                    }
                }
            }
        }
    }
}

// Large tiles for GEMMs with enough of them to fill the CUs: a workgroup of 8 waves
// (2 rows x 4 columns of waves) owns 128 rows x 16 weight-column subtiles (256 weight rows;
// GEMV_SILU: 8 gate and the 8 matching up subtiles, 128 output columns). A stage (two
// 32-element blocks) of both operands and the scales is staged in LDS, loaded once per
// workgroup (8 fragments per wave) through registers one stage ahead of its use; each wave
// then runs 4 x 4 tiles of 16 x 16 per block, reading its fragments from LDS. The per-block
// arithmetic and its order are those of k_pf_gemm_q8, so the two give the same bits.
constexpr int kBigThreads = 512;
constexpr int kBigRows = 128;
constexpr int kBigStageH8 = 64 * 64;  // h8 per stage: 32 A fragments + 32 B fragments of 64 lanes
constexpr int kBigStageBytes = kBigStageH8 * 16 + 256 * 4;
constexpr size_t kBigLdsBytes = 2 * (size_t)kBigStageBytes;

// SPLIT: the grid also splits K into a.ks slices; slice ks writes its row-scaled partial
// sums to a.part[ks][row][output column] and k_pf_reduce applies the epilogue.
template <int MODE, bool SPLIT>
__global__ __launch_bounds__(kBigThreads) void k_pf_gemm_big(const PfGemmArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int b = blockIdx.x;
    {
        const int q = (int)gridDim.x / 8;
        if (b < 8 * q) b = (b % 8) * q + b / 8;
    }
    const int kslice = SPLIT ? b % a.ks : 0;
    if (SPLIT) b /= a.ks;
    const int MT = a.Mpad / kBigRows;
    const int mt = b % MT, nt = b / MT;
    const int K = a.K, nblk = K / 32;
    const int S = SPLIT ? K / 64 / a.ks : K / 64;  // stages of this slice
    const int s0 = kslice * S;                      // its first stage
    const int l16 = lane & 15;
    constexpr bool SILU = MODE == GEMV_SILU;

    // weight-column subtile q (0..15) of this workgroup: output subtile, matrix, tile row
    auto resolve = [&](int q, int& u, int& seg, bool& up) {
        up = SILU && q >= 8;
        u = SILU ? nt * 8 + (q & 7) : nt * 16 + q;
        u = u < a.n_sub ? u : a.n_sub - 1;
        seg = (a.n_seg > 2 && u >= a.seg[2].sub0) ? 2 : ((a.n_seg > 1 && u >= a.seg[1].sub0) ? 1 : 0);
    };
    // this wave's 8 fragment loads per stage: i < 4 A fragments, i >= 4 B fragments
    const TF_GLOBAL h8_t* src[8];
    int step[8];  // h8 per stage
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int f = wave + 8 * i;
        if (i < 4) {
            const int T = f / 4, blk = (f / 2) % 2, hl = f % 2;
            src[i] = (const TF_GLOBAL h8_t*)a.xa + ((int64_t)(mt * 8 + T) * nblk + blk) * 128 + hl * 64 + lane;
            step[i] = 256;
        } else {
            const int g = f - 32, q = g / 2, blk = g % 2;
            int u, seg;
            bool up;
            resolve(q, u, seg, up);
            const int tile = u - PF_SEL(seg, sub0);
            const uint16_t* wf = up ? PF_SEL(seg, wf2) : PF_SEL(seg, wf);
            src[i] = (const TF_GLOBAL h8_t*)wf + ((int64_t)tile * nblk + blk) * 64 + lane;
            step[i] = 128;
        }
    }
    // the scales: thread t (mod 256) loads column j = t of the 256 weight columns
    const uint16_t* dsrc;
    {
        const int j = tid & 255, q = j / 16;
        int u, seg;
        bool up;
        resolve(q, u, seg, up);
        const int c = (u - PF_SEL(seg, sub0)) * 16 + (j & 15);
        const uint8_t* ws = up ? PF_SEL(seg, w2.s) : PF_SEL(seg, w.s);
        dsrc = (const uint16_t*)ws + (int64_t)c * nblk;
    }
    h8_t stg[8];
    uint32_t dstg;
    auto gload = [&](int s) {
        s = s0 + (s < S ? s : S - 1);
#pragma unroll
        for (int i = 0; i < 8; ++i) stg[i] = src[i][(int64_t)s * step[i]];
        dstg = *(const TF_GLOBAL uint32_t*)(dsrc + 2 * s);
    };
    auto lds_write = [&](int buf) {
        h8_t* st = (h8_t*)(lds + buf * kBigStageBytes);
#pragma unroll
        for (int i = 0; i < 8; ++i) st[(wave + 8 * i) * 64 + lane] = stg[i];
        ((uint32_t*)(lds + buf * kBigStageBytes + kBigStageH8 * 16))[tid & 255] = dstg;
    };
    auto barrier = [&]() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    const int wm = wave & 1, wn = wave >> 1;
    int qb[4];  // this wave's weight-column subtiles
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) qb[ni] = SILU ? (ni < 2 ? wn * 2 + ni : 8 + wn * 2 + ni - 2) : wn * 4 + ni;

    f4_t acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int buf) {
        const h8_t* st = (const h8_t*)(lds + buf * kBigStageBytes);
        const uint32_t* sd = (const uint32_t*)(lds + buf * kBigStageBytes + kBigStageH8 * 16);
        uint32_t dd[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) dd[ni] = sd[qb[ni] * 16 + l16];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            h8_t bh[4];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) bh[ni] = st[(32 + qb[ni] * 2 + j) * 64 + lane];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                h8_t ah[2], al[2];
#pragma unroll
                for (int mm = 0; mm < 2; ++mm) {
                    const int T = wm * 4 + half * 2 + mm;
                    ah[mm] = st[((T * 2 + j) * 2 + 0) * 64 + lane];
                    al[mm] = st[((T * 2 + j) * 2 + 1) * 64 + lane];
                }
                f4_t t[2][4];
#pragma unroll
                for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni)
                        t[mm][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mm], bh[ni],
                                                                          (f4_t){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni)
                        t[mm][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mm], bh[ni], t[mm][ni], 0, 0, 0);
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const float dv = h2f(dd[ni] >> (16 * j));
#pragma unroll
                    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            acc[half * 2 + mm][ni][r] = fmaf(dv, t[mm][ni][r], acc[half * 2 + mm][ni][r]);
                }
            }
        }
    };

    gload(0);
    lds_write(0);
    gload(1);
    barrier();
    for (int s = 0; s < S; ++s) {
        compute(s & 1);
        lds_write((s + 1) & 1);  // stage s + 1 (the buffer of stage s - 1, read before the last barrier)
        gload(s + 2);
        barrier();
    }

    // epilogue: lane holds rows 16 T + 4 (lane / 16) + r of weight column 16 q + l16
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        const int r0 = mt * kBigRows + (wm * 4 + mi) * 16 + 4 * (lane >> 4);
        const float4 rsv = *(const float4*)(a.rs + r0);
        const float rsa[4] = {rsv.x, rsv.y, rsv.z, rsv.w};
#pragma unroll
        for (int ni = 0; ni < (SILU ? 2 : 4); ++ni) {
            int u, seg;
            bool up;
            const int uraw = SILU ? nt * 8 + (qb[ni] & 7) : nt * 16 + qb[ni];
            resolve(qb[ni], u, seg, up);
            if (uraw >= a.n_sub) continue;
            if (SPLIT) {
                const int ntot = a.n_sub * 16;
                float* part = a.part + ((int64_t)kslice * a.Mpad) * ntot + u * 16 + l16;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (r0 + r < a.M) part[(int64_t)(r0 + r) * ntot] = acc[mi][ni][r] * rsa[r];
                continue;
            }
            const int c = (u - PF_SEL(seg, sub0)) * 16 + l16;
            float* y = PF_SEL(seg, y);
            const int64_t ldy = PF_SEL(seg, ldy);
            const float* bias = PF_SEL(seg, bias);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = r0 + r;
                if (row >= a.M) continue;
                float* p = y + (int64_t)row * ldy + c;
                if (SILU) {
                    const float gv = acc[mi][ni][r] * rsa[r];
                    const float uv = acc[mi][ni + 2][r] * rsa[r];
                    *p = (gv / (1.0f + expf(-gv))) * uv;
                } else if (MODE == GEMV_STORE) {
                    const float v = acc[mi][ni][r] * rsa[r];
                    *p = bias ? v + bias[c] : v;
                } else {
                    const float nv = *p + acc[mi][ni][r] * rsa[r];
                    *p = nv;
                    if (row == a.tap_row && a.tap) a.tap[c] = nv;
                }
            }
        }
    }
}

// Sums the a.ks partial rows of a split-K GEMM in slice order and applies the epilogue:
// thread per output column of row blockIdx.y.
template <int MODE>
__global__ __launch_bounds__(kBlock) void k_pf_reduce(const PfGemmArgs a) {
    const int row = blockIdx.y;
    const int col = blockIdx.x * kBlock + threadIdx.x;
    const int ntot = a.n_sub * 16;
    if (col >= ntot) return;
    const float* p = a.part + (int64_t)row * ntot + col;
    float v = 0.0f;
    for (int k = 0; k < a.ks; ++k) v += p[(int64_t)k * a.Mpad * ntot];
    const int u = col / 16;
    const int seg = (a.n_seg > 2 && u >= a.seg[2].sub0) ? 2 : ((a.n_seg > 1 && u >= a.seg[1].sub0) ? 1 : 0);
    const int c = col - PF_SEL(seg, sub0) * 16;
    float* y = PF_SEL(seg, y) + (int64_t)row * PF_SEL(seg, ldy) + c;
    if (MODE == GEMV_STORE) {
        const float* bias = PF_SEL(seg, bias);
        *y = bias ? v + bias[c] : v;
    } else {
        const float nv = *y + v;
        *y = nv;
        if (row == a.tap_row && a.tap) a.tap[c] = nv;
    }
}

#undef PF_SEL

// ---------------------------------------------------------------- RoPE and KV store

// Row i is position pos0 + i: q heads rotated in place, k heads rotated into the cache,
// v heads copied into it (the same fmaf pattern as the decode path).
__global__ __launch_bounds__(kBlock) void k_pf_rope_store(float* qkv, int64_t ld, int H, int G, int hd,
                                                          const float* rope_cos, const float* rope_sin, int pos0,
                                                          float* kc, float* vc, int layout, int max_seq) {
    const int i = blockIdx.x, pos = pos0 + i, d2 = hd / 2;
    float* q = qkv + (int64_t)i * ld;
    const float* k = q + (int64_t)H * hd;
    const float* v = k + (int64_t)G * hd;
    const float* cs = rope_cos + (int64_t)pos * d2;
    const float* sn = rope_sin + (int64_t)pos * d2;
    for (int t = threadIdx.x; t < H * d2; t += kBlock) {
        const int h = t / d2, j = t % d2;
        float* qh = q + (int64_t)h * hd;
        const float x0 = qh[j], x1 = qh[j + d2], c = cs[j], s = sn[j];
        qh[j] = fmaf(x0, c, -(x1 * s));
        qh[j + d2] = fmaf(x0, s, x1 * c);
    }
    for (int t = threadIdx.x; t < G * d2; t += kBlock) {
        const int g = t / d2, j = t % d2;
        const float* kh = k + (int64_t)g * hd;
        const float x0 = kh[j], x1 = kh[j + d2], c = cs[j], s = sn[j];
        float* o = kc + kv_offset(layout, G, max_seq, hd, g, pos);
        o[j] = fmaf(x0, c, -(x1 * s));
        o[j + d2] = fmaf(x0, s, x1 * c);
    }
    for (int t = threadIdx.x; t < G * hd; t += kBlock) {
        const int g = t / hd, j = t % hd;
        vc[kv_offset(layout, G, max_seq, hd, g, pos) + j] = v[(int64_t)g * hd + j];
    }
}

// ---------------------------------------------------------------- causal attention

// Workgroup: 16 consecutive queries of one kv head, one wave per query head of the
// group. Per tile of 16 keys a wave computes S^T = K Q^T with HD/4 MFMAs (lane group
// l/16 holds HD/4 consecutive dims of its key row and its query row), so a lane ends up
// with 4 keys of query l%16; the softmax statistics of a query combine the 4 lanes
// l%16 + 16 j. O^T = V^T P^T then takes P^T straight from those registers: MFMA r of a
// tile feeds key 4 (l/16) + r, and V^T as one scalar per lane. Keys run from att_start to
// the last query of the tile; keys past a query's position score -inf.
template <int HD>
__global__ __launch_bounds__(512) void k_pf_attn(const float* q, int64_t ldq, const float* kc, const float* vc,
                                                 int layout, int G, int max_seq, int n_rep, int n, int pos0,
                                                 int att_start, float* out, int64_t ldo) {
    constexpr int DQ = HD / 4;   // dims per lane group in S^T
    constexpr int NT = HD / 16;  // output dim tiles
    const int lane = threadIdx.x & 63, r_head = threadIdx.x >> 6;
    const int qt = (int)gridDim.x - 1 - (int)blockIdx.x;  // longest tiles first
    const int g = blockIdx.y;
    const int h = g * n_rep + r_head;
    const int l16 = lane & 15, grp = lane >> 4;
    const int qi = qt * 16 + l16;
    const int qrow = qi < n ? qi : n - 1;
    const int qpos = pos0 + qrow;
    const int last = qt * 16 + 15 < n ? qt * 16 + 15 : n - 1;
    const int k_hi = pos0 + last;  // last key any query of the tile sees
    const float scale = 1.0f / sqrtf((float)HD);

    float qv[DQ];
    {
        const float* qr = q + (int64_t)qrow * ldq + (int64_t)h * HD + grp * DQ;
#pragma unroll
        for (int s = 0; s < DQ; s += 4) {
            const float4 t = gload_f4(qr + s);
            qv[s] = t.x;
            qv[s + 1] = t.y;
            qv[s + 2] = t.z;
            qv[s + 3] = t.w;
        }
    }
    f4_t ot[NT];
#pragma unroll
    for (int d = 0; d < NT; ++d) ot[d] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    // K rows (lane's key kt + l16, dims grp*DQ ..) and V scalars (MFMA r of dim tile d
    // needs V[kt + 4 grp + r][16 d + l16]) of the tile at kt; keys past k_hi re-read key
    // k_hi (masked). The next tile's loads are issued before the current tile's MFMAs.
    auto load_kv = [&](int kt, float (&kv_)[DQ], float (&vv_)[4][NT]) {
        int key = kt + l16;
        key = key <= k_hi ? key : k_hi;
        const float* kr = kc + kv_offset(layout, G, max_seq, HD, g, key) + grp * DQ;
#pragma unroll
        for (int s = 0; s < DQ; s += 4) {
            const float4 t = gload_f4(kr + s);
            kv_[s] = t.x;
            kv_[s + 1] = t.y;
            kv_[s + 2] = t.z;
            kv_[s + 3] = t.w;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int vkey = kt + 4 * grp + r;
            vkey = vkey <= k_hi ? vkey : k_hi;
            const float* vr = vc + kv_offset(layout, G, max_seq, HD, g, vkey) + l16;
#pragma unroll
            for (int d = 0; d < NT; ++d) vv_[r][d] = *gptr(vr + 16 * d);
        }
    };
    auto tile = [&](int kt, const float (&kv_)[DQ], const float (&vv_)[4][NT]) {
        f4_t st = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < DQ; ++s) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kv_[s], qv[s], st, 0, 0, 0);
        float p[4];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = kt + 4 * grp + r;
            p[r] = key <= qpos ? st[r] * scale : -INFINITY;
            mt = fmaxf(mt, p[r]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);
        const float alpha = expf(m_run - m_new);  // 0 on the first tile
        float ls = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = p[r] == -INFINITY ? 0.0f : expf(p[r] - m_new);
            ls += p[r];
        }
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        l_run = fmaf(l_run, alpha, ls);
        m_run = m_new;
#pragma unroll
        for (int d = 0; d < NT; ++d) {
            f4_t o = ot[d] * alpha;
#pragma unroll
            for (int r = 0; r < 4; ++r) o = __builtin_amdgcn_mfma_f32_16x16x4f32(vv_[r][d], p[r], o, 0, 0, 0);
            ot[d] = o;
        }
    };
    float kva[DQ], vva[4][NT], kvb[DQ], vvb[4][NT];
    load_kv(att_start, kva, vva);
    for (int kt = att_start; kt <= k_hi;) {
        load_kv(kt + 16, kvb, vvb);
        tile(kt, kva, vva);
        kt += 16;
        if (kt > k_hi) break;
        load_kv(kt + 16, kva, vva);
        tile(kt, kvb, vvb);
        kt += 16;
    }
    // lane holds O[query l16][dims 16 d + 4 grp + 0..3]; the 4 lanes of a query share l_run
    if (qi < n) {
        float* orow = out + (int64_t)qi * ldo + (int64_t)h * HD + 4 * grp;
        const float il = 1.0f / l_run;
#pragma unroll
        for (int d = 0; d < NT; ++d)
            *(float4*)(orow + 16 * d) = make_float4(ot[d][0] * il, ot[d][1] * il, ot[d][2] * il, ot[d][3] * il);
    }
}

// The last prompt row becomes the decode input of the lm_head GEMV; the control block
// then describes position pos_last, as after a decode step of that token.
__global__ __launch_bounds__(kBlock) void k_pf_tail(Ctl* ctl, int pos_last, const int32_t* hist, const float* xrow,
                                                    float* x, int D) {
    for (int i = threadIdx.x; i < D; i += kBlock) x[i] = xrow[i];
    if (threadIdx.x == 0) {
        ctl->pos = pos_last;
        ctl->key = 0ull;
        ctl->last_token = hist[pos_last];
    }
}

}  // namespace

bool pf_gemm_supported(int type, int64_t K, int64_t N) {
    return type == TF_HIP_TYPE_Q8_0 && K % 64 == 0 && N % 16 == 0 && K <= kBlock * 8 * kSplitGroups;
}

hipError_t launch_pf_split(const float* x, int64_t ldx, const float* norm_w, float eps, int K, int M, int Mpad,
                           uint16_t* xa, float* rs, hipStream_t st) {
    if (K % 32 != 0 || K > kBlock * 8 * kSplitGroups || ldx % 4 != 0 || Mpad % kPfTileM != 0 || M > Mpad)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_split, dim3(Mpad), dim3(kBlock), 0, st, x, ldx, norm_w, eps, K, M, (h8_t*)xa, rs);
    return hipGetLastError();
}

hipError_t launch_pf_pack_q8(const DevMat& m, uint16_t* wf, hipStream_t st) {
    if (m.type != TF_HIP_TYPE_Q8_0 || m.K % 32 != 0 || m.N % 16 != 0) return hipErrorInvalidValue;
    const int64_t total = m.N / 16 * (m.K / 32) * 64;
    int64_t blocks = (total + kBlock - 1) / kBlock;
    blocks = blocks < 4096 ? blocks : 4096;
    hipLaunchKernelGGL(k_pf_pack_q8, dim3((unsigned)blocks), dim3(kBlock), 0, st, m.q, (int)m.K, m.N, (h8_t*)wf);
    return hipGetLastError();
}

hipError_t launch_pf_gemm(const PfGemmArgs& a, hipStream_t st) {
    if (a.K % 64 != 0 || a.Mpad % kPfTileM != 0 || a.M > a.Mpad || a.M <= 0 || a.n_sub <= 0 || a.n_seg < 1 ||
        a.n_seg > 3)
        return hipErrorInvalidValue;
    for (int s = 0; s < a.n_seg; ++s) {
        const PfSeg& g = a.seg[s];
        if (g.w.type != TF_HIP_TYPE_Q8_0 || g.w.K != a.K || g.w.N % 16 != 0 || !g.y || !g.wf)
            return hipErrorInvalidValue;
        const int next = s + 1 < a.n_seg ? a.seg[s + 1].sub0 : a.n_sub;
        if (next - g.sub0 != g.w.N / 16) return hipErrorInvalidValue;
        if (a.mode == GEMV_SILU && (g.w2.type != TF_HIP_TYPE_Q8_0 || g.w2.K != a.K || g.w2.N != g.w.N || !g.wf2))
            return hipErrorInvalidValue;
    }
    if (a.seg[0].sub0 != 0 || (a.mode == GEMV_SILU && a.n_seg != 1)) return hipErrorInvalidValue;
    // large tiles when they give every CU a workgroup, directly or with K split in slices
    if (a.Mpad % kBigRows == 0) {
        const int per_big = a.mode == GEMV_SILU ? 8 : 16;  // output subtiles per large tile
        const int n_big = (a.n_sub + per_big - 1) / per_big * (a.Mpad / kBigRows);
        const int cus = device_cu_count();
        int ks = 1;
        if (n_big < cus && a.mode != GEMV_SILU && a.part) {
            // the fewest slices that fill the CUs, each at least 8 stages long (shorter
            // slices spend more on filling their pipeline and on the partial rows they
            // write than they save); worth it from half the CUs on
            const int S = a.K / 64;
            const size_t per_slice = (size_t)a.Mpad * a.n_sub * 16;
            for (int k = 2; k <= 16; k *= 2) {
                if (S % k != 0 || S / k < 8 || (size_t)k * per_slice > a.part_floats) break;
                ks = k;
                if (n_big * k >= cus) break;
            }
            if (2 * n_big * ks < cus) ks = 1;
        }
        if (n_big >= cus || ks > 1) {
            static bool attr_set[6] = {false, false, false, false, false, false};
            const void* fns[6] = {(const void*)k_pf_gemm_big<GEMV_STORE, false>,
                                  (const void*)k_pf_gemm_big<GEMV_RESID, false>,
                                  (const void*)k_pf_gemm_big<GEMV_SILU, false>,
                                  (const void*)k_pf_gemm_big<GEMV_STORE, true>,
                                  (const void*)k_pf_gemm_big<GEMV_RESID, true>,
                                  (const void*)k_pf_gemm_big<GEMV_SILU, true>};
            const int fi = a.mode + (ks > 1 ? 3 : 0);
            if (!attr_set[fi]) {
                const hipError_t e =
                    hipFuncSetAttribute(fns[fi], hipFuncAttributeMaxDynamicSharedMemorySize, (int)kBigLdsBytes);
                if (e != hipSuccess) return e;
                attr_set[fi] = true;
            }
            PfGemmArgs b = a;
            b.ks = ks;
            const dim3 grid((unsigned)(n_big * ks));
            switch (fi) {
                case 0: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_STORE, false>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                case 1: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_RESID, false>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                case 2: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_SILU, false>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                case 3: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_STORE, true>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                default: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_RESID, true>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
            }
            hipError_t e = hipGetLastError();
            if (e != hipSuccess || ks == 1) return e;
            const dim3 rgrid((unsigned)((a.n_sub * 16 + kBlock - 1) / kBlock), (unsigned)a.M);
            if (a.mode == GEMV_STORE)
                hipLaunchKernelGGL(k_pf_reduce<GEMV_STORE>, rgrid, dim3(kBlock), 0, st, b);
            else
                hipLaunchKernelGGL(k_pf_reduce<GEMV_RESID>, rgrid, dim3(kBlock), 0, st, b);
            return hipGetLastError();
        }
    }
    // 4 column subtiles per wave; 2 when that leaves fewer than two workgroups per CU
    const int mt = a.Mpad / kPfTileM;
    const int out4 = a.mode == GEMV_SILU ? 2 : 4;
    const int wg4 = (a.n_sub + 2 * out4 - 1) / (2 * out4) * mt;
    const int ni = wg4 >= 2 * device_cu_count() ? 4 : 2;
    const int per_wg = 2 * (a.mode == GEMV_SILU ? ni / 2 : ni);  // output subtiles per workgroup column
    const dim3 grid((unsigned)((a.n_sub + per_wg - 1) / per_wg * mt));
#define PF_LAUNCH(MODE, NI) hipLaunchKernelGGL((k_pf_gemm_q8<MODE, NI>), grid, dim3(256), 0, st, a)
    switch (a.mode * 8 + ni) {
        case GEMV_STORE * 8 + 4: PF_LAUNCH(GEMV_STORE, 4); break;
        case GEMV_STORE * 8 + 2: PF_LAUNCH(GEMV_STORE, 2); break;
        case GEMV_RESID * 8 + 4: PF_LAUNCH(GEMV_RESID, 4); break;
        case GEMV_RESID * 8 + 2: PF_LAUNCH(GEMV_RESID, 2); break;
        case GEMV_SILU * 8 + 4: PF_LAUNCH(GEMV_SILU, 4); break;
        case GEMV_SILU * 8 + 2: PF_LAUNCH(GEMV_SILU, 2); break;
        default: return hipErrorInvalidValue;
    }
#undef PF_LAUNCH
    return hipGetLastError();
}

hipError_t launch_pf_rope_store(float* qkv, int64_t ld, int n, int H, int G, int hd, const float* rope_cos,
                                const float* rope_sin, int pos0, float* kc, float* vc, int layout, int max_seq,
                                hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (pos0 < 0 || pos0 + n > max_seq || hd % 2 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_rope_store, dim3(n), dim3(kBlock), 0, st, qkv, ld, H, G, hd, rope_cos, rope_sin, pos0, kc,
                       vc, layout, max_seq);
    return hipGetLastError();
}

bool pf_attn_supported(int hd, int n_rep) {
    return (hd == 32 || hd == 64 || hd == 128) && n_rep >= 1 && n_rep <= 8;
}

hipError_t launch_pf_attn(const float* q, int64_t ldq, const float* kc, const float* vc, int layout, int H, int G,
                          int hd, int max_seq, int n, int pos0, int att_start, float* out, int64_t ldo,
                          hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int n_rep = H / G;
    if (H % G != 0 || !pf_attn_supported(hd, n_rep) || att_start < 0 || att_start > pos0 || pos0 + n > max_seq ||
        ldq % 4 != 0 || ldo % 4 != 0)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n + 15) / 16), (unsigned)G), block((unsigned)(64 * n_rep));
    switch (hd) {
        case 32:
            hipLaunchKernelGGL(k_pf_attn<32>, grid, block, 0, st, q, ldq, kc, vc, layout, G, max_seq, n_rep, n, pos0,
                               att_start, out, ldo);
            break;
        case 64:
            hipLaunchKernelGGL(k_pf_attn<64>, grid, block, 0, st, q, ldq, kc, vc, layout, G, max_seq, n_rep, n, pos0,
                               att_start, out, ldo);
            break;
        default:
            hipLaunchKernelGGL(k_pf_attn<128>, grid, block, 0, st, q, ldq, kc, vc, layout, G, max_seq, n_rep, n, pos0,
                               att_start, out, ldo);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_pf_tail(Ctl* ctl, int pos_last, const int32_t* hist, const float* xrow, float* x, int D,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_pf_tail, dim3(1), dim3(kBlock), 0, st, ctl, pos_last, hist, xrow, x, D);
    return hipGetLastError();
}

}  // namespace tfk
