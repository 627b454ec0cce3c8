// Prefill of prompt tokens on the matrix cores: Model::prefill and layer_prefill
// (model.cpp:144-195) for a chunk of M tokens at once.
//
// k_pf_split     rmsnorm (layers.cpp:7-12) of each row, or the row as it is, scaled by
//                a power of two and written as fp16 hi + lo in fragment order (the A operand)
// k_pf_gemm_tile / k_pf_gemm_big   matmul (matmul.cpp:64-73) of Q8_0, Q4_0, Q4_1 or F16
//                weights, read in their HBM layout, on v_mfma_f32_16x16x32_f16 (k_pf_gemm_q6k:
//                Q6_K; k_pf_gemm_f32: F32 weights on v_mfma_f32_16x16x4_f32); epilogues:
//                store (+ F32 bias, model.cpp:85-89), residual add (add_inplace,
//                layers.cpp:21-23), silu(gate) * up (layers.cpp:14-19)
// k_pf_rope_store apply_rope_many of q and k (attention.cpp:48-53) and KVCache::store
//                (kvcache.cpp:31-36) of every row
// k_pf_reduce    the slices of a GEMM with K split, added in slice order, + its epilogue;
//                k_pf_reduce_rope / k_pf_reduce_split do that and then k_pf_rope_store's
//                or k_pf_split's work on the rows they hold
// k_pf_pack_kv   the keys and values attention covers, per 32-key tile, as scaled fp16
//                pairs in MFMA fragment order
// k_pf_attn      causal GQA attention of the chunk (attn_prefill, attention.cpp:82-111)
//                on v_mfma_f32_16x16x32_f16 with fp16 operand pairs and an online softmax
//
// Numerics. A Q8_0 weight q is an integer in [-128, 127], a Q4_0 one in [-8, 7], a Q4_1
// code in [0, 15], all exact in fp16, as is an F16 weight; a 32-element block's products
// with the fp16 pair (hi, lo) of an activation are exact in the fp32 accumulator, and
// hi + lo carries 22 significant bits of the fp32 activation (24). Each block's two MFMAs
// start from zero and the block sum is scaled by its fp16 d in fp32 (quant.cpp:266-321
// scales block sums the same way; Q4_1 adds m times the block sum of the activations),
// so the result differs from the fp32 reference by summation order and the 2^-22 split,
// both far inside the 1e-3 parity bound. Scaling rows by 2^e (max |x| in [2^14, 2^15))
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
// of a 16 x 32 operand tile. The activations are stored so that one tile is 64 lanes x 16
// bytes, contiguous: a wave fills a fragment with one coalesced 1 KiB load.
//   activations: xa[row tile][block][hi, lo][lane][8]   (k_pf_split)
// The weights stay where they lie (DevMat streams, no copy): the GEMMs turn the 8 values a
// lane needs (row l % 16 of a 16-row subtile, elements 8 c .. 8 c + 7 of a 32-element block,
// c = l / 16) into fp16 as they go. Each format gives the integers of its blocks, exact in
// fp16, and the block's scale multiplies the block sum afterwards in fp32 (Q4_1's d n + m as
// d sum x n + m sum x); F16 weights are their own fp16 values with scale 1.

// Bytes of a dword, two at a time, as the low bytes of two halves whose high byte is 0x64
// (v_perm_b32: selector byte n < 4 takes byte n of the second operand, 4 byte 0 of the
// first): bytes 0, 1 (hi = 0) or 2, 3 (hi = 1) of w -> the halves 1024 + byte.
__device__ __forceinline__ uint32_t bytes_to_h2(uint32_t w, int hi) {
    return __builtin_amdgcn_perm(0x64646464u, w, hi ? 0x04030402u : 0x04010400u);
}

// Eight int8 bytes q -> their fp16 values: with u = q + 128 (the byte with its top bit
// flipped), 0x64UU is the half 1024 + u, and 1024 + u - 1152 = q exactly.
__device__ __forceinline__ h8_t q8_to_h8(uint2 w) {
    const uint32_t x = w.x ^ 0x80808080u, y = w.y ^ 0x80808080u;
    const tf_u32x4 p = {bytes_to_h2(x, 0), bytes_to_h2(x, 1), bytes_to_h2(y, 0), bytes_to_h2(y, 1)};
    const h8_t off = {1152, 1152, 1152, 1152, 1152, 1152, 1152, 1152};
    return __builtin_bit_cast(h8_t, p) - off;
}

// The 4-bit codes n in the low (hi = 0) or high (hi = 1) nibbles of 8 bytes -> fp16 n - OFF.
template <int OFF>
__device__ __forceinline__ h8_t q4_to_h8(uint2 w, int hi) {
    const int sh = 4 * hi;
    const uint32_t a = (w.x >> sh) & 0x0F0F0F0Fu, b = (w.y >> sh) & 0x0F0F0F0Fu;
    const tf_u32x4 p = {bytes_to_h2(a, 0), bytes_to_h2(a, 1), bytes_to_h2(b, 0), bytes_to_h2(b, 1)};
    constexpr _Float16 o = (_Float16)(1024 + OFF);
    const h8_t off = {o, o, o, o, o, o, o, o};
    return __builtin_bit_cast(h8_t, p) - off;
}

// A layer-matrix format as the GEMMs read it.
//   kBytes  bytes of one row's 32-element block in the q stream
//   kSub    LDS bytes of a 16-row subtile's block (k_pf_gemm_big)
//   kScale  bytes of one row's block in the s stream (0: no scales)
//   kMin    Q4_1's min term
//   off(c)  byte offset in a row's block of the piece lane c = l / 16 reads
//   lds(p, r, c)  that piece of subtile row r from the subtile's LDS block at p
//   cvt(raw, c)   its 8 values as fp16
template <int T>
struct PfW;

// Q8_0 (quant.cpp:66-72): 32 int8 per block. LDS: the 16-byte half h of row r at 16 (16 h + r).
template <>
struct PfW<TF_HIP_TYPE_Q8_0> {
    static constexpr int kBytes = 32, kSub = 512, kScale = 2;
    static constexpr bool kMin = false;
    typedef uint2 Raw;
    __device__ static int off(int c) { return 8 * c; }
    __device__ static Raw load(const TF_GLOBAL uint8_t* p) { return gload_u2((const void*)p); }
    __device__ static Raw lds(const unsigned char* p, int r, int c) {
        return *(const uint2*)(p + 256 * (c >> 1) + 16 * r + 8 * (c & 1));
    }
    __device__ static h8_t cvt(Raw w, int) { return q8_to_h8(w); }
};

// Q4_0 (quant.cpp:74-86): 16 bytes per block, element j in the low nibble of byte j and
// element j + 16 in its high nibble, value n - 8. LDS: row r's 16 bytes at 16 r.
template <>
struct PfW<TF_HIP_TYPE_Q4_0> {
    static constexpr int kBytes = 16, kSub = 256, kScale = 2;
    static constexpr bool kMin = false;
    typedef uint2 Raw;
    __device__ static int off(int c) { return 8 * (c & 1); }
    __device__ static Raw load(const TF_GLOBAL uint8_t* p) { return gload_u2((const void*)p); }
    __device__ static Raw lds(const unsigned char* p, int r, int c) { return *(const uint2*)(p + 16 * r + 8 * (c & 1)); }
    __device__ static h8_t cvt(Raw w, int c) { return q4_to_h8<8>(w, c >> 1); }
};

// Q4_1 (quant.cpp:87-99): the Q4_0 layout with value n d + m; the s stream holds d and m.
template <>
struct PfW<TF_HIP_TYPE_Q4_1> {
    static constexpr int kBytes = 16, kSub = 256, kScale = 4;
    static constexpr bool kMin = true;
    typedef uint2 Raw;
    __device__ static int off(int c) { return 8 * (c & 1); }
    __device__ static Raw load(const TF_GLOBAL uint8_t* p) { return gload_u2((const void*)p); }
    __device__ static Raw lds(const unsigned char* p, int r, int c) { return *(const uint2*)(p + 16 * r + 8 * (c & 1)); }
    __device__ static h8_t cvt(Raw w, int c) { return q4_to_h8<0>(w, c >> 1); }
};

// F16 (quant.cpp:129-131): 64 bytes per block. LDS: the 16-byte piece c of row r at 16 (16 c + r).
template <>
struct PfW<TF_HIP_TYPE_F16> {
    static constexpr int kBytes = 64, kSub = 1024, kScale = 0;
    static constexpr bool kMin = false;
    typedef uint4 Raw;
    __device__ static int off(int c) { return 16 * c; }
    __device__ static Raw load(const TF_GLOBAL uint8_t* p) { return gload_u4((const void*)p); }
    __device__ static Raw lds(const unsigned char* p, int r, int c) { return *(const uint4*)(p + 256 * c + 16 * r); }
    __device__ static h8_t cvt(Raw w, int) { return __builtin_bit_cast(h8_t, w); }
};

// Block blk's scale d and min m from a scale word: a pair of fp16 d (blocks 2 p, 2 p + 1)
// for kScale 2, d | m << 16 of block blk for kScale 4, none for kScale 0.
template <int KS>
__device__ __forceinline__ void pf_scale(uint32_t word, int blk, float& d, float& m) {
    if (KS == 2) {
        d = h2f(word >> (16 * (blk & 1)));
        m = 0.0f;
    } else if (KS == 4) {
        d = h2f(word & 0xFFFFu);
        m = h2f(word >> 16);
    } else {
        d = 1.0f;
        m = 0.0f;
    }
}

constexpr int kSplitGroups = 8;  // 8-element groups per thread: rows up to 256 * 8 * 8 = 16384

// The split of row m whose values thread tid holds as v[i] = 8-element group tid + i ST
// (ST = 64 WPR threads per row; groups past K / 8 hold clamped re-reads, masked here):
// rmsnorm with weight w when given, the power-of-two scale, hi + lo into the fragments.
template <int NG, int WPR>
__device__ __forceinline__ void split_emit(float (&v)[NG][8], int tid, int m, int K, const float* w, float eps,
                                           h8_t* xa, float* rs, double* red_d, float* red_f) {
    constexpr int ST = 64 * WPR;
    const int ng = K / 8, nblk = K / 32;
    h8_t* tile = xa + (int64_t)(m / 16) * nblk * 128 + (m % 16);
    const float4* wr = (const float4*)w;
    float inv = 1.0f;
    if (w) {
        double ss = 0;
#pragma unroll
        for (int i = 0; i < NG; ++i)
            if (tid + i * ST < ng)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += (double)v[i][e] * v[i][e];
        ss = wave_sum_d(ss);
        if (WPR > 1) {
            if ((tid & 63) == 0) red_d[tid >> 6] = ss;
            __syncthreads();
            ss = (red_d[0] + red_d[1]) + (red_d[2] + red_d[3]);
        }
        inv = 1.0f / sqrtf((float)(ss / K) + eps);
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            int j = tid + i * ST;
            j = j < ng ? j : ng - 1;
            const float4 a = wr[2 * j], b = wr[2 * j + 1];
            const float g[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[i][e] = v[i][e] * inv * g[e];
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NG; ++i)
        if (tid + i * ST < ng)
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
    amax = wave_max(amax);
    if (WPR > 1) {
        if ((tid & 63) == 0) red_f[tid >> 6] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    }
    int ex = 0;
    (void)frexpf(amax, &ex);  // amax = f 2^ex, f in [0.5, 1)
    int e2 = amax > 0.0f ? 15 - ex : 0;
    e2 = e2 < -100 ? -100 : (e2 > 100 ? 100 : e2);
    const float sc = ldexpf(1.0f, e2);
    if (tid == 0) rs[m] = ldexpf(1.0f, -e2);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int j = tid + i * ST;
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

// Zeros of padding row m's fragments (rs = 0), ST threads.
template <int ST>
__device__ __forceinline__ void split_zero(int tid, int m, int K, h8_t* xa, float* rs) {
    const int ng = K / 8, nblk = K / 32;
    h8_t* tile = xa + (int64_t)(m / 16) * nblk * 128 + (m % 16);
    const h8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = tid; j < ng; j += ST) {
        h8_t* o = tile + (j / 4) * 128 + 16 * (j % 4);
        o[0] = z;
        o[64] = z;
    }
    if (tid == 0) rs[m] = 0.0f;
}

// WPR waves per row (1: a workgroup takes 4 consecutive rows, a wave each, and reduces
// within the wave; 4: a workgroup per row), the row held in registers (thread t of the row
// owns the 8-element groups t, t + 64 WPR, ..., NG of them: the fewest that cover the row):
// the rmsnorm scale inv (when w is given), a power of two sc putting max |row| in
// [2^14, 2^15) (rs = 1 / sc), then every element as hi + lo into the fragment layout (16
// bytes of a hi and of a lo fragment per group; with a wave per row, the 4 rows of a
// workgroup fill whole 64-byte lines of a fragment). Rows M.. are zeros with rs = 0.
template <int NG, int WPR>
__global__ __launch_bounds__(kBlock) void k_pf_split(const float* x, int64_t ldx, const float* w, float eps, int K,
                                                     int M, h8_t* xa, float* rs) {
    constexpr int ST = 64 * WPR;  // threads per row
    __shared__ double red_d[kWavesPerBlock];
    __shared__ float red_f[kWavesPerBlock];
    const int m = WPR == 1 ? blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6) : blockIdx.x;
    const int tid = WPR == 1 ? threadIdx.x & 63 : threadIdx.x;
    const int ng = K / 8;
    if (m >= M) {
        split_zero<ST>(tid, m, K, xa, rs);
        return;
    }
    const float4* xr = (const float4*)(x + (int64_t)m * ldx);
    float v[NG][8];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int j = tid + i * ST;
        const int jj = j < ng ? j : ng - 1;  // a clamped re-read, masked below
        const float4 a = xr[2 * jj], b = xr[2 * jj + 1];
        v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
        v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
    }
    split_emit<NG, WPR>(v, tid, m, K, w, eps, xa, rs, red_d, red_f);
}

// ---------------------------------------------------------------- GEMM

// Field of the segment holding output subtile u (uniform per wave: scalar selects).
#define PF_SEL(s, f) ((s) == 0 ? a.seg[0].f : ((s) == 1 ? a.seg[1].f : a.seg[2].f))

// A register-streamed tile (k_pf_gemm_tile, k_pf_gemm_f32, k_pf_gemm_q6k): a workgroup of 4
// waves as 2 (rows) x 2 (columns); a wave owns 32 rows from m0 and NI weight-column subtiles
// of 16 (GEMV_SILU: NI / 2 output subtiles, each a gate and an up subtile). Per subtile: its
// segment, the weight row c this lane reads (the output column), whether it is past the
// last subtile (computed on a clamped one, not written).
template <int MODE, int NI, int MI = 2, int WM = 2>
struct TileCtx {
    static constexpr int NO = MODE == GEMV_SILU ? NI / 2 : NI;  // output subtiles per wave
    int lane, l16, lc, m0;
    int kslice = 0;  // K slice of a split launch (ks slices, workgroups slice-fastest)
    int seg[NI], c[NI], gcol[NI];
    bool ok[NI];
    float* y[NI];
    const float* bias[NI];
    int64_t ldy[NI];
    const uint8_t *wq[NI], *wq2[NI], *ws[NI], *ws2[NI];  // the subtile's matrix streams
    __device__ __forceinline__ TileCtx(const PfGemmArgs& a, int ks = 1) {
        lane = threadIdx.x & 63;
        l16 = lane & 15;
        lc = lane >> 4;
        const int wave = threadIdx.x >> 6;
        // XCD-aware order: workgroup b runs on XCD b % 8; give each XCD a contiguous range
        // of tiles, rows fastest, so the row tiles that share a weight tile share an L2.
        int b = blockIdx.x;
        {
            const int q = (int)gridDim.x / 8;
            if (b < 8 * q) b = (b % 8) * q + b / 8;
        }
        kslice = b % ks;
        b /= ks;
        // WM == 2: 64-row tiles, waves 2 (rows, MI = 2 subtiles each) x 2 (columns); WM == 1:
        // tiles of MI 16-row subtiles, all 4 waves along the columns
        const int MT = WM == 2 ? a.Mpad / kPfTileM : (a.M + 16 * MI - 1) / (16 * MI);
        const int mt = b % MT, nt = b / MT;
        m0 = WM == 2 ? mt * kPfTileM + (wave & 1) * 32 : mt * 16 * MI;
        const int wid = WM == 2 ? nt * 2 + (wave >> 1) : nt * 4 + wave;
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
            int u = wid * NO + ni % NO;
            ok[ni] = u < a.n_sub;
            u = u < a.n_sub ? u : a.n_sub - 1;
            seg[ni] = (a.n_seg > 2 && u >= a.seg[2].sub0) ? 2 : ((a.n_seg > 1 && u >= a.seg[1].sub0) ? 1 : 0);
            c[ni] = (u - PF_SEL(seg[ni], sub0)) * 16 + l16;
            gcol[ni] = u * 16 + l16;
            const bool u2 = up(ni);
            const int sg = seg[ni];
            wq[ni] = u2 ? PF_SEL(sg, w2.q) : PF_SEL(sg, w.q);
            wq2[ni] = u2 ? PF_SEL(sg, w2.q2) : PF_SEL(sg, w.q2);
            ws[ni] = u2 ? PF_SEL(sg, w2.s) : PF_SEL(sg, w.s);
            ws2[ni] = u2 ? PF_SEL(sg, w2.s2) : PF_SEL(sg, w.s2);
            y[ni] = PF_SEL(seg[ni], y);
            bias[ni] = PF_SEL(seg[ni], bias);
            ldy[ni] = PF_SEL(seg[ni], ldy);
        }
    }
    __device__ __forceinline__ static bool up(int ni) { return MODE == GEMV_SILU && ni >= NO; }
    // fragment pointers of the wave's two 16-row activation subtiles (lane's 8 halves)
    __device__ __forceinline__ void act(const PfGemmArgs& a, const TF_GLOBAL h8_t* (&ap)[MI]) const {
        const int nblk = a.K / 32;
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
            ap[mi] = (const TF_GLOBAL h8_t*)a.xa + (int64_t)(m0 / 16 + mi) * nblk * 128 + lane;
    }
    // lane holds rows m0 + 16 mi + 4 (lane / 16) + r of output column c[ni], scaled back by
    // the row scales: store (+ bias), residual add (+ the tap row) or silu(gate) * up
    __device__ __forceinline__ void epilogue(const PfGemmArgs& a, const f4_t (&acc)[MI][NI]) const {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
            const int r0 = m0 + 16 * mi + 4 * (lane >> 4);
            const float4 rsv = *(const float4*)(a.rs + r0);
            const float rsa[4] = {rsv.x, rsv.y, rsv.z, rsv.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = r0 + r;
                if (row >= a.M) continue;
#pragma unroll
                for (int ni = 0; ni < NO; ++ni) {
                    if (!ok[ni]) continue;
                    float* p = y[ni] + (int64_t)row * ldy[ni] + c[ni];
                    if (MODE == GEMV_SILU) {
                        const float gv = acc[mi][ni][r] * rsa[r];
                        const float uv = acc[mi][ni + NO][r] * rsa[r];
                        *p = (gv / (1.0f + expf(-gv))) * uv;
                    } else if (MODE == GEMV_STORE) {
                        const float v = acc[mi][ni][r] * rsa[r];
                        *p = bias[ni] ? v + bias[ni][c[ni]] : v;
                    } else {
                        const float nv = *p + acc[mi][ni][r] * rsa[r];
                        *p = nv;
                        if (row == a.tap_row && a.tap) a.tap[c[ni]] = nv;
                    }
                }
            }
        }
    }
    // a K slice's row-scaled partial sums: part[kslice][row][output column] (the big tiles'
    // layout, read by the same reduces)
    // (GEMV_SILU: the gate columns, then the up columns)
    __device__ __forceinline__ void epilogue_part(const PfGemmArgs& a, const f4_t (&acc)[MI][NI]) const {
        const int nout = a.n_sub * 16;
        const int ntot = MODE == GEMV_SILU ? 2 * nout : nout;
        float* part = a.part + (int64_t)kslice * a.Mpad * ntot;
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
            const int r0 = m0 + 16 * mi + 4 * (lane >> 4);
            const float4 rsv = *(const float4*)(a.rs + r0);
            const float rsa[4] = {rsv.x, rsv.y, rsv.z, rsv.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (r0 + r >= a.M) continue;
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
                    if (ok[ni]) part[(int64_t)(r0 + r) * ntot + gcol[ni] + (up(ni) ? nout : 0)] = acc[mi][ni][r] * rsa[r];
            }
        }
    }
};

// Per 32-element block: for each (row subtile, column subtile) an MFMA of the hi part from
// zero, then one of the lo part on top (issued after all eight hi MFMAs, so no MFMA waits on
// the one before it), then acc += d * block sum (Q4_1: + m * the rows' block sums, from the
// same two MFMAs against a fragment of ones). Weight bytes and activation fragments stream
// from L2 into registers, one stage of two blocks ahead; every load is unconditional
// (indices clamped) so the compiler waits only for the stage it consumes.
template <int MODE, int NI, int T, bool SPLIT, int MI, int WM>
__global__ __launch_bounds__(256) void k_pf_gemm_tile(const PfGemmArgs a) {
    using W = PfW<T>;
    const TileCtx<MODE, NI, MI, WM> t(a, SPLIT ? a.ks : 1);
    const int K = a.K, nblk = K / 32;
    constexpr int SW = W::kScale == 4 ? 2 : 1;  // scale words per stage and column
    const TF_GLOBAL uint8_t* bp[NI];
    const TF_GLOBAL uint32_t* sp[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
        bp[ni] = (const TF_GLOBAL uint8_t*)t.wq[ni] + (int64_t)t.c[ni] * nblk * W::kBytes + W::off(t.lc);
        sp[ni] = (const TF_GLOBAL uint32_t*)(t.ws[ni] + (int64_t)t.c[ni] * nblk * W::kScale);
    }
    const TF_GLOBAL h8_t* ap[MI];
    t.act(a, ap);

    f4_t acc[MI][NI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};

    struct Stage {
        h8_t ah[MI][2], al[MI][2];  // [row subtile][block]
        typename W::Raw bw[NI][2];  // [column subtile][block]: the lane's weight bytes
        uint32_t d[NI][SW];         // the scale words of the stage's two blocks
    };
    const int S = SPLIT ? K / 64 / a.ks : K / 64;  // stages (two blocks) of this K slice
    const int sb = SPLIT ? t.kslice * S : 0;       // its first stage
    auto load = [&](int s, Stage& g) {
        s = sb + (s < S ? s : S - 1);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int blk = 2 * s + j;
#pragma unroll
            for (int mi = 0; mi < MI; ++mi) {
                g.ah[mi][j] = ap[mi][blk * 128];
                g.al[mi][j] = ap[mi][blk * 128 + 64];
            }
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) g.bw[ni][j] = W::load(bp[ni] + (int64_t)blk * W::kBytes);
        }
        if (W::kScale)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                for (int w = 0; w < SW; ++w) g.d[ni][w] = sp[ni][SW * s + w];
    };
    const h8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
    auto compute = [&](const Stage& g) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            h8_t bh[NI];
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) bh[ni] = W::cvt(g.bw[ni][j], t.lc);
            f4_t tb[MI][NI], ts[MI];
#pragma unroll
            for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
                    tb[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(g.ah[mi][j], bh[ni],
                                                                       (f4_t){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                if (W::kMin)
                    ts[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(g.ah[mi][j], ones, (f4_t){0.0f, 0.0f, 0.0f, 0.0f},
                                                                    0, 0, 0);
            }
#pragma unroll
            for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
                    tb[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(g.al[mi][j], bh[ni], tb[mi][ni], 0, 0, 0);
                if (W::kMin) ts[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(g.al[mi][j], ones, ts[mi], 0, 0, 0);
            }
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) {
                float dv, mv;
                pf_scale<W::kScale>(g.d[ni][SW == 2 ? j : 0], j, dv, mv);
#pragma unroll
                for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[mi][ni][r] = W::kMin ? fmaf(dv, tb[mi][ni][r], fmaf(mv, ts[mi][r], acc[mi][ni][r]))
                                                 : fmaf(dv, tb[mi][ni][r], acc[mi][ni][r]);
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
    if (SPLIT)
        t.epilogue_part(a, acc);
    else
        t.epilogue(a, acc);
}

// F32 weights on v_mfma_f32_16x16x4_f32. The activations come from the same hi + lo
// fragments (their sum, exact in fp32, is the row's 22-bit value); the weights are loaded as
// they lie. Within a 32-element block, MFMA j (0..7) takes from lane l the element
// k = 8 (l / 16) + j: the 8 consecutive values each lane holds of both operands, a
// reordering of the block's terms. No block scales: every MFMA accumulates into acc.
template <int MODE, int NI>
__global__ __launch_bounds__(256) void k_pf_gemm_f32(const PfGemmArgs a) {
    const TileCtx<MODE, NI> t(a);
    const int K = a.K, nblk = K / 32;
    const float* bp[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) bp[ni] = (const float*)t.wq[ni] + (int64_t)t.c[ni] * K + 8 * t.lc;
    const TF_GLOBAL h8_t* ap[2];
    t.act(a, ap);
    f4_t acc[2][NI];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};
    for (int blk = 0; blk < nblk; ++blk) {
        float x[2][8];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
            const h8_t hi = ap[mi][blk * 128], lo = ap[mi][blk * 128 + 64];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[mi][j] = (float)hi[j] + (float)lo[j];
        }
        float w[NI][8];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
            const float4 u = gload_f4(bp[ni] + 32 * blk), v = gload_f4(bp[ni] + 32 * blk + 4);
            w[ni][0] = u.x; w[ni][1] = u.y; w[ni][2] = u.z; w[ni][3] = u.w;
            w[ni][4] = v.x; w[ni][5] = v.y; w[ni][6] = v.z; w[ni][7] = v.w;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[mi][j], w[ni][j], acc[mi][ni], 0, 0, 0);
    }
    t.epilogue(a, acc);
}

// Q6_K weights (quant.cpp:101-127). A 32-element group of a row: lo[16] (element e < 16 in
// the low nibble of byte e, e + 16 in its high nibble), hi[8] (element e's top two bits at
// bits 2 (e / 8) of byte e % 8), an int8 scale per 16 elements and an fp16 d per 256: the
// value d sc (u - 32) for the 6-bit code u. Lane l's 8 elements 8 c .. 8 c + 7 (c = l / 16)
// share the scale sc of sub-block c / 2, folded into the B operand: sc (u - 32), an integer
// of at most 4096 in magnitude, is the fp16 pair hi (its rounding, v_pk_mul_f16) + lo (the
// exact remainder, at most 1, from v_pk_fma_f16). Per block: the activation hi and lo against
// B hi and the activation hi against B lo (the lo x lo term is below 2^-22 of the product)
// from zero, then acc += d * block sum.
template <int MODE, int NI>
__global__ __launch_bounds__(256) void k_pf_gemm_q6k(const PfGemmArgs a) {
    const TileCtx<MODE, NI> t(a);
    const int K = a.K, nblk = K / 32;
    const TF_GLOBAL uint8_t *lp[NI], *hp[NI], *scp[NI];
    const TF_GLOBAL uint16_t* dp[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
        const int64_t c = t.c[ni];
        lp[ni] = (const TF_GLOBAL uint8_t*)t.wq[ni] + c * (K / 2) + 8 * (t.lc & 1);
        hp[ni] = (const TF_GLOBAL uint8_t*)t.wq2[ni] + c * (K / 4);
        scp[ni] = (const TF_GLOBAL uint8_t*)t.ws[ni] + c * (K / 16) + (t.lc >> 1);
        dp[ni] = (const TF_GLOBAL uint16_t*)(t.ws2[ni] + c * (K / 256) * 2);
    }
    const TF_GLOBAL h8_t* ap[2];
    t.act(a, ap);
    f4_t acc[2][NI];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};
    const f4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int blk = 0; blk < nblk; ++blk) {
        h8_t ah[2], al[2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
            ah[mi] = ap[mi][blk * 128];
            al[mi] = ap[mi][blk * 128 + 64];
        }
        h8_t bh[NI], bl[NI];
        float dv[NI];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
            const uint2 lo = gload_u2((const void*)(lp[ni] + 16 * blk));
            const uint2 hi = gload_u2((const void*)(hp[ni] + 8 * blk));
            const int sh = 4 * (t.lc >> 1), hs = 2 * t.lc;
            const uint32_t u0 = ((lo.x >> sh) & 0x0F0F0F0Fu) | (((hi.x >> hs) & 0x03030303u) << 4);
            const uint32_t u1 = ((lo.y >> sh) & 0x0F0F0F0Fu) | (((hi.y >> hs) & 0x03030303u) << 4);
            const tf_u32x4 p = {bytes_to_h2(u0, 0), bytes_to_h2(u0, 1), bytes_to_h2(u1, 0), bytes_to_h2(u1, 1)};
            const h8_t off = {1056, 1056, 1056, 1056, 1056, 1056, 1056, 1056};
            const h8_t q = __builtin_bit_cast(h8_t, p) - off;  // u - 32, exact
            const _Float16 sc = (_Float16)(int8_t)scp[ni][2 * blk];
            const h8_t scv = {sc, sc, sc, sc, sc, sc, sc, sc};
            bh[ni] = q * scv;
            bl[ni] = __builtin_elementwise_fma(q, scv, -bh[ni]);
            dv[ni] = h2f(dp[ni][blk >> 3]);
        }
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) {
                f4_t tb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mi], bh[ni], zero, 0, 0, 0);
                tb = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mi], bh[ni], tb, 0, 0, 0);
                tb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mi], bl[ni], tb, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[mi][ni][r] = fmaf(dv[ni], tb[r], acc[mi][ni][r]);
            }
    }
    t.epilogue(a, acc);
}

// Large tiles for GEMMs with enough of them to fill the CUs: a workgroup of 8 waves
// (2 rows x 4 columns of waves) owns 128 rows x 16 weight-column subtiles (256 weight rows;
// GEMV_SILU: 8 gate and the 8 matching up subtiles, 128 output columns). A stage (one
// 32-element block) of both operands and the scales goes straight from global memory into
// one of four LDS buffers, four loads per wave, three stages ahead of its use: the 16
// activation fragments (1 KiB each), the 256 weight rows' bytes of the block in the
// format's subtile layout, and their scale words. Each wave then runs 4 x 4 tiles of
// 16 x 16, reading activation fragments and weight bytes from LDS and turning the bytes
// into fp16 in registers (4 waves of 4 x 8 tiles, a third fewer LDS reads per MFMA,
// measured 12% slower: one wave per SIMD leaves the MFMA-to-scale dependencies exposed).
// The per-block arithmetic and its order are those of k_pf_gemm_tile, so the two give the
// same bits.
constexpr int kBigThreads = 512;
constexpr int kBigWaves = kBigThreads / 64;
constexpr int kBigRows = 128;
constexpr int kBigABytes = 16 * 1024;                           // 16 activation fragments (8 row tiles, hi and lo)
constexpr int kBigBBytes = 16 * 1024;                           // 256 weight rows x 64 bytes at most (F16)
constexpr int kBigStageBytes = kBigABytes + kBigBBytes + 1024;  // + a scale word per weight row
constexpr int kBigStages = 4;                                   // LDS buffers: one in use, three loading
constexpr size_t kBigLdsBytes = kBigStages * (size_t)kBigStageBytes;

// SPLIT: the grid also splits K into a.ks slices; slice ks writes its row-scaled partial
// sums to a.part[ks][row][output column] and k_pf_reduce applies the epilogue.
template <int MODE, bool SPLIT, int T>
__global__ __launch_bounds__(kBigThreads) void k_pf_gemm_big(const PfGemmArgs a) {
    using W = PfW<T>;
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
    const int S = SPLIT ? nblk / a.ks : nblk;  // stages (blocks) of this slice
    const int s0 = kslice * S;                 // its first block
    const int l16 = lane & 15, lc = lane >> 4;
    constexpr bool SILU = MODE == GEMV_SILU;

    // weight-column subtile q (0..15) of this workgroup: output subtile, matrix, tile row
    auto resolve = [&](int q, int& u, int& seg, bool& up) {
        up = SILU && q >= 8;
        u = SILU ? nt * 8 + (q & 7) : nt * 16 + q;
        u = u < a.n_sub ? u : a.n_sub - 1;
        seg = (a.n_seg > 2 && u >= a.seg[2].sub0) ? 2 : ((a.n_seg > 1 && u >= a.seg[1].sub0) ? 1 : 0);
    };
    // row r of weight-column subtile q, at byte off of each block
    auto wrow = [&](int q, int r, int off) {
        int u, seg;
        bool up;
        resolve(q, u, seg, up);
        const uint8_t* wq = up ? PF_SEL(seg, w2.q) : PF_SEL(seg, w.q);
        return (const TF_GLOBAL uint8_t*)wq + ((int64_t)(u - PF_SEL(seg, sub0)) * 16 + r) * nblk * W::kBytes + off;
    };
    // this wave's loads per stage: activation fragments f = wave + 8 i (row tile f / 2, hi
    // or lo); weight bytes of subtiles 2 wave, 2 wave + 1 (lane i writes LDS byte 16 i of
    // the wave's part): Q8_0 one 1 KiB load (lane i: half i / 16 % 2 of row i % 16 of
    // subtile 2 wave + i / 32), Q4 one 512-byte load of lanes 0..31 (row i % 16 of subtile
    // 2 wave + i / 16), F16 a 1 KiB load per subtile (piece i / 16 of row i % 16)
    const TF_GLOBAL h8_t* asrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = wave + kBigWaves * i;
        asrc[i] = (const TF_GLOBAL h8_t*)a.xa + (int64_t)(mt * 8 + f / 2) * nblk * 128 + (f % 2) * 64 + lane;
    }
    constexpr int NB = W::kSub == 1024 ? 2 : 1;  // weight loads per wave and stage
    const TF_GLOBAL uint8_t* bsrc[NB];
    if (W::kSub == 512) {
        bsrc[0] = wrow(2 * wave + (lane >> 5), l16, 16 * (lc & 1));
    } else if (W::kSub == 256) {
        bsrc[0] = wrow(2 * wave + (lc & 1), l16, 0);
    } else {
#pragma unroll
        for (int j = 0; j < NB; ++j) bsrc[j] = wrow(2 * wave + j, l16, 16 * lc);
    }
    // the scales: lane i < 32 of wave w loads the scale word of weight column 32 w + i
    // (Q8_0 / Q4_0: the fp16 pair of blocks 2 p, 2 p + 1; Q4_1: d and m of the block)
    const TF_GLOBAL uint32_t* dsrc = nullptr;
    if (W::kScale) {
        const int j = 32 * wave + (lane & 31), q = j / 16;
        int u, seg;
        bool up;
        resolve(q, u, seg, up);
        const int c = (u - PF_SEL(seg, sub0)) * 16 + (j & 15);
        const uint8_t* ws = up ? PF_SEL(seg, w2.s) : PF_SEL(seg, w.s);
        dsrc = (const TF_GLOBAL uint32_t*)(ws + (int64_t)c * nblk * W::kScale);
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
    auto issue = [&](int s) {  // stage s into buffer s % 4: 4 loads per wave
        const int blk = s0 + s;
        const uint32_t base = lds0 + (uint32_t)((s % kBigStages) * kBigStageBytes);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            lds_dma16(asrc[i] + (int64_t)blk * 128,
                      __builtin_amdgcn_readfirstlane(base + (uint32_t)((wave + kBigWaves * i) * 1024)));
        const uint32_t bb = base + kBigABytes;
        if (W::kSub == 512) {
            lds_dma16(bsrc[0] + (int64_t)blk * W::kBytes, __builtin_amdgcn_readfirstlane(bb + 1024u * wave));
        } else if (W::kSub == 256) {
            const uint32_t m0 = __builtin_amdgcn_readfirstlane(bb + 512u * wave);
            if (lane < 32) lds_dma16(bsrc[0] + (int64_t)blk * W::kBytes, m0);
        } else {
#pragma unroll
            for (int j = 0; j < NB; ++j)
                lds_dma16(bsrc[j] + (int64_t)blk * W::kBytes, __builtin_amdgcn_readfirstlane(bb + 1024u * (2 * wave + j)));
        }
        if (W::kScale) {
            const uint32_t m0 = __builtin_amdgcn_readfirstlane(base + (uint32_t)(kBigABytes + kBigBBytes + 128 * wave));
            if (lane < 32) lds_dma4(dsrc + (W::kScale == 2 ? blk / 2 : blk), m0);
        }
    };
    constexpr int kLoads = 2 + NB + (W::kScale ? 1 : 0);
    static_assert(kLoads == 4, "the waits below count 4 loads per stage");

    const int wm = wave & 1, wn = wave >> 1;
    int qb[4];  // this wave's weight-column subtiles
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) qb[ni] = SILU ? (ni < 2 ? wn * 2 + ni : 8 + wn * 2 + ni - 2) : wn * 4 + ni;

    f4_t acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};

    // Software-pipelined: a half's block sums are scaled into acc after the next half's
    // MFMAs are issued (the last half of a block after the first of the next block), so the
    // scaling never waits on MFMAs just issued. Same operations, same order per acc.
    f4_t tp[2][4];  // pending block sums: rows half 1 of the previous block
    f4_t tsp[2];    // Q4_1: their rows' block sums
    float dvp[4], mvp[4];
    auto scale_in = [&](int half, const f4_t (&t)[2][4], const f4_t (&ts)[2], const float (&dv)[4],
                        const float (&mv)[4]) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float o = acc[half * 2 + mm][ni][r];
                    acc[half * 2 + mm][ni][r] =
                        W::kMin ? fmaf(dv[ni], t[mm][ni][r], fmaf(mv[ni], ts[mm][r], o)) : fmaf(dv[ni], t[mm][ni][r], o);
                }
    };
    const h8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
    auto compute = [&](int buf, int blk, bool pending) {
        const h8_t* st = (const h8_t*)(lds + buf * kBigStageBytes);
        const unsigned char* sb = lds + buf * kBigStageBytes + kBigABytes;
        const uint32_t* sd = (const uint32_t*)(lds + buf * kBigStageBytes + kBigABytes + kBigBBytes);
        float dv[4], mv[4];
        h8_t bh[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            pf_scale<W::kScale>(W::kScale ? sd[qb[ni] * 16 + l16] : 0u, blk, dv[ni], mv[ni]);
            bh[ni] = W::cvt(W::lds(sb + qb[ni] * W::kSub, l16, lc), lc);
        }
        auto mfmas = [&](int half, f4_t (&t)[2][4], f4_t (&ts)[2]) {
            h8_t ah[2], al[2];
#pragma unroll
            for (int mm = 0; mm < 2; ++mm) {
                const int T2 = wm * 4 + half * 2 + mm;
                ah[mm] = st[(T2 * 2 + 0) * 64 + lane];
                al[mm] = st[(T2 * 2 + 1) * 64 + lane];
            }
#pragma unroll
            for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni)
                    t[mm][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mm], bh[ni], (f4_t){0.0f, 0.0f, 0.0f, 0.0f},
                                                                      0, 0, 0);
                if (W::kMin)
                    ts[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mm], ones, (f4_t){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            }
#pragma unroll
            for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni)
                    t[mm][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mm], bh[ni], t[mm][ni], 0, 0, 0);
                if (W::kMin) ts[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mm], ones, ts[mm], 0, 0, 0);
            }
        };
        f4_t t0[2][4], ts0[2];
        mfmas(0, t0, ts0);
        if (pending) scale_in(1, tp, tsp, dvp, mvp);
        mfmas(1, tp, tsp);
        scale_in(0, t0, ts0, dv, mv);
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            dvp[ni] = dv[ni];
            mvp[ni] = mv[ni];
        }
    };

    const int pre = S < kBigStages - 1 ? S : kBigStages - 1;
    for (int s = 0; s < pre; ++s) issue(s);
    for (int s = 0; s < S; ++s) {
        // this wave's loads of stage s are done when at most those of the (up to two) stages
        // issued after it are in flight; the barrier then makes every wave's done, and every
        // wave has left compute(s - 1), whose buffer stage s + 3 takes
        const int after = S - 1 - s;
        if (after >= 2)
            asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else if (after == 1)
            asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (s + kBigStages - 1 < S) issue(s + kBigStages - 1);
        compute(s % kBigStages, s0 + s, s > 0);
    }
    if (S > 0) scale_in(1, tp, tsp, dvp, mvp);

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
                // GEMV_SILU: the gate columns, then the up columns
                const int nout = a.n_sub * 16, ntot = SILU ? 2 * nout : nout;
                float* part = a.part + ((int64_t)kslice * a.Mpad) * ntot + u * 16 + l16;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (r0 + r < a.M) {
                        part[(int64_t)(r0 + r) * ntot] = acc[mi][ni][r] * rsa[r];
                        if (SILU) part[(int64_t)(r0 + r) * ntot + nout] = acc[mi][ni + 2][r] * rsa[r];
                    }
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

// Sums the KS (= a.ks) partial rows of a split-K GEMM in slice order and applies the
// epilogue: thread per 4 output columns of row blockIdx.y, the KS slices' loads issued
// together (a loop over a run-time count would wait for each before the next).
template <int MODE, int KS>
__global__ __launch_bounds__(kBlock) void k_pf_reduce(const PfGemmArgs a) {
    const int row = blockIdx.y;
    const int col0 = (blockIdx.x * kBlock + threadIdx.x) * 4;
    const int nout = a.n_sub * 16;
    // GEMV_SILU: the gate columns, then the up columns
    const int ntot = MODE == GEMV_SILU ? 2 * nout : nout;
    if (col0 >= nout) return;
    const float* p = a.part + (int64_t)row * ntot + col0;
    float4 pv[KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) pv[k] = *(const float4*)(p + (int64_t)k * a.Mpad * ntot);
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        v[0] += pv[k].x;
        v[1] += pv[k].y;
        v[2] += pv[k].z;
        v[3] += pv[k].w;
    }
    if (MODE == GEMV_SILU) {
#pragma unroll
        for (int k = 0; k < KS; ++k) pv[k] = *(const float4*)(p + nout + (int64_t)k * a.Mpad * ntot);
        float w[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            w[0] += pv[k].x;
            w[1] += pv[k].y;
            w[2] += pv[k].z;
            w[3] += pv[k].w;
        }
        float* y = a.seg[0].y + (int64_t)row * a.seg[0].ldy + col0;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (v[e] / (1.0f + expf(-v[e]))) * w[e];
        return;
    }
    // a 16-column subtile never straddles two segments, so neither do the 4 columns
    const int u = col0 / 16;
    const int seg = (a.n_seg > 2 && u >= a.seg[2].sub0) ? 2 : ((a.n_seg > 1 && u >= a.seg[1].sub0) ? 1 : 0);
    const int c0 = col0 - PF_SEL(seg, sub0) * 16;
    float* y = PF_SEL(seg, y) + (int64_t)row * PF_SEL(seg, ldy) + c0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (MODE == GEMV_STORE) {
            const float* bias = PF_SEL(seg, bias);
            y[e] = bias ? v[e] + bias[c0 + e] : v[e];
        } else {
            const float nv = y[e] + v[e];
            y[e] = nv;
            if (row == a.tap_row && a.tap) a.tap[c0 + e] = nv;
        }
    }
}

#undef PF_SEL

// k_pf_reduce of the q, k and v segments (GEMV_STORE, K split) fused with
// k_pf_rope_store: thread per rotated pair (j, j + hd / 2) of a q or k head, or per v
// element, of row blockIdx.y. The slices add in slice order and the bias after them, as
// k_pf_reduce does, then the rotation of k_pf_rope_store; q goes back to its segment's
// rows, k and v only to the cache.
template <int KS>
__global__ __launch_bounds__(kBlock) void k_pf_reduce_rope(const PfGemmArgs a) {
    const int i = blockIdx.y, pos = a.pos0 + i;
    const int hd = a.hd, d2 = hd / 2, G = a.n_kv;
    const int nq = a.n_head * d2, nk = G * d2, nv = G * hd;
    const int t = blockIdx.x * kBlock + threadIdx.x;
    if (t >= nq + nk + nv) return;
    const int ntot = a.n_sub * 16;
    const float* p = a.part + (int64_t)i * ntot;
    const int64_t ss = (int64_t)a.Mpad * ntot;
    if (t < nq + nk) {
        const bool isq = t < nq;
        const int u = isq ? t : t - nq, h = u / d2, j = u % d2, c0 = h * hd + j;
        const float* bias = isq ? a.seg[0].bias : a.seg[1].bias;
        const float* ps = p + (isq ? a.seg[0].sub0 : a.seg[1].sub0) * 16 + c0;
        float p0[KS], p1[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            p0[k] = ps[k * ss];
            p1[k] = ps[k * ss + d2];
        }
        float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            x0 += p0[k];
            x1 += p1[k];
        }
        if (bias) {
            x0 = x0 + bias[c0];
            x1 = x1 + bias[c0 + d2];
        }
        const float c = a.rope_cos[(int64_t)pos * d2 + j], s = a.rope_sin[(int64_t)pos * d2 + j];
        const float r0 = fmaf(x0, c, -(x1 * s)), r1 = fmaf(x0, s, x1 * c);
        float* o = isq ? a.seg[0].y + (int64_t)i * a.seg[0].ldy + h * hd
                       : a.kc + kv_offset(a.kv_layout, G, a.max_seq, hd, h, pos);
        o[j] = r0;
        o[j + d2] = r1;
    } else {
        const int u = t - nq - nk, g = u / hd, j = u % hd;
        const float* ps = p + a.seg[2].sub0 * 16 + u;
        float pv[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) pv[k] = ps[k * ss];
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k) v += pv[k];
        if (a.seg[2].bias) v = v + a.seg[2].bias[u];
        a.vc[kv_offset(a.kv_layout, G, a.max_seq, hd, g, pos) + j] = v;
    }
}

// k_pf_reduce of a GEMV_RESID GEMM with one segment, fused with the split of the
// updated rows (k_pf_split with a workgroup per row): thread t owns the 8-column groups
// t, t + 256, ..., adds the KS slices in slice order and then the residual, as
// k_pf_reduce does, stores the row and splits it. Rows M.. get the padding zeros.
template <int KS, int NG>
__global__ __launch_bounds__(kBlock) void k_pf_reduce_split(const PfGemmArgs a) {
    __shared__ double red_d[kWavesPerBlock];
    __shared__ float red_f[kWavesPerBlock];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int K = a.n_sub * 16, ng = K / 8;
    if (m >= a.M) {
        split_zero<kBlock>(tid, m, K, (h8_t*)a.split_xa, a.split_rs);
        return;
    }
    const float* p = a.part + (int64_t)m * K;
    float* y = a.seg[0].y + (int64_t)m * a.seg[0].ldy;
    const int64_t sstride = (int64_t)a.Mpad * K;
    float v[NG][8];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int j = tid + i * kBlock;
        const int jj = j < ng ? j : ng - 1;  // a clamped re-read, masked below
        float4 pv[KS][2];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            pv[k][0] = *(const float4*)(p + k * sstride + 8 * jj);
            pv[k][1] = *(const float4*)(p + k * sstride + 8 * jj + 4);
        }
        const float4 y0 = *(const float4*)(y + 8 * jj), y1 = *(const float4*)(y + 8 * jj + 4);
        float sm[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            sm[0] += pv[k][0].x; sm[1] += pv[k][0].y; sm[2] += pv[k][0].z; sm[3] += pv[k][0].w;
            sm[4] += pv[k][1].x; sm[5] += pv[k][1].y; sm[6] += pv[k][1].z; sm[7] += pv[k][1].w;
        }
        const float yv[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = yv[e] + sm[e];
        if (j < ng) {
            *(float4*)(y + 8 * j) = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
            *(float4*)(y + 8 * j + 4) = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
            if (m == a.tap_row && a.tap)
#pragma unroll
                for (int e = 0; e < 8; ++e) a.tap[8 * j + e] = v[i][e];
        }
    }
    split_emit<NG, 4>(v, tid, m, K, a.split_w, a.split_eps, (h8_t*)a.split_xa, a.split_rs, red_d, red_f);
}


// k_pf_reduce of a GEMV_SILU GEMM (gate columns, then up columns, K split) fused with the
// split of its rows (k_pf_split without a norm, a workgroup per row): thread t owns the
// 8-column groups t, t + 256, ...; each gate and up sum adds the slices in slice order as
// k_pf_reduce does, silu(gate) * up as the GEMM's epilogue computes it, then the row's
// power-of-two scale and its hi + lo fragments. The rows themselves are not stored: only
// the next GEMM reads them, from the fragments. Rows M.. get the padding zeros.
template <int KS, int NG>
__global__ __launch_bounds__(kBlock) void k_pf_reduce_silu_split(const PfGemmArgs a) {
    __shared__ double red_d[kWavesPerBlock];
    __shared__ float red_f[kWavesPerBlock];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int F = a.n_sub * 16, ng = F / 8;
    if (m >= a.M) {
        split_zero<kBlock>(tid, m, F, (h8_t*)a.split_xa, a.split_rs);
        return;
    }
    const float* p = a.part + (int64_t)m * 2 * F;
    const int64_t sstride = (int64_t)a.Mpad * 2 * F;
    float v[NG][8];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int j = tid + i * kBlock;
        const int jj = j < ng ? j : ng - 1;  // a clamped re-read, masked in the split
        float g[8] = {0, 0, 0, 0, 0, 0, 0, 0}, u[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float4 pv[KS][2];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            pv[k][0] = *(const float4*)(p + k * sstride + 8 * jj);
            pv[k][1] = *(const float4*)(p + k * sstride + 8 * jj + 4);
        }
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            g[0] += pv[k][0].x; g[1] += pv[k][0].y; g[2] += pv[k][0].z; g[3] += pv[k][0].w;
            g[4] += pv[k][1].x; g[5] += pv[k][1].y; g[6] += pv[k][1].z; g[7] += pv[k][1].w;
        }
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            pv[k][0] = *(const float4*)(p + F + k * sstride + 8 * jj);
            pv[k][1] = *(const float4*)(p + F + k * sstride + 8 * jj + 4);
        }
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            u[0] += pv[k][0].x; u[1] += pv[k][0].y; u[2] += pv[k][0].z; u[3] += pv[k][0].w;
            u[4] += pv[k][1].x; u[5] += pv[k][1].y; u[6] += pv[k][1].z; u[7] += pv[k][1].w;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = (g[e] / (1.0f + expf(-g[e]))) * u[e];
    }
    split_emit<NG, 4>(v, tid, m, F, nullptr, 0.0f, (h8_t*)a.split_xa, a.split_rs, red_d, red_f);
}

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
//
// Both products of attention run on v_mfma_f32_16x16x32_f16 with every fp32 operand as an
// fp16 pair hi + lo (22 significant bits): x . y = hi_x hi_y + hi_x lo_y + lo_x hi_y, the
// dropped lo_x lo_y being 2^-22 of the product. Rows are scaled by powers of two so that
// hi and lo stay in fp16 range and off its subnormals (max |row| in [2^14, 2^15)), and
// the scales come back out exactly:
//   S^T = K Q^T: each key row k_j by 2^ek_j, each query row by 2^eq; a score is the
//     product times 2^-(ek_j + eq) / sqrt(hd).
//   O^T = V^T P^T: each value row v_j by 2^ev_j; the probability p_ij enters as
//     p_ij 2^(e_i - ev_j), with e_i per query and tile putting the largest of the tile's
//     p_ij 2^-ev_j in [2^14, 2^15): the tile's products come out in units of 2^e_i, the
//     query's running output carries its unit and is rescaled by 2^(e_i - unit) with the
//     softmax's exp(m_old - m_new). Each term keeps 22 bits down to 2^-18 of the tile's
//     largest term |p v| (below that, fp16's subnormal step: at most 2^-40 of it).
// k_pf_pack_kv writes each 32-key tile of a kv head once per layer, already in fragment
// order and scaled (a tile record); k_pf_attn's workgroups stage the records through LDS,
// shared by the query heads of the kv head.

constexpr int kAttnTile = 32;  // keys per tile record

// Max and sum of v over lanes l, l ^ 16, l ^ 32, l ^ 48 (the 4 lanes of one query in the
// MFMA layout) with gfx950's lane swaps, no LDS: a swap leaves each lane its own value in
// one register and its partner's in the other, and every lane adds the lower lane's value
// first, so the 4 lanes get the same bits.
__device__ __forceinline__ float quad_max(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const uint32_t w = __float_as_uint(m);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float quad_sum(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const uint32_t w = __float_as_uint(s);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Tile record of head size HD: K fragments [16-key half][32-dim chunk][hi, lo][lane][8],
// V^T fragments [16-dim tile][hi, lo][lane][8], then 2^-ek_j [32] and 2^-ev_j [32] (0 for
// a zero value row).
// A V^T fragment's lane l holds dim l % 16 and the 8 keys of P^T's lane l: keys
// 4 (l / 16) + 0..3 and 16 + 4 (l / 16) + 0..3, the keys whose scores S^T leaves there.
__host__ __device__ constexpr int attn_rec_bytes(int hd) { return 256 * hd + 512; }
// A record's LDS buffer in k_pf_attn: whole 1 KiB slots (the DMA granule of a wave)
__host__ __device__ constexpr int attn_buf_bytes(int hd) { return (attn_rec_bytes(hd) + 1023) / 1024 * 1024; }
// LDS record buffers of k_pf_attn per key-tile stream: one in use, one loading. With two
// (66 KiB for head size 128) two workgroups share a CU, which measured faster than three or
// four buffers (loads two or three tiles ahead) with one workgroup per CU.
constexpr int kAttnBufs = 2;

constexpr int kZeroRow = 1000;  // row exponent of an all-zero row

__device__ __forceinline__ int pow2_exp(float amax, int if_zero) {
    int ex = 0;
    (void)frexpf(amax, &ex);  // amax = f 2^ex, f in [0.5, 1)
    int e = amax > 0.0f ? 15 - ex : if_zero;
    return e < -100 ? -100 : (e > 100 ? 100 : e);
}

// Grid (tiles, kv heads), 256 threads: tile t of kv head g covers positions key0 + 32 t ..;
// positions past key0 + n_keys are zero rows.
template <int HD>
__global__ __launch_bounds__(kBlock) void k_pf_pack_kv(const float* kc, const float* vc, int layout, int G,
                                                       int max_seq, int key0, int n_keys, unsigned char* recs) {
    constexpr int NC = HD / 32;
    __shared__ float ks[kAttnTile][HD + 1], vs[kAttnTile][HD + 1];
    __shared__ int ex[2][kAttnTile];
    const int t = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    unsigned char* rec = recs + ((int64_t)g * gridDim.x + t) * attn_rec_bytes(HD);
    for (int i = tid; i < kAttnTile * HD / 4; i += kBlock) {
        const int key = i / (HD / 4), d = 4 * (i % (HD / 4));
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
        if (kAttnTile * t + key < n_keys) {
            const int64_t o = kv_offset(layout, G, max_seq, HD, g, key0 + kAttnTile * t + key) + d;
            a = gload_f4(kc + o);
            b = gload_f4(vc + o);
        }
        ks[key][d] = a.x; ks[key][d + 1] = a.y; ks[key][d + 2] = a.z; ks[key][d + 3] = a.w;
        vs[key][d] = b.x; vs[key][d + 1] = b.y; vs[key][d + 2] = b.z; vs[key][d + 3] = b.w;
    }
    __syncthreads();
    {  // row exponents: 4 threads per (K or V, key)
        const int which = tid >> 7, key = (tid >> 2) & 31, part = tid & 3;
        const float* row = which ? vs[key] : ks[key];
        float m = 0.0f;
        for (int d = part; d < HD; d += 4) m = fmaxf(m, fabsf(row[d]));
        m = fmaxf(m, __shfl_xor(m, 1));
        m = fmaxf(m, __shfl_xor(m, 2));
        if (part == 0) ex[which][key] = m > 0.0f ? pow2_exp(m, 0) : kZeroRow;
    }
    __syncthreads();
    h8_t* kf = (h8_t*)rec;
    for (int i = tid; i < 2 * NC * 64; i += kBlock) {
        const int lane = i & 63, hc = i >> 6;
        const int key = 16 * (hc / NC) + (lane & 15), d0 = 32 * (hc % NC) + 8 * (lane >> 4);
        const float sc = ex[0][key] == kZeroRow ? 0.0f : ldexpf(1.0f, ex[0][key]);
        h8_t hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float x = ks[key][d0 + j] * sc;
            hi[j] = (_Float16)x;
            lo[j] = (_Float16)(x - (float)hi[j]);
        }
        kf[hc * 128 + lane] = hi;
        kf[hc * 128 + 64 + lane] = lo;
    }
    h8_t* vf = (h8_t*)(rec + 128 * HD);
    for (int i = tid; i < (HD / 16) * 64; i += kBlock) {
        const int lane = i & 63, dt = i >> 6;
        const int d = 16 * dt + (lane & 15), k0 = 4 * (lane >> 4);
        h8_t hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int key = (j < 4 ? k0 : 16 + k0 - 4) + j;
            const float x = ex[1][key] == kZeroRow ? 0.0f : vs[key][d] * ldexpf(1.0f, ex[1][key]);
            hi[j] = (_Float16)x;
            lo[j] = (_Float16)(x - (float)hi[j]);
        }
        vf[dt * 128 + lane] = hi;
        vf[dt * 128 + 64 + lane] = lo;
    }
    float* fk = (float*)(rec + 256 * HD);
    if (tid < kAttnTile) {
        fk[tid] = ex[0][tid] == kZeroRow ? 0.0f : ldexpf(1.0f, -ex[0][tid]);
        fk[kAttnTile + tid] = ex[1][tid] == kZeroRow ? 0.0f : ldexpf(1.0f, -ex[1][tid]);
    }
}

// Workgroup: QG query blocks of 16 QS queries of one kv head, times its n_rep query
// heads, times KS key streams: wave w takes head w' % n_rep of block w' / n_rep and the key
// tiles t = KS i + w / (n_rep QG), w' = w % (n_rep QG) (4 to 8 waves). With KS = 2 the two
// waves of a head and block each run an online softmax over alternate tiles, which halves
// the longest block's chain of tiles, and merge through LDS at the end. Per tile record
// (loaded into LDS ahead of its use) a wave computes, for
// each of its 16-query subtiles, S^T of 32 keys (lane l: query l % 16, keys 4 (l / 16) + r
// and 16 + 4 (l / 16) + r), the online softmax of those scores, and O^T += V^T P^T with
// P^T straight from the same lanes. Keys run from att_start to the workgroup's last query;
// keys past a query's position score -inf.
template <int HD, int QS, int KS>
__global__ __launch_bounds__(512) void k_pf_attn(const float* q, int64_t ldq, const unsigned char* recs, int T,
                                                 int n_rep, int QG, int n, int pos0, int att_start, float* out,
                                                 int64_t ldo, int G) {
    extern __shared__ uint4 lds_rec[];
    constexpr int NC = HD / 32, NT = HD / 16;
    constexpr int kSlots = attn_buf_bytes(HD) / 1024, RB = attn_buf_bytes(HD), RBYTES = attn_rec_bytes(HD);
    const int tid = threadIdx.x, lane = tid & 63, nthr = blockDim.x;
    const int w = tid >> 6;
    // waves per key stream, this wave's stream and its place in it
    const int nhw = n_rep * QG, khalf = KS > 1 ? w / nhw : 0, wq = KS > 1 ? w % nhw : w;
    // query blocks in order of decreasing length over all kv heads (the kv head fastest), so
    // the longest start first: 4096-token prompt 38.64 -> 38.34 ms against the heads one
    // after the other
    const int g = (int)blockIdx.x % G, h = g * n_rep + wq % n_rep;
    const int blk = (int)gridDim.x / G - 1 - (int)blockIdx.x / G;
    const int q_base = (blk * QG + wq / n_rep) * 16 * QS;
    const int wg_last = min(n - 1, (blk + 1) * QG * 16 * QS - 1);
    const int n_tiles = (pos0 + wg_last - att_start) / kAttnTile + 1;
    const int q_first = __builtin_amdgcn_readfirstlane(pos0 + min(q_base, n - 1));  // the wave's first query
    const int l16 = lane & 15, gq = lane >> 4;
    const float scale = 1.0f / sqrtf((float)HD);

    // Records go straight from global memory into the kAttnBufs KS LDS buffers
    // (global_load_lds, 1 KiB per wave instruction), one step of KS tiles ahead, so no
    // registers hold records in flight. Wave w loads the record's 1 KiB slots w + nw i,
    // i < dpw: slot indices past the last re-load it, lanes past the record's end re-read its
    // last 16 bytes into the buffer's padding, and loads past the last tile re-load it. Load
    // i (tile min(i, n_tiles - 1)) goes to buffer i % nbuf.
    const int nbuf = kAttnBufs * KS;
    const int nw = nthr >> 6, dpw = (kSlots + nw - 1) / nw;
    const unsigned char* src = recs + (int64_t)g * T * RBYTES;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds_rec;
    auto issue = [&](int i) {
        const unsigned char* rec = src + (int64_t)(i < n_tiles ? i : n_tiles - 1) * RBYTES;
        const uint32_t base = lds0 + (uint32_t)((i % nbuf) * RB);
        for (int k = 0; k < dpw; ++k) {
            const int j = min(w + nw * k, kSlots - 1);
            const int off = min(j * 1024 + lane * 16, RBYTES - 16);
            lds_dma16((const TF_GLOBAL unsigned char*)rec + off, __builtin_amdgcn_readfirstlane(base + (uint32_t)(j * 1024)));
        }
    };
    for (int i = 0; i < KS; ++i) issue(i);

    h8_t qh[QS][NC], ql[QS][NC];
    float fq[QS];
    int qpos[QS];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        const int qi = q_base + 16 * qs + l16;
        const int qrow = qi < n ? qi : n - 1;
        qpos[qs] = pos0 + qrow;
        const float* qr = q + (int64_t)qrow * ldq + (int64_t)h * HD + 8 * gq;
        float v[NC][8];
        float amax = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float4 a = gload_f4(qr + 32 * c), b = gload_f4(qr + 32 * c + 4);
            v[c][0] = a.x; v[c][1] = a.y; v[c][2] = a.z; v[c][3] = a.w;
            v[c][4] = b.x; v[c][5] = b.y; v[c][6] = b.z; v[c][7] = b.w;
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[c][j]));
        }
        amax = quad_max(amax);
        const int e = pow2_exp(amax, 0);
        const float sc = ldexpf(1.0f, e);
        fq[qs] = ldexpf(scale, -e) * 1.44269504088896341f;  // the scores in units of log2
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = v[c][j] * sc;
                qh[qs][c][j] = (_Float16)x;
                ql[qs][c][j] = (_Float16)(x - (float)qh[qs][c][j]);
            }
    }
    f4_t acc[QS][NT];
    float m_run[QS], l_run[QS];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        m_run[qs] = -INFINITY;
        l_run[qs] = 0.0f;
#pragma unroll
        for (int d = 0; d < NT; ++d) acc[qs][d] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};
    }
    int unit[QS];  // acc holds O times 2^unit (times l_run), per query
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) unit[qs] = 0;

    auto tile = [&](const unsigned char* rec, int t) {
        const h8_t* kf = (const h8_t*)rec;
        const h8_t* vf = (const h8_t*)(rec + 128 * HD);
        const float* fk = (const float*)(rec + 256 * HD);
        // every K and V fragment of the tile is read up front: the V reads complete under
        // the q.k MFMAs (the softmax's branches would otherwise leave each pair of them to
        // be read, and waited for, right before its MFMAs)
        h8_t kr[NC][2][2], vr[NT][2];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                kr[c][half][0] = kf[(half * NC + c) * 128 + lane];
                kr[c][half][1] = kf[(half * NC + c) * 128 + 64 + lane];
            }
#pragma unroll
        for (int d = 0; d < NT; ++d) {
            vr[d][0] = vf[d * 128 + lane];
            vr[d][1] = vf[d * 128 + 64 + lane];
        }
        f4_t s[QS][2];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) s[qs][0] = s[qs][1] = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const h8_t kh = kr[c][half][0], kl = kr[c][half][1];
#pragma unroll
                for (int qs = 0; qs < QS; ++qs) {
                    f4_t x = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[qs][c], s[qs][half], 0, 0, 0);
                    x = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[qs][c], x, 0, 0, 0);
                    s[qs][half] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[qs][c], x, 0, 0, 0);
                }
            }
#pragma unroll
        for (int d = 0; d < NT; ++d) asm volatile("" : "+v"(vr[d][0]), "+v"(vr[d][1]));
        const float4 k0 = *(const float4*)(fk + 4 * gq), k1 = *(const float4*)(fk + 16 + 4 * gq);
        const float4 v0 = *(const float4*)(fk + kAttnTile + 4 * gq), v1 = *(const float4*)(fk + kAttnTile + 16 + 4 * gq);
        const float fkj[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        const float fvj[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        const int kpos = att_start + kAttnTile * t + 4 * gq;  // key j of the lane: kpos + 16 (j / 4) + j % 4
        // keys past a query only where the tile reaches past the wave's first query
        const bool masked = att_start + kAttnTile * t + kAttnTile - 1 > q_first;
        h8_t ph[QS], pl[QS];
        float resc[QS];
        int unit_new[QS];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
            float p[8];
            float mt = -INFINITY;
#pragma unroll
            for (int j = 0; j < 8; ++j) p[j] = s[qs][j >> 2][j & 3] * fq[qs] * fkj[j];
            if (masked) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (kpos + 16 * (j >> 2) + (j & 3) > qpos[qs]) p[j] = -INFINITY;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) mt = fmaxf(mt, p[j]);
            mt = quad_max(mt);
            // scores are in units of log2 (fq carries log2 e): 2^(x - m) is exp of the score
            // difference; every query has a key in tile 0 (att_start <= its position), so
            // m_new is finite from the first tile on
            // (a second key stream's first tiles can hold no key of a query: m_new stays -inf
            // and the exps take 0 as the reference, so that alpha and p are 0, not NaN)
            const float m_new = fmaxf(m_run[qs], mt);
            const float m_ref = KS > 1 && m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run[qs] - m_ref);  // 0 on the first tile
            float ls = 0.0f, x[8], mx = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                p[j] = __builtin_amdgcn_exp2f(p[j] - m_ref);  // 0 for a masked key
                ls += p[j];
                x[j] = p[j] * fvj[j];
                mx = fmaxf(mx, x[j]);
            }
            ls = quad_sum(ls);
            mx = quad_max(mx);
            l_run[qs] = fmaf(l_run[qs], alpha, ls);
            m_run[qs] = m_new;
            // the tile's unit: the running one while it keeps the tile's largest term in
            // [2^7, 2^15) (so the output needs no rescaling when the max holds), else the one
            // putting it in [2^14, 2^15); no change when the tile adds nothing, and never so
            // far above the running unit that the rescaled output (below 2^43 in its unit,
            // times alpha) could leave fp32's range
            int e = unit[qs];
            if (mx > 0.0f) {
                const int fit = 15 - __builtin_amdgcn_frexp_expf(mx);
                if (fit < unit[qs] || fit > unit[qs] + 7) {
                    e = fit;
                    if (alpha > 0.0f) e = min(e, unit[qs] + 76 - __builtin_amdgcn_frexp_expf(alpha));
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float y = ldexpf(x[j], e);
                ph[qs][j] = (_Float16)y;
                pl[qs][j] = (_Float16)(y - (float)ph[qs][j]);
            }
            resc[qs] = ldexpf(alpha, e - unit[qs]);
            unit_new[qs] = e;
        }
        bool scaled = false;  // some lane's output changes scale (max or unit): rescale all
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
            unit[qs] = unit_new[qs];
            scaled = scaled || resc[qs] != 1.0f;
        }
        if (__builtin_amdgcn_ballot_w64(scaled) != 0)
#pragma unroll
            for (int qs = 0; qs < QS; ++qs)
#pragma unroll
                for (int d = 0; d < NT; ++d) acc[qs][d] = acc[qs][d] * resc[qs];
#pragma unroll
        for (int d = 0; d < NT; ++d) {
            const h8_t vh = vr[d][0], vl = vr[d][1];
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
                f4_t x = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph[qs], acc[qs][d], 0, 0, 0);
                x = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl[qs], x, 0, 0, 0);
                acc[qs][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph[qs], x, 0, 0, 0);
            }
        }
    };

    // this wave's loads of a step's tiles are done (the only ones in flight); the barrier
    // then makes every wave's done, and every wave has left the step before, whose buffers
    // the loads of the next step take
    static_assert(kAttnBufs == 2, "the wait counts no loads issued after a step's own");
    if constexpr (KS == 1) {
        for (int t = 0; t < n_tiles; ++t) {
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            issue(t + 1);
            tile((const unsigned char*)lds_rec + (t % nbuf) * RB, t);
        }
    } else {
        for (int it = 0; it * KS < n_tiles; ++it) {
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
            for (int k = 0; k < KS; ++k) issue(KS * (it + 1) + k);
            const int t = KS * it + khalf;
            if (t < n_tiles) tile((const unsigned char*)lds_rec + (t % nbuf) * RB, t);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the re-loads past the last tile
    if constexpr (KS > 1) {
        // the second stream's waves hand their state (O times 2^unit l, m, l, unit) to the
        // first's through LDS; O = (A0 2^(m0 - M) + A1 2^(m1 - M)) / (l0 2^(m0 - M) + l1 2^(m1 - M))
        // with A = acc 2^-unit and M = max(m0, m1) (m0 is finite: tile 0 is the first stream's)
        constexpr int MW = (4 * NT + 3) * QS;
        static_assert(4 * 64 * MW * 4 <= 2 * kAttnBufs * attn_buf_bytes(HD), "at most 4 waves per stream");
        float* mg = (float*)lds_rec;  // [wave of the first stream][lane][MW]
        __syncthreads();
        if (khalf == 1) {
            float* d = mg + ((int64_t)wq * 64 + lane) * MW;
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
#pragma unroll
                for (int dt = 0; dt < NT; ++dt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) d[(qs * NT + dt) * 4 + r] = acc[qs][dt][r];
                d[4 * NT * QS + 3 * qs] = m_run[qs];
                d[4 * NT * QS + 3 * qs + 1] = l_run[qs];
                d[4 * NT * QS + 3 * qs + 2] = (float)unit[qs];
            }
        }
        __syncthreads();
        if (khalf == 1) return;
        const float* sp = mg + ((int64_t)wq * 64 + lane) * MW;
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
            const float m1 = sp[4 * NT * QS + 3 * qs], l1 = sp[4 * NT * QS + 3 * qs + 1];
            const int u1 = (int)sp[4 * NT * QS + 3 * qs + 2];
            const float M = fmaxf(m_run[qs], m1);
            const float f0 = __builtin_amdgcn_exp2f(m_run[qs] - M), f1 = __builtin_amdgcn_exp2f(m1 - M);
            const float L = fmaf(l_run[qs], f0, l1 * f1);
            const float c0 = ldexpf(f0 / L, -unit[qs]), c1 = ldexpf(f1 / L, -u1);
#pragma unroll
            for (int dt = 0; dt < NT; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[qs][dt][r] = fmaf(acc[qs][dt][r], c0, sp[(qs * NT + dt) * 4 + r] * c1);
            l_run[qs] = 1.0f;  // acc now holds the normalised output
            unit[qs] = 0;
        }
    }
    // lane holds O[query l16][dims 16 d + 4 gq + 0..3] times 2^unit l_run
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        const int qi = q_base + 16 * qs + l16;
        if (qi >= n) continue;
        float* orow = out + (int64_t)qi * ldo + (int64_t)h * HD + 4 * gq;
        const float il = ldexpf(1.0f / l_run[qs], -unit[qs]);
#pragma unroll
        for (int d = 0; d < NT; ++d)
            *(float4*)(orow + 16 * d) =
                make_float4(acc[qs][d][0] * il, acc[qs][d][1] * il, acc[qs][d][2] * il, acc[qs][d][3] * il);
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
    const bool fmt = type == TF_HIP_TYPE_Q8_0 || type == TF_HIP_TYPE_Q4_0 || type == TF_HIP_TYPE_Q4_1 ||
                     type == TF_HIP_TYPE_F16 || type == TF_HIP_TYPE_F32 || type == TF_HIP_TYPE_Q6_K;
    return fmt && K % 64 == 0 && N % 16 == 0 && K <= kBlock * 8 * kSplitGroups &&
           (type != TF_HIP_TYPE_Q6_K || K % 256 == 0);
}

hipError_t launch_pf_split(const float* x, int64_t ldx, const float* norm_w, float eps, int K, int M, int Mpad,
                           uint16_t* xa, float* rs, hipStream_t st) {
    if (K % 32 != 0 || K > kBlock * 8 * kSplitGroups || ldx % 4 != 0 || Mpad % kPfTileM != 0 || M > Mpad)
        return hipErrorInvalidValue;
    // a wave per row while a lane holds at most 20 groups (rows up to 10240), else a workgroup
    const int per1 = (K / 8 + 63) / 64;
#define TF_SPLIT(NG, WPR, rows)                                                                              \
    hipLaunchKernelGGL((k_pf_split<NG, WPR>), dim3((unsigned)(Mpad / (rows))), dim3(kBlock), 0, st, x, ldx, \
                       norm_w, eps, K, M, (h8_t*)xa, rs)
    if (per1 <= 2)
        TF_SPLIT(2, 1, kWavesPerBlock);
    else if (per1 <= 4)
        TF_SPLIT(4, 1, kWavesPerBlock);
    else if (per1 <= 8)
        TF_SPLIT(8, 1, kWavesPerBlock);
    else if (per1 <= 16)
        TF_SPLIT(16, 1, kWavesPerBlock);
    else if (per1 <= 20)
        TF_SPLIT(20, 1, kWavesPerBlock);
    else
        TF_SPLIT(kSplitGroups, 4, 1);  // per4 <= 8: K was checked above
#undef TF_SPLIT
    return hipGetLastError();
}

namespace {

// The reduce of a GEMM whose K ran in ks slices (2, 4, 8 or 16; partial sums in b.part): the
// QKV reduce fused with RoPE and the cache store, the residual reduce fused with the next
// GEMM's activation split, or the plain reduce; *fused says whether the fused work ran.
hipError_t launch_split_reduce(const PfGemmArgs& a, int ks, hipStream_t st, bool* fused) {
    hipError_t e = hipSuccess;
    if (a.mode == GEMV_STORE && a.rope_cos && a.rope_sin && a.kc && a.vc && a.n_seg == 3 && a.hd % 2 == 0 &&
        a.seg[0].w.N == (int64_t)a.n_head * a.hd && a.seg[1].w.N == (int64_t)a.n_kv * a.hd &&
        a.seg[2].w.N == (int64_t)a.n_kv * a.hd) {
        const int items = (a.n_head + a.n_kv) * (a.hd / 2) + a.n_kv * a.hd;
        const dim3 qgrid((unsigned)((items + kBlock - 1) / kBlock), (unsigned)a.M);
#define PF_RROPE(KS) hipLaunchKernelGGL((k_pf_reduce_rope<KS>), qgrid, dim3(kBlock), 0, st, a)
        switch (ks) {
            case 2: PF_RROPE(2); break;
            case 4: PF_RROPE(4); break;
            case 8: PF_RROPE(8); break;
            case 16: PF_RROPE(16); break;
            default: return hipErrorInvalidValue;
        }
#undef PF_RROPE
        e = hipGetLastError();
        if (e == hipSuccess && fused) *fused = true;
        return e;
    }
    const int ngr = a.n_sub * 2;  // 8-column groups of an output row
    if (a.mode == GEMV_RESID && a.split_xa && a.split_rs && a.n_seg == 1 && a.seg[0].ldy % 4 == 0 && a.seg[0].ldy >= ngr * 8 &&
        ((uintptr_t)a.seg[0].y & 15) == 0 && ngr <= 4 * kBlock) {
        const int ng = ngr <= kBlock ? 1 : (ngr <= 2 * kBlock ? 2 : 4);
#define PF_RSPLIT(KS, NG) hipLaunchKernelGGL((k_pf_reduce_split<KS, NG>), dim3((unsigned)a.Mpad), dim3(kBlock), 0, st, a)
        switch (ks * 8 + ng) {  // ks is 2, 4, 8 or 16 here
            case 17: PF_RSPLIT(2, 1); break;
            case 18: PF_RSPLIT(2, 2); break;
            case 20: PF_RSPLIT(2, 4); break;
            case 33: PF_RSPLIT(4, 1); break;
            case 34: PF_RSPLIT(4, 2); break;
            case 36: PF_RSPLIT(4, 4); break;
            case 65: PF_RSPLIT(8, 1); break;
            case 66: PF_RSPLIT(8, 2); break;
            case 68: PF_RSPLIT(8, 4); break;
            case 129: PF_RSPLIT(16, 1); break;
            case 130: PF_RSPLIT(16, 2); break;
            case 132: PF_RSPLIT(16, 4); break;
            default: return hipErrorInvalidValue;
        }
#undef PF_RSPLIT
        e = hipGetLastError();
        if (e == hipSuccess && fused) *fused = true;
        return e;
    }
    const int ngs = a.n_sub * 2 <= kBlock ? 1 : (a.n_sub * 2 <= 2 * kBlock ? 2 : (a.n_sub * 2 <= 4 * kBlock ? 4 : 8));
    // (a thread's partial loads, ks x groups, kept to 16 so that they stay in registers)
    if (a.mode == GEMV_SILU && a.split_xa && a.split_rs && a.n_sub * 2 <= 8 * kBlock && ks * ngs <= 16) {
        const int ng = ngs;  // 8-column groups of an output row per thread
#define PF_RSS(KS, NG) hipLaunchKernelGGL((k_pf_reduce_silu_split<KS, NG>), dim3((unsigned)a.Mpad), dim3(kBlock), 0, st, a)
        switch (ks * 16 + ng) {  // ks is 2, 4, 8 or 16 here
            case 33: PF_RSS(2, 1); break;
            case 34: PF_RSS(2, 2); break;
            case 36: PF_RSS(2, 4); break;
            case 40: PF_RSS(2, 8); break;
            case 65: PF_RSS(4, 1); break;
            case 66: PF_RSS(4, 2); break;
            case 68: PF_RSS(4, 4); break;
            case 129: PF_RSS(8, 1); break;
            case 130: PF_RSS(8, 2); break;
            case 257: PF_RSS(16, 1); break;
            default: return hipErrorInvalidValue;
        }
#undef PF_RSS
        const hipError_t e = hipGetLastError();
        if (e == hipSuccess && fused) *fused = true;
        return e;
    }
    const dim3 rgrid((unsigned)((a.n_sub * 4 + kBlock - 1) / kBlock), (unsigned)a.M);
#define PF_REDUCE(MODE, KS) hipLaunchKernelGGL((k_pf_reduce<MODE, KS>), rgrid, dim3(kBlock), 0, st, a)
    switch (a.mode * 32 + ks) {  // ks is 2, 4, 8 or 16 here
        case 2: PF_REDUCE(GEMV_STORE, 2); break;
        case 4: PF_REDUCE(GEMV_STORE, 4); break;
        case 8: PF_REDUCE(GEMV_STORE, 8); break;
        case 16: PF_REDUCE(GEMV_STORE, 16); break;
        case 34: PF_REDUCE(GEMV_RESID, 2); break;
        case 36: PF_REDUCE(GEMV_RESID, 4); break;
        case 40: PF_REDUCE(GEMV_RESID, 8); break;
        case 48: PF_REDUCE(GEMV_RESID, 16); break;
        case 66: PF_REDUCE(GEMV_SILU, 2); break;
        case 68: PF_REDUCE(GEMV_SILU, 4); break;
        case 72: PF_REDUCE(GEMV_SILU, 8); break;
        case 80: PF_REDUCE(GEMV_SILU, 16); break;
        default: return hipErrorInvalidValue;
    }
#undef PF_REDUCE
    return hipGetLastError();
}

// Row counts up to which the register-streamed tiles put all four waves along the columns
// (33-64 rows as two 32-row tiles measured the same as one 64-row tile).
constexpr int kSmallRows = 32;

// The launch of launch_pf_gemm for weights of format T (arguments checked).
template <int T>
hipError_t launch_gemm_t(const PfGemmArgs& a, hipStream_t st, bool* fused) {
    // large tiles when they give every CU a workgroup, directly or with K split in slices
    if (a.Mpad % kBigRows == 0) {
        const int per_big = a.mode == GEMV_SILU ? 8 : 16;  // output subtiles per large tile
        const int n_big = (a.n_sub + per_big - 1) / per_big * (a.Mpad / kBigRows);
        const int cus = device_cu_count();
        int ks = 1;
        bool big = n_big >= cus;
        if (!big && a.part) {
            // K slices by the span they give: rounds of workgroups over the CUs times
            // stages per slice; the fewest slices with the shortest span (each split adds
            // its reduce), each slice at least 8 stages long (shorter slices spend more on
            // filling their pipeline and on the partial rows they write than they save), or
            // 4 when that fits the CUs in one round. Big tiles when at least half the CUs
            // get one.
            const int S = a.K / 64;
            const size_t per_slice = (size_t)a.Mpad * a.n_sub * 16 * (a.mode == GEMV_SILU ? 2 : 1);
            int64_t best = (int64_t)((n_big + cus - 1) / cus) * S;
            for (int k = 2; k <= 16; k *= 2) {
                if (S % k != 0 || S / k < 4 || (S / k < 8 && n_big * k > cus) ||
                    (size_t)k * per_slice > a.part_floats)
                    break;
                const int64_t span = (int64_t)((n_big * k + cus - 1) / cus) * (S / k);
                if (span < best) {
                    best = span;
                    ks = k;
                }
            }
            big = 2 * n_big * ks >= cus;
        }
        if (big) {
            static bool attr_set[6] = {false, false, false, false, false, false};
            const void* fns[6] = {(const void*)k_pf_gemm_big<GEMV_STORE, false, T>,
                                  (const void*)k_pf_gemm_big<GEMV_RESID, false, T>,
                                  (const void*)k_pf_gemm_big<GEMV_SILU, false, T>,
                                  (const void*)k_pf_gemm_big<GEMV_STORE, true, T>,
                                  (const void*)k_pf_gemm_big<GEMV_RESID, true, T>,
                                  (const void*)k_pf_gemm_big<GEMV_SILU, true, T>};
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
                case 0: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_STORE, false, T>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                case 1: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_RESID, false, T>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                case 2: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_SILU, false, T>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                case 3: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_STORE, true, T>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                case 4: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_RESID, true, T>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
                default: hipLaunchKernelGGL((k_pf_gemm_big<GEMV_SILU, true, T>), grid, dim3(kBigThreads), kBigLdsBytes, st, b); break;
            }
            hipError_t e = hipGetLastError();
            if (e != hipSuccess || ks == 1) return e;
            return launch_split_reduce(b, ks, st, fused);
        }
    }
    // 64-row tiles with two waves along the rows, or, for at most 32 rows, tiles of 16 rows
    // (at most 16) or 32 with all four waves along the columns (fewer activation reads per
    // weight byte); 4 column subtiles per wave, 2 when that leaves fewer than two workgroups
    // per CU
    const int cus = device_cu_count();
    const int shape = a.M <= 16 ? 1 : (a.M <= kSmallRows ? 2 : 0);  // 16-row, 32-row or 64-row tiles
    const int mt = shape == 0 ? a.Mpad / kPfTileM : (a.M + 16 * shape - 1) / (16 * shape);
    const int wcols = shape ? 4 : 2;  // waves along the columns
    const int out4 = a.mode == GEMV_SILU ? 2 : 4;
    const int wg4 = (a.n_sub + wcols * out4 - 1) / (wcols * out4) * mt;
    const int ni = wg4 >= 2 * cus ? 4 : 2;
    const int per_wg = wcols * (a.mode == GEMV_SILU ? ni / 2 : ni);  // output subtiles per workgroup column
    const int n_wg = (a.n_sub + per_wg - 1) / per_wg * mt;
    // Few tiles (a short prompt: every weight byte is read once whatever the row count, so
    // the time is the weight stream's): K in slices too, by the same span rule with two
    // workgroups per CU, slices of at least 2 stages (4 blocks)
    int ks = 1;
    if (n_wg < 2 * cus && a.part) {
        const int S = a.K / 64, slots = 2 * cus;
        const size_t per_slice = (size_t)a.Mpad * a.n_sub * 16 * (a.mode == GEMV_SILU ? 2 : 1);
        int64_t best = (int64_t)((n_wg + slots - 1) / slots) * S;
        for (int k = 2; k <= 16; k *= 2) {
            if (S % k != 0 || S / k < 2 || (size_t)k * per_slice > a.part_floats) break;
            const int64_t span = (int64_t)((n_wg * k + slots - 1) / slots) * (S / k);
            if (span < best) {
                best = span;
                ks = k;
            }
        }
    }
    PfGemmArgs b = a;
    b.ks = ks;
    const dim3 grid((unsigned)(n_wg * ks));
#define PF_LAUNCH(MODE, NI, SP)                                                                      \
    do {                                                                                           \
        if (shape == 1)                                                                            \
            hipLaunchKernelGGL((k_pf_gemm_tile<MODE, NI, T, SP, 1, 1>), grid, dim3(256), 0, st, b); \
        else if (shape == 2)                                                                       \
            hipLaunchKernelGGL((k_pf_gemm_tile<MODE, NI, T, SP, 2, 1>), grid, dim3(256), 0, st, b); \
        else                                                                                       \
            hipLaunchKernelGGL((k_pf_gemm_tile<MODE, NI, T, SP, 2, 2>), grid, dim3(256), 0, st, b); \
    } while (0)
    switch (a.mode * 16 + ni * 2 + (ks > 1 ? 1 : 0)) {
        case GEMV_STORE * 16 + 8: PF_LAUNCH(GEMV_STORE, 4, false); break;
        case GEMV_STORE * 16 + 4: PF_LAUNCH(GEMV_STORE, 2, false); break;
        case GEMV_STORE * 16 + 9: PF_LAUNCH(GEMV_STORE, 4, true); break;
        case GEMV_STORE * 16 + 5: PF_LAUNCH(GEMV_STORE, 2, true); break;
        case GEMV_RESID * 16 + 8: PF_LAUNCH(GEMV_RESID, 4, false); break;
        case GEMV_RESID * 16 + 4: PF_LAUNCH(GEMV_RESID, 2, false); break;
        case GEMV_RESID * 16 + 9: PF_LAUNCH(GEMV_RESID, 4, true); break;
        case GEMV_RESID * 16 + 5: PF_LAUNCH(GEMV_RESID, 2, true); break;
        case GEMV_SILU * 16 + 8: PF_LAUNCH(GEMV_SILU, 4, false); break;
        case GEMV_SILU * 16 + 4: PF_LAUNCH(GEMV_SILU, 2, false); break;
        case GEMV_SILU * 16 + 9: PF_LAUNCH(GEMV_SILU, 4, true); break;
        case GEMV_SILU * 16 + 5: PF_LAUNCH(GEMV_SILU, 2, true); break;
        default: return hipErrorInvalidValue;
    }
#undef PF_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || ks == 1) return e;
    return launch_split_reduce(b, ks, st, fused);
}

}  // namespace

hipError_t launch_pf_gemm(const PfGemmArgs& a, hipStream_t st, bool* fused) {
    if (fused) *fused = false;
    if (a.K % 64 != 0 || a.Mpad % kPfTileM != 0 || a.M > a.Mpad || a.M <= 0 || a.n_sub <= 0 || a.n_seg < 1 ||
        a.n_seg > 3)
        return hipErrorInvalidValue;
    // one format for every matrix of the launch
    const int t = a.seg[0].w.type;
    for (int s = 0; s < a.n_seg; ++s) {
        const PfSeg& g = a.seg[s];
        if (!pf_gemm_supported(g.w.type, g.w.K, g.w.N) || g.w.type != t || g.w.K != a.K || !g.y)
            return hipErrorInvalidValue;
        const int next = s + 1 < a.n_seg ? a.seg[s + 1].sub0 : a.n_sub;
        if (next - g.sub0 != g.w.N / 16) return hipErrorInvalidValue;
        if (a.mode == GEMV_SILU && (g.w2.type != t || g.w2.K != a.K || g.w2.N != g.w.N)) return hipErrorInvalidValue;
    }
    if (a.seg[0].sub0 != 0 || (a.mode == GEMV_SILU && a.n_seg != 1)) return hipErrorInvalidValue;
    if (t == TF_HIP_TYPE_F32 || t == TF_HIP_TYPE_Q6_K) {
        // register-streamed tiles only: 4 column subtiles per wave, 2 when that leaves
        // fewer than two workgroups per CU
        const int mt = a.Mpad / kPfTileM;
        const int out4 = a.mode == GEMV_SILU ? 2 : 4;
        const int wg4 = (a.n_sub + 2 * out4 - 1) / (2 * out4) * mt;
        const int ni = wg4 >= 2 * device_cu_count() ? 4 : 2;
        const int per_wg = 2 * (a.mode == GEMV_SILU ? ni / 2 : ni);
        const dim3 grid((unsigned)((a.n_sub + per_wg - 1) / per_wg * mt));
#define PF_OWN(KERNEL, MODE, NI) hipLaunchKernelGGL((KERNEL<MODE, NI>), grid, dim3(256), 0, st, a)
#define PF_OWN_ALL(KERNEL)                                             \
    switch (a.mode * 8 + ni) {                                         \
        case GEMV_STORE * 8 + 4: PF_OWN(KERNEL, GEMV_STORE, 4); break; \
        case GEMV_STORE * 8 + 2: PF_OWN(KERNEL, GEMV_STORE, 2); break; \
        case GEMV_RESID * 8 + 4: PF_OWN(KERNEL, GEMV_RESID, 4); break; \
        case GEMV_RESID * 8 + 2: PF_OWN(KERNEL, GEMV_RESID, 2); break; \
        case GEMV_SILU * 8 + 4: PF_OWN(KERNEL, GEMV_SILU, 4); break;   \
        case GEMV_SILU * 8 + 2: PF_OWN(KERNEL, GEMV_SILU, 2); break;   \
        default: return hipErrorInvalidValue;                          \
    }
        if (t == TF_HIP_TYPE_F32) {
            PF_OWN_ALL(k_pf_gemm_f32)
        } else {
            PF_OWN_ALL(k_pf_gemm_q6k)
        }
#undef PF_OWN_ALL
#undef PF_OWN
        return hipGetLastError();
    }
    switch (t) {
        case TF_HIP_TYPE_Q8_0: return launch_gemm_t<TF_HIP_TYPE_Q8_0>(a, st, fused);
        case TF_HIP_TYPE_Q4_0: return launch_gemm_t<TF_HIP_TYPE_Q4_0>(a, st, fused);
        case TF_HIP_TYPE_Q4_1: return launch_gemm_t<TF_HIP_TYPE_Q4_1>(a, st, fused);
        case TF_HIP_TYPE_F16: return launch_gemm_t<TF_HIP_TYPE_F16>(a, st, fused);
    }
    return hipErrorInvalidValue;
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

size_t pf_attn_ws_bytes(int hd, int G, int n_keys) {
    return (size_t)((n_keys + kAttnTile - 1) / kAttnTile) * G * attn_rec_bytes(hd);
}

namespace {

template <int HD, int QS, int KS>
hipError_t launch_attn_t(const float* q, int64_t ldq, const unsigned char* recs, int T, int G, int n_rep, int QG,
                         int n, int pos0, int att_start, float* out, int64_t ldo, hipStream_t st) {
    const size_t lds = (size_t)kAttnBufs * KS * attn_buf_bytes(HD);
    static hipError_t attr = hipFuncSetAttribute((const void*)k_pf_attn<HD, QS, KS>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    const int per_blk = 16 * QS * QG;
    const dim3 grid((unsigned)((n + per_blk - 1) / per_blk * G)), block((unsigned)(64 * n_rep * QG * KS));
    hipLaunchKernelGGL((k_pf_attn<HD, QS, KS>), grid, block, lds, st, q, ldq, recs, T, n_rep, QG, n, pos0, att_start,
                       out, ldo, G);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_attn_hd(const float* q, int64_t ldq, const float* kc, const float* vc, int layout, int G,
                          int max_seq, int n_rep, int n, int pos0, int att_start, float* out, int64_t ldo,
                          unsigned char* recs, hipStream_t st) {
    const int n_keys = pos0 + n - att_start, T = (n_keys + kAttnTile - 1) / kAttnTile;
    hipLaunchKernelGGL(k_pf_pack_kv<HD>, dim3((unsigned)T, (unsigned)G), dim3(kBlock), 0, st, kc, vc, layout, G,
                       max_seq, att_start, n_keys, recs);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // 4 to 8 waves per workgroup, one 16-query subtile per wave (a prompt chunk of 4096
    // rows gives 256 query blocks per kv head)
    const int QG = (4 + n_rep - 1) / n_rep;
    // two key streams where the waves of one stream leave room for a second
    if (2 * n_rep * QG <= 8) return launch_attn_t<HD, 1, 2>(q, ldq, recs, T, G, n_rep, QG, n, pos0, att_start, out, ldo, st);
    return launch_attn_t<HD, 1, 1>(q, ldq, recs, T, G, n_rep, QG, n, pos0, att_start, out, ldo, st);
}

}  // namespace

hipError_t launch_pf_attn(const float* q, int64_t ldq, const float* kc, const float* vc, int layout, int H, int G,
                          int hd, int max_seq, int n, int pos0, int att_start, float* out, int64_t ldo, void* ws,
                          size_t ws_bytes, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int n_rep = H / G;
    if (H % G != 0 || !pf_attn_supported(hd, n_rep) || att_start < 0 || att_start > pos0 || pos0 + n > max_seq ||
        ldq % 4 != 0 || ldo % 4 != 0 || !ws || ws_bytes < pf_attn_ws_bytes(hd, G, pos0 + n - att_start))
        return hipErrorInvalidValue;
    unsigned char* recs = (unsigned char*)ws;
    switch (hd) {
        case 32:
            return launch_attn_hd<32>(q, ldq, kc, vc, layout, G, max_seq, n_rep, n, pos0, att_start, out, ldo, recs,
                                      st);
        case 64:
            return launch_attn_hd<64>(q, ldq, kc, vc, layout, G, max_seq, n_rep, n, pos0, att_start, out, ldo, recs,
                                      st);
        default:
            return launch_attn_hd<128>(q, ldq, kc, vc, layout, G, max_seq, n_rep, n, pos0, att_start, out, ldo, recs,
                                       st);
    }
}

hipError_t launch_pf_tail(Ctl* ctl, int pos_last, const int32_t* hist, const float* xrow, float* x, int D,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_pf_tail, dim3(1), dim3(kBlock), 0, st, ctl, pos_last, hist, xrow, x, D);
    return hipGetLastError();
}

}  // namespace tfk
