// Embedding lookup, weight repacking, dequantization, and the single-op kernels
// behind the op-level entry points (rmsnorm, argmax) and the HBM read roof.
#include <mutex>
#include <vector>

#include "formats.hpp"

namespace tfk {

namespace {

// dequant_row of the token's embedding row (model.cpp:199). The token is the one the
// host staged at hist[pos] (mode 0) or the previous step's argmax (mode 1), which is
// recorded there; the argmax key is cleared for this step's lm_head.
template <int T>
__global__ __launch_bounds__(kBlock) void k_embed(const DevMat emb, float* x, Ctl* ctl, int32_t* hist, int D) {
    using F = Fmt<T>;
    __shared__ int tok;
    if (threadIdx.x == 0) {
        const int p = ctl->pos;
        int t = ctl->mode ? key_to_index(ctl->key) : hist[p];
        if (t < 0 || t >= emb.N) {
            ctl->err = 1;
            t = 0;
        }
        tok = t;
        hist[p] = t;
        ctl->last_token = t;
        ctl->key = 0ull;
    }
    __syncthreads();
    const RowPtr rp = F::row(emb, tok);
    for (int s = threadIdx.x; s < D / F::E; s += kBlock) {
        float v[F::E];
        F::dequant(F::load(rp, s), v);
#pragma unroll
        for (int i = 0; i < F::E; i += 4) *(float4*)(x + (int64_t)s * F::E + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
    }
}

// dequant_row of each prompt token's embedding row (model.cpp:186): row i of x is
// token tok[i] (tokens are range-checked by the host).
template <int T>
__global__ __launch_bounds__(kBlock) void k_embed_rows(const DevMat emb, const int32_t* tok, float* x, int D) {
    using F = Fmt<T>;
    const RowPtr rp = F::row(emb, tok[blockIdx.x]);
    float* xr = x + (int64_t)blockIdx.x * D;
    for (int s = threadIdx.x; s < D / F::E; s += kBlock) {
        float v[F::E];
        F::dequant(F::load(rp, s), v);
#pragma unroll
        for (int i = 0; i < F::E; i += 4) *(float4*)(xr + (int64_t)s * F::E + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
    }
}

template <int T>
__global__ __launch_bounds__(kBlock) void k_dequant_rows(const DevMat m, int64_t row0, int64_t nrows, float* out) {
    using F = Fmt<T>;
    const int64_t steps = m.K / F::E;
    const int64_t total = nrows * steps;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
        const int64_t r = i / steps;
        const int s = (int)(i % steps);
        float v[F::E];
        F::dequant(F::load(F::row(m, row0 + r), s), v);
#pragma unroll
        for (int j = 0; j < F::E; ++j) out[r * m.K + (int64_t)s * F::E + j] = v[j];
    }
}

// GGUF rows -> DevMat streams. One thread per GGUF block (Q6_K: per 32-element group).
__global__ __launch_bounds__(kBlock) void k_repack(int type, const uint8_t* raw, int64_t K, int64_t N, DevMat m) {
    const int64_t nb = K / 32;  // 32-element groups per row
    const int64_t total = N * nb;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
        const int64_t r = i / nb, b = i % nb;
        if (type == TF_HIP_TYPE_Q8_0) {
            const uint8_t* src = raw + r * nb * 34 + b * 34;
            uint8_t* q = m.q + r * K + b * 32;
            for (int j = 0; j < 32; ++j) q[j] = src[2 + j];  // int8 q
            ((uint16_t*)m.s)[r * nb + b] = (uint16_t)(src[0] | (src[1] << 8));
        } else if (type == TF_HIP_TYPE_Q4_0) {
            const uint8_t* src = raw + r * nb * 18 + b * 18;
            uint8_t* q = m.q + r * (K / 2) + b * 16;
            for (int j = 0; j < 16; ++j) q[j] = src[2 + j];
            ((uint16_t*)m.s)[r * nb + b] = (uint16_t)(src[0] | (src[1] << 8));
        } else if (type == TF_HIP_TYPE_Q4_1) {
            const uint8_t* src = raw + r * nb * 20 + b * 20;
            uint8_t* q = m.q + r * (K / 2) + b * 16;
            for (int j = 0; j < 16; ++j) q[j] = src[4 + j];
            ((uint16_t*)m.s)[2 * (r * nb + b)] = (uint16_t)(src[0] | (src[1] << 8));
            ((uint16_t*)m.s)[2 * (r * nb + b) + 1] = (uint16_t)(src[2] | (src[3] << 8));
        } else if (type == TF_HIP_TYPE_Q6_K) {
            // group b of row r: elements e = 32 (b % 8) + j of super-block b / 8
            const int64_t sb = b / 8;
            const int c = (int)(b % 8);
            const uint8_t* blk = raw + r * (K / 256) * 210 + sb * 210;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            uint8_t u[32];
            for (int j = 0; j < 32; ++j) {
                // GGUF position of element e = 128h + 32k + l (quant.cpp:101-127)
                const int e = 32 * c + j;
                const int h = e / 128, k = (e % 128) / 32, l = e % 32;
                const uint8_t lb = ql[64 * h + l + 32 * (k & 1)];
                const int nib = k < 2 ? (lb & 0x0F) : (lb >> 4);
                const int top = (qh[32 * h + l] >> (2 * k)) & 3;
                u[j] = (uint8_t)(nib | (top << 4));
            }
            uint8_t* lo = m.q + r * (K / 2) + b * 16;
            uint8_t* hi = m.q2 + r * (K / 4) + b * 8;
            for (int j = 0; j < 16; ++j) lo[j] = (uint8_t)((u[j] & 0x0F) | ((u[j + 16] & 0x0F) << 4));
            for (int j = 0; j < 8; ++j)
                hi[j] = (uint8_t)((u[j] >> 4) | ((u[j + 8] >> 4) << 2) | ((u[j + 16] >> 4) << 4) | ((u[j + 24] >> 4) << 6));
            m.s[r * (K / 16) + 2 * b] = blk[192 + 2 * c];
            m.s[r * (K / 16) + 2 * b + 1] = blk[192 + 2 * c + 1];
            if (c == 0) ((uint16_t*)m.s2)[r * (K / 256) + sb] = (uint16_t)(blk[208] | (blk[209] << 8));
        }
    }
}

// rmsnorm (layers.cpp:7-12), one workgroup per row.
__global__ __launch_bounds__(kBlock) void k_rmsnorm_rows(const float* x, const float* w, int n, float eps, float* out) {
    __shared__ double red[kWavesPerBlock];
    const float* xr = x + (int64_t)blockIdx.x * n;
    float* o = out + (int64_t)blockIdx.x * n;
    double ss = 0;
    for (int k = threadIdx.x; k < n; k += kBlock) ss += (double)xr[k] * (double)xr[k];
    ss = wave_sum_d(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int k = threadIdx.x; k < n; k += kBlock) o[k] = xr[k] * inv * w[k];
}

// apply_rope_many (attention.cpp:48-53): thread i rotates pair j of (row, head) i / d2 with
// the angles of position pos0 + row from the host tables, as rope_one (attention.cpp:31-41)
// in the reference's build, which contracts each output's first product into an fma.
__global__ __launch_bounds__(kBlock) void k_rope_rows(float* x, int64_t n_pairs, int n_heads, int hd, int pos0,
                                                      const float* cos_tab, const float* sin_tab) {
    const int d2 = hd / 2;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n_pairs; i += (int64_t)gridDim.x * kBlock) {
        const int64_t rh = i / d2;  // row * n_heads + head
        const int j = (int)(i - rh * d2);
        const int64_t pos = pos0 + rh / n_heads;
        float* v = x + rh * hd;
        const float c = cos_tab[pos * d2 + j], s = sin_tab[pos * d2 + j];
        const float x0 = v[j], x1 = v[j + d2];
        v[j] = fmaf(x0, c, -(x1 * s));
        v[j + d2] = fmaf(x0, s, x1 * c);
    }
}

__global__ __launch_bounds__(kBlock) void k_argmax(const float* x, int n, Ctl* ctl) {
    __shared__ unsigned long long wb[kWavesPerBlock];
    unsigned long long best = 0;
    for (int i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) {
        const unsigned long long k = argmax_key(x[i], i);
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < kWavesPerBlock; ++i) best = wb[i] > best ? wb[i] : best;
        best = wb[0] > best ? wb[0] : best;
        atomicMax(&ctl->key, best);
    }
}

// Read-only stream (bench/stream.c:128-141 on the GPU): every byte read once per launch.
// The words are summed as integers (mod 2^32), so the total does not depend on the order
// and says whether every word was read: out[wave] holds each wave's partial sum.
__global__ __launch_bounds__(kBlock) void k_read_stream(const uint4* p, size_t n4, uint32_t* out) {
    uint32_t acc = 0;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += (size_t)gridDim.x * kBlock) {
        const uint4 v = p[i];
        acc += (v.x + v.y) + (v.z + v.w);
    }
    acc = wave_sum_u32(acc);
    if ((threadIdx.x & 63) == 0) out[(size_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)] = acc;
}

// The streams' fill pattern: 32-bit word i holds i * kStreamMul (mod 2^32), so the sum of
// n words is kStreamMul * n (n - 1) / 2 (mod 2^32).
__global__ __launch_bounds__(kBlock) void k_fill_stream(uint4* p, size_t n4) {
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += (size_t)gridDim.x * kBlock) {
        const uint32_t w = (uint32_t)(4 * i);
        p[i] = make_uint4(w * kStreamMul, (w + 1) * kStreamMul, (w + 2) * kStreamMul, (w + 3) * kStreamMul);
    }
}

// Copy stream (bench/stream.c:106-115 on the GPU): every byte read once and written once.
__global__ __launch_bounds__(kBlock) void k_copy_stream(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                        size_t n4) {
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += (size_t)gridDim.x * kBlock) dst[i] = src[i];
}

int grid_for(int64_t work) {
    const int64_t cap = 16LL * device_cu_count();
    int64_t b = (work + kBlock - 1) / kBlock;
    if (b < 1) b = 1;
    return (int)(b < cap ? b : cap);
}

}  // namespace

int device_cu_count() {
    static std::once_flag once;
    static int cus = 256;
    std::call_once(once, [] {
        int dev = 0;
        if (hipGetDevice(&dev) == hipSuccess) {
            int v = 0;
            if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
        }
    });
    return cus;
}

#define TF_DISPATCH_TYPE(type, CALL)                                  \
    switch (type) {                                                    \
        case TF_HIP_TYPE_Q8_0: { constexpr int T_ = TF_HIP_TYPE_Q8_0; CALL; break; } \
        case TF_HIP_TYPE_Q4_0: { constexpr int T_ = TF_HIP_TYPE_Q4_0; CALL; break; } \
        case TF_HIP_TYPE_Q4_1: { constexpr int T_ = TF_HIP_TYPE_Q4_1; CALL; break; } \
        case TF_HIP_TYPE_Q6_K: { constexpr int T_ = TF_HIP_TYPE_Q6_K; CALL; break; } \
        case TF_HIP_TYPE_F16: { constexpr int T_ = TF_HIP_TYPE_F16; CALL; break; }   \
        case TF_HIP_TYPE_F32: { constexpr int T_ = TF_HIP_TYPE_F32; CALL; break; }   \
        default: return hipErrorInvalidValue;                          \
    }

hipError_t launch_embed(const DevMat& emb, float* x, Ctl* ctl, int32_t* hist, int D, hipStream_t st) {
    TF_DISPATCH_TYPE(emb.type, hipLaunchKernelGGL((k_embed<T_>), dim3(1), dim3(kBlock), 0, st, emb, x, ctl, hist, D));
    return hipGetLastError();
}

hipError_t launch_embed_rows(const DevMat& emb, const int32_t* tok, int n, float* x, int D, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    TF_DISPATCH_TYPE(emb.type, hipLaunchKernelGGL((k_embed_rows<T_>), dim3(n), dim3(kBlock), 0, st, emb, tok, x, D));
    return hipGetLastError();
}

hipError_t launch_dequant_rows(const DevMat& m, int64_t row0, int64_t nrows, float* out, hipStream_t st) {
    const int64_t steps = m.K / fmt_step_elems(m.type);
    const int blocks = grid_for(nrows * steps);
    TF_DISPATCH_TYPE(m.type, hipLaunchKernelGGL((k_dequant_rows<T_>), dim3(blocks), dim3(kBlock), 0, st, m, row0, nrows, out));
    return hipGetLastError();
}

hipError_t launch_repack(int type, const uint8_t* raw, int64_t K, int64_t N, DevMat& m, hipStream_t st) {
    hipLaunchKernelGGL(k_repack, dim3(grid_for(N * (K / 32))), dim3(kBlock), 0, st, type, raw, K, N, m);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float* x, const float* w, int n, int rows, float eps, float* out, hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(rows), dim3(kBlock), 0, st, x, w, n, eps, out);
    return hipGetLastError();
}

hipError_t launch_rope_rows(float* x, int seq, int n_heads, int hd, int pos0, const float* cos_tab,
                            const float* sin_tab, hipStream_t st) {
    const int64_t n_pairs = (int64_t)seq * n_heads * (hd / 2);
    hipLaunchKernelGGL(k_rope_rows, dim3(grid_for(n_pairs)), dim3(kBlock), 0, st, x, n_pairs, n_heads, hd, pos0, cos_tab,
                       sin_tab);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* x, int n, Ctl* ctl, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax, dim3(grid_for(n)), dim3(kBlock), 0, st, x, n, ctl);
    return hipGetLastError();
}

hipError_t launch_copy_stream(uint4* dst, const uint4* src, size_t n4, int blocks, hipStream_t st) {
    hipLaunchKernelGGL(k_copy_stream, dim3(blocks), dim3(kBlock), 0, st, dst, src, n4);
    return hipGetLastError();
}

hipError_t launch_read_stream(const uint4* p, size_t n4, uint32_t* out, int blocks, hipStream_t st) {
    hipLaunchKernelGGL(k_read_stream, dim3(blocks), dim3(kBlock), 0, st, p, n4, out);
    return hipGetLastError();
}

hipError_t launch_fill_stream(uint4* p, size_t n4, int blocks, hipStream_t st) {
    hipLaunchKernelGGL(k_fill_stream, dim3(blocks), dim3(kBlock), 0, st, p, n4);
    return hipGetLastError();
}

}  // namespace tfk
