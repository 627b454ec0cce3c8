// Fused dequant-GEMV for the decode step (the matmul of matmul.cpp:22-32 with M = 1,
// which is 99% of the reference's decode time).
//
// One workgroup = 4 wavefronts. The prologue stages x (optionally RMSNorm-ed, the
// rmsnorm of layers.cpp:7-12 fused in) and its 16-element partial sums in LDS. Each
// wavefront then owns groups of R consecutive output rows: lanes stride over the row
// in 16-byte steps (formats.hpp), keep U steps of all R rows in flight, and fold the
// 64 lane partials with a butterfly. Epilogues fuse the QKV bias (model.cpp:122-124),
// the residual adds (model.cpp:131, 141), SiLU*up (layers.cpp:14-19) and the greedy
// argmax of the lm_head (sampler.cpp:8-13).
#include "formats.hpp"

namespace tfk {

namespace {

constexpr int kUnroll = 2;

__device__ void stage_x(const GemvArgs& a, float* xs, float* x16, bool need_sums) {
    const int K = (int)a.K;
    const int tid = threadIdx.x;
    if (a.norm_w) {
        __shared__ double red[kWavesPerBlock];
        double ss = 0;
        for (int k = tid; k < K; k += kBlock) {
            const double v = (double)a.x[k];
            ss += v * v;  // exact in fp64, as the reference's accumulation terms
        }
        ss = wave_sum_d(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = 1.0f / sqrtf((float)(ss / K) + a.eps);
        for (int k = tid; k < K; k += kBlock) xs[k] = a.x[k] * inv * a.norm_w[k];
    } else {
        for (int k = tid; k < K; k += kBlock) xs[k] = a.x[k];
    }
    __syncthreads();
    if (a.norm_out && blockIdx.x == 0)
        for (int k = tid; k < K; k += kBlock) a.norm_out[k] = xs[k];
    if (need_sums) {
        for (int c = tid; c < K / 16; c += kBlock) {
            const float4* p = (const float4*)(xs + 16 * c);
            const float4 u = p[0], v = p[1], w = p[2], z = p[3];
            x16[c] = ((u.x + u.y) + (u.z + u.w)) + ((v.x + v.y) + (v.z + v.w)) + ((w.x + w.y) + (w.z + w.w)) +
                     ((z.x + z.y) + (z.z + z.w));
        }
        __syncthreads();
    }
}

template <int NR>
__device__ __forceinline__ float pick(const float (&v)[NR], int i) {
    float r = v[0];
#pragma unroll
    for (int j = 1; j < NR; ++j) r = (i == j) ? v[j] : r;
    return r;
}

// R rows per group; SILU pairs R gate rows with the same R up rows (NR = 2R streams).
template <int T, int R, int MODE>
__global__ __launch_bounds__(kBlock) void k_gemv(const GemvArgs a) {
    using F = Fmt<T>;
    constexpr bool SILU = MODE == GEMV_SILU;
    constexpr int NR = SILU ? 2 * R : R;
    extern __shared__ float smem[];
    float* xs = smem;
    float* x16 = smem + a.K;
    stage_x(a, xs, x16, F::kNeedSums);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int S = (int)(a.K / F::E);
    unsigned long long best = 0;

    for (int64_t g = (int64_t)blockIdx.x * kWavesPerBlock + wave; g < a.total_groups;
         g += (int64_t)gridDim.x * kWavesPerBlock) {
        int si = 0;
        int64_t gg = g;
        while (si + 1 < a.n_seg && gg >= a.seg[si].groups) {
            gg -= a.seg[si].groups;
            ++si;
        }
        const GemvSeg& sg = a.seg[si];
        const int64_t row0 = gg * R;
        const int64_t N = sg.a.N;
        RowPtr rp[NR];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = row0 + r < N ? row0 + r : N - 1;  // tail rows re-read a valid row
            rp[r] = F::row(sg.a, row);
            if (SILU) rp[R + r] = F::row(sg.b, row);
        }
        float acc[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = 0.0f;

        for (int s0 = lane; s0 < S; s0 += kWave * kUnroll) {
            typename F::Raw w[kUnroll][NR];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int s = s0 + u * kWave;
                if (s < S) {
#pragma unroll
                    for (int r = 0; r < NR; ++r) w[u][r] = F::load(rp[r], s);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int s = s0 + u * kWave;
                if (s < S) {
#pragma unroll
                    for (int r = 0; r < NR; ++r) acc[r] += F::dot(w[u][r], xs, x16, s);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = wave_sum(acc[r]);

        const int64_t row = row0 + lane;
        if (lane < R && row < N) {
            const float v = pick<NR>(acc, lane);
            if (SILU) {
                const float up = pick<NR>(acc, lane + R);
                sg.y[row] = (v / (1.0f + expf(-v))) * up;
            } else if (MODE == GEMV_STORE) {
                sg.y[row] = sg.bias ? v + sg.bias[row] : v;
            } else if (MODE == GEMV_RESID) {
                const float nv = sg.y[row] + v;
                sg.y[row] = nv;
                if (sg.tap) sg.tap[row] = nv;
            } else {  // GEMV_LOGITS
                if (sg.y) sg.y[row] = v;
                const unsigned long long k = argmax_key(v, row);
                best = k > best ? k : best;
            }
        }
    }

    if (MODE == GEMV_LOGITS) {
        __shared__ unsigned long long wbest[kWavesPerBlock];
        best = wave_max_u64(best);
        if (lane == 0) wbest[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long b = wbest[0];
            for (int i = 1; i < kWavesPerBlock; ++i) b = wbest[i] > b ? wbest[i] : b;
            atomicMax(&a.ctl->key, b);
            if (a.bump_pos && blockIdx.x == 0) a.ctl->pos += 1;
        }
    }
}

template <int T, int R>
hipError_t launch_t(const GemvArgs& a, int blocks, size_t lds, hipStream_t st) {
    switch (a.mode) {
        case GEMV_STORE: hipLaunchKernelGGL((k_gemv<T, R, GEMV_STORE>), dim3(blocks), dim3(kBlock), lds, st, a); break;
        case GEMV_RESID: hipLaunchKernelGGL((k_gemv<T, R, GEMV_RESID>), dim3(blocks), dim3(kBlock), lds, st, a); break;
        case GEMV_SILU: hipLaunchKernelGGL((k_gemv<T, R, GEMV_SILU>), dim3(blocks), dim3(kBlock), lds, st, a); break;
        case GEMV_LOGITS: hipLaunchKernelGGL((k_gemv<T, R, GEMV_LOGITS>), dim3(blocks), dim3(kBlock), lds, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int T>
hipError_t launch_r(const GemvArgs& a, int R, int blocks, size_t lds, hipStream_t st) {
    switch (R) {
        case 1: return launch_t<T, 1>(a, blocks, lds, st);
        case 2: return launch_t<T, 2>(a, blocks, lds, st);
        case 4: return launch_t<T, 4>(a, blocks, lds, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

int64_t gemv_groups(int64_t n_rows, int rows_per_wave) { return (n_rows + rows_per_wave - 1) / rows_per_wave; }

size_t gemv_lds_bytes(int64_t K) { return (size_t)K * 4 + (size_t)(K / 16) * 4; }

hipError_t launch_gemv(const GemvArgs& a, int R, hipStream_t st) {
    if (a.total_groups <= 0) return hipSuccess;
    const int cap = 4 * device_cu_count();
    const int64_t want = (a.total_groups + kWavesPerBlock - 1) / kWavesPerBlock;
    const int blocks = (int)(want < cap ? want : cap);
    const size_t lds = gemv_lds_bytes(a.K);
    switch (a.type) {
        case TF_HIP_TYPE_Q8_0: return launch_r<TF_HIP_TYPE_Q8_0>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_Q4_0: return launch_r<TF_HIP_TYPE_Q4_0>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_Q4_1: return launch_r<TF_HIP_TYPE_Q4_1>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_Q6_K: return launch_r<TF_HIP_TYPE_Q6_K>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_F16: return launch_r<TF_HIP_TYPE_F16>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_F32: return launch_r<TF_HIP_TYPE_F32>(a, R, blocks, lds, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace tfk
