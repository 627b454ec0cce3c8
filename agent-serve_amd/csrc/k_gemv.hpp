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
#pragma once
#include "formats.hpp"

namespace tfk {
namespace gemv_detail {

constexpr int kStageVec = 9;  // float4 of x per thread: K <= 9 * 4 * kBlock = 9216

// x (optionally RMSNorm-ed) and its 16-element partial sums into LDS. Every load of x
// and of the norm weight is issued before the first one is used, and the prologue ends
// with every load complete, the first weight tile's included (issued earlier, it has
// landed by the time x has): the main loop then starts with no stale pending loads in
// the compiler's wait bookkeeping.
__device__ void stage_x(const GemvArgs& a, float* xs, float* x16, bool need_sums) {
    const int K4 = (int)(a.K / 4);
    const int nv = (K4 + kBlock - 1) / kBlock;  // float4 of x per thread actually needed
    const int tid = threadIdx.x;
    const float4* x4 = (const float4*)a.x;
    // indices past the end re-load the last element (never stored)
    float4 xv[kStageVec];
#pragma unroll
    for (int i = 0; i < kStageVec; ++i) {
        const int j = tid + i * kBlock;
        if (i < nv) xv[i] = x4[j < K4 ? j : K4 - 1];
    }
    if (a.norm_w) {
        const float4* w4 = (const float4*)a.norm_w;
        float4 wv[kStageVec];
#pragma unroll
        for (int i = 0; i < kStageVec; ++i) {
            const int j = tid + i * kBlock;
            if (i < nv) wv[i] = w4[j < K4 ? j : K4 - 1];
        }
        __shared__ double red[kWavesPerBlock];
        double ss = 0;  // every x*x is exact in fp64, as in the reference's accumulation
#pragma unroll
        for (int i = 0; i < kStageVec; ++i) {
            if (i < nv) {
                const float4 v = xv[i];
                const double t = (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
                ss += tid + i * kBlock < K4 ? t : 0.0;
            }
        }
        ss = wave_sum_d(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = 1.0f / sqrtf((float)(ss / a.K) + a.eps);
#pragma unroll
        for (int i = 0; i < kStageVec; ++i) {
            if (i < nv) {
                const float4 v = xv[i], w = wv[i];
                xv[i] = make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kStageVec; ++i) {
        const int j = tid + i * kBlock;
        if (i < nv && j < K4) {
            ((float4*)xs)[j] = xv[i];
            if (a.norm_out && blockIdx.x == 0) ((float4*)a.norm_out)[j] = xv[i];
        }
    }
    __syncthreads();
    if (need_sums) {
        for (int c = tid; c < (int)(a.K / 16); c += kBlock) {
            const float4* p = (const float4*)(xs + 16 * c);
            const float4 u = p[0], v = p[1], w = p[2], z = p[3];
            x16[c] = ((u.x + u.y) + (u.z + u.w)) + ((v.x + v.y) + (v.z + v.w)) + ((w.x + w.y) + (w.z + w.w)) +
                     ((z.x + z.y) + (z.z + z.w));
        }
        __syncthreads();
    }
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt = expcnt = lgkmcnt = 0
}

// R rows per group; SILU pairs R gate rows with the same R up rows (NR = 2R streams).
// A wave walks tiles (group g, tile ti): tile ti of a group covers steps
// ti*64U + 64u + lane (u < U) of its NR rows. Tiles are double-buffered in registers:
// the loads of tile t+1 are in flight while tile t is consumed, and the loads of a
// wave's first tile are issued before the x prologue, which does not need them.
template <int T, int R, int MODE, int U>
__global__ __launch_bounds__(kBlock) void k_gemv(const GemvArgs a) {
    using F = Fmt<T>;
    using Raw = typename F::Raw;
    constexpr bool SILU = MODE == GEMV_SILU;
    constexpr int NR = SILU ? 2 * R : R;
    extern __shared__ float smem[];
    float* xs = smem;
    float* x16 = smem + a.K;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // groups are wave-uniform
    const int S = (int)(a.K / F::E);
    const int TPG = (S + kWave * U - 1) / (kWave * U);

    // the segment holding group g, chosen with compile-time indices: a runtime index into
    // the kernel arguments would become a vector load whose wait drains the weight loads
    // in flight
    auto locate = [&](int g, int& row0) -> const GemvSeg& {
        if (a.n_seg > 1 && g >= (int)a.seg[0].groups) {
            g -= (int)a.seg[0].groups;
            if (a.n_seg > 2 && g >= (int)a.seg[1].groups) {
                row0 = (g - (int)a.seg[1].groups) * R;
                return a.seg[2];
            }
            row0 = g * R;
            return a.seg[1];
        }
        row0 = g * R;
        return a.seg[0];
    };
    // a tile's weight loads, plus what the group's epilogue reads (the residual row for
    // RESID, the bias row for STORE; a harmless word of x where there is none), issued
    // with the tile so that its wait is the tile's
    auto load_tile = [&](int g, int ti, Raw (&w)[U][NR], float& extra) {
        int row0;
        const GemvSeg& sg = locate(g, row0);
        const int N = (int)sg.a.N;
        if (MODE == GEMV_RESID || MODE == GEMV_STORE) {
            int re = row0 + (lane < R ? lane : R - 1);
            re = re < N ? re : N - 1;
            const float* ep = MODE == GEMV_RESID ? sg.y : sg.bias;
            extra = ep ? ep[re] : a.x[0];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + r < N ? row0 + r : N - 1;  // tail rows re-read a valid row
            const RowPtr pa = F::row(sg.a, row);
            RowPtr pb = pa;
            if (SILU) pb = F::row(sg.b, row);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // steps past the row end re-load its last step (masked out in step()): the
                // loads stay unconditional, so their wait counts stay exact
                int s = ti * kWave * U + u * kWave + lane;
                s = s < S ? s : S - 1;
                w[u][r] = F::load(pa, s);
                if (SILU) w[u][R + r] = F::load(pb, s);
            }
        }
    };

    // groups g, g + stride, ... of this wave, TPG tiles each: the tile count is known up
    // front, so the loop below has a single back edge and no exit path with loads pending
    const int total = (int)a.total_groups;
    const int stride = gridDim.x * kWavesPerBlock;
    int g = blockIdx.x * kWavesPerBlock + wave;
    const int n_tiles = g < total ? ((total - 1 - g) / stride + 1) * TPG : 0;
    int ti = 0;
    Raw wa[U][NR], wb[U][NR];
    float ea = 0.0f, eb = 0.0f;
    if (n_tiles > 0) load_tile(g, 0, wa, ea);
    stage_x(a, xs, x16, F::kNeedSums);

    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
    unsigned long long best = 0;

    // lane r writes row r of the group (every lane holds every row's total)
    auto epilogue = [&](int gq, float extra) {
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = wave_sum(acc[r]);
        int row0;
        const GemvSeg& sg = locate(gq, row0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + r;
            if (lane == r && row < (int)sg.a.N) {
                const float v = acc[r];
                if (SILU) {
                    sg.y[row] = (v / (1.0f + expf(-v))) * acc[R + r];
                } else if (MODE == GEMV_STORE) {
                    sg.y[row] = sg.bias ? v + extra : v;
                } else if (MODE == GEMV_RESID) {
                    const float nv = extra + v;
                    sg.y[row] = nv;
                    if (sg.tap) sg.tap[row] = nv;
                } else {  // GEMV_LOGITS
                    if (sg.y) sg.y[row] = v;
                    const unsigned long long k = argmax_key(v, row);
                    best = k > best ? k : best;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
    };
    // consume `cur` (tile ti of group g) while `nxt` receives the following tile; past
    // the wave's last tile the load re-reads the current one (an L2 hit) so that it
    // stays unconditional: a load under a branch makes the compiler's wait before the
    // next use a full drain
    auto step = [&](Raw (&cur)[U][NR], float& ecur, Raw (&nxt)[U][NR], float& enxt) {
        int gn = g;
        int tn = ti + 1;
        if (tn == TPG) {
            tn = 0;
            gn = g + stride;
        }
        const bool more = gn < total;
        load_tile(more ? gn : g, more ? tn : ti, nxt, enxt);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = ti * kWave * U + u * kWave + lane;
            const bool in_row = s < S;
            const int sc = in_row ? s : S - 1;
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const float d = F::dot(cur[u][r], xs, x16, sc);
                acc[r] += in_row ? d : 0.0f;
            }
        }
        if (ti == TPG - 1) epilogue(g, ecur);
        g = gn;
        ti = tn;
    };
    int k = 0;
    for (; k + 2 <= n_tiles; k += 2) {
        step(wa, ea, wb, eb);
        step(wb, eb, wa, ea);
    }
    if (k < n_tiles) step(wa, ea, wb, eb);

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

template <int T, int R, int U>
hipError_t launch_t(const GemvArgs& a, int blocks, size_t lds, hipStream_t st) {
    switch (a.mode) {
        case GEMV_STORE: hipLaunchKernelGGL((k_gemv<T, R, GEMV_STORE, U>), dim3(blocks), dim3(kBlock), lds, st, a); break;
        case GEMV_RESID: hipLaunchKernelGGL((k_gemv<T, R, GEMV_RESID, U>), dim3(blocks), dim3(kBlock), lds, st, a); break;
        case GEMV_SILU: hipLaunchKernelGGL((k_gemv<T, R, GEMV_SILU, U>), dim3(blocks), dim3(kBlock), lds, st, a); break;
        case GEMV_LOGITS: hipLaunchKernelGGL((k_gemv<T, R, GEMV_LOGITS, U>), dim3(blocks), dim3(kBlock), lds, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Steps in flight per row and tile (U): enough to cover the row (up to 8 x 16 B per lane),
// fewer when many rows share a wave.
template <int T>
hipError_t launch_r(const GemvArgs& a, int R, int blocks, size_t lds, hipStream_t st) {
    const int S = (int)(a.K / Fmt<T>::E);
    // steps in flight per row and tile: the whole row where it fits 4 x 16 B per lane
    int U = (S + kWave - 1) / kWave;
    U = U >= 4 ? 4 : U >= 2 ? 2 : 1;
    switch (R * 16 + U) {
        case 1 * 16 + 1: return launch_t<T, 1, 1>(a, blocks, lds, st);
        case 1 * 16 + 2: return launch_t<T, 1, 2>(a, blocks, lds, st);
        case 1 * 16 + 4: return launch_t<T, 1, 4>(a, blocks, lds, st);
        case 2 * 16 + 1: return launch_t<T, 2, 1>(a, blocks, lds, st);
        case 2 * 16 + 2: return launch_t<T, 2, 2>(a, blocks, lds, st);
        case 2 * 16 + 4: return launch_t<T, 2, 4>(a, blocks, lds, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace gemv_detail

// Instantiated once per format in k_gemv_<format>.hip.
template <int T>
hipError_t launch_gemv_fmt(const GemvArgs& a, int R, int blocks, size_t lds, hipStream_t st) {
    return gemv_detail::launch_r<T>(a, R, blocks, lds, st);
}

}  // namespace tfk
