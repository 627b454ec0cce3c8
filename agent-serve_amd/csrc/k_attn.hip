// Decode attention over the HBM-resident fp32 KV cache (attn_decode, attention.cpp:55-80),
// with the RoPE of q and k (attention.cpp:31-46) and the KV store (kvcache.cpp:31-36)
// folded in.
//
// Grid = kv heads x S splits of the position range (flash-decoding). A workgroup
// rotates its n_rep query heads and the new key, scores its positions (one thread per
// position, the reference's 8-lane dot order), takes a local softmax and accumulates
// P.V; the last workgroup of a kv head to finish (atomic ticket) merges the S
// partial (max, sum, o) triples into the output heads and re-arms the ticket.
#include "dev_common.hpp"
#include "tf_internal.hpp"

namespace tfk {

namespace {

constexpr int kMinChunk = 32;
constexpr int kMaxRep = 8;  // query heads per kv head supported (GQA ratio)

__device__ __forceinline__ int64_t kv_index(int layout, int G, int max_seq, int hd, int g, int p) {
    return layout == TF_HIP_KV_HEAD_MAJOR ? ((int64_t)g * max_seq + p) * hd : ((int64_t)p * G + g) * hd;
}

__global__ __launch_bounds__(kBlock) void k_attn_decode(const AttnArgs a) {
    const int g = blockIdx.x / a.S;
    const int s = blockIdx.x % a.S;
    const int hd = a.hd, d2 = hd / 2;
    const int n_rep = a.H / a.G;
    const int pos = a.fixed_pos >= 0 ? a.fixed_pos : a.ctl->pos;
    const int start = a.fixed_pos >= 0 ? a.fixed_start : a.ctl->att_start;
    const int n = pos + 1 - start;
    int n_act = (n + kMinChunk - 1) / kMinChunk;
    n_act = n_act < a.S ? n_act : a.S;
    const int chunk = (n + n_act - 1) / n_act;
    const int p0 = start + s * chunk;
    const int p1 = min(pos + 1, p0 + chunk);
    const int tid = threadIdx.x;

    extern __shared__ float sm[];
    float* qs = sm;                  // [n_rep][hd] rotated queries
    float* kn = qs + n_rep * hd;     // [hd] rotated new key
    float* vn = kn + hd;             // [hd] new value
    float* pr = vn + hd;             // [n_rep][chunk] scores, then exp weights
    float* red = pr + n_rep * chunk; // [n_rep][2] (max, sum)
    float* acc_part = red + 2 * n_rep; // [4][n_rep][hd] partial P.V per thread group
    __shared__ int is_last;

    if (s < n_act) {
        const float* cs = a.rope_cos + (int64_t)pos * d2;
        const float* sn = a.rope_sin + (int64_t)pos * d2;
        for (int i = tid; i < n_rep * d2; i += kBlock) {
            const int r = i / d2, j = i % d2;
            const float* qh = a.q + (int64_t)(g * n_rep + r) * hd;
            const float x0 = qh[j], x1 = qh[j + d2];
            if (a.rope) {
                qs[r * hd + j] = fmaf(x0, cs[j], -(x1 * sn[j]));
                qs[r * hd + j + d2] = fmaf(x0, sn[j], x1 * cs[j]);
            } else {
                qs[r * hd + j] = x0;
                qs[r * hd + j + d2] = x1;
            }
        }
        for (int j = tid; j < d2; j += kBlock) {
            const float* kh = a.knew + (int64_t)g * hd;
            const float x0 = kh[j], x1 = kh[j + d2];
            if (a.rope) {
                kn[j] = fmaf(x0, cs[j], -(x1 * sn[j]));
                kn[j + d2] = fmaf(x0, sn[j], x1 * cs[j]);
            } else {
                kn[j] = x0;
                kn[j + d2] = x1;
            }
        }
        for (int j = tid; j < hd; j += kBlock) vn[j] = a.vnew[(int64_t)g * hd + j];
        __syncthreads();
        // The split holding the new position publishes k and v to the cache.
        if (a.store_kv && p1 == pos + 1) {
            const int64_t o = kv_index(a.layout, a.G, a.max_seq, hd, g, pos);
            for (int j = tid; j < hd; j += kBlock) {
                a.kc[o + j] = kn[j];
                a.vc[o + j] = vn[j];
            }
        }
        // scores: one thread per position, all n_rep heads at once, in the order of dot_f32
        // (8 lanes, FMAs over i = 0, 8, 16, ..., then hsum8; quant.cpp:198-214)
        const float scale = 1.0f / sqrtf((float)hd);
        for (int pp = tid; pp < p1 - p0; pp += kBlock) {
            const int p = p0 + pp;
            const float* kp = p == pos ? kn : a.kc + kv_index(a.layout, a.G, a.max_seq, hd, g, p);
            float acc[kMaxRep][8];
#pragma unroll
            for (int r = 0; r < kMaxRep; ++r)
#pragma unroll
                for (int l = 0; l < 8; ++l) acc[r][l] = 0.0f;
            for (int i = 0; i < hd; i += 8) {
                const float4 ka = *(const float4*)(kp + i), kb = *(const float4*)(kp + i + 4);
                const float kk[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
#pragma unroll
                for (int r = 0; r < kMaxRep; ++r) {
                    if (r < n_rep) {
                        const float* qr = qs + r * hd + i;
#pragma unroll
                        for (int l = 0; l < 8; ++l) acc[r][l] = fmaf(qr[l], kk[l], acc[r][l]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < kMaxRep; ++r) {
                if (r < n_rep) {
                    const float* c = acc[r];
                    const float dt = ((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7]));
                    pr[r * chunk + pp] = scale * dt;
                }
            }
        }
        __syncthreads();
        // local softmax statistics: wave w handles heads r = w, w + 4, ...
        const int lane = tid & 63, wave = tid >> 6;
        const int len = p1 - p0;
        for (int r = wave; r < n_rep; r += kWavesPerBlock) {
            float m = -INFINITY;
            for (int i = lane; i < len; i += kWave) m = fmaxf(m, pr[r * chunk + i]);
            m = wave_max(m);
            float l = 0.0f;
            for (int i = lane; i < len; i += kWave) {
                const float e = expf(pr[r * chunk + i] - m);
                pr[r * chunk + i] = e;
                l += e;
            }
            l = wave_sum(l);
            if (lane == 0) {
                red[2 * r] = m;
                red[2 * r + 1] = l;
            }
        }
        __syncthreads();
        // P.V: thread (grp, d) sums positions grp, grp + ngrp, ... for every head of the group
        const int ngrp = kBlock / hd;  // 4 for hd 64, 2 for hd 128
        const int grp = tid / hd, d = tid % hd;
        if (grp < ngrp) {
            float o[kMaxRep];
#pragma unroll
            for (int r = 0; r < kMaxRep; ++r) o[r] = 0.0f;
            for (int pp = grp; pp < len; pp += ngrp) {
                const int p = p0 + pp;
                const float vv = p == pos ? vn[d] : a.vc[kv_index(a.layout, a.G, a.max_seq, hd, g, p) + d];
#pragma unroll
                for (int r = 0; r < kMaxRep; ++r)
                    if (r < n_rep) o[r] = fmaf(pr[r * chunk + pp], vv, o[r]);
            }
#pragma unroll
            for (int r = 0; r < kMaxRep; ++r)
                if (r < n_rep) acc_part[(grp * n_rep + r) * hd + d] = o[r];
        }
        __syncthreads();
        for (int i = tid; i < n_rep * hd; i += kBlock) {
            const int r = i / hd, dd = i % hd;
            float o = 0.0f;
            for (int q = 0; q < ngrp; ++q) o += acc_part[(q * n_rep + r) * hd + dd];
            const int h = g * n_rep + r;
            a.part_o[((int64_t)h * a.S + s) * hd + dd] = o;
        }
        if (tid < n_rep) {
            const int h = g * n_rep + tid;
            a.part_ml[((int64_t)h * a.S + s) * 2] = red[2 * tid];
            a.part_ml[((int64_t)h * a.S + s) * 2 + 1] = red[2 * tid + 1];
        }
    }
    // ticket: the last of the S workgroups of this kv head merges the partials
    __threadfence();
    __syncthreads();
    if (tid == 0) is_last = atomicAdd(&a.counter[g], 1u) == (unsigned)(a.S - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int i = tid; i < n_rep * hd; i += kBlock) {
        const int r = i / hd, dd = i % hd;
        const int h = g * n_rep + r;
        const float* ml = a.part_ml + (int64_t)h * a.S * 2;
        float M = -INFINITY;
        for (int t = 0; t < n_act; ++t) M = fmaxf(M, ml[2 * t]);
        float L = 0.0f, o = 0.0f;
        for (int t = 0; t < n_act; ++t) {
            const float w = expf(ml[2 * t] - M);
            L = fmaf(ml[2 * t + 1], w, L);
            o = fmaf(a.part_o[((int64_t)h * a.S + t) * hd + dd], w, o);
        }
        a.out[(int64_t)h * hd + dd] = o / L;
    }
    if (tid == 0) a.counter[g] = 0u;
}

}  // namespace

hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t st) {
    const int n_rep = a.H / a.G;
    int chunk_max = (a.max_seq + a.S - 1) / a.S;
    if (chunk_max < kMinChunk) chunk_max = kMinChunk;
    const int ngrp = kBlock / a.hd;
    const size_t lds = sizeof(float) * ((size_t)n_rep * a.hd + 2 * (size_t)a.hd + (size_t)n_rep * chunk_max +
                                        2 * (size_t)n_rep + (size_t)ngrp * n_rep * a.hd);
    hipLaunchKernelGGL(k_attn_decode, dim3(a.G * a.S), dim3(kBlock), lds, st, a);
    return hipGetLastError();
}

}  // namespace tfk
