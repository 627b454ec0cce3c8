// Decode attention over the HBM-resident fp32 KV cache (attn_decode, attention.cpp:55-80),
// with the RoPE of q and k (attention.cpp:31-46) and the KV store (kvcache.cpp:31-36)
// folded in.
//
// k_attn_decode: grid = kv heads x S splits of the position range (flash-decoding). A
// workgroup rotates its n_rep query heads and the new key, then walks its positions in
// LDS tiles of K and V rows (one memory round per tile): scores in the reference's
// 8-lane dot order, an online softmax across tiles, and P.V. With one active split it
// writes the output heads itself; otherwise it writes (max, sum, o) partials and
// k_attn_combine merges them in a second launch.
// No workgroup waits on another inside a launch: on this multi-XCD part a device-scope
// fence writes back the XCD's L2, which costs more than the kernel boundary.
#include "dev_common.hpp"
#include "tf_internal.hpp"

namespace tfk {

namespace {

constexpr int kMaxRep = 8;     // query heads per kv head supported (GQA ratio)
constexpr int kAttnTile = 32;  // positions per K/V tile in LDS
constexpr int kMaxPairs = kMaxRep * 256 / kBlock;  // (head, dim) pairs per thread, head_dim <= 256

__device__ __forceinline__ int64_t kv_index(int layout, int G, int max_seq, int hd, int g, int p) {
    return layout == TF_HIP_KV_HEAD_MAJOR ? ((int64_t)g * max_seq + p) * hd : ((int64_t)p * G + g) * hd;
}

struct Split {
    int pos, start, n_act, chunk;
};

// Active splits: positions [start, pos] cut into chunks of at least kAttnMinChunk.
__device__ __forceinline__ Split split_of(const AttnArgs& a) {
    Split sp;
    sp.pos = a.fixed_pos >= 0 ? a.fixed_pos : a.ctl->pos;
    sp.start = a.fixed_pos >= 0 ? a.fixed_start : a.ctl->att_start;
    const int n = sp.pos + 1 - sp.start;
    int n_act = (n + kAttnMinChunk - 1) / kAttnMinChunk;
    sp.n_act = n_act < a.S ? n_act : a.S;
    sp.chunk = (n + sp.n_act - 1) / sp.n_act;
    return sp;
}

__global__ __launch_bounds__(kBlock) void k_attn_decode(const AttnArgs a) {
    const int g = blockIdx.x / a.S;
    const int s = blockIdx.x % a.S;
    const int hd = a.hd, d2 = hd / 2, hd4 = hd / 4;
    const int n_rep = a.H / a.G;
    const Split sp = split_of(a);
    if (s >= sp.n_act) return;
    const int pos = sp.pos;
    const int p0 = sp.start + s * sp.chunk;
    const int p1 = min(pos + 1, p0 + sp.chunk);
    const int tid = threadIdx.x;
    const int ks = hd + 4;  // padded K-tile row: rows fall in different LDS banks

    extern __shared__ float sm[];
    float* qs = sm;                        // [n_rep][hd] rotated queries
    float* kn = qs + n_rep * hd;           // [hd] rotated new key
    float* vn = kn + hd;                   // [hd] new value
    float* kt = vn + hd;                   // [kAttnTile][hd + 4] K tile
    float* vt = kt + kAttnTile * ks;       // [kAttnTile][hd] V tile
    float* pr = vt + kAttnTile * hd;       // [n_rep][kAttnTile] scores, then weights
    float* st = pr + n_rep * kAttnTile;    // [n_rep][3] running max, running sum, rescale

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
    if (tid < n_rep) {
        st[3 * tid] = -INFINITY;
        st[3 * tid + 1] = 0.0f;
    }
    __syncthreads();
    // the split holding the new position publishes k and v to the cache
    if (a.store_kv && p1 == pos + 1) {
        const int64_t o = kv_index(a.layout, a.G, a.max_seq, hd, g, pos);
        for (int j = tid; j < hd; j += kBlock) {
            a.kc[o + j] = kn[j];
            a.vc[o + j] = vn[j];
        }
    }
    const float scale = 1.0f / sqrtf((float)hd);
    float o_acc[kMaxPairs];
#pragma unroll
    for (int k = 0; k < kMaxPairs; ++k) o_acc[k] = 0.0f;

    for (int t0 = p0; t0 < p1; t0 += kAttnTile) {
        const int tn = min(kAttnTile, p1 - t0);
        // K and V rows of the tile, one memory round for the whole tile
        for (int i = tid; i < tn * hd4; i += kBlock) {
            const int j = i / hd4, c = i % hd4;
            const int p = t0 + j;
            float4 kv, vv;
            if (p == pos) {
                kv = *(const float4*)(kn + 4 * c);
                vv = *(const float4*)(vn + 4 * c);
            } else {
                const int64_t o = kv_index(a.layout, a.G, a.max_seq, hd, g, p) + 4 * c;
                kv = *(const float4*)(a.kc + o);
                vv = *(const float4*)(a.vc + o);
            }
            *(float4*)(kt + j * ks + 4 * c) = kv;
            *(float4*)(vt + j * hd + 4 * c) = vv;
        }
        __syncthreads();
        // scores in the order of dot_f32 (8 lanes over i = 0, 8, ..., then hsum8; quant.cpp:198-214)
        for (int i = tid; i < n_rep * tn; i += kBlock) {
            const int r = i / tn, j = i % tn;
            const float* qr = qs + r * hd;
            const float* kr = kt + j * ks;
            float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int e = 0; e < hd; e += 8) {
                const float4 qa = *(const float4*)(qr + e), qb = *(const float4*)(qr + e + 4);
                const float4 ka = *(const float4*)(kr + e), kb = *(const float4*)(kr + e + 4);
                c[0] = fmaf(qa.x, ka.x, c[0]);
                c[1] = fmaf(qa.y, ka.y, c[1]);
                c[2] = fmaf(qa.z, ka.z, c[2]);
                c[3] = fmaf(qa.w, ka.w, c[3]);
                c[4] = fmaf(qb.x, kb.x, c[4]);
                c[5] = fmaf(qb.y, kb.y, c[5]);
                c[6] = fmaf(qb.z, kb.z, c[6]);
                c[7] = fmaf(qb.w, kb.w, c[7]);
            }
            pr[r * kAttnTile + j] = scale * (((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7])));
        }
        __syncthreads();
        // online softmax statistics: wave w handles heads r = w, w + 4, ...
        const int lane = tid & 63, wave = tid >> 6;
        for (int r = wave; r < n_rep; r += kWavesPerBlock) {
            const float v = lane < tn ? pr[r * kAttnTile + lane] : -INFINITY;
            const float m_old = st[3 * r];
            const float m_new = fmaxf(m_old, wave_max(v));
            const float e = lane < tn ? expf(v - m_new) : 0.0f;
            if (lane < tn) pr[r * kAttnTile + lane] = e;
            const float l_tile = wave_sum(e);
            if (lane == 0) {
                const float alpha = expf(m_old - m_new);  // 0 on the first tile
                st[3 * r] = m_new;
                st[3 * r + 1] = fmaf(st[3 * r + 1], alpha, l_tile);
                st[3 * r + 2] = alpha;
            }
        }
        __syncthreads();
        // P.V: thread owns (head, dim) pairs tid, tid + 256, ...
#pragma unroll
        for (int k = 0; k < kMaxPairs; ++k) {
            const int pi = tid + k * kBlock;
            if (pi < n_rep * hd) {
                const int r = pi / hd, d = pi % hd;
                float o = o_acc[k] * st[3 * r + 2];
                for (int j = 0; j < tn; ++j) o = fmaf(pr[r * kAttnTile + j], vt[j * hd + d], o);
                o_acc[k] = o;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < kMaxPairs; ++k) {
        const int pi = tid + k * kBlock;
        if (pi < n_rep * hd) {
            const int r = pi / hd, d = pi % hd;
            const int h = g * n_rep + r;
            if (sp.n_act == 1)
                a.out[(int64_t)h * hd + d] = o_acc[k] / st[3 * r + 1];
            else
                a.part_o[((int64_t)h * a.S + s) * hd + d] = o_acc[k];
        }
    }
    if (sp.n_act > 1 && tid < n_rep) {
        const int h = g * n_rep + tid;
        a.part_ml[((int64_t)h * a.S + s) * 2] = st[3 * tid];
        a.part_ml[((int64_t)h * a.S + s) * 2 + 1] = st[3 * tid + 1];
    }
}

// Merges the split partials: out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M).
__global__ __launch_bounds__(kBlock) void k_attn_combine(const AttnArgs a) {
    const Split sp = split_of(a);
    if (sp.n_act <= 1) return;  // k_attn_decode wrote the output
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= a.H * a.hd) return;
    const int h = i / a.hd, dd = i % a.hd;
    const float* ml = a.part_ml + (int64_t)h * a.S * 2;
    float M = -INFINITY;
    for (int t = 0; t < sp.n_act; ++t) M = fmaxf(M, ml[2 * t]);
    float L = 0.0f, o = 0.0f;
    for (int t = 0; t < sp.n_act; ++t) {
        const float w = expf(ml[2 * t] - M);
        L = fmaf(ml[2 * t + 1], w, L);
        o = fmaf(a.part_o[((int64_t)h * a.S + t) * a.hd + dd], w, o);
    }
    a.out[(int64_t)h * a.hd + dd] = o / L;
}

}  // namespace

int attn_splits(int max_seq) {
    if (max_seq <= 512) return 1;
    int s = (max_seq + kAttnMinChunk - 1) / kAttnMinChunk;
    return s < 2 ? 2 : (s > 64 ? 64 : s);
}

hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t st) {
    const int n_rep = a.H / a.G;
    const size_t lds = sizeof(float) * ((size_t)n_rep * a.hd + 2 * (size_t)a.hd + (size_t)kAttnTile * (a.hd + 4) +
                                        (size_t)kAttnTile * a.hd + (size_t)n_rep * kAttnTile + 3 * (size_t)n_rep);
    hipLaunchKernelGGL(k_attn_decode, dim3(a.G * a.S), dim3(kBlock), lds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.S == 1) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3((a.H * a.hd + kBlock - 1) / kBlock), dim3(kBlock), 0, st, a);
    return hipGetLastError();
}

}  // namespace tfk
