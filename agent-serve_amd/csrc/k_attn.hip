// Decode attention over the HBM-resident fp32 KV cache (attn_decode, attention.cpp:55-80),
// with the RoPE of q and k (attention.cpp:31-46) and the KV store (kvcache.cpp:31-36)
// folded in.
//
// k_attn_decode: grid = kv heads x S splits of the position range (flash-decoding). A
// workgroup rotates its n_rep query heads and the new key, then walks its positions in
// LDS tiles of K and V rows (one memory round per tile): scores in the reference's
// 8-lane dot order, an online softmax across tiles, and P.V. With one active split it
// writes the output heads itself; otherwise it writes (max, sum, o) partials and
// k_attn_combine merges them in a second launch. Splits are one tile long until there
// are kAttnMaxSplits of them, so a long context is read by many workgroups in one memory
// round each instead of a few walking tiles one after the other.
// No workgroup waits on another inside a launch: on this multi-XCD part a device-scope
// fence writes back the XCD's L2, which costs more than the kernel boundary.
#include "dev_common.hpp"
#include "tf_internal.hpp"

namespace tfk {

namespace {

constexpr int kMaxRep = 8;     // query heads per kv head supported (GQA ratio)
constexpr int kAttnTile = 32;  // positions per K/V tile in LDS

// Per-thread register counts for head_dim <= HDM (64, 128 or 256).
template <int HDM>
struct AttnShape {
    static constexpr int kPairs = kMaxRep * HDM / kBlock;             // (head, dim) pairs of P.V
    static constexpr int kQPairs = kMaxRep * HDM / 2 / kBlock;        // rotation pairs
    static constexpr int kTileVec = kAttnTile * HDM / 4 / kBlock;     // float4 of a K (or V) tile
};

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

template <int HDM>
__global__ __launch_bounds__(kBlock) void k_attn_decode(const AttnArgs a) {
    constexpr int kMaxPairs = AttnShape<HDM>::kPairs;
    constexpr int kQPairs = AttnShape<HDM>::kQPairs;
    constexpr int kTileVec = AttnShape<HDM>::kTileVec;
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

    // K/V rows of a tile, kTileVec float4 of each per thread, loaded into registers;
    // indices past the tile re-load its last element (never stored) so the loads
    // stay unconditional
    auto load_tile = [&](int t0, float4 (&kr)[kTileVec], float4 (&vr)[kTileVec]) {
        const int tn = min(kAttnTile, p1 - t0);
#pragma unroll
        for (int k = 0; k < kTileVec; ++k) {
            int i = tid + k * kBlock;
            i = i < tn * hd4 ? i : tn * hd4 - 1;
            const int j = i / hd4, c = i % hd4;
            const int64_t o = kv_index(a.layout, a.G, a.max_seq, hd, g, t0 + j) + 4 * c;
            kr[k] = *(const float4*)(a.kc + o);
            vr[k] = *(const float4*)(a.vc + o);
        }
    };
    // one memory round for everything the first tile needs
    const int nq = n_rep * d2;
    float qa[kQPairs], qb[kQPairs], ca[kQPairs], sa[kQPairs];
    // without RoPE the angles are loaded but unused: row 0 of the table then, so that a
    // stand-in table of d2 floats (the op-level entry points pass q) is never read past
    const int64_t ro = a.rope ? (int64_t)pos * d2 : 0;
    const float* cs = a.rope_cos + ro;
    const float* sn = a.rope_sin + ro;
#pragma unroll
    for (int k = 0; k < kQPairs; ++k) {
        int i = tid + k * kBlock;
        i = i < nq ? i : nq - 1;
        const int r = i / d2, j = i % d2;
        const float* qh = a.q + (int64_t)(g * n_rep + r) * hd;
        qa[k] = qh[j];
        qb[k] = qh[j + d2];
        ca[k] = cs[j];
        sa[k] = sn[j];
    }
    const int jk = tid < d2 ? tid : d2 - 1;
    // the new row: knew / vnew, or (null) the cache's row at pos, already stored
    const int64_t o_new = kv_index(a.layout, a.G, a.max_seq, hd, g, pos);
    const float* kh = a.knew ? a.knew + (int64_t)g * hd : a.kc + o_new;
    const float* vh = a.vnew ? a.vnew + (int64_t)g * hd : a.vc + o_new;
    const float k0 = kh[jk], k1 = kh[jk + d2], kc0 = cs[jk], ks0 = sn[jk];
    const int jv = tid < hd ? tid : hd - 1;
    const float v0 = vh[jv];
    float4 kr_a[kTileVec], vr_a[kTileVec], kr_b[kTileVec], vr_b[kTileVec];
    load_tile(p0, kr_a, vr_a);

#pragma unroll
    for (int k = 0; k < kQPairs; ++k) {
        const int i = tid + k * kBlock;
        if (i < nq) {
            const int r = i / d2, j = i % d2;
            if (a.rope) {
                qs[r * hd + j] = fmaf(qa[k], ca[k], -(qb[k] * sa[k]));
                qs[r * hd + j + d2] = fmaf(qa[k], sa[k], qb[k] * ca[k]);
            } else {
                qs[r * hd + j] = qa[k];
                qs[r * hd + j + d2] = qb[k];
            }
        }
    }
    if (tid < d2) {
        kn[tid] = a.rope ? fmaf(k0, kc0, -(k1 * ks0)) : k0;
        kn[tid + d2] = a.rope ? fmaf(k0, ks0, k1 * kc0) : k1;
    }
    if (tid < hd) vn[tid] = v0;
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

    auto tile = [&](int t0, float4 (&kr)[kTileVec], float4 (&vr)[kTileVec], float4 (&kn_r)[kTileVec],
                    float4 (&vn_r)[kTileVec]) {
        const int tn = min(kAttnTile, p1 - t0);
        if (t0 + kAttnTile < p1) load_tile(t0 + kAttnTile, kn_r, vn_r);  // next tile in flight
#pragma unroll
        for (int k = 0; k < kTileVec; ++k) {
            const int i = tid + k * kBlock;
            if (i < tn * hd4) {
                const int j = i / hd4, c = i % hd4;
                const bool is_new = t0 + j == pos;  // not in the cache yet: the rotated k and v
                *(float4*)(kt + j * ks + 4 * c) = is_new ? *(const float4*)(kn + 4 * c) : kr[k];
                *(float4*)(vt + j * hd + 4 * c) = is_new ? *(const float4*)(vn + 4 * c) : vr[k];
            }
        }
        __syncthreads();
        // scores in the order of dot_f32 (8 lanes over i = 0, 8, ..., then hsum8; quant.cpp:198-214)
        for (int i = tid; i < n_rep * tn; i += kBlock) {
            const int r = i / tn, j = i % tn;
            const float* qr = qs + r * hd;
            const float* krow = kt + j * ks;
            float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int e = 0; e < hd; e += 8) {
                const float4 q0 = *(const float4*)(qr + e), q1 = *(const float4*)(qr + e + 4);
                const float4 x0 = *(const float4*)(krow + e), x1 = *(const float4*)(krow + e + 4);
                c[0] = fmaf(q0.x, x0.x, c[0]);
                c[1] = fmaf(q0.y, x0.y, c[1]);
                c[2] = fmaf(q0.z, x0.z, c[2]);
                c[3] = fmaf(q0.w, x0.w, c[3]);
                c[4] = fmaf(q1.x, x1.x, c[4]);
                c[5] = fmaf(q1.y, x1.y, c[5]);
                c[6] = fmaf(q1.z, x1.z, c[6]);
                c[7] = fmaf(q1.w, x1.w, c[7]);
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
    };
    for (int t0 = p0; t0 < p1;) {
        tile(t0, kr_a, vr_a, kr_b, vr_b);
        t0 += kAttnTile;
        if (t0 >= p1) break;
        tile(t0, kr_b, vr_b, kr_a, vr_a);
        t0 += kAttnTile;
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

// Merges the split partials of head blockIdx.x: out = sum_s o_s e^(m_s - M) / sum_s l_s
// e^(m_s - M), M = max_s m_s. One workgroup per head: the weights e^(m_s - M) go to LDS
// once, thread (d, group) sums o_s[d] over the splits s = group, group + groups, ..., and
// the groups are added in group order (a fixed order for a given split count).
constexpr int kCombThreads = 1024;

__global__ __launch_bounds__(kCombThreads) void k_attn_combine(const AttnArgs a) {
    const Split sp = split_of(a);
    if (sp.n_act <= 1) return;  // k_attn_decode wrote the output
    __shared__ float w[kAttnMaxSplits];
    __shared__ float red[kCombThreads / kWave];
    __shared__ float part[kCombThreads];
    const int h = blockIdx.x, n = sp.n_act, hd = a.hd;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* ml = a.part_ml + (int64_t)h * a.S * 2;
    float m = -INFINITY;
    for (int t = tid; t < n; t += kCombThreads) m = fmaxf(m, ml[2 * t]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    float M = red[0];
    for (int i = 1; i < kCombThreads / kWave; ++i) M = fmaxf(M, red[i]);
    __syncthreads();  // red is reused below
    float l = 0.0f;
    for (int t = tid; t < n; t += kCombThreads) {
        const float wt = expf(ml[2 * t] - M);
        w[t] = wt;
        l = fmaf(ml[2 * t + 1], wt, l);
    }
    l = wave_sum(l);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    float L = 0.0f;
    for (int i = 0; i < kCombThreads / kWave; ++i) L += red[i];
    const int groups = kCombThreads / hd;
    const int d = tid % hd, grp = tid / hd;
    float o = 0.0f;
    if (grp < groups) {
        const float* po = a.part_o + (int64_t)h * a.S * hd + d;
#pragma unroll 8
        for (int t = grp; t < n; t += groups) o = fmaf(po[(int64_t)t * hd], w[t], o);
    }
    part[tid] = o;
    __syncthreads();
    if (tid < hd) {
        float sum = 0.0f;
        for (int g = 0; g < groups; ++g) sum += part[g * hd + tid];
        a.out[(int64_t)h * hd + tid] = sum / L;
    }
}

}  // namespace

int attn_splits(int max_seq) {
    if (max_seq <= 512) return 1;
    int s = (max_seq + kAttnMinChunk - 1) / kAttnMinChunk;
    return s < 2 ? 2 : (s > kAttnMaxSplits ? kAttnMaxSplits : s);
}

hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t st) {
    const int n_rep = a.H / a.G;
    const size_t lds = sizeof(float) * ((size_t)n_rep * a.hd + 2 * (size_t)a.hd + (size_t)kAttnTile * (a.hd + 4) +
                                        (size_t)kAttnTile * a.hd + (size_t)n_rep * kAttnTile + 3 * (size_t)n_rep);
    if (a.hd <= 64)
        hipLaunchKernelGGL(k_attn_decode<64>, dim3(a.G * a.S), dim3(kBlock), lds, st, a);
    else if (a.hd <= 128)
        hipLaunchKernelGGL(k_attn_decode<128>, dim3(a.G * a.S), dim3(kBlock), lds, st, a);
    else
        hipLaunchKernelGGL(k_attn_decode<256>, dim3(a.G * a.S), dim3(kBlock), lds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.S == 1) return e;
    if (a.hd > kCombThreads) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.H), dim3(kCombThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace tfk
