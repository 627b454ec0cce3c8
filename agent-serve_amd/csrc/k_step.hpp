// Persistent decode step: one cooperative launch runs n tokens of the token loop
// (Model::decode, model.cpp:197-208, and the per-token layers of Model::prefill,
// model.cpp:144-195) with one workgroup of 8 waves per CU.
//
// Per layer (layer_decode, model.cpp:108-142), five phases:
//   1 QKV GEMV, attn_norm fused, bias added          -> q, k, v   (model.cpp:110-124)
//   2 attention, one workgroup per kv head            -> att       (model.cpp:125-130)
//   3 wo GEMV + residual                              -> x         (model.cpp:131)
//   4 gate/up GEMV, ffn_norm fused, SiLU(gate)*up     -> h         (model.cpp:133-139)
//   5 down GEMV + residual                            -> x         (model.cpp:140-141)
// then output_norm + lm_head + greedy argmax (model.cpp:204-207, sampler.cpp:8-13).
//
// Workgroups hand activations to each other as 64-bit words (epoch << 32 | float bits)
// stored and loaded with agent-scope relaxed atomics. Each (token, layer, phase) has its
// own epoch, so a consumer knows a word is current when it carries that epoch: no fence,
// counter or grid barrier is involved. Every workgroup also publishes one word at the end
// of a layer and the next layer waits for all of them, which makes each layer boundary a
// barrier; exchange buffers alternate by layer parity, so a buffer is rewritten only after
// every workgroup has finished reading it. Each wave issues the loads of its first two
// weight tiles before it waits for its phase's input, so HBM keeps streaming while the
// hand-off completes. Every wait is bounded: past the limit, or once another workgroup
// has flagged a failure, it flags ctl->err and goes on, and the host reports the error.
#pragma once
#include <type_traits>

#include "formats.hpp"

namespace tfk {
namespace step_detail {

typedef unsigned long long u64;

constexpr int kT = kStepThreads;   // threads per workgroup
constexpr int kNW = kT / kWave;    // waves per workgroup
constexpr int kGD = 8;             // exchange words per thread for d_model-sized inputs (<= 4096)
// Copies of the wo output's exchange words at most; a build writes RX of them and workgroup w
// reads copy w % RX, so that the workgroups' polls of that d_model vector spread over RX
// times the memory lines
constexpr int kXRep = 8;
constexpr int kGF = 20;            // and for d_ff-sized ones (<= 10240)
constexpr int kGW = 2;             // and for per-workgroup words (<= 1024)
constexpr int kMaxRep = 8;         // query heads per kv head
constexpr int kTile = 32;          // attention positions per LDS tile
constexpr int kSpinLimit = 1 << 20;  // about a second of polling
constexpr int kErrToken = 1;
constexpr int kErrTimeout = 2;


__device__ __forceinline__ void put(u64* p, float v, uint32_t e) {
    __hip_atomic_store(gptr(p), ((u64)e << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 get(u64* p) {
    return __hip_atomic_load(gptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes read at agent scope (two 8-byte loads that miss any stale copy in this XCD's L2).
// c ? a : b on values. (The conditional operator on two float4 lvalues selects between their
// addresses and copies, which keeps register arrays in scratch.)
__device__ __forceinline__ float4 sel4(bool c, float4 a, float4 b) {
    return make_float4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}
__device__ __forceinline__ float4 gload_f4_agent(const float* p) {
    const u64 a = __hip_atomic_load((const TF_GLOBAL u64*)gptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const u64 b = __hip_atomic_load((const TF_GLOBAL u64*)gptr(p + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
                       __uint_as_float((uint32_t)(b >> 32)));
}
__device__ __forceinline__ int get_err(Ctl* c) {
    return __hip_atomic_load(gptr(&c->err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void set_err(Ctl* c, int v) {
    __hip_atomic_store(gptr(&c->err), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits for the na words pa[0..na) of epoch ea and writes their values to da (LDS), and
// for the nb words pb[0..nb) of epoch eb (arrival words; values unused). Thread tid reads
// words tid + i*kT. Every load of the first pass is issued before any is checked; a word
// that does not carry its epoch yet is read again (bit i of `pend`) until it does.
// Needs na <= NA * kT, nb <= NB * kT, NA + NB <= 32.
template <int NA, int NB>
__device__ __forceinline__ void gather(u64* pa, int na, uint32_t ea, float* da, u64* pb, int nb, uint32_t eb,
                                       Ctl* ctl) {
    const int tid = threadIdx.x;
    u64 wa[NA], wb[NB];
#pragma unroll
    for (int i = 0; i < NA; ++i)
        if (tid + i * kT < na) wa[i] = get(pa + tid + i * kT);
#pragma unroll
    for (int i = 0; i < NB; ++i)
        if (tid + i * kT < nb) wb[i] = get(pb + tid + i * kT);
    uint32_t pend = 0;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int j = tid + i * kT;
        if (j < na) {
            if ((uint32_t)(wa[i] >> 32) == ea)
                da[j] = __uint_as_float((uint32_t)wa[i]);
            else
                pend |= 1u << i;
        }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i)
        if (tid + i * kT < nb && (uint32_t)(wb[i] >> 32) != eb) pend |= 1u << (NA + i);
    for (int spin = 0; pend; ++spin) {
        if (spin >= kSpinLimit || ((spin & 1023) == 1023 && get_err(ctl))) {
            if (!get_err(ctl)) set_err(ctl, kErrTimeout);  // the first failure's code stays
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            if (pend & (1u << i)) {
                const int j = tid + i * kT;
                const u64 w = get(pa + j);
                if ((uint32_t)(w >> 32) == ea) {
                    da[j] = __uint_as_float((uint32_t)w);
                    pend &= ~(1u << i);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (pend & (1u << (NA + i))) {
                const u64 w = get(pb + tid + i * kT);
                if ((uint32_t)(w >> 32) == eb) pend &= ~(1u << (NA + i));
            }
        }
    }
}

// gather() of words base[idx(j)], j < n, of epoch e into d[j] (LDS).
template <int NA, class Idx>
__device__ __forceinline__ void gather_idx(u64* base, Idx&& idx, int n, uint32_t e, float* d, Ctl* ctl) {
    const int tid = threadIdx.x;
    u64 w[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i)
        if (tid + i * kT < n) w[i] = get(base + idx(tid + i * kT));
    uint32_t pend = 0;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int j = tid + i * kT;
        if (j < n) {
            if ((uint32_t)(w[i] >> 32) == e)
                d[j] = __uint_as_float((uint32_t)w[i]);
            else
                pend |= 1u << i;
        }
    }
    for (int spin = 0; pend; ++spin) {
        if (spin >= kSpinLimit || ((spin & 1023) == 1023 && get_err(ctl))) {
            if (!get_err(ctl)) set_err(ctl, kErrTimeout);  // the first failure's code stays
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            if (pend & (1u << i)) {
                const int j = tid + i * kT;
                const u64 v = get(base + idx(j));
                if ((uint32_t)(v >> 32) == e) {
                    d[j] = __uint_as_float((uint32_t)v);
                    pend &= ~(1u << i);
                }
            }
        }
    }
}

// xs = rmsnorm(xr) (layers.cpp:7-12: fp64 sum of squares, inv = 1/sqrtf(ss/n + eps),
// x * inv * w) when w is set, else a copy; then the 16-element sums of xs when wanted.
// wr holds this thread's norm weights xs[tid + i*kT], loaded by the caller.
template <int NWR>
__device__ __forceinline__ void stage(const float* xr, int K, bool norm, const float (&wr)[NWR], float eps, float* xs, float* x16,
                      bool sums, double* red) {
    const int tid = threadIdx.x;
    __syncthreads();  // xr / xs written by the gather
    if (norm) {
        double ss = 0;
        for (int j = tid; j < K; j += kT) {
            const double v = xr[j];
            ss += v * v;
        }
        ss = wave_sum_d(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
        const float inv = 1.0f / sqrtf((float)(ss / K) + eps);
#pragma unroll
        for (int i = 0; i < NWR; ++i) {
            const int j = tid + i * kT;
            if (j < K) xs[j] = (xr[j] * inv) * wr[i];
        }
        __syncthreads();
    }
    if (sums) {
        for (int c = tid; c < K / 16; c += kT) {
            const float4* p = (const float4*)(xs + 16 * c);
            const float4 u = p[0], v = p[1], w = p[2], z = p[3];
            x16[c] = ((u.x + u.y) + (u.z + u.w)) + ((v.x + v.y) + (v.z + v.w)) + ((w.x + w.y) + (w.z + w.w)) +
                     ((z.x + z.y) + (z.z + z.w));
        }
    }
    __syncthreads();
}

// Norm weights of this thread (elements tid + i*kT), read before the phase's weight tiles
// so that waiting for them never waits for the tiles.
template <int NWR>
__device__ __forceinline__ void load_norm(const float* w, int K, float (&wr)[NWR]) {
#pragma unroll
    for (int i = 0; i < NWR; ++i) {
        const int j = threadIdx.x + i * kT;
        wr[i] = w ? *gptr(w + (j < K ? j : K - 1)) : 1.0f;
    }
}

// Rows of up to three matrices of one format (the segments), grouped R rows at a time;
// wave wid of nw takes groups wid, wid + nw, ... (wid < 0: no rows). A group's rows are
// walked in tiles of U*64 lane steps, double-buffered in registers; the first two tiles
// are loaded before prep() (the phase's input hand-off), the rest stream behind the
// compute. Loads are unconditional (indices clamped, contributions masked) so that the
// compiler's waits stay partial. seg_of(si, 0 | 1) is segment si's matrix (1: the up
// matrix of SILU), bias_of(si) its bias or nullptr; epi(si, row, v, v_up, bias) runs on
// lane r for row r. The workgroup synchronises before prep(), so prep may overwrite the
// LDS the previous phase read.
template <int T, int R, int MODE, int U, class SegOf, class BiasOf, class Prep, class Epi>
__device__ __forceinline__ void gemv_phase(int nseg, const int (&groups)[3], SegOf&& seg_of, BiasOf&& bias_of, int K,
                                           int wid, int nw, const float* xs, const float* x16, Prep&& prep,
                                           Epi&& epi) {
    using F = Fmt<T>;
    using Raw = typename F::Raw;
    constexpr bool SILU = MODE == GEMV_SILU;
    constexpr int NR = SILU ? 2 * R : R;
    const int lane = threadIdx.x & 63;
    const int S = K / F::E;
    const int TPG = (S + kWave * U - 1) / (kWave * U);
    const int total = groups[0] + (nseg > 1 ? groups[1] : 0) + (nseg > 2 ? groups[2] : 0);
    const int n_tiles = (wid >= 0 && wid < total) ? ((total - 1 - wid) / nw + 1) * TPG : 0;

    // segment and first row of group g (compile-time segment indices only)
    auto locate = [&](int g, int& row0) -> int {
        if (nseg > 1 && g >= groups[0]) {
            g -= groups[0];
            if (nseg > 2 && g >= groups[1]) {
                row0 = (g - groups[1]) * R;
                return 2;
            }
            row0 = g * R;
            return 1;
        }
        row0 = g * R;
        return 0;
    };
    auto load_k = [&](int k, Raw (&w)[U][NR], float& extra) {
        k = k < n_tiles ? k : n_tiles - 1;
        const int g = wid + (k / TPG) * nw;
        const int ti = k - (k / TPG) * TPG;
        int row0;
        const int si = locate(g, row0);
        const DevMat& ma = seg_of(si, 0);
        const int N = (int)ma.N;
        if (MODE == GEMV_STORE) {
            const float* bias = bias_of(si);
            int re = row0 + (lane < R ? lane : R - 1);
            re = re < N ? re : N - 1;
            extra = bias ? *gptr(bias + re) : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + r < N ? row0 + r : N - 1;
            const RowPtr pa = F::row(ma, row);
            RowPtr pb = pa;
            if (SILU) pb = F::row(seg_of(si, 1), row);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int s = ti * kWave * U + u * kWave + lane;
                s = s < S ? s : S - 1;
                w[u][r] = F::load(pa, s);
                if (SILU) w[u][R + r] = F::load(pb, s);
            }
        }
    };
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
    auto consume = [&](int k, Raw (&w)[U][NR], float extra) {
        const int g = wid + (k / TPG) * nw;
        const int ti = k - (k / TPG) * TPG;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = ti * kWave * U + u * kWave + lane;
            const bool in_row = s < S;
            const int sc = in_row ? s : S - 1;
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const float d = F::dot(w[u][r], xs, x16, sc);
                acc[r] += in_row ? d : 0.0f;
            }
        }
        if (ti == TPG - 1) {
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[r] = wave_sum(acc[r]);
            int row0;
            const int si = locate(g, row0);
            const int N = (int)seg_of(si, 0).N;
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (lane == r && row0 + r < N) epi(si, row0 + r, acc[r], SILU ? acc[R + r] : 0.0f, extra);
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
        }
    };

    Raw wa[U][NR], wb[U][NR];
    float ea = 0.0f, eb = 0.0f;
    __builtin_amdgcn_sched_barrier(0);  // keep this phase's code out of the previous one's
    if (n_tiles > 0) {
        load_k(0, wa, ea);
        load_k(1, wb, eb);
    }
    __syncthreads();
    prep();
    // the last one or two tiles are consumed without loading past them: a load issued there
    // (clamped, so a re-read) would sit in front of the next phase's exchange reads, which
    // complete after it
    int k = 0;
    for (; k + 2 < n_tiles; k += 2) {
        consume(k, wa, ea);
        load_k(k + 2, wa, ea);
        consume(k + 1, wb, eb);
        load_k(k + 3, wb, eb);
    }
    if (k < n_tiles) consume(k, wa, ea);
    if (k + 1 < n_tiles) consume(k + 1, wb, eb);
}

__device__ __forceinline__ int64_t kv_at(int layout, int G, int max_seq, int hd, int g, int p) {
    return layout == TF_HIP_KV_HEAD_MAJOR ? ((int64_t)g * max_seq + p) * hd : ((int64_t)p * G + g) * hd;
}

// Attention of kv head g's n_rep query heads over cache positions [p0, p1) (attn_decode,
// attention.cpp:55-80), with the RoPE of the query heads and the key (attention.cpp:31-46)
// and the store of the new K/V row at pos (kvcache.cpp:31-36). fetch() fills qkv (LDS) with
// the head block [n_rep q heads | k | v] the QKV phase produced; it runs after the first K/V
// tiles' loads are issued (the cached rows do not depend on this token), so the cache
// latency overlaps the hand-off. NB = 4 (spans of more than two 32-position tiles): four
// tiles are in flight at a time, each tile's registers reloaded with the tile four ahead as
// soon as they are in LDS; NB = 1 or 2 (spans of that many tiles): all of them load up
// front and nothing is reloaded (a load past the span would delay the hand-off's polls,
// which wait for every load in flight). The
// loads past the span re-read row p1 - 1 instead of being skipped: no load sits behind a
// branch, and every wait for a tile is a fixed count of the loads issued after it.
//   kPart false (attn_head, spans up to StepArgs::split_from): [p0, p1) = [start, pos]; out =
//     the normalised heads, [n_rep][hd]. The same workgroup runs head g for every such
//     token of a launch, so the rows it reads are its own or written before the launch.
//   kPart true (attn_part, longer spans): one split of [start, pos] (flash-decoding, split
//     over workgroups). out[r * (hd + 2) ...] = the unnormalised o (P.V with P = e^(s - m)),
//     then m and l (the running max and sum of the online softmax); the combine phase
//     merges the splits. The cache is read at agent scope. An empty split leaves m = -inf,
//     l = 0, o = 0 and does not wait for the head block.
//   Both store the new row at agent scope (a later, split token of the launch reads it from
//   other XCDs). With wait_row they wait for the stores before returning, i.e. before their
//   next puts; without it the caller waits for them (s_waitcnt vmcnt(0) in the waves with
//   tid < hd) before the workgroup's end-of-layer word, which every later reader of the row
//   waits for.
// bar() synchronises the kT threads that run the attention (a workgroup barrier, or the
// compute waves' barrier of a kernel whose other waves do not take part). a supplies H, G,
// hd, max_seq, layout and the RoPE tables, ly the layer's K and V cache (kc, vc).
template <int HDM, bool kPart, int NB, class A, class Ly, class Fetch, class Bar>
__device__ __forceinline__ void attn_span(const A& a, const Ly& ly, int g, int pos, int p0, int p1,
                                          float* qkv, float* sm, float* out, Fetch&& fetch, Bar&& bar,
                                          bool wait_row = true) {
    constexpr int kTV = (kTile * HDM / 4 + kT - 1) / kT;  // float4 of a K (or V) tile per thread
    const int hd = a.hd, d2 = hd / 2, hd4 = hd / 4;
    const int n_rep = a.H / a.G;
    const int tid = threadIdx.x;
    const int ks = hd + 4;
    const int ho = hd + 2;
    float* qs = qkv;                  // [n_rep][hd], rotated in place
    float* kn = qkv + n_rep * hd;     // [hd]
    float* vn = kn + hd;              // [hd]
    float* kt = sm;                   // [kTile][hd + 4]
    float* vt = kt + kTile * ks;      // [kTile][hd]
    if (kPart && p0 >= p1) {
        for (int i = tid; i < n_rep * ho; i += kT) {
            const int d = i % ho;
            out[i] = d == hd ? -INFINITY : 0.0f;
        }
        bar();
        return;
    }
    const TF_GLOBAL float* cs = gptr(a.rope_cos + (int64_t)pos * d2);
    const TF_GLOBAL float* sn = gptr(a.rope_sin + (int64_t)pos * d2);

    // tile i of the span, clamped to its last row
    auto tile_at = [&](int i) { return min(p0 + i * kTile, p1 - 1); };
    auto load_tile = [&](int t0, float4 (&kr)[kTV], float4 (&vr)[kTV]) __attribute__((always_inline)) {
        const int tn = min(kTile, p1 - t0);
#pragma unroll
        for (int k = 0; k < kTV; ++k) {
            int i = tid + k * kT;
            i = i < tn * hd4 ? i : tn * hd4 - 1;
            const int j = i / hd4, c = i % hd4;
            const int64_t o = kv_at(a.layout, a.G, a.max_seq, hd, g, t0 + j) + 4 * c;
            if constexpr (kPart) {
                kr[k] = gload_f4_agent(ly.kc + o);
                vr[k] = gload_f4_agent(ly.vc + o);
            } else {
                kr[k] = gload_f4(ly.kc + o);
                vr[k] = gload_f4(ly.vc + o);
            }
        }
    };
    // four named buffers (an array of them indexed by an unrolled loop ends up in scratch)
    float4 kr0[kTV], vr0[kTV], kr1[kTV], vr1[kTV], kr2[kTV], vr2[kTV], kr3[kTV], vr3[kTV];
    load_tile(tile_at(0), kr0, vr0);
    if constexpr (NB >= 2) load_tile(tile_at(1), kr1, vr1);
    if constexpr (NB == 4) {
        load_tile(tile_at(2), kr2, vr2);
        load_tile(tile_at(3), kr3, vr3);
    }
    // this thread's RoPE cos/sin, read before the hand-off (after it they would cost another
    // memory round trip on the attention's critical path)
    constexpr int kRope = ((kMaxRep + 1) * HDM / 2 + kT - 1) / kT;
    float rc[kRope], rs[kRope];
#pragma unroll
    for (int k = 0; k < kRope; ++k) {
        const int j = (tid + k * kT) % d2;
        rc[k] = cs[j];
        rs[k] = sn[j];
    }
    fetch();
    // RoPE (rope_one, with the reference build's contractions)
#pragma unroll
    for (int k = 0; k < kRope; ++k) {
        const int i = tid + k * kT;
        if (i < (n_rep + 1) * d2) {
            const int r = i / d2, j = i % d2;
            float* v = qs + r * hd;  // r == n_rep is the key
            const float x0 = v[j], x1 = v[j + d2], c = rc[k], s = rs[k];
            v[j] = fmaf(x0, c, -(x1 * s));
            v[j + d2] = fmaf(x0, s, x1 * c);
        }
    }
    bar();
    const bool stores_row = pos >= p0 && pos < p1;
    if (stores_row) {
        const int64_t o = kv_at(a.layout, a.G, a.max_seq, hd, g, pos);
        // agent scope in both layouts: a launch whose later tokens split reads this row from
        // workgroups on other XCDs
        for (int j = tid; j < hd; j += kT) {
            __hip_atomic_store(gptr(ly.kc + o + j), kn[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(gptr(ly.vc + o + j), vn[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Query head r = wave (n_rep <= kNW): its online-softmax state and its outputs (dims
    // lane + 64 c) stay in the wave's registers; lane j scores position j of a tile.
    constexpr int kOD = (HDM + kWave - 1) / kWave;
    const bool head_wave = wave < n_rep;
    const float* qr = qs + (head_wave ? wave : 0) * hd;
    float m_run = -INFINITY, l_run = 0.0f;
    float o_acc[kOD];
#pragma unroll
    for (int c = 0; c < kOD; ++c) o_acc[c] = 0.0f;

    auto step = [&](int ti, float4 (&kr)[kTV], float4 (&vr)[kTV]) __attribute__((always_inline)) {
            const int t0 = p0 + ti * kTile;
            const int tn = min(kTile, p1 - t0);  // <= 0 past the last tile
#pragma unroll
            for (int k = 0; k < kTV; ++k) {
                const int i = tid + k * kT;
                if (i < tn * hd4) {
                    const int j = i / hd4, c = i % hd4;
                    const bool is_new = t0 + j == pos;  // the cache row may still be the old one
                    *(float4*)(kt + j * ks + 4 * c) = sel4(is_new, *(const float4*)(kn + 4 * c), kr[k]);
                    *(float4*)(vt + j * hd + 4 * c) = sel4(is_new, *(const float4*)(vn + 4 * c), vr[k]);
                }
            }
            if constexpr (NB == 4) load_tile(tile_at(ti + 4), kr, vr);
            if (tn > 0) {
                bar();
                if (head_wave) {
                    // score of position lane in dot_f32's 8-lane order (quant.cpp:198-214).
                    // Unguarded and fully unrolled when hd is the instantiation's head size,
                    // so the LDS reads pipeline.
                    float v = -INFINITY;
                    if (HDM == 128 && hd == HDM) {
                        // 128-dim heads: both halves of the wave, lane j (< 32) takes the first
                        // half of position j's dims, lane j + 32 the second half (tiles are at
                        // most 32 positions), each in dot_f32's 8-lane order; the halves' sums
                        // then add across the lane swap. Halves the score's dependent chain:
                        // 1.3% per token at 4096 positions (Qwen2.5-1.5B shape); the 64-dim
                        // builds keep one lane per position (0.7% faster at 6-38 positions)
                        const int pj = lane & 31, h0 = (lane >> 5) * (HDM / 2);
                        float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                        if (pj < tn) {
                            const float* krow = kt + pj * ks + h0;
                            const float* qh = qr + h0;
#pragma unroll
                            for (int e = 0; e < HDM / 2; e += 8) {
                                const float4 q0 = *(const float4*)(qh + e), q1 = *(const float4*)(qh + e + 4);
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
                        }
                        const float sh = ((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7]));
                        const uint32_t u = __float_as_uint(sh);
                        const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
                        // lanes < 32: sw[0] is their own half, sw[1] lane + 32's
                        if (lane < tn) v = scale * (__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
                    } else if (lane < tn) {
                        const float* krow = kt + lane * ks;
                        float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                        auto dot8 = [&](int e) __attribute__((always_inline)) {
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
                        };
                        if (hd == HDM) {
#pragma unroll
                            for (int e = 0; e < HDM; e += 8) dot8(e);
                        } else {
                            for (int e = 0; e < hd; e += 8) dot8(e);
                        }
                        v = scale * (((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7])));
                    }
                    // online softmax over the tile (softmax, layers.cpp:25-35, one tile at a time)
                    const float m_new = fmaxf(m_run, wave_max(v));
                    const float e = lane < tn ? expf(v - m_new) : 0.0f;
                    const float l_tile = wave_sum(e);
                    const float alpha = expf(m_run - m_new);
                    m_run = m_new;
                    l_run = fmaf(l_run, alpha, l_tile);
                    // P.V: dim lane + 64 c, positions in order; p_j read from lane j
#pragma unroll
                    for (int c = 0; c < kOD; ++c) {
                        const int d = lane + c * kWave;
                        if (c * kWave < hd) {
                            const int dd = d < hd ? d : hd - 1;
                            float o = o_acc[c] * alpha;
                            // eight positions at a time with their V reads issued together
                            // (readlane is convergent: the compiler does not unroll a loop
                            // with a run-time trip count around it)
                            int j = 0;
                            for (; j + 8 <= tn; j += 8) {
                                float vv[8];
#pragma unroll
                                for (int u = 0; u < 8; ++u) vv[u] = vt[(j + u) * hd + dd];
#pragma unroll
                                for (int u = 0; u < 8; ++u)
                                    o = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j + u)), vv[u], o);
                            }
                            for (; j < tn; ++j)
                                o = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j)), vt[j * hd + dd], o);
                            o_acc[c] = o;
                        }
                    }
                }
                bar();
            }
    };
    if constexpr (NB == 4) {
        const int n_tiles = (p1 - p0 + kTile - 1) / kTile;
        for (int it = 0; it < n_tiles; it += 4) {
            step(it, kr0, vr0);
            step(it + 1, kr1, vr1);
            step(it + 2, kr2, vr2);
            step(it + 3, kr3, vr3);
        }
    } else {
        step(0, kr0, vr0);
        if constexpr (NB == 2) step(1, kr1, vr1);
    }
    if (head_wave) {
        const int r = wave;
#pragma unroll
        for (int c = 0; c < kOD; ++c) {
            const int d = lane + c * kWave;
            if (d < hd) {
                if constexpr (kPart)
                    out[r * ho + d] = o_acc[c];
                else
                    out[r * hd + d] = o_acc[c] / l_run;
            }
        }
        if constexpr (kPart) {
            if (lane == 0) {
                out[r * ho + hd] = m_run;
                out[r * ho + hd + 1] = l_run;
            }
        }
    }
    // the row's stores are done before this workgroup's next puts
    if (stores_row && wait_row) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    bar();
}

template <int HDM, class A, class Ly, class Fetch, class Bar>
__device__ __forceinline__ void attn_head(const A& a, const Ly& ly, int g, int pos, int start, float* qkv,
                                          float* sm, float* out, Fetch&& fetch, Bar&& bar, bool wait_row = true) {
    const int n = pos + 1 - start;
    if (n > 2 * kTile)
        attn_span<HDM, false, 4>(a, ly, g, pos, start, pos + 1, qkv, sm, out, fetch, bar, wait_row);
    else if (n > kTile)
        attn_span<HDM, false, 2>(a, ly, g, pos, start, pos + 1, qkv, sm, out, fetch, bar, wait_row);
    else
        attn_span<HDM, false, 1>(a, ly, g, pos, start, pos + 1, qkv, sm, out, fetch, bar, wait_row);
}

template <int HDM, class A, class Ly, class Fetch, class Bar>
__device__ __forceinline__ void attn_part(const A& a, const Ly& ly, int g, int pos, int p0, int p1,
                                          float* qkv, float* sm, float* out, Fetch&& fetch, Bar&& bar,
                                          bool wait_row = true) {
    if (p1 - p0 > 2 * kTile)
        attn_span<HDM, true, 4>(a, ly, g, pos, p0, p1, qkv, sm, out, fetch, bar, wait_row);
    else if (p1 - p0 > kTile)
        attn_span<HDM, true, 2>(a, ly, g, pos, p0, p1, qkv, sm, out, fetch, bar, wait_row);
    else
        attn_span<HDM, true, 1>(a, ly, g, pos, p0, p1, qkv, sm, out, fetch, bar, wait_row);
}

// Floats of LDS the attention scratch needs.
__host__ __device__ inline int attn_lds_floats(int n_rep, int hd) {
    return kTile * (hd + 4) + kTile * hd + n_rep * kTile + 3 * n_rep;
}

// The shared region: a GEMV input and its 16-element sums, the attention scratch, or the
// 2 * n_wg argmax words, whichever is largest.
__host__ __device__ inline int region_floats(int D, int F, int n_rep, int hd, int n_wg) {
    const int kmax = D > F ? D : F;
    int r = kmax + kmax / 16;
    const int att = attn_lds_floats(n_rep, hd);
    r = att > r ? att : r;
    return 2 * n_wg > r ? 2 * n_wg : r;
}

// Slices per query head in the layout where every workgroup splits: the largest power of
// two dividing hd with one workgroup per (head, slice) pair.
__host__ __device__ inline int split_all_parts(int H, int hd, int n_wg) {
    int parts = 1;
    while (2 * parts <= hd && hd % (2 * parts) == 0 && H * 2 * parts <= n_wg) parts *= 2;
    return parts;
}

// LDS bytes of one staged Q8_0 row of K elements (ffn_down staged one row per wave): the q
// bytes padded to whole 1 KiB load instructions, then the fp16 scales padded to 256-byte ones.
__host__ __device__ inline int row_slot_bytes(int K) {
    return (K + 1023) / 1024 * 1024 + (K / 16 + 255) / 256 * 256;
}

// ffn_down staged in LDS, split over K inside each workgroup (models with fewer down rows
// than half the waves, where one row per wave would leave most waves idle): workgroup w takes rows
// [w * R, w * R + R) of the D rows (R = down_rows), wave v a run of the F columns in units
// of 64 (two Q8_0 blocks, so a wave's fp16 scales are whole 4-byte words): the first F/64 % 8
// waves take one unit more. The waves of a workgroup thus read one eighth of the FFN's
// hidden vector each instead of all of it; the 8 partial sums of a row are added in wave
// order. A wave's slot: the R rows' q bytes (the largest run each), then their scales
// (4 bytes per unit, 16-byte aligned per row).
constexpr int kDownRowsMax = 4;  // R limit (d_model <= 4 x workgroups: the layout is for few rows)
__host__ __device__ inline int down_rows(int D, int n_wg) { return (D + n_wg - 1) / n_wg; }
__host__ __device__ inline int down_units_max(int F) { return (F / 64 + kNW - 1) / kNW; }
__host__ __device__ inline int down_unit0(int F, int v) { return v * (F / 64 / kNW) + min(v, F / 64 % kNW); }
__host__ __device__ inline int down_units(int F, int v) { return F / 64 / kNW + (v < F / 64 % kNW ? 1 : 0); }
__host__ __device__ inline int down_qstride(int F) { return 64 * down_units_max(F); }
__host__ __device__ inline int down_dstride(int F) { return (4 * down_units_max(F) + 15) / 16 * 16; }
__host__ __device__ inline int down_slot_bytes(int D, int F, int n_wg) {
    return down_rows(D, n_wg) * (down_qstride(F) + down_dstride(F));
}
__host__ __device__ inline bool down_split_ok(int D, int F, int n_wg) {
    return F % 64 == 0 && F / 64 >= kNW && down_units_max(F) <= kWave && down_rows(D, n_wg) <= kDownRowsMax;
}

// Launch constants, kept in LDS: phases re-read what they need after their barriers
// instead of holding dozens of kernel-wide values in registers across the whole launch.
struct StepConst {
    StepArgs a;
    int L, D, F, G, hd, n_rep, Hd, HB, nwg, P, attn_wg0;
    int A, parts, A_all, parts_all, PW;  // split attention: splits per kv head and slices per head of both layouts
    int o_xr, o_xs, o_x16, o_qkv, o_att;  // LDS byte offsets of the arrays below the layer table
    int o_down, down_slot;                // staged ffn_down rows (o_down 0: not staged), bytes per wave
    uint32_t e0;
    int pos0;
    u64 key0;
    // exchange buffers (word offsets into a.ex), each twice (layer or token parity)
    int XA, XB, QKV, ATT, HH, DONE, BEST, PART;
};

// TL: the layer matrices' format; TA: a second format wo and ffn_down may have, layer by
// layer (the runtime type picks the instantiation); TO: the lm_head's (and embedding's).
// DSPLIT: ffn_down staged split over K in each workgroup (else a row per wave, when staged);
// a template argument so that the row-per-wave build carries none of the split's code.
// UQ: lane steps per tile of the d_model-long Q8_0 rows (QKV, wo, gate/up, lm_head): 2 covers a
// 2048-element row in one tile; 1 for rows of at most 1024 elements (one tile of 64 lanes
// already covers them, and a second step would be masked out on most lanes: the
// Qwen2.5-0.5B shape's 896-element rows decode 7% faster with 1, the 2048-element rows of
// Llama-3.2-1B 3% slower).
template <int TL, int TO, int HDM, int TA, bool DSPLIT, int UQ>
__global__ __launch_bounds__(kT, 1) void k_step(const StepArgs args) {
    using FE = Fmt<TO>;  // the embedding table has the lm_head's format (checked by the host)
    constexpr bool kSums = Fmt<TL>::kNeedSums || Fmt<TA>::kNeedSums;  // inputs of wo and ffn_down
    // lane steps per tile of the d_model-long rows (QKV, wo, gate/up, lm_head): one for the
    // 32-element formats, whose 2048-element rows are 64 steps (a second would be masked
    // out on every lane); ffn_down's n_ff-long rows keep two
    constexpr int UL = Fmt<TL>::E >= 32 ? 1 : UQ, UA = Fmt<TA>::E >= 32 ? 1 : UQ, UO = Fmt<TO>::E >= 32 ? 1 : UQ;
    // copies of the wo output words: measured faster for the Q8_0 head-size-64 builds
    // (Llama-3.2-1B shape 0.511 -> 0.501, Qwen2.5-0.5B 0.599 -> 0.589 ms per token), slower for
    // the others (mixed Q4, Qwen2.5-1.5B: +0.9 %); copies of the ffn_down output words too
    // gave most of the gain back
    constexpr int RX = TL == TF_HIP_TYPE_Q8_0 && HDM == 64 ? kXRep : 1;
    constexpr int NWR = 8;  // norm weights per thread: d_model <= 4096
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ __align__(16) unsigned char sc_raw[sizeof(StepConst)];  // StepConst is not trivially constructible
    StepConst& sc = *reinterpret_cast<StepConst*>(sc_raw);
    __shared__ double red[kNW];
    __shared__ u64 wbest[kNW];
    __shared__ float dpart[DSPLIT ? kNW * kDownRowsMax : 1];  // split ffn_down: partial sums [wave][row]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x;
    StepLayer* lay = (StepLayer*)smem;
    if (tid == 0) {
        StepConst& c = sc;
        c.a = args;
        c.L = args.n_layer;
        c.D = args.D;
        c.F = args.F;
        c.G = args.G;
        c.hd = args.hd;
        c.n_rep = args.H / args.G;
        c.Hd = args.H * args.hd;
        c.HB = (c.n_rep + 2) * args.hd;  // words of one kv head block [q heads | k | v]
        c.nwg = gridDim.x;
        c.P = 6 * c.L + 8;               // epochs per token
        c.A = args.split;                // > 0: splits per kv head of the long-cache attention (trailing layout)
        c.attn_wg0 = c.nwg - c.G * (c.A ? c.A : 1);  // workgroups attn_wg0.. run a split token's attention
        c.parts = c.A ? c.A / c.n_rep : 1;  // each attention workgroup then merges hd / parts outputs of one head
        c.A_all = args.split_all;        // > 0: splits per kv head when every workgroup splits
        c.parts_all = split_all_parts(args.H, c.hd, c.nwg);
        c.PW = args.H * (c.A > c.A_all ? c.A : c.A_all) * (c.hd + 2);  // words of one parity of PART
        const int kmax = c.D > c.F ? c.D : c.F;
        c.o_xr = (int)(((size_t)c.L * sizeof(StepLayer) + 15) / 16 * 16);
        c.o_xs = c.o_xr + 4 * ((c.D + 3) / 4 * 4);
        c.o_x16 = c.o_xs + 4 * kmax;
        c.o_qkv = c.o_xs + 4 * ((region_floats(c.D, c.F, c.n_rep, c.hd, c.nwg) + 3) / 4 * 4);
        c.o_att = c.o_qkv + 4 * c.HB;
        c.down_slot = DSPLIT ? down_slot_bytes(c.D, c.F, c.nwg) : row_slot_bytes(c.F);
        c.o_down = (args.stage_lds & 3) ? (c.o_att + 4 * c.n_rep * (c.hd + 2) + 15) / 16 * 16 : 0;
        c.e0 = args.ctl->epoch;
        c.pos0 = args.ctl->pos;
        c.key0 = args.ctl->key;
        c.XA = 0;
        c.XB = c.XA + 2 * c.D;
        c.QKV = c.XB + 2 * RX * c.D;
        c.ATT = c.QKV + 2 * c.G * c.HB;
        c.HH = c.ATT + 2 * c.Hd;
        c.DONE = c.HH + 2 * c.F;
        c.BEST = c.DONE + 2 * c.nwg;
        c.PART = c.BEST + 4 * c.nwg;
    }
    {
        const u64* src = (const u64*)args.layers;
        u64* dst = (u64*)lay;
        const int nw = (int)(args.n_layer * sizeof(StepLayer) / 8);
        for (int i = tid; i < nw; i += kT) dst[i] = src[i];
    }
    __syncthreads();
    float* xr = (float*)(smem + sc.o_xr);
    float* xs = (float*)(smem + sc.o_xs);
    float* x16 = (float*)(smem + sc.o_x16);
    auto E = [&](int t, int l, int p) -> uint32_t { return sc.e0 + (uint32_t)(t * sc.P + 6 * l + p); };
    auto X = [&](int off) -> u64* { return sc.a.ex + off; };
    auto no_bias = [](int) -> const float* { return nullptr; };
    const int n_tokens = args.n_tokens;
    int tok = 0;
    // Staged weight rows: a wave copies a Q8_0 or Q4_0 row (qbytes of quants, then its fp16
    // scales, K / 16 bytes for both formats) into an LDS slot of its own with direct
    // global->LDS loads, ahead of the phase that reads it: lane i of a load lands at slot +
    // 16 i (4 i for the scales). The scales start at the slot's Q8_0 offset (K rounded up to
    // 1 KiB) for both formats. Lanes past the row's end re-read its last bytes; what they
    // write past the row is never read.
    auto stage_row = [&](const uint8_t* q, int qbytes, const uint8_t* d, int K, unsigned char* slot) {
        const int qsteps = (qbytes + 1023) / 1024, dbytes = K / 16, dsteps = (dbytes + 255) / 256;
        for (int i = 0; i < qsteps; ++i) {
            int o = 1024 * i + 16 * lane;
            o = o < qbytes ? o : qbytes - 16;
            __builtin_amdgcn_global_load_lds((const TF_GLOBAL void*)(q + o),
                                             (__attribute__((address_space(3))) void*)(slot + 1024 * i), 16, 0, 0);
        }
        unsigned char* dslot = slot + (K + 1023) / 1024 * 1024;
        for (int i = 0; i < dsteps; ++i) {
            int o = 256 * i + 4 * lane;
            o = o < dbytes ? o : dbytes - 4;
            __builtin_amdgcn_global_load_lds((const TF_GLOBAL void*)(d + o),
                                             (__attribute__((address_space(3))) void*)(dslot + 256 * i), 4, 0, 0);
        }
    };
    // Dot of the staged row in `slot` with xs (format TL), in gemv_phase's lane-step order
    // and reduction, so the same bits as the register path.
    auto staged_dot = [&](const unsigned char* slot, int K) -> float {
        using FS = Fmt<TL == TF_HIP_TYPE_Q4_0 ? TF_HIP_TYPE_Q4_0 : TF_HIP_TYPE_Q8_0>;
        const uint16_t* dsl = (const uint16_t*)(slot + (K + 1023) / 1024 * 1024);
        float acc = 0.0f;
        for (int s = lane; s < K / FS::E; s += kWave) {
            typename FS::Raw w;
            w.q = *(const uint4*)(slot + 16 * s);
            w.d = FS::E == 16 ? dsl[s >> 1] : dsl[s];  // one fp16 scale per 32 elements
            acc += FS::dot(w, xs, x16, s);
        }
        return wave_sum(acc);
    };
    // Staged ffn_down (Q8_0), split layout: wave v copies its run of columns of its workgroup's R rows into
    // its own LDS slot with direct global->LDS loads, ahead of the down phase (lane i of a
    // load lands at +16 i for the q bytes, +4 i for the scales). Lanes past the run load
    // nothing.
    auto issue_down = [&](const StepLayer& ly) {
        if constexpr (TL == TF_HIP_TYPE_Q8_0 || TL == TF_HIP_TYPE_Q4_0) {
            if constexpr (!DSPLIT) {
                // one row per wave: row wid. (One return for both conditions: with two, the
                // compiler's wait-count pass put an s_waitcnt vmcnt(0) after the staging, for
                // the LDS reads that follow, and the gate/up phase then waited for the row;
                // measured as 2% of the Qwen2.5-1.5B shape's token time.)
                // A layer whose ffn_down has the other format (TA) is not staged.
                const int wid = wg * kNW + wave;
                if (sc.o_down == 0 || wid >= (int)ly.wd.N || (int)ly.wd.type != TL) return;
                const int K = sc.F, qbytes = TL == TF_HIP_TYPE_Q8_0 ? K : K / 2;
                stage_row(ly.wd.q + (int64_t)wid * qbytes, qbytes, ly.wd.s + (int64_t)wid * (K / 16), K,
                          smem + sc.o_down + wave * sc.down_slot);
                return;
            }
            if (sc.o_down == 0) return;
            const int F = sc.F, R = down_rows(sc.D, sc.nwg), u0 = down_unit0(F, wave), nu = down_units(F, wave);
            const int r0 = wg * R, nr = min(R, (int)ly.wd.N - r0);
            const int qs = down_qstride(F), ds = down_dstride(F);
            unsigned char* slot = smem + sc.o_down + wave * sc.down_slot;
            unsigned char* dslot = slot + R * qs;
            for (int r = 0; r < nr; ++r) {
                const uint8_t* q = ly.wd.q + (int64_t)(r0 + r) * F + 64 * u0;
                const uint8_t* d = ly.wd.s + (int64_t)(r0 + r) * (F / 16) + 4 * u0;
                for (int i = 0; i < 64 * nu; i += 1024)
                    if (i + 16 * lane < 64 * nu)
                        __builtin_amdgcn_global_load_lds((const TF_GLOBAL void*)(q + i + 16 * lane),
                                                         (__attribute__((address_space(3))) void*)(slot + r * qs + i),
                                                         16, 0, 0);
                if (lane < nu)
                    __builtin_amdgcn_global_load_lds((const TF_GLOBAL void*)(d + 4 * lane),
                                                     (__attribute__((address_space(3))) void*)(dslot + r * ds), 4, 0,
                                                     0);
            }
        }
    };
    // The down phase on the staged slices: wave v's partial sums of its rows over its
    // columns (lane steps of 16 elements in order, each a Q8_0 step dot as in the GEMV, then
    // the wave reduction), into dpart[v][r]; the caller adds the 8 partials of a row. RM is
    // a compile-time row count >= the workgroup's rows: each step's inputs are read once for
    // all rows, and rows past nr re-read the last row (no branch between the LDS reads).
    auto staged_down_rm = [&](float* dpart, auto rm) {
        constexpr int RM = decltype(rm)::value;
        using F8 = Fmt<TF_HIP_TYPE_Q8_0>;
        const int F = sc.F, R = down_rows(sc.D, sc.nwg), u0 = down_unit0(F, wave), nu = down_units(F, wave);
        const int nr = min(R, sc.D - wg * R);
        if (nr <= 0) return;
        const int qs = down_qstride(F), ds = down_dstride(F);
        const unsigned char* slot = smem + sc.o_down + wave * sc.down_slot;
        const unsigned char* dslot = slot + R * qs;
        float acc[RM];
#pragma unroll
        for (int r = 0; r < RM; ++r) acc[r] = 0.0f;
        for (int j = lane; j < 4 * nu; j += kWave) {
            const float4* x4 = (const float4*)(xs + 16 * (4 * u0 + j));  // the step's inputs in the whole row
            const float4 x[4] = {x4[0], x4[1], x4[2], x4[3]};
#pragma unroll
            for (int r = 0; r < RM; ++r) {
                const int rr = r < nr ? r : nr - 1;
                typename F8::Raw w;
                w.q = *(const uint4*)(slot + rr * qs + 16 * j);
                w.d = ((const uint16_t*)(dslot + rr * ds))[j >> 1];
                acc[r] += F8::dot_x(w, x);
            }
        }
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            const float v = wave_sum(acc[r]);
            if (lane == 0 && r < nr) dpart[wave * kDownRowsMax + r] = v;
        }
    };
    auto staged_down = [&](float* dpart) {
        const int R = down_rows(sc.D, sc.nwg);
        if (R <= 2) staged_down_rm(dpart, std::integral_constant<int, 2>());
        else staged_down_rm(dpart, std::integral_constant<int, kDownRowsMax>());
    };

    for (int t = 0; t < n_tokens; ++t) {
        const bool last = t == n_tokens - 1;
        for (int l = 0; l < sc.L; ++l) {
            const StepLayer& ly = lay[l];
            const int par = l & 1;
            // split attention layout of this token (caches longer than 512 positions), see phase 2
            const int span = sc.pos0 + t + 1 - sc.a.att_start;
            const bool all = sc.A_all && span > sc.a.split_all_from;
            // short spans attend on one workgroup per kv head (attn_head), longer ones split
            const bool split = sc.A && (all || span > sc.a.split_from);
            const int attn_wg0 = split ? sc.attn_wg0 : sc.nwg - sc.G;
            // copies of the wo output words this token (one when every workgroup splits the
            // attention: measured slower with copies, Llama-3.2-1B shape after 2,000 tokens)
            const int rx = all ? 1 : RX;
            // ---- 1: QKV (attn_norm fused)
            {
                const int D = sc.D;
                float wr[NWR];
                load_norm(ly.attn_norm, D, wr);
                const int groups[3] = {(int)ly.wq.N, (int)ly.wk.N, (int)ly.wv.N};
                auto seg = [&](int si, int) -> const DevMat& { return si == 0 ? ly.wq : si == 1 ? ly.wk : ly.wv; };
                auto bias = [&](int si) -> const float* { return si == 0 ? ly.bq : si == 1 ? ly.bk : ly.bv; };
                auto prep = [&]() {
                    const StepArgs& a = sc.a;
                    const int pos = sc.pos0 + t;
                    if (l == 0) {
                        // the token: staged in hist, or the previous token's argmax
                        if (t > 0) {
                            if (a.greedy) {
                                float* kb = xs;  // free: the barrier before prep has passed
                                gather<kGW, 1>(X(sc.BEST) + ((t - 1) & 1) * 2 * sc.nwg, 2 * sc.nwg, E(t - 1, sc.L, 6),
                                               kb, nullptr, 0, 0, a.ctl);
                                __syncthreads();
                                if (tid == 0) {
                                    u64 b = 0;
                                    for (int i = 0; i < sc.nwg; ++i) {
                                        const u64 k = ((u64)__float_as_uint(kb[2 * i]) << 32) |
                                                      (u64)__float_as_uint(kb[2 * i + 1]);
                                        b = k > b ? k : b;
                                    }
                                    wbest[0] = b;
                                }
                                __syncthreads();
                                tok = key_to_index(wbest[0]);
                            } else {
                                gather<1, kGW>(nullptr, 0, 0, nullptr, X(sc.DONE) + ((sc.L - 1) & 1) * sc.nwg, sc.nwg,
                                               E(t - 1, sc.L - 1, 5), a.ctl);
                                tok = *gptr(a.hist + pos);
                            }
                        } else {
                            tok = a.greedy ? key_to_index(sc.key0) : *gptr(a.hist + pos);
                        }
                        if (tok < 0 || tok >= (int)a.embd.N) {
                            if (tid == 0) set_err(a.ctl, kErrToken);
                            tok = 0;
                        }
                        if (wg == 0 && tid == 0) {
                            *gptr(a.hist + pos) = tok;
                            *gptr(&a.ctl->last_token) = tok;
                        }
                        // dequant_row of the token's row (model.cpp:199)
                        const RowPtr rp = FE::row(a.embd, tok);
                        for (int s = tid; s < D / FE::E; s += kT) {
                            float v[FE::E];
                            FE::dequant(FE::load(rp, s), v);
#pragma unroll
                            for (int i = 0; i < FE::E; ++i) xr[s * FE::E + i] = v[i];
                        }
                    } else {
                        gather<kGD, kGW>(X(sc.XA) + ((l - 1) & 1) * D, D, E(t, l - 1, 5), xr,
                                         X(sc.DONE) + ((l - 1) & 1) * sc.nwg, sc.nwg, E(t, l - 1, 5), a.ctl);
                    }
                    stage(xr, D, true, wr, a.eps, xs, x16, Fmt<TL>::kNeedSums, red);
                };
                auto epi = [&](int si, int row, float v, float, float extra) {
                    const int hd = sc.hd, n_rep = sc.n_rep, HB = sc.HB;
                    int idx;
                    if (si == 0) {  // q row of head h = row / hd
                        const int h = row / hd;
                        idx = (h / n_rep) * HB + (h % n_rep) * hd + row % hd;
                    } else {        // k or v row of kv head row / hd
                        idx = (row / hd) * HB + (n_rep + si - 1) * hd + row % hd;
                    }
                    put(X(sc.QKV) + par * sc.G * HB + idx, bias(si) ? v + extra : v, E(t, l, 1));
                };
                gemv_phase<TL, 1, GEMV_STORE, UL>(3, groups, seg, bias, D, wg * kNW + wave, sc.nwg * kNW, xs, x16,
                                                 prep, epi);
            }
            // ---- 2: attention (kv head g on workgroup attn_wg0 + g), then 4: gate/up
            // ---- 3: wo + residual (workgroups without an attention head), then 4: gate/up
            // The workgroups without an attention head issue their gate/up tiles and stage
            // their ffn_down row before they wait for the attention output: a 1B model's 53 MB
            // of gate/up and down per layer stream in while attention runs, not after wo. (The
            // attention workgroups take no wo rows: with their gate/up and ffn_down loads issued
            // before wo they are wo's stragglers, after it gate/up's.)
            {
                const int D = sc.D;
                float wr[NWR];
                load_norm(ly.ffn_norm, D, wr);
                // gate/up rows per group: one for Q8_0 (gate/up rows are then dealt one at a
                // time, so no wave holds a whole group more than another: 8960 rows on 2048
                // waves give 5 or 4 instead of 3 or 2 pairs, and two streams per wave keep
                // enough loads in flight), two for the 4-bit formats (their rows are half the
                // bytes; one row per group measured 1.8% slower on the mixed-Q4 model)
                constexpr int kGuR = TL == TF_HIP_TYPE_Q8_0 ? 1 : 2;
                const int gu_groups[3] = {(int)((ly.wg.N + kGuR - 1) / kGuR), 0, 0};
                auto gu_seg = [&](int, int what) -> const DevMat& { return what == 1 ? ly.wu : ly.wg; };
                auto gu_epi = [&](int, int row, float v, float up, float) {
                    put(X(sc.HH) + par * sc.F + row, (v / (1.0f + expf(-v))) * up, E(t, l, 4));
                };
                auto gu_input = [&]() {
                    gather<kGD, 1>(X(sc.XB) + (par * RX + wg % rx) * D, D, E(t, l, 3), xr, nullptr, 0, 0, sc.a.ctl);
                    stage(xr, D, true, wr, sc.a.eps, xs, x16, Fmt<TL>::kNeedSums, red);
                };
                // ---- 3: wo + residual, rows dealt over nw waves from wave 0
                auto wo_phase = [&](int nw) {
                    const int Hd = sc.Hd;
                    // rows dealt round the waves starting where the QKV rows ended, so that a
                    // wave with a QKV row more than the rest does not also get one more wo row
                    const int rot = (int)((ly.wq.N + ly.wk.N + ly.wv.N) % (sc.nwg * kNW)) % nw;
                    const int wid = (wg * kNW + wave + nw - rot) % nw;
                    float wo_wr[1];
                    const int groups[3] = {(int)ly.wo.N, 0, 0};
                    auto seg = [&](int, int) -> const DevMat& { return ly.wo; };
                    auto prep = [&]() {
                        gather<kGD, 1>(X(sc.ATT) + par * Hd, Hd, E(t, l, 2), xs, nullptr, 0, 0, sc.a.ctl);
                        stage(xs, Hd, false, wo_wr, 0.0f, xs, x16, kSums, red);
                    };
                    auto epi = [&](int, int row, float v, float, float) {
                        const float nv = xr[row] + v;
#pragma unroll
                        for (int r = 0; r < RX; ++r)
                            if (r < rx) put(X(sc.XB) + (par * RX + r) * sc.D + row, nv, E(t, l, 3));
                    };
                    if (TA != TL && ly.wo.type == TA)
                        gemv_phase<TA, 1, GEMV_RESID, UA>(1, groups, seg, no_bias, Hd, wid, nw, xs, x16, prep, epi);
                    else
                        gemv_phase<TL, 1, GEMV_RESID, UL>(1, groups, seg, no_bias, Hd, wid, nw, xs, x16, prep, epi);
                };
                // ---- 2 (caches longer than 512 positions): kv head g's positions split over
                // A workgroups, then each (query head, slice of hd / parts outputs) merged
                // from the A partials by one workgroup. Two layouts, chosen per token from
                // the span's length (the same on every workgroup):
                //   trailing: the G * A workgroups from attn_wg0 on split and merge while the
                //     others start the FFN's and wo's loads; best while a split's share of the
                //     scores and P.V is small (spans up to split_all_from);
                //   all: workgroups 0.. split (A_all per kv head) and merge, then every
                //     workgroup runs wo; more splits, shorter ones, for long spans.
                // The partials carry epoch slot 6 of the layer (unused by the other phases;
                // the argmax words use it only past the last layer; never 0).
                if (split && (all || wg >= attn_wg0)) {
                    const int A = all ? sc.A_all : sc.A, parts = all ? sc.parts_all : sc.parts;
                    const int G = sc.G, HB = sc.HB, n_rep = sc.n_rep, hd = sc.hd, ho = hd + 2;
                    const int aw = all ? wg : wg - attn_wg0;
                    u64* pb = X(sc.PART) + par * sc.PW;
                    float* qkv = (float*)(smem + sc.o_qkv);
                    float* part = (float*)(smem + sc.o_att);
                    __syncthreads();  // the QKV phase's waves are done with xs
                    if (aw < G * A) {
                        const int g = aw % G, s = aw / G;
                        const int pos = sc.pos0 + t, start = sc.a.att_start;
                        const int chunk = (pos + 1 - start + A - 1) / A;
                        const int p0 = start + s * chunk, p1 = min(pos + 1, p0 + chunk);
                        // trailing layout: the stored row is waited for after attention, off the
                        // chain (the workgroup then waits for wo's output anyway)
                        attn_part<HDM>(sc.a, ly, g, pos, p0, p1, qkv, xs, part, [&]() {
                            gather<kGD, 1>(X(sc.QKV) + par * G * HB + g * HB, HB, E(t, l, 1), qkv, nullptr, 0, 0,
                                           sc.a.ctl);
                            __syncthreads();
                        }, [] { __syncthreads(); }, all);
                        u64* pw_base = pb + (size_t)(g * A + s) * n_rep * ho;
                        for (int i = tid; i < n_rep * ho; i += kT) put(pw_base + i, part[i], E(t, l, 6));
                    }
                    if (aw < sc.a.H * parts) {
                        const int sz = hd / parts;
                        const int h = aw / parts, d0 = (aw % parts) * sz;
                        const int g = h / n_rep, r = h % n_rep, w = sz + 2;
                        float* buf = xs;  // [A][sz, m, l]
                        __syncthreads();
                        gather_idx<3>(pb, [&](int j) {
                            const int s = j / w, k = j % w;
                            return (size_t)((g * A + s) * n_rep + r) * ho + (k < sz ? d0 + k : hd + k - sz);
                        }, A * w, E(t, l, 6), buf, sc.a.ctl);
                        __syncthreads();
                        for (int k = wave; k < sz; k += kNW) {
                            float m = -INFINITY;
                            for (int s = lane; s < A; s += kWave) m = fmaxf(m, buf[s * w + sz]);
                            m = wave_max(m);
                            float lsum = 0.0f, osum = 0.0f;
                            for (int s = lane; s < A; s += kWave) {
                                const float wt = expf(buf[s * w + sz] - m);
                                lsum = fmaf(buf[s * w + sz + 1], wt, lsum);
                                osum = fmaf(buf[s * w + k], wt, osum);
                            }
                            lsum = wave_sum(lsum);
                            osum = wave_sum(osum);
                            if (lane == 0) put(X(sc.ATT) + par * sc.Hd + h * hd + d0 + k, osum / lsum, E(t, l, 2));
                        }
                    }
                }
                // an attention workgroup that left its K/V row stores in flight waits for them
                // (the waves that stored) before it issues the FFN's loads: wo's output is
                // still a hand-off away, and the end-of-layer word comes after this
                auto row_stores_done = [&]() {
                    if (wave * kWave < sc.hd) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                };
                if (split && !all && wg >= attn_wg0) {
                    auto down_then_input = [&]() {
                        row_stores_done();
                        issue_down(ly);
                        gu_input();
                    };
                    gemv_phase<TL, kGuR, GEMV_SILU, UL>(1, gu_groups, gu_seg, no_bias, D, wg * kNW + wave, sc.nwg * kNW, xs,
                                                    x16, down_then_input, gu_epi);
                } else if (!split && wg >= attn_wg0) {
                    const int g = wg - attn_wg0;
                    const int HB = sc.HB;
                    float* qkv = (float*)(smem + sc.o_qkv);
                    float* att_out = (float*)(smem + sc.o_att);
                    __syncthreads();  // the QKV phase's waves are done with xs
                    attn_head<HDM>(sc.a, ly, g, sc.pos0 + t, sc.a.att_start, qkv, xs, att_out, [&]() {
                        gather<kGD, 1>(X(sc.QKV) + par * sc.G * HB + g * HB, HB, E(t, l, 1), qkv, nullptr, 0, 0,
                                       sc.a.ctl);
                        __syncthreads();
                    }, [] { __syncthreads(); }, false);
                    const int nh = sc.n_rep * sc.hd;
                    for (int i = tid; i < nh; i += kT) put(X(sc.ATT) + par * sc.Hd + g * nh + i, att_out[i], E(t, l, 2));
                    auto down_then_input = [&]() {
                        row_stores_done();
                        issue_down(ly);
                        gu_input();
                    };
                    gemv_phase<TL, kGuR, GEMV_SILU, UL>(1, gu_groups, gu_seg, no_bias, D, wg * kNW + wave, sc.nwg * kNW, xs,
                                                    x16, down_then_input, gu_epi);
                } else if (all) {
                    // Every workgroup split the attention: the merged output comes right after
                    // the merge, so gate/up's tiles wait until wo is done. (A wave's loads
                    // complete in issue order and the CU's vector memory path is one queue:
                    // every load issued before the attention-output polls delays them.)
                    issue_down(ly);
                    wo_phase(sc.nwg * kNW);
                    gemv_phase<TL, kGuR, GEMV_SILU, UL>(1, gu_groups, gu_seg, no_bias, D, wg * kNW + wave, sc.nwg * kNW, xs,
                                                    x16, gu_input, gu_epi);
                } else {
                    // The attention runs on other workgroups for several microseconds: gate/up's
                    // first tiles and the ffn_down rows stream in meanwhile.
                    auto wo_then_input = [&]() {
                        issue_down(ly);
                        wo_phase(attn_wg0 * kNW);
                        __syncthreads();  // every wave's wo rows are read out of xs before the input is staged
                        gu_input();
                    };
                    gemv_phase<TL, kGuR, GEMV_SILU, UL>(1, gu_groups, gu_seg, no_bias, D, wg * kNW + wave, sc.nwg * kNW, xs,
                                                    x16, wo_then_input, gu_epi);
                }
            }
            // ---- 5: down + residual
            {
                const int F = sc.F;
                float wr[1];
                const int groups[3] = {(int)ly.wd.N, 0, 0};
                auto seg = [&](int, int) -> const DevMat& { return ly.wd; };
                auto prep = [&]() {
                    gather<kGF, 1>(X(sc.HH) + par * F, F, E(t, l, 4), xs, nullptr, 0, 0, sc.a.ctl);
                    stage(xs, F, false, wr, 0.0f, xs, x16, kSums, red);
                };
                auto epi = [&](int, int row, float v, float, float) {
                    const float nv = xr[row] + v;
                    put(X(sc.XA) + par * sc.D + row, nv, E(t, l, 5));
                    if (last && sc.a.taps) *gptr(sc.a.taps + (size_t)l * sc.D + row) = nv;
                };
                bool staged = false;
                if constexpr (TL == TF_HIP_TYPE_Q8_0 || TL == TF_HIP_TYPE_Q4_0) {
                    if (sc.o_down && (int)ly.wd.type == TL) {
                        // the slices were staged in LDS during gate/up
                        staged = true;
                        __syncthreads();
                        prep();
                        // a wave's loads complete in order and the exchange loads of prep came
                        // after its staged slices or row: the waits below are already satisfied
                        if constexpr (DSPLIT) {
                            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                            staged_down(dpart);
                            __syncthreads();
                            const int R = down_rows(sc.D, sc.nwg), r0 = wg * R;
                            if (tid < R && r0 + tid < sc.D) {
                                float v = dpart[tid];
                                for (int w = 1; w < kNW; ++w) v += dpart[w * kDownRowsMax + tid];
                                epi(0, r0 + tid, v, 0.0f, 0.0f);
                            }
                        } else {
                            const int wid = wg * kNW + wave;
                            if (wid < (int)ly.wd.N) {  // waves without a row do not wait
                                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                                const float acc = staged_dot(smem + sc.o_down + wave * sc.down_slot, F);
                                if (lane == 0) epi(0, wid, acc, 0.0f, 0.0f);
                            }
                        }
                    }
                }
                if (!staged) {
                    if (TA != TL && ly.wd.type == TA)
                        gemv_phase<TA, 1, GEMV_RESID, 2>(1, groups, seg, no_bias, F, wg * kNW + wave, sc.nwg * kNW,
                                                         xs, x16, prep, epi);
                    else
                        gemv_phase<TL, 1, GEMV_RESID, 2>(1, groups, seg, no_bias, F, wg * kNW + wave, sc.nwg * kNW,
                                                         xs, x16, prep, epi);
                }
                __syncthreads();
                if (tid == 0) put(X(sc.DONE) + par * sc.nwg + wg, 0.0f, E(t, l, 5));
            }
        }
        // ---- output_norm + lm_head + greedy argmax
        if (sc.a.lm_every || last) {
            const int D = sc.D;
            float wr[NWR];
            load_norm(sc.a.out_norm, D, wr);
            const int groups[3] = {(int)((sc.a.out.N + 1) / 2), 0, 0};
            auto seg = [&](int, int) -> const DevMat& { return sc.a.out; };
            auto prep = [&]() {
                const int Lm = sc.L - 1;
                gather<kGD, kGW>(X(sc.XA) + (Lm & 1) * D, D, E(t, Lm, 5), xr, X(sc.DONE) + (Lm & 1) * sc.nwg, sc.nwg,
                                 E(t, Lm, 5), sc.a.ctl);
                stage(xr, D, true, wr, sc.a.eps, xs, x16, Fmt<TO>::kNeedSums, red);
                if (last && sc.a.taps && wg == 0)
                    for (int j = tid; j < D; j += kT) *gptr(sc.a.taps + (size_t)sc.L * D + j) = xs[j];
            };
            u64 best = 0;
            auto epi = [&](int, int row, float v, float, float) {
                if (last && sc.a.logits) *gptr(sc.a.logits + row) = v;
                const u64 k = argmax_key(v, row);
                best = k > best ? k : best;
            };
            gemv_phase<TO, 2, GEMV_LOGITS, UO>(1, groups, seg, no_bias, D, wg * kNW + wave, sc.nwg * kNW, xs, x16,
                                              prep, epi);
            best = wave_max_u64(best);
            if (lane == 0) wbest[wave] = best;
            __syncthreads();
            if (tid == 0) {
                u64 b = wbest[0];
                for (int i = 1; i < kNW; ++i) b = wbest[i] > b ? wbest[i] : b;
                u64* bw = X(sc.BEST) + (t & 1) * 2 * sc.nwg + 2 * wg;
                put(bw, __uint_as_float((uint32_t)(b >> 32)), E(t, sc.L, 6));
                put(bw + 1, __uint_as_float((uint32_t)b), E(t, sc.L, 6));
            }
            __syncthreads();
        }
    }
    // workgroup 0 folds the last token's keys and advances the control block
    if (wg == 0) {
        const int t = n_tokens - 1;
        float* kb = xs;
        __syncthreads();
        gather<kGW, 1>(X(sc.BEST) + (t & 1) * 2 * sc.nwg, 2 * sc.nwg, E(t, sc.L, 6), kb, nullptr, 0, 0, sc.a.ctl);
        __syncthreads();
        if (tid == 0) {
            u64 b = 0;
            for (int i = 0; i < sc.nwg; ++i) {
                const u64 k = ((u64)__float_as_uint(kb[2 * i]) << 32) | (u64)__float_as_uint(kb[2 * i + 1]);
                b = k > b ? k : b;
            }
            TF_GLOBAL Ctl* ctl = gptr(sc.a.ctl);
            ctl->key = b;
            ctl->pos = sc.pos0 + n_tokens;
            ctl->epoch = sc.e0 + (uint32_t)(n_tokens * sc.P);
        }
    }
}

// Cooperative launch of one build, with the dynamic LDS the launch's arguments need.
template <int TL, int TO, int HDM, int TA = TL, bool DSPLIT = false, int UQ = 2>
hipError_t launch_t(const StepArgs& a, int n_wg, hipStream_t st) {
    const void* fn = (const void*)k_step<TL, TO, HDM, TA, DSPLIT, UQ>;
    const size_t lds = step_lds_bytes(a.n_layer, a.D, a.F, a.H, a.G, a.hd, n_wg, a.stage_lds);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kStepThreads, lds);
    if (e != hipSuccess) return e;
    if (per_cu < 1 || n_wg > per_cu * device_cu_count()) return hipErrorCooperativeLaunchTooLarge;
    StepArgs arg = a;
    void* params[] = {(void*)&arg};
    return hipLaunchCooperativeKernel(fn, dim3(n_wg), dim3(kStepThreads), params, (unsigned)lds, st);
}

}  // namespace step_detail
}  // namespace tfk
