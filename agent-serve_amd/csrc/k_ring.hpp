// Ring decode step: the step kernel's token loop (k_step.hpp: Model::decode, model.cpp:197-208,
// and the per-token layers of Model::prefill, model.cpp:144-195) with each CU's weights
// streamed through an LDS ring by a loader wave of its own.
//
// One cooperative launch, one workgroup of 9 waves per CU. Waves 0-7 compute: per layer the
// same five phases as the step kernel (QKV with attn_norm and bias, attention, wo +
// residual, gate/up with ffn_norm and SiLU, down + residual; then output_norm + lm_head +
// greedy argmax), the same epoch-word hand-offs between workgroups and the same attention
// code. Wave 8 is the loader: it copies, in the order the compute waves consume them, the
// workgroup's share of every phase -- norm weights, biases, then batches of 8 weight items
// -- from HBM into the ring with direct global->LDS loads, keeping at most RingArgs::cap of
// them in flight. A CU's memory path serves all its waves in order, so a deep burst of weight
// loads (the step kernel issues every wave's tiles ahead) makes the hand-off polls behind
// it slow; a bounded, continuous stream keeps HBM busy while the polls stay short, and the
// ring carries the weights across the latency-bound stretches of a layer (attention, the
// hand-offs) instead of registers.
//
// Protocol inside a workgroup (all in LDS, no global traffic):
//   landed    loader: units [0, landed) of the stream are in the ring (its loads complete in
//             order, so after s_waitcnt vmcnt(k) all but the last k have landed);
//   done[w]   compute wave w: units below done[w] are consumed (the loader refills only
//             below min(done) + ring size);
//   arrive    the compute waves' barrier: each adds one and waits until the count reaches
//             8 times the barriers it has passed (the loader takes no part, so it may block
//             on its loads at any time).
// Both sides walk the same schedule (phases, row shares, batch layout from RingArgs::ph), so
// unit positions agree without being exchanged. Every wait is bounded; past the limit a
// wave flags ctl->err and goes on, and the host reports the error.
#pragma once

#include "k_step.hpp"

namespace tfk {
namespace ring_detail {

using namespace step_detail;

constexpr int kRT = kT + kWave;  // 8 compute waves + the loader
constexpr int kUnit = 256;       // bytes per ring unit (one dword load of a wave)
constexpr int kCapMax = 48;      // loader loads in flight at most (RingArgs::cap)
constexpr int kLpiMax = 3;       // 1 KiB lines per item (P <= 3072)
constexpr int kBiasMax = 64;     // rows per workgroup of a phase with biases
#ifndef TF_RING_POLL_SLEEP
#define TF_RING_POLL_SLEEP 8
#endif
constexpr int kPollSleep = TF_RING_POLL_SLEEP;  // s_sleep between the hand-off polls' rounds
// Ctl::err codes of the ring's own waits (the exchange's is kErrTimeout)
constexpr int kErrLanded = 3;    // a compute wave waited too long for weights to land
constexpr int kErrSpace = 4;     // the loader waited too long for ring space

typedef __attribute__((address_space(3))) uint32_t lds_u32;

struct RingCtl {
    uint32_t landed, arrive, pad0, pad1;
    uint32_t done[kNW];
    unsigned long long wbest[kNW];
    int tok;
    int pad2[3];
};

__host__ __device__ inline int r_al16(int x) { return (x + 15) / 16 * 16; }

// LDS layout (byte offsets), the same on host and device.
struct RingLds {
    int args, table, ctl, xr, xr2, xin, qkv, att, part, bias, ring, total;
};
__host__ __device__ inline RingLds ring_lds(int L, int D, int F, int H, int G, int hd, int nwg, int part_floats,
                                            int ring_units) {
    RingLds o;
    const int n_rep = H / G;
    o.args = 0;
    o.table = r_al16((int)sizeof(RingArgs));
    o.ctl = r_al16(o.table + L * (int)sizeof(RingLayer));
    o.xr = r_al16(o.ctl + (int)sizeof(RingCtl));
    o.xr2 = r_al16(o.xr + 4 * D);
    o.xin = r_al16(o.xr2 + 4 * D);
    o.qkv = r_al16(o.xin + 4 * region_floats(D, F, n_rep, hd, nwg));
    o.att = r_al16(o.qkv + 4 * (n_rep + 2) * hd);
    o.part = r_al16(o.att + 4 * n_rep * (hd + 2));
    o.bias = r_al16(o.part + 4 * part_floats);
    o.ring = (o.bias + 4 * kBiasMax + 1023) / 1024 * 1024;
    o.total = o.ring + ring_units * kUnit;
    return o;
}

// Contiguous row share [r0, r1) of participant idx of n.
__device__ __forceinline__ void share(int N, int n, int idx, int& r0, int& r1) {
    r0 = (int)((int64_t)N * idx / n);
    r1 = (int)((int64_t)N * (idx + 1) / n);
}

__device__ __forceinline__ uint32_t lds_ld(const lds_u32* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_st(lds_u32* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// a - b < 0 for counters that may wrap
__device__ __forceinline__ bool before(uint32_t a, uint32_t b) { return (int32_t)(a - b) < 0; }

// s_waitcnt vmcnt(n), n <= kCapMax (larger n wait for everything).
__device__ __forceinline__ void wait_vm(int n) {
    switch (n) {
#define TF_W(k) \
    case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
        TF_W(0) TF_W(1) TF_W(2) TF_W(3) TF_W(4) TF_W(5) TF_W(6) TF_W(7)
        TF_W(8) TF_W(9) TF_W(10) TF_W(11) TF_W(12) TF_W(13) TF_W(14) TF_W(15)
        TF_W(16) TF_W(17) TF_W(18) TF_W(19) TF_W(20) TF_W(21) TF_W(22) TF_W(23)
        TF_W(24) TF_W(25) TF_W(26) TF_W(27) TF_W(28) TF_W(29) TF_W(30) TF_W(31)
        TF_W(32) TF_W(33) TF_W(34) TF_W(35) TF_W(36) TF_W(37) TF_W(38) TF_W(39)
        TF_W(40) TF_W(41) TF_W(42) TF_W(43) TF_W(44) TF_W(45) TF_W(46) TF_W(47)
        TF_W(48)
#undef TF_W
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

// Makes v opaque to the optimizer at this point: values computed from it afterwards are
// not hoisted above it. The thread index goes through this at every phase, so that lane
// masks and addresses derived from it are not computed once and held (spilled) across the
// whole launch.
template <class T>
__device__ __forceinline__ void opaque_v(T& v) {
    asm volatile("" : "+v"(v));
}

// A value every lane holds the same, as a scalar. Values read from the LDS copy of the
// arguments land in vector registers, and the compiler then treats them as lane-varying: a
// switch on one (wait_vm) becomes a chain of exec-masked blocks whose s_waitcnt all execute,
// down to vmcnt(0), and loops bounded by one re-read it from LDS every iteration.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ RingPhase uni(const RingPhase& p) {
    RingPhase q;
    q.N = uni(p.N);
    q.K = uni(p.K);
    q.sk = uni(p.sk);
    q.lsk = uni(p.lsk);
    q.P = uni(p.P);
    q.lpi = uni(p.lpi);
    q.spi = uni(p.spi);
    q.mats = uni(p.mats);
    q.qu = uni(p.qu);
    q.su = uni(p.su);
    q.ub = uni(p.ub);
    q.nu = uni(p.nu);
    q.bu = uni(p.bu);
    return q;
}

// Rows of the QKV phase: matrix (0 q, 1 k, 2 v) and row within it.
__device__ __forceinline__ int qkv_mat(int row, int Nq, int Nk, int& r) {
    if (row < Nq) {
        r = row;
        return 0;
    }
    if (row < Nq + Nk) {
        r = row - Nq;
        return 1;
    }
    r = row - Nq - Nk;
    return 2;
}

// The launch's arguments and layer table are copied to LDS and read there where they are
// used: held in registers across the launch, the kernel's many uniform values spill.
template <int HDM>
__global__ __launch_bounds__(kRT, 1) void k_ring(const RingArgs args) {
    extern __shared__ __align__(16) unsigned char smem[];
    int tid = threadIdx.x;
    int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x;
    const int nwg = gridDim.x;
    {
        const uint32_t* src = (const uint32_t*)&args;
        uint32_t* dst = (uint32_t*)smem;
        for (int i = tid; i < (int)(sizeof(RingArgs) / 4); i += kRT) dst[i] = src[i];
    }
    const RingArgs& a = *(const RingArgs*)smem;
    const RingLds o = ring_lds(args.n_layer, args.D, args.F, args.H, args.G, args.hd, nwg, args.part_floats,
                               args.ring_units);
    RingLayer* lay = (RingLayer*)(smem + o.table);
    RingCtl* rc = (RingCtl*)(smem + o.ctl);
    // the residual stream: xr holds a layer's input (QKV, wo's residual, the lm_head's input),
    // xr2 the wo output (gate/up, down's residual), so that a phase's gather never overwrites
    // what the previous phase's epilogue may still be reading
    float* xr = (float*)(smem + o.xr);
    float* xr2 = (float*)(smem + o.xr2);
    float* xin = (float*)(smem + o.xin);
    float* qkvb = (float*)(smem + o.qkv);
    float* att_out = (float*)(smem + o.att);
    float* part = (float*)(smem + o.part);
    float* bias_l = (float*)(smem + o.bias);
    unsigned char* ring = smem + o.ring;
    const uint32_t R = (uint32_t)args.ring_units;  // (the LDS copy is complete only after the barrier below)
    const uint32_t ring_lds_addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)ring;
    lds_u32* landed = (lds_u32*)&rc->landed;
    lds_u32* arrive = (lds_u32*)&rc->arrive;
    lds_u32* done = (lds_u32*)rc->done;

    {
        const uint64_t* src = (const uint64_t*)args.layers;
        uint64_t* dst = (uint64_t*)lay;
        const int nw = (int)(args.n_layer * sizeof(RingLayer) / 8);
        for (int i = tid; i < nw; i += kRT) dst[i] = src[i];
        if (tid < (int)(sizeof(RingCtl) / 4)) ((uint32_t*)rc)[tid] = 0;
    }
    __syncthreads();
    const int L = uni(a.n_layer), D = uni(a.D), F = uni(a.F), G = uni(a.G), hd = uni(a.hd), H = uni(a.H);
    const int n_rep = H / G, Hd = H * hd, HB = (n_rep + 2) * hd;

    const uint32_t e0 = uni(a.ctl->epoch);
    const int pos0 = uni(a.ctl->pos);
    const int P_ep = 6 * L + 8;  // epochs per token
    auto E = [&](int t, int l, int p) -> uint32_t { return e0 + (uint32_t)(t * P_ep + 6 * l + p); };
    // exchange buffers, each twice (layer or token parity): the step kernel's layout with one
    // copy of the wo output
    const int XA = 0, XB = XA + 2 * D, QKV = XB + 2 * kXRep * D, ATT = QKV + 2 * G * HB, HH = ATT + 2 * Hd,
              DONE = HH + 2 * F, BEST = DONE + 2 * nwg, PART = BEST + 4 * nwg;
    const int A_all = uni(a.split_all), parts_all = split_all_parts(H, hd, nwg);
    const int PW = H * A_all * (hd + 2);
    const int n_tokens = uni(a.n_tokens), att_start = uni(a.att_start), split_from = uni(a.split_from);
    const int lm_every = uni(a.lm_every), greedy = uni(a.greedy);
    auto X = [&](int off) -> u64* { return a.ex + off; };
    // ring position of unit u as (u mod R), once per batch; then wrap(o + d) for the units
    // d < R after it (no division in the loops)
    auto wrap = [&](uint32_t x) -> uint32_t { return x >= R ? x - R : x; };
    auto ring_ptr = [&](uint32_t ro, uint32_t d) -> unsigned char* { return ring + wrap(ro + d) * kUnit; };
    // the token's attention layout: every workgroup splits (spans past split_from), or
    // one workgroup per kv head on the last G workgroups, wo on the others
    auto all_split = [&](int t) { return A_all > 0 && pos0 + t + 1 - att_start > split_from; };
    // participants of a phase: (index of this workgroup, count), index < 0 when it has no rows
    auto wo_share = [&](bool all, int& idx, int& n) {
        n = all ? nwg : nwg - G;
        idx = wg < n ? wg : -1;
    };

    if (wave == kNW) {
        // ------------------------------------------------------------ the loader
        // Loads of the same wave complete in order: `issued` and `completed` count them, and
        // lane i of `fifo` holds the end unit of the load numbered i (mod 64), so that once
        // all but the last k have completed the landed front is known without any memory
        // access. Ring space is checked once per block of loads (a batch, a norm vector)
        // against `md`, the compute waves' smallest consumed front, which is re-read only
        // when the block does not fit.
        // the loader's wave is issued ahead of the compute waves of its SIMD: its loads are
        // what they wait for, and it needs few issue cycles
        __builtin_amdgcn_s_setprio(3);
        const int cap = uni(a.cap);
        uint32_t issued = 0, completed = 0, md = 0;
        int fifo = 0;
        bool stop = false;
        auto retire = [&](int keep) {
            wait_vm(keep);
            completed = issued - (uint32_t)keep;
            if (completed != 0)
                lds_st(landed, (uint32_t)__builtin_amdgcn_readlane(fifo, (int)((completed - 1) & 63)));
        };
        auto refresh = [&]() {
            typedef uint32_t v4 __attribute__((ext_vector_type(4)));
            typedef const volatile __attribute__((address_space(3))) v4 lds_v4;
            const v4 x = ((lds_v4*)done)[0], y = ((lds_v4*)done)[1];
            const uint32_t d[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
            uint32_t m = d[0];
#pragma unroll
            for (int w = 1; w < kNW; ++w) m = before(d[w], m) ? d[w] : m;
            md = m;
        };
        // ring space for every unit below u_end
        auto reserve = [&](uint32_t u_end) {
            for (int spin = 0; !stop && before(md + R, u_end); ++spin) {
                if (issued != completed) {
                    retire((int)(issued - completed) - 1);
                } else {
                    if (spin >= 4 * kSpinLimit) {
                        set_err(a.ctl, kErrSpace);
                        stop = true;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                refresh();
            }
        };
        // a free in-flight slot, then the load (its LDS address uniform), then its end unit
        auto put16 = [&](const uint8_t* src, uint32_t lds, uint32_t u_end) {
            if (issued - completed >= (uint32_t)cap) retire(cap - 1);
            lds_dma16(gptr(src), __builtin_amdgcn_readfirstlane(lds));
            fifo = lane == (int)(issued & 63) ? (int)u_end : fifo;
            ++issued;
        };
        auto put4 = [&](const void* src, uint32_t lds, uint32_t u_end) {
            if (issued - completed >= (uint32_t)cap) retire(cap - 1);
            lds_dma4(gptr(src), __builtin_amdgcn_readfirstlane(lds));
            fifo = lane == (int)(issued & 63) ? (int)u_end : fifo;
            ++issued;
        };
        uint32_t U = 0;
        // one phase's stream: participant idx of n (idx < 0: no rows, nothing streamed)
        auto stream = [&](const RingPhase& ph_lds, int idx, int n, const float* norm, auto&& qrow, auto&& srow,
                          auto&& brow) {
            const RingPhase ph = uni(ph_lds);
            if (idx < 0) return;
            int r0, r1;
            share(ph.N, n, idx, r0, r1);
            const int n_items = (r1 - r0) * ph.sk;
            if (n_items <= 0) return;
            const uint32_t base = U;
            if (ph.nu || ph.bu) {
                reserve(base + ph.nu + ph.bu);
                if (stop) return;
                const uint32_t ro = base % R;
                for (int i = 0; i < ph.nu / 4; ++i) {
                    int off = 1024 * i + 16 * lane;
                    off = off < 4 * ph.K ? off : 4 * ph.K - 16;
                    put16((const uint8_t*)norm + off, ring_lds_addr + wrap(ro + 4 * i) * kUnit, base + 4 * (i + 1));
                }
                if (ph.bu) {
                    const int r = r0 + (lane < r1 - r0 ? lane : 0);
                    put4(brow(r), ring_lds_addr + wrap(ro + ph.nu) * kUnit, base + ph.nu + 1);
                }
            }
            const uint32_t b0 = base + ph.nu + ph.bu;
            const int nb = (n_items + 7) / 8;
            const int ipb = ph.mats * ph.spi;  // scale dwords per item slot
            for (int b = 0; b < nb; ++b) {
                const uint32_t bu = b0 + (uint32_t)b * ph.ub;
                reserve(bu + ph.ub);
                if (stop) return;
                const uint32_t ro = bu % R;
                for (int s = 0; s < 8 && 8 * b + s < n_items; ++s) {
                    const int item = 8 * b + s, row = r0 + (item >> ph.lsk), pt = item & (ph.sk - 1);
                    for (int m = 0; m < ph.mats; ++m) {
                        const uint8_t* q = qrow(m, row) + (int64_t)pt * ph.P;
                        for (int j = 0; j < ph.lpi; ++j) {
                            int off = 1024 * j + 16 * lane;
                            off = off < ph.P ? off : ph.P - 16;
                            const uint32_t d = 4 * ((s * ph.mats + m) * ph.lpi + j);
                            put16(q + off, ring_lds_addr + wrap(ro + d) * kUnit, bu + d + 4);
                        }
                    }
                }
                for (int k = 0; k < ph.su; ++k) {
                    int e = 64 * k + lane;  // scale dword of the batch
                    int s = e / ipb;
                    if (s >= 8 || 8 * b + s >= n_items) {
                        s = 0;
                        e = 0;
                    }
                    const int item = 8 * b + s, row = r0 + (item >> ph.lsk), pt = item & (ph.sk - 1);
                    const int m = (e % ipb) / ph.spi, kd = (e % ipb) % ph.spi;
                    const uint8_t* sp = srow(m, row) + (int64_t)pt * (ph.P / 16) + 4 * kd;
                    const uint32_t d = ph.qu + k;
                    put4(sp, ring_lds_addr + wrap(ro + d) * kUnit, bu + d + 1);
                }
            }
            U = b0 + (uint32_t)nb * ph.ub;
        };
        const int Nq = H * hd, Nk = G * hd;
        for (int t = 0; t < n_tokens; ++t) {
            const bool all = all_split(t);
            for (int l = 0; l < L; ++l) {
                const RingLayer& ly = lay[l];
                stream(a.ph[RP_QKV], wg, nwg, ly.attn_norm,
                       [&](int, int row) -> const uint8_t* {
                           int r;
                           const int mt = qkv_mat(row, Nq, Nk, r);
                           return ly.q[mt] + (int64_t)r * D;
                       },
                       [&](int, int row) -> const uint8_t* {
                           int r;
                           const int mt = qkv_mat(row, Nq, Nk, r);
                           return ly.s[mt] + (int64_t)r * (D / 16);
                       },
                       [&](int row) -> const float* {
                           int r;
                           const int mt = qkv_mat(row, Nq, Nk, r);
                           const float* bp = mt == 0 ? ly.bq : mt == 1 ? ly.bk : ly.bv;
                           return bp + r;
                       });
                int wi, wn;
                wo_share(all, wi, wn);
                stream(a.ph[RP_WO], wi, wn, nullptr,
                       [&](int, int row) -> const uint8_t* { return ly.q[3] + (int64_t)row * Hd; },
                       [&](int, int row) -> const uint8_t* { return ly.s[3] + (int64_t)row * (Hd / 16); },
                       [&](int) -> const float* { return nullptr; });
                stream(a.ph[RP_GU], wg, nwg, ly.ffn_norm,
                       [&](int m, int row) -> const uint8_t* { return ly.q[4 + m] + (int64_t)row * D; },
                       [&](int m, int row) -> const uint8_t* { return ly.s[4 + m] + (int64_t)row * (D / 16); },
                       [&](int) -> const float* { return nullptr; });
                stream(a.ph[RP_DOWN], wg, nwg, nullptr,
                       [&](int, int row) -> const uint8_t* { return ly.q[6] + (int64_t)row * F; },
                       [&](int, int row) -> const uint8_t* { return ly.s[6] + (int64_t)row * (F / 16); },
                       [&](int) -> const float* { return nullptr; });
            }
            if (lm_every || t == n_tokens - 1)
                stream(a.ph[RP_LM], wg, nwg, a.out_norm,
                       [&](int, int row) -> const uint8_t* { return a.out.q + (int64_t)row * D; },
                       [&](int, int row) -> const uint8_t* { return a.out.s + (int64_t)row * (D / 16); },
                       [&](int) -> const float* { return nullptr; });
        }
        retire(0);
        return;
    }

    // ---------------------------------------------------------------- compute waves
    Ctl* const ctl = a.ctl;
    // barrier of the 8 compute waves: this wave's earlier LDS accesses are done before it
    // arrives, and LDS serves a CU's requests in order, so what the others wrote before
    // arriving is visible once the count is reached
    uint32_t nbar = 0;
    auto cbar = [&]() {
        nbar += kNW;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        // (the spin sleeps between reads: a late wave is usually waiting for the loader's
        // loads, and reads spinning at full rate take LDS cycles and issue slots from them)
        for (int spin = 0; before(lds_ld(arrive), nbar); ++spin) {
            if (spin >= 16 * kSpinLimit) {
                if (lane == 0 && !get_err(ctl)) set_err(ctl, kErrTimeout);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        asm volatile("" ::: "memory");
    };
    auto wait_landed = [&](uint32_t need) {
        for (int spin = 0; before(lds_ld(landed), need); ++spin) {
            if (spin >= 4 * kSpinLimit || ((spin & 1023) == 1023 && get_err(ctl))) {
                if (lane == 0 && !get_err(ctl)) set_err(ctl, kErrLanded);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    };
    auto consumed = [&](uint32_t u) {
        asm volatile("" ::: "memory");  // after this wave's reads of the units below u
        if (lane == 0) lds_st(done + wave, u);
    };
    uint32_t U = 0;
    float xv[kLpiMax][16];
    // RMSNorm scale of the D floats of x (layers.cpp:7-12: fp64 sum of squares, then
    // 1 / sqrtf(ss / n + eps)); every wave computes it in the same order
    auto inv_norm = [&](const float* x) -> float {
        double ss = 0;
        for (int j = lane; j < D; j += kWave) {
            const double v = x[j];
            ss += v * v;
        }
        ss = wave_sum_d(ss);
        return 1.0f / sqrtf((float)(ss / D) + a.eps);
    };
    // this wave's inputs of its items: element pt * P + 1024 j + 16 lane + i of src (normed
    // with the weights at ring unit nu0 when norm)
    auto load_x = [&](const RingPhase& ph, const float* src, bool norm, uint32_t nu0, float inv) {
        const int pt = wave & (ph.sk - 1);
        const uint32_t no = nu0 % R;
#pragma unroll
        for (int j = 0; j < kLpiMax; ++j) {
            const int e = 1024 * j + 16 * lane;
            const bool ok = j < ph.lpi && e < ph.P;
            const int c = pt * ph.P + (ok ? e : 0);
            const float4* xs4 = (const float4*)(src + c);
            float4 v[4] = {xs4[0], xs4[1], xs4[2], xs4[3]};
            if (norm) {
                const float4* w4 = (const float4*)(ring_ptr(no, (uint32_t)(c >> 6)) + 4 * (c & 63));
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 w = w4[k];
                    v[k] = make_float4((v[k].x * inv) * w.x, (v[k].y * inv) * w.y, (v[k].z * inv) * w.z,
                                       (v[k].w * inv) * w.w);
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                xv[j][4 * k + 0] = ok ? v[k].x : 0.0f;
                xv[j][4 * k + 1] = ok ? v[k].y : 0.0f;
                xv[j][4 * k + 2] = ok ? v[k].z : 0.0f;
                xv[j][4 * k + 3] = ok ? v[k].w : 0.0f;
            }
        }
    };
    // The batches of a phase from unit b0: item 8 b + wave of each batch (n_items in all) is
    // this wave's; on_item(item, dot of matrix 0, dot of matrix 1) runs on every lane with the
    // wave's sums (dot_q8_0_f32's per-block d scaling, quant.cpp:266-321; Fmt<Q8_0>::dot_x's
    // order within a 16-element step).
    auto consume = [&](const RingPhase& ph, uint32_t b0, int n_items, auto&& on_item) {
        const int nb = (n_items + 7) / 8;
        for (int b = 0; b < nb; ++b) {
            const int item = 8 * b + wave;
            const uint32_t bu = b0 + (uint32_t)b * ph.ub;
            if (item < n_items) {
                wait_landed(bu + ph.qu + ph.su);
                const uint32_t ro = bu % R;
                float acc[2] = {0.0f, 0.0f};
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    if (m < ph.mats) {
#pragma unroll
                        for (int j = 0; j < kLpiMax; ++j) {
                            if (j < ph.lpi) {
                                const bool ok = 1024 * j + 16 * lane < ph.P;
                                const uint4 q = *(const uint4*)(ring_ptr(ro, 4 * ((wave * ph.mats + m) * ph.lpi + j)) +
                                                                16 * lane);
                                const int e = (wave * ph.mats + m) * ph.spi + 16 * j + (lane >> 2);
                                const uint16_t d = *(const uint16_t*)(ring_ptr(ro, ph.qu + (uint32_t)(e >> 6)) +
                                                                      4 * (e & 63) + 2 * ((lane >> 1) & 1));
                                const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                                float t = 0.0f;
#pragma unroll
                                for (int i = 0; i < 4; ++i) {
                                    t = fmaf(xv[j][4 * i + 0], sb0(qw[i]), t);
                                    t = fmaf(xv[j][4 * i + 1], sb1(qw[i]), t);
                                    t = fmaf(xv[j][4 * i + 2], sb2(qw[i]), t);
                                    t = fmaf(xv[j][4 * i + 3], sb3(qw[i]), t);
                                }
                                acc[m] += ok ? h2f(d) * t : 0.0f;
                            }
                        }
                    }
                }
                const float v0 = wave_sum(acc[0]);
                const float v1 = ph.mats > 1 ? wave_sum(acc[1]) : 0.0f;
                consumed(bu + ph.ub);
                on_item(item, v0, v1);
            } else {
                consumed(bu + ph.ub);
            }
        }
    };
    // One GEMV phase on this workgroup's share: input() gathers the phase's input into src
    // (RMSNormed when norm); the batches are consumed, and after
    // a barrier thread r < rows runs epi(row, value, up value, bias) with the item sums of
    // row r0 + r added in part order.
    auto gemv = [&](const RingPhase& ph_lds, int idx, int n, const float* src, bool norm, auto&& input, auto&& epi) {
        const RingPhase ph = uni(ph_lds);
        opaque_v(tid);
        lane = tid & 63;
        input();
        cbar();
        int r0 = 0, r1 = 0;
        if (idx >= 0) share(ph.N, n, idx, r0, r1);
        const int n_items = (r1 - r0) * ph.sk;
        const uint32_t base = U;
        if (n_items > 0) {
            const float inv = norm ? inv_norm(src) : 1.0f;
            if (ph.nu || ph.bu) wait_landed(base + ph.nu + ph.bu);
            load_x(ph, src, norm, base, inv);
            if (ph.bu && tid < r1 - r0) bias_l[tid] = *(const float*)(ring_ptr(base % R, ph.nu) + 4 * tid);
            const uint32_t b0 = base + ph.nu + ph.bu;
            consumed(b0);
            consume(ph, b0, n_items, [&](int item, float v0, float v1) {
                if (lane == 0) {
                    part[item] = v0;
                    if (ph.mats > 1) part[a.part_floats / 2 + item] = v1;
                }
            });
            U = b0 + (uint32_t)((n_items + 7) / 8) * ph.ub;
            consumed(U);
        }
        cbar();
        if (tid < r1 - r0) {
            float v = part[tid * ph.sk], u = ph.mats > 1 ? part[a.part_floats / 2 + tid * ph.sk] : 0.0f;
            for (int p = 1; p < ph.sk; ++p) {
                v += part[tid * ph.sk + p];
                if (ph.mats > 1) u += part[a.part_floats / 2 + tid * ph.sk + p];
            }
            epi(r0 + tid, v, u, ph.bu ? bias_l[tid] : 0.0f);
        }
    };

    const int Nq = H * hd, Nk = G * hd;
    const RingPhase& pq = a.ph[RP_QKV];
    int tok = 0;
    for (int t = 0; t < n_tokens; ++t) {
        const bool last = t == n_tokens - 1;
        const bool all = all_split(t);
        const int pos = pos0 + t;
        for (int l = 0; l < L; ++l) {
            opaque_v(tid);
            lane = tid & 63;
            const RingLayer& ly = lay[l];
            const int par = l & 1;
            // ---- 1: QKV (attn_norm fused, bias added)
            gemv(pq, wg, nwg, xr, true,
                 [&]() {
                     if (l == 0) {
                         if (t > 0) {
                             if (greedy) {
                                 gather<kGW, 1, kPollSleep>(X(BEST) + ((t - 1) & 1) * 2 * nwg, 2 * nwg, E(t - 1, L, 6), xin,
                                                nullptr, 0, 0, ctl);
                                 cbar();
                                 if (tid == 0) {
                                     u64 b = 0;
                                     for (int i = 0; i < nwg; ++i) {
                                         const u64 k = ((u64)__float_as_uint(xin[2 * i]) << 32) |
                                                       (u64)__float_as_uint(xin[2 * i + 1]);
                                         b = k > b ? k : b;
                                     }
                                     rc->tok = key_to_index(b);
                                 }
                                 cbar();
                                 tok = rc->tok;
                             } else {
                                 gather<1, kGW, kPollSleep>(nullptr, 0, 0, nullptr, X(DONE) + ((L - 1) & 1) * nwg, nwg,
                                                E(t - 1, L - 1, 5), ctl);
                                 tok = *gptr(a.hist + pos);
                             }
                         } else {
                             tok = greedy ? key_to_index(ctl->key) : *gptr(a.hist + pos);
                         }
                         if (tok < 0 || tok >= (int)a.embd.N) {
                             if (tid == 0) set_err(ctl, kErrToken);
                             tok = 0;
                         }
                         if (wg == 0 && tid == 0) {
                             *gptr(a.hist + pos) = tok;
                             *gptr(&ctl->last_token) = tok;
                         }
                         // dequant_row of the token's row (model.cpp:199)
                         using FE = Fmt<TF_HIP_TYPE_Q8_0>;
                         const RowPtr rp = FE::row(a.embd, tok);
                         for (int s = tid; s < D / FE::E; s += kT) {
                             float v[FE::E];
                             FE::dequant(FE::load(rp, s), v);
#pragma unroll
                             for (int i = 0; i < FE::E; ++i) xr[s * FE::E + i] = v[i];
                         }
                     } else {
                         gather<kGD, kGW, kPollSleep>(X(XA) + ((l - 1) & 1) * D, D, E(t, l - 1, 5), xr,
                                          X(DONE) + ((l - 1) & 1) * nwg, nwg, E(t, l - 1, 5), ctl);
                     }
                 },
                 [&](int row, float v, float, float b) {
                     int r;
                     const int mt = qkv_mat(row, Nq, Nk, r);
                     const int idx = mt == 0 ? (r / hd / n_rep) * HB + ((r / hd) % n_rep) * hd + r % hd
                                             : (r / hd) * HB + (n_rep + mt - 1) * hd + r % hd;
                     put(X(QKV) + par * G * HB + idx, v + b, E(t, l, 1));
                 });
            // ---- 2: attention
            opaque_v(tid);
            lane = tid & 63;
            if (all) {
                // every workgroup: one split of one kv head's positions, then one (query head,
                // slice) merge of the splits (the step kernel's all-split layout)
                const int A = A_all, parts = parts_all, ho = hd + 2;
                u64* pb = X(PART) + par * PW;
                const int start = att_start;
                if (wg < G * A) {
                    const int g = wg % G, s = wg / G;
                    const int chunk = (pos + 1 - start + A - 1) / A;
                    const int p0 = start + s * chunk, p1 = min(pos + 1, p0 + chunk);
                    attn_part<HDM>(a, ly, g, pos, p0, p1, qkvb, xin, att_out, [&]() {
                        gather<kGD, 1, kPollSleep>(X(QKV) + par * G * HB + g * HB, HB, E(t, l, 1), qkvb, nullptr, 0, 0, ctl);
                        cbar();
                    }, cbar, true);
                    u64* pw_base = pb + (size_t)(g * A + s) * n_rep * ho;
                    for (int i = tid; i < n_rep * ho; i += kT) put(pw_base + i, att_out[i], E(t, l, 6));
                }
                cbar();
                if (wg < a.H * parts) {
                    const int sz = hd / parts;
                    const int h = wg / parts, d0 = (wg % parts) * sz;
                    const int g = h / n_rep, r = h % n_rep, w = sz + 2;
                    gather_idx<3>(pb, [&](int j) {
                        const int s = j / w, k = j % w;
                        return (size_t)((g * A + s) * n_rep + r) * ho + (k < sz ? d0 + k : hd + k - sz);
                    }, A * w, E(t, l, 6), xin, ctl);
                    cbar();
                    for (int k = wave; k < sz; k += kNW) {
                        float m = -INFINITY;
                        for (int s = lane; s < A; s += kWave) m = fmaxf(m, xin[s * w + sz]);
                        m = wave_max(m);
                        float lsum = 0.0f, osum = 0.0f;
                        for (int s = lane; s < A; s += kWave) {
                            const float wt = expf(xin[s * w + sz] - m);
                            lsum = fmaf(xin[s * w + sz + 1], wt, lsum);
                            osum = fmaf(xin[s * w + k], wt, osum);
                        }
                        lsum = wave_sum(lsum);
                        osum = wave_sum(osum);
                        if (lane == 0) put(X(ATT) + par * Hd + h * hd + d0 + k, osum / lsum, E(t, l, 2));
                    }
                }
                cbar();  // xin (the merge's input) is read before wo gathers into it
            } else if (wg >= nwg - G) {
                const int g = wg - (nwg - G);
                attn_head<HDM>(a, ly, g, pos, a.att_start, qkvb, xin, att_out, [&]() {
                    gather<kGD, 1, kPollSleep>(X(QKV) + par * G * HB + g * HB, HB, E(t, l, 1), qkvb, nullptr, 0, 0, ctl);
                    cbar();
                }, cbar, true);
                const int nh = n_rep * hd;
                for (int i = tid; i < nh; i += kT) put(X(ATT) + par * Hd + g * nh + i, att_out[i], E(t, l, 2));
            }
            // ---- 3: wo + residual
            {
                int wi, wn;
                wo_share(all, wi, wn);
                if (wi >= 0)
                    gemv(a.ph[RP_WO], wi, wn, xin, false,
                         [&]() { gather<kGD, 1, kPollSleep>(X(ATT) + par * Hd, Hd, E(t, l, 2), xin, nullptr, 0, 0, ctl); },
                         [&](int row, float v, float, float) { put(X(XB) + par * D + row, xr[row] + v, E(t, l, 3)); });
            }
            // ---- 4: gate/up (ffn_norm fused), SiLU(gate) * up
            gemv(a.ph[RP_GU], wg, nwg, xr2, true,
                 [&]() { gather<kGD, 1, kPollSleep>(X(XB) + par * D, D, E(t, l, 3), xr2, nullptr, 0, 0, ctl); },
                 [&](int row, float g, float u, float) {
                     put(X(HH) + par * F + row, (g / (1.0f + expf(-g))) * u, E(t, l, 4));
                 });
            // ---- 5: down + residual
            gemv(a.ph[RP_DOWN], wg, nwg, xin, false,
                 [&]() { gather<kGF, 1, kPollSleep>(X(HH) + par * F, F, E(t, l, 4), xin, nullptr, 0, 0, ctl); },
                 [&](int row, float v, float, float) {
                     const float nv = xr2[row] + v;
                     put(X(XA) + par * D + row, nv, E(t, l, 5));
                     if (last && a.taps) *gptr(a.taps + (size_t)l * D + row) = nv;
                 });
            cbar();
            if (tid == 0) put(X(DONE) + par * nwg + wg, 0.0f, E(t, l, 5));
        }
        // ---- output_norm + lm_head + greedy argmax
        if (lm_every || last) {
            opaque_v(tid);
            lane = tid & 63;
            const RingPhase ph = uni(a.ph[RP_LM]);
            const int Lm = L - 1;
            gather<kGD, kGW, kPollSleep>(X(XA) + (Lm & 1) * D, D, E(t, Lm, 5), xr, X(DONE) + (Lm & 1) * nwg, nwg, E(t, Lm, 5),
                             ctl);
            cbar();
            int r0, r1;
            share(ph.N, nwg, wg, r0, r1);
            const uint32_t base = U;
            const float inv = inv_norm(xr);
            wait_landed(base + ph.nu);
            load_x(ph, xr, true, base, inv);
            if (last && a.taps && wg == 0)
                for (int j = tid; j < D; j += kT)
                    *gptr(a.taps + (size_t)L * D + j) =
                        (xr[j] * inv) * *(const float*)(ring_ptr(base % R, (uint32_t)(j >> 6)) + 4 * (j & 63));
            const uint32_t b0 = base + ph.nu;
            consumed(b0);
            u64 best = 0;
            const int n_items = r1 - r0;
            consume(ph, b0, n_items, [&](int item, float v, float) {
                const int row = r0 + item;
                if (lane == 0 && last && a.logits) *gptr(a.logits + row) = v;
                const u64 k = argmax_key(v, row);
                best = k > best ? k : best;
            });
            U = b0 + (uint32_t)((n_items + 7) / 8) * ph.ub;
            consumed(U);
            if (lane == 0) rc->wbest[wave] = best;
            cbar();
            if (tid == 0) {
                u64 b = rc->wbest[0];
                for (int i = 1; i < kNW; ++i) b = rc->wbest[i] > b ? rc->wbest[i] : b;
                u64* bw = X(BEST) + (t & 1) * 2 * nwg + 2 * wg;
                put(bw, __uint_as_float((uint32_t)(b >> 32)), E(t, L, 6));
                put(bw + 1, __uint_as_float((uint32_t)b), E(t, L, 6));
            }
        }
    }
    // workgroup 0 folds the last token's keys and advances the control block
    if (wg == 0) {
        const int t = n_tokens - 1;
        gather<kGW, 1, kPollSleep>(X(BEST) + (t & 1) * 2 * nwg, 2 * nwg, E(t, L, 6), xin, nullptr, 0, 0, ctl);
        cbar();
        if (tid == 0) {
            u64 b = 0;
            for (int i = 0; i < nwg; ++i) {
                const u64 k = ((u64)__float_as_uint(xin[2 * i]) << 32) | (u64)__float_as_uint(xin[2 * i + 1]);
                b = k > b ? k : b;
            }
            TF_GLOBAL Ctl* c = gptr(ctl);
            c->key = b;
            c->pos = pos0 + n_tokens;
            c->epoch = e0 + (uint32_t)(n_tokens * P_ep);
        }
    }
}

}  // namespace ring_detail
}  // namespace tfk
