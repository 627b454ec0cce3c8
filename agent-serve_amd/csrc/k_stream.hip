// The streaming persistent decode step (k_stream.hpp): repack of the Q8_0 weights into
// per-(workgroup, compute wave) streams, the kernel, and its host-side sizes and launch.
#include <type_traits>

#include "k_stream.hpp"


namespace tfk {

using namespace step_detail;

namespace {

// LDS layout of the stream kernel (byte offsets), the same on host and device.
struct SLds {
    int layers, steps, xr, xs, qkv, att, part0, part1, ring, total;
};
__host__ __device__ inline int al16(int x) { return (x + 15) / 16 * 16; }
__host__ __device__ inline SLds s_lds(int L, int D, int F, int H, int G, int hd, int nwg, int steps_max, int part_max,
                                      int rs) {
    SLds o;
    const int n_rep = H / G;
    o.layers = 0;
    o.steps = al16(L * (int)sizeof(SLayer));
    o.xr = al16(o.steps + kSCW * steps_max);
    o.xs = al16(o.xr + 4 * D);
    o.qkv = al16(o.xs + 4 * region_floats(D, F, n_rep, hd, nwg));
    o.att = al16(o.qkv + 4 * (n_rep + 2) * hd);
    o.part0 = al16(o.att + 4 * n_rep * (hd + 2));
    o.part1 = al16(o.part0 + 4 * part_max);
    o.ring = al16(o.part1 + 4 * part_max);
    o.total = o.ring + kSCW * rs * kSlotBytes;
    return o;
}

// Optional time stamps (built with -DTF_STREAM_PROBE only): where each wave spends its
// time, in 10 ns ticks of s_memrealtime, written to StreamArgs::dbg at the end.
#ifdef TF_STREAM_PROBE
#define SP_NOW() __builtin_amdgcn_s_memrealtime()
#define SP_ACC(var, t0) (var) += SP_NOW() - (t0)
#else
#define SP_NOW() 0ull
#define SP_ACC(var, t0) ((void)(var), (void)(t0))
#endif

// Units (row tiles) of the largest phase share of one workgroup: the size of part0/part1.
__host__ __device__ inline int s_part_max(const SPlan& pl, int nwg) {
    int m = 1;
    for (int i = 0; i < SP_COUNT; ++i) {
        const int rows = (pl.ph[i].n_rows + nwg - 1) / nwg;
        m = rows * pl.ph[i].T > m ? rows * pl.ph[i].T : m;
    }
    return m;
}

// s_waitcnt vmcnt(n) for n < 32, n even (two loads per slot).
__device__ __forceinline__ void wait_vm_even(int n) {
    switch (n) {
#define TF_W(k) \
    case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
        TF_W(0) TF_W(2) TF_W(4) TF_W(6) TF_W(8) TF_W(10) TF_W(12) TF_W(14)
        TF_W(16) TF_W(18) TF_W(20) TF_W(22) TF_W(24) TF_W(26) TF_W(28) TF_W(30)
        TF_W(32) TF_W(34) TF_W(36) TF_W(38) TF_W(40) TF_W(42) TF_W(44) TF_W(46)
        TF_W(48) TF_W(50) TF_W(52) TF_W(54) TF_W(56) TF_W(58) TF_W(60) TF_W(62)
#undef TF_W
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(3))) void lds_cvoid;

// LDS byte offset of a pointer into the kernel's LDS.
__device__ __forceinline__ uint32_t lds_off(const void* p) { return (uint32_t)(uintptr_t)(lds_cvoid*)p; }

// Direct global->LDS loads as inline asm: lane i of the wave copies 16 (or 4) bytes from
// its address to LDS offset lds + 16 i (4 i). Issued through the compiler's builtin, every
// later LDS access of the wave would first wait for all of them (vmcnt(0)); the loader
// tracks their completion itself. The LDS address goes through M0, which the compiler
// treats as reserved and warns about in a clobber list; on gfx950 it emits no M0 use of its
// own in this file (no LDS-parameter, message or relative-move instructions), so these two
// writes are the only ones and the warning is silenced here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(lds), "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" : : "s"(lds), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop

// ---------------------------------------------------------------- repack

// One block per (workgroup c, compute wave w) stream: copies the slots that wave consumes
// in one token, in order, from the DevMat layout (q bytes [N][K], fp16 d [N][K/32]) into
// the stream, and records each slot's lane steps.
struct PackArgs {
    const StepLayer* layers;
    DevMat out;
    uint8_t* stream;
    const uint64_t* sbase;
    uint8_t* ssteps;
    const uint32_t* sfirst;
    int n_layer, nwg;
    SPlan plan;
};

__global__ __launch_bounds__(64) void k_stream_pack(const PackArgs a) {
    const int cw = blockIdx.x, c = cw / kSCW, w = cw % kSCW;
    const int lane = threadIdx.x;
    uint8_t* dst = a.stream + a.sbase[cw];
    uint8_t* st = a.ssteps + a.sfirst[cw];
    uint64_t off = 0;
    uint32_t k = 0;
    auto copy_slot = [&](const DevMat& m, int row, int j, int steps) {
        const uint8_t* q = m.q + (int64_t)row * m.K + (int64_t)j * kSlotQ;
        const uint8_t* s = m.s + (int64_t)row * (m.K / 32) * 2 + (int64_t)j * 64;
        if (lane < steps) *(uint4*)(dst + off + 16 * lane) = *(const uint4*)(q + 16 * lane);
        for (int b = lane; b < (steps + 15) / 16 * 16; b += 64) dst[off + 16 * steps + b] = b < steps ? s[b] : 0;
        if (lane == 0) st[k] = (uint8_t)steps;
        off += (uint64_t)s_gbytes(steps);
        ++k;
    };
    auto phase = [&](int pi, auto&& mat_of) {
        const SPhase& p = a.plan.ph[pi];
        const SUnits su = s_units(p, c, a.nwg, w);
        for (int u = su.u0; u < su.u1; ++u) {
            const int rl = u / p.T, j = u - rl * p.T, row = su.r0 + rl;
            for (int sl = 0; sl < p.spu; ++sl) {
                int r;
                const DevMat& m = mat_of(row, sl, r);
                copy_slot(m, r, j, s_steps(p, j));
            }
        }
    };
    for (int l = 0; l < a.n_layer; ++l) {
        const StepLayer& ly = a.layers[l];
        phase(SP_QKV, [&](int row, int, int& r) -> const DevMat& {
            if (row < ly.wq.N) { r = row; return ly.wq; }
            if (row < ly.wq.N + ly.wk.N) { r = row - (int)ly.wq.N; return ly.wk; }
            r = row - (int)(ly.wq.N + ly.wk.N);
            return ly.wv;
        });
        phase(SP_WO, [&](int row, int, int& r) -> const DevMat& { r = row; return ly.wo; });
        phase(SP_GU, [&](int row, int sl, int& r) -> const DevMat& { r = row; return sl ? ly.wu : ly.wg; });
        phase(SP_DOWN, [&](int row, int, int& r) -> const DevMat& { r = row; return ly.wd; });
    }
    phase(SP_LM, [&](int row, int, int& r) -> const DevMat& { r = row; return a.out; });
}

// ---------------------------------------------------------------- the kernel

struct SConst {
    StreamArgs a;
    SPlan plan;
    SLds lds;
    int nwg, n_rep, Hd, HB, P, A_all, parts_all, PW, RS;
    uint32_t e0;
    int pos0;
    unsigned long long key0;
    int XA, XB, QKV, ATT, HH, DONE, BEST, PART;
};

// One wave's feed of its ring (wave-uniform state). iss: slots issued over the launch, clr:
// slots known to be in LDS, cons: slots consumed. The next slot to issue is slot fk of token
// ftok's stream, fg bytes into it, ring position fw.
struct Feed {
    const uint8_t* base;   // the wave's stream
    const uint8_t* steps;  // lane steps of each slot of a token's stream (LDS)
    uint32_t ring_o;       // LDS byte offset of the wave's ring
    int RS, n_tok, nl, nt, depth, lane;
    bool lm_all;
    uint32_t iss, clr, cons, fg;
    int fk, ftok, fw;

    __device__ __forceinline__ int n_cur(int t) const { return (lm_all || t == n_tok - 1) ? nt : nl; }
    __device__ __forceinline__ void skip_empty() {
        while (ftok < n_tok && n_cur(ftok) == 0) ++ftok;
    }
    __device__ __forceinline__ void issue_one() {
        const int st = __builtin_amdgcn_readfirstlane((int)steps[fk]);
        const uint8_t* src = base + fg;
        const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane((int)(ring_o + (uint32_t)(fw * kSlotBytes)));
        if (lane < st) dma16(src + 16 * lane, dst);
        if (4 * lane < st) dma4(src + 16 * st + 4 * lane, dst + kSlotQ);
        ++iss;
        fw = fw + 1 == RS ? 0 : fw + 1;
        fg += (uint32_t)s_gbytes(st);
        if (++fk >= n_cur(ftok)) {
            fk = 0;
            fg = 0;
            ++ftok;
            skip_empty();
        }
    }
    // issue while the ring has room and fewer than p slots are in flight
    __device__ __forceinline__ void topup(int p) {
        while (ftok < n_tok && (int)(iss - cons) < RS && (int)(iss - clr) < p) issue_one();
    }
    // slots cons .. n - 1 in LDS
    __device__ __forceinline__ void need(uint32_t n) {
        while (iss < n) issue_one();
        if (n > clr) {
            wait_vm_even(2 * (int)(iss - n));
            clr = n;
        }
    }
    __device__ __forceinline__ void top() { topup(depth); }
    // every load issued so far is complete
    __device__ __forceinline__ void pass() {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        clr = iss;
    }
};

// gather() of k_step.hpp with the feed kept going: top() runs before the first round of
// loads and before every re-poll (it issues the wave's next slots, ring and depth
// permitting), pass() after each round (every load the wave issued before the round is
// then complete). The re-poll loop runs while any lane of the wave has a word pending, so
// top() always runs with the whole wave.
template <int NA, int NB>
__device__ __forceinline__ void fgather(u64* pa, int na, uint32_t ea, float* da, u64* pb, int nb, uint32_t eb,
                                        Ctl* ctl, Feed& f) {
    const int tid = threadIdx.x;
    f.top();
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
    f.pass();
    for (int spin = 0; __builtin_amdgcn_ballot_w64(pend != 0) != 0; ++spin) {
        if (spin >= kSpinLimit || ((spin & 1023) == 1023 && get_err(ctl))) {
            set_err(ctl, kErrTimeout);
            break;
        }
        f.top();
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
        f.pass();
    }
}

template <int HDM>
__global__ __launch_bounds__(kSThreads, 1) void k_stream(const StreamArgs args) {
    using F8 = Fmt<TF_HIP_TYPE_Q8_0>;
    constexpr int NWR = 8;  // norm weights per thread: d_model <= 4096
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ __align__(16) unsigned char sc_raw[sizeof(SConst)];
    SConst& sc = *reinterpret_cast<SConst*>(sc_raw);
    __shared__ double red[kSCW];
    __shared__ unsigned long long wbest[kSCW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x;
    if (tid == 0) {
        SConst& c = sc;
        c.a = args;
        c.nwg = gridDim.x;
        c.plan = s_plan(args.D, args.F, args.H, args.G, args.hd, args.V);
        c.lds = s_lds(args.n_layer, args.D, args.F, args.H, args.G, args.hd, c.nwg, args.steps_max,
                      s_part_max(c.plan, c.nwg), args.ring_slots);
        c.n_rep = args.H / args.G;
        c.Hd = args.H * args.hd;
        c.HB = (c.n_rep + 2) * args.hd;
        c.P = 6 * args.n_layer + 8;
        c.A_all = args.split_all;
        c.parts_all = split_all_parts(args.H, args.hd, c.nwg);
        c.PW = args.H * c.A_all * (args.hd + 2);
        c.RS = args.ring_slots;
        c.e0 = args.ctl->epoch;
        c.pos0 = args.ctl->pos;
        c.key0 = args.ctl->key;
        c.XA = 0;
        c.XB = c.XA + 2 * args.D;
        c.QKV = c.XB + 2 * args.D;
        c.ATT = c.QKV + 2 * args.G * c.HB;
        c.HH = c.ATT + 2 * c.Hd;
        c.DONE = c.HH + 2 * args.F;
        c.BEST = c.DONE + 2 * c.nwg;
        c.PART = c.BEST + 4 * c.nwg;
    }
    __syncthreads();
    const SLds& LO = sc.lds;
    SLayer* lay = (SLayer*)(smem + LO.layers);
    uint8_t* steps_tab = smem + LO.steps;
    {
        const uint64_t* src = (const uint64_t*)args.layers;
        uint64_t* dst = (uint64_t*)lay;
        const int nw = (int)(args.n_layer * sizeof(SLayer) / 8);
        for (int i = tid; i < nw; i += kSThreads) dst[i] = src[i];
        for (int w = 0; w < kSCW; ++w) {
            const int cw = wg * kSCW + w;
            const uint8_t* s = args.ssteps + args.sfirst[cw];
            const int n = (int)args.snt[cw];
            for (int i = tid; i < n; i += kSThreads) steps_tab[w * args.steps_max + i] = s[i];
        }
    }
    __syncthreads();

    // Barrier over the workgroup's LDS accesses only: the feed's loads stay in flight.
    auto bar = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    // ------------------------------------------------------------ the feed
    const StreamArgs& A0 = sc.a;
    const int RS = __builtin_amdgcn_readfirstlane(sc.RS);
    const int depth = __builtin_amdgcn_readfirstlane(A0.depth);
    const int depth_lm = __builtin_amdgcn_readfirstlane(A0.depth_lm);
    Feed fd;
    {
        const int cwi = wg * kSCW + wave;
        const uint64_t fb_u = (uint64_t)(args.stream + args.sbase[cwi]);
        fd.base = (const uint8_t*)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(fb_u >> 32)) << 32) |
                                   (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)fb_u));
        fd.steps = steps_tab + wave * args.steps_max;
        fd.ring_o = __builtin_amdgcn_readfirstlane((int)lds_off(smem + LO.ring + (size_t)wave * RS * kSlotBytes));
        fd.RS = RS;
        fd.n_tok = __builtin_amdgcn_readfirstlane(args.n_tokens);
        fd.nl = __builtin_amdgcn_readfirstlane((int)args.snl[cwi]);
        fd.nt = __builtin_amdgcn_readfirstlane((int)args.snt[cwi]);
        fd.depth = depth;
        fd.lane = lane;
        fd.lm_all = __builtin_amdgcn_readfirstlane(args.lm_every) != 0;
        fd.iss = fd.clr = fd.cons = fd.fg = 0;
        fd.fk = fd.ftok = fd.fw = 0;
        fd.skip_empty();
    }
    const unsigned char* const ring_w = smem + LO.ring + (size_t)wave * RS * kSlotBytes;
    int cw_r = 0;  // ring position of the next slot to consume

    float* xr = (float*)(smem + LO.xr);
    float* xs = (float*)(smem + LO.xs);
    float* part0 = (float*)(smem + LO.part0);
    float* part1 = (float*)(smem + LO.part1);
    const int ct = tid;

    uint64_t pc_feed = 0, pc_gather = 0, pc_units = 0, pc_attn = 0, pc_lm = 0;
    const uint64_t pc_t0 = SP_NOW();
    (void)pc_t0;
    auto E = [&](int t, int l, int p) -> uint32_t { return sc.e0 + (uint32_t)(t * sc.P + 6 * l + p); };
    auto X = [&](int off) -> u64* { return sc.a.ex + off; };

    // xs = rmsnorm(src) (layers.cpp:7-12) or a copy, as stage() of k_step.hpp
    auto sstage = [&](const float* src, int K, bool norm, const float (&wr)[NWR], float eps) {
        bar();
        if (norm) {
            double ss = 0;
            for (int j = ct; j < K; j += kT) {
                const double v = src[j];
                ss += v * v;
            }
            ss = wave_sum_d(ss);
            if (lane == 0) red[wave] = ss;
            bar();
            ss = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
            const float inv = 1.0f / sqrtf((float)(ss / K) + eps);
#pragma unroll
            for (int i = 0; i < NWR; ++i) {
                const int j = ct + i * kT;
                if (j < K) xs[j] = (src[j] * inv) * wr[i];
            }
        }
        bar();
    };

    // The units of phase p this wave owns, read from its ring: partial dot products of
    // each unit's row tile with xs, summed over the wave's consecutive tiles of a row and
    // written at the run's last unit (0 at the others), so a row's value is the fixed-order
    // sum of its T entries. The slot's ring position is refilled once its bytes are read.
    const int nwg_r = __builtin_amdgcn_readfirstlane(sc.nwg);
    auto run_units_t = [&](auto spu_c, const SPhase& pp, int p_depth) __attribute__((always_inline)) {
        constexpr int SPU = decltype(spu_c)::value;
        const int T = __builtin_amdgcn_readfirstlane(pp.T);
        const int tail = __builtin_amdgcn_readfirstlane(pp.tail);
        const int n_rows = __builtin_amdgcn_readfirstlane(pp.n_rows);
        const int r0 = split_lo(n_rows, wg, nwg_r);
        const int U = (split_lo(n_rows, wg + 1, nwg_r) - r0) * T;
        const int u0 = split_lo(U, wave, kSCW), u1 = split_lo(U, wave + 1, kSCW);
        const uint64_t tu = SP_NOW();
        float a0 = 0.0f, a1 = 0.0f;
        int j = u0 % T;  // tile of unit u, advanced below
        for (int u = u0; u < u1; ++u) {
            const int steps = j == T - 1 ? tail : 64;
            {
                const uint64_t tf = SP_NOW();
                fd.need(fd.cons + (uint32_t)SPU);
                SP_ACC(pc_feed, tf);
            }
            const bool act = lane < steps;
            const int ls = act ? lane : 0;
            const int ridx1 = cw_r + 1 == RS ? 0 : cw_r + 1;
            const unsigned char* s0 = ring_w + cw_r * kSlotBytes;
            typename F8::Raw w0;
            w0.q = *(const uint4*)(s0 + 16 * ls);
            w0.d = *(const uint16_t*)(s0 + kSlotQ + 2 * (ls >> 1));
            typename F8::Raw w1 = w0;
            if constexpr (SPU == 2) {
                const unsigned char* s1 = ring_w + ridx1 * kSlotBytes;
                w1.q = *(const uint4*)(s1 + 16 * ls);
                w1.d = *(const uint16_t*)(s1 + kSlotQ + 2 * (ls >> 1));
            }
            const float* xj = xs + j * (kSlotQ);  // 64 steps x 16 elements per tile
            const float d0 = F8::dot(w0, xj, nullptr, ls);
            float d1 = 0.0f;
            if constexpr (SPU == 2) d1 = F8::dot(w1, xj, nullptr, ls);
            // the slots' bytes are in registers before their ring positions are refilled
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            fd.cons += (uint32_t)SPU;
            cw_r = SPU == 2 ? (ridx1 + 1 == RS ? 0 : ridx1 + 1) : ridx1;
            fd.topup(p_depth);
            a0 += act ? d0 : 0.0f;
            if constexpr (SPU == 2) a1 += act ? d1 : 0.0f;
            const bool end = j == T - 1 || u == u1 - 1;
            float r0v = 0.0f, r1v = 0.0f;
            if (end) {
                r0v = wave_sum(a0);
                if constexpr (SPU == 2) r1v = wave_sum(a1);
                a0 = a1 = 0.0f;
            }
            if (lane == 0) {
                part0[u] = r0v;
                if constexpr (SPU == 2) part1[u] = r1v;
            }
            if (++j == T) j = 0;
        }
        SP_ACC(pc_units, tu);
    };
    auto run_units = [&](const SPhase& p, int p_depth) {
        if (p.spu == 2)
            run_units_t(std::integral_constant<int, 2>{}, p, p_depth);
        else
            run_units_t(std::integral_constant<int, 1>{}, p, p_depth);
    };
    // value of row rl (workgroup-local) of phase p after run_units and a barrier
    auto row_sum = [&](const SPhase& p, const float* part, int rl) -> float {
        float v = 0.0f;
        for (int j = 0; j < p.T; ++j) v += part[rl * p.T + j];
        return v;
    };

    const int n_tokens = sc.a.n_tokens;
    int tok = 0;
    for (int t = 0; t < n_tokens; ++t) {
        const bool last = t == n_tokens - 1;
        for (int l = 0; l < sc.a.n_layer; ++l) {
            const SLayer& ly = lay[l];
            const int par = l & 1;
            const int D = sc.a.D;
            const int span = sc.pos0 + t + 1 - sc.a.att_start;
            const bool split = sc.A_all && span > sc.a.split_from;
            // ---- 1: QKV (attn_norm fused, bias added)
            {
                const SPhase& p = sc.plan.ph[SP_QKV];
                float wr[NWR];
                load_norm(ly.attn_norm, D, wr);
                const int nq = sc.Hd, nk = sc.a.G * sc.a.hd;
                const int r0 = split_lo(p.n_rows, wg, sc.nwg), rows = split_lo(p.n_rows, wg + 1, sc.nwg) - r0;
                float bias = 0.0f;
                if (ct < rows) {
                    const int row = r0 + ct;
                    const float* b = row < nq ? ly.bq : (row < nq + nk ? ly.bk : ly.bv);
                    const int rr = row < nq ? row : (row < nq + nk ? row - nq : row - nq - nk);
                    bias = b ? *gptr(b + rr) : 0.0f;
                }
                const StreamArgs& a = sc.a;
                const int pos = sc.pos0 + t;
                if (l == 0) {
                    if (t > 0) {
                        if (a.greedy) {
                            float* kb = xs;
                            bar();
                            fgather<kGW, 1>(X(sc.BEST) + ((t - 1) & 1) * 2 * sc.nwg, 2 * sc.nwg,
                                            E(t - 1, a.n_layer, 6), kb, nullptr, 0, 0, a.ctl, fd);
                            bar();
                            if (ct == 0) {
                                u64 b = 0;
                                for (int i = 0; i < sc.nwg; ++i) {
                                    const u64 k = ((u64)__float_as_uint(kb[2 * i]) << 32) |
                                                  (u64)__float_as_uint(kb[2 * i + 1]);
                                    b = k > b ? k : b;
                                }
                                wbest[0] = b;
                            }
                            bar();
                            tok = key_to_index(wbest[0]);
                        } else {
                            fgather<1, kGW>(nullptr, 0, 0, nullptr, X(sc.DONE) + ((a.n_layer - 1) & 1) * sc.nwg, sc.nwg,
                                            E(t - 1, a.n_layer - 1, 5), a.ctl, fd);
                            tok = *gptr(a.hist + pos);
                        }
                    } else {
                        tok = a.greedy ? key_to_index(sc.key0) : *gptr(a.hist + pos);
                    }
                    if (tok < 0 || tok >= (int)a.embd.N) {
                        if (ct == 0) set_err(a.ctl, kErrToken);
                        tok = 0;
                    }
                    if (wg == 0 && ct == 0) {
                        *gptr(a.hist + pos) = tok;
                        *gptr(&a.ctl->last_token) = tok;
                    }
                    bar();  // xs (the key scratch) is read before the embedding row lands in xr
                    const RowPtr rp = F8::row(a.embd, tok);
                    for (int s = ct; s < D / F8::E; s += kT) {
                        float v[F8::E];
                        F8::dequant(F8::load(rp, s), v);
#pragma unroll
                        for (int i = 0; i < F8::E; ++i) xr[s * F8::E + i] = v[i];
                    }
                } else {
                    const uint64_t tg = SP_NOW();
                    fgather<kGD, kGW>(X(sc.XA) + ((l - 1) & 1) * D, D, E(t, l - 1, 5), xr,
                                      X(sc.DONE) + ((l - 1) & 1) * sc.nwg, sc.nwg, E(t, l - 1, 5), a.ctl, fd);
                    SP_ACC(pc_gather, tg);
                }
                sstage(xr, D, true, wr, a.eps);
                run_units(p, depth);
                bar();
                if (ct < rows) {
                    const int row = r0 + ct;
                    const float v = row_sum(p, part0, ct) + bias;
                    const int hd = a.hd, n_rep = sc.n_rep, HB = sc.HB;
                    int idx;
                    if (row < nq) {
                        const int h = row / hd;
                        idx = (h / n_rep) * HB + (h % n_rep) * hd + row % hd;
                    } else {
                        const int kr = row - nq, si = kr < nk ? 0 : 1, r = kr - si * nk;
                        idx = (r / hd) * HB + (n_rep + si) * hd + r % hd;
                    }
                    put(X(sc.QKV) + par * a.G * HB + idx, v, E(t, l, 1));
                }
            }
            // ---- 2: attention
            const uint64_t ta = SP_NOW();
            {
                const StreamArgs& a = sc.a;
                const int G = a.G, HB = sc.HB, n_rep = sc.n_rep, hd = a.hd;
                float* qkv = (float*)(smem + LO.qkv);
                float* aout = (float*)(smem + LO.att);
                const int pos = sc.pos0 + t;
                if (!split) {
                    // kv head g on workgroup nwg - G + g
                    if (wg >= sc.nwg - G) {
                        const int g = wg - (sc.nwg - G);
                        bar();  // xs is free: every wave is past its QKV units
                        attn_head<HDM>(a, ly, g, pos, a.att_start, qkv, xs, aout, [&]() {
                            gather<kGD, 1>(X(sc.QKV) + par * G * HB + g * HB, HB, E(t, l, 1), qkv, nullptr, 0, 0, a.ctl);
                            bar();
                        }, bar);
                        const int nh = n_rep * hd;
                        for (int i = ct; i < nh; i += kT) put(X(sc.ATT) + par * sc.Hd + g * nh + i, aout[i], E(t, l, 2));
                    }
                } else {
                    // every workgroup takes one split of one kv head, then one (query head,
                    // slice of hd / parts) merge of the splits' partials (flash-decoding)
                    const int A = sc.A_all, parts = sc.parts_all, ho = hd + 2;
                    u64* pb = X(sc.PART) + par * sc.PW;
                    bar();
                    if (wg < G * A) {
                        const int g = wg % G, s = wg / G;
                        const int start = a.att_start;
                        const int chunk = (pos + 1 - start + A - 1) / A;
                        const int p0 = start + s * chunk, p1 = min(pos + 1, p0 + chunk);
                        attn_part<HDM>(a, ly, g, pos, p0, p1, qkv, xs, aout, [&]() {
                            gather<kGD, 1>(X(sc.QKV) + par * G * HB + g * HB, HB, E(t, l, 1), qkv, nullptr, 0, 0, a.ctl);
                            bar();
                        }, bar);
                        u64* pw_base = pb + (size_t)(g * A + s) * n_rep * ho;
                        for (int i = ct; i < n_rep * ho; i += kT) put(pw_base + i, aout[i], E(t, l, 6));
                    }
                    if (wg < a.H * parts) {
                        const int sz = hd / parts;
                        const int h = wg / parts, d0 = (wg % parts) * sz;
                        const int g = h / n_rep, r = h % n_rep, w = sz + 2;
                        float* buf = xs;
                        bar();
                        gather_idx<3>(pb, [&](int j) {
                            const int s = j / w, k = j % w;
                            return (size_t)((g * A + s) * n_rep + r) * ho + (k < sz ? d0 + k : hd + k - sz);
                        }, A * w, E(t, l, 6), buf, a.ctl);
                        bar();
                        for (int k = wave; k < sz; k += kSCW) {
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
            }
            SP_ACC(pc_attn, ta);
            // ---- 3: wo + residual
            {
                const SPhase& p = sc.plan.ph[SP_WO];
                float no_w[NWR];
                bar();  // the attention's LDS use (xs) is over
                {
                    const uint64_t tg = SP_NOW();
                    fgather<kGD, 1>(X(sc.ATT) + par * sc.Hd, sc.Hd, E(t, l, 2), xs, nullptr, 0, 0, sc.a.ctl, fd);
                    SP_ACC(pc_gather, tg);
                }
                sstage(xs, sc.Hd, false, no_w, 0.0f);
                run_units(p, depth);
                bar();
                const int r0 = split_lo(p.n_rows, wg, sc.nwg), rows = split_lo(p.n_rows, wg + 1, sc.nwg) - r0;
                if (ct < rows) {
                    const int row = r0 + ct;
                    put(X(sc.XB) + par * D + row, xr[row] + row_sum(p, part0, ct), E(t, l, 3));
                }
            }
            // ---- 4: gate/up (ffn_norm fused), SiLU(gate) * up
            {
                const SPhase& p = sc.plan.ph[SP_GU];
                float wr[NWR];
                load_norm(ly.ffn_norm, D, wr);
                bar();  // every wave has read xr's residual for its wo rows
                {
                    const uint64_t tg = SP_NOW();
                    fgather<kGD, 1>(X(sc.XB) + par * D, D, E(t, l, 3), xr, nullptr, 0, 0, sc.a.ctl, fd);
                    SP_ACC(pc_gather, tg);
                }
                sstage(xr, D, true, wr, sc.a.eps);
                run_units(p, depth);
                bar();
                const int r0 = split_lo(p.n_rows, wg, sc.nwg), rows = split_lo(p.n_rows, wg + 1, sc.nwg) - r0;
                for (int i = ct; i < rows; i += kT) {
                    const float g = row_sum(p, part0, i), u = row_sum(p, part1, i);
                    put(X(sc.HH) + par * sc.a.F + r0 + i, (g / (1.0f + expf(-g))) * u, E(t, l, 4));
                }
            }
            // ---- 5: down + residual
            {
                const SPhase& p = sc.plan.ph[SP_DOWN];
                float no_w[NWR];
                bar();
                {
                    const uint64_t tg = SP_NOW();
                    fgather<kGF, 1>(X(sc.HH) + par * sc.a.F, sc.a.F, E(t, l, 4), xs, nullptr, 0, 0, sc.a.ctl, fd);
                    SP_ACC(pc_gather, tg);
                }
                sstage(xs, sc.a.F, false, no_w, 0.0f);
                run_units(p, depth);
                bar();
                const int r0 = split_lo(p.n_rows, wg, sc.nwg), rows = split_lo(p.n_rows, wg + 1, sc.nwg) - r0;
                if (ct < rows) {
                    const int row = r0 + ct;
                    const float nv = xr[row] + row_sum(p, part0, ct);
                    put(X(sc.XA) + par * D + row, nv, E(t, l, 5));
                    if (last && sc.a.taps) *gptr(sc.a.taps + (size_t)l * D + row) = nv;
                }
                bar();
                if (ct == 0) put(X(sc.DONE) + par * sc.nwg + wg, 0.0f, E(t, l, 5));
            }
        }
        // ---- output_norm + lm_head + greedy argmax
        if (sc.a.lm_every || last) {
            const uint64_t tl = SP_NOW();
            const SPhase& p = sc.plan.ph[SP_LM];
            const int D = sc.a.D, Lm = sc.a.n_layer - 1;
            float wr[NWR];
            load_norm(sc.a.out_norm, D, wr);
            bar();
            fgather<kGD, kGW>(X(sc.XA) + (Lm & 1) * D, D, E(t, Lm, 5), xr, X(sc.DONE) + (Lm & 1) * sc.nwg, sc.nwg,
                              E(t, Lm, 5), sc.a.ctl, fd);
            sstage(xr, D, true, wr, sc.a.eps);
            if (last && sc.a.taps && wg == 0)
                for (int j = ct; j < D; j += kT) *gptr(sc.a.taps + (size_t)sc.a.n_layer * D + j) = xs[j];
            run_units(p, depth_lm);
            bar();
            const int r0 = split_lo(p.n_rows, wg, sc.nwg), rows = split_lo(p.n_rows, wg + 1, sc.nwg) - r0;
            u64 best = 0;
            for (int i = ct; i < rows; i += kT) {
                const float v = row_sum(p, part0, i);
                if (last && sc.a.logits) *gptr(sc.a.logits + r0 + i) = v;
                const u64 k = argmax_key(v, r0 + i);
                best = k > best ? k : best;
            }
            best = wave_max_u64(best);
            if (lane == 0) wbest[wave] = best;
            bar();
            if (ct == 0) {
                u64 b = wbest[0];
                for (int i = 1; i < kSCW; ++i) b = wbest[i] > b ? wbest[i] : b;
                u64* bw = X(sc.BEST) + (t & 1) * 2 * sc.nwg + 2 * wg;
                put(bw, __uint_as_float((uint32_t)(b >> 32)), E(t, sc.a.n_layer, 6));
                put(bw + 1, __uint_as_float((uint32_t)b), E(t, sc.a.n_layer, 6));
            }
            SP_ACC(pc_lm, tl);
        }
    }
    // no load of the feed outlives the workgroup
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#ifdef TF_STREAM_PROBE
    if (lane == 0 && sc.a.dbg) {
        unsigned long long* o = sc.a.dbg + (size_t)wg * 64 + wave * 8;
        o[0] = pc_feed;
        o[1] = pc_gather;
        o[2] = pc_units;
        o[3] = pc_attn;
        o[4] = pc_lm;
        o[5] = SP_NOW() - pc_t0;
        o[6] = fd.iss;
    }
#endif
    // workgroup 0 folds the last token's keys and advances the control block
    if (wg == 0) {
        const int t = n_tokens - 1;
        float* kb = xs;
        bar();
        gather<kGW, 1>(X(sc.BEST) + (t & 1) * 2 * sc.nwg, 2 * sc.nwg, E(t, sc.a.n_layer, 6), kb, nullptr, 0, 0,
                       sc.a.ctl);
        bar();
        if (ct == 0) {
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

}  // namespace

// ---------------------------------------------------------------- host side

bool stream_supported(int tl, int to, int hd, int n_rep, int D, int F, int H) {
    return tl == TF_HIP_TYPE_Q8_0 && to == TF_HIP_TYPE_Q8_0 && hd <= 128 && n_rep <= kMaxRep && D % 64 == 0 &&
           F % 64 == 0 && (H * hd) % 64 == 0 && D <= 4096 && F <= 10240;
}

int stream_plan(int n_layer, int D, int F, int H, int G, int hd, int V, int nwg, std::vector<uint64_t>& sbase,
                std::vector<uint32_t>& sfirst, std::vector<uint32_t>& snl, std::vector<uint32_t>& snt,
                uint64_t* stream_bytes, uint32_t* steps_total, int* steps_max) {
    const SPlan pl = s_plan(D, F, H, G, hd, V);
    const int n = nwg * kSCW;
    sbase.assign((size_t)n, 0);
    sfirst.assign((size_t)n, 0);
    snl.assign((size_t)n, 0);
    snt.assign((size_t)n, 0);
    uint64_t off = 0;
    uint32_t first = 0;
    int smax = 0;
    for (int c = 0; c < nwg; ++c)
        for (int w = 0; w < kSCW; ++w) {
            const int cw = c * kSCW + w;
            uint64_t bytes = 0;
            uint32_t slots = 0;
            auto add = [&](int pi) {
                const SPhase& p = pl.ph[pi];
                const SUnits su = s_units(p, c, nwg, w);
                for (int u = su.u0; u < su.u1; ++u) {
                    const int j = u % p.T;
                    bytes += (uint64_t)p.spu * s_gbytes(s_steps(p, j));
                    slots += (uint32_t)p.spu;
                }
            };
            for (int l = 0; l < n_layer; ++l)
                for (int pi = SP_QKV; pi <= SP_DOWN; ++pi) add(pi);
            snl[(size_t)cw] = slots;
            add(SP_LM);
            snt[(size_t)cw] = slots;
            sbase[(size_t)cw] = off;
            sfirst[(size_t)cw] = first;
            off += (bytes + 255) / 256 * 256;
            first += slots;
            smax = (int)slots > smax ? (int)slots : smax;
        }
    *stream_bytes = off;
    *steps_total = first;
    *steps_max = (smax + 15) / 16 * 16;
    return 0;
}

size_t stream_lds_bytes(int n_layer, int D, int F, int H, int G, int hd, int V, int nwg, int steps_max, int rs) {
    const SPlan pl = s_plan(D, F, H, G, hd, V);
    return (size_t)s_lds(n_layer, D, F, H, G, hd, nwg, steps_max, s_part_max(pl, nwg), rs).total;
}

// The largest ring (slots per compute wave) the LDS holds, or 0 when fewer than 4 fit.
int stream_ring_slots(int n_layer, int D, int F, int H, int G, int hd, int V, int nwg, int steps_max) {
    int dev = 0, max_lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return 0;
    const size_t fixed = stream_lds_bytes(n_layer, D, F, H, G, hd, V, nwg, steps_max, 0);
    const size_t budget = (size_t)max_lds - 2048;  // the kernel's static LDS (constants, reductions)
    if (fixed >= budget) return 0;
    const int rs = (int)((budget - fixed) / ((size_t)kSCW * kSlotBytes));
    return rs >= 4 ? (rs > 64 ? 64 : rs) : 0;
}

hipError_t launch_stream_pack(const StepLayer* d_layers, const DevMat& out, int n_layer, int D, int F, int H, int G,
                              int hd, int V, int nwg, uint8_t* stream, const uint64_t* sbase, uint8_t* ssteps,
                              const uint32_t* sfirst, hipStream_t st) {
    PackArgs a;
    a.layers = d_layers;
    a.out = out;
    a.stream = stream;
    a.sbase = sbase;
    a.ssteps = ssteps;
    a.sfirst = sfirst;
    a.n_layer = n_layer;
    a.nwg = nwg;
    a.plan = s_plan(D, F, H, G, hd, V);
    hipLaunchKernelGGL(k_stream_pack, dim3(nwg * kSCW), dim3(64), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_stream(const StreamArgs& a, int nwg, hipStream_t st) {
    const void* fn = a.hd <= 64 ? (const void*)k_stream<64> : (const void*)k_stream<128>;
    const size_t lds = stream_lds_bytes(a.n_layer, a.D, a.F, a.H, a.G, a.hd, a.V, nwg, a.steps_max, a.ring_slots);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kSThreads, lds);
    if (e != hipSuccess) return e;
    if (per_cu < 1 || nwg > per_cu * device_cu_count()) return hipErrorCooperativeLaunchTooLarge;
    StreamArgs arg = a;
    void* params[] = {(void*)&arg};
    return hipLaunchCooperativeKernel(fn, dim3(nwg), dim3(kSThreads), params, (unsigned)lds, st);
}

}  // namespace tfk
