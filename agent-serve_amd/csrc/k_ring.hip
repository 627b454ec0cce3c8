// The ring decode step (k_ring.hpp): its plan for a model, LDS size and cooperative launch.
#include <algorithm>

#include "k_ring.hpp"

namespace tfk {

using namespace ring_detail;

namespace {

int max_lds_bytes() {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return 0;
    return v;
}

// Items per row for a phase whose workgroups hold at most rmax rows of K elements: the
// choice with the fewest batch steps for the busiest wave (a batch costs its 1 KiB lines
// plus about one line of fixed work: the wait, the wave reduction, the hand-back).
int pick_parts(int K, int rmax) {
    int best = 0;
    long best_cost = 0;
    for (int sk = 1; sk <= 8; sk *= 2) {
        if (K % (64 * sk) != 0 || K / sk > kLpiMax * 1024) continue;
        const int lpi = (K / sk + 1023) / 1024;
        const long cost = (long)((rmax * sk + 7) / 8) * (lpi + 1);
        if (best == 0 || cost < best_cost) {
            best = sk;
            best_cost = cost;
        }
    }
    return best;
}

void plan_phase(RingPhase& p, int N, int K, int sk, int mats, bool norm, bool bias) {
    p.N = N;
    p.K = K;
    p.sk = sk;
    p.lsk = sk == 8 ? 3 : sk == 4 ? 2 : sk == 2 ? 1 : 0;
    p.P = K / sk;
    p.lpi = (p.P + 1023) / 1024;
    p.spi = p.P / 64;
    p.mats = mats;
    p.qu = 4 * 8 * mats * p.lpi;
    p.su = (8 * mats * p.spi + 63) / 64;
    p.ub = (p.qu + p.su + 3) / 4 * 4;
    p.nu = norm ? 4 * ((4 * K + 1023) / 1024) : 0;
    p.bu = bias ? 4 : 0;
}

}  // namespace

bool ring_plan(int L, int D, int F, int H, int G, int hd, int V, int n_wg, int max_seq, int split_all, int split_from,
               bool has_bias, RingArgs* a) {
    const int n_rep = H / G, Hd = H * hd, Nqkv = H * hd + 2 * G * hd;
    if (hd > 128 || n_rep > kNW || n_rep < 1 || n_wg <= G || V < n_wg) return false;
    if (D % 64 || F % 64 || Hd % 64) return false;
    // spans past split_from split over every workgroup (the all-split layout; the ring kernel
    // has no trailing-split layout); a cache that never needs it still keeps the option, since
    // split_from can be lowered at run time
    (void)max_seq;
    (void)split_from;
    if (split_all <= 0) return false;
    auto rmax = [](int N, int n) { return (N + n - 1) / n; };
    if (has_bias && rmax(Nqkv, n_wg) > kBiasMax) return false;
    const int sk_qkv = pick_parts(D, rmax(Nqkv, n_wg));
    const int sk_wo = pick_parts(Hd, rmax(D, n_wg - G));
    const int sk_gu = pick_parts(D, rmax(F, n_wg));
    const int sk_dn = pick_parts(F, rmax(D, n_wg));
    if (!sk_qkv || !sk_wo || !sk_gu || !sk_dn || D > kLpiMax * 1024) return false;
    plan_phase(a->ph[RP_QKV], Nqkv, D, sk_qkv, 1, true, has_bias);
    plan_phase(a->ph[RP_WO], D, Hd, sk_wo, 1, false, false);
    plan_phase(a->ph[RP_GU], F, D, sk_gu, 2, true, false);
    plan_phase(a->ph[RP_DOWN], D, F, sk_dn, 1, false, false);
    plan_phase(a->ph[RP_LM], V, D, 1, 1, true, false);
    int items = rmax(Nqkv, n_wg) * sk_qkv;
    items = std::max(items, rmax(D, n_wg - G) * sk_wo);
    items = std::max(items, rmax(F, n_wg) * sk_gu);
    items = std::max(items, rmax(D, n_wg) * sk_dn);
    a->part_floats = 2 * items;
    const int max_lds = max_lds_bytes();
    const RingLds o = ring_lds(L, D, F, H, G, hd, n_wg, a->part_floats, 0);
    if (max_lds <= o.ring) return false;
    a->ring_units = (max_lds - o.ring) / kUnit / 4 * 4;
    a->cap = 16;
    // room for the largest phase head (norm + bias) and two of the largest batches
    int need = 0;
    for (int i = 0; i < RP_COUNT; ++i) need = std::max(need, a->ph[i].nu + a->ph[i].bu + 2 * a->ph[i].ub);
    return a->ring_units >= need;
}

size_t ring_lds_bytes(const RingArgs& a, int n_wg) {
    return (size_t)ring_lds(a.n_layer, a.D, a.F, a.H, a.G, a.hd, n_wg, a.part_floats, a.ring_units).total;
}

hipError_t launch_ring(const RingArgs& a, int n_wg, hipStream_t st) {
    const void* fn = a.hd <= 64 ? (const void*)k_ring<64> : (const void*)k_ring<128>;
    const size_t lds = ring_lds_bytes(a, n_wg);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kRT, lds);
    if (e != hipSuccess) return e;
    if (per_cu < 1 || n_wg > per_cu * device_cu_count()) return hipErrorCooperativeLaunchTooLarge;
    RingArgs arg = a;
    void* params[] = {(void*)&arg};
    return hipLaunchCooperativeKernel(fn, dim3(n_wg), dim3(kRT), params, (unsigned)lds, st);
}

}  // namespace tfk
