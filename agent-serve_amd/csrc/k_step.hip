// Dispatch of the persistent step kernel (k_step.hpp): exchange and LDS sizes, the
// compiled (layer format, lm_head format, head size) combinations, cooperative launch.
#include "k_step.hpp"

namespace tfk {

using step_detail::attn_lds_floats;
using step_detail::kXRep;

size_t step_exchange_words(int D, int F, int H, int G, int hd, int n_wg, int split) {
    const size_t n_rep = (size_t)(H / G);
    return 2 * ((size_t)D + (size_t)kXRep * D + (size_t)G * (n_rep + 2) * hd + (size_t)H * hd + (size_t)F +
                (size_t)n_wg + 2 * (size_t)n_wg + (size_t)H * split * (hd + 2));
}

int step_split(int D, int F, int H, int G, int hd, int n_wg) {
    // A = n_rep * parts splits per kv head on G * A workgroups (at most half of them, the
    // rest stream the FFN weights meanwhile); parts (a power of two dividing hd) slices of
    // each head's outputs, one per attention workgroup, for the merge
    const int n_rep = H / G;
    int parts = 0;
    for (int p = 1; p <= hd && hd % p == 0 && H * p <= n_wg / 2; p *= 2) parts = p;
    if (parts < 1) return 0;
    const int A = n_rep * parts, sz = hd / parts;
    if (A < 2 || A * (sz + 2) > 3 * step_detail::kT || A * (sz + 2) > step_detail::region_floats(D, F, n_rep, hd, n_wg))
        return 0;
    return A;
}

int step_split_all_from(int H, int G, int hd, int split) {
    // Every workgroup splitting gives up the trailing layout's overlap of attention with the
    // FFN's weight loads; it pays once a trailing split's share of the scores and P.V,
    // span / split * n_rep * hd, passes about 25,600 (measured on MI355X: the crossover is
    // near 1,500 positions for the Llama-3.2-1B shape, 16 splits of 4 heads x 64, and near
    // 1,750 for the Qwen2.5-1.5B shape, 48 splits of 6 heads x 128; both give 1,600 here)
    const int64_t w = (int64_t)(H / G) * hd;
    return split > 0 ? (int)((25600LL * split + w - 1) / w) : 0;
}

int step_split_all(int D, int F, int H, int G, int hd, int n_wg) {
    // one split of every kv head per workgroup, as far as the merge's gather (3 words per
    // thread) and the LDS region hold A (sz + 2) words
    const int n_rep = H / G;
    const int sz = hd / step_detail::split_all_parts(H, hd, n_wg);
    int A = n_wg / G;
    while (A > 1 && (A * (sz + 2) > 3 * step_detail::kT || A * (sz + 2) > step_detail::region_floats(D, F, n_rep, hd, n_wg)))
        --A;
    return A < 2 ? 0 : A;
}

size_t step_lds_bytes(int n_layer, int D, int F, int H, int G, int hd, int n_wg, int stage_lds) {
    const int n_rep = H / G;
    const int region = step_detail::region_floats(D, F, n_rep, hd, n_wg);
    const size_t table = ((size_t)n_layer * sizeof(StepLayer) + 15) / 16 * 16;
    const size_t floats = (size_t)(D + 3) / 4 * 4 + (size_t)(region + 3) / 4 * 4 + (size_t)(n_rep + 2) * hd +
                          (size_t)n_rep * (hd + 2);
    const size_t staged = (stage_lds & 2)   ? 16 + (size_t)step_detail::kNW * step_detail::down_slot_bytes(D, F, n_wg)
                          : (stage_lds & 1) ? 16 + (size_t)step_detail::kNW * step_detail::row_slot_bytes(F)
                                            : 0;
    return table + 4 * floats + staged;
}

int step_stage_lds(int tl, int n_layer, int D, int F, int H, int G, int hd, int n_wg) {
    if ((tl != TF_HIP_TYPE_Q8_0 && tl != TF_HIP_TYPE_Q4_0) || F % 32 != 0 || D % 32 != 0 || D < 64 || F < 64)
        return 0;
    int dev = 0, max_lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return 0;
    // the kernel's static LDS (StepConst, reductions) stays under 2 KiB
    auto fits = [&](int mode) { return step_lds_bytes(n_layer, D, F, H, G, hd, n_wg, mode) + 2048 <= (size_t)max_lds; };
    // fewer down rows than half the waves: split each workgroup's rows over K (every wave
    // busy) instead of leaving most waves without a row (measured on the Qwen2.5-0.5B shape,
    // 896 rows: 0.668 against 0.688 ms per token; with 1536 and 2048 rows the row per wave is
    // faster)
    if (tl == TF_HIP_TYPE_Q8_0 && 2 * D < n_wg * step_detail::kNW && step_detail::down_split_ok(D, F, n_wg) && fits(2))
        return 2;
    if (D <= n_wg * step_detail::kNW && fits(1)) return 1;
    return 0;
}

int step_alt_type(int tl) { return tl == TF_HIP_TYPE_Q4_0 ? TF_HIP_TYPE_Q4_1 : tl; }

bool step_supported(int tl, int to, int hd, int n_rep) {
    if (hd > 128 || n_rep > step_detail::kMaxRep) return false;
    return (tl == TF_HIP_TYPE_Q8_0 && to == TF_HIP_TYPE_Q8_0) ||
           (tl == TF_HIP_TYPE_F32 && to == TF_HIP_TYPE_F32 && hd <= 64) ||
           (tl == TF_HIP_TYPE_Q4_0 && to == TF_HIP_TYPE_Q6_K && hd <= 64);
}

hipError_t launch_step(const StepArgs& a, int tl, int to, int n_wg, hipStream_t st) {
    using step_detail::launch_t;
    constexpr int Q8 = TF_HIP_TYPE_Q8_0;
    if (tl == Q8 && to == Q8) {
        if (a.stage_lds & 2) return launch_step_split(a, n_wg, st);
        return a.hd <= 64 ? launch_t<Q8, Q8, 64>(a, n_wg, st) : launch_t<Q8, Q8, 128>(a, n_wg, st);
    }
    if (tl == TF_HIP_TYPE_F32 && to == TF_HIP_TYPE_F32 && a.hd <= 64)
        return launch_t<TF_HIP_TYPE_F32, TF_HIP_TYPE_F32, 64>(a, n_wg, st);
    if (tl == TF_HIP_TYPE_Q4_0 && to == TF_HIP_TYPE_Q6_K && a.hd <= 64)
        return launch_t<TF_HIP_TYPE_Q4_0, TF_HIP_TYPE_Q6_K, 64, TF_HIP_TYPE_Q4_1>(a, n_wg, st);
    return hipErrorInvalidValue;
}

}  // namespace tfk
