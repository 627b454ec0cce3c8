// Dispatch of the fused dequant-GEMV (k_gemv.hpp) by format; the kernels of each
// format are compiled in their own translation unit (k_gemv_<format>.hip).
#include "k_gemv.hpp"

namespace tfk {

#define TF_GEMV_EXTERN(T) extern template hipError_t launch_gemv_fmt<T>(const GemvArgs&, int, int, size_t, hipStream_t);
TF_GEMV_EXTERN(TF_HIP_TYPE_Q8_0)
TF_GEMV_EXTERN(TF_HIP_TYPE_Q4_0)
TF_GEMV_EXTERN(TF_HIP_TYPE_Q4_1)
TF_GEMV_EXTERN(TF_HIP_TYPE_Q6_K)
TF_GEMV_EXTERN(TF_HIP_TYPE_F16)
TF_GEMV_EXTERN(TF_HIP_TYPE_F32)

int64_t gemv_groups(int64_t n_rows, int rows_per_wave) { return (n_rows + rows_per_wave - 1) / rows_per_wave; }

size_t gemv_lds_bytes(int64_t K) { return (size_t)K * 4 + (size_t)(K / 16) * 4; }

hipError_t launch_gemv(const GemvArgs& a, int R, hipStream_t st) {
    if (a.total_groups <= 0) return hipSuccess;
    // Workgroups per CU by matrix height (swept on MI355X for the decode shapes):
    // one for N <= 4096 rows, two up to 16384, four above (the lm_head).
    int64_t rows = 0;
    for (int i = 0; i < a.n_seg; ++i) rows += a.seg[i].a.N * (a.mode == GEMV_SILU ? 2 : 1);
    const int per_cu = rows <= 4096 ? 1 : rows <= 16384 ? 2 : 4;
    const int cap = per_cu * device_cu_count();
    const int64_t want = (a.total_groups + kWavesPerBlock - 1) / kWavesPerBlock;
    const int blocks = (int)(want < cap ? want : cap);
    const size_t lds = gemv_lds_bytes(a.K);
    switch (a.type) {
        case TF_HIP_TYPE_Q8_0: return launch_gemv_fmt<TF_HIP_TYPE_Q8_0>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_Q4_0: return launch_gemv_fmt<TF_HIP_TYPE_Q4_0>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_Q4_1: return launch_gemv_fmt<TF_HIP_TYPE_Q4_1>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_Q6_K: return launch_gemv_fmt<TF_HIP_TYPE_Q6_K>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_F16: return launch_gemv_fmt<TF_HIP_TYPE_F16>(a, R, blocks, lds, st);
        case TF_HIP_TYPE_F32: return launch_gemv_fmt<TF_HIP_TYPE_F32>(a, R, blocks, lds, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace tfk
