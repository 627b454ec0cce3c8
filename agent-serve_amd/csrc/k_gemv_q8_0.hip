// GEMV kernels for Q8_0 weights (k_gemv.hpp).
#include "k_gemv.hpp"

namespace tfk {
template hipError_t launch_gemv_fmt<TF_HIP_TYPE_Q8_0>(const GemvArgs&, int, int, size_t, hipStream_t);
}  // namespace tfk
