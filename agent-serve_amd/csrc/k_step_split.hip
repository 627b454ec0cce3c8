// The step kernel's Q8_0 builds with ffn_down staged split over K (k_step.hpp, DSPLIT), in
// a translation unit of their own: each translation unit is a code object of its own, so
// the other builds' code keeps its place. The split is chosen for models with d_model under
// half the waves; on MI355X (2048 waves) those are the models whose d_model-long rows fit one
// 64-lane tile, and these builds take one lane step per tile (UQ = 1); other combinations
// would be correct with either build, only slower.
#include "k_step.hpp"

namespace tfk {

hipError_t launch_step_split(const StepArgs& a, int n_wg, hipStream_t st) {
    constexpr int Q8 = TF_HIP_TYPE_Q8_0;
    return a.hd <= 64 ? step_detail::launch_t<Q8, Q8, 64, Q8, true, 1>(a, n_wg, st)
                      : step_detail::launch_t<Q8, Q8, 128, Q8, true, 1>(a, n_wg, st);
}

}  // namespace tfk
