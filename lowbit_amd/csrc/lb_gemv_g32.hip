// Instantiations of the small-M kernels (lb_gemv.h) for int4 weights with groups of
// 32 (F_W4A16G32, F_W4A8G32), compiled apart from lb_kernels.hip so that the two
// translation units build in parallel.
#include "lb_gemv.h"

namespace lbk {

hipError_t launch_gemv_g32(int fmt, const GemmArgs &a, int num_cus, size_t lds, hipStream_t s, GemvPlan *plan) {
  if (fmt == F_W4A16G32) return launch_gemv_f<F_W4A16G32>(a, num_cus, lds, s, plan);
  if (fmt == F_W4A8G32) return launch_gemv_f<F_W4A8G32>(a, num_cus, lds, s, plan);
  return hipErrorInvalidValue;
}

}  // namespace lbk
