// SpMM kernel instances for f32 features (see spmm_kernels.h).
#include "spmm_kernels.h"

namespace ogn {
namespace spmm {

void launch_f32(const Plan& pl, bool mm, dim3 grid, hipStream_t s, const SpmmParams& p, bool i64) {
  if (i64) launch_main<OGN_F32, int64_t>(pl, mm, grid, s, p);
  else launch_main<OGN_F32, int32_t>(pl, mm, grid, s, p);
}

}  // namespace spmm
}  // namespace ogn
