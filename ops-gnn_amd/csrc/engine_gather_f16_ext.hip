// CSR engine instances: column-gather mode, f16 features -- extrema and
// log-sum-exp (the sums are in engine_gather_f16.hip).
#include "csr_engine.h"

namespace ogn {
namespace eng {

void launch_gather_f16_ext(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  launch_gather_ext_dt<OGN_F16>(pl, rk, i64, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
