// CSR engine instances: column-gather mode, i8 features -- extrema and
// log-sum-exp (the sums are in engine_gather_i8.hip).
#include "csr_engine.h"

namespace ogn {
namespace eng {

void launch_gather_i8_ext(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  launch_gather_ext_dt<OGN_I8>(pl, rk, i64, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
