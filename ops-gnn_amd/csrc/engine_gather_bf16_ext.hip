// CSR engine instances: column-gather mode, bf16 features -- extrema and
// log-sum-exp (the sums are in engine_gather_bf16.hip).
#include "csr_engine.h"

namespace ogn {
namespace eng {

void launch_gather_bf16_ext(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  launch_gather_ext_dt<OGN_BF16>(pl, rk, i64, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
