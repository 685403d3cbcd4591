// CSR engine instances: column-gather (SpMM) mode, bf16 features.
#include "csr_engine.h"

namespace ogn {
namespace eng {

void launch_gather_bf16(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  if (rk == RK_SUM) launch_gather_sum_dt<OGN_BF16>(pl, i64, grid, s, p);
  else launch_gather_bf16_ext(pl, rk, i64, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
