// CSR engine instances: column-gather (SpMM) mode, int8 features with int32
// results (torch_sparse int8 SpMM).
#include "csr_engine.h"

namespace ogn {
namespace eng {

void launch_gather_i8(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  if (rk == RK_SUM) launch_gather_sum_dt<OGN_I8>(pl, i64, grid, s, p);
  else launch_gather_i8_ext(pl, rk, i64, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
