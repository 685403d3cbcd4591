// CSR engine instances: contiguous-segment mode, f16 features, fast variants
// with non-temporal source loads (sources above the last-level cache).
#include "csr_engine.h"

namespace ogn {
namespace eng {

void launch_contig_f16_nt(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  launch_contig_dt<OGN_F16, true>(pl, rk, i64, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
