// CSR engine instances: contiguous-segment mode, f32 features, fast variants
// with non-temporal source loads (sources above the last-level cache).
#include "csr_engine.h"

namespace ogn {
namespace eng {

void launch_contig_f32_nt(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  launch_contig_dt<OGN_F32, true>(pl, rk, i64, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
