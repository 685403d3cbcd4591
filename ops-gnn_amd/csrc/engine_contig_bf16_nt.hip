// CSR engine instances: contiguous-segment mode, bf16 features, fast variants
// with non-temporal source loads (sources above the last-level cache).
#include "csr_engine.h"

namespace ogn {
namespace eng {

void launch_contig_bf16_nt(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  launch_contig_dt<OGN_BF16, true>(pl, rk, i64, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
