// ind2ptr / ptr2ind (torch_sparse index conversions) for gfx950.
//
// ind2ptr: out[i] = #{ j : ind[j] < i }, i in [0, rows] -- a lower_bound of i
// in the sorted index.  One thread per output does a branch-free binary
// search; the top levels of every search hit the same cache lines, so the
// kernel reads far less than the whole index when rows << numel.
//
// ptr2ind: out[e] = r with ptr[r] <= e < ptr[r+1].  Each thread owns 8
// consecutive edges: one upper_bound search for the first, then a forward
// walk over rowptr; the 8 results leave as two 32-byte stores.
#include "ogn_device.h"

#include <algorithm>

namespace ogn {
namespace {

constexpr int kEdgesPerThread = 8;

template <typename IDX>
__device__ __forceinline__ int64_t lower_bound_idx(const IDX* __restrict__ a, int64_t n, int64_t key) {
  int64_t lo = 0, len = n;
  while (len > 0) {
    const int64_t half = len >> 1;
    const int64_t mid = lo + half;
    const bool go_right = (int64_t)a[mid] < key;
    lo = go_right ? mid + 1 : lo;
    len = go_right ? len - half - 1 : half;
  }
  return lo;
}

template <typename IDX>
__device__ __forceinline__ int64_t upper_bound_idx(const IDX* __restrict__ a, int64_t n, int64_t key) {
  int64_t lo = 0, len = n;
  while (len > 0) {
    const int64_t half = len >> 1;
    const int64_t mid = lo + half;
    const bool go_right = (int64_t)a[mid] <= key;
    lo = go_right ? mid + 1 : lo;
    len = go_right ? len - half - 1 : half;
  }
  return lo;
}

template <typename IDX>
__global__ __launch_bounds__(256) void ind2ptr_kernel(const IDX* __restrict__ ind, int64_t numel,
                                                      int64_t rows, int64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i > rows) return;
  out[i] = lower_bound_idx(ind, numel, i);
}

template <typename IDX>
__global__ __launch_bounds__(256) void ptr2ind_kernel(const IDX* __restrict__ ptr, int64_t rows,
                                                      int64_t numel, int64_t* __restrict__ out) {
  const int64_t e0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kEdgesPerThread;
  if (e0 >= numel) return;
  // Row of edge e0: the last r with ptr[r] <= e0 (rows with ptr[r] == ptr[r+1]
  // are skipped because the search lands on the last equal pointer).
  int64_t r = upper_bound_idx(ptr, rows + 1, e0) - 1;
  r = std::min<int64_t>(std::max<int64_t>(r, 0), std::max<int64_t>(rows - 1, 0));
  int64_t next = ptr[r + 1];
  int64_t res[kEdgesPerThread];
#pragma unroll
  for (int i = 0; i < kEdgesPerThread; ++i) {
    const int64_t e = e0 + i;
    while (e >= next && r + 1 < rows) {
      ++r;
      next = ptr[r + 1];
    }
    res[i] = r;
  }
  if (e0 + kEdgesPerThread <= numel) {
    longlong2* o = reinterpret_cast<longlong2*>(out + e0);
#pragma unroll
    for (int i = 0; i < kEdgesPerThread / 2; ++i) o[i] = make_longlong2(res[2 * i], res[2 * i + 1]);
  } else {
    for (int i = 0; i < kEdgesPerThread && e0 + i < numel; ++i) out[e0 + i] = res[i];
  }
}

}  // namespace
}  // namespace ogn

using namespace ogn;

extern "C" {

int ogn_ind2ptr(const void* ind, int index_dtype, int64_t numel, int64_t rows, int64_t* out,
                void* stream) {
  if (numel < 0 || rows < 0) return fail(OGN_EINVAL, "ogn_ind2ptr: negative size");
  if (!out || (numel > 0 && !ind)) return fail(OGN_EINVAL, "ogn_ind2ptr: null pointer");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_ind2ptr: index dtype must be int32 or int64");
  hipStream_t s = static_cast<hipStream_t>(stream);
  TimedLaunch t("ind2ptr", s);
  const dim3 g((unsigned)((rows + 1 + 255) / 256));
  if (index_dtype == OGN_I64)
    hipLaunchKernelGGL(ind2ptr_kernel<int64_t>, g, dim3(256), 0, s, static_cast<const int64_t*>(ind),
                       numel, rows, out);
  else
    hipLaunchKernelGGL(ind2ptr_kernel<int32_t>, g, dim3(256), 0, s, static_cast<const int32_t*>(ind),
                       numel, rows, out);
  return check_launch("ogn_ind2ptr");
}

int ogn_ptr2ind(const void* ptr, int index_dtype, int64_t rows, int64_t numel, int64_t* out,
                void* stream) {
  if (numel < 0 || rows < 0) return fail(OGN_EINVAL, "ogn_ptr2ind: negative size");
  if (numel == 0) return OGN_OK;
  if (rows == 0) return fail(OGN_EINVAL, "ogn_ptr2ind: numel > 0 needs at least one row");
  if (!out || !ptr) return fail(OGN_EINVAL, "ogn_ptr2ind: null pointer");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_ptr2ind: index dtype must be int32 or int64");
  if ((uintptr_t)out % 16 != 0) return fail(OGN_EINVAL, "ogn_ptr2ind: out must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  TimedLaunch t("ptr2ind", s);
  const int64_t threads = (numel + kEdgesPerThread - 1) / kEdgesPerThread;
  const dim3 g((unsigned)((threads + 255) / 256));
  if (index_dtype == OGN_I64)
    hipLaunchKernelGGL(ptr2ind_kernel<int64_t>, g, dim3(256), 0, s, static_cast<const int64_t*>(ptr),
                       rows, numel, out);
  else
    hipLaunchKernelGGL(ptr2ind_kernel<int32_t>, g, dim3(256), 0, s, static_cast<const int32_t*>(ptr),
                       rows, numel, out);
  return check_launch("ogn_ptr2ind");
}

}  // extern "C"
