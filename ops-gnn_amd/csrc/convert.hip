// ind2ptr / ptr2ind (torch_sparse index conversions) for gfx950.
//
// ind2ptr: out[i] = #{ j : ind[j] < i }, i in [0, rows] -- a lower_bound of i
// in the sorted index.  One thread per output does a branch-free binary
// search; the top levels of every search hit the same cache lines, so the
// kernel reads far less than the whole index when rows << numel.
//
// ptr2ind: out[e] = r with ptr[r] <= e < ptr[r+1].  A block owns 2048
// consecutive edges and stages the pointer entries they can touch in LDS;
// each thread owns 8 edges: one search in LDS for the first, then a forward
// walk; the tile's results are transposed through LDS and leave as
// coalesced 4 KiB store instructions.
#include "ogn_device.h"
#include "search.h"

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

constexpr int kTileThreads = 256;
constexpr int64_t kTileEdges = (int64_t)kTileThreads * kEdgesPerThread;
constexpr int kWindow = 2176;  // pointer entries staged in LDS per tile (17 KiB: 9 blocks per CU)

// A block owns a tile of 2048 edges.  Its first wavefront finds the rows of
// the tile's first and last edges; the pointer entries between them (the
// only rows the tile can touch) go to LDS, and every thread finds the row of
// its first edge by binary search in LDS, then walks its 8 edges.  A tile
// that spans more than kWindow pointer entries (long runs of empty rows)
// searches global memory instead.
template <typename IDX>
__global__ __launch_bounds__(kTileThreads) void ptr2ind_kernel(const IDX* __restrict__ ptr, int64_t rows,
                                                              int64_t numel, int64_t* __restrict__ out) {
  __shared__ int64_t win[kWindow];
  __shared__ int64_t bounds[2];
  const int64_t t0 = (int64_t)blockIdx.x * kTileEdges;
  const int64_t t1 = std::min<int64_t>(t0 + kTileEdges, numel) - 1;
  if (threadIdx.x < kWave) {
    const int64_t ub = wave_upper_bound2(ptr, rows + 1, t0, t1);
    if (threadIdx.x == 0) bounds[0] = ub;
    if (threadIdx.x == 32) bounds[1] = ub;
  }
  __syncthreads();
  const int64_t last = std::max<int64_t>(rows - 1, 0);
  const int64_t r_lo = std::min<int64_t>(std::max<int64_t>(bounds[0] - 1, 0), last);
  const int64_t r_hi = std::min<int64_t>(std::max<int64_t>(bounds[1] - 1, 0), last);
  const int64_t nwin = r_hi - r_lo + 2;  // ptr[r_lo .. r_hi + 1]
  const bool staged = nwin <= kWindow;
  if (staged) {
    for (int64_t i = threadIdx.x; i < nwin; i += kTileThreads) win[i] = (int64_t)ptr[r_lo + i];
  }
  __syncthreads();
  const int64_t e0 = t0 + (int64_t)threadIdx.x * kEdgesPerThread;
  int64_t r = 0;
  if (e0 >= numel) {
    // no edges: nothing to find (the thread still joins the barrier below)
  } else if (staged) {
    // last window entry <= e0 (entry 0 holds ptr[r_lo] <= t0 <= e0, unless e0
    // precedes every row start: then row r_lo, as the clamp above gives)
    int64_t lo = 0, len = nwin;
    while (len > 0) {
      const int64_t h = len >> 1;
      const bool right = win[lo + h] <= e0;
      lo = right ? lo + h + 1 : lo;
      len = right ? len - h - 1 : h;
    }
    r = std::min<int64_t>(std::max<int64_t>(r_lo + lo - 1, 0), last);
  } else {
    r = std::min<int64_t>(std::max<int64_t>(upper_bound_idx(ptr, rows + 1, e0) - 1, 0), last);
  }
  const auto ptr_at = [&](int64_t i) -> int64_t {
    return staged && i - r_lo < nwin ? win[i - r_lo] : (int64_t)ptr[i];
  };
  int64_t res[kEdgesPerThread];
  if (e0 < numel) {
    int64_t next = ptr_at(r + 1);
#pragma unroll
    for (int i = 0; i < kEdgesPerThread; ++i) {
      const int64_t e = e0 + i;
      while (e >= next && r + 1 < rows) {
        ++r;
        next = ptr_at(r + 1);
      }
      res[i] = r;
    }
  }
  // Transpose through LDS (reusing the window) so that every store
  // instruction writes 256 consecutive 16-byte pieces (4 KiB) of the tile.
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kEdgesPerThread; ++i) win[threadIdx.x * kEdgesPerThread + i] = res[i];
  __syncthreads();
  const int64_t n_tile = t1 - t0 + 1;
  typedef long long v2i64 __attribute__((ext_vector_type(2)));
  const v2i64* w2 = reinterpret_cast<const v2i64*>(win);
  if (n_tile == kTileEdges) {
    v2i64* o = reinterpret_cast<v2i64*>(out + t0);
#pragma unroll
    for (int k = 0; k < kEdgesPerThread / 2; ++k) {
      const int q = k * kTileThreads + threadIdx.x;
      __builtin_nontemporal_store(w2[q], &o[q]);
    }
  } else {
    for (int64_t q = threadIdx.x; q < n_tile; q += kTileThreads) out[t0 + q] = win[q];
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
  const dim3 g((unsigned)((numel + kTileEdges - 1) / kTileEdges));
  if (index_dtype == OGN_I64)
    hipLaunchKernelGGL(ptr2ind_kernel<int64_t>, g, dim3(256), 0, s, static_cast<const int64_t*>(ptr),
                       rows, numel, out);
  else
    hipLaunchKernelGGL(ptr2ind_kernel<int32_t>, g, dim3(256), 0, s, static_cast<const int32_t*>(ptr),
                       rows, numel, out);
  return check_launch("ogn_ptr2ind");
}

}  // extern "C"
