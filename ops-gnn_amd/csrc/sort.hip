// Stable sort of bounded row keys: the permutation step of COO -> CSR (sort
// the edges by row) and of CSR -> CSC (sort by column) that the torch_sparse
// frontends run before an SpMM or its transposed backward (reference
// python/ops_gnn/torch_sparse_spmm.py:273-342, argsort there).
//
// Keys are int64 row ids known to lie in [0, max_key].  A general int64 sort
// radix-sorts all 64 key bits with 64-bit keys and values: eight passes of
// 32 bytes per element.  Here the keys and positions are narrowed to 32 bits
// (one fused pass), hipCUB's LSD radix sort (stable) runs over only the
// ceil(log2(max_key + 1)) low bits -- 3 passes of 8 bytes per element for a
// million rows -- and one pass widens the sorted keys and the permutation
// back to int64.  Not capturable in a HIP graph (the library sort clears its
// histograms with memset nodes).

#include <hipcub/hipcub.hpp>

#include "ogn_device.h"

namespace {

using namespace ogn;

__global__ __launch_bounds__(256) void narrow_kernel(const int64_t* __restrict__ keys, int64_t n,
                                                     uint32_t* __restrict__ k32, uint32_t* __restrict__ v32) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    k32[i] = (uint32_t)keys[i];
    v32[i] = (uint32_t)i;
  }
}

__global__ __launch_bounds__(256) void widen_kernel(const uint32_t* __restrict__ k32, const uint32_t* __restrict__ v32,
                                                    int64_t n, int64_t* __restrict__ keys_out,
                                                    int64_t* __restrict__ perm) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    if (keys_out) keys_out[i] = (int64_t)k32[i];
    perm[i] = (int64_t)v32[i];
  }
}

int key_bits(int64_t max_key) {
  int b = 1;
  while (b < 63 && (max_key >> b) > 0) ++b;
  return b;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct SortLayout {
  size_t k_in, v_in, k_out, v_out, temp, temp_bytes, total;
};

// Buffers in the workspace: narrowed keys and positions (in and out), then
// the library's temporary storage.
bool sort_layout(int64_t n, int bits, hipStream_t stream, SortLayout* l) {
  size_t temp = 0;
  if (hipcub::DeviceRadixSort::SortPairs(nullptr, temp, static_cast<const uint32_t*>(nullptr),
                                         static_cast<uint32_t*>(nullptr), static_cast<const uint32_t*>(nullptr),
                                         static_cast<uint32_t*>(nullptr), (int)n, 0, bits, stream) != hipSuccess)
    return false;
  const size_t a = align256((size_t)n * sizeof(uint32_t));
  l->k_in = 0;
  l->v_in = a;
  l->k_out = 2 * a;
  l->v_out = 3 * a;
  l->temp = 4 * a;
  l->temp_bytes = temp;
  l->total = 4 * a + align256(temp);
  return true;
}

constexpr int64_t kMaxItems = 0x7fffffff;  // 32-bit positions and item count

}  // namespace

extern "C" {

size_t ogn_sort_rows_workspace_size(int64_t n, int64_t max_key) {
  if (n <= 0 || n > kMaxItems || max_key < 0 || max_key > 0xffffffffLL) return 0;
  SortLayout l;
  if (!sort_layout(n, key_bits(max_key), nullptr, &l)) return 0;
  return l.total;
}

int ogn_sort_rows(const int64_t* keys, int64_t n, int64_t max_key, int64_t* sorted_keys, int64_t* perm,
                  void* workspace, size_t workspace_bytes, void* stream) {
  if (n < 0 || max_key < 0) return fail(OGN_EINVAL, "ogn_sort_rows: negative size");
  if (n > kMaxItems || max_key > 0xffffffffLL)
    return fail(OGN_EUNSUPPORTED, "ogn_sort_rows: more than 2^31 - 1 keys or keys above 2^32 - 1");
  if (n == 0) return OGN_OK;
  if (!keys || !perm) return fail(OGN_EINVAL, "ogn_sort_rows: null pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int bits = key_bits(max_key);
  SortLayout l;
  if (!sort_layout(n, bits, s, &l)) return fail(OGN_EHIP, "ogn_sort_rows: radix sort size query failed");
  if (!workspace || workspace_bytes < l.total) return fail(OGN_EINVAL, "ogn_sort_rows: workspace too small");
  char* ws = static_cast<char*>(workspace);
  uint32_t* k_in = reinterpret_cast<uint32_t*>(ws + l.k_in);
  uint32_t* v_in = reinterpret_cast<uint32_t*>(ws + l.v_in);
  uint32_t* k_out = reinterpret_cast<uint32_t*>(ws + l.k_out);
  uint32_t* v_out = reinterpret_cast<uint32_t*>(ws + l.v_out);
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 1 << 16));
  {
    TimedLaunch t("sort_rows_narrow", s);
    hipLaunchKernelGGL(narrow_kernel, dim3(grid), dim3(256), 0, s, keys, n, k_in, v_in);
  }
  {
    TimedLaunch t("sort_rows_radix", s);
    size_t temp = l.temp_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(ws + l.temp, temp, k_in, k_out, v_in, v_out, (int)n, 0, bits, s) !=
        hipSuccess)
      return fail(OGN_EHIP, "ogn_sort_rows: radix sort failed");
  }
  {
    TimedLaunch t("sort_rows_widen", s);
    hipLaunchKernelGGL(widen_kernel, dim3(grid), dim3(256), 0, s, k_out, v_out, n, sorted_keys, perm);
  }
  return check_launch("ogn_sort_rows");
}

}  // extern "C"
