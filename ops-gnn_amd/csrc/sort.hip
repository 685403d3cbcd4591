// Stable sort of bounded row keys: the permutation step of COO -> CSR (sort
// the edges by row) and of CSR -> CSC (sort by column) that the torch_sparse
// frontends run before an SpMM or its transposed backward (reference
// python/ops_gnn/torch_sparse_spmm.py:273-342, argsort there, then the
// columns and values indexed by it).
//
// Keys are int64 row ids known to lie in [0, max_key].  A general int64 sort
// radix-sorts all 64 key bits with 64-bit keys and values: eight passes of
// 32 bytes per element.  Here the keys are narrowed to 32 bits and hipCUB's
// LSD radix sort (stable) runs over only the ceil(log2(max_key + 1)) low
// bits -- 3 passes for a million rows.  The sorted value is a record of the
// element's position and up to two companion elements (the columns and the
// edge values, 4 or 8 bytes each), so the companions move with the keys in
// the sequential passes instead of being gathered afterwards through the
// permutation (a random read per element and companion).  One pass before
// the sort builds the narrowed keys and records; one after it widens the
// keys and positions to int64 and unpacks the companions.  Not capturable in
// a HIP graph (the library sort clears its histograms with memset nodes).

#include <hipcub/hipcub.hpp>

#include "ogn_device.h"

namespace {

using namespace ogn;

template <int BYTES>
struct Word;
template <> struct Word<0> { using T = uint32_t; };  // unused slot
template <> struct Word<4> { using T = uint32_t; };
template <> struct Word<8> { using T = uint64_t; };

// The sorted value: the position and the companion elements (wider first, so
// the record packs without padding when the widths are 8 and 4).
template <int AB, int BB>
struct Rec;
template <> struct Rec<0, 0> { uint32_t pos; };
template <> struct Rec<4, 0> { uint32_t pos, a; };
template <> struct Rec<8, 0> { uint64_t a; uint32_t pos; };
template <> struct Rec<4, 4> { uint32_t pos, a, b; };
template <> struct Rec<8, 4> { uint64_t a; uint32_t pos, b; };
template <> struct Rec<4, 8> { uint64_t b; uint32_t pos, a; };
template <> struct Rec<8, 8> { uint64_t a, b; uint32_t pos; };

struct Companions {
  const void* a;
  void* a_out;
  const void* b;
  void* b_out;
};

template <int AB, int BB>
__global__ __launch_bounds__(256) void pack_kernel(const int64_t* __restrict__ keys, int64_t n, uint32_t* __restrict__ k32,
                                                   Rec<AB, BB>* __restrict__ rec, Companions c) {
  using TA = typename Word<AB>::T;
  using TB = typename Word<BB>::T;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    k32[i] = (uint32_t)keys[i];
    Rec<AB, BB> r;
    r.pos = (uint32_t)i;
    if constexpr (AB != 0) r.a = static_cast<const TA*>(c.a)[i];
    if constexpr (BB != 0) r.b = static_cast<const TB*>(c.b)[i];
    rec[i] = r;
  }
}

template <int AB, int BB>
__global__ __launch_bounds__(256) void unpack_kernel(const uint32_t* __restrict__ k32, const Rec<AB, BB>* __restrict__ rec,
                                                     int64_t n, int64_t* __restrict__ keys_out,
                                                     int64_t* __restrict__ perm, Companions c) {
  using TA = typename Word<AB>::T;
  using TB = typename Word<BB>::T;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const Rec<AB, BB> r = rec[i];
    perm[i] = (int64_t)r.pos;
    if (keys_out) keys_out[i] = (int64_t)k32[i];
    if constexpr (AB != 0) static_cast<TA*>(c.a_out)[i] = r.a;
    if constexpr (BB != 0) static_cast<TB*>(c.b_out)[i] = r.b;
  }
}

int key_bits(int64_t max_key) {
  int b = 1;
  while (b < 63 && (max_key >> b) > 0) ++b;
  return b;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct SortLayout {
  size_t k_in, r_in, k_out, r_out, temp, temp_bytes, total;
};

// Workspace: narrowed keys and records (in and out), then the library's
// temporary storage.
template <int AB, int BB>
bool sort_layout(int64_t n, int bits, hipStream_t stream, SortLayout* l) {
  using R = Rec<AB, BB>;
  size_t temp = 0;
  if (hipcub::DeviceRadixSort::SortPairs(nullptr, temp, static_cast<const uint32_t*>(nullptr),
                                         static_cast<uint32_t*>(nullptr), static_cast<const R*>(nullptr),
                                         static_cast<R*>(nullptr), (int)n, 0, bits, stream) != hipSuccess)
    return false;
  const size_t kb = align256((size_t)n * sizeof(uint32_t)), rb = align256((size_t)n * sizeof(R));
  l->k_in = 0;
  l->k_out = kb;
  l->r_in = 2 * kb;
  l->r_out = 2 * kb + rb;
  l->temp = 2 * kb + 2 * rb;
  l->temp_bytes = temp;
  l->total = l->temp + align256(temp);
  return true;
}

template <int AB, int BB>
int sort_impl(const int64_t* keys, int64_t n, int bits, int64_t* sorted_keys, int64_t* perm, const Companions& c,
              void* workspace, size_t workspace_bytes, hipStream_t s) {
  using R = Rec<AB, BB>;
  SortLayout l;
  if (!sort_layout<AB, BB>(n, bits, s, &l)) return fail(OGN_EHIP, "ogn_sort_rows: radix sort size query failed");
  if (!workspace || workspace_bytes < l.total) return fail(OGN_EINVAL, "ogn_sort_rows: workspace too small");
  char* ws = static_cast<char*>(workspace);
  uint32_t* k_in = reinterpret_cast<uint32_t*>(ws + l.k_in);
  uint32_t* k_out = reinterpret_cast<uint32_t*>(ws + l.k_out);
  R* r_in = reinterpret_cast<R*>(ws + l.r_in);
  R* r_out = reinterpret_cast<R*>(ws + l.r_out);
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 1 << 16));
  {
    TimedLaunch t("sort_rows_pack", s);
    hipLaunchKernelGGL((pack_kernel<AB, BB>), dim3(grid), dim3(256), 0, s, keys, n, k_in, r_in, c);
  }
  {
    TimedLaunch t("sort_rows_radix", s);
    size_t temp = l.temp_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(ws + l.temp, temp, k_in, k_out, r_in, r_out, (int)n, 0, bits, s) !=
        hipSuccess)
      return fail(OGN_EHIP, "ogn_sort_rows: radix sort failed");
  }
  {
    TimedLaunch t("sort_rows_unpack", s);
    hipLaunchKernelGGL((unpack_kernel<AB, BB>), dim3(grid), dim3(256), 0, s, k_out, r_out, n, sorted_keys, perm, c);
  }
  return check_launch("ogn_sort_rows");
}

// The (a_bytes, b_bytes) instance; a is the first non-empty companion.
template <typename F>
bool dispatch(int ab, int bb, F&& f) {
  switch (ab * 16 + bb) {
    case 0: f(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}); return true;
    case 4 * 16: f(std::integral_constant<int, 4>{}, std::integral_constant<int, 0>{}); return true;
    case 8 * 16: f(std::integral_constant<int, 8>{}, std::integral_constant<int, 0>{}); return true;
    case 4 * 16 + 4: f(std::integral_constant<int, 4>{}, std::integral_constant<int, 4>{}); return true;
    case 8 * 16 + 4: f(std::integral_constant<int, 8>{}, std::integral_constant<int, 4>{}); return true;
    case 4 * 16 + 8: f(std::integral_constant<int, 4>{}, std::integral_constant<int, 8>{}); return true;
    case 8 * 16 + 8: f(std::integral_constant<int, 8>{}, std::integral_constant<int, 8>{}); return true;
    default: return false;
  }
}

constexpr int64_t kMaxItems = 0x7fffffff;  // 32-bit positions and item count

bool sizes_ok(int64_t n, int64_t max_key) { return n <= kMaxItems && max_key <= 0xffffffffLL; }

}  // namespace

extern "C" {

size_t ogn_sort_rows_workspace_size(int64_t n, int64_t max_key, int a_bytes, int b_bytes) {
  if (n <= 0 || max_key < 0 || !sizes_ok(n, max_key) || (a_bytes == 0 && b_bytes != 0)) return 0;
  size_t total = 0;
  const bool known = dispatch(a_bytes, b_bytes, [&](auto ac, auto bc) {
    SortLayout l;
    if (sort_layout<decltype(ac)::value, decltype(bc)::value>(n, key_bits(max_key), nullptr, &l)) total = l.total;
  });
  return known ? total : 0;
}

int ogn_sort_rows(const int64_t* keys, int64_t n, int64_t max_key, int64_t* sorted_keys, int64_t* perm,
                  const void* a, void* a_out, int a_bytes, const void* b, void* b_out, int b_bytes,
                  void* workspace, size_t workspace_bytes, void* stream) {
  if (n < 0 || max_key < 0) return fail(OGN_EINVAL, "ogn_sort_rows: negative size");
  if (!sizes_ok(n, max_key))
    return fail(OGN_EUNSUPPORTED, "ogn_sort_rows: more than 2^31 - 1 keys or keys above 2^32 - 1");
  for (int eb : {a_bytes, b_bytes})
    if (eb != 0 && eb != 4 && eb != 8) return fail(OGN_EINVAL, "ogn_sort_rows: companion elements are 4 or 8 bytes");
  if (a_bytes == 0 && b_bytes != 0) return fail(OGN_EINVAL, "ogn_sort_rows: companion b without companion a");
  if (n == 0) return OGN_OK;
  if (!keys || !perm) return fail(OGN_EINVAL, "ogn_sort_rows: null pointer");
  if ((a_bytes && (!a || !a_out)) || (b_bytes && (!b || !b_out)))
    return fail(OGN_EINVAL, "ogn_sort_rows: null companion pointer");
  const Companions c{a, a_out, b, b_out};
  int rc = OGN_OK;
  dispatch(a_bytes, b_bytes, [&](auto ac, auto bc) {
    rc = sort_impl<decltype(ac)::value, decltype(bc)::value>(keys, n, key_bits(max_key), sorted_keys, perm, c,
                                                             workspace, workspace_bytes,
                                                             static_cast<hipStream_t>(stream));
  });
  return rc;
}

}  // extern "C"
