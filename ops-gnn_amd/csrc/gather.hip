// gather_csr / gather_coo for gfx950: expand segment rows back over their
// positions (the inverse of a segment reduction, and its backward for sum).
//
//   gather_csr: out[b, i, :] = src[b, s, :] for ptr[s] <= i < ptr[s+1];
//               rows before ptr[0] are zero.
//   gather_coo: out[b, e, :] = src[b, index[b, e], :].
//
// Rows are raw bytes (any dtype, bit-exact copies, NaN payloads kept).  A
// block owns a tile of 64 output rows: one thread per row finds its source
// row (a branch-free upper_bound over the pointer row for CSR, a load for
// COO) into LDS, then the block copies the tile's packets -- 16, 8, 4, 2 or
// 1 bytes each, the widest that divides the row and both base addresses --
// with consecutive threads on consecutive packets, so reads of one source
// row and writes of the tile are coalesced.
#include "ogn_device.h"
#include "search.h"

#include <algorithm>

namespace ogn {
namespace {

constexpr int kTileRows = 64;
constexpr int kThreads = 256;

struct GatherArgs {
  const int64_t* ptr;    // csr: [ptr_batches, segments + 1]
  const int64_t* index;  // coo: [batch, entries]
  int64_t ptr_bstride;   // 0 when one pointer row is shared
  const char* src;       // [batch, src_rows, row_bytes]
  char* out;             // [batch, out_rows, row_bytes]
  int64_t src_rows, out_rows, row_bytes;
  FastDiv ppr;           // packets per row
};

template <int P>
struct Packet;
// Output packets are written once and not read back here: non-temporal
// stores (config 2 expansion, 512 MB out: 125 -> 89 us).
template <typename T>
__device__ __forceinline__ void store_out(T* p, T v) {
  if constexpr (sizeof(T) == 16) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 q = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(p));
  } else if constexpr (sizeof(T) == 8) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 q = {v.x, v.y};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x2*>(p));
  } else {
    __builtin_nontemporal_store(v, p);
  }
}
template <> struct Packet<16> { using T = uint4; };
template <> struct Packet<8> { using T = uint2; };
template <> struct Packet<4> { using T = uint32_t; };
template <> struct Packet<2> { using T = uint16_t; };
template <> struct Packet<1> { using T = uint8_t; };

// Pointer entries a CSR tile stages in LDS: its 64 rows touch at most 64
// non-empty segments; longer runs of empty segments search global memory.
constexpr int kPtrWindow = 128;

template <int P, bool CSR>
__global__ __launch_bounds__(kThreads) void gather_kernel(GatherArgs a) {
  using T = typename Packet<P>::T;
  __shared__ int64_t rows[kTileRows];
  __shared__ int64_t win[CSR ? kPtrWindow : 1];
  __shared__ int64_t bounds[2];
  const int64_t b = blockIdx.y;
  const int64_t i0 = (int64_t)blockIdx.x * kTileRows;
  const int64_t nrows = std::min<int64_t>(kTileRows, a.out_rows - i0);
  int64_t s_lo = 0, nwin = 0;
  if constexpr (CSR) {
    // the segments of the tile's first and last rows (one 32-way search per
    // wavefront instead of a binary search per row), then their pointer
    // entries into LDS
    const int64_t* ptr = a.ptr + b * a.ptr_bstride;
    if (threadIdx.x < kWave) {
      const int64_t ub = wave_upper_bound2(ptr, a.src_rows + 1, i0, i0 + nrows - 1);
      if (threadIdx.x == 0) bounds[0] = ub;
      if (threadIdx.x == 32) bounds[1] = ub;
    }
    __syncthreads();
    s_lo = std::max<int64_t>(bounds[0] - 1, 0);
    nwin = std::min<int64_t>(bounds[1], a.src_rows + 1) - s_lo;  // ptr[s_lo .. ub(last) - 1]
    if (nwin <= kPtrWindow && threadIdx.x < nwin) win[threadIdx.x] = ptr[s_lo + threadIdx.x];
    __syncthreads();
  }
  if (threadIdx.x < nrows) {
    const int64_t i = i0 + threadIdx.x;
    int64_t s;
    if constexpr (CSR) {
      // last s with ptr[s] <= i (segments = src_rows); -1 before ptr[0]
      int64_t lo, n;
      if (nwin <= kPtrWindow) {
        // every entry of ptr before s_lo is <= i, every entry past the window > i
        lo = 0;
        n = nwin;
        while (n > 0) {
          const int64_t half = n >> 1;
          const bool right = win[lo + half] <= i;
          lo = right ? lo + half + 1 : lo;
          n = right ? n - half - 1 : half;
        }
        lo += s_lo;
      } else {
        const int64_t* ptr = a.ptr + b * a.ptr_bstride;
        lo = 0;
        n = a.src_rows + 1;  // search ptr[0 .. segments]
        while (n > 0) {
          const int64_t half = n >> 1;
          const bool right = ptr[lo + half] <= i;
          lo = right ? lo + half + 1 : lo;
          n = right ? n - half - 1 : half;
        }
      }
      s = lo - 1;  // number of entries <= i, minus one
      if (s >= a.src_rows) s = -1;  // past the last segment end (not produced)
    } else {
      s = a.index[b * a.out_rows + i];
      s = std::min<int64_t>(std::max<int64_t>(s, 0), a.src_rows - 1);
    }
    rows[threadIdx.x] = s;
  }
  __syncthreads();
  const int64_t ppr = (int64_t)a.ppr.d;
  const int64_t total = nrows * ppr;
  const T* __restrict__ src = reinterpret_cast<const T*>(a.src + b * a.src_rows * a.row_bytes);
  T* __restrict__ out = reinterpret_cast<T*>(a.out + (b * a.out_rows + i0) * a.row_bytes);
  // 8 packets per thread per round, all loads issued before the stores: a
  // tile of 512-byte rows is one round, so no load waits behind a store
  // (with plain stores this alone was 2 % slower than 4 packets)
  constexpr int kU = 8;
  for (int64_t p0 = threadIdx.x; p0 < total; p0 += kThreads * kU) {
    T v[kU];
    int64_t o[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t p = p0 + u * kThreads;
      o[u] = -1;
      v[u] = T{};
      if (p < total) {
        const int64_t r = fdiv(p, a.ppr);
        const int64_t q = p - r * ppr;
        const int64_t s = rows[r];
        o[u] = r * ppr + q;
        if (s >= 0) v[u] = src[s * ppr + q];
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (o[u] >= 0) store_out(out + o[u], v[u]);
  }
}

int packet_for(const void* src, const void* out, int64_t row_bytes) {
  for (int p : {16, 8, 4, 2}) {
    if (row_bytes % p == 0 && (uintptr_t)src % p == 0 && (uintptr_t)out % p == 0) return p;
  }
  return 1;
}

template <bool CSR>
int launch(GatherArgs& a, int64_t batch, const void* src, void* out, hipStream_t s, const char* name) {
  const int p = packet_for(src, out, a.row_bytes);
  a.ppr = make_fastdiv(a.row_bytes / p);
  const dim3 grid((unsigned)((a.out_rows + kTileRows - 1) / kTileRows), (unsigned)batch);
  TimedLaunch t(name, s);
  switch (p) {
    case 16: hipLaunchKernelGGL((gather_kernel<16, CSR>), grid, dim3(kThreads), 0, s, a); break;
    case 8: hipLaunchKernelGGL((gather_kernel<8, CSR>), grid, dim3(kThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((gather_kernel<4, CSR>), grid, dim3(kThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((gather_kernel<2, CSR>), grid, dim3(kThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((gather_kernel<1, CSR>), grid, dim3(kThreads), 0, s, a); break;
  }
  return check_launch(name);
}

}  // namespace
}  // namespace ogn

using namespace ogn;

extern "C" {

int ogn_gather_csr(const int64_t* indptr, int64_t ptr_batches, const void* src, int64_t batch, int64_t segments,
                   int64_t row_bytes, int64_t out_rows, void* out, void* stream) {
  if (ptr_batches < 0 || batch < 0 || segments < 0 || row_bytes < 0 || out_rows < 0)
    return fail(OGN_EINVAL, "ogn_gather_csr: negative size");
  if (batch == 0 || out_rows == 0 || row_bytes == 0) return OGN_OK;
  if (ptr_batches != 1 && ptr_batches != batch)
    return fail(OGN_EINVAL, "ogn_gather_csr: ptr_batches must be 1 or batch");
  if (batch > 65535) return fail(OGN_EUNSUPPORTED, "ogn_gather_csr: batch > 65535");
  if (!indptr || !out || (segments > 0 && !src)) return fail(OGN_EINVAL, "ogn_gather_csr: null pointer");
  GatherArgs a{};
  a.ptr = indptr;
  a.ptr_bstride = ptr_batches == 1 ? 0 : segments + 1;
  a.src = static_cast<const char*>(src);
  a.out = static_cast<char*>(out);
  a.src_rows = segments;
  a.out_rows = out_rows;
  a.row_bytes = row_bytes;
  return launch<true>(a, batch, src, out, static_cast<hipStream_t>(stream), "gather_csr");
}

int ogn_gather_coo(const int64_t* index, const void* src, int64_t batch, int64_t src_rows, int64_t entries,
                   int64_t row_bytes, void* out, void* stream) {
  if (batch < 0 || src_rows < 0 || entries < 0 || row_bytes < 0)
    return fail(OGN_EINVAL, "ogn_gather_coo: negative size");
  if (batch == 0 || entries == 0 || row_bytes == 0) return OGN_OK;
  if (src_rows == 0) return fail(OGN_EINVAL, "ogn_gather_coo: entries need a non-empty src");
  if (batch > 65535) return fail(OGN_EUNSUPPORTED, "ogn_gather_coo: batch > 65535");
  if (!index || !src || !out) return fail(OGN_EINVAL, "ogn_gather_coo: null pointer");
  GatherArgs a{};
  a.index = index;
  a.src = static_cast<const char*>(src);
  a.out = static_cast<char*>(out);
  a.src_rows = src_rows;
  a.out_rows = entries;
  a.row_bytes = row_bytes;
  return launch<false>(a, batch, src, out, static_cast<hipStream_t>(stream), "gather_coo");
}

}  // extern "C"
