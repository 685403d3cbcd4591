// Measurement kernels: the practical memory ceilings reported beside the
// 8 TB/s HBM peak.  ogn_calibrate_gather reads the rows a workload gathers
// (same index, same table, same row width) and nothing else -- a floor for
// any kernel that gathers them; ogn_calibrate_stream is a streaming copy
// (dst given) or read (dst null) of 16-byte packets.  No counterpart in the
// reference; the results are reduced into a sink word only under a
// condition that never holds, which keeps every load live.
#include "ogn_device.h"

#include <string>

using namespace ogn;

namespace {

constexpr int kBlock = 256;
constexpr uint32_t kNever = 0x9E3779B9u;

// One wavefront per chunk of 64 * W index entries; G lanes (16 bytes each)
// per row, S = 64 / G rows per step, U steps in flight.
template <int G>
__global__ __launch_bounds__(kBlock) void gather_floor_kernel(const char* __restrict__ table, int64_t rows,
                                                              uint32_t row_bytes, const int64_t* __restrict__ idx,
                                                              int64_t n, int64_t chunk, uint32_t* sink) {
  constexpr int S = kWave / G;
  constexpr int NSTEPS = kWave / S;
  constexpr int U = NSTEPS < 8 ? NSTEPS : 8;
  const int lane = lane_id();
  const int sub = lane / G;
  const int gl = lane % G;
  const int64_t lo = ((int64_t)blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6)) * chunk;
  if (lo >= n) return;
  const int64_t hi = std::min<int64_t>(lo + chunk, n);
  uint32_t acc = 0;
  for (int64_t wb = lo; wb < hi; wb += kWave) {
    const int64_t e = wb + lane;
    const int32_t cl = e < hi ? (int32_t)std::min<int64_t>(std::max<int64_t>(idx[e], 0), rows - 1) : 0;
    const int nw = (int)std::min<int64_t>(kWave, hi - wb);
#pragma unroll
    for (int j0 = 0; j0 < NSTEPS; j0 += U) {
      uint4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int src = (j0 + u) * S + sub;
        const uint32_t c = (uint32_t)shfl32(cl, src & (kWave - 1));
        x[u] = src < nw ? load16(table + c * row_bytes + (uint32_t)gl * 16u) : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= x[u].x + x[u].y + x[u].z + x[u].w;
    }
  }
  if (acc == kNever) sink[0] = acc;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kBlock) void stream_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                        int64_t packets, uint32_t* sink) {
  constexpr int U = 8;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  uint32_t acc = 0;
  for (int64_t base = (int64_t)blockIdx.x * kBlock * U + threadIdx.x; base < packets; base += stride * U) {
    u32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * kBlock;
      x[u] = __builtin_nontemporal_load(src + std::min<int64_t>(i, packets - 1));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * kBlock;
      if (dst) {
        if (i < packets) __builtin_nontemporal_store(x[u], dst + i);
      } else {
        acc ^= x[u].x + x[u].y + x[u].z + x[u].w;
      }
    }
  }
  if (acc == kNever) sink[0] = acc;
}

}  // namespace

extern "C" {

int ogn_calibrate_gather(const void* table, int64_t rows, int64_t row_bytes, const int64_t* index, int64_t n,
                         void* sink, void* stream) {
  if (rows <= 0 || n < 0) return fail(OGN_EINVAL, "ogn_calibrate_gather: bad sizes");
  const int64_t g = row_bytes / 16;
  if (row_bytes % 16 != 0 || g < 1 || g > kWave || (g & (g - 1)) != 0)
    return fail(OGN_EUNSUPPORTED, "ogn_calibrate_gather: row_bytes must be 16 * a power of two, at most 1024");
  if ((uint64_t)rows * (uint64_t)row_bytes > (1ull << 32))
    return fail(OGN_EUNSUPPORTED, "ogn_calibrate_gather: table above 4 GiB");
  if (!table || !sink || (n > 0 && !index)) return fail(OGN_EINVAL, "ogn_calibrate_gather: null pointer");
  if (n == 0) return OGN_OK;
  if (((uintptr_t)table % 16) != 0) return fail(OGN_EINVAL, "ogn_calibrate_gather: table not 16-byte aligned");
  // 512 rows per wave as the SpMM engine's gather chunks
  const int64_t chunk = 512;
  const int64_t waves = (n + chunk - 1) / chunk;
  const dim3 grid((unsigned)((waves + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* t = static_cast<const char*>(table);
  uint32_t* k = static_cast<uint32_t*>(sink);
  const uint32_t rb = (uint32_t)row_bytes;
  switch (g) {
#define OGN_G(GV) \
  case GV: hipLaunchKernelGGL(gather_floor_kernel<GV>, grid, dim3(kBlock), 0, s, t, rows, rb, index, n, chunk, k); break;
    OGN_G(1) OGN_G(2) OGN_G(4) OGN_G(8) OGN_G(16) OGN_G(32) OGN_G(64)
#undef OGN_G
    default: break;
  }
  return check_launch("ogn_calibrate_gather");
}

int ogn_calibrate_stream(const void* src, void* dst, int64_t bytes, void* sink, void* stream) {
  if (bytes < 0 || bytes % 16 != 0) return fail(OGN_EINVAL, "ogn_calibrate_stream: bytes must be a multiple of 16");
  if (!src || !sink) return fail(OGN_EINVAL, "ogn_calibrate_stream: null pointer");
  if (((uintptr_t)src % 16) != 0 || ((uintptr_t)dst % 16) != 0)
    return fail(OGN_EINVAL, "ogn_calibrate_stream: buffers must be 16-byte aligned");
  const int64_t packets = bytes / 16;
  if (packets == 0) return OGN_OK;
  // 8 packets per thread per pass; about 8 blocks per CU
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((packets + kBlock * 8 - 1) / (kBlock * 8), 2048));
  hipLaunchKernelGGL(stream_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), packets, static_cast<uint32_t*>(sink));
  return check_launch("ogn_calibrate_stream");
}

}  // extern "C"
