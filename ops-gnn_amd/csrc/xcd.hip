// XCD-tiled SDDMM (dot) and SpMM (sum) for gfx950.
//
// An MI355X has 8 XCDs, each with its own 4 MB L2, and the dispatcher hands
// workgroup b to XCD b % 8.  A feature table of 4-64 MB (the K or V operand
// of an attention layer) does not fit one L2, so random row gathers miss and
// are served by the MALL at ~8.4 TB/s; one eighth of it does fit, and rows
// gathered only from that eighth are L2 hits (20.3 TB/s measured for 128-byte
// rows).  So the columns are cut into 8 tiles and workgroup b only gathers
// columns of tile b % 8.
//
// Plan (per graph; columns sorted within each row): row-aligned chunks of
// about kChunk edges (a row is never split between chunks), and for every
// row r the start of each tile's columns, split[t][r] (split[0][r] = rowptr[r],
// split[8][r] = rowptr[r + 1]): tile t's edges of row r are the contiguous
// range [split[t][r], split[t + 1][r]).  Workgroup b takes tile b % 8 of
// chunks 4 (b / 8) .. 4 (b / 8) + 3, one wavefront per chunk.  Inside a
// wavefront, 64 rows at a time: lane k holds row k's segment of the tile, a
// lane scan gives each segment's "virtual" start, and virtual positions are
// mapped back to edges with a 6-step lane search; from there the schedule is
// the SDDMM / SpMM one (S = 64 / G edges per step, G lanes per feature row).
//
// SDDMM writes each edge's score in place.  SpMM writes, per tile, a partial
// row sum in fp32 for every row ([8, m, k], zeros for rows with no edge in
// the tile), and a combine pass adds the 8 tiles in order: deterministic.
#include "csr_engine.h"
#include "dot.h"

#include <string>

using namespace ogn;

namespace {

constexpr int kBlock = 256;
constexpr int kTiles = 8;
constexpr int64_t kChunk = 8192;

int64_t plan_chunks(int64_t nnz) { return std::max<int64_t>(1, (nnz + kChunk - 1) / kChunk); }
int64_t tile_width(int64_t n_cols) { return std::max<int64_t>(1, (n_cols + kTiles - 1) / kTiles); }

struct XcdPlan {
  const int64_t* chunk_row;  // [nchunks + 1]
  const int64_t* split;      // [kTiles + 1][m]
  const uint16_t* col16;     // [nnz]: column minus its tile's first column
  int64_t m, nchunks;
};

// Tile-relative 16-bit columns are kept when a tile spans at most 2^16
// columns (n_cols <= 2^19) and the rows are sorted.
constexpr int64_t kCol16MaxCols = (int64_t)kTiles << 16;

// Plan memory: a 256-byte header (word 0: the build's unsorted-row flag),
// chunk_row padded to 32 entries, then split.
constexpr int64_t kHeaderWords = 32;

XcdPlan plan_view(const void* plan, int64_t m, int64_t nnz) {
  XcdPlan p;
  p.nchunks = plan_chunks(nnz);
  p.chunk_row = static_cast<const int64_t*>(plan) + kHeaderWords;
  p.split = p.chunk_row + ((p.nchunks + 1 + 31) / 32 * 32);
  p.col16 = reinterpret_cast<const uint16_t*>(p.split + (int64_t)(kTiles + 1) * m);
  p.m = m;
  return p;
}

size_t plan_bytes(int64_t m, int64_t nnz) {
  const int64_t nc = plan_chunks(nnz);
  return sizeof(int64_t) *
             ((size_t)kHeaderWords + (size_t)((nc + 1 + 31) / 32 * 32) + (size_t)(kTiles + 1) * (size_t)m) +
         sizeof(uint16_t) * (size_t)((nnz + 127) / 128 * 128);
}

// ------------------------------------------------------------------ plan
template <typename IDX>
__global__ __launch_bounds__(kBlock) void plan_chunk_rows_kernel(const IDX* __restrict__ ptr, int64_t m,
                                                                  int64_t nchunks, int64_t* chunk_row) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c > nchunks) return;
  if (c == nchunks) {
    chunk_row[c] = m;
    return;
  }
  // first row whose start is at or after the chunk's first edge
  const int64_t key = (int64_t)ptr[0] + c * kChunk;
  int64_t lo = 0, hi = m;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)ptr[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  chunk_row[c] = c == 0 ? 0 : lo;
}

template <typename IDX>
__global__ __launch_bounds__(kBlock) void plan_split_kernel(const IDX* __restrict__ ptr, const IDX* __restrict__ col,
                                                             int64_t m, int64_t tile_w, int64_t* split) {
  const int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (r >= m) return;
  const int64_t a = ptr[r], z = ptr[r + 1];
  split[r] = a;
  split[(int64_t)kTiles * m + r] = z;
  int64_t lo = a;
  for (int t = 1; t < kTiles; ++t) {
    const int64_t key = (int64_t)t * tile_w;
    int64_t hi = z;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if ((int64_t)col[mid] < key) lo = mid + 1;
      else hi = mid;
    }
    split[(int64_t)t * m + r] = lo;
  }
}

// One wavefront per row: flags a column smaller than its predecessor.
template <typename IDX>
__global__ __launch_bounds__(kBlock) void plan_sorted_kernel(const IDX* __restrict__ ptr, const IDX* __restrict__ col,
                                                              int64_t m, int* unsorted) {
  const int64_t r = (int64_t)blockIdx.x * (kBlock / kWave) + wave_in_block();
  if (r >= m) return;
  const int64_t a = ptr[r], z = ptr[r + 1];
  bool bad = false;
  for (int64_t e = a + 1 + lane_id(); e < z; e += kWave) bad |= col[e] < col[e - 1];
  if (__ballot(bad) && lane_id() == 0) atomicOr(unsorted, 1);
}

template <typename IDX>
__global__ __launch_bounds__(kBlock) void plan_col16_kernel(const IDX* __restrict__ col, int64_t nnz, int64_t tile_w,
                                                             uint16_t* __restrict__ col16) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= nnz) return;
  const int64_t c = std::max<int64_t>((int64_t)col[e], 0);
  const int64_t t = std::min<int64_t>(c / tile_w, kTiles - 1);
  col16[e] = (uint16_t)std::min<int64_t>(c - t * tile_w, 65535);
}

__global__ void zero_int_kernel(int* p) { *p = 0; }

// ------------------------------------------------------------------ shared walk
// 64 rows rb .. rb + nr - 1 of tile t: lane k gets its row's segment
// [sa, sa + len); incl = inclusive lane scan of len; d = sa - (incl - len)
// maps a virtual position v of lane k's segment to the edge v + d.
struct RowWindow {
  int32_t incl;
  int64_t d;
  int32_t total;
};

__device__ __forceinline__ RowWindow row_window(const XcdPlan& pl, int t, int64_t rb, int nr) {
  const int lane = lane_id();
  const int64_t r = rb + lane;
  const bool valid = lane < nr;
  const int64_t sa = valid ? pl.split[(int64_t)t * pl.m + r] : 0;
  const int64_t sz = valid ? pl.split[(int64_t)(t + 1) * pl.m + r] : 0;
  const int32_t len = (int32_t)(sz - sa);
  int32_t incl = len;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int32_t o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  RowWindow w;
  w.incl = incl;
  w.d = sa - (int64_t)(incl - len);
  w.total = __builtin_amdgcn_readlane(incl, kWave - 1);
  return w;
}

// The lane (row of the window) whose segment holds virtual position v < total.
__device__ __forceinline__ int row_of(int32_t incl, int32_t v) {
  int k = 0;
#pragma unroll
  for (int step = 32; step >= 1; step >>= 1)
    if (shfl32(incl, k + step - 1) <= v) k += step;
  return k;
}

struct XcdArgs {
  XcdPlan pl;
  int64_t tile_w;   // columns per tile (tile t starts at t * tile_w)
  const void* col;
  const void* lhs;
  const void* rhs;  // the gathered table (SDDMM rhs, SpMM mat)
  const void* val;
  void* out;
  float* partial;
  int64_t lhs_rows, rhs_rows, k;
  int dt;
};

// ------------------------------------------------------------------ SDDMM dot
template <int DT, typename IDX, int G, bool C16>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4)))
void sddmm_dot_xcd_kernel(XcdArgs a) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr int NE = E::VEC;
  constexpr int S = kWave / G;
  constexpr int NSTEPS = kWave / S;
  constexpr int U = NSTEPS < 4 ? NSTEPS : 4;  // L2-hit gathers: 4 steps in flight, more waves
  const int lane = lane_id();
  const int sub = lane / G;
  const int gl = lane % G;
  const int t = (int)(blockIdx.x % kTiles);
  const int64_t c = (int64_t)(blockIdx.x / kTiles) * (kBlock / kWave) + wave_in_block();
  const XcdPlan& pl = a.pl;
  if (c >= pl.nchunks) return;
  const int64_t R0 = pl.chunk_row[c], R1 = pl.chunk_row[c + 1];
  const IDX* __restrict__ col = static_cast<const IDX*>(a.col);
  // edge e's column: from the plan's 16-bit tile-relative copy (2 bytes per
  // edge streamed instead of 4 or 8), or from col
  const int64_t tile0 = (int64_t)t * a.tile_w;
  auto column = [&](int64_t e) -> int64_t {
    if constexpr (C16) return tile0 + (int64_t)load_stream(a.pl.col16 + e);
    else return (int64_t)load_stream(col + e);
  };
  const char* __restrict__ lhs = static_cast<const char*>(a.lhs);
  const char* __restrict__ rhs = static_cast<const char*>(a.rhs);
  const uint32_t row_bytes = (uint32_t)(a.k * sizeof(S_t));
  const uint32_t k_off = (uint32_t)(gl * NE * sizeof(S_t));
  int64_t held = -1;
  uint4 keep = make_uint4(0u, 0u, 0u, 0u);
  for (int64_t rb = R0; rb < R1; rb += kWave) {
    const int nr = (int)std::min<int64_t>(kWave, R1 - rb);
    const RowWindow w = row_window(pl, t, rb, nr);
    for (int32_t vb = 0; vb < w.total; vb += kWave) {
      const int32_t v = vb + lane;
      const int nw = std::min<int32_t>(kWave, w.total - vb);
      const int kl = row_of(w.incl, std::min<int32_t>(v, w.total - 1));
      const int64_t e = v + shfl64(w.d, kl);
      const int32_t cl = v < w.total ? (int32_t)std::min<int64_t>(std::max<int64_t>(column(e), 0), a.rhs_rows - 1) : 0;
      float mine = 0.f;
      for (int j0 = 0; j0 < NSTEPS; j0 += U) {
        uint4 xr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int p = (j0 + u) * S + sub;
          const uint32_t co = (uint32_t)shfl32(cl, p) * row_bytes + k_off;
          xr[u] = p < nw ? load16(rhs + co) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int p = (j0 + u) * S + sub;
          const int64_t row = rb + shfl32(kl, p);
          if (p < nw && row != held) {  // a new row for this sub-group
            held = row;
            keep = held < a.lhs_rows ? load16(lhs + (uint64_t)held * row_bytes + k_off) : make_uint4(0u, 0u, 0u, 0u);
          }
          const float dsum = group_sum<G>(packet_dot<DT>(keep, xr[u], 0.f));
          if (gl == j0 + u) mine = dsum;
        }
      }
      // lane s * G + j holds the score of window position j * S + s
      const int pmine = gl * S + sub;
      const int64_t emine = shfl64(e, pmine);
      if (pmine < nw) store_floats<1, true>(a.out, a.dt, emine, &mine);
    }
  }
}

// ------------------------------------------------------------------ SpMM sum
template <int DT, typename IDX, int G, bool C16>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4)))
void spmm_sum_xcd_kernel(XcdArgs a) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr int NE = E::VEC;
  constexpr int S = kWave / G;
  constexpr int NSTEPS = kWave / S;
  constexpr int U = NSTEPS < 4 ? NSTEPS : 4;  // L2-hit gathers: 4 steps in flight, more waves
  const int lane = lane_id();
  const int sub = lane / G;
  const int gl = lane % G;
  const int t = (int)(blockIdx.x % kTiles);
  const int64_t c = (int64_t)(blockIdx.x / kTiles) * (kBlock / kWave) + wave_in_block();
  const XcdPlan& pl = a.pl;
  if (c >= pl.nchunks) return;
  const int64_t R0 = pl.chunk_row[c], R1 = pl.chunk_row[c + 1];
  const IDX* __restrict__ col = static_cast<const IDX*>(a.col);
  // edge e's column: from the plan's 16-bit tile-relative copy (2 bytes per
  // edge streamed instead of 4 or 8), or from col
  const int64_t tile0 = (int64_t)t * a.tile_w;
  auto column = [&](int64_t e) -> int64_t {
    if constexpr (C16) return tile0 + (int64_t)load_stream(a.pl.col16 + e);
    else return (int64_t)load_stream(col + e);
  };
  const S_t* __restrict__ val = static_cast<const S_t*>(a.val);
  const char* __restrict__ mat = static_cast<const char*>(a.rhs);
  float* __restrict__ part = a.partial + (size_t)t * (size_t)pl.m * (size_t)a.k;
  const uint32_t row_bytes = (uint32_t)(a.k * sizeof(S_t));
  const uint32_t k_off = (uint32_t)(gl * NE * sizeof(S_t));
  const int64_t k0 = (int64_t)gl * NE;
  float acc[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) acc[i] = 0.f;
  for (int64_t rb = R0; rb < R1; rb += kWave) {
    const int nr = (int)std::min<int64_t>(kWave, R1 - rb);
    const RowWindow w = row_window(pl, t, rb, nr);
    int kr = 0;  // current row of the window and its virtual end
    int32_t re = nr > 0 ? __builtin_amdgcn_readlane(w.incl, 0) : INT32_MAX;
    // finish row kr: sub-group partials summed across the wave (fixed
    // butterfly order), sub-group 0 writes the tile's fp32 partial row
    auto flush = [&]() {
      if constexpr (S >= 2) {
#pragma unroll
        for (int i = 0; i < NE; ++i) {
          if constexpr (G <= 1) acc[i] += xor_shfl<1>(acc[i]);
          if constexpr (G <= 2) acc[i] += xor_shfl<2>(acc[i]);
          if constexpr (G <= 4) acc[i] += xor_shfl<4>(acc[i]);
          if constexpr (G <= 8) acc[i] += xor_shfl<8>(acc[i]);
          if constexpr (G <= 16) acc[i] += xor_shfl<16>(acc[i]);
          if constexpr (G <= 32) acc[i] += xor_shfl<32>(acc[i]);
        }
      }
      if (sub == 0) store_floats<NE, true>(part, OGN_F32, (rb + kr) * a.k + k0, acc);
#pragma unroll
      for (int i = 0; i < NE; ++i) acc[i] = 0.f;
      ++kr;
      re = kr < nr ? __builtin_amdgcn_readlane(w.incl, kr) : INT32_MAX;
    };
    for (int32_t vb = 0; vb < w.total; vb += kWave) {
      const int32_t v = vb + lane;
      const int nw = std::min<int32_t>(kWave, w.total - vb);
      const int nsteps = (nw + S - 1) / S;
      const int kl = row_of(w.incl, std::min<int32_t>(v, w.total - 1));
      const int64_t e = v + shfl64(w.d, kl);
      const bool ok = v < w.total;
      const int32_t cl = ok ? (int32_t)std::min<int64_t>(std::max<int64_t>(column(e), 0), a.rhs_rows - 1) : 0;
      // the edge weight, streamed past L2 (which holds the tile's rows)
      float wl = 0.f;
      if (ok) {
        if constexpr (DT == OGN_F32) wl = __uint_as_float(load_stream(reinterpret_cast<const uint32_t*>(val) + e));
        else wl = E::load1(val, e);
      }
      for (int j0 = 0; j0 < nsteps; j0 += U) {
        uint4 xr[U];
        float wv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int p = (j0 + u) * S + sub;
          const uint32_t co = (uint32_t)shfl32(cl, p & (kWave - 1)) * row_bytes + k_off;
          wv[u] = shflf(wl, p & (kWave - 1));
          xr[u] = p < nw ? load16(mat + co) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (j0 + u >= nsteps) break;
          const int32_t vfirst = vb + (j0 + u) * S;
          const int32_t last = std::min<int32_t>(vfirst + S, w.total) - 1;
          const int32_t vm = vfirst + sub;
          float x[NE];
          E::unpack(xr[u], x);
          bool added = false;
          while (true) {
            if (!added && vm < w.total && vm < re) {
#pragma unroll
              for (int i = 0; i < NE; ++i) acc[i] = __builtin_fmaf(x[i], wv[u], acc[i]);
              added = true;
            }
            if (last < re) break;
            flush();
          }
        }
      }
    }
    while (kr < nr) flush();  // rows ending at the last position and empty ones after
  }
}

// out[r, :] = sum over tiles of partial[t, r, :], in tile order.
template <int ODT>
__global__ __launch_bounds__(kBlock) void combine_kernel(const float* __restrict__ partial, int64_t mk,
                                                         void* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * 4;
  if (i >= mk) return;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 q = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(partial + (size_t)t * mk + i));
    s[0] += q[0];
    s[1] += q[1];
    s[2] += q[2];
    s[3] += q[3];
  }
  store_floats<4, true>(out, ODT, i, s);
}

template <int DT, typename IDX, bool C16>
void launch_dot_c(int g, dim3 grid, hipStream_t s, const XcdArgs& a) {
  switch (g) {
    case 4: hipLaunchKernelGGL((sddmm_dot_xcd_kernel<DT, IDX, 4, C16>), grid, dim3(kBlock), 0, s, a); break;
    case 8: hipLaunchKernelGGL((sddmm_dot_xcd_kernel<DT, IDX, 8, C16>), grid, dim3(kBlock), 0, s, a); break;
    case 16: hipLaunchKernelGGL((sddmm_dot_xcd_kernel<DT, IDX, 16, C16>), grid, dim3(kBlock), 0, s, a); break;
    default: hipLaunchKernelGGL((sddmm_dot_xcd_kernel<DT, IDX, 32, C16>), grid, dim3(kBlock), 0, s, a); break;
  }
}

template <int DT, typename IDX>
void launch_dot(int g, bool c16, dim3 grid, hipStream_t s, const XcdArgs& a) {
  c16 ? launch_dot_c<DT, IDX, true>(g, grid, s, a) : launch_dot_c<DT, IDX, false>(g, grid, s, a);
}

template <int DT, typename IDX, bool C16>
void launch_sum_c(int g, dim3 grid, hipStream_t s, const XcdArgs& a) {
  switch (g) {
    case 4: hipLaunchKernelGGL((spmm_sum_xcd_kernel<DT, IDX, 4, C16>), grid, dim3(kBlock), 0, s, a); break;
    case 8: hipLaunchKernelGGL((spmm_sum_xcd_kernel<DT, IDX, 8, C16>), grid, dim3(kBlock), 0, s, a); break;
    case 16: hipLaunchKernelGGL((spmm_sum_xcd_kernel<DT, IDX, 16, C16>), grid, dim3(kBlock), 0, s, a); break;
    default: hipLaunchKernelGGL((spmm_sum_xcd_kernel<DT, IDX, 32, C16>), grid, dim3(kBlock), 0, s, a); break;
  }
}

template <int DT, typename IDX>
void launch_sum(int g, bool c16, dim3 grid, hipStream_t s, const XcdArgs& a) {
  c16 ? launch_sum_c<DT, IDX, true>(g, grid, s, a) : launch_sum_c<DT, IDX, false>(g, grid, s, a);
}

// Feature rows of 64, 128, 256 or 512 bytes (G = 4 .. 32 lanes of 16 bytes).
int row_lanes(int64_t k, int dtype) {
  const int64_t bytes = k * dtype_size(dtype);
  if (bytes != 64 && bytes != 128 && bytes != 256 && bytes != 512) return 0;
  return (int)(bytes / 16);
}

dim3 xcd_grid(const XcdPlan& pl) {
  return dim3((unsigned)(((pl.nchunks + 3) / 4) * kTiles));
}

}  // namespace

extern "C" {

size_t ogn_xcd_plan_bytes(int64_t m, int64_t nnz) {
  if (m < 0 || nnz < 0) return 0;
  return plan_bytes(m, nnz);
}

int ogn_xcd_plan(const void* rowptr, const void* col, int index_dtype, int64_t m, int64_t n_cols, int64_t nnz,
                 void* plan, size_t plan_size, int* sorted, void* stream) {
  if (m <= 0 || n_cols <= 0 || nnz <= 0) return fail(OGN_EINVAL, "ogn_xcd_plan: empty graph");
  if (nnz >= (int64_t)1 << 31) return fail(OGN_EUNSUPPORTED, "ogn_xcd_plan: 2^31 or more edges");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64) return fail(OGN_EINVAL, "ogn_xcd_plan: index dtype");
  if (!rowptr || !col || !plan || !sorted) return fail(OGN_EINVAL, "ogn_xcd_plan: null pointer");
  if (plan_size < plan_bytes(m, nnz)) return fail(OGN_EINVAL, "ogn_xcd_plan: plan buffer too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const XcdPlan pl = plan_view(plan, m, nnz);
  int64_t* chunk_row = const_cast<int64_t*>(pl.chunk_row);
  int64_t* split = const_cast<int64_t*>(pl.split);
  int* flag = static_cast<int*>(plan);
  hipLaunchKernelGGL(zero_int_kernel, dim3(1), dim3(1), 0, s, flag);
  const unsigned cb = (unsigned)((pl.nchunks + 1 + kBlock - 1) / kBlock);
  const unsigned rbk = (unsigned)((m + kBlock - 1) / kBlock);
  const unsigned wb = (unsigned)((m + 3) / 4);
  const int64_t tw = tile_width(n_cols);
  const unsigned eb = (unsigned)((nnz + kBlock - 1) / kBlock);
  if (index_dtype == OGN_I64) {
    const int64_t* p = static_cast<const int64_t*>(rowptr);
    const int64_t* c = static_cast<const int64_t*>(col);
    hipLaunchKernelGGL(plan_chunk_rows_kernel<int64_t>, dim3(cb), dim3(kBlock), 0, s, p, m, pl.nchunks, chunk_row);
    hipLaunchKernelGGL(plan_split_kernel<int64_t>, dim3(rbk), dim3(kBlock), 0, s, p, c, m, tw, split);
    hipLaunchKernelGGL(plan_sorted_kernel<int64_t>, dim3(wb), dim3(kBlock), 0, s, p, c, m, flag);
    if (n_cols <= kCol16MaxCols)
      hipLaunchKernelGGL(plan_col16_kernel<int64_t>, dim3(eb), dim3(kBlock), 0, s, c, nnz, tw,
                         const_cast<uint16_t*>(pl.col16));
  } else {
    const int32_t* p = static_cast<const int32_t*>(rowptr);
    const int32_t* c = static_cast<const int32_t*>(col);
    hipLaunchKernelGGL(plan_chunk_rows_kernel<int32_t>, dim3(cb), dim3(kBlock), 0, s, p, m, pl.nchunks, chunk_row);
    hipLaunchKernelGGL(plan_split_kernel<int32_t>, dim3(rbk), dim3(kBlock), 0, s, p, c, m, tw, split);
    hipLaunchKernelGGL(plan_sorted_kernel<int32_t>, dim3(wb), dim3(kBlock), 0, s, p, c, m, flag);
    if (n_cols <= kCol16MaxCols)
      hipLaunchKernelGGL(plan_col16_kernel<int32_t>, dim3(eb), dim3(kBlock), 0, s, c, nnz, tw,
                         const_cast<uint16_t*>(pl.col16));
  }
  int host = 1;
  if (hipMemcpyAsync(&host, flag, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(OGN_EHIP, "ogn_xcd_plan: reading the sortedness flag failed");
  // 1: sorted rows; 2: sorted, and the 16-bit tile-relative columns are kept
  *sorted = host != 0 ? 0 : (n_cols <= kCol16MaxCols ? 2 : 1);
  return check_launch("ogn_xcd_plan");
}

int ogn_sddmm_dot_xcd(const void* plan, int64_t m, int64_t nnz, const void* col, int index_dtype, const void* lhs,
                      int64_t lhs_rows, const void* rhs, int64_t rhs_rows, int64_t k, int dtype, void* out,
                      int plan_state, void* stream) {
  if (!plan || !col || !lhs || !rhs || !out) return fail(OGN_EINVAL, "ogn_sddmm_dot_xcd: null pointer");
  if (m <= 0 || nnz <= 0 || nnz >= (int64_t)1 << 31) return fail(OGN_EINVAL, "ogn_sddmm_dot_xcd: sizes");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_sddmm_dot_xcd: dtype must be float32, float16 or bfloat16");
  const int g = row_lanes(k, dtype);
  if (!g) return fail(OGN_EUNSUPPORTED, "ogn_sddmm_dot_xcd: feature rows must be 64, 128, 256 or 512 bytes");
  if (((uintptr_t)lhs % 16) || ((uintptr_t)rhs % 16)) return fail(OGN_EINVAL, "ogn_sddmm_dot_xcd: unaligned features");
  if ((uint64_t)rhs_rows * (uint64_t)(k * dtype_size(dtype)) >= (1ull << 32) ||
      (uint64_t)lhs_rows * (uint64_t)(k * dtype_size(dtype)) >= (1ull << 32))
    return fail(OGN_EUNSUPPORTED, "ogn_sddmm_dot_xcd: feature tables above 4 GiB");
  XcdArgs a{};
  a.pl = plan_view(plan, m, nnz);
  a.tile_w = tile_width(rhs_rows);
  a.col = col;
  a.lhs = lhs;
  a.rhs = rhs;
  a.out = out;
  a.lhs_rows = lhs_rows;
  a.rhs_rows = rhs_rows;
  a.k = k;
  a.dt = dtype;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // plan_state: what ogn_xcd_plan reported; 2 = 16-bit columns kept (the
  // plan was built with n_cols = rhs_rows)
  const bool c16 = plan_state == 2;
  TimedLaunch tl("sddmm_xcd", s);
  const bool i64 = index_dtype == OGN_I64;
  const dim3 grid = xcd_grid(a.pl);
  switch (dtype) {
    case OGN_F32: i64 ? launch_dot<OGN_F32, int64_t>(g, c16, grid, s, a) : launch_dot<OGN_F32, int32_t>(g, c16, grid, s, a); break;
    case OGN_F16: i64 ? launch_dot<OGN_F16, int64_t>(g, c16, grid, s, a) : launch_dot<OGN_F16, int32_t>(g, c16, grid, s, a); break;
    default: i64 ? launch_dot<OGN_BF16, int64_t>(g, c16, grid, s, a) : launch_dot<OGN_BF16, int32_t>(g, c16, grid, s, a); break;
  }
  return check_launch("ogn_sddmm_dot_xcd");
}

size_t ogn_spmm_sum_xcd_workspace_size(int64_t m, int64_t k) {
  if (m <= 0 || k <= 0) return 0;
  return sizeof(float) * (size_t)kTiles * (size_t)m * (size_t)k;
}

int ogn_spmm_sum_xcd(const void* plan, int64_t m, int64_t nnz, const void* col, int index_dtype, const void* value,
                     const void* mat, int64_t n, int64_t k, int dtype, void* out, int out_dtype, void* workspace,
                     size_t workspace_bytes, int plan_state, void* stream) {
  if (!plan || !col || !value || !mat || !out) return fail(OGN_EINVAL, "ogn_spmm_sum_xcd: null pointer");
  if (m <= 0 || nnz <= 0 || nnz >= (int64_t)1 << 31) return fail(OGN_EINVAL, "ogn_spmm_sum_xcd: sizes");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_spmm_sum_xcd: dtype must be float32, float16 or bfloat16");
  if (out_dtype != dtype && out_dtype != OGN_F32)
    return fail(OGN_EUNSUPPORTED, "ogn_spmm_sum_xcd: output dtype must be the input dtype or float32");
  const int g = row_lanes(k, dtype);
  if (!g) return fail(OGN_EUNSUPPORTED, "ogn_spmm_sum_xcd: feature rows must be 64, 128, 256 or 512 bytes");
  if (((uintptr_t)mat % 16) || ((uintptr_t)out % 16)) return fail(OGN_EINVAL, "ogn_spmm_sum_xcd: unaligned");
  if ((uint64_t)n * (uint64_t)(k * dtype_size(dtype)) >= (1ull << 32))
    return fail(OGN_EUNSUPPORTED, "ogn_spmm_sum_xcd: feature table above 4 GiB");
  if (!workspace || workspace_bytes < ogn_spmm_sum_xcd_workspace_size(m, k) || ((uintptr_t)workspace % 16))
    return fail(OGN_EINVAL, "ogn_spmm_sum_xcd: workspace too small or unaligned");
  XcdArgs a{};
  a.pl = plan_view(plan, m, nnz);
  a.tile_w = tile_width(n);
  a.col = col;
  a.rhs = mat;
  a.val = value;
  a.partial = static_cast<float*>(workspace);
  a.rhs_rows = n;
  a.k = k;
  a.dt = dtype;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool i64 = index_dtype == OGN_I64;
  const bool c16 = plan_state == 2;
  {
    TimedLaunch tl("spmm_xcd", s);
    const dim3 grid = xcd_grid(a.pl);
    switch (dtype) {
      case OGN_F32: i64 ? launch_sum<OGN_F32, int64_t>(g, c16, grid, s, a) : launch_sum<OGN_F32, int32_t>(g, c16, grid, s, a); break;
      case OGN_F16: i64 ? launch_sum<OGN_F16, int64_t>(g, c16, grid, s, a) : launch_sum<OGN_F16, int32_t>(g, c16, grid, s, a); break;
      default: i64 ? launch_sum<OGN_BF16, int64_t>(g, c16, grid, s, a) : launch_sum<OGN_BF16, int32_t>(g, c16, grid, s, a); break;
    }
  }
  {
    TimedLaunch tl("spmm_xcd_combine", s);
    const int64_t mk = m * k;
    const dim3 grid((unsigned)((mk / 4 + kBlock - 1) / kBlock));
    switch (out_dtype) {
      case OGN_F32: hipLaunchKernelGGL(combine_kernel<OGN_F32>, grid, dim3(kBlock), 0, s, a.partial, mk, out); break;
      case OGN_F16: hipLaunchKernelGGL(combine_kernel<OGN_F16>, grid, dim3(kBlock), 0, s, a.partial, mk, out); break;
      default: hipLaunchKernelGGL(combine_kernel<OGN_BF16>, grid, dim3(kBlock), 0, s, a.partial, mk, out); break;
    }
  }
  return check_launch("ogn_spmm_sum_xcd");
}

}  // extern "C"
