// CSR SpMM (torch_sparse semantics) for gfx950.
//
// Schedule: nnz-split.  The edge list [0, nnz) is cut into fixed chunks of C
// edges and one wavefront owns one chunk, so every wave does the same amount
// of gather work whatever the row-length distribution (power-law hub rows of
// 20 000 edges are spread over many waves, runs of short rows share one).
//
// Inside a wave the 64 lanes are split into S = 64 / G sub-groups of G lanes;
// a sub-group covers one feature row of `mat` with one 16-byte load per lane
// (G = K * sizeof(T) / 16), so a step gathers S edges at once and U steps are
// issued before any is consumed (S * U feature rows in flight per wave).
// Column indices and edge weights are staged with one coalesced load per 64
// edges and handed to the sub-groups with ds_bpermute; row ends come from a
// 64-row window of rowptr held one entry per lane (v_readlane).
//
// Ownership: a row is written by the chunk holding its last edge (empty rows
// by the chunk where their position falls).  A row that crosses a chunk
// boundary leaves a partial record: "tail" in each chunk it leaves, "head" in
// the chunk where it ends.  A fix-up kernel folds tail[c1..c2-1] + head[c2]
// in chunk order and finalises the row, so results are deterministic and no
// atomics are used.
#pragma once
#include "ogn_device.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace ogn {
namespace spmm {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kUnroll = 8;
constexpr int64_t kNone = INT64_MAX;

struct SpmmParams {
  const void* ptr;
  const void* col;
  const void* val;
  const void* mat;
  void* out;
  int64_t* arg;
  const int64_t* chunk_row;
  float* sum_head;
  float* sum_tail;
  double* mm_head;
  double* mm_tail;
  int64_t* arg_head;
  int64_t* arg_tail;
  int64_t m, n, k, nnz, chunk, nchunks;
  int val_mode;  // 0 none, 1 one weight per edge, 2 k weights per edge
  int out_dt;
  int reduce;
};

template <typename MT>
__device__ __forceinline__ bool mm_better(MT v, MT best, bool is_min) {
  return is_min ? v < best : v > best;
}

// Row ids of the first edge of every chunk: row r owns the chunk starts that
// fall inside [ptr[r], ptr[r+1]).
template <typename IDX>
__global__ __launch_bounds__(256) void chunk_rows_kernel(const IDX* __restrict__ ptr, int64_t m,
                                                         int64_t chunk, int64_t nchunks,
                                                         int64_t* __restrict__ chunk_row) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= m) return;
  const int64_t a = ptr[r], z = ptr[r + 1];
  if (z <= a) return;
  int64_t c0 = (a + chunk - 1) / chunk, c1 = (z - 1) / chunk;
  c0 = std::max<int64_t>(c0, 0);
  c1 = std::min<int64_t>(c1, nchunks - 1);
  for (int64_t c = c0; c <= c1; ++c) chunk_row[c] = r;
}

template <int DT, typename IDX, int G, bool VL, bool MM>
__global__ __launch_bounds__(kBlock) void spmm_chunk_kernel(SpmmParams p) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr int NE = VL ? E::VEC : 1;
  constexpr int S = kWave / G;
  using MT = std::conditional_t<DT == OGN_F32, double, float>;

  const int lane = lane_id();
  const int sub = lane / G;
  const int gl = lane % G;
  const int64_t c = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (c >= p.nchunks) return;
  const int64_t b = blockIdx.z;
  const int64_t K = p.k;
  const int64_t M = p.m;
  const int64_t k0 = (int64_t)blockIdx.y * (G * NE) + gl * NE;
  const bool kok = VL || k0 < K;
  const IDX* __restrict__ ptr = static_cast<const IDX*>(p.ptr);
  const IDX* __restrict__ col = static_cast<const IDX*>(p.col);
  const S_t* __restrict__ matb = static_cast<const S_t*>(p.mat) + b * p.n * K;
  const S_t* __restrict__ val = static_cast<const S_t*>(p.val);
  const bool is_min = p.reduce == OGN_REDUCE_MIN;
  const bool is_mean = p.reduce == OGN_REDUCE_MEAN;

  const int64_t lo = c * p.chunk;
  const int64_t hi = std::min(lo + p.chunk, p.nnz);
  int64_t r = c == 0 ? 0 : std::min<int64_t>(std::max<int64_t>(p.chunk_row[c], 0), M - 1);

  // rowptr window: lane j holds ptr[wb + 1 + j].
  int64_t wb = r;
  IDX pw = ptr[std::min<int64_t>(wb + 1 + lane, M)];
  auto rowend = [&](int64_t rr) -> int64_t {
    if (rr >= M) return kNone;
    if (rr - wb >= kWave) {
      wb = rr;
      pw = ptr[std::min<int64_t>(wb + 1 + lane, M)];
    }
    return (int64_t)readlane64(pw, (int)(rr - wb));
  };
  int64_t rs = (int64_t)ptr[r];
  int64_t re = rowend(r);
  const bool head_split = rs < lo;
  bool first = true;

  float acc[NE];
  MT best[NE];
  int64_t barg[NE];
  auto reset = [&]() {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      acc[i] = 0.f;
      best[i] = 0;
      barg[i] = kNone;
    }
  };
  reset();

  // Combine the S sub-group partials of the current row (all lanes end up
  // with the combined value).
  auto combine = [&]() {
#pragma unroll
    for (int off = G; off < kWave; off <<= 1) {
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        if constexpr (MM) {
          const MT ob = (MT)(sizeof(MT) == 8 ? shfld((double)best[i], lane ^ off)
                                             : shflf((float)best[i], lane ^ off));
          const int64_t oa = shfl64(barg[i], lane ^ off);
          const bool take = oa != kNone &&
                            (barg[i] == kNone || mm_better(ob, best[i], is_min) ||
                             (ob == best[i] && oa < barg[i]));
          if (take) {
            best[i] = ob;
            barg[i] = oa;
          }
        } else {
          acc[i] += shflf(acc[i], lane ^ off);
        }
      }
    }
  };

  const int64_t rec_base = (b * p.nchunks + c) * K + k0;
  auto write_record = [&](bool head) {
    if (sub != 0 || !kok) return;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      if (!VL && k0 + i >= K) break;
      if constexpr (MM) {
        (head ? p.mm_head : p.mm_tail)[rec_base + i] = (double)best[i];
        (head ? p.arg_head : p.arg_tail)[rec_base + i] = barg[i];
      } else {
        (head ? p.sum_head : p.sum_tail)[rec_base + i] = acc[i];
      }
    }
  };

  auto flush = [&]() {
    combine();
    if (head_split && first) {
      write_record(true);
    } else if (sub == 0 && kok) {
      const int64_t off = (b * M + r) * K + k0;
      float v[NE];
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        if constexpr (MM) {
          v[i] = barg[i] == kNone ? 0.f : (float)best[i];
        } else {
          const int64_t deg = re - rs;
          v[i] = is_mean ? (deg > 0 ? acc[i] / (float)deg : 0.f) : acc[i];
        }
      }
      store_floats<NE>(p.out, p.out_dt, off, v);
      if constexpr (MM) {
#pragma unroll
        for (int i = 0; i < NE; ++i) p.arg[off + i] = barg[i] == kNone ? p.nnz : barg[i];
      }
    }
    first = false;
    reset();
  };

  for (int64_t wbase = lo; wbase < hi; wbase += kWave) {
    const int64_t el = wbase + lane;
    const bool ev = el < hi;
    int64_t cl = ev ? (int64_t)load_stream(col + el) : 0;
    cl = std::min<int64_t>(std::max<int64_t>(cl, 0), p.n - 1);
    const IDX cli = (IDX)cl;
    float vl = 1.f;
    if (p.val_mode == 1) vl = ev ? E::load1(val, el) : 0.f;
    const int nw = (int)std::min<int64_t>(kWave, hi - wbase);
    const int nsteps = (nw + S - 1) / S;
    for (int j0 = 0; j0 < nsteps; j0 += kUnroll) {
      float x[kUnroll][NE];
      float w[kUnroll][VL ? NE : 1];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int idx = (j0 + u) * S + sub;
        const int64_t cc = (int64_t)shfl64(cli, idx & (kWave - 1));
        const float ws = shflf(vl, idx & (kWave - 1));
        const bool ok = (j0 + u) < nsteps && idx < nw && kok;
        if constexpr (VL) {
          if (ok) {
            E::unpack(load16(matb + cc * K + k0), x[u]);
          } else {
#pragma unroll
            for (int i = 0; i < NE; ++i) x[u][i] = 0.f;
          }
#pragma unroll
          for (int i = 0; i < NE; ++i) w[u][i] = ws;
          if (p.val_mode == 2 && ok) {
            float wv[NE];
            E::unpack(load16(val + (wbase + idx) * K + k0), wv);
#pragma unroll
            for (int i = 0; i < NE; ++i) w[u][i] = wv[i];
          }
        } else {
          x[u][0] = ok ? E::load1(matb, cc * K + k0) : 0.f;
          w[u][0] = ws;
          if (p.val_mode == 2 && ok) w[u][0] = E::load1(val, (wbase + idx) * K + k0);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (j0 + u >= nsteps) break;
        const int64_t e_first = wbase + (int64_t)(j0 + u) * S;
        const int64_t last = std::min<int64_t>(e_first + S, hi) - 1;
        const int64_t e_mine = e_first + sub;
        const bool valid = e_mine < hi;
        bool added = false;
        while (true) {
          if (!added && valid && e_mine < re) {
#pragma unroll
            for (int i = 0; i < NE; ++i) {
              const float wi = w[u][VL ? i : 0];
              if constexpr (MM) {
                const MT pv = (MT)x[u][i] * (MT)wi;
                if (!__builtin_isnan(pv) &&
                    (barg[i] == kNone || mm_better(pv, best[i], is_min))) {
                  best[i] = pv;
                  barg[i] = e_mine;
                }
              } else {
                acc[i] = __builtin_fmaf(x[u][i], wi, acc[i]);
              }
            }
            added = true;
          }
          if (last < re) break;
          flush();
          ++r;
          rs = re;
          re = rowend(r);
        }
      }
    }
  }
  // Rows that end exactly at `hi` and the empty rows behind them.
  while (r < M && re <= hi) {
    flush();
    ++r;
    rs = re;
    re = rowend(r);
  }
  if (r < M && rs < hi) {
    combine();
    write_record(false);
  }
}

// Finalise rows that cross chunk boundaries: one wave per chunk that holds
// the first piece of such a row.
template <typename IDX, bool MM>
__global__ __launch_bounds__(kBlock) void spmm_fixup_kernel(SpmmParams p) {
  const int lane = lane_id();
  const int64_t c = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (c + 1 >= p.nchunks) return;
  const int64_t b = blockIdx.z;
  const IDX* __restrict__ ptr = static_cast<const IDX*>(p.ptr);
  const int64_t lo = c * p.chunk, hi = lo + p.chunk;
  const int64_t r = std::min<int64_t>(std::max<int64_t>(p.chunk_row[c + 1], 0), p.m - 1);
  const int64_t rs = ptr[r];
  if (!(rs < hi && rs >= lo)) return;
  const int64_t re = ptr[r + 1];
  const int64_t c2 = std::min<int64_t>((re - 1) / p.chunk, p.nchunks - 1);
  const int64_t K = p.k;
  const bool is_min = p.reduce == OGN_REDUCE_MIN;
  for (int64_t k = lane; k < K; k += kWave) {
    const int64_t off = (b * p.m + r) * K + k;
    float v;
    if constexpr (MM) {
      double best = p.mm_tail[(b * p.nchunks + c) * K + k];
      int64_t barg = p.arg_tail[(b * p.nchunks + c) * K + k];
      for (int64_t cc = c + 1; cc <= c2; ++cc) {
        const int64_t ri = (b * p.nchunks + cc) * K + k;
        const double ob = cc < c2 ? p.mm_tail[ri] : p.mm_head[ri];
        const int64_t oa = cc < c2 ? p.arg_tail[ri] : p.arg_head[ri];
        if (oa != kNone && (barg == kNone || mm_better(ob, best, is_min))) {
          best = ob;
          barg = oa;
        }
      }
      v = barg == kNone ? 0.f : (float)best;
      p.arg[off] = barg == kNone ? p.nnz : barg;
    } else {
      float a = p.sum_tail[(b * p.nchunks + c) * K + k];
      for (int64_t cc = c + 1; cc < c2; ++cc) a += p.sum_tail[(b * p.nchunks + cc) * K + k];
      a += p.sum_head[(b * p.nchunks + c2) * K + k];
      if (p.reduce == OGN_REDUCE_MEAN) a = a / (float)(re - rs);
      v = a;
    }
    store_floats<1>(p.out, p.out_dt, off, &v);
  }
}

struct Plan {
  bool vec;
  int g;
  int64_t tiles;
  int64_t chunk;
  int64_t nchunks;
};

template <int DT, typename IDX, bool VL, bool MM>
void launch_g(int g, dim3 grid, hipStream_t s, const SpmmParams& p) {
  switch (g) {
#define OGN_G(GV) \
  case GV: hipLaunchKernelGGL((spmm_chunk_kernel<DT, IDX, GV, VL, MM>), grid, dim3(kBlock), 0, s, p); break;
    OGN_G(1) OGN_G(2) OGN_G(4) OGN_G(8) OGN_G(16) OGN_G(32) OGN_G(64)
#undef OGN_G
    default: break;
  }
}

template <int DT, typename IDX>
void launch_main(const Plan& pl, bool mm, dim3 grid, hipStream_t s, const SpmmParams& p) {
  if (pl.vec) {
    if (mm) launch_g<DT, IDX, true, true>(pl.g, grid, s, p);
    else launch_g<DT, IDX, true, false>(pl.g, grid, s, p);
  } else {
    // Scalar fallback (k not a multiple of 16 bytes or unaligned): one lane
    // per feature, one edge per step.
    if (mm) hipLaunchKernelGGL((spmm_chunk_kernel<DT, IDX, 64, false, true>), grid, dim3(kBlock), 0, s, p);
    else hipLaunchKernelGGL((spmm_chunk_kernel<DT, IDX, 64, false, false>), grid, dim3(kBlock), 0, s, p);
  }
}


void launch_f32(const Plan&, bool, dim3, hipStream_t, const SpmmParams&, bool i64);
void launch_f16(const Plan&, bool, dim3, hipStream_t, const SpmmParams&, bool i64);
void launch_bf16(const Plan&, bool, dim3, hipStream_t, const SpmmParams&, bool i64);

}  // namespace spmm
}  // namespace ogn
