// Generalised CSR SDDMM for gfx950:  out[e] = phi(lhs[t_l(e)], rhs[t_r(e)])
// with targets 0 = row of e (src), 1 = e itself (edge), 2 = col[e] (dst) and
// phi in {dot, add, sub, mul, div, copy_lhs, copy_rhs}.  dot reduces the
// feature axis (out [nnz]); the others keep it (out [nnz, k]).
//
// Schedule: nnz-split, like the CSR engine -- one wavefront per chunk of C
// edges.  Inside a wave, S = 64 / G sub-groups each take one edge per step
// and G lanes cover its feature row with 16-byte loads (vector mode) or one
// element per lane (scalar mode).  The row of every edge comes from a
// wave-uniform walk over a 64-entry rowptr window (no per-edge search, no
// row-index array in memory).  dot is reduced across the G lanes of a
// sub-group with ds_bpermute.  fp16 / bf16 compute in fp32 and round once.
#include "csr_engine.h"
#include "dot.h"

#include <string>

using namespace ogn;

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kU = 4;
constexpr int64_t kNoRow = INT64_MAX;

enum { SD_DOT = 0, SD_ADD = 1, SD_SUB = 2, SD_MUL = 3, SD_DIV = 4, SD_COPY_LHS = 5, SD_COPY_RHS = 6 };

struct SddmmParams {
  const void* ptr;
  const void* col;
  const void* lhs;
  const void* rhs;
  void* out;
  const int64_t* chunk_row;
  int64_t m, nnz, k, lhs_rows, rhs_rows, chunk, nchunks;
  int op, lt, rt;
  int dt;
};

template <typename IDX>
__global__ __launch_bounds__(256) void sddmm_chunk_rows(const IDX* __restrict__ ptr, int64_t m, int64_t chunk,
                                                       int64_t nchunks, int64_t* __restrict__ chunk_row) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= m) return;
  const int64_t a = ptr[r], z = ptr[r + 1];
  if (z <= a) return;
  const int64_t c0 = std::max<int64_t>((a + chunk - 1) / chunk, 0);
  const int64_t c1 = std::min<int64_t>((z - 1) / chunk, nchunks - 1);
  for (int64_t c = c0; c <= c1; ++c) chunk_row[c] = r;
}

template <int DT, typename IDX, int G, bool VL>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4))) void sddmm_kernel(SddmmParams p) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr int NE = VL ? E::VEC : 1;
  constexpr int S = kWave / G;
  const int lane = lane_id();
  const int sub = lane / G;
  const int gl = lane % G;
  const int64_t c = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (c >= p.nchunks) return;
  const IDX* __restrict__ ptr = static_cast<const IDX*>(p.ptr);
  const IDX* __restrict__ col = static_cast<const IDX*>(p.col);
  const S_t* __restrict__ lhs = static_cast<const S_t*>(p.lhs);
  const S_t* __restrict__ rhs = static_cast<const S_t*>(p.rhs);
  const int64_t K = p.k;
  const int64_t M = p.m;
  const int64_t lo = c * p.chunk;
  const int64_t hi = std::min(lo + p.chunk, p.nnz);
  const bool need_row = p.lt == 0 || p.rt == 0;
  const bool use_l = p.op != SD_COPY_RHS, use_r = p.op != SD_COPY_LHS;
  // feature passes: scalar mode covers k in chunks of G lanes
  const int64_t kpass = VL ? 1 : (K + G - 1) / G;

  int64_t r = std::min<int64_t>(std::max<int64_t>(p.chunk_row[c], 0), std::max<int64_t>(M - 1, 0));
  int64_t wb = r;
  IDX pw = ptr[std::min<int64_t>(wb + 1 + lane, M)];
  auto rowend = [&](int64_t rr) -> int64_t {
    if (rr >= M) return kNoRow;
    if (rr - wb >= kWave) {
      wb = rr;
      pw = ptr[std::min<int64_t>(wb + 1 + lane, M)];
    }
    return (int64_t)readlane64(pw, (int)(rr - wb));
  };
  int64_t re = need_row ? rowend(r) : kNoRow;

  // An operand gathered by row (target 0) is loaded once per row change of
  // the sub-group and kept in registers; `held_*` is the row it holds.
  int64_t held_l = -1, held_r = -1;
  uint4 keep_l = make_uint4(0u, 0u, 0u, 0u), keep_r = keep_l;

  for (int64_t wbase = lo; wbase < hi; wbase += kWave) {
    const int64_t el = wbase + lane;
    int64_t cl = el < hi ? (int64_t)load_stream(col + el) : 0;
    const int nw = (int)std::min<int64_t>(kWave, hi - wbase);
    const int nsteps = (nw + S - 1) / S;
    for (int j0 = 0; j0 < nsteps; j0 += kU) {
      // Phase 1: rows of the U steps (wave-uniform walk) and column shuffles.
      int64_t row[kU], cc[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        row[u] = 0;
        cc[u] = (int64_t)shfl64(cl, ((j0 + u) * S + sub) & (kWave - 1));
        if (!need_row || j0 + u >= nsteps) continue;
        const int64_t e_first = wbase + (int64_t)(j0 + u) * S;
        const int64_t last = std::min<int64_t>(e_first + S, hi) - 1;
        const int64_t e_mine = e_first + sub;
        bool got = false;
        while (true) {
          if (!got && e_mine < re) {
            row[u] = r;
            got = true;
          }
          if (last < re) break;
          ++r;
          re = rowend(r);
        }
      }
      float dsum[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) dsum[u] = 0.f;
      for (int64_t kp = 0; kp < kpass; ++kp) {
        const int64_t k0 = VL ? (int64_t)gl * NE : kp * G + gl;
        const bool kok = VL || k0 < K;
        // Phase 2: issue every gather of the U steps back to back (raw).
        uint4 rl[kU], rr[kU];
        float sl[kU], sr[kU];
        bool ok[kU], new_l[kU], new_r[kU];
        int64_t pl_ = held_l, pr_ = held_r;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int idx = (j0 + u) * S + sub;
          const int64_t e = wbase + idx;
          ok[u] = (j0 + u) < nsteps && idx < nw;
          const int64_t li = p.lt == 0 ? row[u] : (p.lt == 1 ? e : cc[u]);
          const int64_t ri = p.rt == 0 ? row[u] : (p.rt == 1 ? e : cc[u]);
          const bool lok = ok[u] && kok && use_l && li >= 0 && li < p.lhs_rows;
          const bool rok = ok[u] && kok && use_r && ri >= 0 && ri < p.rhs_rows;
          // reuse only in vector mode (one pass holds the whole feature row)
          new_l[u] = !(VL && p.lt == 0 && li == pl_);
          new_r[u] = !(VL && p.rt == 0 && ri == pr_);
          if (VL && p.lt == 0 && ok[u]) pl_ = li;
          if (VL && p.rt == 0 && ok[u]) pr_ = ri;
          rl[u] = make_uint4(0u, 0u, 0u, 0u);
          rr[u] = rl[u];
          sl[u] = 0.f;
          sr[u] = 0.f;
          if constexpr (VL) {
            if (lok && new_l[u]) rl[u] = load16(lhs + li * K + k0);
            if (rok && new_r[u]) rr[u] = load16(rhs + ri * K + k0);
          } else {
            if (lok) sl[u] = E::load1(lhs, li * K + k0);
            if (rok) sr[u] = E::load1(rhs, ri * K + k0);
          }
          if (!lok) new_l[u] = true;  // a skipped operand reads as zero
          if (!rok) new_r[u] = true;
        }
        held_l = pl_;
        held_r = pr_;
        // Phase 3: consume in order.
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          float xl[NE], xr[NE];
          if constexpr (VL) {
            // steps past the end of the window leave the held rows alone
            if (ok[u] && new_l[u]) keep_l = rl[u];
            if (ok[u] && new_r[u]) keep_r = rr[u];
            E::unpack(keep_l, xl);
            E::unpack(keep_r, xr);
          } else {
            xl[0] = sl[u];
            xr[0] = sr[u];
          }
          if (p.op == SD_DOT) {
#pragma unroll
            for (int i = 0; i < NE; ++i) dsum[u] = __builtin_fmaf(xl[i], xr[i], dsum[u]);
          } else if (ok[u] && kok) {
            float v[NE];
#pragma unroll
            for (int i = 0; i < NE; ++i) {
              const float a = xl[i], b = xr[i];
              switch (p.op) {
                case SD_ADD: v[i] = a + b; break;
                case SD_SUB: v[i] = a - b; break;
                case SD_MUL: v[i] = a * b; break;
                case SD_DIV: v[i] = a / b; break;
                case SD_COPY_LHS: v[i] = a; break;
                default: v[i] = b; break;
              }
            }
            store_floats<NE>(p.out, p.dt, (wbase + (j0 + u) * S + sub) * K + k0, v);
          }
        }
      }
      if (p.op == SD_DOT) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          float d = dsum[u];
          // reduce over the G lanes of the sub-group (fixed order: all lanes agree)
#pragma unroll
          for (int off = G >> 1; off > 0; off >>= 1) {
            const float o = shflf(d, lane ^ off);
            d = (lane & off) ? o + d : d + o;
          }
          const int idx = (j0 + u) * S + sub;
          if (gl == 0 && (j0 + u) < nsteps && idx < nw) store_floats<1>(p.out, p.dt, wbase + idx, &d);
        }
      }
    }
  }
}

// Sum over the G lanes of a sub-group (G a power of two, lanes aligned to
// G); every lane of the sub-group ends with the same value.  Within 16-lane
// rows DPP permutes do it without the LDS unit: xor 1 and xor 2 by quad
// permutation, then the half-row and row mirrors pair each lane with one in
// the other half; wider groups add swizzle / bpermute rounds.


// dot(lhs[row(e)], rhs[col(e)]) -- the GAT score and the SpMM edge-weight
// gradient.  Specialises the generic kernel for that case: the lhs row is
// held in registers and reloaded only when a sub-group's row changes, rhs
// rows are gathered U at a time with 32-bit byte offsets from a uniform
// base, packets are dotted with the dot2 instructions, the sub-group
// reduction uses DPP, and column indices of the next window are loaded one
// window ahead.  A block of U steps lying inside the current row (most of
// them: rows are long) skips the per-step row walk.  The 64 results of a
// window are gathered one per lane -- lane s * G + j keeps step j of
// sub-group s -- and written with one store.
template <int DT, typename IDX, int G>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4)))
void sddmm_dot_kernel(SddmmParams p) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr int NE = E::VEC;
  constexpr int S = kWave / G;
  constexpr int NSTEPS = kWave / S;  // steps per 64-edge window (= G)
  constexpr int U = NSTEPS < 8 ? NSTEPS : 8;
  const int lane = lane_id();
  const int sub = lane / G;
  const int gl = lane % G;
  const int64_t c = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (c >= p.nchunks) return;
  const IDX* __restrict__ ptr = static_cast<const IDX*>(p.ptr);
  const IDX* __restrict__ col = static_cast<const IDX*>(p.col);
  const char* __restrict__ lhs = static_cast<const char*>(p.lhs);
  const char* __restrict__ rhs = static_cast<const char*>(p.rhs);
  const uint32_t row_bytes = (uint32_t)(p.k * sizeof(S_t));
  const uint32_t k_off = (uint32_t)(gl * NE * sizeof(S_t));
  const int64_t M = p.m;
  const int64_t lo = c * p.chunk;
  const int64_t hi = std::min(lo + p.chunk, p.nnz);

  int64_t r = std::min<int64_t>(std::max<int64_t>(p.chunk_row[c], 0), std::max<int64_t>(M - 1, 0));
  int64_t wb = r;
  IDX pw = ptr[std::min<int64_t>(wb + 1 + lane, M)];
  auto rowend = [&](int64_t rr) -> int64_t {
    if (rr >= M) return kNoRow;
    if (rr - wb >= kWave) {
      wb = rr;
      pw = ptr[std::min<int64_t>(wb + 1 + lane, M)];
    }
    return (int64_t)readlane64(pw, (int)(rr - wb));
  };
  int64_t re = rowend(r);

  int64_t held = -1;
  uint4 keep = make_uint4(0u, 0u, 0u, 0u);
  auto hold = [&](int64_t row) {
    if (row != held) {  // rare: a new row for this sub-group
      held = row;
      keep = held < p.lhs_rows ? load16(lhs + (uint64_t)held * row_bytes + k_off) : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  int32_t cl_next = 0;
  auto stage = [&](int64_t w) {
    const int64_t el = w + lane;
    cl_next = el < hi ? (int32_t)load_stream(col + el) : 0;
  };
  stage(lo);
  for (int64_t wbase = lo; wbase < hi; wbase += kWave) {
    const int32_t cl = std::min<int32_t>(std::max<int32_t>(cl_next, 0), (int32_t)(p.rhs_rows - 1));
    if (wbase + kWave < hi) stage(wbase + kWave);
    const int nw = (int)std::min<int64_t>(kWave, hi - wbase);
    const int nsteps = (nw + S - 1) / S;
    float mine = 0.f;  // this lane's result: step gl of sub-group sub
    for (int j0 = 0; j0 < nsteps; j0 += U) {
      uint32_t co[U];
#pragma unroll
      for (int u = 0; u < U; ++u) co[u] = (uint32_t)shfl32(cl, ((j0 + u) * S + sub) & (kWave - 1)) * row_bytes + k_off;
      uint4 xr[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = (j0 + u) < nsteps && (j0 + u) * S + sub < nw;
        xr[u] = ok ? load16(rhs + co[u]) : make_uint4(0u, 0u, 0u, 0u);
      }
      const int64_t block_last = wbase + std::min<int64_t>((int64_t)(j0 + U) * S, nw) - 1;
      if (block_last < re) {
        // every edge of the block is in row r
        hold(r);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float d = group_sum<G>(packet_dot<DT>(keep, xr[u], 0.f));
          if (gl == j0 + u) mine = d;
        }
        continue;
      }
      int64_t row[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        row[u] = 0;
        if (j0 + u >= nsteps) continue;
        const int64_t e_first = wbase + (int64_t)(j0 + u) * S;
        const int64_t last = std::min<int64_t>(e_first + S, hi) - 1;
        const int64_t e_mine = e_first + sub;
        bool got = false;
        while (true) {
          if (!got && e_mine < re) {
            row[u] = r;
            got = true;
          }
          if (last < re) break;
          ++r;
          re = rowend(r);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = (j0 + u) < nsteps && (j0 + u) * S + sub < nw;
        if (ok) hold(row[u]);
        const float d = group_sum<G>(packet_dot<DT>(keep, xr[u], 0.f));
        if (gl == j0 + u) mine = d;
      }
    }
    const int idx = gl * S + sub;  // window edge of this lane's result
    if (idx < nw) store_floats<1>(p.out, p.dt, wbase + idx, &mine);
  }
}

template <int DT, typename IDX>
void launch(bool vec, int g, dim3 grid, hipStream_t s, const SddmmParams& p) {
  if (!vec) {
    switch (g) {
      case 1: hipLaunchKernelGGL((sddmm_kernel<DT, IDX, 1, false>), grid, dim3(kBlock), 0, s, p); break;
      case 8: hipLaunchKernelGGL((sddmm_kernel<DT, IDX, 8, false>), grid, dim3(kBlock), 0, s, p); break;
      default: hipLaunchKernelGGL((sddmm_kernel<DT, IDX, 64, false>), grid, dim3(kBlock), 0, s, p); break;
    }
    return;
  }
  switch (g) {
#define OGN_G(GV) \
  case GV: hipLaunchKernelGGL((sddmm_kernel<DT, IDX, GV, true>), grid, dim3(kBlock), 0, s, p); break;
    OGN_G(1) OGN_G(2) OGN_G(4) OGN_G(8) OGN_G(16) OGN_G(32) OGN_G(64)
#undef OGN_G
    default: break;
  }
}

template <int DT, typename IDX>
void launch_dot(int g, dim3 grid, hipStream_t s, const SddmmParams& p) {
  switch (g) {
#define OGN_G(GV) \
  case GV: hipLaunchKernelGGL((sddmm_dot_kernel<DT, IDX, GV>), grid, dim3(kBlock), 0, s, p); break;
    OGN_G(1) OGN_G(2) OGN_G(4) OGN_G(8) OGN_G(16) OGN_G(32) OGN_G(64)
#undef OGN_G
    default: break;
  }
}

struct SdPlan {
  bool vec;
  int g;
  int64_t chunk, nchunks;
};

SdPlan sd_plan(int64_t nnz, int64_t k, int dt, bool aligned) {
  SdPlan pl{};
  const int esz = dtype_size(dt);
  const int vec = 16 / esz;
  const int64_t kv = k / vec;
  if (aligned && k % vec == 0 && kv >= 1 && kv <= 64 && (kv & (kv - 1)) == 0) {
    pl.vec = true;
    pl.g = (int)kv;
  } else {
    pl.vec = false;
    pl.g = k == 1 ? 1 : (k <= 8 ? 8 : 64);
  }
  const int64_t row_bytes = std::max<int64_t>(1, std::min<int64_t>(k, 64 * vec) * esz);
  int64_t chunk = (65536 / row_bytes + 63) / 64 * 64;
  pl.chunk = std::min<int64_t>(std::max<int64_t>(chunk, 64), 8192);
  pl.nchunks = std::max<int64_t>(1, (nnz + pl.chunk - 1) / pl.chunk);
  return pl;
}

bool is_aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

extern "C" {

size_t ogn_sddmm_csr_workspace_size(int64_t nnz, int64_t k, int dtype) {
  if (nnz < 0 || k <= 0) return 0;
  return (size_t)std::max(sd_plan(nnz, k, dtype, true).nchunks, sd_plan(nnz, k, dtype, false).nchunks) *
             sizeof(int64_t) + 256;
}

int ogn_sddmm_csr(const void* rowptr, const void* col, int index_dtype, int64_t m, int64_t nnz,
                  const void* lhs, int64_t lhs_rows, int lhs_target, const void* rhs, int64_t rhs_rows,
                  int rhs_target, int64_t k, int dtype, int op, void* out, void* workspace,
                  size_t workspace_bytes, void* stream) {
  if (m < 0 || nnz < 0 || k < 0 || lhs_rows < 0 || rhs_rows < 0) return fail(OGN_EINVAL, "ogn_sddmm_csr: negative size");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_sddmm_csr: index dtype must be int32 or int64");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_sddmm_csr: dtype must be float32, float16 or bfloat16");
  if (op < SD_DOT || op > SD_COPY_RHS) return fail(OGN_EINVAL, "ogn_sddmm_csr: unknown op");
  if (lhs_target < 0 || lhs_target > 2 || rhs_target < 0 || rhs_target > 2)
    return fail(OGN_EINVAL, "ogn_sddmm_csr: targets must be 0, 1 or 2");
  if (nnz == 0 || k == 0) return OGN_OK;
  if (!rowptr || !col || !out || (op != SD_COPY_RHS && !lhs) || (op != SD_COPY_LHS && !rhs))
    return fail(OGN_EINVAL, "ogn_sddmm_csr: null pointer");
  if (m == 0) return fail(OGN_EINVAL, "ogn_sddmm_csr: nnz > 0 needs rows");
  const bool aligned = (op == SD_COPY_RHS || is_aligned(lhs, 16)) && (op == SD_COPY_LHS || is_aligned(rhs, 16)) &&
                       (op == SD_DOT || is_aligned(out, 16));
  const SdPlan pl = sd_plan(nnz, k, dtype, aligned);
  if (!workspace || workspace_bytes < (size_t)pl.nchunks * sizeof(int64_t))
    return fail(OGN_EINVAL, "ogn_sddmm_csr: workspace too small");
  SddmmParams p{};
  p.ptr = rowptr;
  p.col = col;
  p.lhs = lhs;
  p.rhs = rhs;
  p.out = out;
  p.chunk_row = static_cast<const int64_t*>(workspace);
  p.m = m;
  p.nnz = nnz;
  p.k = k;
  p.lhs_rows = lhs_rows;
  p.rhs_rows = rhs_rows;
  p.chunk = pl.chunk;
  p.nchunks = pl.nchunks;
  p.op = op;
  p.lt = lhs_target;
  p.rt = rhs_target;
  p.dt = dtype;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool i64 = index_dtype == OGN_I64;
  {
    TimedLaunch t("sddmm_chunk_rows", s);
    const dim3 g((unsigned)((m + 255) / 256));
    if (i64)
      hipLaunchKernelGGL(sddmm_chunk_rows<int64_t>, g, dim3(256), 0, s, static_cast<const int64_t*>(rowptr), m,
                         pl.chunk, pl.nchunks, static_cast<int64_t*>(workspace));
    else
      hipLaunchKernelGGL(sddmm_chunk_rows<int32_t>, g, dim3(256), 0, s, static_cast<const int32_t*>(rowptr), m,
                         pl.chunk, pl.nchunks, static_cast<int64_t*>(workspace));
  }
  const dim3 grid((unsigned)((pl.nchunks + kWaves - 1) / kWaves));
  TimedLaunch t("sddmm_main", s);
  // dot(lhs[row], rhs[col]) with vector rows and 32-bit offsets -> the specialised kernel
  const uint64_t rbytes = (uint64_t)rhs_rows * (uint64_t)k * (uint64_t)dtype_size(dtype);
  if (op == SD_DOT && lhs_target == 0 && rhs_target == 2 && pl.vec && rbytes < (1ull << 32) && rhs_rows > 0) {
    switch (dtype) {
      case OGN_F32: i64 ? launch_dot<OGN_F32, int64_t>(pl.g, grid, s, p) : launch_dot<OGN_F32, int32_t>(pl.g, grid, s, p); break;
      case OGN_F16: i64 ? launch_dot<OGN_F16, int64_t>(pl.g, grid, s, p) : launch_dot<OGN_F16, int32_t>(pl.g, grid, s, p); break;
      default: i64 ? launch_dot<OGN_BF16, int64_t>(pl.g, grid, s, p) : launch_dot<OGN_BF16, int32_t>(pl.g, grid, s, p); break;
    }
    return check_launch("ogn_sddmm_csr");
  }
  switch (dtype) {
    case OGN_F32: i64 ? launch<OGN_F32, int64_t>(pl.vec, pl.g, grid, s, p) : launch<OGN_F32, int32_t>(pl.vec, pl.g, grid, s, p); break;
    case OGN_F16: i64 ? launch<OGN_F16, int64_t>(pl.vec, pl.g, grid, s, p) : launch<OGN_F16, int32_t>(pl.vec, pl.g, grid, s, p); break;
    default: i64 ? launch<OGN_BF16, int64_t>(pl.vec, pl.g, grid, s, p) : launch<OGN_BF16, int32_t>(pl.vec, pl.g, grid, s, p); break;
  }
  return check_launch("ogn_sddmm_csr");
}

}  // extern "C"
