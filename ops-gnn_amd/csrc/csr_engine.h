// CSR reduction engine for gfx950: the one kernel family behind CSR SpMM,
// segment_csr, segment_coo, sorted-index scatter and segment log-sum-exp.
//
//   out[b, r, k] = R_{e in [ptr[r], ptr[r+1])} w(e, k) * x[b, row(e), k]
//
// row(e) = col[e] (gather mode, SpMM) or e itself (contiguous mode: segment
// reductions, where each segment is a run of consecutive rows of src).
// R = sum / mean / prod, min / max (+ arg), or log-sum-exp.
//
// Schedule: nnz-split.  The position range [ptr[0], ptr[m]) is cut into
// chunks of C positions and one wavefront owns one chunk, so every wave does
// the same amount of work whatever the row-length distribution (power-law
// hub rows are spread over many waves; runs of short rows share one).
//
// Inside a wave the 64 lanes form S = 64 / G sub-groups of G lanes; a
// sub-group covers one feature row with one 16-byte load per lane (vector
// mode, G = K * sizeof(T) / 16) or one element per lane (scalar mode), so a
// step touches S positions and U steps are in flight before any is consumed.
// Column indices and edge weights are staged with one coalesced load per 64
// positions and handed to the sub-groups with ds_bpermute; row ends come
// from a 64-row window of the pointer array held one entry per lane.
//
// Ownership: a row is finished by the chunk holding its last position (empty
// rows by the chunk their position falls in).  A row crossing a chunk
// boundary leaves partial records -- "tail" in each chunk it leaves, "head"
// in the chunk where it ends -- and a fix-up kernel folds
// tail[c1..c2-1] + head[c2] in chunk order and finishes the row.  Results are
// deterministic (no atomics; fixed combination order).
#pragma once

#include "ogn_device.h"
#include "search.h"

#include <algorithm>
#include <type_traits>

namespace ogn {
namespace eng {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kUnrollSum = 8;
constexpr int kUnrollSum32 = 8;  // 12 measured no faster at K=128 fp32
constexpr int kUnrollWide = 4;
constexpr int64_t kNone = INT64_MAX;
constexpr int32_t kNone32 = INT32_MAX;

// Reduction kinds (template parameter RK).
enum { RK_SUM = 0, RK_MINMAX = 1, RK_LSE = 2 };

// Extremum finishing rules.
enum {
  MM_SPMM = 0,    // torch_sparse: NaN ignored, first tie, none -> 0 / arg_empty
  MM_SEGCSR = 1,  // segment_csr: strict improvement from +-inf (arg = segment start)
  MM_LATER = 2,   // segment_coo / scatter: fold from a seed with >= / <=, later tie
  MM_NANPROP = 3  // DGL spmm: a NaN message makes the result NaN; empty -> 0, no arg
};
// Message = x (op) w for each position (w = edge weight, 1 when absent).
enum { OP_MUL = 0, OP_ADD = 1, OP_SUB = 2, OP_DIV = 3 };

template <typename T>
__device__ __forceinline__ T apply_op(T x, T w, int op) {
  switch (op) {
    case OP_ADD: return x + w;
    case OP_SUB: return x - w;
    case OP_DIV: return x / w;
    default: return x * w;
  }
}
// Seeds for MM_LATER.
enum {
  SEED_NONE = 0,
  SEED_OUT = 1,    // the current value of out (arg = arg_empty)
  SEED_FIRST = 2,  // the first element of the segment (arg = its position)
  SEED_LIMIT = 3   // +-limit (finite dtype extreme); still the seed at the end -> 0
};

struct Params {
  const void* ptr;
  int64_t ptr_bstride;  // elements between the pointer rows of batches (0 = shared)
  const void* col;      // gather mode
  const void* val;
  int val_mode;         // 0 none, 1 one weight per position, 2 k weights per position
  int val_op;           // OP_*: how a weight combines with the gathered feature
  const void* src;
  int src_dt;
  int64_t src_bstride;  // elements between batches of src
  void* out;
  int out_dt;
  int64_t out_bstride;  // elements between batches of out
  int64_t* arg;
  int64_t* chunk_row;   // [ptr batches][nchunks]
  longlong4* fix;       // [ptr batches][nchunks] {r, ptr[r], ptr[r + 1], -} of the
                        // row crossing chunk c's end from inside c; r = -1: none
  void* rec_head;       // [batch][nchunks][k] partial values
  void* rec_tail;
  int64_t* arg_head;    // [batch][nchunks][k] partial args (min/max)
  int64_t* arg_tail;
  int64_t m;            // rows of the output (segments)
  int64_t n;            // rows of src addressable (gather bound / length)
  int64_t k;            // features
  int64_t nnz_bound;    // host bound on ptr[m] - ptr[0] (sizes the grid)
  int64_t chunk;
  int64_t nchunks;
  int reduce;           // OGN_REDUCE_*
  int mm_mode;
  int seed_mode;
  int sum_seed;         // sum / mean start from the current out value
  int mean_keep_empty;  // mean of an empty row keeps the seed (else 0)
  float limit;
  int64_t arg_empty;
  float* aux;           // log-sum-exp statistics mode: out <- max, aux <- sum of exp
  int short_rows;       // contiguous fast variants: chunks of short rows take short_chunk
                        // (1), their finished rows staged in LDS (2)
  int src_nt;           // contiguous source read with non-temporal loads (NTS instances)
  int out_nt;           // staged extremum positions written with non-temporal stores
};

template <typename MT>
__device__ __forceinline__ bool better(MT v, MT best, bool is_min) {
  return is_min ? v < best : v > best;
}

__device__ __forceinline__ float clampf_max(float m) {
  return fminf(fmaxf(m, -3.402823466e38f), 3.402823466e38f);
}

// Log-sum-exp state merge: (m, s) = running max and sum of exp(x - clamp(m)).
__device__ __forceinline__ void lse_merge(float& m, float& s, float om, float os) {
  const float nm = fmaxf(m, om);
  const float cn = clampf_max(nm);
  const float a = s == 0.f ? 0.f : s * fast_exp(clampf_max(m) - cn);
  const float bb = os == 0.f ? 0.f : os * fast_exp(clampf_max(om) - cn);
  m = nm;
  s = a + bb;
}

__device__ __forceinline__ void lse_add(float& m, float& s, float x) {
  // Branch-free online update (lanes of a wave rarely agree on a new max):
  // nm = max(m, x) ignores NaN, so a NaN x leaves m and turns s into NaN;
  // +inf makes s infinite; -inf adds exp(-inf) = 0.  m never becomes NaN,
  // so the rescale factor exp(clamp(m) - clamp(nm)) lies in [0, 1].
  const float nm = fmaxf(m, x);
  const float cn = clampf_max(nm);
  s = __builtin_fmaf(s, fast_exp(clampf_max(m) - cn), fast_exp(x - cn));
  m = nm;
}

// int8 SpMM sum / mean from the exact int32 sum: an int32 output truncates
// the mean toward zero; an fp32 output takes the exact sum, or the quotient
// rounded once (fp64 divide, then one rounding to fp32).
__device__ __forceinline__ void finish_int(const Params& p, int64_t off, int32_t a, int64_t cnt) {
  const bool mean = p.reduce == OGN_REDUCE_MEAN;
  if (p.out_dt == OGN_I32) {
    static_cast<int32_t*>(p.out)[off] = mean ? (cnt > 0 ? a / (int32_t)cnt : 0) : a;
  } else {
    const double v = mean ? (cnt > 0 ? (double)a / (double)cnt : 0.0) : (double)a;
    static_cast<float*>(p.out)[off] = (float)v;
  }
}

// Finish one output element from its combined partial state.
//   sum kinds: a = sum (or product); mean divides by the row length.
//   min/max: (best, barg) resolved against the seed of the mode.
//   lse: (best = m, a = s).
template <int RK, typename MT>
__device__ __forceinline__ void finish_elem(const Params& p, int64_t b, int64_t r, int64_t k,
                                            int64_t rs, int64_t re, float a, MT best, int64_t barg,
                                            float* outv, int64_t* outarg) {
  const int64_t off = b * p.out_bstride + r * p.k + k;
  const int64_t cnt = re - rs;
  if constexpr (RK == RK_SUM) {
    float v = a;
    if (p.sum_seed) {
      const float seed = load_float(p.out, p.out_dt, off);
      v = p.reduce == OGN_REDUCE_PROD ? seed * v : seed + v;
    }
    if (p.reduce == OGN_REDUCE_MEAN) {
      if (cnt > 0) v = v / (float)cnt;
      else v = p.mean_keep_empty ? load_float(p.out, p.out_dt, off) : 0.f;
    }
    *outv = v;
  } else if constexpr (RK == RK_LSE) {
    if (p.aux) {
      *outv = cnt > 0 ? (float)best : -__builtin_inff();
      p.aux[off] = cnt > 0 ? a : 0.f;
    } else {
      *outv = cnt > 0 ? clampf_max(best) + logf(a) : -__builtin_inff();
    }
  } else {
    const bool is_min = p.reduce == OGN_REDUCE_MIN;
    const bool has = barg != kNone;
    if (p.mm_mode == MM_SPMM || p.mm_mode == MM_NANPROP) {
      *outv = has ? (float)best : 0.f;
      *outarg = has ? barg : p.arg_empty;
    } else if (p.mm_mode == MM_SEGCSR) {
      if (cnt <= 0) {
        *outv = 0.f;
        *outarg = p.arg_empty;
      } else {
        const MT sentinel = is_min ? (MT)__builtin_inff() : (MT)-__builtin_inff();
        const bool take = has && better(best, sentinel, is_min);
        *outv = take ? (float)best : (float)sentinel;
        *outarg = take ? barg : rs;
      }
    } else {
      MT sv;
      int64_t sa = p.arg_empty;
      if (p.seed_mode == SEED_OUT) {
        sv = (MT)load_float(p.out, p.out_dt, off);
      } else if (p.seed_mode == SEED_FIRST) {
        if (cnt <= 0) {
          *outv = 0.f;
          *outarg = p.arg_empty;
          return;
        }
        sv = (MT)load_float(p.src, p.src_dt, b * p.src_bstride + rs * p.k + k);
        sa = rs;
      } else {
        sv = is_min ? (MT)p.limit : (MT)-p.limit;
      }
      const bool take = has && !(sv != sv) && (is_min ? best <= sv : best >= sv);
      float v = take ? (float)best : (float)sv;
      const int64_t ra = take ? barg : sa;
      if (p.seed_mode == SEED_LIMIT && ra == p.arg_empty) v = 0.f;
      *outv = v;
      *outarg = ra;
    }
  }
}

// Row ids of the first position of every chunk (chunk_row[c]: the row r
// with ptr[r] <= base + c * chunk < ptr[r + 1]), and the fix-up entries
// (fix[c - 1]: that row when it starts inside chunk c - 1, so crosses its
// end; r = -1 otherwise).  One lane per chunk: the block brackets the rows of
// its 256 chunk starts with one 32-way wave search, stages that window of
// ptr in LDS when it holds at most kRowWindow entries, and each lane
// binary-searches its own start there (in global memory for a wider
// window).  A hub row spanning thousands of chunks costs no thread more than
// any other.  Every entry below the chunk count is rewritten on every call.
constexpr int kRowWindow = 4096;
template <typename IDX>
__global__ __launch_bounds__(256) void chunk_rows_kernel(Params p) {
  __shared__ int64_t win[kRowWindow];
  __shared__ int64_t bracket[2];
  const int64_t cb = (int64_t)blockIdx.x * blockDim.x;  // the block's first chunk
  const int64_t c = cb + threadIdx.x;
  const IDX* __restrict__ ptr = static_cast<const IDX*>(p.ptr) + blockIdx.y * p.ptr_bstride;
  const int64_t base = ptr[0];
  // the data end, computed as engine_kernel and fixup_kernel compute it
  const int64_t total = std::max<int64_t>(std::min<int64_t>((int64_t)ptr[p.m] - base, p.nnz_bound), 0);
  const int64_t nce = std::min<int64_t>(p.nchunks, (total + p.chunk - 1) / p.chunk);
  if (cb >= nce) return;  // whole block
  const int64_t clast = std::min<int64_t>(cb + (int64_t)blockDim.x - 1, nce - 1);
  if (threadIdx.x < kWave) {
    const int64_t ub = wave_upper_bound2(ptr, p.m + 1, base + cb * p.chunk, base + clast * p.chunk);
    if (threadIdx.x == 0 || threadIdx.x == 32) bracket[threadIdx.x >> 5] = ub;
  }
  __syncthreads();
  const int64_t L = bracket[0], H = bracket[1];  // every answer lies in [L, H]
  const bool staged = H - L <= kRowWindow;
  if (staged) {
    for (int64_t i = threadIdx.x; i < H - L; i += blockDim.x) win[i] = ptr[L + i];
    __syncthreads();
  }
  if (c > clast) return;
  const int64_t key = base + c * p.chunk;
  int64_t lo = L, hi = H;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    const int64_t v = staged ? win[mid - L] : (int64_t)ptr[mid];
    if (v <= key) lo = mid + 1;
    else hi = mid;
  }
  const int64_t r = std::min<int64_t>(std::max<int64_t>(lo - 1, 0), p.m - 1);
  p.chunk_row[blockIdx.y * p.nchunks + c] = r;
  if (c >= 1) {
    // ptr[r] and ptr[r + 1] from the staged window when it holds them
    const int64_t rs = staged && r >= L && r < H ? win[r - L] : (int64_t)ptr[r];
    const int64_t re = staged && r + 1 >= L && r + 1 < H ? win[r + 1 - L] : (int64_t)ptr[r + 1];
    const bool crosses = rs >= base + (c - 1) * p.chunk && rs < base + c * p.chunk;
    p.fix[blockIdx.y * p.nchunks + c - 1] = crosses ? make_longlong4(r, rs, re, 0) : make_longlong4(-1, 0, 0, 0);
  }
}

// Chunk c holds rows r0 (the row of its first position) up to r_end, the
// first row that ends past the chunk (m for the last chunk).
__device__ __forceinline__ int64_t chunk_row_end(const Params& p, int64_t pb, int64_t c, int64_t nce) {
  if (c + 1 >= nce) return p.m;
  return std::min<int64_t>(std::max<int64_t>(p.chunk_row[pb * p.nchunks + c + 1], 0), p.m - 1);
}

// Chunks that run short_chunk instead of the step schedule: those where
// some row both starts and ends (two or more row boundaries), or on average
// at most S positions (one step) per row.  The step schedule finishes every
// row with a cross-lane combine, which short_chunk spends only on rows long
// enough to be folded by the whole wave; chunks with at most one row
// boundary are the interior and the ends of long rows, where the step
// schedule's long runs fold whole windows.  Config 5 scatter (Zipf degrees:
// rows of 1-2 positions around hub rows) main kernel: sum / max / logsumexp
// 1.28 / 1.53 / 1.46 ms with the mean rule alone, 1.24 / 1.41 / 1.28 ms.
// Argument positions of NE consecutive features, written once: with `nt`
// (outputs larger than the last-level cache), pairs as 16-byte non-temporal
// stores where the address allows.  Config 5 scatter max (384 MB of values
// and arguments): 1.411 -> 1.360 ms; config 2 segment max (96 MB) is 3 %
// slower that way, and unchanged with plain 16-byte stores.
template <int NE>
__device__ __forceinline__ void store_args(int64_t* a, const int64_t* v, bool nt) {
  if constexpr (NE % 2 == 0) {
    if (nt && ((uintptr_t)a & 15) == 0) {
      typedef long long i64x2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int i = 0; i < NE; i += 2) {
        const i64x2 q = {(long long)v[i], (long long)v[i + 1]};
        __builtin_nontemporal_store(q, reinterpret_cast<i64x2*>(a + i));
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < NE; ++i) a[i] = v[i];
}

constexpr int64_t kWaveRowMin = 16;
// LDS words per wave staging short_chunk's finished rows (8 KiB; 32 KiB per
// block leaves room for the 16 resident waves per CU the engine targets)
constexpr int kStageWords = 2048;
__device__ __forceinline__ bool chunk_is_short(int64_t r0, int64_t r_end, int64_t lo, int64_t hi, int S) {
  return r_end - r0 >= 2 || (r_end - r0) * S >= hi - lo;
}

// Variants.  V_FIRST and V_LATER fix the common cases at compile time --
// messages x * w with at most one weight per position, no product
// reduction, NaN-ignoring extrema with the first (V_FIRST) or the last
// (V_LATER) tie winning -- which keeps the per-lane state small; V_GENERIC
// reads every rule from Params.
// V_FIRST32 is V_FIRST for a gathered operand below 4 GiB: row offsets are
// 32-bit byte offsets from a uniform base (one VGPR per address, one
// ds_bpermute per column).
enum { V_GENERIC = 0, V_FIRST = 1, V_LATER = 2, V_FIRST32 = 3 };

// Occupancy target per instance (waves per SIMD), enforced through the
// register budget: 4 (<= 128 VGPRs) for the fast variants, 3 for 16-bit
// min/max and log-sum-exp, whose 8 elements per lane need more state.
template <int DT, int RK, int VAR, int G, bool VL>
constexpr int engine_waves() {
  if constexpr (VAR == V_GENERIC) return 1;
  // one 16-byte row per lane: 8 staged positions per lane per window
  if constexpr (G == 1 && VL) return 3;
  return DT != OGN_F32 && RK != RK_SUM ? 3 : 4;
}

// Chunks of many row boundaries (contiguous mode, fast variants; see
// chunk_is_short), run by engine_kernel's wave for chunk c instead of the
// step schedule: the chunk's rows are dealt to the S sub-groups in turn, each
// sub-group folds its row's positions (four loads in flight) on its own --
// no cross-lane combine -- and finishes the row, or leaves the same head /
// tail record as the step schedule for a row that crosses the chunk's edge.
// Rows with more positions in the chunk than L are skipped there and folded
// afterwards by the whole wave, one at a time: sub-group s takes positions
// s, s + S, ... (eight loads in flight) and the S partials are merged in
// position order.  The extremum direction is a template parameter, and
// argument positions are int32 offsets from the chunk start.
template <int DT, int G, bool VL, int RK, int VAR, bool MIN, bool NTS>
__device__ __forceinline__ void short_chunk(const Params& p, int64_t c, int64_t lo, int64_t hi, int64_t r0,
                                            int64_t r_end, uint32_t* __restrict__ stage) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr int NE = VL ? E::VEC : 1;
  constexpr int S = kWave / G;
  constexpr int kU = 4;
  const int lane = lane_id();
  const int sub = lane / G;
  const int gl = lane % G;
  const int64_t b = blockIdx.z;
  const int64_t pb = p.ptr_bstride ? b : 0;
  const int64_t K = p.k;
  const int64_t M = p.m;
  const int64_t k0 = (int64_t)blockIdx.y * (G * NE) + gl * NE;
  const bool kok = VL || k0 < K;
  const int64_t kc = kok ? k0 : 0;  // a feature in range for the loads
  const int64_t* __restrict__ ptr = static_cast<const int64_t*>(p.ptr) + pb * p.ptr_bstride;
  const S_t* __restrict__ srcb = static_cast<const S_t*>(p.src) + b * p.src_bstride;
  // rows r0 .. r_end - 1 end inside the chunk; r_end (< m) may start inside it
  const int64_t r_last = std::min<int64_t>(r_end, M - 1);
  // Rows with more than L positions inside the chunk (L: twice the chunk's
  // mean row length, at least kWaveRowMin) are left to the whole wave
  // (below), so that one long row does not hold up the sub-groups that fold
  // the short rows dealt beside it.
  const int64_t L = std::max<int64_t>(kWaveRowMin, 2 * (hi - lo) / std::max<int64_t>(1, r_last - r0 + 1));
  // Finished rows are staged in LDS (p.short_rows == 2) and written kSlots
  // rows per sub-group at a time, usually once at the end of the chunk.  A
  // wave's loads and stores share one completion counter here, and with a
  // store outstanding the compiler can only wait for all of them: a store
  // after every row made the next row's loads wait for its write as well.
  constexpr bool kArgs = RK == RK_MINMAX;
  constexpr int kSlotWords = NE * (kArgs ? 2 : 1);
  constexpr int kSlots = std::min(32, kStageWords / (kWave * kSlotWords));
  const bool staged = p.short_rows == 2;
  int slot = 0;
  auto init = [&](float* acc, float* best, int32_t* barg) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      acc[i] = 0.f;
      // later tie: -+inf start, "nothing taken" while the arg is unset;
      // first tie: NaN start (no ordered compare with it holds)
      best[i] = RK == RK_LSE ? -__builtin_inff()
                             : (VAR == V_LATER ? (MIN ? __builtin_inff() : -__builtin_inff()) : __builtin_nanf(""));
      barg[i] = kNone32;
    }
  };
  auto fold = [&](const float* x, int32_t off, float* acc, float* best, int32_t* barg) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const float pv = x[i];
      if constexpr (RK == RK_MINMAX) {
        bool take;
        if constexpr (VAR == V_LATER) take = MIN ? pv <= best[i] : pv >= best[i];
        else take = !(MIN ? pv >= best[i] : pv <= best[i]) && pv == pv;
        best[i] = take ? pv : best[i];
        barg[i] = take ? off : barg[i];
      } else if constexpr (RK == RK_LSE) {
        lse_add(best[i], acc[i], pv);
      } else {
        acc[i] += pv;
      }
    }
  };
  // Write row r's result (whole row in the chunk) or its head / tail record.
  auto emit = [&](int64_t r, int64_t rs, int64_t re, const float* acc, const float* best, const int32_t* barg,
                  int sl) {
    if (re > hi || rs < lo) {
      // partial row: tail if it goes on past the chunk, else head (it began before)
      const bool head = re <= hi;
      const int64_t rb = (b * p.nchunks + c) * K + k0;
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        if constexpr (RK == RK_MINMAX) {
          static_cast<double*>(head ? p.rec_head : p.rec_tail)[rb + i] = (double)best[i];
          (head ? p.arg_head : p.arg_tail)[rb + i] = barg[i] == kNone32 ? kNone : lo + barg[i];
        } else if constexpr (RK == RK_LSE) {
          static_cast<float2*>(head ? p.rec_head : p.rec_tail)[rb + i] = make_float2(best[i], acc[i]);
        } else {
          static_cast<float*>(head ? p.rec_head : p.rec_tail)[rb + i] = acc[i];
        }
      }
    } else {
      const int64_t off = b * p.out_bstride + r * K + k0;
      float v[NE];
      int64_t ag[NE];
#pragma unroll
      for (int i = 0; i < NE; ++i)
        finish_elem<RK, float>(p, b, r, k0 + i, rs, re, acc[i], best[i], barg[i] == kNone32 ? kNone : lo + barg[i],
                               &v[i], &ag[i]);
      if (sl >= 0) {
        // staged: values, then (min / max) the argument as an offset from
        // the chunk start -- every argument of a row inside the chunk lies
        // in [lo, hi) or is the empty-row value, coded kNone32
        uint32_t* q = stage + (sl * kWave + lane) * kSlotWords;
#pragma unroll
        for (int i = 0; i < NE; ++i) q[i] = __float_as_uint(v[i]);
        if constexpr (kArgs) {
#pragma unroll
          for (int i = 0; i < NE; ++i) q[NE + i] = (uint32_t)(ag[i] == p.arg_empty ? kNone32 : (int32_t)(ag[i] - lo));
        }
        return;
      }
      store_floats<NE, true>(p.out, p.out_dt, off, v);
      if constexpr (RK == RK_MINMAX) {
        if (p.arg) {
#pragma unroll
          for (int i = 0; i < NE; ++i) p.arg[off + i] = ag[i];
        }
      }
    }
  };
  // Staged rows of this lane's sub-group: slot j holds row gbase + j * S.
  uint32_t pend = 0;
  int64_t gbase = r0 + sub;
  auto flush = [&]() {
    while (pend) {
      const int j = __builtin_ctz(pend);
      pend &= pend - 1;
      const int64_t off = b * p.out_bstride + (gbase + (int64_t)j * S) * K + k0;
      const uint32_t* q = stage + (j * kWave + lane) * kSlotWords;
      float v[NE];
#pragma unroll
      for (int i = 0; i < NE; ++i) v[i] = __uint_as_float(q[i]);
      store_floats<NE, true>(p.out, p.out_dt, off, v);
      if constexpr (kArgs) {
        if (p.arg) {
          int64_t ag[NE];
#pragma unroll
          for (int i = 0; i < NE; ++i) {
            const int32_t code = (int32_t)q[NE + i];
            ag[i] = code == kNone32 ? p.arg_empty : lo + code;
          }
          store_args<NE>(p.arg + off, ag, p.out_nt);
        }
      }
    }
  };
  for (int64_t r = r0 + sub; r <= r_last; r += S) {
    if (staged && slot == kSlots) {
      flush();
      gbase = r;
      slot = 0;
    }
    const int my = slot++;
    const int64_t rs = ptr[r], re = ptr[r + 1];
    if (r == r_end && rs >= hi) break;  // starts in the next chunk
    const int64_t a = std::max<int64_t>(rs, lo), z = std::min<int64_t>(std::min<int64_t>(re, hi), p.n);
    if (z - a > L) continue;  // the wave's
    float acc[NE], best[NE];
    int32_t barg[NE];
    init(acc, best, barg);
    for (int64_t e0 = a; e0 < z; e0 += kU) {
      float x[kU][NE];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        // conditional: most of these rows hold 1-2 positions, and loading
        // all four packets regardless was measured 15 % slower
        const bool ok = e0 + u < z;
        if constexpr (VL) {
          E::unpack(ok ? load16_once<NTS>(srcb + (e0 + u) * K + kc) : make_uint4(0u, 0u, 0u, 0u), x[u]);
        } else {
          x[u][0] = ok ? E::load1(srcb, (e0 + u) * K + kc) : 0.f;
        }
      }
      const int32_t off = (int32_t)(e0 - lo);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (e0 + u >= z) break;
        fold(x[u], off + u, acc, best, barg);
      }
    }
    if (!kok) continue;
    const bool whole = rs >= lo && re <= hi;
    emit(r, rs, re, acc, best, barg, staged && whole ? my : -1);
    if (staged && whole) pend |= 1u << my;
  }
  flush();
  // Long rows: sub-group s folds positions a + s, a + s + S, ... (kW steps
  // in flight), then the sub-group partials are merged in position order.
  constexpr int kW = 8;
  for (int64_t w = r0; w <= r_last; w += kWave) {
    bool lg = false;
    if (w + lane <= r_last) {
      const int64_t rr = w + lane;
      const int64_t rs = ptr[rr], re = ptr[rr + 1];
      const int64_t a = std::max<int64_t>(rs, lo), z = std::min<int64_t>(std::min<int64_t>(re, hi), p.n);
      lg = !(rr == r_end && rs >= hi) && z - a > L;
    }
    uint64_t mask = __ballot(lg);
    while (mask) {
      const int j = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int64_t r = w + j;
      const int64_t rs = ptr[r], re = ptr[r + 1];
      const int64_t a = std::max<int64_t>(rs, lo), z = std::min<int64_t>(std::min<int64_t>(re, hi), p.n);
      float acc[NE], best[NE];
      int32_t barg[NE];
      init(acc, best, barg);
      int64_t e0 = a;
      for (; e0 + kW * S <= z; e0 += kW * S) {
        float x[kW][NE];
#pragma unroll
        for (int u = 0; u < kW; ++u) {
          if constexpr (VL) E::unpack(load16_once<NTS>(srcb + (e0 + sub + u * S) * K + kc), x[u]);
          else x[u][0] = E::load1(srcb, (e0 + sub + u * S) * K + kc);
        }
#pragma unroll
        for (int u = 0; u < kW; ++u) fold(x[u], (int32_t)(e0 + sub + u * S - lo), acc, best, barg);
      }
      {
        float x[kW][NE];
#pragma unroll
        for (int u = 0; u < kW; ++u) {
          const bool ok = e0 + sub + u * S < z;
          if constexpr (VL) {
            E::unpack(ok ? load16_once<NTS>(srcb + (e0 + sub + u * S) * K + kc) : make_uint4(0u, 0u, 0u, 0u), x[u]);
          } else {
            x[u][0] = ok ? E::load1(srcb, (e0 + sub + u * S) * K + kc) : 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < kW; ++u)
          if (e0 + sub + u * S < z) fold(x[u], (int32_t)(e0 + sub + u * S - lo), acc, best, barg);
      }
      // butterfly over sub-groups; lower sub-groups hold earlier positions
      auto round = [&](auto offc) {
        constexpr int off = decltype(offc)::value;
        const bool upper = (lane & off) != 0;
#pragma unroll
        for (int i = 0; i < NE; ++i) {
          if constexpr (RK == RK_MINMAX) {
            const float ob = xor_shfl<off>(best[i]);
            const int32_t oa = xor_shfl<off>(barg[i]);
            const bool tie = VAR == V_LATER ? oa > barg[i] : oa < barg[i];
            const bool take = oa != kNone32 && (barg[i] == kNone32 || (MIN ? ob < best[i] : ob > best[i]) ||
                                                (ob == best[i] && tie));
            best[i] = take ? ob : best[i];
            barg[i] = take ? oa : barg[i];
          } else if constexpr (RK == RK_LSE) {
            const float om = xor_shfl<off>(best[i]);
            const float os = xor_shfl<off>(acc[i]);
            float m1 = upper ? om : best[i], s1 = upper ? os : acc[i];
            const float m2 = upper ? best[i] : om, s2 = upper ? acc[i] : os;
            lse_merge(m1, s1, m2, s2);
            best[i] = m1;
            acc[i] = s1;
          } else {
            const float o = xor_shfl<off>(acc[i]);
            acc[i] = upper ? o + acc[i] : acc[i] + o;
          }
        }
      };
      if constexpr (G <= 1) round(std::integral_constant<int, 1>{});
      if constexpr (G <= 2) round(std::integral_constant<int, 2>{});
      if constexpr (G <= 4) round(std::integral_constant<int, 4>{});
      if constexpr (G <= 8) round(std::integral_constant<int, 8>{});
      if constexpr (G <= 16) round(std::integral_constant<int, 16>{});
      if constexpr (G <= 32) round(std::integral_constant<int, 32>{});
      if (sub == 0 && kok) emit(r, rs, re, acc, best, barg, -1);
    }
  }
}

// NTS: the contiguous source is read with non-temporal loads (chosen per call
// by its size, see run()).
template <int DT, typename IDX, int G, bool VL, int RK, bool GATHER, int VAR, bool NTS = false>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(engine_waves<DT, RK, VAR, G, VL>())))
void engine_kernel(Params p) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr bool FAST = VAR != V_GENERIC;
  constexpr bool OFF32 = VAR == V_FIRST32;
  static_assert(!OFF32 || (VL && GATHER), "32-bit offsets are for vector gathers");
  constexpr int NE = VL ? E::VEC : 1;
  constexpr int S = kWave / G;
  // Steps in flight per wave: fewer for the wider min/max and log-sum-exp state.
  constexpr int kUnroll = RK == RK_SUM ? (DT == OGN_F32 ? kUnrollSum32 : kUnrollSum) : kUnrollWide;
  // min/max of weighted fp32 messages compare exact fp64 products (fp16/bf16
  // products are exact in fp32); contiguous mode and the later-tie gather
  // variant (scatter through a permutation) have no weights, so their fp32
  // comparisons are exact as they are.
  using MT = std::conditional_t<RK == RK_MINMAX && DT == OGN_F32 && GATHER && VAR != V_LATER, double, float>;

  const int lane = lane_id();
  const int sub = lane / G;
  const int gl = lane % G;
  const int64_t c = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (c >= p.nchunks) return;
  const int64_t b = blockIdx.z;
  const int64_t pb = p.ptr_bstride ? b : 0;
  const int64_t K = p.k;
  const int64_t M = p.m;
  const int64_t k0 = (int64_t)blockIdx.y * (G * NE) + gl * NE;
  const bool kok = VL || k0 < K;
  const IDX* __restrict__ ptr = static_cast<const IDX*>(p.ptr) + pb * p.ptr_bstride;
  const IDX* __restrict__ col = static_cast<const IDX*>(p.col);
  const S_t* __restrict__ srcb = static_cast<const S_t*>(p.src) + b * p.src_bstride;
  const S_t* __restrict__ val = static_cast<const S_t*>(p.val);
  const bool is_min = p.reduce == OGN_REDUCE_MIN;
  const bool is_prod = !FAST && p.reduce == OGN_REDUCE_PROD;
  const bool later = VAR == V_LATER || (VAR == V_GENERIC && p.mm_mode == MM_LATER);
  const bool nanprop = !FAST && p.mm_mode == MM_NANPROP;
  const int vop = FAST ? (int)OP_MUL : p.val_op;
  const int val_mode = FAST ? std::min(p.val_mode, 1) : p.val_mode;
  constexpr int NW = (VL && !FAST) ? NE : 1;  // weights held per step

  const int64_t base = ptr[0];
  const int64_t end = std::max<int64_t>(std::min<int64_t>((int64_t)ptr[M] - base, p.nnz_bound), 0);
  const int64_t nce = std::max<int64_t>(1, (end + p.chunk - 1) / p.chunk);
  if (c >= nce) return;
  const int64_t lo = base + c * p.chunk;
  const int64_t hi = base + std::min<int64_t>((c + 1) * p.chunk, end);
  int64_t r = c == 0 ? 0 : std::min<int64_t>(std::max<int64_t>(p.chunk_row[pb * p.nchunks + c], 0), M - 1);
  if constexpr (!GATHER && FAST) {
    if (p.short_rows) {
      __shared__ uint32_t stage[kWavesPerBlock * kStageWords];
      uint32_t* ws = stage + wave_in_block() * kStageWords;
      const int64_t r_end = chunk_row_end(p, pb, c, nce);
      if (chunk_is_short(r, r_end, lo, hi, S)) {
        if (RK == RK_MINMAX && is_min) short_chunk<DT, G, VL, RK, VAR, true, NTS>(p, c, lo, hi, r, r_end, ws);
        else short_chunk<DT, G, VL, RK, VAR, false, NTS>(p, c, lo, hi, r, r_end, ws);
        return;
      }
    }
  }

  // Pointer window: lane j holds ptr[wb + 1 + j].
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

  // int8 sums accumulate exactly in int32 (torch_sparse int8 -> int32)
  constexpr bool IS_INT = DT == OGN_I8;
  using AT = std::conditional_t<IS_INT, int32_t, float>;
  AT acc[NE];
  MT best[NE];
  // Extremum positions are held as int32 offsets from the chunk start (a
  // chunk is at most 8192 positions); kNone32 marks "nothing taken".
  int32_t barg[NE];
  // Fast variants keep extrema in "max space": a min reduction folds -x with
  // the max rules (flipv negates under a uniform mask, one VALU, no
  // per-element choice between two compares), and values are flipped back
  // where they leave the wave (records, finishing).  Negation is exact, so
  // values, ties and signed zeros come back unchanged.
  constexpr bool MAXSPACE = FAST && RK == RK_MINMAX;
  const bool flip_mm = MAXSPACE && is_min;
  auto flipv = [&](MT v) -> MT {
    if constexpr (!MAXSPACE) {
      return v;
    } else if constexpr (std::is_same<MT, double>::value) {
      const uint64_t u = (uint64_t)__double_as_longlong(v) ^ (flip_mm ? 0x8000000000000000ull : 0ull);
      return __longlong_as_double((long long)u);
    } else {
      return __uint_as_float(__float_as_uint(v) ^ (flip_mm ? 0x80000000u : 0u));
    }
  };
  const bool mm_min = MAXSPACE ? false : is_min;  // direction of the compares below
  auto reset = [&]() {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      acc[i] = is_prod ? (AT)1 : (AT)0;
      // min/max start from NaN, "nothing taken yet": every ordered compare
      // with it is false, so the first non-NaN message is taken without a
      // separate test (barg stays kNone32 until then).  The later-tie fast
      // variant starts from -inf instead (max space): taking on >= then
      // needs one compare, and -inf with no arg is "nothing taken" to every
      // rule that reads the state.
      best[i] = RK == RK_LSE ? (MT)-__builtin_inff()
                             : (VAR == V_LATER ? (MT)-__builtin_inff() : (MT)__builtin_nan(""));
      barg[i] = kNone32;
    }
  };
  reset();

  // One butterfly round over sub-groups OFF apart (OFF a compile-time lane
  // distance, see xor_shfl).
  auto combine_round = [&](auto offc) {
    constexpr int off = decltype(offc)::value;
    const bool upper = (lane & off) != 0;  // partner holds earlier positions
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      if constexpr (RK == RK_MINMAX) {
        const MT ob = xor_shfl<off>(best[i]);
        const int32_t oa = xor_shfl<off>(barg[i]);
        bool take;
        if (nanprop) {
          // a NaN beats any number; between two NaNs, or equal numbers, the
          // earlier position wins, so every lane ends with the same arg
          const bool mine_nan = best[i] != best[i], their_nan = ob != ob;
          take = oa != kNone32 &&
                 (barg[i] == kNone32 ||
                  (their_nan ? (!mine_nan || oa < barg[i])
                             : (!mine_nan && (better(ob, best[i], mm_min) || (ob == best[i] && oa < barg[i])))));
        } else if (later) {
          take = oa != kNone32 && (barg[i] == kNone32 || better(ob, best[i], mm_min) ||
                                   (ob == best[i] && oa > barg[i]));
        } else {
          take = oa != kNone32 && (barg[i] == kNone32 || better(ob, best[i], mm_min) ||
                                   (ob == best[i] && oa < barg[i]));
        }
        best[i] = take ? ob : best[i];
        barg[i] = take ? oa : barg[i];
      } else if constexpr (RK == RK_LSE) {
        const float om = xor_shfl<off>((float)best[i]);
        const float os = xor_shfl<off>(acc[i]);
        // merge in position order so every lane computes the same value
        float m1 = upper ? om : (float)best[i], s1 = upper ? os : acc[i];
        const float m2 = upper ? (float)best[i] : om, s2 = upper ? acc[i] : os;
        lse_merge(m1, s1, m2, s2);
        best[i] = m1;
        acc[i] = s1;
      } else {
        const AT o = xor_shfl<off>(acc[i]);
        const AT lo_v = upper ? o : acc[i], hi_v = upper ? acc[i] : o;
        acc[i] = is_prod ? lo_v * hi_v : lo_v + hi_v;
      }
    }
  };
  // Combine the S sub-group partials of the current row; all lanes end with
  // the combined state.  Lower sub-groups hold earlier positions.
  auto combine = [&]() {
    if constexpr (G <= 1) combine_round(std::integral_constant<int, 1>{});
    if constexpr (G <= 2) combine_round(std::integral_constant<int, 2>{});
    if constexpr (G <= 4) combine_round(std::integral_constant<int, 4>{});
    if constexpr (G <= 8) combine_round(std::integral_constant<int, 8>{});
    if constexpr (G <= 16) combine_round(std::integral_constant<int, 16>{});
    if constexpr (G <= 32) combine_round(std::integral_constant<int, 32>{});
  };

  auto write_record = [&](bool head) {
    if (sub != 0 || !kok) return;
    const int64_t rb = (b * p.nchunks + c) * K + k0;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      if (!VL && k0 + i >= K) break;
      if constexpr (RK == RK_MINMAX) {
        static_cast<double*>(head ? p.rec_head : p.rec_tail)[rb + i] = (double)flipv(best[i]);
        (head ? p.arg_head : p.arg_tail)[rb + i] = barg[i] == kNone32 ? kNone : lo + barg[i];
      } else if constexpr (RK == RK_LSE) {
        static_cast<float2*>(head ? p.rec_head : p.rec_tail)[rb + i] = make_float2((float)best[i], (float)acc[i]);
      } else {
        static_cast<AT*>(head ? p.rec_head : p.rec_tail)[rb + i] = acc[i];
      }
    }
  };

  // Gather-mode fp32 sums hold a finished row's result in registers and store it
  // just after the next batch of gathers is issued: loads and stores share
  // one completion counter, and a store issued before the gathers made their
  // wait include its write acknowledgement.
  constexpr bool DEFER = GATHER && FAST && VL && RK == RK_SUM && DT == OGN_F32;
  float pv_out[DEFER ? NE : 1];
  int64_t pv_off = -1;  // -1: nothing pending
  auto store_pending = [&]() {
    if constexpr (DEFER) {
      if (pv_off >= 0) {
        store_floats<NE, true>(p.out, p.out_dt, pv_off, pv_out);
        pv_off = -1;
      }
    }
  };

  auto flush = [&]() {
    combine();
    if (head_split && first) {
      write_record(true);
    } else if (sub == 0 && kok) {
      float v[NE];
      int64_t ag[NE];
      const int64_t off = b * p.out_bstride + r * K + k0;
      if constexpr (DEFER) {
#pragma unroll
        for (int i = 0; i < NE; ++i)
          finish_elem<RK, MT>(p, b, r, k0 + i, rs, re, (float)acc[i], flipv(best[i]), kNone, &v[i], &ag[i]);
        store_pending();
#pragma unroll
        for (int i = 0; i < NE; ++i) pv_out[i] = v[i];
        pv_off = off;
        first = false;
        reset();
        return;
      }
      if constexpr (IS_INT && RK == RK_SUM) {
#pragma unroll
        for (int i = 0; i < NE; ++i) {
          if (!VL && k0 + i >= K) break;
          finish_int(p, off + i, acc[i], re - rs);
        }
      } else {
#pragma unroll
        for (int i = 0; i < NE; ++i)
          finish_elem<RK, MT>(p, b, r, k0 + i, rs, re, (float)acc[i], flipv(best[i]),
                              barg[i] == kNone32 ? kNone : lo + barg[i], &v[i], &ag[i]);
        if (VL || k0 + NE <= K) {
          store_floats<NE, true>(p.out, p.out_dt, off, v);
        }
      }
      if constexpr (RK == RK_MINMAX) {
        if (p.arg) {
#pragma unroll
          for (int i = 0; i < NE; ++i) p.arg[off + i] = ag[i];
        }
      }
    }
    first = false;
    reset();
  };

  // Column indices and weights of the next 64-position window are loaded
  // one window ahead, so a window's gathers never wait for its staging load.
  // A window is the run of positions whose col / value are staged together:
  // 64 positions (one per lane) when a step covers fewer than 64 positions,
  // and kUnroll x 64 when one step already covers 64 (S == 64: one lane per
  // feature row or one feature), so that kUnroll steps can still be in
  // flight; each lane then stages its own position of every step.
  constexpr int WSTEPS = S == kWave ? kUnroll : 1;
  constexpr int64_t WPOS = (int64_t)kWave * WSTEPS;
  int64_t cl_next[WSTEPS];
  float vl_next[WSTEPS];
  auto stage = [&](int64_t wb2) {
#pragma unroll
    for (int t = 0; t < WSTEPS; ++t) {
      const int64_t el = wb2 + t * kWave + lane;
      const bool ev = el < hi;
      if constexpr (GATHER) cl_next[t] = ev ? (int64_t)load_stream(col + el) : 0;
      vl_next[t] = 1.f;
      if (val_mode == 1) vl_next[t] = ev ? E::load1(val, el) : 0.f;
    }
  };
  // Long runs (contiguous mode, fast variants, no weights): windows lying
  // wholly inside the current row -- the bulk of a hub row -- are folded
  // with no per-step row-end or chunk-end test.  Lane positions and the fold
  // order per lane are those of the step schedule, so sums and extrema are
  // the same bits; loads step through src at a uniform stride, FU steps in
  // flight.  Extrema take 3 VALU per element with the later-tie rule (the
  // "nothing taken" NaN start becomes -+inf, which every rule treats alike
  // while the arg is unset); log-sum-exp takes the batch maximum first and
  // rescales once per batch, one exponential per element.
  auto long_run = [&](auto minc, int64_t w0, int64_t nwin) {
    constexpr bool MIN = decltype(minc)::value;
    constexpr int NSW = kWave / S;           // steps per window
    constexpr int FU = NSW < 8 ? NSW : 8;    // steps per batch
    const int64_t stride = (int64_t)S * K;   // elements between steps
    const S_t* q = srcb + (w0 + sub) * K + k0;
    int32_t off = (int32_t)(w0 - lo) + sub;  // this lane's position in the chunk
    if constexpr (RK == RK_MINMAX) {
      // the state is kept in max space; fold in the real direction here
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        best[i] = flipv(best[i]);
        if constexpr (VAR == V_LATER)
          if (best[i] != best[i]) best[i] = MIN ? (MT)__builtin_inff() : (MT)-__builtin_inff();
      }
    }
    const int64_t nb = nwin * (NSW / FU);
    for (int64_t bi = 0; bi < nb; ++bi) {
      uint4 xr[FU];
#pragma unroll
      for (int u = 0; u < FU; ++u) xr[u] = load16_once<NTS>(q + u * stride);
      q += FU * stride;
      float x[FU][NE];
#pragma unroll
      for (int u = 0; u < FU; ++u) E::unpack(xr[u], x[u]);
      if constexpr (RK == RK_SUM) {
#pragma unroll
        for (int u = 0; u < FU; ++u)
#pragma unroll
          for (int i = 0; i < NE; ++i) acc[i] = __builtin_fmaf(x[u][i], 1.f, acc[i]);
      } else if constexpr (RK == RK_MINMAX) {
#pragma unroll
        for (int u = 0; u < FU; ++u) {
          const int32_t pos = off + u * S;
#pragma unroll
          for (int i = 0; i < NE; ++i) {
            const MT pv = (MT)x[u][i];
            bool take;
            if constexpr (VAR == V_LATER) take = MIN ? pv <= best[i] : pv >= best[i];
            else take = !(MIN ? pv >= best[i] : pv <= best[i]) && pv == pv;
            best[i] = take ? pv : best[i];
            barg[i] = take ? pos : barg[i];
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < NE; ++i) {
          float mx = x[0][i];
#pragma unroll
          for (int u = 1; u < FU; ++u) mx = fmaxf(mx, x[u][i]);
          const float m = (float)best[i];
          const float nm = fmaxf(m, mx);
          const float cn = clampf_max(nm);
          float t = 0.f;
#pragma unroll
          for (int u = 0; u < FU; ++u) t += fast_exp(x[u][i] - cn);
          acc[i] = __builtin_fmaf(acc[i], fast_exp(clampf_max(m) - cn), t);
          best[i] = nm;
        }
      }
      off += FU * S;
    }
    if constexpr (RK == RK_MINMAX) {
#pragma unroll
      for (int i = 0; i < NE; ++i) best[i] = flipv(best[i]);
    }
  };

  stage(lo);
  for (int64_t wbase = lo; wbase < hi; wbase += WPOS) {
    if constexpr (!GATHER && FAST && VL && WSTEPS == 1 && !IS_INT) {
      if (val_mode == 0 && r < M) {
        const int64_t stop = std::min<int64_t>(std::min<int64_t>(re, hi), p.n);
        const int64_t nwin = (stop - wbase) / WPOS;
        if (nwin > 0) {
          if constexpr (RK == RK_MINMAX) {
            if (is_min) long_run(std::true_type{}, wbase, nwin);
            else long_run(std::false_type{}, wbase, nwin);
          } else {
            long_run(std::false_type{}, wbase, nwin);
          }
          wbase += nwin * WPOS;
          if (wbase >= hi) break;
        }
      }
    }
    // One-step windows copy the staged col / value out and restage at once;
    // multi-step windows read the staged arrays in phase 1 and restage after
    // the gathers are issued (no second copy of the arrays).
    int64_t cl = 0;
    float vl = 1.f;
    if constexpr (WSTEPS == 1) {
      if constexpr (GATHER) {
        cl = cl_next[0];
      } else {
        cl = wbase + lane;
      }
      cl = std::min<int64_t>(std::max<int64_t>(cl, 0), p.n - 1);
      vl = vl_next[0];
      if (wbase + WPOS < hi) stage(wbase + WPOS);
    }
    const int nw = (int)std::min<int64_t>(WPOS, hi - wbase);
    const int nsteps = (nw + S - 1) / S;
    for (int j0 = 0; j0 < nsteps; j0 += kUnroll) {
      // Raw 16-byte loads are kept as issued and unpacked when consumed, so
      // 16-bit features occupy half the registers and no load is waited for
      // before the last one has been issued.
      uint4 xr[kUnroll];
      float xs[kUnroll];
      float w[kUnroll][NW];
      // Phase 1: every lane shuffle of the U steps (positions and weights).
      // Doing them before any gather is issued keeps the wait for the staged
      // col/value loads ahead of the gathers, so the U gathers overlap.
      int64_t cc[kUnroll];
      uint32_t co[kUnroll];  // OFF32: byte offset of the gathered packet
      float ws[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int idx = (j0 + u) * S + sub;
        if constexpr (WSTEPS > 1) {
          // S == 64: step u is this lane's own staged position u
          int64_t c1;
          if constexpr (GATHER) {
            c1 = cl_next[u];
          } else {
            c1 = wbase + u * kWave + lane;
          }
          c1 = std::min<int64_t>(std::max<int64_t>(c1, 0), p.n - 1);
          if constexpr (GATHER && OFF32) {
            co[u] = (uint32_t)c1 * (uint32_t)(K * sizeof(S_t)) + (uint32_t)(k0 * sizeof(S_t));
          } else {
            cc[u] = c1;
          }
          ws[u] = vl_next[u];
        } else {
          if constexpr (GATHER) {
            if constexpr (OFF32) {
              co[u] = (uint32_t)shfl32((int32_t)cl, idx & (kWave - 1)) * (uint32_t)(K * sizeof(S_t)) +
                      (uint32_t)(k0 * sizeof(S_t));
            } else {
              cc[u] = (int64_t)shfl64((IDX)cl, idx & (kWave - 1));
            }
          } else {
            cc[u] = std::min<int64_t>(wbase + idx, p.n - 1);
          }
          ws[u] = shflf(vl, idx & (kWave - 1));
        }
      }
      // Phase 2: issue the U gathers back to back.
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int idx = (j0 + u) * S + sub;
        const bool ok = (j0 + u) < nsteps && idx < nw && kok;
        if constexpr (VL) {
          if constexpr (OFF32) {
            xr[u] = ok ? load16(reinterpret_cast<const char*>(srcb) + co[u]) : make_uint4(0u, 0u, 0u, 0u);
          } else {
            xr[u] = ok ? load16_once<!GATHER && NTS>(srcb + cc[u] * K + k0) : make_uint4(0u, 0u, 0u, 0u);
          }
#pragma unroll
          for (int i = 0; i < NW; ++i) w[u][i] = ws[u];
          if constexpr (NW > 1) {
            if (val_mode == 2 && ok) {
              float wv[NE];
              E::unpack(load16(val + (wbase + idx) * K + k0), wv);
#pragma unroll
              for (int i = 0; i < NE; ++i) w[u][i] = wv[i];
            }
          }
        } else {
          xs[u] = ok ? E::load1(srcb, cc[u] * K + k0) : 0.f;
          w[u][0] = ws[u];
          if (val_mode == 2 && ok) w[u][0] = E::load1(val, (wbase + idx) * K + k0);
        }
      }
      if constexpr (WSTEPS > 1) {
        if (wbase + WPOS < hi) stage(wbase + WPOS);  // every step of this window is issued
      }
      store_pending();
      // Phase 3: consume the steps in order (fully unrolled, so the staged
      // steps stay in registers).
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (j0 + u >= nsteps) break;
        const int64_t e_first = wbase + (int64_t)(j0 + u) * S;
        const int64_t last = std::min<int64_t>(e_first + S, hi) - 1;
        const int64_t e_mine = e_first + sub;
        const bool valid = e_mine < hi;
        float x[NE];
        if constexpr (VL) E::unpack(xr[u], x);
        else x[0] = xs[u];
        float wcur[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) wcur[i] = w[u][i];
        bool added = false;
        while (true) {
          if (!added && valid && e_mine < re) {
#pragma unroll
            for (int i = 0; i < NE; ++i) {
              const float wi = wcur[NW > 1 ? i : 0];
              if constexpr (RK == RK_MINMAX) {
                // selects, not branches: lanes disagree on `take` all the time
                const MT pv = flipv(apply_op<MT>((MT)x[i], (MT)wi, vop));
                const bool isnan_pv = pv != pv;
                bool take;
                if constexpr (FAST) {
                  // max space, NaN-ignoring: later tie takes on >= from the
                  // -inf start; first tie on >, where the NaN start takes
                  // any number
                  if constexpr (VAR == V_LATER) take = pv >= best[i];
                  else take = !(pv <= best[i]) && !isnan_pv;
                } else {
                  // NaN-propagating: the first NaN is kept (its position is the arg)
                  take = nanprop ? (barg[i] == kNone32 || (isnan_pv && best[i] == best[i]) ||
                                    better(pv, best[i], is_min))
                                 : (!isnan_pv && (barg[i] == kNone32 || better(pv, best[i], is_min) ||
                                                  (later && pv == best[i])));
                }
                best[i] = take ? pv : best[i];
                barg[i] = take ? (int32_t)(e_mine - lo) : barg[i];
              } else if constexpr (RK == RK_LSE) {
                float m = (float)best[i];
                lse_add(m, acc[i], apply_op<float>(x[i], wi, vop));
                best[i] = m;
              } else if constexpr (IS_INT) {
                acc[i] += (int32_t)(x[i] * wi);  // exact: |x w| <= 2^14
              } else {
                if (vop == OP_MUL)
                  acc[i] = is_prod ? acc[i] * (x[i] * wi) : __builtin_fmaf(x[i], wi, acc[i]);
                else
                  acc[i] = is_prod ? acc[i] * apply_op<float>(x[i], wi, vop)
                                   : acc[i] + apply_op<float>(x[i], wi, vop);
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
  store_pending();
}

// Finish rows that cross chunk boundaries: one wave per chunk that holds the
// first piece of such a row.  With K > 32 every lane takes a feature and
// folds the row's records in chunk order (8 loads in flight).  With K <= 32
// the wave's lanes split into NG = 64 / KW lane groups (KW = K rounded up to
// a power of two); group g folds
// the row's records c + 1 + g, c + 1 + g + NG, ... (8 loads in flight), and
// the group partials are merged in a butterfly -- so a hub row spread over
// hundreds of chunks is folded by every lane of the wave, not only by the K
// lanes of its features.  Merges of min/max partials compare (value,
// position), so the tie rules hold whatever the fold order.
// INT: int32 sum records (int8 SpMM), finished by finish_int.
// Long rows: a row whose records span more than kLongSpan chunks has the
// tail records of its interior chunks (c1, c2) pre-folded in runs that end at
// multiples of kPiece -- one run per aligned group of kPiece chunks -- into
// each run's first record, so the fix-up folds about span / kPiece records
// instead of span (a hub row of config 5 spans ~2000 chunks).
constexpr int64_t kLongSpan = 64;
constexpr int64_t kPiece = 32;

struct RowRecords {
  int64_t c1, c2, first, count;  // first: the first run start past c1 + 1
  bool lng;
  // chunk of record t (1 <= t <= count); record count is the head in c2
  __device__ __forceinline__ int64_t chunk(int64_t t) const {
    if (!lng) return c1 + t;
    if (t >= count) return c2;
    return t == 1 ? c1 + 1 : first + (t - 2) * kPiece;
  }
};

__device__ __forceinline__ RowRecords row_records(int64_t c1, int64_t c2) {
  RowRecords rr;
  rr.c1 = c1;
  rr.c2 = c2;
  rr.lng = c2 - c1 > kLongSpan;
  rr.first = (c1 + 1) / kPiece * kPiece + kPiece;
  const int64_t mids = rr.lng && rr.first <= c2 - 1 ? (c2 - 1 - rr.first) / kPiece + 1 : 0;
  rr.count = rr.lng ? mids + 2 : c2 - c1;
  return rr;
}

template <typename MT>
__device__ __forceinline__ void mm_merge(MT& best, int64_t& barg, MT ob, int64_t oa, bool is_min, bool later,
                                         bool nanprop) {
  if (oa == kNone) return;
  bool take;
  if (barg == kNone) {
    take = true;
  } else if (nanprop && (best != best || ob != ob)) {
    // the earliest NaN wins (nothing replaces a NaN in position order)
    take = (ob != ob) && (!(best != best) || oa < barg);
  } else if (better(ob, best, is_min)) {
    take = true;
  } else if (ob == best) {
    take = later ? oa > barg : oa < barg;
  } else {
    take = false;
  }
  if (take) {
    best = ob;
    barg = oa;
  }
}

// Pre-fold of long rows (see kLongSpan): one wave per aligned group of
// kPiece chunks.  Lane l looks at chunk ca + l: it is interior to a long row
// when the row of its first position started in an earlier chunk c1, ends in
// a later chunk c2, and c2 - c1 > kLongSpan (the fix-up's test, from the
// same pointers).  A run starts at max(ca, c1 + 1) and ends at
// min(ca + kPiece - 1, c2 - 1); its tail records are folded in chunk order
// (lane groups over records, then a butterfly) into its first record.
template <typename IDX, int RK, bool F32MM, bool INT = false>
__global__ __launch_bounds__(kBlock) void prefold_kernel(Params p) {
  using MT = std::conditional_t<F32MM, double, float>;
  using AT = std::conditional_t<INT, int32_t, float>;
  const int lane = lane_id();
  const int64_t ca = ((int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * kPiece;
  const int64_t b = blockIdx.z;
  const int64_t pb = p.ptr_bstride ? b : 0;
  const IDX* __restrict__ ptr = static_cast<const IDX*>(p.ptr) + pb * p.ptr_bstride;
  const int64_t base = ptr[0];
  const int64_t end = std::max<int64_t>(std::min<int64_t>((int64_t)ptr[p.m] - base, p.nnz_bound), 0);
  const int64_t nce = std::max<int64_t>(1, (end + p.chunk - 1) / p.chunk);
  if (ca >= nce) return;
  const int64_t c = ca + lane;
  bool start = false;
  int64_t c2 = 0;
  if (lane < kPiece && c >= 1 && c < nce) {
    const int64_t r = std::min<int64_t>(std::max<int64_t>(p.chunk_row[pb * p.nchunks + c], 0), p.m - 1);
    const int64_t rs = ptr[r], re = ptr[r + 1];
    const int64_t c1 = (rs - base) / p.chunk;
    c2 = std::min<int64_t>((re - 1 - base) / p.chunk, nce - 1);
    start = c > c1 && c < c2 && c2 - c1 > kLongSpan && (c == ca || c == c1 + 1);
  }
  uint64_t starts = __ballot(start);
  if (!starts) return;
  const int64_t K = p.k;
  const bool is_min = p.reduce == OGN_REDUCE_MIN;
  const bool is_prod = p.reduce == OGN_REDUCE_PROD;
  const bool later = p.mm_mode == MM_LATER;
  const bool nanprop = p.mm_mode == MM_NANPROP;
  int kw = 1;
  while (kw < K && kw < kWave) kw <<= 1;
  const int ng = kWave / kw;
  const int g = lane / kw;
  while (starts) {
    const int sl = __builtin_ctzll(starts);
    starts &= starts - 1;
    const int64_t cs = ca + sl;
    const int64_t ce = std::min<int64_t>(ca + kPiece - 1, (int64_t)readlane64(c2, sl) - 1);
    if (ce <= cs) continue;
    for (int64_t k = lane % kw; k < K; k += kw) {
      const int64_t base_rec = (b * p.nchunks) * K + k;
      AT a = is_prod ? (AT)1 : (AT)0;
      MT best = RK == RK_LSE ? (MT)-__builtin_inff() : (MT)0;
      int64_t barg = kNone;
      constexpr int B = 8;
      for (int64_t c0 = cs + g; c0 <= ce; c0 += (int64_t)B * ng) {
        AT va[B];
        float vb[B];
        double vd[B];
        int64_t vg[B];
#pragma unroll
        for (int j = 0; j < B; ++j) {
          const int64_t cc = c0 + (int64_t)j * ng;
          const bool ok = cc <= ce;
          const int64_t ri = base_rec + std::min<int64_t>(cc, ce) * K;
          if constexpr (RK == RK_MINMAX) {
            vd[j] = ok ? static_cast<const double*>(p.rec_tail)[ri] : 0.0;
            vg[j] = ok ? p.arg_tail[ri] : kNone;
          } else if constexpr (RK == RK_LSE) {
            const float2 t = ok ? static_cast<const float2*>(p.rec_tail)[ri] : make_float2(-__builtin_inff(), 0.f);
            va[j] = t.x;
            vb[j] = t.y;
          } else {
            va[j] = ok ? static_cast<const AT*>(p.rec_tail)[ri] : (is_prod ? (AT)1 : (AT)0);
          }
        }
#pragma unroll
        for (int j = 0; j < B; ++j) {
          if constexpr (RK == RK_MINMAX) {
            mm_merge<MT>(best, barg, (MT)vd[j], vg[j], is_min, later, nanprop);
          } else if constexpr (RK == RK_LSE) {
            float m = (float)best;
            float sa = (float)a;
            lse_merge(m, sa, (float)va[j], vb[j]);
            best = m;
            a = (AT)sa;
          } else {
            a = is_prod ? a * va[j] : a + va[j];
          }
        }
      }
      for (int d = kw; d < kWave; d <<= 1) {
        if constexpr (RK == RK_MINMAX) {
          const MT ob = (MT)__shfl_xor((double)best, d);
          const int64_t oa = __shfl_xor(barg, d);
          mm_merge<MT>(best, barg, ob, oa, is_min, later, nanprop);
        } else if constexpr (RK == RK_LSE) {
          const float om = __shfl_xor((float)best, d), os = __shfl_xor((float)a, d);
          float m = (float)best;
          float sa = (float)a;
          lse_merge(m, sa, om, os);
          best = m;
          a = (AT)sa;
        } else {
          const AT o = __shfl_xor(a, d);
          a = is_prod ? a * o : a + o;
        }
      }
      if (g != 0) continue;
      const int64_t wi = base_rec + cs * K;
      if constexpr (RK == RK_MINMAX) {
        static_cast<double*>(p.rec_tail)[wi] = (double)best;
        p.arg_tail[wi] = barg;
      } else if constexpr (RK == RK_LSE) {
        static_cast<float2*>(p.rec_tail)[wi] = make_float2((float)best, (float)a);
      } else {
        static_cast<AT*>(p.rec_tail)[wi] = a;
      }
    }
  }
}

template <typename IDX, int RK, bool F32MM, bool INT = false>
__global__ __launch_bounds__(kBlock) void fixup_kernel(Params p) {
  using MT = std::conditional_t<F32MM, double, float>;
  using AT = std::conditional_t<INT, int32_t, float>;
  const int lane = lane_id();
  const int64_t c = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  const int64_t b = blockIdx.z;
  const int64_t pb = p.ptr_bstride ? b : 0;
  const IDX* __restrict__ ptr = static_cast<const IDX*>(p.ptr) + pb * p.ptr_bstride;
  // The row that starts inside chunk c and ends past it, from the chunk-row
  // pass (one load instead of chunk_row -> ptr[r] -> ptr[r + 1]).  Loaded
  // together with ptr[0] and ptr[m] (the index is clamped into the array;
  // entries at or past the last chunk are never used).
  const longlong4 fx = p.fix[pb * p.nchunks + std::min<int64_t>(c, p.nchunks - 1)];
  const int64_t base = ptr[0];
  const int64_t end = std::max<int64_t>(std::min<int64_t>((int64_t)ptr[p.m] - base, p.nnz_bound), 0);
  const int64_t nce = std::max<int64_t>(1, (end + p.chunk - 1) / p.chunk);
  if (c + 1 >= nce) return;
  if (fx.x < 0 || fx.x >= p.m) return;
  const int64_t r = fx.x, rs = fx.y, re = fx.z;
  const int64_t c2 = std::min<int64_t>((re - 1 - base) / p.chunk, nce - 1);
  // Records after the start one, numbered t = 1 .. T: chunks c + 1 .. c2,
  // or for a long row (prefold_kernel has folded each run of its interior
  // chunks into the run's first record) c + 1, the run starts at multiples
  // of kPiece, then c2.
  const RowRecords rr = row_records(c, c2);
  const int64_t T = rr.count;
  const int64_t K = p.k;
  const bool is_min = p.reduce == OGN_REDUCE_MIN;
  const bool is_prod = p.reduce == OGN_REDUCE_PROD;
  const bool later = p.mm_mode == MM_LATER;
  const bool nanprop = p.mm_mode == MM_NANPROP;
  constexpr int kBatch = 8;
  if (K > kWave / 2) {
    // every lane on a feature: one fold in chunk order.  A lane folds its
    // features k and k + 64 together (NF = 2), so the record loads of both
    // are in flight at once and a wave walks its row's chain of dependent
    // loads once for K <= 128 instead of once per 64 features.
    constexpr int NF = 2;
    for (int64_t k0 = lane; k0 < K; k0 += NF * kWave) {
      bool fok[NF];
      int64_t base_rec[NF];
      AT a[NF];
      MT best[NF];
      int64_t barg[NF];
  #pragma unroll
      for (int f = 0; f < NF; ++f) {
        const int64_t k = k0 + f * kWave;
        fok[f] = k < K;
        base_rec[f] = (b * p.nchunks) * K + (fok[f] ? k : k0);
        a[f] = 0;
        best[f] = 0;
        barg[f] = kNone;
        if constexpr (RK == RK_MINMAX) {
          best[f] = (MT)static_cast<const double*>(p.rec_tail)[base_rec[f] + c * K];
          barg[f] = p.arg_tail[base_rec[f] + c * K];
        } else if constexpr (RK == RK_LSE) {
          const float2 t = static_cast<const float2*>(p.rec_tail)[base_rec[f] + c * K];
          best[f] = t.x;
          a[f] = t.y;
        } else {
          a[f] = static_cast<const AT*>(p.rec_tail)[base_rec[f] + c * K];
        }
      }
      for (int64_t t0 = 1; t0 <= T; t0 += kBatch) {
        AT va[NF][kBatch];
        float vb[NF][kBatch];
        double vd[NF][kBatch];
        int64_t vg[NF][kBatch];
  #pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const bool ok = t0 + j <= T;
          const int64_t cc = rr.chunk(std::min<int64_t>(t0 + j, T));
          const bool head = cc >= c2;
  #pragma unroll
          for (int f = 0; f < NF; ++f) {
            const int64_t ri = base_rec[f] + cc * K;
            if constexpr (RK == RK_MINMAX) {
              vd[f][j] = ok ? static_cast<const double*>(head ? p.rec_head : p.rec_tail)[ri] : 0.0;
              vg[f][j] = ok ? (head ? p.arg_head : p.arg_tail)[ri] : kNone;
            } else if constexpr (RK == RK_LSE) {
              const float2 t = ok ? static_cast<const float2*>(head ? p.rec_head : p.rec_tail)[ri]
                                  : make_float2(-__builtin_inff(), 0.f);
              va[f][j] = t.x;
              vb[f][j] = t.y;
            } else {
              va[f][j] = ok ? static_cast<const AT*>(head ? p.rec_head : p.rec_tail)[ri]
                            : (is_prod ? (AT)1 : (AT)0);
            }
          }
        }
  #pragma unroll
        for (int f = 0; f < NF; ++f) {
  #pragma unroll
          for (int j = 0; j < kBatch; ++j) {
            if constexpr (RK == RK_MINMAX) {
              const MT ob = (MT)vd[f][j];
              const int64_t oa = vg[f][j];
              // later records hold later positions
              if (oa != kNone && !(nanprop && best[f] != best[f]) &&
                  (barg[f] == kNone || better(ob, best[f], is_min) || (later && ob == best[f]) ||
                   (nanprop && ob != ob))) {
                best[f] = ob;
                barg[f] = oa;
              }
            } else if constexpr (RK == RK_LSE) {
              float m = (float)best[f];
              float sa = (float)a[f];
              lse_merge(m, sa, (float)va[f][j], vb[f][j]);
              best[f] = m;
              a[f] = (AT)sa;
            } else {
              a[f] = is_prod ? a[f] * va[f][j] : a[f] + va[f][j];
            }
          }
        }
      }
  #pragma unroll
      for (int f = 0; f < NF; ++f) {
        if (!fok[f]) continue;
        const int64_t k = k0 + f * kWave;
        const int64_t off = b * p.out_bstride + r * K + k;
        if constexpr (INT && RK == RK_SUM) {
          finish_int(p, off, a[f], re - rs);
          continue;
        }
        float v;
        int64_t ag = 0;
        finish_elem<RK, MT>(p, b, r, k, rs, re, (float)a[f], best[f], barg[f], &v, &ag);
        store_floats<1>(p.out, p.out_dt, off, &v);
        if constexpr (RK == RK_MINMAX) {
          if (p.arg) p.arg[off] = ag;
        }
      }
    }
    return;
  }
  int kw = 1;
  while (kw < K && kw < kWave) kw <<= 1;
  const int ng = kWave / kw;
  const int g = lane / kw;
  for (int64_t k = lane % kw; k < K; k += kw) {
    const int64_t base_rec = (b * p.nchunks) * K + k;
    AT a = is_prod ? (AT)1 : (AT)0;
    MT best = 0;
    int64_t barg = kNone;
    if constexpr (RK == RK_LSE) best = -__builtin_inff();
    if (g == 0) {  // the row's first piece
      if constexpr (RK == RK_MINMAX) {
        best = (MT) static_cast<const double*>(p.rec_tail)[base_rec + c * K];
        barg = p.arg_tail[base_rec + c * K];
      } else if constexpr (RK == RK_LSE) {
        const float2 t = static_cast<const float2*>(p.rec_tail)[base_rec + c * K];
        best = t.x;
        a = t.y;
      } else {
        a = static_cast<const AT*>(p.rec_tail)[base_rec + c * K];
      }
    }
    // fold records t = c0, c0 + ng, ... (B loads in flight per lane; full: only
    // whole batches; returns where it stopped)
    auto fold = [&](auto bc, int64_t from, int64_t to, bool full) -> int64_t {
      constexpr int B = decltype(bc)::value;
      int64_t c0 = from;
      for (; full ? c0 + (int64_t)(B - 1) * ng <= to : c0 <= to; c0 += (int64_t)B * ng) {
        AT va[B];
        float vb[B];
        double vd[B];
        int64_t vg[B];
#pragma unroll
        for (int j = 0; j < B; ++j) {
          const int64_t t = c0 + (int64_t)j * ng;
          const bool ok = t <= to;
          const int64_t cc = rr.chunk(std::min<int64_t>(t, T));
          const int64_t ri = base_rec + cc * K;
          const bool head = cc >= c2;
          if constexpr (RK == RK_MINMAX) {
            vd[j] = ok ? static_cast<const double*>(head ? p.rec_head : p.rec_tail)[ri] : 0.0;
            vg[j] = ok ? (head ? p.arg_head : p.arg_tail)[ri] : kNone;
          } else if constexpr (RK == RK_LSE) {
            const float2 t = ok ? static_cast<const float2*>(head ? p.rec_head : p.rec_tail)[ri]
                                : make_float2(-__builtin_inff(), 0.f);
            va[j] = t.x;
            vb[j] = t.y;
          } else {
            va[j] = ok ? static_cast<const AT*>(head ? p.rec_head : p.rec_tail)[ri] : (is_prod ? (AT)1 : (AT)0);
          }
        }
#pragma unroll
        for (int j = 0; j < B; ++j) {
          if constexpr (RK == RK_MINMAX) {
            mm_merge<MT>(best, barg, (MT)vd[j], vg[j], is_min, later, nanprop);
          } else if constexpr (RK == RK_LSE) {
            float m = (float)best;
            float sa = (float)a;
            lse_merge(m, sa, (float)va[j], vb[j]);
            best = m;
            a = (AT)sa;
          } else {
            a = is_prod ? a * va[j] : a + va[j];
          }
        }
      }
      return c0;
    };
    fold(std::integral_constant<int, 8>{}, 1 + g, T, false);
    // merge the lane groups (partners kw, 2kw, ... lanes apart)
    for (int d = kw; d < kWave; d <<= 1) {
      if constexpr (RK == RK_MINMAX) {
        const MT ob = (MT)__shfl_xor((double)best, d);
        const int64_t oa = __shfl_xor(barg, d);
        mm_merge<MT>(best, barg, ob, oa, is_min, later, nanprop);
      } else if constexpr (RK == RK_LSE) {
        const float om = __shfl_xor((float)best, d), os = __shfl_xor((float)a, d);
        float m = (float)best;
        float sa = (float)a;
        lse_merge(m, sa, om, os);
        best = m;
        a = (AT)sa;
      } else {
        const AT o = __shfl_xor(a, d);
        a = is_prod ? a * o : a + o;
      }
    }
    if (g != 0) continue;
    const int64_t off = b * p.out_bstride + r * K + k;
    if constexpr (INT && RK == RK_SUM) {
      finish_int(p, off, a, re - rs);
      continue;
    }
    float v;
    int64_t ag = 0;
    finish_elem<RK, MT>(p, b, r, k, rs, re, (float)a, best, barg, &v, &ag);
    store_floats<1>(p.out, p.out_dt, off, &v);
    if constexpr (RK == RK_MINMAX) {
      if (p.arg) p.arg[off] = ag;
    }
  }
}

// ------------------------------------------------------------------ host side
struct Plan {
  bool vec;
  int g;
  int64_t tiles;
  int64_t chunk;
  int64_t nchunks;
};

// gather: SpMM (feature rows gathered through col) rather than contiguous rows.
Plan make_plan(int64_t nnz_bound, int64_t k, int in_dtype, bool aligned, bool gather = false);

struct Workspace {
  size_t chunk_row, fix, head, tail, arg_head, arg_tail, total;
};

Workspace workspace_layout(const Plan& pl, int64_t k, int64_t batch, int64_t ptr_batches, int rk);

// Run the engine: chunk-row pass, main pass, fix-up pass.  `name` labels the
// launches for the opt-in timer (<name>_main etc.).
// Layout options of run(): no row longer than 64 * the smallest chunk (4096
// positions: the long-row pre-fold is skipped), and keeping / reusing the
// chunk layout (chunk_row, fix) of a workspace across calls with one
// pointer array.
enum { LAYOUT_SHORT_ROWS = 1, LAYOUT_KEEP = 2, LAYOUT_REUSE = 4 };
constexpr int64_t kShortRowsMax = 4096;

// Fingerprint of a layout kept in a caller workspace: the workspace, the
// pointer array and the plan values it was computed for (v[0] names the
// layout kind: 0 engine chunk layout, 1 grouped-softmax long-row list).
struct KeptKey {
  const void* ws;
  const void* ptr;
  int64_t v[8];
  int64_t payload[8];  // host facts kept with the layout (not part of the key)
  bool same(const KeptKey& o) const {
    if (ws != o.ws || ptr != o.ptr) return false;
    for (int i = 0; i < 8; ++i)
      if (v[i] != o.v[i]) return false;
    return true;
  }
};
bool kept_layout_match(const KeptKey& k);
// as kept_layout_match, also copying out the stored payload on a match
bool kept_layout_find(const KeptKey& k, int64_t* payload);
void kept_layout_store(const KeptKey& k);

int run(const Plan& pl, Params& p, int in_dtype, int index_dtype, bool gather, int rk, int64_t batch,
        void* workspace, size_t workspace_bytes, hipStream_t s, const char* name, int layout = 0);

// Per-dtype / per-mode instantiations (engine_<mode>_<dt>.hip).
#define OGN_ENGINE_DECL(NAME) \
  void NAME(const Plan&, int rk, bool i64, dim3, hipStream_t, const Params&);
OGN_ENGINE_DECL(launch_gather_f32)
OGN_ENGINE_DECL(launch_gather_f16)
OGN_ENGINE_DECL(launch_gather_bf16)
OGN_ENGINE_DECL(launch_contig_f32)
OGN_ENGINE_DECL(launch_contig_f16)
OGN_ENGINE_DECL(launch_contig_bf16)
// contiguous fast variants with non-temporal source loads (engine_contig_<dt>_nt.hip)
OGN_ENGINE_DECL(launch_contig_f32_nt)
OGN_ENGINE_DECL(launch_contig_f16_nt)
OGN_ENGINE_DECL(launch_contig_bf16_nt)
OGN_ENGINE_DECL(launch_gather_i8)
// gather-mode extrema and log-sum-exp (engine_gather_<dt>_ext.hip; their
// own translation units, so that the build's longest compile is shorter)
OGN_ENGINE_DECL(launch_gather_f32_ext)
OGN_ENGINE_DECL(launch_gather_f16_ext)
OGN_ENGINE_DECL(launch_gather_bf16_ext)
OGN_ENGINE_DECL(launch_gather_i8_ext)
#undef OGN_ENGINE_DECL

template <int DT, typename IDX, bool VL, int RK, bool GATHER, int VAR, bool NTS = false>
void launch_g(int g, dim3 grid, hipStream_t s, const Params& p) {
  switch (g) {
#define OGN_G(GV) \
  case GV: hipLaunchKernelGGL((engine_kernel<DT, IDX, GV, VL, RK, GATHER, VAR, NTS>), grid, dim3(kBlock), 0, s, p); break;
    OGN_G(1) OGN_G(2) OGN_G(4) OGN_G(8) OGN_G(16) OGN_G(32) OGN_G(64)
#undef OGN_G
    default: break;
  }
}

template <int DT, typename IDX, int RK, bool GATHER, int VAR, bool NTS = false>
void launch_rk_f(const Plan& pl, dim3 grid, hipStream_t s, const Params& p) {
  if (pl.vec) {
    launch_g<DT, IDX, true, RK, GATHER, VAR, NTS>(pl.g, grid, s, p);
  } else if (pl.g == 1) {
    hipLaunchKernelGGL((engine_kernel<DT, IDX, 1, false, RK, GATHER, VAR, NTS>), grid, dim3(kBlock), 0, s, p);
  } else {
    hipLaunchKernelGGL((engine_kernel<DT, IDX, 64, false, RK, GATHER, VAR, NTS>), grid, dim3(kBlock), 0, s, p);
  }
}

// Which variant serves a request: the fast ones need x * w messages with a
// scalar (or no) weight, no product reduction, and for min/max the
// NaN-ignoring first-tie rule (torch_sparse SpMM, segment_csr) or the
// later-tie rule (segment_coo, scatter).
inline int variant_of(int rk, bool gather, const Params& p) {
  if (p.val_op != OP_MUL || p.val_mode == 2 || p.reduce == OGN_REDUCE_PROD) return V_GENERIC;
  if (rk != RK_MINMAX) return V_FIRST;
  if (p.mm_mode == MM_SPMM || p.mm_mode == MM_SEGCSR) return V_FIRST;
  if (p.mm_mode == MM_LATER) return gather && p.val_mode != 0 ? V_GENERIC : V_LATER;  // V_LATER: unweighted
  return V_GENERIC;
}

// NTS (contiguous mode): non-temporal source loads in the fast variants; the
// generic variant keeps plain loads.
template <int DT, typename IDX, int RK, bool GATHER, bool NTS = false>
void launch_rk(const Plan& pl, dim3 grid, hipStream_t s, const Params& p) {
  const int v = variant_of(RK, GATHER, p);
  if constexpr (GATHER) {
    // every gathered byte offset (row * K + k) * size fits in 32 bits
    const uint64_t bytes = (uint64_t)p.n * (uint64_t)p.k * sizeof(typename Elem<DT>::S);
    if (v == V_FIRST && pl.vec && bytes < (1ull << 32)) {
      launch_g<DT, IDX, true, RK, GATHER, V_FIRST32>(pl.g, grid, s, p);
      return;
    }
  }
  // later-tie extrema: contiguous segments, and gather mode with int64 rows
  // (the unsorted scatter reducing through its sort permutation)
  if constexpr (RK == RK_MINMAX && (!GATHER || std::is_same<IDX, int64_t>::value)) {
    if (v == V_LATER) {
      launch_rk_f<DT, IDX, RK, GATHER, V_LATER, NTS>(pl, grid, s, p);
      return;
    }
  }
  if (v == V_FIRST) launch_rk_f<DT, IDX, RK, GATHER, V_FIRST, NTS>(pl, grid, s, p);
  else if constexpr (!NTS) launch_rk_f<DT, IDX, RK, GATHER, V_GENERIC>(pl, grid, s, p);
}

// Gather mode (SpMM, and scatter / grouped statistics through a permutation)
// instantiates int32 and int64 indices with sum / min-max and int64 rows for
// log-sum-exp; contiguous mode (segments) uses int64 pointers with every
// reduction kind.
template <int DT>
void launch_gather_sum_dt(const Plan& pl, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  i64 ? launch_rk<DT, int64_t, RK_SUM, true>(pl, grid, s, p) : launch_rk<DT, int32_t, RK_SUM, true>(pl, grid, s, p);
}

template <int DT>
void launch_gather_ext_dt(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  if (rk == RK_LSE) {
    // log-sum-exp statistics through a permutation (int64 rows, unweighted):
    // the grouped softmax over an unsorted index
    if constexpr (DT != OGN_I8) launch_rk_f<DT, int64_t, RK_LSE, true, V_FIRST>(pl, grid, s, p);
  } else {
    i64 ? launch_rk<DT, int64_t, RK_MINMAX, true>(pl, grid, s, p)
        : launch_rk<DT, int32_t, RK_MINMAX, true>(pl, grid, s, p);
  }
}

template <int DT, bool NTS = false>
void launch_contig_dt(const Plan& pl, int rk, bool i64, dim3 grid, hipStream_t s, const Params& p) {
  (void)i64;  // segment pointers are int64
  if (rk == RK_MINMAX) launch_rk<DT, int64_t, RK_MINMAX, false, NTS>(pl, grid, s, p);
  else if (rk == RK_LSE) launch_rk<DT, int64_t, RK_LSE, false, NTS>(pl, grid, s, p);
  else launch_rk<DT, int64_t, RK_SUM, false, NTS>(pl, grid, s, p);
}

}  // namespace eng
}  // namespace ogn
