// Segment and scatter reductions for the exact dtypes: int8, uint8, int16,
// int32, int64 (and float64 for scatter).
//
// These dtypes have no fp32 arithmetic: every sum, product and mean is exact
// integer arithmetic in the source dtype's wrap-around ring (accumulated in
// 64 bits, narrowed once -- narrowing is a ring homomorphism, so the result
// equals the step-by-step typed fold), and min/max are exact compares.
//
// Contiguous segments (segment_csr, segment_coo, sorted-index scatter): one
// thread per (batch, segment, 16-byte feature packet) folds the segment's
// rows in order -- deterministic, one writer per output, loads of one row
// coalesced across the threads of a segment.  Integer segments longer than
// kLongSeg rows are first cut into fixed pieces of kPieceRows positions,
// folded in parallel (piece_kernel) into partial records, and the segment's
// thread then folds its records in position order: ring sums and products
// do not depend on the grouping, and extremum records carry their position
// and follow the same tie rule, so results are those of the serial fold
// while a hub segment no longer serialises on one thread.  float64 keeps
// the serial fold (its sum depends on the order).  Unsorted scatter: 64-bit
// atomics into a workspace (integer add/min/max are associative, so the
// result does not depend on the order; float64 sum/prod does, as in any
// atomic scatter), a second pass for the "later writer wins" arg, and a
// finishing pass that narrows, divides and writes.
//
// Per-operator rules (the mean's count narrowing and rounding differ):
//   segment_csr  reference csrc/npu/segment_csr/op_kernel/arch35/segment_csr.cpp:143-149,
//                283-296 (int64 accumulator; mean = narrow(sum) / narrow(count),
//                truncating, 0 when the narrowed count is 0), :386-407 (first
//                extremum wins); test/segment_csr/arch35/golden.py:21-60.
//   segment_coo  reference csrc/npu/segment_coo/op_kernel/arch35/segment_coo.cpp:18-31
//                (byte mean: narrow both operands, exact mean when the narrowed
//                count is 0), :114-153 (mean seeded from out, sum not; min/max
//                seeded from out or the first row, <= / >= so the last
//                extremum wins).
//   scatter      reference python/ops_gnn/scatter.py:430-458 (mean: typed sum,
//                count narrowed to the dtype for 8/16-bit types and clamped to
//                >= 1, floor division), test/scatter/arch35/golden.py:49-127
//                (seeds, <= / >= folds, untouched min/max cells give 0).
#include "typed.h"

#include <algorithm>
#include <limits>
#include <type_traits>

namespace ogn {
namespace {

template <int DT> struct Store;
template <> struct Store<OGN_I8> { using T = int8_t; };
template <> struct Store<OGN_U8> { using T = uint8_t; };
template <> struct Store<OGN_I16> { using T = int16_t; };
template <> struct Store<OGN_I32> { using T = int32_t; };
template <> struct Store<OGN_I64> { using T = int64_t; };
template <> struct Store<OGN_F64> { using T = double; };

template <int DT>
using Acc = std::conditional_t<DT == OGN_F64, double, int64_t>;

// 64-bit wrap-around add / multiply (no signed-overflow UB)
__device__ __forceinline__ int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
__device__ __forceinline__ double wadd(double a, double b) { return a + b; }
__device__ __forceinline__ int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
__device__ __forceinline__ double wmul(double a, double b) { return a * b; }

// value of the source dtype that `v` wraps to
template <int DT>
__device__ __forceinline__ Acc<DT> narrow(Acc<DT> v) {
  return (Acc<DT>)(typename Store<DT>::T)v;
}

// q = floor(a / b), b != 0
__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) {
  const int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}

template <int DT>
__device__ __forceinline__ Acc<DT> limit_of(bool is_max) {
  using T = typename Store<DT>::T;
  if constexpr (DT == OGN_F64) {
    return is_max ? -1.7976931348623157e308 : 1.7976931348623157e308;
  } else {
    return is_max ? (int64_t)std::numeric_limits<T>::min() : (int64_t)std::numeric_limits<T>::max();
  }
}

// Mean of a finished sum over `rows` >= 1 entries, per operator.
template <int DT>
__device__ __forceinline__ Acc<DT> finish_mean(Acc<DT> acc, int64_t rows, int sem) {
  if constexpr (DT == OGN_F64) {
    return acc / (double)rows;
  } else {
    const int64_t w = narrow<DT>(acc);
    const int64_t c = narrow<DT>(rows);
    if (sem == OGN_SEM_SEGMENT_CSR) return c == 0 ? 0 : narrow<DT>(w / c);
    if (sem == OGN_SEM_SEGMENT_COO) return c == 0 ? narrow<DT>(acc / rows) : narrow<DT>(w / c);
    // torch_scatter: 8/16-bit counts wrap in the dtype and are clamped to 1
    const int64_t d = sizeof(typename Store<DT>::T) <= 2 ? std::max<int64_t>(c, 1) : rows;
    return narrow<DT>(floor_div(w, d));
  }
}

template <int DT>
__device__ __forceinline__ bool takes(Acc<DT> x, Acc<DT> cur, bool is_max, bool strict) {
  return strict ? (is_max ? x > cur : x < cur) : (is_max ? x >= cur : x <= cur);
}

template <typename T, int V>
struct alignas(sizeof(T) * V) Pack {
  T v[V];
};

// ------------------------------------------------------------------ contiguous segments
enum { RC_SUM = 0, RC_PROD = 1, RC_MINMAX = 2 };

// Segments of more rows than kLongSeg take the piece records; a piece is
// kPieceRows positions (so a long segment spans at least three pieces).
constexpr int64_t kLongSeg = 4096;
constexpr int64_t kPieceRows = 2048;

struct SegArgs {
  // piece records, or null: value rec[((b * npieces + piece) * 2 + w) * k + f]
  // (w = 0: the segment holding the piece's first position, w = 1: the one
  // holding its last position, when that is another segment) and, for
  // min / max, the extremum's position at the same index of recpos
  int64_t* rec;
  int64_t* recpos;
  int64_t npieces;
  const int64_t* ptr;
  int64_t ptr_bstride;
  const void* src;
  void* out;
  int64_t* arg;
  int64_t length, segs, k, batch;
  int64_t total;    // batch * segs * packets
  FastDiv packets;  // packets per row (k / V)
  FastDiv segs_d;
  int sem, has_out, mean, is_max;
};

// Index of the segment holding position x (ptr[s] <= x < ptr[s + 1]), or -1.
__device__ __forceinline__ int64_t segment_of(const int64_t* ptr, int64_t segs, int64_t x) {
  int64_t lo = 0, hi = segs + 1;  // first index with ptr[i] > x
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ptr[mid] <= x) lo = mid + 1;
    else hi = mid;
  }
  const int64_t s = lo - 1;
  return s >= 0 && s < segs && x < ptr[s + 1] ? s : -1;
}

// One thread per (batch, piece, packet): the partial records of the (at most
// two) long segments overlapping the piece.
template <int DT, int V, int RC>
__global__ __launch_bounds__(256) void piece_kernel(SegArgs a) {
  using T = typename Store<DT>::T;
  using A = Acc<DT>;
  const int64_t packets = a.k / V;
  const int64_t total = a.batch * a.npieces * packets;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t c = i % packets;
    const int64_t t = i / packets;
    const int64_t pc = t % a.npieces;
    const int64_t b = t / a.npieces;
    const int64_t* ptr = a.ptr + b * a.ptr_bstride;
    const int64_t lo = pc * kPieceRows, hi = std::min<int64_t>(lo + kPieceRows, a.length);
    const Pack<T, V>* src = reinterpret_cast<const Pack<T, V>*>(static_cast<const T*>(a.src) + (b * a.length) * a.k + c * V);
    const int64_t row_step = a.k / V;
    const int64_t s1 = segment_of(ptr, a.segs, lo);
    const int64_t s2 = hi > lo ? segment_of(ptr, a.segs, hi - 1) : -1;
#pragma unroll 1
    for (int w = 0; w < 2; ++w) {
      const int64_t s = w == 0 ? s1 : (s2 != s1 ? s2 : -1);
      if (s < 0) continue;
      const int64_t beg = ptr[s], end = ptr[s + 1];
      if (end - beg <= kLongSeg) continue;
      const int64_t from = std::max(beg, lo), to = std::min(end, hi);
      A acc[V];
      int64_t best[V];
      {
        const Pack<T, V> x = src[from * row_step];
#pragma unroll
        for (int j = 0; j < V; ++j) {
          acc[j] = (A)x.v[j];
          best[j] = from;
        }
      }
      const bool strict = a.sem == OGN_SEM_SEGMENT_CSR;
#pragma unroll 4
      for (int64_t r = from + 1; r < to; ++r) {
        const Pack<T, V> x = src[r * row_step];
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const A xv = (A)x.v[j];
          if constexpr (RC == RC_SUM) acc[j] = wadd(acc[j], xv);
          if constexpr (RC == RC_PROD) acc[j] = wmul(acc[j], xv);
          if constexpr (RC == RC_MINMAX) {
            if (takes<DT>(xv, acc[j], a.is_max, strict)) {
              acc[j] = xv;
              best[j] = r;
            }
          }
        }
      }
      const int64_t o = ((b * a.npieces + pc) * 2 + w) * a.k + c * V;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        a.rec[o + j] = (int64_t)acc[j];
        if constexpr (RC == RC_MINMAX) a.recpos[o + j] = best[j];
      }
    }
  }
}

template <int DT, int V, int RC>
__global__ __launch_bounds__(256) void seg_kernel(SegArgs a) {
  using T = typename Store<DT>::T;
  using A = Acc<DT>;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.total; i += stride) {
    const int64_t t = fdiv(i, a.packets);
    const int64_t c = i - t * (int64_t)a.packets.d;
    const int64_t b = fdiv(t, a.segs_d);
    const int64_t s = t - b * a.segs;
    const int64_t* ptr = a.ptr + b * a.ptr_bstride;
    const int64_t beg = ptr[s], end = ptr[s + 1];
    const int64_t rows = std::max<int64_t>(end - beg, 0);
    const int64_t o = (b * a.segs + s) * a.k + c * V;
    const Pack<T, V>* src = reinterpret_cast<const Pack<T, V>*>(static_cast<const T*>(a.src) + (b * a.length) * a.k + c * V);
    const int64_t row_step = a.k / V;
    Pack<T, V>* out = reinterpret_cast<Pack<T, V>*>(static_cast<T*>(a.out) + o);
    A acc[V];
    int64_t best[V];
    Pack<T, V> seed;
    const bool seeded = a.has_out && (a.sem == OGN_SEM_SCATTER || (a.sem == OGN_SEM_SEGMENT_COO && (RC == RC_MINMAX || a.mean)));
    if (seeded) seed = *out;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      best[j] = a.length;
      if constexpr (RC == RC_SUM) acc[j] = seeded ? (A)seed.v[j] : (A)0;
      if constexpr (RC == RC_PROD) acc[j] = seeded ? (A)seed.v[j] : (A)1;
      if constexpr (RC == RC_MINMAX) acc[j] = seeded ? (A)seed.v[j] : limit_of<DT>(a.is_max);
    }
    if (a.rec && rows > kLongSeg) {
      // fold the piece records in position order: the first piece's record
      // 0 when the segment starts on the piece boundary, else its record 1;
      // record 0 of every later piece
      const int64_t pb = beg / kPieceRows, pe = (end - 1) / kPieceRows;
      const int w0 = beg % kPieceRows != 0 ? 1 : 0;
      auto rec_at = [&](int64_t pc, int w) { return ((b * a.npieces + pc) * 2 + w) * a.k + c * V; };
      int64_t pc = pb;
      bool strict = false;
      if constexpr (RC == RC_MINMAX) {
        // segment_csr / unseeded segment_coo start from the first record
        // (taken here, not through a loop-carried "first" flag: with one,
        // the gfx950 code kept later takes' positions but not their values)
        if (!seeded && a.sem != OGN_SEM_SCATTER) {
          const int64_t ro = rec_at(pb, w0);
#pragma unroll
          for (int j = 0; j < V; ++j) {
            acc[j] = (A)a.rec[ro + j];
            best[j] = a.recpos[ro + j];
          }
          pc = pb + 1;
        }
        strict = a.sem == OGN_SEM_SEGMENT_CSR;
      }
#pragma unroll 4
      for (; pc <= pe; ++pc) {
        const int64_t ro = rec_at(pc, pc == pb ? w0 : 0);
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const A xv = (A)a.rec[ro + j];
          if constexpr (RC == RC_SUM) acc[j] = wadd(acc[j], xv);
          if constexpr (RC == RC_PROD) acc[j] = wmul(acc[j], xv);
          if constexpr (RC == RC_MINMAX) {
            const int64_t xp = a.recpos[ro + j];  // loaded unconditionally: the loads pipeline
            const bool tk = takes<DT>(xv, acc[j], a.is_max, strict);
            acc[j] = tk ? xv : acc[j];
            best[j] = tk ? xp : best[j];
          }
        }
      }
    } else {
      int64_t r0 = beg;
      bool strict = false;
      if constexpr (RC == RC_MINMAX) {
        // segment_csr / unseeded segment_coo start from the segment's first row
        if (!seeded && a.sem != OGN_SEM_SCATTER && rows > 0) {
          const Pack<T, V> x = src[beg * row_step];
#pragma unroll
          for (int j = 0; j < V; ++j) {
            acc[j] = (A)x.v[j];
            best[j] = beg;
          }
          r0 = beg + 1;
        }
        strict = a.sem == OGN_SEM_SEGMENT_CSR;
      }
#pragma unroll 4
      for (int64_t r = r0; r < end; ++r) {
        const Pack<T, V> x = src[r * row_step];
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const A xv = (A)x.v[j];
          if constexpr (RC == RC_SUM) acc[j] = wadd(acc[j], xv);
          if constexpr (RC == RC_PROD) acc[j] = wmul(acc[j], xv);
          if constexpr (RC == RC_MINMAX) {
            if (takes<DT>(xv, acc[j], a.is_max, strict)) {
              acc[j] = xv;
              best[j] = r;
            }
          }
        }
      }
    }
    Pack<T, V> res;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      A v = acc[j];
      if constexpr (RC == RC_SUM) {
        if (a.mean && rows > 0) v = finish_mean<DT>(v, rows, a.sem);
      }
      if constexpr (RC == RC_MINMAX) {
        if (best[j] == a.length && !seeded) v = 0;
        if (a.arg) a.arg[o + j] = best[j];
      }
      res.v[j] = (T)v;
    }
    *out = res;
  }
}

unsigned grid_for(int64_t total) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((total + 255) / 256, 1 << 20));
}

template <int DT, int V>
void launch_seg(const SegArgs& a, int rc, hipStream_t s) {
  if constexpr (DT != OGN_F64) {
    if (a.rec) {
      TimedLaunch t("segment_exact_pieces", s);
      const dim3 g(grid_for(a.batch * a.npieces * (a.k / V)));
      if (rc == RC_SUM) hipLaunchKernelGGL((piece_kernel<DT, V, RC_SUM>), g, dim3(256), 0, s, a);
      else if (rc == RC_PROD) hipLaunchKernelGGL((piece_kernel<DT, V, RC_PROD>), g, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((piece_kernel<DT, V, RC_MINMAX>), g, dim3(256), 0, s, a);
    }
  }
  TimedLaunch t("segment_exact", s);
  const dim3 grid(grid_for(a.total));
  if (rc == RC_SUM) hipLaunchKernelGGL((seg_kernel<DT, V, RC_SUM>), grid, dim3(256), 0, s, a);
  else if (rc == RC_PROD) hipLaunchKernelGGL((seg_kernel<DT, V, RC_PROD>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((seg_kernel<DT, V, RC_MINMAX>), grid, dim3(256), 0, s, a);
}

template <int DT>
void launch_seg_dt(const SegArgs& a, int v, int rc, hipStream_t s) {
  constexpr int VW = 16 / (int)sizeof(typename Store<DT>::T);
  if (v == VW) launch_seg<DT, VW>(a, rc, s);
  else launch_seg<DT, 1>(a, rc, s);
}

// ------------------------------------------------------------------ unsorted scatter
struct ScatArgs {
  const void* src;
  const int64_t* index;
  int64_t isb, isl, isf;
  int64_t before, len, after, size;
  void* out;
  int64_t* arg;
  void* acc;       // [cells] int64 / double
  int64_t* count;  // [cells] (mean)
  int reduce, has_out;
  Split3 sp;
};

__device__ __forceinline__ void atomic_fold(int64_t* p, int64_t x, int reduce) {
  unsigned long long* u = reinterpret_cast<unsigned long long*>(p);
  switch (reduce) {
    case OGN_REDUCE_MIN: atomicMin(reinterpret_cast<long long*>(p), (long long)x); break;
    case OGN_REDUCE_MAX: atomicMax(reinterpret_cast<long long*>(p), (long long)x); break;
    case OGN_REDUCE_PROD: {
      unsigned long long old = __atomic_load_n(u, __ATOMIC_RELAXED);
      while (!__atomic_compare_exchange_n(u, &old, old * (unsigned long long)x, false, __ATOMIC_RELAXED,
                                          __ATOMIC_RELAXED)) {
      }
      break;
    }
    default: atomicAdd(u, (unsigned long long)x); break;
  }
}

__device__ __forceinline__ void atomic_fold(double* p, double x, int reduce) {
  if (reduce == OGN_REDUCE_SUM || reduce == OGN_REDUCE_MEAN) {
    atomicAdd(p, x);
    return;
  }
  unsigned long long* u = reinterpret_cast<unsigned long long*>(p);
  unsigned long long old = __atomic_load_n(u, __ATOMIC_RELAXED);
  while (true) {
    const double cur = __longlong_as_double((long long)old);
    double want;
    if (reduce == OGN_REDUCE_PROD) {
      want = cur * x;
    } else {
      // strict improvement only: ties and -0/+0 are settled by the arg pass
      if (!(reduce == OGN_REDUCE_MIN ? x < cur : x > cur)) return;
      want = x;
    }
    if (__atomic_compare_exchange_n(u, &old, (unsigned long long)__double_as_longlong(want), false,
                                    __ATOMIC_RELAXED, __ATOMIC_RELAXED))
      return;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void scat_init_kernel(ScatArgs a) {
  using T = typename Store<DT>::T;
  using A = Acc<DT>;
  const int64_t cells = a.before * a.size * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  A* acc = static_cast<A*>(a.acc);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cells; i += stride) {
    const bool mm = a.reduce == OGN_REDUCE_MIN || a.reduce == OGN_REDUCE_MAX;
    A v = a.reduce == OGN_REDUCE_PROD ? (A)1 : mm ? limit_of<DT>(a.reduce == OGN_REDUCE_MAX) : (A)0;
    if (a.has_out) v = (A) static_cast<const T*>(a.out)[i];
    acc[i] = v;
    if (a.count) a.count[i] = 0;
    if (a.arg) a.arg[i] = -1;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void scat_main_kernel(ScatArgs a) {
  using T = typename Store<DT>::T;
  using A = Acc<DT>;
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  A* acc = static_cast<A*>(a.acc);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t b, l, f;
    split3(i, a.sp, b, l, f);
    const int64_t t = a.index[b * a.isb + l * a.isl + f * a.isf];
    if (t < 0 || t >= a.size) continue;
    const int64_t o = (b * a.size + t) * a.after + f;
    atomic_fold(&acc[o], (A) static_cast<const T*>(a.src)[i], a.reduce);
    if (a.count) atomicAdd(reinterpret_cast<unsigned long long*>(&a.count[o]), 1ull);
  }
}

// Largest position whose value equals the final extremum (later writer wins).
template <int DT>
__global__ __launch_bounds__(256) void scat_arg_kernel(ScatArgs a) {
  using T = typename Store<DT>::T;
  using A = Acc<DT>;
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const A* acc = static_cast<const A*>(a.acc);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t b, l, f;
    split3(i, a.sp, b, l, f);
    const int64_t t = a.index[b * a.isb + l * a.isl + f * a.isf];
    if (t < 0 || t >= a.size) continue;
    const int64_t o = (b * a.size + t) * a.after + f;
    if ((A) static_cast<const T*>(a.src)[i] == acc[o]) atomicMax(reinterpret_cast<long long*>(&a.arg[o]), (long long)l);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void scat_finish_kernel(ScatArgs a) {
  using T = typename Store<DT>::T;
  using A = Acc<DT>;
  const int64_t cells = a.before * a.size * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const A* acc = static_cast<const A*>(a.acc);
  T* out = static_cast<T*>(a.out);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cells; i += stride) {
    A v = acc[i];
    if (a.arg) {
      const int64_t where = a.arg[i] < 0 ? a.len : a.arg[i];
      a.arg[i] = where;
      if (where == a.len) {
        v = a.has_out ? (A)out[i] : (A)0;
      } else {
        // the winning element itself (keeps -0.0 / +0.0 of the later writer)
        const int64_t f = i % a.after;
        const int64_t b = i / (a.after * a.size);
        v = (A) static_cast<const T*>(a.src)[(b * a.len + where) * a.after + f];
      }
    } else if (a.count && a.count[i] > 0) {
      v = finish_mean<DT>(v, a.count[i], OGN_SEM_SCATTER);
    }
    out[i] = (T)v;
  }
}

template <int DT>
void launch_scat(ScatArgs& a, hipStream_t s) {
  const int64_t cells = a.before * a.size * a.after;
  const int64_t total = a.before * a.len * a.after;
  {
    TimedLaunch t("scatter_init", s);
    hipLaunchKernelGGL(scat_init_kernel<DT>, dim3(grid_for(cells)), dim3(256), 0, s, a);
  }
  if (total > 0) {
    TimedLaunch t("scatter_main", s);
    hipLaunchKernelGGL(scat_main_kernel<DT>, dim3(grid_for(total)), dim3(256), 0, s, a);
  }
  if (a.arg && total > 0) {
    TimedLaunch t("scatter_arg", s);
    hipLaunchKernelGGL(scat_arg_kernel<DT>, dim3(grid_for(total)), dim3(256), 0, s, a);
  }
  TimedLaunch t("scatter_finish", s);
  hipLaunchKernelGGL(scat_finish_kernel<DT>, dim3(grid_for(cells)), dim3(256), 0, s, a);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

bool is_exact_dtype(int dt) {
  return dt == OGN_I8 || dt == OGN_U8 || dt == OGN_I16 || dt == OGN_I32 || dt == OGN_I64 || dt == OGN_F64;
}

size_t exact_segment_workspace_size(int64_t batch, int64_t length, int64_t k, int dtype, int reduce) {
  if (dtype == OGN_F64 || batch <= 0 || length <= kLongSeg || k <= 0) return 0;
  const int64_t npieces = (length + kPieceRows - 1) / kPieceRows;
  const size_t one = ((size_t)batch * npieces * 2 * k * sizeof(int64_t) + 255) / 256 * 256;
  return (reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX) ? 2 * one : one;
}

int exact_segment_reduce(const int64_t* indptr, int64_t ptr_batches, const void* src, int dtype, int64_t batch,
                         int64_t length, int64_t segments, int64_t k, void* out, int64_t* arg, int reduce,
                         int semantics, int has_out, bool short_segments, void* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  if (reduce == OGN_REDUCE_LSE || semantics == OGN_SEM_DGL)
    return fail(OGN_EUNSUPPORTED, "ogn_segment_reduce: logsumexp and DGL reductions need a floating dtype");
  if (reduce == OGN_REDUCE_PROD && semantics != OGN_SEM_SCATTER)
    return fail(OGN_EINVAL, "ogn_segment_reduce: prod is a scatter reduction");
  SegArgs a{};
  const int size = dtype_size(dtype);
  const int vw = 16 / size;
  const bool vec = k % vw == 0 && aligned16(src) && aligned16(out);
  const int v = vec ? vw : 1;
  a.ptr = indptr;
  a.ptr_bstride = ptr_batches > 1 ? segments + 1 : 0;
  a.src = src;
  a.out = out;
  a.arg = (reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX) ? arg : nullptr;
  a.length = length;
  a.segs = segments;
  a.k = k;
  a.packets = make_fastdiv(k / v);
  a.segs_d = make_fastdiv(segments);
  a.total = batch * segments * (k / v);
  a.sem = semantics;
  a.has_out = has_out;
  a.mean = reduce == OGN_REDUCE_MEAN;
  a.is_max = reduce == OGN_REDUCE_MAX;
  const int rc = reduce == OGN_REDUCE_PROD ? RC_PROD : (reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX) ? RC_MINMAX : RC_SUM;
  a.batch = batch;
  // long segments: piece records, when the caller's workspace holds them
  // (without it, or with the short-segments hint, every segment is folded
  // serially, with the same result)
  const size_t need = exact_segment_workspace_size(batch, length, k, dtype, reduce);
  if (need > 0 && !short_segments && workspace && workspace_bytes >= need) {
    a.npieces = (length + kPieceRows - 1) / kPieceRows;
    a.rec = static_cast<int64_t*>(workspace);
    a.recpos = rc == RC_MINMAX ? reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + need / 2) : nullptr;
  }
  switch (dtype) {
    case OGN_I8: launch_seg_dt<OGN_I8>(a, v, rc, stream); break;
    case OGN_U8: launch_seg_dt<OGN_U8>(a, v, rc, stream); break;
    case OGN_I16: launch_seg_dt<OGN_I16>(a, v, rc, stream); break;
    case OGN_I32: launch_seg_dt<OGN_I32>(a, v, rc, stream); break;
    case OGN_I64: launch_seg_dt<OGN_I64>(a, v, rc, stream); break;
    default: launch_seg_dt<OGN_F64>(a, v, rc, stream); break;
  }
  return check_launch("ogn_segment_reduce");
}

size_t exact_scatter_workspace_size(int64_t cells, int reduce) {
  const size_t c = (size_t)std::max<int64_t>(cells, 0);
  return (c * 8 + 255) / 256 * 256 + (reduce == OGN_REDUCE_MEAN ? (c * 8 + 255) / 256 * 256 : 0) + 256;
}

int exact_scatter_atomic(const void* src, int dtype, const int64_t* index, int64_t isb, int64_t isl, int64_t isf,
                         int64_t before, int64_t len, int64_t after, int64_t size, void* out, int64_t* arg,
                         int reduce, int has_out, void* workspace, hipStream_t stream) {
  const int64_t cells = before * size * after;
  ScatArgs a{};
  a.src = src;
  a.index = index;
  a.isb = isb;
  a.isl = isl;
  a.isf = isf;
  a.before = before;
  a.len = len;
  a.after = after;
  a.size = size;
  a.sp = make_split3(len, after);
  a.out = out;
  a.arg = (reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX) ? arg : nullptr;
  char* ws = static_cast<char*>(workspace);
  a.acc = ws;
  a.count = reduce == OGN_REDUCE_MEAN ? reinterpret_cast<int64_t*>(ws + ((size_t)cells * 8 + 255) / 256 * 256) : nullptr;
  a.reduce = reduce;
  a.has_out = has_out;
  switch (dtype) {
    case OGN_I8: launch_scat<OGN_I8>(a, stream); break;
    case OGN_U8: launch_scat<OGN_U8>(a, stream); break;
    case OGN_I16: launch_scat<OGN_I16>(a, stream); break;
    case OGN_I32: launch_scat<OGN_I32>(a, stream); break;
    case OGN_I64: launch_scat<OGN_I64>(a, stream); break;
    default: launch_scat<OGN_F64>(a, stream); break;
  }
  return check_launch("ogn_scatter_atomic");
}

}  // namespace ogn
