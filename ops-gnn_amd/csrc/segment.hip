// Segment reductions over contiguous rows (segment_csr, segment_coo,
// sorted-index scatter, segment_logsumexp): the CSR engine in contiguous mode,
// plus the index helpers those paths need (batched ind2ptr, index facts).
#include "csr_engine.h"
#include "typed.h"

#include <cstdlib>
#include <string>

using namespace ogn;
using namespace ogn::eng;

namespace {

bool is_aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int rk_of(int reduce) {
  if (reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX) return RK_MINMAX;
  if (reduce == OGN_REDUCE_LSE) return RK_LSE;
  return RK_SUM;
}

// out[b][i] = #{ j : ind[b][j] < i }, i in [0, rows].
__global__ __launch_bounds__(256) void ind2ptr_batched_kernel(const int64_t* __restrict__ ind, int64_t numel,
                                                              int64_t rows, int64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i > rows) return;
  const int64_t* a = ind + (int64_t)blockIdx.y * numel;
  int64_t lo = 0, len = numel;
  while (len > 0) {
    const int64_t half = len >> 1;
    const bool right = a[lo + half] < i;
    lo = right ? lo + half + 1 : lo;
    len = right ? len - half - 1 : half;
  }
  out[(int64_t)blockIdx.y * (rows + 1) + i] = lo;
}

// facts[0] = 1 if some ind[j] > ind[j+1] (unsorted), facts[1] = min, facts[2] = max.
__global__ void facts_init_kernel(int64_t* facts) {
  facts[0] = 0;
  facts[1] = INT64_MAX;
  facts[2] = INT64_MIN;
}

// Each thread reads 16-byte pairs (ind[j], ind[j + 1]) at 4 pairs in flight,
// plus the element after each pair for the order test across pairs; j
// starts at `first` (0, or 1 when ind is only 8-byte aligned), and thread 0
// also takes the elements outside the pairs.  One atomic per block.
__global__ __launch_bounds__(256) void index_facts_kernel(const int64_t* __restrict__ ind, int64_t numel,
                                                          int64_t first, int64_t* facts) {
  int64_t unsorted = 0, mn = INT64_MAX, mx = INT64_MIN;
  auto take = [&](int64_t v) {
    mn = v < mn ? v : mn;
    mx = v > mx ? v : mx;
  };
  const int64_t npairs = (numel - first) / 2;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  constexpr int kU = 4;
  for (int64_t p0 = t0; p0 < npairs; p0 += kU * stride) {
    longlong2 v[kU];
    int64_t nx[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t p = p0 + u * stride;
      const int64_t j = first + 2 * p;
      v[u] = p < npairs ? *reinterpret_cast<const longlong2*>(ind + j) : make_longlong2(INT64_MAX, INT64_MAX);
      nx[u] = p < npairs && j + 2 < numel ? ind[j + 2] : INT64_MAX;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (p0 + u * stride >= npairs) break;
      take(v[u].x);
      take(v[u].y);
      unsorted |= (v[u].x > v[u].y) | (v[u].y > nx[u]);
    }
  }
  if (t0 == 0) {
    if (first == 1) {  // ind[0], before the first pair
      take(ind[0]);
      if (numel > 1 && ind[0] > ind[1]) unsorted = 1;
    }
    if ((numel - first) % 2 == 1) take(ind[numel - 1]);  // after the last pair (its order tested there)
  }
  for (int off = 32; off > 0; off >>= 1) {
    unsorted |= __shfl_xor(unsorted, off);
    const int64_t omn = __shfl_xor(mn, off), omx = __shfl_xor(mx, off);
    mn = omn < mn ? omn : mn;
    mx = omx > mx ? omx : mx;
  }
  __shared__ int64_t red[3][4];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = unsorted;
    red[1][w] = mn;
    red[2][w] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) {
      unsorted |= red[0][i];
      mn = red[1][i] < mn ? red[1][i] : mn;
      mx = red[2][i] > mx ? red[2][i] : mx;
    }
    if (unsorted) atomicMax((unsigned long long*)&facts[0], 1ull);
    atomicMin((long long*)&facts[1], (long long)mn);
    atomicMax((long long*)&facts[2], (long long)mx);
  }
}

// One-feature rows (k == 1) that are long on average: one wavefront per
// (batch, row).  Lanes read the row as aligned 16-byte packets (8 fp16/bf16
// or 4 fp32 positions), fold each packet into the log-sum-exp state (m, s)
// with one rescale, and combine the 64 lane states with a max butterfly and
// a sum butterfly (fmax and + commute, so every lane ends with the same
// bits).  The general engine
// spreads one-feature rows over 64 lanes with one 2-byte load each; here
// every load is a full packet, and only the two packets a row shares with
// its neighbours pay for per-position masks.
template <int DT>
__device__ __forceinline__ void load_packet(const typename Elem<DT>::S* row, int64_t q, int64_t rs, int64_t re,
                                            int64_t length, float* x) {
  using E = Elem<DT>;
  constexpr int V = E::VEC;
  if (q >= rs && q + V <= re) {  // interior packet (re <= length)
    E::unpack(*reinterpret_cast<const uint4*>(row + q), x);
    return;
  }
#pragma unroll
  for (int i = 0; i < V; ++i)  // outside the row: -inf, exp(-inf) = 0
    x[i] = (q + i >= rs && q + i < re) ? E::load1(row, q + i) : -__builtin_inff();
}

template <int DT>
__device__ __forceinline__ void row_lse_k1(const typename Elem<DT>::S* row, int64_t rs, int64_t re, int64_t length,
                                           float& m, float& sacc) {
  constexpr int V = Elem<DT>::VEC;
  m = -__builtin_inff();
  sacc = 0.f;
#pragma unroll 2
  for (int64_t q = rs / V * V + (int64_t)lane_id() * V; q < re; q += (int64_t)kWave * V) {
    float x[V];
    load_packet<DT>(row, q, rs, re, length, x);
    float pm = m;
#pragma unroll
    for (int i = 0; i < V; ++i) pm = fmaxf(pm, x[i]);  // NaN-ignoring, as lse_add
    const float cn = clampf_max(pm);
    float t = sacc * fast_exp(clampf_max(m) - cn);
#pragma unroll
    for (int i = 0; i < V; ++i) t += fast_exp(x[i] - cn);
    m = pm;
    sacc = t;
  }
  // Across the 64 lanes: the row maximum first (a max butterfly), then each
  // lane rescales its sum to that maximum once and a sum butterfly adds
  // them -- two cheap butterflies instead of six log-sum-exp merges.
  float gm = m;
  gm = fmaxf(gm, xor_shfl<1>(gm));
  gm = fmaxf(gm, xor_shfl<2>(gm));
  gm = fmaxf(gm, xor_shfl<4>(gm));
  gm = fmaxf(gm, xor_shfl<8>(gm));
  gm = fmaxf(gm, xor_shfl<16>(gm));
  gm = fmaxf(gm, xor_shfl<32>(gm));
  float sv = sacc == 0.f ? 0.f : sacc * fast_exp(clampf_max(m) - clampf_max(gm));
  sv += xor_shfl<1>(sv);
  sv += xor_shfl<2>(sv);
  sv += xor_shfl<4>(sv);
  sv += xor_shfl<8>(sv);
  sv += xor_shfl<16>(sv);
  sv += xor_shfl<32>(sv);
  m = gm;
  sacc = sv;
}

// 4 wavefronts per block, one row each.
template <int DT>
__global__ __launch_bounds__(256) void row_stats_k1_kernel(const int64_t* __restrict__ ptr, const void* __restrict__ src,
                                                           int64_t length, int64_t segments, float* __restrict__ m_out,
                                                           float* __restrict__ s_out) {
  const int64_t r = (int64_t)blockIdx.x * 4 + wave_in_block();
  if (r >= segments) return;
  const int64_t b = blockIdx.y;
  const int64_t rs = std::max<int64_t>(ptr[r], 0);
  const int64_t re = std::min<int64_t>(ptr[r + 1], length);
  float m, sacc;
  row_lse_k1<DT>(static_cast<const typename Elem<DT>::S*>(src) + b * length, rs, re, length, m, sacc);
  if (lane_id() == 0) {
    m_out[b * segments + r] = m;
    s_out[b * segments + r] = sacc;
  }
}

// Per-row constants of the softmax outputs: inv = 1 / s and ls = ln s from
// the hardware reciprocal and log2 (about 1 ulp each; an output is
// e * inv or (x - m) - ls, well inside the fp32 tolerance), both NaN for a
// row holding +inf, so that every output of such a row is NaN.
__device__ __forceinline__ void softmax_row_constants(float m, float s, float& inv, float& ls) {
  const bool poisoned = m == __builtin_inff();
  inv = poisoned ? __builtin_nanf("") : __builtin_amdgcn_rcpf(s);
  ls = poisoned ? __builtin_nanf("") : __builtin_amdgcn_logf(s) * 0.693147180559945309f;
}

// 64-lane reduction for the row kernels: four DPP steps inside each 16-lane
// row (quad_perm xor 1, quad_perm xor 2, half-row mirror, row mirror), after
// which every lane of a row holds the row's result, then the four row
// results are read as uniform values and combined.  Every lane returns the
// same bits (each step combines the same two operands on both partners).
template <bool MAX>
__device__ __forceinline__ float wave_reduce64(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  v = op(v, dpp(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  v = op(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row_mirror
  const int b = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
  return op(op(r0, r1), op(r2, r3));
}

// Softmax / log_softmax of one one-feature row held in registers: the row
// spans at most 64 * U aligned 16-byte packets; lane l holds packets l,
// l + 64, ...  fetch_row_packets issues the U loads (all in flight at once;
// packets past the row read as zero), finish_row_packets masks positions
// outside [rs, re) to -inf and computes the max, the sum of exponentials and
// the outputs from registers: one read and one exponential per position.
// A row holding +inf gives NaN throughout (torch.softmax).
// Every lane issues its U loads unconditionally, so that all of them are in
// flight before the first is used (a load under a branch, merged with a
// default value, makes the compiler wait for it on the spot).  A packet
// outside the row, or not wholly inside the buffer, re-reads a packet the
// row already reads (addresses stay in bounds; its values are masked or
// reloaded element by element in finish_row_packets).
template <int DT>
__device__ __forceinline__ int64_t packet_address(int64_t q, int64_t q0, int64_t re, int64_t length) {
  constexpr int V = Elem<DT>::VEC;
  const int64_t last_full = (length - V) / V * V;  // length >= V
  return q < re && q + V <= length ? q : std::min<int64_t>(q0, last_full);
}

template <int DT, int U>
__device__ __forceinline__ void fetch_row_packets(const typename Elem<DT>::S* __restrict__ row, int64_t rs,
                                                  int64_t re, int64_t length, uint4* raw) {
  constexpr int V = Elem<DT>::VEC;
  if (length < V) return;  // no whole packet: finish_row_packets loads elements
  const int64_t q0 = rs / V * V;
  const int lane = (int)lane_id();
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t q = q0 + (int64_t)(u * kWave + lane) * V;
    raw[u] = load16(row + packet_address<DT>(q, q0, re, length));
  }
}

template <int DT, int U>
__device__ __forceinline__ void finish_row_packets(const typename Elem<DT>::S* __restrict__ row,
                                                   void* __restrict__ out, int64_t obase, int64_t rs, int64_t re,
                                                   int64_t length, int log_mode, const uint4* raw) {
  using E = Elem<DT>;
  constexpr int V = E::VEC;
  const int64_t q0 = rs / V * V;
  const int lane = (int)lane_id();
  const uint32_t n = (uint32_t)(re - rs);
  float x[U][V];
  float pm = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t q = q0 + (int64_t)(u * kWave + lane) * V;
    if (q < re && q + V > length) {  // the buffer's last, partial packet
#pragma unroll
      for (int i = 0; i < V; ++i) x[u][i] = q + i < length ? E::load1(row, q + i) : 0.f;
    } else {
      E::unpack(raw[u], x[u]);
    }
    const int32_t d = (int32_t)(q - rs);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      x[u][i] = (uint32_t)(d + i) < n ? x[u][i] : -__builtin_inff();
      pm = fmaxf(pm, x[u][i]);  // NaN-ignoring
    }
  }
  const float m = wave_reduce64<true>(pm);
  const float cm = clampf_max(m);
  float ps = 0.f;
  if (log_mode) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < V; ++i) ps += fast_exp(x[u][i] - cm);
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < V; ++i) {
        x[u][i] = fast_exp(x[u][i] - cm);
        ps += x[u][i];
      }
  }
  const float s = wave_reduce64<false>(ps);
  float inv, ls;
  softmax_row_constants(m, s, inv, ls);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t q = q0 + (int64_t)(u * kWave + lane) * V;
    if (q >= re) continue;
    const int32_t d = (int32_t)(q - rs);
    float v[V];
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = log_mode ? (x[u][i] - cm) - ls : x[u][i] * inv;
    if (d >= 0 && (uint32_t)(d + V) <= n) {
      store_floats<V, true>(out, DT, obase + q, v);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i)
        if ((uint32_t)(d + i) < n) store_floats<1>(out, DT, obase + q + i, &v[i]);
    }
  }
}

template <int DT, int U>
__device__ __forceinline__ void softmax_row_in_registers(const typename Elem<DT>::S* __restrict__ row,
                                                         void* __restrict__ out, int64_t obase, int64_t rs,
                                                         int64_t re, int64_t length, int log_mode) {
  uint4 raw[U];
  fetch_row_packets<DT, U>(row, rs, re, length, raw);
  finish_row_packets<DT, U>(row, out, obase, rs, re, length, log_mode, raw);
}

// Rows of up to kWaveRowPackets packets: one wavefront each, in registers.
// Longer rows (the tail of a lognormal or power-law degree distribution) are
// listed by that kernel and done by row_softmax_long_kernel, a block per row.
constexpr int64_t kWaveRowPackets = 4 * kWave;

template <int DT>
__device__ __forceinline__ int64_t row_packets(int64_t rs, int64_t re) {
  constexpr int V = Elem<DT>::VEC;
  return re > rs ? (re - rs / V * V + V - 1) / V : 0;
}

// Workspace of ogn_segment_group_softmax: a long-row counter, then the list
// of long rows (b * segments + r), at most one per kWaveRowPackets * VEC
// positions of each batch.
struct LongRowList {
  unsigned long long* count;
  int64_t* rows;
};
constexpr size_t kListHeader = 256;
inline int64_t long_row_capacity(int64_t batch, int64_t length, int64_t segments, int vec) {
  return batch * std::min<int64_t>(segments, length / (kWaveRowPackets * vec) + 1);
}

__global__ void zero_u64_kernel(unsigned long long* p) { *p = 0; }

// One row per wavefront (4 per block): rows of up to 64 * 4 packets in
// registers (tier chosen by length, wave-uniform); a longer row is appended
// to the long-row list.
template <int DT>
__global__ __launch_bounds__(256) void row_softmax_k1_kernel(const int64_t* __restrict__ ptr,
                                                             const void* __restrict__ src, int64_t length,
                                                             int64_t segments, void* __restrict__ out, int log_mode,
                                                             LongRowList list) {
  using E = Elem<DT>;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave_in_block();
  if (r >= segments) return;
  const int64_t b = blockIdx.y;
  const int64_t rs = std::max<int64_t>(ptr[r], 0);
  const int64_t re = std::min<int64_t>(ptr[r + 1], length);
  const int64_t packets = row_packets<DT>(rs, re);
  if (packets == 0) return;
  const typename E::S* row = static_cast<const typename E::S*>(src) + b * length;
  const int64_t obase = b * length;
  if (packets <= kWave) return softmax_row_in_registers<DT, 1>(row, out, obase, rs, re, length, log_mode);
  if (packets <= 2 * kWave) return softmax_row_in_registers<DT, 2>(row, out, obase, rs, re, length, log_mode);
  if (packets <= 3 * kWave) return softmax_row_in_registers<DT, 3>(row, out, obase, rs, re, length, log_mode);
  if (packets <= 4 * kWave) return softmax_row_in_registers<DT, 4>(row, out, obase, rs, re, length, log_mode);
  // a long row: listed for row_softmax_long_kernel (no list: a kept plan
  // already holds the long rows)
  if (list.rows && lane_id() == 0) list.rows[atomicAdd(list.count, 1ull)] = b * segments + r;
}

// Reduction over a 256-thread block: wave_reduce64, then the 4 wave
// results combined in wave order from LDS (every thread gets the same bits).
template <bool MAX>
__device__ __forceinline__ float block_reduce256(float v, float* red) {
  v = wave_reduce64<MAX>(v);
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = MAX ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return r;
}

// One long row in registers over a 256-thread block: UB packets per thread.
template <int DT, int UB>
__device__ __forceinline__ void block_row_in_registers(const typename Elem<DT>::S* __restrict__ row,
                                                       void* __restrict__ out, int64_t obase, int64_t rs, int64_t re,
                                                       int64_t length, int log_mode, float* red) {
  using E = Elem<DT>;
  constexpr int V = E::VEC;
  constexpr int T = 256;
  const int t = (int)threadIdx.x;
  const int64_t q0 = rs / V * V;
  const uint32_t n = (uint32_t)(re - rs);
    uint4 raw[UB];
#pragma unroll
    for (int u = 0; u < UB; ++u)
      raw[u] = load16(row + packet_address<DT>(q0 + (int64_t)(u * T + t) * V, q0, re, length));
    float x[UB][V];
    float pm = -__builtin_inff();
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int64_t q = q0 + (int64_t)(u * T + t) * V;
      if (q < re && q + V > length) {
#pragma unroll
        for (int i = 0; i < V; ++i) x[u][i] = q + i < length ? E::load1(row, q + i) : 0.f;
      } else {
        E::unpack(raw[u], x[u]);
      }
      const int32_t d = (int32_t)(q - rs);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        x[u][i] = (uint32_t)(d + i) < n ? x[u][i] : -__builtin_inff();
        pm = fmaxf(pm, x[u][i]);
      }
    }
    const float m = block_reduce256<true>(pm, red);
    const float cm = clampf_max(m);
    float ps = 0.f;
#pragma unroll
    for (int u = 0; u < UB; ++u)
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float e = fast_exp(x[u][i] - cm);
        ps += e;
        if (!log_mode) x[u][i] = e;
      }
    const float s = block_reduce256<false>(ps, red);
    float inv, ls;
    softmax_row_constants(m, s, inv, ls);
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int64_t q = q0 + (int64_t)(u * T + t) * V;
      if (q >= re) continue;
      const int32_t d = (int32_t)(q - rs);
      float v[V];
#pragma unroll
      for (int i = 0; i < V; ++i) v[i] = log_mode ? (x[u][i] - cm) - ls : x[u][i] * inv;
      if (d >= 0 && (uint32_t)(d + V) <= n) {
        store_floats<V, true>(out, DT, obase + q, v);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i)
          if ((uint32_t)(d + i) < n) store_floats<1>(out, DT, obase + q + i, &v[i]);
      }
    }
}

// The listed long rows, a 256-thread block per row (blocks stride over the
// list).  Rows of up to 256 * 8 packets (16 384 fp16 positions) stay in
// registers (8 loads in flight per thread); longer rows take two passes over
// chunks of 256 * 8 packets (log-sum-exp statistics, then the outputs), each
// chunk's 8 loads per thread issued together.
// One long row, [rs, re) of `row`, over a 256-thread block: rows of up to
// 256 * UB packets in registers (UB loads in flight per thread), longer rows
// in two passes over chunks of 256 * UB packets (log-sum-exp statistics,
// then the outputs), each chunk's UB loads per thread issued together.
template <int DT, int UB>
__device__ __forceinline__ void long_row_block(const typename Elem<DT>::S* __restrict__ row, void* __restrict__ out,
                                               int64_t obase, int64_t rs, int64_t re, int64_t length, int log_mode,
                                               float* red) {
  using E = Elem<DT>;
  constexpr int V = E::VEC;
  constexpr int T = 256;
  const int t = (int)threadIdx.x;
  const int64_t q0 = rs / V * V;
  const uint32_t n = (uint32_t)(re - rs);
  const int64_t pk = row_packets<DT>(rs, re);
  if (pk <= 2 * T) {
    block_row_in_registers<DT, 2>(row, out, obase, rs, re, length, log_mode, red);
  } else if (pk <= 4 * T) {
    block_row_in_registers<DT, 4>(row, out, obase, rs, re, length, log_mode, red);
  } else if (pk <= (int64_t)UB * T) {
    block_row_in_registers<DT, UB>(row, out, obase, rs, re, length, log_mode, red);
  } else {
    // statistics: per-thread online (m, s) over chunks, then block max and
    // rescaled sum
    constexpr int64_t kChunk = (int64_t)UB * T * V;
    float m = -__builtin_inff(), sacc = 0.f;
    for (int64_t c0 = q0; c0 < re; c0 += kChunk) {
      uint4 raw[UB];
#pragma unroll
      for (int u = 0; u < UB; ++u)
        raw[u] = load16(row + packet_address<DT>(c0 + (int64_t)(u * T + t) * V, q0, re, length));
      float pm = m;
      float x[UB][V];
#pragma unroll
      for (int u = 0; u < UB; ++u) {
        const int64_t q = c0 + (int64_t)(u * T + t) * V;
        if (q < re && q + V > length) {
#pragma unroll
          for (int i = 0; i < V; ++i) x[u][i] = q + i < length ? E::load1(row, q + i) : 0.f;
        } else {
          E::unpack(raw[u], x[u]);
        }
        const int64_t d = q - rs;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          x[u][i] = (uint64_t)(d + i) < (uint64_t)n ? x[u][i] : -__builtin_inff();
          pm = fmaxf(pm, x[u][i]);
        }
      }
      const float cn = clampf_max(pm);
      float acc = sacc * fast_exp(clampf_max(m) - cn);
#pragma unroll
      for (int u = 0; u < UB; ++u)
#pragma unroll
        for (int i = 0; i < V; ++i) acc += fast_exp(x[u][i] - cn);
      m = pm;
      sacc = acc;
    }
    const float gm = block_reduce256<true>(m, red);
    const float sv = sacc == 0.f ? 0.f : sacc * fast_exp(clampf_max(m) - clampf_max(gm));
    const float s = block_reduce256<false>(sv, red);
    const float cm = clampf_max(gm);
    float inv, ls;
    softmax_row_constants(gm, s, inv, ls);
    for (int64_t c0 = q0; c0 < re; c0 += kChunk) {
      uint4 raw[UB];
#pragma unroll
      for (int u = 0; u < UB; ++u)
        raw[u] = load16(row + packet_address<DT>(c0 + (int64_t)(u * T + t) * V, q0, re, length));
#pragma unroll
      for (int u = 0; u < UB; ++u) {
        const int64_t q = c0 + (int64_t)(u * T + t) * V;
        if (q >= re) continue;
        float x[V], v[V];
        if (q + V > length) {
#pragma unroll
          for (int i = 0; i < V; ++i) x[i] = q + i < length ? E::load1(row, q + i) : 0.f;
        } else {
          E::unpack(raw[u], x);
        }
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = log_mode ? (x[i] - cm) - ls : fast_exp(x[i] - cm) * inv;
        const int64_t d = q - rs;
        if (d >= 0 && d + V <= (int64_t)n) {
          store_floats<V, true>(out, DT, obase + q, v);
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i)
            if ((uint64_t)(d + i) < (uint64_t)n) store_floats<1>(out, DT, obase + q + i, &v[i]);
        }
      }
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void row_softmax_long_kernel(const int64_t* __restrict__ ptr,
                                                               const void* __restrict__ src, int64_t length,
                                                               int64_t segments, void* __restrict__ out,
                                                               int log_mode, LongRowList list,
                                                               const longlong2* __restrict__ bounds) {
  using E = Elem<DT>;
  __shared__ float red[4];
  const int64_t count = (int64_t)*list.count;
  for (int64_t item = blockIdx.x; item < count; item += gridDim.x) {
    // a row code b * segments + r of the list, or (bounds given: a kept
    // plan) the row's clamped [start, end) in batch blockIdx.y
    int64_t b, rs, re;
    if (bounds) {
      const longlong2 bd = bounds[item];
      b = blockIdx.y;
      rs = bd.x;
      re = bd.y;
    } else {
      const int64_t code = list.rows[item];
      b = code / segments;
      const int64_t r = code - b * segments;
      rs = std::max<int64_t>(ptr[r], 0);
      re = std::min<int64_t>(ptr[r + 1], length);
    }
    long_row_block<DT, 8>(static_cast<const typename E::S*>(src) + b * length, out, b * length, rs, re, length,
                          log_mode, red);
  }
}

// ---------------------------------------------------------------- binned rows
// A kept softmax plan (one per pointer array, built on a KEEP call) lists the
// rows by class of 16-byte packets per row:
//   0: <= 8 packets -- 8-lane groups, 8 rows per wavefront
//   1: <= 16        -- 16-lane groups, 4 rows per wavefront
//   2: <= 32        -- 32-lane groups, 2 rows per wavefront
//   3..6: <= 64 / 128 / 192 / 256 -- one wavefront, 1..4 packets per lane
//   7: longer       -- a 256-thread block per row (row_softmax_long_kernel)
// Empty rows are in no class.  Rows of one wavefront each leave most lanes
// idle when they are short (a 64-position fp16 row is 8 packets); packing
// them lets every lane load a packet.  The binned launch orders classes
// from the largest rows to the smallest.
constexpr int kSmClasses = 8;
constexpr int kSmPacked = 7;  // classes run by the binned kernel

__host__ __device__ constexpr int sm_rows_per_wave(int c) { return c == 0 ? 8 : (c == 1 ? 4 : (c == 2 ? 2 : 1)); }

__device__ __forceinline__ int sm_class(int64_t packets) {
  if (packets <= 0) return -1;
  if (packets <= 8) return 0;
  if (packets <= 16) return 1;
  if (packets <= 32) return 2;
  if (packets <= 64) return 3;
  if (packets <= 128) return 4;
  if (packets <= 192) return 5;
  if (packets <= 256) return 6;
  return 7;
}

struct SmPlan {
  int64_t row_off[kSmClasses + 1];  // class c's rows: rows[row_off[c] .. row_off[c + 1])
  int64_t wave_off[kSmPacked];      // first wavefront of class c in the binned launch
  int64_t waves[kSmPacked];         // wavefronts of class c
  int64_t total;                    // wavefronts of the classes above
  int64_t long_blocks;              // leading blocks of the launch: one per long row
};

// Binning pays when short rows are common: with fewer than 1/8 of the rows
// in the 8 / 16 / 32-lane classes, rows run one wavefront each in row order
// (row_softmax_k1_kernel), which measured faster for rows of 33-256 packets
// (uniform 491-position fp16 rows: 0.093 ms in row order, 0.113 ms binned).
bool sm_plan_binned(const int64_t* counts) {
  int64_t shortr = 0, all = 0;
  for (int c = 0; c < kSmClasses; ++c) {
    all += counts[c];
    if (c < 3) shortr += counts[c];
  }
  return shortr * 8 >= all;
}

SmPlan sm_plan_from_counts(const int64_t* counts) {
  SmPlan pl{};
  pl.row_off[0] = 0;
  for (int c = 0; c < kSmClasses; ++c) pl.row_off[c + 1] = pl.row_off[c] + counts[c];
  int64_t w = 0;
  for (int c = kSmPacked - 1; c >= 0; --c) {  // largest rows first
    pl.wave_off[c] = w;
    pl.waves[c] = (counts[c] + sm_rows_per_wave(c) - 1) / sm_rows_per_wave(c);
    w += pl.waves[c];
  }
  pl.total = w;
  pl.long_blocks = counts[kSmClasses - 1];
  return pl;
}

// Workspace of the plan: counts[8], cursor[8] (u64), then the rows'
// clamped bounds (16 bytes each: one load gives a wavefront its row).
struct SmPlanSpace {
  unsigned long long* counts;
  unsigned long long* cursor;
  longlong2* rows;  // clamped [start, end) of each listed row
};

__global__ void sm_zero_kernel(unsigned long long* p, int n) {
  if ((int)threadIdx.x < n) p[threadIdx.x] = 0ull;
}

template <int DT>
__global__ __launch_bounds__(256) void sm_plan_count_kernel(const int64_t* __restrict__ ptr, int64_t length,
                                                            int64_t segments, unsigned long long* counts) {
  __shared__ unsigned int h[kSmClasses];
  if (threadIdx.x < kSmClasses) h[threadIdx.x] = 0u;
  __syncthreads();
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r < segments) {
    const int64_t rs = std::max<int64_t>(ptr[r], 0), re = std::min<int64_t>(ptr[r + 1], length);
    const int c = sm_class(row_packets<DT>(rs, re));
    if (c >= 0) atomicAdd(&h[c], 1u);
  }
  __syncthreads();
  if (threadIdx.x < kSmClasses && h[threadIdx.x]) atomicAdd(&counts[threadIdx.x], (unsigned long long)h[threadIdx.x]);
}

__global__ void sm_plan_scan_kernel(const unsigned long long* counts, unsigned long long* cursor) {
  if (threadIdx.x != 0) return;
  unsigned long long a = 0;
  for (int c = 0; c < kSmClasses; ++c) {
    cursor[c] = a;
    a += counts[c];
  }
}

template <int DT>
__global__ __launch_bounds__(256) void sm_plan_scatter_kernel(const int64_t* __restrict__ ptr, int64_t length,
                                                              int64_t segments, unsigned long long* cursor,
                                                              longlong2* __restrict__ rows) {
  __shared__ unsigned int h[kSmClasses];
  __shared__ unsigned long long base[kSmClasses];
  if (threadIdx.x < kSmClasses) h[threadIdx.x] = 0u;
  __syncthreads();
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int c = -1;
  unsigned int local = 0;
  int64_t rs = 0, re = 0;
  if (r < segments) {
    rs = std::max<int64_t>(ptr[r], 0);
    re = std::min<int64_t>(ptr[r + 1], length);
    c = sm_class(row_packets<DT>(rs, re));
    if (c >= 0) local = atomicAdd(&h[c], 1u);
  }
  __syncthreads();
  if (threadIdx.x < kSmClasses && h[threadIdx.x])
    base[threadIdx.x] = atomicAdd(&cursor[threadIdx.x], (unsigned long long)h[threadIdx.x]);
  __syncthreads();
  if (c >= 0) rows[base[c] + local] = make_longlong2(rs, re);
}

// Reduction over aligned groups of L lanes (8, 16 or 32): DPP inside each
// 16-lane row, then one cross-row exchange for 32.  Every lane of a group
// ends with the same bits.
template <int L, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  v = op(v, dpp(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  if constexpr (L >= 16) v = op(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row_mirror
  if constexpr (L >= 32) v = op(v, xor_shfl<16>(v));
  return v;
}

// Softmax / log_softmax of up to 64 / L rows of at most L packets, one per
// L-lane group, one packet per lane; `valid` false: the group has no row.
template <int DT, int L>
__device__ __forceinline__ void softmax_rows_grouped(const typename Elem<DT>::S* __restrict__ row,
                                                     void* __restrict__ out, int64_t obase, int64_t rs, int64_t re,
                                                     int64_t length, int log_mode) {
  using E = Elem<DT>;
  constexpr int V = E::VEC;
  const int gl = (int)lane_id() % L;
  const int64_t q0 = rs / V * V;
  const int64_t q = q0 + (int64_t)gl * V;
  const uint32_t n = (uint32_t)(re - rs);
  const uint4 raw = length >= V ? load16(row + packet_address<DT>(q, q0, re, length)) : make_uint4(0u, 0u, 0u, 0u);
  float x[V];
  if (q < re && q + V > length) {
#pragma unroll
    for (int i = 0; i < V; ++i) x[i] = q + i < length ? E::load1(row, q + i) : 0.f;
  } else {
    E::unpack(raw, x);
  }
  const int32_t d = (int32_t)(q - rs);
  float pm = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < V; ++i) {
    x[i] = (uint32_t)(d + i) < n ? x[i] : -__builtin_inff();
    pm = fmaxf(pm, x[i]);
  }
  const float m = group_reduce<L, true>(pm);
  const float cm = clampf_max(m);
  float ps = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const float e = fast_exp(x[i] - cm);
    ps += e;
    if (!log_mode) x[i] = e;
  }
  const float s = group_reduce<L, false>(ps);
  float inv, ls;
  softmax_row_constants(m, s, inv, ls);
  if (q >= re) return;
  float v[V];
#pragma unroll
  for (int i = 0; i < V; ++i) v[i] = log_mode ? (x[i] - cm) - ls : x[i] * inv;
  if (d >= 0 && (uint32_t)(d + V) <= n) {
    store_floats<V, true>(out, DT, obase + q, v);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i)
      if ((uint32_t)(d + i) < n) store_floats<1>(out, DT, obase + q + i, &v[i]);
  }
}

template <int DT, int L>
__device__ __forceinline__ void binned_groups(const typename Elem<DT>::S* row, void* out, int64_t obase,
                                              int64_t length, int log_mode, const longlong2* __restrict__ rows,
                                              int64_t first, int64_t last) {
  const int64_t i = first + (int64_t)(lane_id() / L);
  const longlong2 bd = i < last ? rows[i] : make_longlong2(0, 0);
  softmax_rows_grouped<DT, L>(row, out, obase, bd.x, bd.y, length, log_mode);
}

template <int DT>
__global__ __launch_bounds__(256) void row_softmax_binned_kernel(const void* __restrict__ src, int64_t length,
                                                                 void* __restrict__ out, int log_mode,
                                                                 const longlong2* __restrict__ rows, SmPlan plan) {
  using E = Elem<DT>;
  __shared__ float red[4];
  const int64_t b = blockIdx.y;
  const typename E::S* row = static_cast<const typename E::S*>(src) + b * length;
  const int64_t obase = b * length;
  if ((int64_t)blockIdx.x < plan.long_blocks) {
    // the long rows lead the grid, a block each (up to 1024 packets in
    // registers, two passes beyond), so that they overlap the rest
    const longlong2 bd = rows[plan.row_off[kSmClasses - 1] + blockIdx.x];
    return long_row_block<DT, 4>(row, out, obase, bd.x, bd.y, length, log_mode, red);
  }
  const int64_t w = ((int64_t)blockIdx.x - plan.long_blocks) * 4 + wave_in_block();
  if (w >= plan.total) return;
  int c = 0;
#pragma unroll
  for (int k = 0; k < kSmPacked; ++k)
    if (w >= plan.wave_off[k] && w < plan.wave_off[k] + plan.waves[k]) c = k;
  const int64_t idx = w - plan.wave_off[c];
  const int64_t first = plan.row_off[c] + idx * sm_rows_per_wave(c), last = plan.row_off[c + 1];
  switch (c) {
    case 0: return binned_groups<DT, 8>(row, out, obase, length, log_mode, rows, first, last);
    case 1: return binned_groups<DT, 16>(row, out, obase, length, log_mode, rows, first, last);
    case 2: return binned_groups<DT, 32>(row, out, obase, length, log_mode, rows, first, last);
    default: break;
  }
  const longlong2 bd = rows[first];
  const int64_t rs = bd.x, re = bd.y;
  if (c == 3) return softmax_row_in_registers<DT, 1>(row, out, obase, rs, re, length, log_mode);
  if (c == 4) return softmax_row_in_registers<DT, 2>(row, out, obase, rs, re, length, log_mode);
  if (c == 5) return softmax_row_in_registers<DT, 3>(row, out, obase, rs, re, length, log_mode);
  return softmax_row_in_registers<DT, 4>(row, out, obase, rs, re, length, log_mode);
}

template <int DT>
void launch_softmax_plan(hipStream_t st, const int64_t* ptr, const void* src, int64_t batch, int64_t length,
                         int64_t segments, void* out, int lm, SmPlanSpace sp, const SmPlan& plan, bool binned) {
  if (!binned) {
    const dim3 grid((unsigned)((segments + 3) / 4), (unsigned)batch);
    hipLaunchKernelGGL(row_softmax_k1_kernel<DT>, grid, dim3(256), 0, st, ptr, src, length, segments, out, lm,
                       LongRowList{nullptr, nullptr});
  } else {
    if (plan.total + plan.long_blocks > 0) {
      const dim3 g((unsigned)(plan.long_blocks + (plan.total + 3) / 4), (unsigned)batch);
      hipLaunchKernelGGL(row_softmax_binned_kernel<DT>, g, dim3(256), 0, st, src, length, out, lm, sp.rows, plan);
    }
    return;
  }
  const int64_t nlong = plan.row_off[kSmClasses] - plan.row_off[kSmClasses - 1];
  if (nlong > 0) {
    // long rows from their kept bounds, batch = blockIdx.y
    LongRowList list{sp.counts + (kSmClasses - 1), nullptr};
    const dim3 g((unsigned)std::min<int64_t>(nlong, 4096), (unsigned)batch);
    hipLaunchKernelGGL(row_softmax_long_kernel<DT>, g, dim3(256), 0, st, ptr, src, length, segments, out, lm, list,
                       sp.rows + plan.row_off[kSmClasses - 1]);
  }
}

template <int DT>
void build_softmax_plan(hipStream_t st, const int64_t* ptr, int64_t length, int64_t segments, SmPlanSpace sp) {
  const unsigned blocks = (unsigned)((segments + 255) / 256);
  hipLaunchKernelGGL(sm_zero_kernel, dim3(1), dim3(64), 0, st, sp.counts, 2 * kSmClasses);
  hipLaunchKernelGGL(sm_plan_count_kernel<DT>, dim3(blocks), dim3(256), 0, st, ptr, length, segments, sp.counts);
  hipLaunchKernelGGL(sm_plan_scan_kernel, dim3(1), dim3(64), 0, st, sp.counts, sp.cursor);
  hipLaunchKernelGGL(sm_plan_scatter_kernel<DT>, dim3(blocks), dim3(256), 0, st, ptr, length, segments, sp.cursor,
                     sp.rows);
}

template <int DT>
void launch_softmax_rows(dim3 grid, hipStream_t st, const int64_t* ptr, const void* src, int64_t length,
                         int64_t segments, void* out, int lm, LongRowList list, int64_t capacity) {
  hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(1), 0, st, list.count);
  hipLaunchKernelGGL(row_softmax_k1_kernel<DT>, grid, dim3(256), 0, st, ptr, src, length, segments, out, lm, list);
  const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(capacity, 4096));
  hipLaunchKernelGGL(row_softmax_long_kernel<DT>, dim3(blocks), dim3(256), 0, st, ptr, src, length, segments, out,
                     lm, list, nullptr);
}

void launch_stats_rows(int dtype, int64_t batch, hipStream_t st, const int64_t* ptr, const void* src, int64_t length,
                       int64_t segments, float* m, float* s) {
  const dim3 grid((unsigned)((segments + 3) / 4), (unsigned)batch);
  if (dtype == OGN_F32)
    hipLaunchKernelGGL(row_stats_k1_kernel<OGN_F32>, grid, dim3(256), 0, st, ptr, src, length, segments, m, s);
  else if (dtype == OGN_F16)
    hipLaunchKernelGGL(row_stats_k1_kernel<OGN_F16>, grid, dim3(256), 0, st, ptr, src, length, segments, m, s);
  else
    hipLaunchKernelGGL(row_stats_k1_kernel<OGN_BF16>, grid, dim3(256), 0, st, ptr, src, length, segments, m, s);
}

}  // namespace

extern "C" {

size_t ogn_segment_reduce_workspace_size(int64_t batch, int64_t length, int64_t segments, int64_t k,
                                         int64_t ptr_batches, int in_dtype, int reduce) {
  if (batch <= 0 || length < 0 || segments < 0 || k <= 0) return 0;
  if (is_exact_dtype(in_dtype)) return exact_segment_workspace_size(batch, length, k, in_dtype, reduce);
  const int rk = rk_of(reduce);
  const Plan pa = make_plan(length, k, in_dtype, true);
  const Plan pu = make_plan(length, k, in_dtype, false);
  const int64_t pbat = ptr_batches > 1 ? batch : 1;
  return std::max(workspace_layout(pa, k, batch, pbat, rk).total, workspace_layout(pu, k, batch, pbat, rk).total);
}

int ogn_segment_reduce(const int64_t* indptr, int64_t ptr_batches, const void* src, int dtype,
                       int64_t batch, int64_t length, int64_t segments, int64_t k, void* out,
                       int64_t* arg, int reduce, int semantics, int flags, void* workspace,
                       size_t workspace_bytes, void* stream) {
  if (batch < 0 || length < 0 || segments < 0 || k < 0)
    return fail(OGN_EINVAL, "ogn_segment_reduce: negative size");
  const bool exact = is_exact_dtype(dtype);
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16 && !exact)
    return fail(OGN_EUNSUPPORTED, "ogn_segment_reduce: unsupported src dtype");
  if (reduce < OGN_REDUCE_SUM || reduce > OGN_REDUCE_LSE)
    return fail(OGN_EINVAL, "ogn_segment_reduce: unknown reduce code");
  if (semantics < OGN_SEM_SEGMENT_CSR || semantics > OGN_SEM_DGL)
    return fail(OGN_EINVAL, "ogn_segment_reduce: unknown semantics code");
  if (ptr_batches != 1 && ptr_batches != batch)
    return fail(OGN_EINVAL, "ogn_segment_reduce: ptr_batches must be 1 or batch");
  const int rk = rk_of(reduce);
  if (batch == 0 || segments == 0 || k == 0) return OGN_OK;
  if (!indptr || !out) return fail(OGN_EINVAL, "ogn_segment_reduce: null pointer");
  if (length > 0 && !src) return fail(OGN_EINVAL, "ogn_segment_reduce: null src");
  const bool has_out = (flags & OGN_SEG_HAS_OUT) != 0;
  if (exact)
    return exact_segment_reduce(indptr, ptr_batches, src, dtype, batch, length, segments, k, out, arg, reduce,
                                semantics, has_out ? 1 : 0, (flags & OGN_SEG_SHORT_SEGMENTS) != 0, workspace,
                                workspace_bytes, static_cast<hipStream_t>(stream));

  const bool aligned = is_aligned(src, 16) && is_aligned(out, 16);
  const Plan pl = make_plan(length, k, dtype, aligned);
  Params p{};
  p.ptr = indptr;
  p.ptr_bstride = ptr_batches > 1 ? segments + 1 : 0;
  p.src = src;
  p.src_dt = dtype;
  p.src_bstride = length * k;
  p.out = out;
  p.out_dt = dtype;
  p.out_bstride = segments * k;
  p.arg = arg;
  p.m = segments;
  p.n = std::max<int64_t>(length, 1);
  p.k = k;
  p.nnz_bound = length;
  p.reduce = reduce;
  p.arg_empty = length;
  p.seed_mode = SEED_NONE;
  switch (semantics) {
    case OGN_SEM_SEGMENT_CSR:
      p.mm_mode = MM_SEGCSR;
      break;
    case OGN_SEM_DGL:
      p.mm_mode = MM_NANPROP;
      break;
    case OGN_SEM_SEGMENT_COO:
      p.mm_mode = MM_LATER;
      p.seed_mode = has_out ? SEED_OUT : SEED_FIRST;
      p.sum_seed = reduce == OGN_REDUCE_MEAN && has_out;
      p.mean_keep_empty = has_out;
      break;
    default:  // torch_scatter
      p.mm_mode = MM_LATER;
      p.seed_mode = has_out ? SEED_OUT : SEED_LIMIT;
      p.sum_seed = has_out;
      p.mean_keep_empty = has_out;
      p.limit = dtype == OGN_F32 ? 3.4028234663852886e38f : (dtype == OGN_F16 ? 65504.f : 3.3895313892515355e38f);
      break;
  }
  const int layout = ((flags & OGN_SEG_SHORT_SEGMENTS) ? LAYOUT_SHORT_ROWS : 0) |
                     ((flags & OGN_SEG_KEEP_LAYOUT) ? LAYOUT_KEEP : 0) |
                     ((flags & OGN_SEG_REUSE_LAYOUT) ? LAYOUT_REUSE : 0);
  return run(pl, p, dtype, OGN_I64, false, rk, batch, workspace, workspace_bytes,
             static_cast<hipStream_t>(stream), "segment", layout);
}

// arg[j] = rows[arg[j]] for a winning position, unchanged (the empty marker) otherwise.
__global__ __launch_bounds__(256) void map_arg_kernel(int64_t* __restrict__ arg, int64_t cells,
                                                      const int64_t* __restrict__ rows, int64_t length) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cells; i += stride) {
    const int64_t a = arg[i];
    if (a >= 0 && a < length) arg[i] = rows[a];
  }
}

size_t ogn_segment_reduce_gather_workspace_size(int64_t length, int64_t segments, int64_t k, int dtype,
                                                int reduce) {
  if (length < 0 || segments < 0 || k <= 0 || is_exact_dtype(dtype)) return 0;
  const int rk = rk_of(reduce);
  const Plan pa = make_plan(length, k, dtype, true, true);
  const Plan pu = make_plan(length, k, dtype, false, true);
  return std::max(workspace_layout(pa, k, 1, 1, rk).total, workspace_layout(pu, k, 1, 1, rk).total);
}

int ogn_segment_reduce_gather(const int64_t* indptr, const int64_t* rows, const void* src, int dtype,
                              int64_t src_rows, int64_t length, int64_t segments, int64_t k, void* out,
                              int64_t* arg, int reduce, int semantics, int flags, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (src_rows < 0 || length < 0 || segments < 0 || k < 0)
    return fail(OGN_EINVAL, "ogn_segment_reduce_gather: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_segment_reduce_gather: src dtype must be float32, float16 or bfloat16");
  if (reduce < OGN_REDUCE_SUM || reduce > OGN_REDUCE_PROD)
    return fail(OGN_EUNSUPPORTED, "ogn_segment_reduce_gather: sum, mean, min, max or prod");
  if (semantics != OGN_SEM_SCATTER) return fail(OGN_EUNSUPPORTED, "ogn_segment_reduce_gather: scatter semantics");
  if (segments == 0 || k == 0) return OGN_OK;
  if (!indptr || !out || (length > 0 && (!rows || !src)))
    return fail(OGN_EINVAL, "ogn_segment_reduce_gather: null pointer");
  if (length > 0 && src_rows == 0) return fail(OGN_EINVAL, "ogn_segment_reduce_gather: positions need src rows");
  const bool has_out = (flags & OGN_SEG_HAS_OUT) != 0;
  const int rk = rk_of(reduce);
  const bool aligned = is_aligned(src, 16) && is_aligned(out, 16);
  const Plan pl = make_plan(length, k, dtype, aligned, true);
  Params p{};
  p.ptr = indptr;
  p.ptr_bstride = 0;
  p.col = rows;
  p.src = src;
  p.src_dt = dtype;
  p.src_bstride = 0;
  p.out = out;
  p.out_dt = dtype;
  p.out_bstride = segments * k;
  p.arg = arg;
  p.m = segments;
  p.n = std::max<int64_t>(src_rows, 1);
  p.k = k;
  p.nnz_bound = length;
  p.reduce = reduce;
  p.arg_empty = src_rows;
  // torch_scatter rules, as ogn_segment_reduce with OGN_SEM_SCATTER
  p.mm_mode = MM_LATER;
  p.seed_mode = has_out ? SEED_OUT : SEED_LIMIT;
  p.sum_seed = has_out;
  p.mean_keep_empty = has_out;
  p.limit = dtype == OGN_F32 ? 3.4028234663852886e38f : (dtype == OGN_F16 ? 65504.f : 3.3895313892515355e38f);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc = run(pl, p, dtype, OGN_I64, true, rk, 1, workspace, workspace_bytes, s, "segment_gather", 0);
  if (rc != OGN_OK || !arg || rk != RK_MINMAX || length == 0) return rc;
  // the engine's argument is a position in `rows` order; report the src row
  const int64_t cells = segments * k;
  TimedLaunch t("segment_gather_arg", s);
  hipLaunchKernelGGL(map_arg_kernel, dim3((unsigned)std::min<int64_t>((cells + 255) / 256, 4096)), dim3(256), 0, s,
                     arg, cells, rows, length);
  return check_launch("ogn_segment_reduce_gather");
}

int ogn_segment_group_stats(const int64_t* indptr, const void* src, int dtype, int64_t batch, int64_t length,
                            int64_t segments, int64_t k, float* m_out, float* s_out, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (batch < 0 || length < 0 || segments < 0 || k < 0)
    return fail(OGN_EINVAL, "ogn_segment_group_stats: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_segment_group_stats: src dtype must be float32, float16 or bfloat16");
  if (batch == 0 || segments == 0 || k == 0) return OGN_OK;
  if (!indptr || !m_out || !s_out || (length > 0 && !src))
    return fail(OGN_EINVAL, "ogn_segment_group_stats: null pointer");
  // One-feature rows that average >= 64 positions: whole wavefronts per row.
  const int esize = dtype_size(dtype);
  if (k == 1 && length >= 64 * segments && is_aligned(src, 16) && (batch == 1 || (length * esize) % 16 == 0) &&
      batch <= 65535) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    TimedLaunch t("segment_stats_main", st);
    launch_stats_rows(dtype, batch, st, indptr, src, length, segments, m_out, s_out);
    return check_launch("ogn_segment_group_stats");
  }
  const bool aligned = is_aligned(src, 16) && is_aligned(m_out, 16);
  const Plan pl = make_plan(length, k, dtype, aligned);
  Params p{};
  p.ptr = indptr;
  p.src = src;
  p.src_dt = dtype;
  p.src_bstride = length * k;
  p.out = m_out;
  p.out_dt = OGN_F32;
  p.out_bstride = segments * k;
  p.aux = s_out;
  p.m = segments;
  p.n = std::max<int64_t>(length, 1);
  p.k = k;
  p.nnz_bound = length;
  p.reduce = OGN_REDUCE_LSE;
  p.arg_empty = length;
  return run(pl, p, dtype, OGN_I64, false, RK_LSE, batch, workspace, workspace_bytes,
             static_cast<hipStream_t>(stream), "segment_stats");
}

int ogn_segment_group_stats_gather(const int64_t* indptr, const int64_t* rows, const void* src, int dtype,
                                   int64_t src_rows, int64_t length, int64_t segments, int64_t k, float* m_out,
                                   float* s_out, void* workspace, size_t workspace_bytes, void* stream) {
  if (src_rows < 0 || length < 0 || segments < 0 || k < 0)
    return fail(OGN_EINVAL, "ogn_segment_group_stats_gather: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_segment_group_stats_gather: src dtype must be float32, float16 or bfloat16");
  if (segments == 0 || k == 0) return OGN_OK;
  if (!indptr || !m_out || !s_out || (length > 0 && (!rows || !src)))
    return fail(OGN_EINVAL, "ogn_segment_group_stats_gather: null pointer");
  if (length > 0 && src_rows == 0) return fail(OGN_EINVAL, "ogn_segment_group_stats_gather: positions need src rows");
  const bool aligned = is_aligned(src, 16) && is_aligned(m_out, 16);
  const Plan pl = make_plan(length, k, dtype, aligned, true);
  Params p{};
  p.ptr = indptr;
  p.col = rows;
  p.src = src;
  p.src_dt = dtype;
  p.src_bstride = 0;
  p.out = m_out;
  p.out_dt = OGN_F32;
  p.out_bstride = segments * k;
  p.aux = s_out;
  p.m = segments;
  p.n = std::max<int64_t>(src_rows, 1);
  p.k = k;
  p.nnz_bound = length;
  p.reduce = OGN_REDUCE_LSE;
  p.arg_empty = src_rows;
  return run(pl, p, dtype, OGN_I64, true, RK_LSE, 1, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
             "segment_stats_gather");
}

// Workspace: the long-row list (header + capacity), then the kept plan
// (counts and cursors, 256 bytes, then 16 bytes of bounds per segment).
static size_t softmax_list_bytes(int64_t batch, int64_t length, int64_t segments, int vec) {
  return (kListHeader + sizeof(int64_t) * (size_t)long_row_capacity(batch, length, segments, vec) + 255) / 256 * 256;
}

size_t ogn_segment_group_softmax_workspace_size(int64_t batch, int64_t length, int64_t segments, int dtype) {
  if (batch <= 0 || length < 0 || segments < 0) return 0;
  const int vec = 16 / dtype_size(dtype);
  return softmax_list_bytes(batch, length, segments, vec) + 256 + sizeof(longlong2) * (size_t)segments;
}

int ogn_segment_group_softmax(const int64_t* indptr, const void* src, int dtype, int64_t batch, int64_t length,
                              int64_t segments, void* out, int log_softmax, int flags, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (batch < 0 || length < 0 || segments < 0) return fail(OGN_EINVAL, "ogn_segment_group_softmax: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_segment_group_softmax: src dtype must be float32, float16 or bfloat16");
  if (batch == 0 || segments == 0 || length == 0) return OGN_OK;
  if (!indptr || !src || !out) return fail(OGN_EINVAL, "ogn_segment_group_softmax: null pointer");
  if (!is_aligned(src, 16) || !is_aligned(out, 16) || (batch > 1 && (length * dtype_size(dtype)) % 16 != 0))
    return fail(OGN_EINVAL, "ogn_segment_group_softmax: src / out rows must be 16-byte aligned");
  if (batch > 65535) return fail(OGN_EUNSUPPORTED, "ogn_segment_group_softmax: batch > 65535");
  const size_t need = ogn_segment_group_softmax_workspace_size(batch, length, segments, dtype);
  if (!workspace || workspace_bytes < need || !is_aligned(workspace, 256))
    return fail(OGN_EINVAL, "ogn_segment_group_softmax: workspace too small or not 256-byte aligned (need " +
                                std::to_string(need) + " bytes)");
  const int vec = 16 / dtype_size(dtype);
  LongRowList list{static_cast<unsigned long long*>(workspace),
                   reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + kListHeader)};
  const int64_t capacity = long_row_capacity(batch, length, segments, vec);
  hipStream_t st = static_cast<hipStream_t>(stream);
  TimedLaunch t("segment_softmax", st);
  const dim3 grid((unsigned)((segments + 3) / 4), (unsigned)batch);
  const int lm = log_softmax ? 1 : 0;
  char* plan_base = static_cast<char*>(workspace) + softmax_list_bytes(batch, length, segments, vec);
  SmPlanSpace sp{reinterpret_cast<unsigned long long*>(plan_base),
                 reinterpret_cast<unsigned long long*>(plan_base) + kSmClasses,
                 reinterpret_cast<longlong2*>(plan_base + 256)};
  KeptKey key{workspace, indptr, {2, batch, length, segments, vec, 0, 0, 0}, {}};
  int64_t counts[8];
  if ((flags & OGN_SEG_REUSE_LAYOUT) && kept_layout_find(key, counts)) {
    // the kept plan of this pointer array: rows binned by length
    const SmPlan plan = sm_plan_from_counts(counts);
    const bool bn = sm_plan_binned(counts);
    if (dtype == OGN_F32) launch_softmax_plan<OGN_F32>(st, indptr, src, batch, length, segments, out, lm, sp, plan, bn);
    else if (dtype == OGN_F16) launch_softmax_plan<OGN_F16>(st, indptr, src, batch, length, segments, out, lm, sp, plan, bn);
    else launch_softmax_plan<OGN_BF16>(st, indptr, src, batch, length, segments, out, lm, sp, plan, bn);
    return check_launch("ogn_segment_group_softmax");
  }
  if (dtype == OGN_F32) launch_softmax_rows<OGN_F32>(grid, st, indptr, src, length, segments, out, lm, list, capacity);
  else if (dtype == OGN_F16) launch_softmax_rows<OGN_F16>(grid, st, indptr, src, length, segments, out, lm, list, capacity);
  else launch_softmax_rows<OGN_BF16>(grid, st, indptr, src, length, segments, out, lm, list, capacity);
  if (flags & (OGN_SEG_KEEP_LAYOUT | OGN_SEG_REUSE_LAYOUT)) {
    // build the plan for later calls: four small kernels and one 64-byte
    // read of the class counts (this call waits for it)
    if (dtype == OGN_F32) build_softmax_plan<OGN_F32>(st, indptr, length, segments, sp);
    else if (dtype == OGN_F16) build_softmax_plan<OGN_F16>(st, indptr, length, segments, sp);
    else build_softmax_plan<OGN_BF16>(st, indptr, length, segments, sp);
    unsigned long long host[kSmClasses];
    if (hipMemcpyAsync(host, sp.counts, sizeof(host), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return fail(OGN_EHIP, "ogn_segment_group_softmax: reading the row-class counts failed");
    for (int c = 0; c < kSmClasses; ++c) key.payload[c] = (int64_t)host[c];
    kept_layout_store(key);
  }
  return check_launch("ogn_segment_group_softmax");
}

int ogn_ind2ptr_batched(const int64_t* ind, int64_t batches, int64_t numel, int64_t rows, int64_t* out,
                        void* stream) {
  if (batches < 0 || numel < 0 || rows < 0) return fail(OGN_EINVAL, "ogn_ind2ptr_batched: negative size");
  if (batches == 0) return OGN_OK;
  if (!out || (numel > 0 && !ind)) return fail(OGN_EINVAL, "ogn_ind2ptr_batched: null pointer");
  if (batches > 65535) return fail(OGN_EUNSUPPORTED, "ogn_ind2ptr_batched: more than 65535 batches");
  hipStream_t s = static_cast<hipStream_t>(stream);
  TimedLaunch t("ind2ptr_batched", s);
  hipLaunchKernelGGL(ind2ptr_batched_kernel, dim3((unsigned)((rows + 1 + 255) / 256), (unsigned)batches),
                     dim3(256), 0, s, ind, numel, rows, out);
  return check_launch("ogn_ind2ptr_batched");
}

int ogn_index_facts(const int64_t* ind, int64_t numel, int64_t* facts, void* stream) {
  if (numel < 0) return fail(OGN_EINVAL, "ogn_index_facts: negative size");
  if (!facts || (numel > 0 && !ind)) return fail(OGN_EINVAL, "ogn_index_facts: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  TimedLaunch t("index_facts", s);
  hipLaunchKernelGGL(facts_init_kernel, dim3(1), dim3(1), 0, s, facts);
  if (numel > 0) {
    const int64_t first = (reinterpret_cast<uintptr_t>(ind) & 15) ? 1 : 0;
    const int blocks = (int)std::max<int64_t>(1, std::min<int64_t>((numel / 2 + 255) / 256, 2048));
    hipLaunchKernelGGL(index_facts_kernel, dim3(blocks), dim3(256), 0, s, ind, numel, first, facts);
  }
  return check_launch("ogn_index_facts");
}

}  // extern "C"
