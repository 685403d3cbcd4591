// Segment reductions over contiguous rows (segment_csr, segment_coo,
// sorted-index scatter, segment_logsumexp): the CSR engine in contiguous mode,
// plus the index helpers those paths need (batched ind2ptr, index facts).
#include "csr_engine.h"
#include "typed.h"

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

__global__ __launch_bounds__(256) void index_facts_kernel(const int64_t* __restrict__ ind, int64_t numel,
                                                          int64_t* facts) {
  int64_t unsorted = 0, mn = INT64_MAX, mx = INT64_MIN;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel; i += stride) {
    const int64_t v = ind[i];
    mn = v < mn ? v : mn;
    mx = v > mx ? v : mx;
    if (i + 1 < numel && ind[i + 1] < v) unsorted = 1;
  }
  // wave-level reduction, then one atomic per wave
  for (int off = 32; off > 0; off >>= 1) {
    unsorted |= __shfl_xor(unsorted, off);
    const int64_t omn = __shfl_xor(mn, off), omx = __shfl_xor(mx, off);
    mn = omn < mn ? omn : mn;
    mx = omx > mx ? omx : mx;
  }
  if ((threadIdx.x & 63) == 0) {
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
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
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

// Fused softmax / log_softmax of one-feature rows: the statistics as above,
// then a second pass over the row (just read, so served by the caches) that
// writes exp(x - clamp(m)) / s or (x - clamp(m)) - log(s); a row holding
// +inf gives NaN throughout (torch.softmax).  Packets shared with a
// neighbouring row are written element by element.
template <int DT>
__global__ __launch_bounds__(256) void row_softmax_k1_kernel(const int64_t* __restrict__ ptr,
                                                             const void* __restrict__ src, int64_t length,
                                                             int64_t segments, void* __restrict__ out, int log_mode) {
  using E = Elem<DT>;
  constexpr int V = E::VEC;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= segments) return;
  const int64_t b = blockIdx.y;
  const int64_t rs = std::max<int64_t>(ptr[r], 0);
  const int64_t re = std::min<int64_t>(ptr[r + 1], length);
  const typename E::S* row = static_cast<const typename E::S*>(src) + b * length;
  float m, sacc;
  row_lse_k1<DT>(row, rs, re, length, m, sacc);
  const float cm = clampf_max(m);
  const float ls = logf(sacc);
  const float inv = 1.f / sacc;
  const bool poisoned = m == __builtin_inff();
#pragma unroll 2
  for (int64_t q = rs / V * V + (int64_t)lane_id() * V; q < re; q += (int64_t)kWave * V) {
    float x[V], v[V];
    load_packet<DT>(row, q, rs, re, length, x);
#pragma unroll
    for (int i = 0; i < V; ++i)
      v[i] = log_mode ? (x[i] - cm) - ls : fast_exp(x[i] - cm) * inv;
    if (poisoned) {
#pragma unroll
      for (int i = 0; i < V; ++i) v[i] = __builtin_nanf("");
    }
    const int64_t o = b * length + q;
    if (q >= rs && q + V <= re) {
      store_floats<V, true>(out, DT, o, v);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i)
        if (q + i >= rs && q + i < re) store_floats<1>(out, DT, o + i, &v[i]);
    }
  }
}

template <int DT>
void launch_row_kernel(bool softmax, dim3 grid, hipStream_t st, const int64_t* ptr, const void* src, int64_t length,
                       int64_t segments, float* m, float* s, void* out, int lm) {
  if (softmax)
    hipLaunchKernelGGL(row_softmax_k1_kernel<DT>, grid, dim3(256), 0, st, ptr, src, length, segments, out, lm);
  else
    hipLaunchKernelGGL(row_stats_k1_kernel<DT>, grid, dim3(256), 0, st, ptr, src, length, segments, m, s);
}

void launch_rows(bool softmax, int dtype, int64_t batch, hipStream_t st, const int64_t* ptr, const void* src,
                 int64_t length, int64_t segments, float* m, float* s, void* out, int lm) {
  const dim3 grid((unsigned)((segments + 3) / 4), (unsigned)batch);
  if (dtype == OGN_F32) launch_row_kernel<OGN_F32>(softmax, grid, st, ptr, src, length, segments, m, s, out, lm);
  else if (dtype == OGN_F16) launch_row_kernel<OGN_F16>(softmax, grid, st, ptr, src, length, segments, m, s, out, lm);
  else launch_row_kernel<OGN_BF16>(softmax, grid, st, ptr, src, length, segments, m, s, out, lm);
}

}  // namespace

extern "C" {

size_t ogn_segment_reduce_workspace_size(int64_t batch, int64_t length, int64_t segments, int64_t k,
                                         int64_t ptr_batches, int in_dtype, int reduce) {
  if (batch <= 0 || length < 0 || segments < 0 || k <= 0 || is_exact_dtype(in_dtype)) return 0;
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
                                semantics, has_out ? 1 : 0, static_cast<hipStream_t>(stream));

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
  return run(pl, p, dtype, OGN_I64, false, rk, batch, workspace, workspace_bytes,
             static_cast<hipStream_t>(stream), "segment");
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
    launch_rows(false, dtype, batch, st, indptr, src, length, segments, m_out, s_out, nullptr, 0);
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

int ogn_segment_group_softmax(const int64_t* indptr, const void* src, int dtype, int64_t batch, int64_t length,
                              int64_t segments, void* out, int log_softmax, void* stream) {
  if (batch < 0 || length < 0 || segments < 0) return fail(OGN_EINVAL, "ogn_segment_group_softmax: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_segment_group_softmax: src dtype must be float32, float16 or bfloat16");
  if (batch == 0 || segments == 0 || length == 0) return OGN_OK;
  if (!indptr || !src || !out) return fail(OGN_EINVAL, "ogn_segment_group_softmax: null pointer");
  if (!is_aligned(src, 16) || !is_aligned(out, 16) || (batch > 1 && (length * dtype_size(dtype)) % 16 != 0))
    return fail(OGN_EINVAL, "ogn_segment_group_softmax: src / out rows must be 16-byte aligned");
  if (batch > 65535) return fail(OGN_EUNSUPPORTED, "ogn_segment_group_softmax: batch > 65535");
  hipStream_t st = static_cast<hipStream_t>(stream);
  TimedLaunch t("segment_softmax", st);
  launch_rows(true, dtype, batch, st, indptr, src, length, segments, nullptr, nullptr, out, log_softmax ? 1 : 0);
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
    const int blocks = (int)std::min<int64_t>((numel + 255) / 256, 2048);
    hipLaunchKernelGGL(index_facts_kernel, dim3(blocks), dim3(256), 0, s, ind, numel, facts);
  }
  return check_launch("ogn_index_facts");
}

}  // extern "C"
