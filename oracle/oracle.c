/*
 * oracle.c -- CPU restatement of the ops-gnn reference goldens for the sparse
 * message-passing hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (ops_gnn, libogn_hip.so)
 * links, loads or calls this file; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, as the checker and as the timed CPU
 * baseline.
 *
 * Every function reduces each output cell in index order and accumulates in
 * double, as the reference goldens do (they compute in float64 and cast
 * once).  Inputs are float32 (fp16 / bf16 tensors widen to float32 exactly);
 * outputs are double so that callers can apply the golden's final cast.
 * OpenMP parallelises over independent output rows/segments only, so results
 * do not depend on the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_NONE INT64_MAX

/* ---------------------------------------------------------------- SpMM
 * torch_sparse SpMM golden: reference test/torch_sparse_spmm/arch35/golden.py:91-116.
 *   out[b,r,k] = R_e value[e,(k|0)] * mat[b,col[e],k] over e in [ptr[r], ptr[r+1]).
 * sum/mean (mean divides by the row length, golden :103-104); min/max ignore
 * NaN products (golden :106-108), the first edge attaining the extremum wins
 * (the `.max(-2)` over a boolean mask returns the first True, golden :109),
 * and an empty or all-NaN row gives 0 with arg = nnz (golden :93, :111-113).
 * value_width is 0 (no value), 1, or k.
 */
void oracle_spmm_csr(const int64_t* ptr, const int64_t* col, const float* value,
                     int64_t value_width, const float* mat, int64_t batch, int64_t m,
                     int64_t n, int64_t k, int reduce, double* out, int64_t* arg) {
  const int64_t nnz = ptr[m];
  for (int64_t b = 0; b < batch; ++b) {
    const float* mb = mat + b * n * k;
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t r = 0; r < m; ++r) {
      const int64_t a = ptr[r], z = ptr[r + 1];
      double* o = out + (b * m + r) * k;
      int64_t* ag = arg ? arg + (b * m + r) * k : 0;
      if (reduce <= 1) {
        for (int64_t j = 0; j < k; ++j) o[j] = 0.0;
        for (int64_t e = a; e < z; ++e) {
          const float* row = mb + col[e] * k;
          for (int64_t j = 0; j < k; ++j) {
            const double w = value_width == 0 ? 1.0
                           : (double)value[value_width == 1 ? e : e * k + j];
            o[j] += (double)row[j] * w;
          }
        }
        if (reduce == 1 && z > a)
          for (int64_t j = 0; j < k; ++j) o[j] /= (double)(z - a);
      } else {
        const int is_min = reduce == 2;
        for (int64_t j = 0; j < k; ++j) {
          double best = 0.0;
          int64_t where = ORACLE_NONE;
          for (int64_t e = a; e < z; ++e) {
            const double w = value_width == 0 ? 1.0
                           : (double)value[value_width == 1 ? e : e * k + j];
            const double p = (double)mb[col[e] * k + j] * w;
            if (isnan(p)) continue;
            if (where == ORACLE_NONE || (is_min ? p < best : p > best)) {
              best = p;
              where = e;
            }
          }
          o[j] = where == ORACLE_NONE ? 0.0 : best;
          if (ag) ag[j] = where == ORACLE_NONE ? nnz : where;
        }
      }
    }
  }
}

/* ---------------------------------------------------------------- ind2ptr / ptr2ind
 * reference test/sparse/arch35/golden.py:6-27 (torch_sparse convert_cpu.cpp):
 * out[i] = number of entries of the sorted `ind` that are < i, i in [0, rows].
 */
void oracle_ind2ptr(const int64_t* ind, int64_t numel, int64_t rows, int64_t* out) {
  if (numel == 0) {
    for (int64_t i = 0; i <= rows; ++i) out[i] = 0;
    return;
  }
  for (int64_t i = 0; i <= ind[0] && i <= rows; ++i) out[i] = 0;
  for (int64_t i = 0; i + 1 < numel; ++i)
    for (int64_t r = ind[i]; r < ind[i + 1]; ++r)
      if (r + 1 <= rows) out[r + 1] = i + 1;
  for (int64_t i = ind[numel - 1] + 1; i <= rows; ++i) out[i] = numel;
}

/* reference test/sparse/arch35/golden.py:30-43: out[e] = r with ptr[r] <= e < ptr[r+1]. */
void oracle_ptr2ind(const int64_t* ptr, int64_t rows, int64_t numel, int64_t* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t e = ptr[r]; e < ptr[r + 1] && e < numel; ++e) out[e] = r;
}

/* ---------------------------------------------------------------- segment_csr
 * reference test/segment_csr/arch35/golden.py:21-103 and the arch35 kernel
 * csrc/npu/segment_csr/op_kernel/arch35/segment_csr.cpp:16-34,
 * :506-640.  src is viewed as [batch, len, feat]; ptr as [batch | 1, segs+1]
 * (ptr_stride 0 broadcasts one pointer vector).  sum/mean accumulate in
 * double; empty segments give 0 (and arg = len).  min/max start from +-inf
 * and update on strict improvement only, so the first extremum wins and NaN
 * never enters (the arch35 kernel's rule; the golden's torch.min/max agrees
 * on NaN-free data).  End pointers are clamped to len (golden :64).
 */
void oracle_segment_csr(const float* src, const int64_t* ptr, int64_t ptr_stride,
                        int64_t batch, int64_t len, int64_t feat, int64_t segs, int reduce,
                        double* out, int64_t* arg) {
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t* p = ptr + b * ptr_stride;
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t s = 0; s < segs; ++s) {
      int64_t a = p[s], z = p[s + 1];
      if (z > len) z = len;
      double* o = out + (b * segs + s) * feat;
      int64_t* ag = arg ? arg + (b * segs + s) * feat : 0;
      for (int64_t j = 0; j < feat; ++j) {
        if (a >= z) {
          o[j] = 0.0;
          if (ag) ag[j] = len;
          continue;
        }
        if (reduce <= 1) {
          double acc = 0.0;
          for (int64_t i = a; i < z; ++i) acc += (double)src[(b * len + i) * feat + j];
          o[j] = reduce == 1 ? acc / (double)(z - a) : acc;
        } else {
          const int is_min = reduce == 2;
          double best = is_min ? INFINITY : -INFINITY;
          int64_t where = a;
          for (int64_t i = a; i < z; ++i) {
            const double v = (double)src[(b * len + i) * feat + j];
            if (is_min ? v < best : v > best) {
              best = v;
              where = i;
            }
          }
          o[j] = best;
          if (ag) ag[j] = where;
        }
      }
    }
  }
}

/* ---------------------------------------------------------------- segment_coo (Ascend 950 rules)
 * reference csrc/npu/segment_coo/op_kernel/arch35/segment_coo.cpp:114-153
 * (ReduceSegments), restated as an in-order fold over the sorted index:
 * src [batch, len, feat]; index [ib, len] (ib = 1 broadcasts); out/arg
 * [batch, segs, feat].  has_out: `out` holds the caller's values on entry.
 *  sum: overwrite (start 0).  mean: start from out if has_out, divide by the
 *  count when non-empty (empty keeps the start value).  min/max: start from
 *  out (arg = len) if has_out, else from the segment's first element; take
 *  x when x <= v (min) / x >= v (max), so the LAST extremum wins and NaN
 *  never enters (a NaN start value stays).  Empty: value 0 (no out) / arg len.
 */
void oracle_segment_coo(const float* src, const int64_t* index, int64_t ib, int64_t batch,
                        int64_t len, int64_t feat, int64_t segs, int reduce, int has_out,
                        double* out, int64_t* arg) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t* idx = index + (ib == 1 ? 0 : b * len);
    double* o = out + b * segs * feat;
    int64_t* ag = arg ? arg + b * segs * feat : 0;
    for (int64_t i = 0; i < segs * feat; ++i) {
      if (reduce == 0 || !has_out) o[i] = 0.0; /* sum always overwrites */
      if (ag) ag[i] = len;
    }
    int64_t j = 0;
    while (j < len) {
      const int64_t s = idx[j];
      int64_t z = j;
      while (z < len && idx[z] == s) ++z;
      if (s >= 0 && s < segs) {
        for (int64_t f = 0; f < feat; ++f) {
          double v;
          int64_t where = len;
          int64_t start = j;
          if (reduce <= 1) {
            v = (reduce == 1 && has_out) ? o[s * feat + f] : 0.0;
          } else if (has_out) {
            v = o[s * feat + f];
          } else {
            v = (double)src[(b * len + j) * feat + f];
            where = j;
            start = j + 1;
          }
          for (int64_t t = (reduce <= 1 ? j : start); t < z; ++t) {
            const double x = (double)src[(b * len + t) * feat + f];
            if (reduce <= 1) v += x;
            else if (reduce == 2 ? x <= v : x >= v) {
              v = x;
              where = t;
            }
          }
          if (reduce == 1) v /= (double)(z - j);
          o[s * feat + f] = v;
          if (ag && reduce >= 2) ag[s * feat + f] = where;
        }
      }
      j = z;
    }
  }
}

/* ---------------------------------------------------------------- scatter (torch_scatter)
 * reference test/scatter/arch35/golden.py:35-127: an in-order fold over every
 * element of src [before, len, after] into out [before, size, after] at
 * index (same shape as src, already broadcast).  sum/mean add, prod
 * multiplies; min/max take x when x <= out / x >= out (later tie); mean
 * divides by the count where the count is non-zero.  Without has_out, out
 * starts at 0 (sum/mean), 1 (prod) or the dtype's finite extreme `limit`
 * (min/max), and positions never taken by min/max become 0.  arg = len when
 * nothing was taken.  reduce codes: 0 sum 1 mean 2 min 3 max 4 prod.
 */
static void scatter_fold(const float* src32, const double* src64, const int64_t* index, int64_t before,
                         int64_t len, int64_t after, int64_t size, int reduce, int has_out, double limit,
                         double* out, int64_t* arg) {
  const int64_t total = before * size * after;
  int64_t* count = 0;
  if (reduce == 1) {
    count = (int64_t*)calloc((size_t)total, sizeof(int64_t));
  }
  for (int64_t i = 0; i < total; ++i) {
    if (!has_out) out[i] = reduce == 4 ? 1.0 : reduce == 2 ? limit : reduce == 3 ? -limit : 0.0;
    if (arg) arg[i] = len;
  }
  for (int64_t b = 0; b < before; ++b)
    for (int64_t l = 0; l < len; ++l)
      for (int64_t f = 0; f < after; ++f) {
        const int64_t t = index[(b * len + l) * after + f];
        if (t < 0 || t >= size) continue;
        const int64_t e = (b * len + l) * after + f;
        const double x = src32 ? (double)src32[e] : src64[e];
        const int64_t key = (b * size + t) * after + f;
        if (reduce == 0 || reduce == 1) {
          out[key] += x;
          if (count) count[key] += 1;
        } else if (reduce == 4) {
          out[key] *= x;
        } else if (reduce == 2 ? x <= out[key] : x >= out[key]) {
          out[key] = x;
          if (arg) arg[key] = l;
        }
      }
  if (count) {
    for (int64_t i = 0; i < total; ++i)
      if (count[i] > 0) out[i] /= (double)count[i];
    free(count);
  }
  if (!has_out && (reduce == 2 || reduce == 3) && arg) {
    for (int64_t i = 0; i < total; ++i)
      if (arg[i] == len) out[i] = 0.0;
  }
}

void oracle_scatter(const float* src, const int64_t* index, int64_t before, int64_t len, int64_t after,
                    int64_t size, int reduce, int has_out, double limit, double* out, int64_t* arg) {
  scatter_fold(src, 0, index, before, len, after, size, reduce, has_out, limit, out, arg);
}

/* float64 scatter: the same fold on double inputs (the golden computes in
 * the source dtype, float64 here, in element order). */
void oracle_scatter_f64(const double* src, const int64_t* index, int64_t before, int64_t len, int64_t after,
                        int64_t size, int reduce, int has_out, double* out, int64_t* arg) {
  scatter_fold(0, src, index, before, len, after, size, reduce, has_out, 1.7976931348623157e308, out, arg);
}

/* ---------------------------------------------------------------- log-sum-exp
 * reference test/segment_logsumexp/golden.py:25-44 (torch.logsumexp in
 * float64 per CSR segment; empty -> -inf).  torch.logsumexp returns NaN if a
 * NaN is present, +inf if +inf is present, -inf if every term is -inf.
 */
static double lse_of(const float* x, int64_t n, int64_t stride) {
  if (n <= 0) return -INFINITY;
  double m = -INFINITY;
  for (int64_t i = 0; i < n; ++i) {
    const double v = (double)x[i * stride];
    if (isnan(v)) return NAN;
    if (v > m) m = v;
  }
  if (isinf(m)) return m;
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += exp((double)x[i * stride] - m);
  return m + log(s);
}

void oracle_segment_lse(const float* src, const int64_t* ptr, int64_t ptr_stride, int64_t batch,
                        int64_t len, int64_t feat, int64_t segs, double* out) {
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t* p = ptr + b * ptr_stride;
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t s = 0; s < segs; ++s) {
      int64_t a = p[s], z = p[s + 1];
      if (z > len) z = len;
      for (int64_t f = 0; f < feat; ++f)
        out[(b * segs + s) * feat + f] = a < z ? lse_of(src + (b * len + a) * feat + f, z - a, feat) : -INFINITY;
    }
  }
}

/* ---------------------------------------------------------------- grouped softmax family
 * reference test/common/grouped_softmax_golden.py:31-82: groups are the
 * positions along `dim` sharing an index value; every group is reduced with
 * torch.softmax / torch.log_softmax / torch.logsumexp in float64.
 * torch.softmax(v) = exp(v - max) / sum(exp(v - max)) with max the plain
 * maximum (NaN if a NaN is present), so +-inf and NaN follow IEEE from there.
 * mode 0 softmax, 1 log_softmax -> out [before, len, after];
 * mode 2 logsumexp -> out [before, groups, after] (empty group -> -inf).
 */
void oracle_group_softmax(const float* src, const int64_t* index, int64_t before, int64_t len,
                          int64_t after, int64_t groups, int mode, double* out) {
  int64_t* cnt = (int64_t*)calloc((size_t)(groups + 1), sizeof(int64_t));
  for (int64_t l = 0; l < len; ++l)
    if (index[l] >= 0 && index[l] < groups) cnt[index[l] + 1]++;
  for (int64_t g = 0; g < groups; ++g) cnt[g + 1] += cnt[g];
  int64_t* pos = (int64_t*)malloc((size_t)(len > 0 ? len : 1) * sizeof(int64_t));
  int64_t* fill = (int64_t*)calloc((size_t)(groups > 0 ? groups : 1), sizeof(int64_t));
  for (int64_t l = 0; l < len; ++l) {
    const int64_t g = index[l];
    if (g >= 0 && g < groups) pos[cnt[g] + fill[g]++] = l;
  }
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t g = 0; g < groups; ++g) {
    const int64_t* ps = pos + cnt[g];
    const int64_t n = cnt[g + 1] - cnt[g];
    for (int64_t b = 0; b < before; ++b)
      for (int64_t f = 0; f < after; ++f) {
        double m = -INFINITY;
        int nan = 0;
        for (int64_t i = 0; i < n; ++i) {
          const double v = (double)src[(b * len + ps[i]) * after + f];
          if (isnan(v)) nan = 1;
          else if (v > m) m = v;
        }
        if (nan) m = NAN;
        if (mode == 2) {
          double r;
          if (n == 0) r = -INFINITY;
          else if (isnan(m)) r = NAN;
          else if (isinf(m)) r = m;
          else {
            double s = 0.0;
            for (int64_t i = 0; i < n; ++i) s += exp((double)src[(b * len + ps[i]) * after + f] - m);
            r = m + log(s);
          }
          out[(b * groups + g) * after + f] = r;
          continue;
        }
        double s = 0.0;
        for (int64_t i = 0; i < n; ++i) s += exp((double)src[(b * len + ps[i]) * after + f] - m);
        for (int64_t i = 0; i < n; ++i) {
          const double v = (double)src[(b * len + ps[i]) * after + f] - m;
          out[(b * len + ps[i]) * after + f] = mode == 0 ? exp(v) / s : v - log(s);
        }
      }
  }
  if (mode != 2) {
    /* positions whose index is out of range keep 0 (golden result starts as zeros) */
    for (int64_t l = 0; l < len; ++l)
      if (index[l] < 0 || index[l] >= groups)
        for (int64_t b = 0; b < before; ++b)
          for (int64_t f = 0; f < after; ++f) out[(b * len + l) * after + f] = 0.0;
  }
  free(cnt);
  free(pos);
  free(fill);
}

/* ---------------------------------------------------------------- grouped softmax backward
 * Gradient of oracle_group_softmax w.r.t. src, computed from the float64
 * forward -- what autograd of the reference's float64 golden gives
 * (test/common/grouped_softmax_golden.py:86-98 for logsumexp; softmax and
 * log_softmax through torch's own Jacobians):
 *   softmax:     y * (g - sum_group(y * g))
 *   log_softmax: g - exp(y) * sum_group(g)
 *   logsumexp:   g[group] * exp(x - lse[group])   (grad is [before, groups, after])
 * Positions outside every group get 0.
 */
void oracle_group_softmax_backward(const float* src, const float* grad, const int64_t* index, int64_t before,
                                   int64_t len, int64_t after, int64_t groups, int mode, double* gsrc) {
  const int64_t total = before * len * after;
  const int64_t ocells = mode == 2 ? before * groups * after : total;
  double* y = (double*)malloc((size_t)(ocells > 0 ? ocells : 1) * sizeof(double));
  oracle_group_softmax(src, index, before, len, after, groups, mode, y);
  for (int64_t i = 0; i < total; ++i) gsrc[i] = 0.0;
  if (mode == 2) {
    for (int64_t b = 0; b < before; ++b)
      for (int64_t l = 0; l < len; ++l) {
        const int64_t g = index[l];
        if (g < 0 || g >= groups) continue;
        for (int64_t f = 0; f < after; ++f) {
          const int64_t o = (b * groups + g) * after + f, i = (b * len + l) * after + f;
          gsrc[i] = (double)grad[o] * exp((double)src[i] - y[o]);
        }
      }
    free(y);
    return;
  }
  const int64_t cells = before * groups * after;
  double* t = (double*)calloc((size_t)(cells > 0 ? cells : 1), sizeof(double));
  for (int64_t b = 0; b < before; ++b)
    for (int64_t l = 0; l < len; ++l) {
      const int64_t g = index[l];
      if (g < 0 || g >= groups) continue;
      for (int64_t f = 0; f < after; ++f) {
        const int64_t i = (b * len + l) * after + f;
        t[(b * groups + g) * after + f] += mode == 0 ? y[i] * (double)grad[i] : (double)grad[i];
      }
    }
  for (int64_t b = 0; b < before; ++b)
    for (int64_t l = 0; l < len; ++l) {
      const int64_t g = index[l];
      if (g < 0 || g >= groups) continue;
      for (int64_t f = 0; f < after; ++f) {
        const int64_t i = (b * len + l) * after + f;
        const double tt = t[(b * groups + g) * after + f];
        gsrc[i] = mode == 0 ? y[i] * ((double)grad[i] - tt) : (double)grad[i] - exp(y[i]) * tt;
      }
    }
  free(t);
  free(y);
}

/* ---------------------------------------------------------------- SDDMM
 * reference test/sddmm_csr/arch22/golden.py:18-90: per edge e with row r
 * (ptr[r] <= e < ptr[r+1]) and column col[e], the operands are
 * lhs[t_l(e)] / rhs[t_r(e)] with t = 0 -> r, 1 -> e, 2 -> col[e].
 * op 0 dot (sum over k, double), 1 add, 2 sub, 3 mul, 4 div, 5 copy_lhs,
 * 6 copy_rhs.  out: [nnz] for dot, [nnz, k] otherwise.
 */
void oracle_sddmm(const int64_t* ptr, const int64_t* col, int64_t m, const float* lhs, const float* rhs,
                  int lt, int rt, int op, int64_t k, double* out) {
  for (int64_t r = 0; r < m; ++r) {
    for (int64_t e = ptr[r]; e < ptr[r + 1]; ++e) {
      const int64_t li = lt == 0 ? r : (lt == 1 ? e : col[e]);
      const int64_t ri = rt == 0 ? r : (rt == 1 ? e : col[e]);
      if (op == 0) {
        double s = 0.0;
        for (int64_t j = 0; j < k; ++j) s += (double)lhs[li * k + j] * (double)rhs[ri * k + j];
        out[e] = s;
        continue;
      }
      for (int64_t j = 0; j < k; ++j) {
        const double a = op == 6 ? 0.0 : (double)lhs[li * k + j];
        const double b = op == 5 ? 0.0 : (double)rhs[ri * k + j];
        double v;
        switch (op) {
          case 1: v = a + b; break;
          case 2: v = a - b; break;
          case 3: v = a * b; break;
          case 4: v = a / b; break;
          case 5: v = a; break;
          default: v = b; break;
        }
        out[e * k + j] = v;
      }
    }
  }
}

/* ---------------------------------------------------------------- DGL spmm
 * reference test/unified_spmm/arch22/golden.py:13-92 (messages, then
 * index_add for sum/mean and scatter_reduce amax/amin with include_self from
 * -inf/+inf for max/min, empty rows -> 0).  torch's amax/amin propagate NaN,
 * so a row holding a NaN message is NaN.  msg: 0 copy (x), 1 add, 2 sub,
 * 3 mul, 4 div with w[e, (j | 0)] (width 1 or k); w may be NULL for copy.
 * copy_rhs is msg 5 (the edge value itself, x unused).
 * reduce: 0 sum, 1 mean, 2 min, 3 max.
 */
void oracle_spmm_dgl(const int64_t* ptr, const int64_t* col, int64_t m, const float* x, const float* w,
                     int64_t width, int msg, int reduce, int64_t k, double* out) {
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t r = 0; r < m; ++r) {
    for (int64_t j = 0; j < k; ++j) {
      const int64_t a = ptr[r], z = ptr[r + 1];
      double acc = reduce == 2 ? INFINITY : (reduce == 3 ? -INFINITY : 0.0);
      int nan = 0;
      for (int64_t e = a; e < z; ++e) {
        const double xv = msg == 5 ? 0.0 : (double)x[col[e] * k + j];
        const double wv = w ? (double)w[width == 1 ? e : e * k + j] : 0.0;
        double v;
        switch (msg) {
          case 1: v = xv + wv; break;
          case 2: v = xv - wv; break;
          case 3: v = xv * wv; break;
          case 4: v = xv / wv; break;
          case 5: v = wv; break;
          default: v = xv; break;
        }
        if (reduce <= 1) acc += v;
        else if (isnan(v)) nan = 1;
        else if (reduce == 2 ? v < acc : v > acc) acc = v;
      }
      if (reduce == 1 && z > a) acc /= (double)(z - a);
      if (reduce >= 2) acc = (z == a) ? 0.0 : (nan ? NAN : acc);
      out[r * k + j] = acc;
    }
  }
}

/* ---------------------------------------------------------------- gather
 * reference test/gather_csr/arch35/golden.py:63-90 (gather_csr_cpu): out row
 * i of batch b is src row s with ptr[s] <= i < ptr[s+1], rows before ptr[0]
 * stay zero; rows are copied as raw bytes.  gather_coo
 * (test/gather_coo/arch35/test_gather_coo.py:87-106): out[b, e] = src[b, index[b, e]].
 */
void oracle_gather_csr(const int64_t* ptr, int64_t ptr_batches, const unsigned char* src, int64_t batch,
                       int64_t segments, int64_t row_bytes, int64_t out_rows, unsigned char* out) {
  memset(out, 0, (size_t)(batch * out_rows * row_bytes));
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t* p = ptr + (ptr_batches == 1 ? 0 : b) * (segments + 1);
    for (int64_t s = 0; s < segments; ++s)
      for (int64_t i = p[s]; i < p[s + 1]; ++i)
        memcpy(out + (b * out_rows + i) * row_bytes, src + (b * segments + s) * row_bytes, (size_t)row_bytes);
  }
}

void oracle_gather_coo(const int64_t* index, const unsigned char* src, int64_t batch, int64_t src_rows,
                       int64_t entries, int64_t row_bytes, unsigned char* out) {
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t e = 0; e < entries; ++e)
      memcpy(out + (b * entries + e) * row_bytes, src + (b * src_rows + index[b * entries + e]) * row_bytes,
             (size_t)row_bytes);
}

/* ---------------------------------------------------------------- exact integer dtypes
 * Integer segment_csr / segment_coo / scatter.  Values travel as int64 (any
 * int8 / uint8 / int16 / int32 / int64 input widens exactly); `bits` and
 * `is_unsigned` name the source dtype, and narrow() gives the value of that
 * dtype an int64 wraps to -- the golden's `.to(dtype)`.  Every fold runs in
 * element order and wraps in the dtype at each step (uint64 arithmetic, then
 * narrow), exactly as the goldens' typed tensors do.
 */
static int64_t narrow(int64_t v, int bits, int is_unsigned) {
  if (bits >= 64) return v;
  const uint64_t m = (1ull << bits) - 1;
  const uint64_t u = (uint64_t)v & m;
  if (!is_unsigned && (u >> (bits - 1))) return (int64_t)(u | ~m);
  return (int64_t)u;
}

static int64_t trunc_div(int64_t a, int64_t b) { return a / b; } /* C division truncates */

static int64_t floor_div(int64_t a, int64_t b) {
  const int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}

static int64_t int_limit(int bits, int is_unsigned, int want_max) {
  if (is_unsigned) return want_max ? (int64_t)((1ull << bits) - 1) : 0;
  if (bits >= 64) return want_max ? INT64_MAX : INT64_MIN;
  return want_max ? (int64_t)((1ull << (bits - 1)) - 1) : -(int64_t)(1ull << (bits - 1));
}

/* segment_csr, reference test/segment_csr/arch35/golden.py:21-103: per
 * segment, sum = typed sum (`selected.sum(0).to(dtype)`); mean =
 * _mean_from_typed_sum (golden :21-34): count narrowed to the dtype, truncating
 * division, 0 where the narrowed count is 0; min/max = torch.min/max over the
 * rows, first extremum for arg (segment_argminmax_cpu, golden :84-103).
 * Empty segments: 0, arg = len.  End pointers clamp to len (golden :64). */
void oracle_int_segment_csr(const int64_t* src, const int64_t* ptr, int64_t ptr_stride, int64_t batch,
                            int64_t len, int64_t feat, int64_t segs, int reduce, int bits, int is_unsigned,
                            int64_t* out, int64_t* arg) {
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t* p = ptr + b * ptr_stride;
    for (int64_t s = 0; s < segs; ++s) {
      int64_t a = p[s], z = p[s + 1];
      if (z > len) z = len;
      for (int64_t j = 0; j < feat; ++j) {
        const int64_t o = (b * segs + s) * feat + j;
        if (arg) arg[o] = len;
        if (a >= z) {
          out[o] = 0;
          continue;
        }
        if (reduce <= 1) {
          int64_t acc = 0;
          for (int64_t i = a; i < z; ++i) acc = narrow((int64_t)((uint64_t)acc + (uint64_t)src[(b * len + i) * feat + j]), bits, is_unsigned);
          if (reduce == 1) {
            const int64_t c = narrow(z - a, bits, is_unsigned);
            acc = c == 0 ? 0 : narrow(trunc_div(acc, c), bits, is_unsigned);
          }
          out[o] = acc;
        } else {
          int64_t best = src[(b * len + a) * feat + j], where = a;
          for (int64_t i = a + 1; i < z; ++i) {
            const int64_t v = src[(b * len + i) * feat + j];
            if (reduce == 2 ? v < best : v > best) {
              best = v;
              where = i;
            }
          }
          out[o] = best;
          if (arg) arg[o] = where;
        }
      }
    }
  }
}

/* segment_coo, reference csrc/npu/segment_coo/op_kernel/arch35/segment_coo.cpp:114-153
 * (ReduceSegments) with FinishMean (:18-31), as an in-order fold over the
 * sorted index (same layout and seeding rules as oracle_segment_coo above).
 * mean: sum from out (has_out) or 0; a non-empty segment gives
 * narrow(narrow(sum) / narrow(count)), or the exact sum / count when the
 * narrowed count is 0 (a byte count divisible by 256). */
void oracle_int_segment_coo(const int64_t* src, const int64_t* index, int64_t ib, int64_t batch, int64_t len,
                            int64_t feat, int64_t segs, int reduce, int has_out, int bits, int is_unsigned,
                            int64_t* out, int64_t* arg) {
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t* idx = index + (ib == 1 ? 0 : b * len);
    int64_t* o = out + b * segs * feat;
    int64_t* ag = arg ? arg + b * segs * feat : 0;
    for (int64_t i = 0; i < segs * feat; ++i) {
      if (reduce == 0 || !has_out) o[i] = 0;
      if (ag) ag[i] = len;
    }
    int64_t j = 0;
    while (j < len) {
      const int64_t s = idx[j];
      int64_t z = j;
      while (z < len && idx[z] == s) ++z;
      if (s >= 0 && s < segs) {
        for (int64_t f = 0; f < feat; ++f) {
          int64_t v, where = len, start = j;
          if (reduce <= 1) {
            v = (reduce == 1 && has_out) ? o[s * feat + f] : 0; /* exact (64-bit) sum */
          } else if (has_out) {
            v = o[s * feat + f];
          } else {
            v = src[(b * len + j) * feat + f];
            where = j;
            start = j + 1;
          }
          for (int64_t t = (reduce <= 1 ? j : start); t < z; ++t) {
            const int64_t x = src[(b * len + t) * feat + f];
            if (reduce <= 1) v = (int64_t)((uint64_t)v + (uint64_t)x);
            else if (reduce == 2 ? x <= v : x >= v) {
              v = x;
              where = t;
            }
          }
          if (reduce == 1) {
            const int64_t c = narrow(z - j, bits, is_unsigned);
            v = c != 0 ? trunc_div(narrow(v, bits, is_unsigned), c) : trunc_div(v, z - j);
          }
          o[s * feat + f] = narrow(v, bits, is_unsigned);
          if (ag && reduce >= 2) ag[s * feat + f] = where;
        }
      }
      j = z;
    }
  }
}

/* scatter, reference test/scatter/arch35/golden.py:49-127: in-order fold into
 * typed out cells (each += / *= wraps in the dtype), min/max with <= / >=
 * from out or the dtype's limits (untouched cells -> 0 without out), and the
 * mean's finish (golden :106-118, python/ops_gnn/scatter.py:443-456): where
 * the count is non-zero, floor division by the count, which for 8/16-bit
 * dtypes is first narrowed to the dtype and clamped to >= 1.  reduce codes:
 * 0 sum 1 mean 2 min 3 max 4 prod. */
void oracle_int_scatter(const int64_t* src, const int64_t* index, int64_t before, int64_t len, int64_t after,
                        int64_t size, int reduce, int has_out, int bits, int is_unsigned, int64_t* out,
                        int64_t* arg) {
  const int64_t total = before * size * after;
  int64_t* count = reduce == 1 ? (int64_t*)calloc((size_t)(total > 0 ? total : 1), sizeof(int64_t)) : 0;
  for (int64_t i = 0; i < total; ++i) {
    if (!has_out)
      out[i] = reduce == 4 ? 1 : reduce == 2 ? int_limit(bits, is_unsigned, 1)
             : reduce == 3 ? int_limit(bits, is_unsigned, 0) : 0;
    if (arg) arg[i] = len;
  }
  for (int64_t b = 0; b < before; ++b)
    for (int64_t l = 0; l < len; ++l)
      for (int64_t f = 0; f < after; ++f) {
        const int64_t t = index[(b * len + l) * after + f];
        if (t < 0 || t >= size) continue;
        const int64_t x = src[(b * len + l) * after + f];
        const int64_t key = (b * size + t) * after + f;
        if (reduce == 0 || reduce == 1) {
          out[key] = narrow((int64_t)((uint64_t)out[key] + (uint64_t)x), bits, is_unsigned);
          if (count) count[key] += 1;
        } else if (reduce == 4) {
          out[key] = narrow((int64_t)((uint64_t)out[key] * (uint64_t)x), bits, is_unsigned);
        } else if (reduce == 2 ? x <= out[key] : x >= out[key]) {
          out[key] = x;
          if (arg) arg[key] = l;
        }
      }
  if (count) {
    for (int64_t i = 0; i < total; ++i) {
      if (count[i] <= 0) continue;
      int64_t d = count[i];
      if (bits <= 16) {
        d = narrow(d, bits, is_unsigned);
        if (d < 1) d = 1;
      }
      out[i] = narrow(floor_div(out[i], d), bits, is_unsigned);
    }
    free(count);
  }
  if (!has_out && (reduce == 2 || reduce == 3) && arg) {
    for (int64_t i = 0; i < total; ++i)
      if (arg[i] == len) out[i] = 0;
  }
}
