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
