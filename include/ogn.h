/*
 * ogn.h -- C ABI of libogn_hip.so, the gfx950 (MI355X) implementation of the
 * ops-gnn sparse message-passing hot path.
 *
 * Conventions shared by every entry point:
 *  - All tensor arguments are raw device pointers to contiguous row-major
 *    storage; sizes are int64 element counts.  Nothing crossing this ABI is a
 *    torch type.
 *  - `stream` is a hipStream_t (NULL = legacy default stream).  Every call is
 *    asynchronous on that stream and never synchronises the device, except
 *    where a function says otherwise.
 *  - The library never allocates caller-visible memory.  Functions that need
 *    scratch memory have a *_workspace_size() query; the caller passes a
 *    device buffer of at least that many bytes (256-byte aligned).
 *  - Return value: OGN_OK (0) or an OGN_E* code; ogn_last_error() returns a
 *    thread-local message for the last failing call on the calling thread.
 *  - Index tensors (indptr / col / index) are int32 or int64 as given by the
 *    `index_dtype` argument (OGN_I32 / OGN_I64).
 *  - Reduction codes follow the reference's torch_sparse adapter
 *    (python/ops_gnn/torch_sparse_spmm.py:27): sum 0, mean 1, min 2, max 3.
 *  - dtype codes: see ogn_dtype.  The reference's output-type codes
 *    (python/ops_gnn/torch_sparse_spmm.py:28) are remapped by the host layer.
 *
 * Inputs are trusted to be valid CSR/COO (the host layer validates them with
 * ogn_validate_csr, exactly as the reference validates before launching);
 * kernels additionally clamp every gathered index into range so that a
 * malformed input gives wrong numbers, never an out-of-bounds access.
 */
#ifndef OGN_H_
#define OGN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  OGN_F32 = 0,
  OGN_F16 = 1,
  OGN_BF16 = 2,
  OGN_I8 = 3,
  OGN_I32 = 4,
  OGN_I64 = 5,
  OGN_F64 = 6,
  OGN_U8 = 7
} ogn_dtype;

typedef enum {
  OGN_REDUCE_SUM = 0,
  OGN_REDUCE_MEAN = 1,
  OGN_REDUCE_MIN = 2,
  OGN_REDUCE_MAX = 3
} ogn_reduce;

enum {
  OGN_OK = 0,
  OGN_EINVAL = 1,       /* bad argument (shape, dtype, size, null pointer) */
  OGN_EUNSUPPORTED = 2, /* valid request this build does not implement */
  OGN_EHIP = 3          /* HIP runtime error (launch failure) */
};

/* Thread-local description of the last error on this thread ("" if none). */
const char* ogn_last_error(void);
/* Target architecture the kernels were built for ("gfx950"). */
const char* ogn_arch(void);
/* ABI version; bumped on any incompatible change. */
int ogn_abi_version(void);

/* Opt-in kernel timing (diagnostics; no reference counterpart -- it replaces
 * the NPU-event timing of the reference benchmarks).  While enabled, every
 * kernel this library launches is bracketed by two HIP events on its stream.
 * ogn_timing_enable() (on or off) drops earlier records.
 * ogn_timing_query() waits for the recorded events of kernels named `kernel`
 * and returns their summed duration and launch count. */
int ogn_timing_enable(int on);
int ogn_timing_query(const char* kernel, double* total_ms, int64_t* launches);

/* ------------------------------------------------------------------ CSR
 * Device CSR validation.  Replaces ValidateCompute
 * (reference csrc/npu/torch_sparse_spmm/op_kernel/arch35/torch_sparse_spmm_kernel.h:399-425)
 * and TorchSparseSpmmValidate
 * (reference csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:136-147).
 * Writes one int32 to *status (device memory): 0 = valid, 1 = bad rowptr
 * (ptr[0] != 0, ptr[m] != nnz, decreasing, or outside [0, nnz]),
 * 2 = column outside [0, n).  The larger code wins when both occur.
 * col may be NULL to check rowptr only.
 */
int ogn_validate_csr(const void* rowptr, const void* col, int index_dtype, int64_t m,
                     int64_t nnz, int64_t n, int32_t* status, void* stream);

/* ------------------------------------------------------------------ SpMM
 * Weighted CSR SpMM, torch_sparse semantics.  Replaces TorchSparseSpmmForward
 * (reference csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:97-135)
 * and its kernels CsrCompute / CsrComputeFour / CsrPrefetchCompute
 * (reference .../op_kernel/arch35/torch_sparse_spmm_kernel.h:37-254).
 *
 *   out[b, r, k] = R_{e in [ptr[r], ptr[r+1])} value[e, (k | 0)] * mat[b, col[e], k]
 *
 * mat: [batch, n, k] of in_dtype (f32/f16/bf16).  value: NULL (all ones), or
 * [nnz] (value_width 1) or [nnz, k] (value_width k), same dtype as mat.
 * out: [batch, m, k] of out_dtype (f32/f16/bf16); arg: [batch, m, k] int64,
 * required for min/max, ignored otherwise.  Arithmetic is fp32 (min/max of
 * fp32 inputs compare exact fp64 products).  min/max ignore NaN products,
 * the first edge wins ties, and an empty or all-NaN row gives 0 / arg = nnz.
 * mean divides by the row length (duplicates included); empty rows give 0.
 * Deterministic: identical inputs give bit-identical outputs.
 */
size_t ogn_spmm_csr_workspace_size(int64_t m, int64_t nnz, int64_t k, int64_t batch,
                                   int in_dtype, int reduce);
int ogn_spmm_csr(const void* rowptr, const void* col, int index_dtype, const void* value,
                 int64_t value_width, const void* mat, int in_dtype, int64_t batch,
                 int64_t m, int64_t n, int64_t k, int64_t nnz, void* out, int out_dtype,
                 int64_t* arg, int reduce, void* workspace, size_t workspace_bytes,
                 void* stream);

/* ------------------------------------------------------------------ index conversion
 * ind2ptr: out[i] = #{ j : ind[j] < i } for i in [0, rows]; `ind` sorted
 * non-decreasing (numel entries).  out: int64 [rows + 1].  numel == 0 gives
 * zeros.  Replaces Ind2Ptr (reference csrc/npu/ind2ptr/op_kernel/arch35/ind2ptr.cpp:146)
 * and the ind2ptr half of TorchSparseSpmmConvert
 * (reference csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:170-184).
 */
int ogn_ind2ptr(const void* ind, int index_dtype, int64_t numel, int64_t rows, int64_t* out,
                void* stream);
/* ptr2ind: out[e] = r with ptr[r] <= e < ptr[r+1], e in [0, numel); ptr has
 * rows + 1 entries.  out: int64 [numel], 16-byte aligned.  Replaces Ptr2Ind
 * (reference csrc/npu/ptr2ind/op_kernel/arch35/ptr2ind.cpp:56).
 */
int ogn_ptr2ind(const void* ptr, int index_dtype, int64_t rows, int64_t numel, int64_t* out,
                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OGN_H_ */
