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
  OGN_U8 = 7,
  OGN_I16 = 8
} ogn_dtype;

typedef enum {
  OGN_REDUCE_SUM = 0,
  OGN_REDUCE_MEAN = 1,
  OGN_REDUCE_MIN = 2,
  OGN_REDUCE_MAX = 3,
  OGN_REDUCE_PROD = 4, /* scatter "mul" */
  OGN_REDUCE_LSE = 5   /* log-sum-exp */
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
 * mat: [batch, n, k] of in_dtype (f32/f16/bf16, or i8).  value: NULL (all
 * ones), or [nnz] (value_width 1) or [nnz, k] (value_width k), same dtype as
 * mat.  out: [batch, m, k] of out_dtype, by the reference's table
 * (torch_sparse_spmm.cpp:88-90): f32 -> f32; f16 -> f32 | f16;
 * bf16 -> f32 | bf16; i8 -> i32 | f32.  i8 sums accumulate exactly in int32;
 * an i32 mean truncates toward zero, an f32 mean is the exact quotient
 * rounded once.  Other pairs return OGN_EUNSUPPORTED.  arg: [batch, m, k] int64,
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

/* ogn_spmm_csr without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The engine
 * workspace is a library-owned device array of OGN_SPMM_NOALLOC_SCRATCH_BYTES
 * (128 MiB), one per GPU, held until the process ends; the call uses the
 * array of the current device (hipGetDevice), which must be the device of
 * `stream` and of the operands.  A call whose ogn_spmm_csr_workspace_size()
 * exceeds the maximum returns OGN_EINVAL and launches nothing (config-3 sized
 * fp32 / bf16 sums fit; min/max at that size do not).  Nothing here calls
 * hipMalloc / hipFree.  Every call on a GPU shares that GPU's array: calls
 * that overlap on one GPU (several streams or host threads) race and must
 * be serialised by the caller.  The array needs no clearing: every entry a
 * call reads was written earlier in the same call.  Results are bitwise
 * those of ogn_spmm_csr.
 */
#define OGN_SPMM_NOALLOC_SCRATCH_BYTES ((size_t)134217728)
int ogn_spmm_csr_noalloc(const void* rowptr, const void* col, int index_dtype, const void* value,
                         int64_t value_width, const void* mat, int in_dtype, int64_t batch,
                         int64_t m, int64_t n, int64_t k, int64_t nnz, void* out, int out_dtype,
                         int64_t* arg, int reduce, void* stream);

/* Generalised CSR aggregation (DGL-style spmm / bspmm):
 *   out[b, r, k] = R_{e in row r} msg(mat[b, col[e], k], value[e, (k | 0)])
 * msg: OGN_MSG_MUL (x * w; w = 1 without value), OGN_MSG_ADD (x + w),
 * OGN_MSG_SUB (x - w), OGN_MSG_DIV (x / w).
 * semantics: OGN_SPMM_TORCH_SPARSE (as ogn_spmm_csr) or OGN_SPMM_DGL
 * (reference python/ops_gnn/spmm.py:148-208, csrc/npu/common/spmm/spmm_utils.h:389-406:
 * min/max propagate NaN -- a row holding a NaN message gives NaN -- empty rows
 * give 0, and arg may be NULL).  Replaces RunSpmmCopyLhs / UnifiedSpmmCsr
 * (reference csrc/npu/common/spmm/spmm_utils.h:188-204,
 * csrc/npu/unified_spmm/op_host/unified_spmm.cpp:116-158) and the torch
 * composition for binary messages (python/ops_gnn/spmm.py:148-208); fp16
 * accumulates in fp32.  Workspace: ogn_spmm_csr_workspace_size(). */
enum { OGN_MSG_MUL = 0, OGN_MSG_ADD = 1, OGN_MSG_SUB = 2, OGN_MSG_DIV = 3 };
enum { OGN_SPMM_TORCH_SPARSE = 0, OGN_SPMM_DGL = 1 };
int ogn_spmm_csr_ex(const void* rowptr, const void* col, int index_dtype, const void* value,
                    int64_t value_width, const void* mat, int in_dtype, int64_t batch, int64_t m,
                    int64_t n, int64_t k, int64_t nnz, void* out, int out_dtype, int64_t* arg,
                    int reduce, int message_op, int semantics, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ------------------------------------------------------------------ SDDMM
 * out[e] = phi(lhs[t_l(e)], rhs[t_r(e)]) on a CSR graph (reference
 * SddmmCsrForward csrc/npu/sddmm_csr/op_host/sddmm_csr.cpp:415-461, golden
 * test/sddmm_csr/arch22/golden.py:74-90).  Targets: 0 = row of e (src),
 * 1 = e (edge), 2 = col[e] (dst).  lhs [lhs_rows, k], rhs [rhs_rows, k],
 * both of `dtype` (f32/f16/bf16).  op: OGN_SDDMM_DOT -> out [nnz] (feature
 * reduction), ADD/SUB/MUL/DIV -> out [nnz, k], COPY_LHS / COPY_RHS -> the
 * gathered operand [nnz, k] (the unused operand may be NULL).  fp32 compute,
 * one rounding to dtype.  Workspace: ogn_sddmm_csr_workspace_size(). */
enum { OGN_SDDMM_DOT = 0, OGN_SDDMM_ADD = 1, OGN_SDDMM_SUB = 2, OGN_SDDMM_MUL = 3, OGN_SDDMM_DIV = 4,
       OGN_SDDMM_COPY_LHS = 5, OGN_SDDMM_COPY_RHS = 6 };
size_t ogn_sddmm_csr_workspace_size(int64_t nnz, int64_t k, int dtype);
int ogn_sddmm_csr(const void* rowptr, const void* col, int index_dtype, int64_t m, int64_t nnz,
                  const void* lhs, int64_t lhs_rows, int lhs_target, const void* rhs, int64_t rhs_rows,
                  int rhs_target, int64_t k, int dtype, int op, void* out, void* workspace,
                  size_t workspace_bytes, void* stream);

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

/* ------------------------------------------------------------------ segment reductions
 * Reductions over runs of consecutive rows.  src is viewed as
 * [batch, length, k] (batch = product of the dims before the reduction dim,
 * k = product of the dims after it); out / arg as [batch, segments, k].
 * indptr: int64 [ptr_batches, segments + 1], ptr_batches 1 (shared by every
 * batch) or `batch`; non-decreasing, within [0, length].  Segment s covers
 * rows [indptr[s], indptr[s+1]); rows outside [indptr[0], indptr[segments])
 * are ignored.  dtype: f32 / f16 / bf16 for src and out, arithmetic in fp32;
 * or an exact dtype (int8, uint8, int16, int32, int64, float64): sums and
 * products wrap in the dtype, min/max compare exactly, and the integer mean
 * follows each operator's rule (segment_csr: narrow(sum) / narrow(count)
 * truncating, 0 for a zero narrowed count; segment_coo: the same with the
 * exact mean for a zero narrowed count; scatter: floor division by the count,
 * narrowed and clamped to >= 1 for 8/16-bit types).  Exact dtypes support
 * sum, mean, min, max (and prod for scatter).  For the integer dtypes the
 * workspace holds partial results of segments longer than 4096 rows, folded
 * in parallel pieces; with a smaller workspace (or none) such segments are
 * folded by one thread per feature packet, with the same result.  float64
 * needs no workspace (its sums keep the serial order).
 * reduce: sum, mean, min, max, prod, lse.  arg (int64, optional, min/max
 * only) gets positions along the reduction dim.
 *
 * semantics selects the reference operator whose rules apply:
 *  OGN_SEM_SEGMENT_CSR -- segment_csr (reference test/segment_csr/arch35/golden.py:21-103,
 *    csrc/npu/segment_csr/op_kernel/arch35/segment_csr.cpp:506-640): out is
 *    overwritten; min/max start from +-inf and move on strict improvement
 *    (first extremum wins, NaN never enters, an all-NaN segment gives +-inf
 *    with arg = its first row); empty segments give 0 / arg = length.
 *  OGN_SEM_SEGMENT_COO -- Ascend 950 segment_coo (reference
 *    csrc/npu/segment_coo/op_kernel/arch35/segment_coo.cpp:114-153): sum
 *    overwrites; mean adds to out when OGN_SEG_HAS_OUT; min/max fold with
 *    <= / >= from the seed (out with arg = length if OGN_SEG_HAS_OUT, else
 *    the segment's first row), so the LAST extremum wins.
 *  OGN_SEM_SCATTER -- torch_scatter scatter on a sorted index (reference
 *    test/scatter/arch35/golden.py:35-127): sum/mean/prod accumulate into out
 *    when OGN_SEG_HAS_OUT (else start from 0 / 1); mean divides by the count
 *    (empty: out unchanged); min/max fold with <= / >= from out (or from the
 *    dtype's finite extreme, a position never written giving 0), last
 *    extremum wins, arg = length when nothing was taken.
 *  OGN_SEM_DGL -- DGL copy_rhs aggregation (reference python/ops_gnn/spmm.py:165-208):
 *    min/max propagate NaN, empty segments give 0.
 *  reduce = lse gives log(sum(exp(x))) with the shift clamped to +-FLT_MAX
 *    (reference csrc/npu/segment_logsumexp/op_kernel/common/segment_logsumexp_kernel.h:10-45);
 *    empty segments give -inf.
 * Replaces the segment_csr / segment_coo / segment_logsumexp host+kernel
 * pairs (reference csrc/npu/segment_csr/op_host/segment_csr.cpp:1663-1702,
 * csrc/npu/segment_coo/op_host/segment_coo.cpp:1127-1175).
 */
enum { OGN_SEM_SEGMENT_CSR = 0, OGN_SEM_SEGMENT_COO = 1, OGN_SEM_SCATTER = 2, OGN_SEM_DGL = 3 };
/* flags:
 *  OGN_SEG_HAS_OUT -- out holds seeds (see semantics above).
 *  OGN_SEG_SHORT_SEGMENTS -- the caller knows that no segment holds more
 *    than 4096 rows; the pass that pre-folds the partial results of segments
 *    spanning many wavefront chunks (integer dtypes: the piece pass) is then
 *    not launched.
 *  OGN_SEG_KEEP_LAYOUT -- the caller keeps `workspace` for later calls with
 *    the same indptr (same address, same contents) on the same stream; the
 *    library records which pointer array and chunk plan the workspace's
 *    chunk layout (row of every chunk's first position, rows crossing chunk
 *    ends) was computed for.
 *  OGN_SEG_REUSE_LAYOUT -- `workspace` was last used with KEEP or REUSE for
 *    this indptr, whose contents have not changed since: the chunk-row pass
 *    is skipped when the recorded pointer address and plan match this call
 *    (otherwise the layout is recomputed and recorded).  The rest of the
 *    workspace is rewritten by every call, so calls sharing one workspace
 *    must not overlap.
 * No counterpart in the reference (its host tiling is recomputed per call);
 * they serve callers that run one graph many times. */
enum { OGN_SEG_HAS_OUT = 1, OGN_SEG_SHORT_SEGMENTS = 2, OGN_SEG_KEEP_LAYOUT = 4, OGN_SEG_REUSE_LAYOUT = 8 };
size_t ogn_segment_reduce_workspace_size(int64_t batch, int64_t length, int64_t segments, int64_t k,
                                         int64_t ptr_batches, int dtype, int reduce);
int ogn_segment_reduce(const int64_t* indptr, int64_t ptr_batches, const void* src, int dtype,
                       int64_t batch, int64_t length, int64_t segments, int64_t k, void* out,
                       int64_t* arg, int reduce, int semantics, int flags, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ogn_segment_reduce over rows read through an index: position i of the
 * segments (indptr, int64 [segments + 1], as ogn_segment_reduce with one
 * batch) is row rows[i] of src [src_rows, k]; torch_scatter semantics only
 * (OGN_SEM_SCATTER: flags OGN_SEG_HAS_OUT seeds from out; min/max take the
 * LATER position on ties, in `rows` order), float32 / float16 / bfloat16,
 * reduce sum, mean, min, max or prod.  arg (optional, min/max) gets the src
 * row of each winner (rows[i]), src_rows when nothing was taken.  The
 * unsorted scatter sorts its index stably (ogn_sort_rows) and reduces here,
 * so that every output row is folded by one wavefront schedule instead of
 * contended atomics (reference scatter_kernel_atomic.h:338-412 and the arg
 * pass scatter_kernel_minmax.h:120-175 for the same operation).  Workspace:
 * ogn_segment_reduce_gather_workspace_size. */
size_t ogn_segment_reduce_gather_workspace_size(int64_t length, int64_t segments, int64_t k, int dtype,
                                                int reduce);
int ogn_segment_reduce_gather(const int64_t* indptr, const int64_t* rows, const void* src, int dtype,
                              int64_t src_rows, int64_t length, int64_t segments, int64_t k, void* out,
                              int64_t* arg, int reduce, int semantics, int flags, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ogn_segment_group_stats over rows read through an index (one batch):
 * position i of the groups (indptr [segments + 1]) is row rows[i] of src
 * [src_rows, k].  The grouped softmax / logsumexp over an unsorted index
 * sort it (ogn_sort_rows) and take their statistics here instead of with
 * contended atomics.  Workspace: ogn_segment_reduce_gather_workspace_size
 * with reduce = OGN_REDUCE_LSE. */
int ogn_segment_group_stats_gather(const int64_t* indptr, const int64_t* rows, const void* src, int dtype,
                                   int64_t src_rows, int64_t length, int64_t segments, int64_t k, float* m_out,
                                   float* s_out, void* workspace, size_t workspace_bytes, void* stream);

/* Batched ind2ptr over int64 sorted indices: ind [batches, numel] ->
 * out [batches, rows + 1].  Used to turn a sorted COO index into segment
 * pointers (reference segment_coo BuildPointers,
 * csrc/npu/segment_coo/op_kernel/arch35/segment_coo.cpp:67-82). */
int ogn_ind2ptr_batched(const int64_t* ind, int64_t batches, int64_t numel, int64_t rows, int64_t* out,
                        void* stream);

/* Facts about an int64 index (device memory, 3 x int64): facts[0] = 1 if
 * not non-decreasing, facts[1] = min, facts[2] = max (INT64_MAX / INT64_MIN
 * when empty).  Replaces the cached index min/max probe of the reference
 * scatter (python/ops_gnn/scatter.py:134-178). */
int ogn_index_facts(const int64_t* ind, int64_t numel, int64_t* facts, void* stream);

/* Stable sort of n int64 keys known to lie in [0, max_key] (max_key below
 * 2^32, n below 2^31): perm[i] = position of the i-th smallest key, equal keys
 * in position order; sorted_keys (optional, may be NULL) = the keys in that
 * order; up to two companion arrays a, b (elements of a_bytes / b_bytes = 4
 * or 8 bytes; 0 = none; b only with a) permuted alike: a_out[i] =
 * a[perm[i]].  The COO -> CSR and CSR -> CSC permutation step (reference
 * python/ops_gnn/torch_sparse_spmm.py:273-342: a stable argsort, then the
 * columns and values indexed by it).  Radix sort over the
 * ceil(log2(max_key + 1)) low key bits with 32-bit keys; the companions
 * travel with the positions through the sort's passes.  The workspace
 * (ogn_sort_rows_workspace_size with the same sizes and companion widths: 0
 * when they are out of range or no GPU answers the query) holds the keys,
 * the records and the sort's temporary storage.  Not capturable in a HIP
 * graph. */
size_t ogn_sort_rows_workspace_size(int64_t n, int64_t max_key, int a_bytes, int b_bytes);
int ogn_sort_rows(const int64_t* keys, int64_t n, int64_t max_key, int64_t* sorted_keys, int64_t* perm,
                  const void* a, void* a_out, int a_bytes, const void* b, void* b_out, int b_bytes,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Log-sum-exp statistics of sorted groups (contiguous segments, shared
 * indptr [segments + 1]): m_out[b, g, f] = max (unclamped; -inf for an empty
 * group) and s_out[b, g, f] = sum(exp(x - clamp(max, +-FLT_MAX))), both fp32.
 * Workspace: ogn_segment_reduce_workspace_size(batch, length, segments, k, 1,
 * dtype, OGN_REDUCE_LSE).  First pass of scatter_softmax / scatter_log_softmax
 * on a sorted index (reference csrc/npu/scatter_softmax/common/grouped_softmax_shared.h:178-209
 * phases 1-2). */
int ogn_segment_group_stats(const int64_t* indptr, const void* src, int dtype, int64_t batch, int64_t length,
                            int64_t segments, int64_t k, float* m_out, float* s_out, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Fused softmax (log_softmax = 0) or log_softmax (1) of one-feature rows:
 * src / out [batch, length] (the per-edge score layout, after = 1), row r of
 * every batch = positions [indptr[r], indptr[r+1]) (shared indptr
 * [segments + 1]).  out = exp(x - clamp(m)) / s or (x - clamp(m)) - log(s)
 * with (m, s) as ogn_segment_group_stats; a row holding +inf is NaN
 * throughout.  Positions outside [indptr[0], indptr[segments]) are not
 * written.  One wavefront per row of up to 2048 (fp16 / bf16) or 1024 (fp32)
 * positions, a 256-thread block per longer row: meant for rows of >= ~64
 * positions on average.  src and out 16-byte aligned, and length * element
 * size a multiple of 16 when batch > 1.  Workspace (256-byte aligned, its
 * contents need no initialisation): the long-row list and a row plan,
 * ogn_segment_group_softmax_workspace_size() bytes.  flags: with
 * OGN_SEG_KEEP_LAYOUT (or REUSE without a kept plan) the call also bins the
 * rows by length into the workspace (a plan for later calls; this call then
 * waits for a 64-byte read of the bin counts); with OGN_SEG_REUSE_LAYOUT and a
 * plan kept for this workspace, indptr address and shape, short rows share
 * wavefronts (8, 16 or 32 lanes per row) and the rows run largest first.
 * Calls sharing a kept workspace must not overlap; indptr must be unchanged
 * since the plan was built.  ABI 3 added `flags`.  Fuses the sorted-index
 * forward phases of scatter_softmax / scatter_log_softmax (reference
 * csrc/npu/scatter_softmax/common/grouped_softmax_shared.h:178-209). */
size_t ogn_segment_group_softmax_workspace_size(int64_t batch, int64_t length, int64_t segments, int dtype);
int ogn_segment_group_softmax(const int64_t* indptr, const void* src, int dtype, int64_t batch, int64_t length,
                              int64_t segments, void* out, int log_softmax, int flags, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ unsorted scatter
 * torch_scatter scatter with an arbitrary int64 index (same rules as
 * OGN_SEM_SCATTER above).  src: [before, len, after] contiguous; index read
 * at b*index_stride_before + l*index_stride_len + f*index_stride_after
 * (strides in elements, 0 = broadcast); out/arg: [before, size, after]; when
 * has_out, out holds the starting values.  reduce: sum, mean, min, max,
 * prod.  arg (int64) is required for min/max.  Entries of index outside
 * [0, size) are skipped.  dtype: f32 / f16 / bf16 (fp32 atomics: sum/mean/prod
 * order may vary between runs; min/max and arg are exact), int8 / uint8 /
 * int16 / int32 / int64 (64-bit integer atomics: every result exact and
 * order-independent) or float64 (sum/prod order may vary).  Replaces scatter_forward
 * (reference csrc/npu/scatter/op_host/scatter.cpp:242-269) and its atomic and
 * min/max kernels (csrc/npu/scatter/op_kernel/arch35/scatter_kernel_atomic.h:338-412,
 * scatter_kernel_minmax.h:120-175). */
size_t ogn_scatter_atomic_workspace_size(int64_t before, int64_t size, int64_t after, int reduce);
int ogn_scatter_atomic(const void* src, int dtype, const int64_t* index, int64_t index_stride_before,
                       int64_t index_stride_len, int64_t index_stride_after, int64_t before, int64_t len,
                       int64_t after, int64_t size, void* out, int64_t* arg, int reduce, int has_out,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ grouped softmax
 * Groups = positions l along the reduction dim sharing index[l] (1-D int32 or
 * int64 index of length len); src/out [before, len, after].
 * ogn_group_stats_atomic: m/s statistics as ogn_segment_group_stats for an
 *   unsorted index, with atomics (m, s: [before, groups, after] fp32;
 *   scratch_key: same size, uint32).
 * ogn_group_softmax_apply: out = exp(x - m') / s (softmax) or
 *   (x - m') - log(s) (log_softmax), m' = clamp(m, +-FLT_MAX); NaN for a group
 *   holding +inf; positions whose index is outside [0, groups) get 0.
 * ogn_group_lse_from_stats: out = m' + log(s) over `cells` entries.
 * Replace the three-phase RunForward of the reference
 * (csrc/npu/scatter_softmax/common/grouped_softmax_shared.h:178-209,
 * csrc/npu/scatter_logsumexp/common/grouped_logsumexp_shared.h:50-90). */
int ogn_group_stats_atomic(const void* src, int dtype, const void* index, int index_dtype, int64_t before,
                           int64_t len, int64_t after, int64_t groups, float* m, float* s, uint32_t* scratch_key,
                           void* stream);
int ogn_group_softmax_apply(const void* src, int dtype, const void* index, int index_dtype, int64_t before,
                            int64_t len, int64_t after, int64_t groups, const float* m, const float* s,
                            void* out, int log_softmax, void* stream);
int ogn_group_lse_from_stats(const float* m, const float* s, int64_t cells, void* out, int dtype, void* stream);

/* Backward of the grouped softmax family (reference RunBackward,
 * csrc/npu/scatter_softmax/common/grouped_softmax_shared.h:212-250 and
 * csrc/npu/scatter_logsumexp/common/grouped_logsumexp_shared.h:92-136; Python
 * python/ops_gnn/_grouped_softmax.py:122-133, scatter_logsumexp.py:78-84).
 *  mode 0 softmax:     grad_src = out * (g - T),      T = group sum of out * g
 *  mode 1 log_softmax: grad_src = g - exp(out) * T,   T = group sum of g
 *    saved = forward output, grad = its gradient, both [before, len, after];
 *    workspace: before * groups * after fp32 (cleared by the call).
 *  mode 2 logsumexp:   grad_src = g[group] * exp(x - out[group])
 *    saved = forward src [before, len, after], reduced = forward output and
 *    grad = its gradient, both [before, groups, after]; no workspace.
 * Positions whose index is outside [0, groups) get 0.  fp32 math; group sums
 * use atomics (one per run of equal targets in a wavefront), unless mode
 * carries OGN_GROUP_BWD_TOTALS_GIVEN: the workspace then already holds the
 * group sums T (the unsorted-index path computes them without atomics:
 * ogn_group_bwd_messages, then ogn_segment_reduce_gather over the index's
 * sort permutation) and only the elementwise pass runs. */
enum { OGN_GROUP_BWD_TOTALS_GIVEN = 4 };
int ogn_group_softmax_backward(const void* saved, const void* grad, const void* reduced, int dtype,
                               const void* index, int index_dtype, int64_t before, int64_t len, int64_t after,
                               int64_t groups, int mode, void* grad_src, float* workspace, size_t workspace_bytes,
                               void* stream);
/* The terms T sums, per position, in fp32: msg[i] = saved[i] * grad[i]
 * (mode 0) or grad[i] (mode 1), n elements.  No counterpart in the
 * reference (its sums are fused atomics). */
int ogn_group_bwd_messages(const void* saved, const void* grad, int dtype, int64_t n, int mode, float* msg,
                           void* stream);

/* ------------------------------------------------------------------ gather
 * Expansion of segment rows (raw bytes: any dtype, bit-exact).
 * ogn_gather_csr: out[b, i, :] = src[b, s, :] for indptr[s] <= i < indptr[s+1]
 *   (the last such s); rows before indptr[0] are zero.  indptr: int64
 *   [ptr_batches, segments + 1], ptr_batches 1 (shared) or batch, each row
 *   non-decreasing and ending at out_rows.  src [batch, segments, row_bytes],
 *   out [batch, out_rows, row_bytes].  Replaces gather_csr (reference
 *   csrc/npu/gather_csr/op_host/gather_csr.cpp:338, golden
 *   test/gather_csr/arch35/golden.py:63-90).
 * ogn_gather_coo: out[b, e, :] = src[b, index[b, e], :]; index int64
 *   [batch, entries], values clamped into [0, src_rows).  Replaces gather_coo
 *   (reference csrc/npu/gather_coo/op_host/gather_coo.cpp, golden
 *   test/gather_coo/arch35/test_gather_coo.py:87-106). */
int ogn_gather_csr(const int64_t* indptr, int64_t ptr_batches, const void* src, int64_t batch, int64_t segments,
                   int64_t row_bytes, int64_t out_rows, void* out, void* stream);
int ogn_gather_coo(const int64_t* index, const void* src, int64_t batch, int64_t src_rows, int64_t entries,
                   int64_t row_bytes, void* out, void* stream);

/* ------------------------------------------------------------------ XCD tiles
 * Column-tiled SDDMM dot and SpMM sum, for graphs whose gathered feature
 * table is larger than one XCD's 4 MB L2 but small enough that an eighth of
 * it fits (the 29.8 MB K / V of an attention layer).  Workgroup b runs on XCD
 * b % 8 and gathers only columns of tile b % 8, so its rows stay in that
 * XCD's L2.  No counterpart in the reference (its kernels have no cache
 * tiers to target); results: SDDMM bit-identical to ogn_sddmm_csr's dot, SpMM
 * the same sum in another order (per-tile fp32 partials, added in tile
 * order: deterministic).
 * ogn_xcd_plan: builds the plan of (rowptr, col) into `plan`
 *   (ogn_xcd_plan_bytes bytes): row-aligned chunks of about 8192 edges and,
 *   for every row, where each of 8 column tiles (n_cols / 8 columns wide)
 *   starts in its edge range.  *sorted (the plan state) = 0 when a row's
 *   columns are not sorted (the tiles then do not follow column ranges; the
 *   results are right either way), 1 when they are, 2 when they are and
 *   n_cols <= 2^19, so that the plan also holds every column as a 16-bit
 *   offset from its tile's first column (2 bytes per edge streamed instead
 *   of the index).  Waits for a 4-byte read.  Fewer than 2^31 edges.
 * The run functions take that state as plan_state (2: read the 16-bit
 *   columns, which needs rhs_rows / n equal to the plan's n_cols; else col).
 * ogn_sddmm_dot_xcd: out[e] = dot(lhs[row(e)], rhs[col[e]]) (lhs_target =
 *   row, rhs_target = col), k * element size 64, 128, 256 or 512 bytes.
 * ogn_spmm_sum_xcd: out[r] = sum_e value[e] * mat[col[e]] (one weight per
 *   edge, batch 1), out dtype = mat dtype or float32; workspace
 *   ogn_spmm_sum_xcd_workspace_size(m, k) bytes (8 fp32 partial outputs). */
size_t ogn_xcd_plan_bytes(int64_t m, int64_t nnz);
int ogn_xcd_plan(const void* rowptr, const void* col, int index_dtype, int64_t m, int64_t n_cols, int64_t nnz,
                 void* plan, size_t plan_bytes, int* sorted, void* stream);
int ogn_sddmm_dot_xcd(const void* plan, int64_t m, int64_t nnz, const void* col, int index_dtype, const void* lhs,
                      int64_t lhs_rows, const void* rhs, int64_t rhs_rows, int64_t k, int dtype, void* out,
                      int plan_state, void* stream);
size_t ogn_spmm_sum_xcd_workspace_size(int64_t m, int64_t k);
int ogn_spmm_sum_xcd(const void* plan, int64_t m, int64_t nnz, const void* col, int index_dtype, const void* value,
                     const void* mat, int64_t n, int64_t k, int dtype, void* out, int out_dtype, void* workspace,
                     size_t workspace_bytes, int plan_state, void* stream);

/* ------------------------------------------------------------------ measurement
 * Practical memory ceilings, reported by bench.py beside the 8 TB/s HBM
 * peak.  No counterpart in the reference; they serve measurement only.
 * ogn_calibrate_gather: reads table rows index[0 .. n) (row_bytes each, 16 *
 *   a power of two up to 1024; table 16-byte aligned, below 4 GiB; indices
 *   clamped into [0, rows)) exactly as a gathering kernel would, and nothing
 *   else: the time floor of any kernel gathering those rows.
 * ogn_calibrate_stream: streaming copy of `bytes` (a multiple of 16) from
 *   src to dst, or a streaming read of src when dst is NULL.
 * sink: one 4-byte device word, written only under a condition that never
 * holds (it keeps the loads live). */
int ogn_calibrate_gather(const void* table, int64_t rows, int64_t row_bytes, const int64_t* index, int64_t n,
                         void* sink, void* stream);
int ogn_calibrate_stream(const void* src, void* dst, int64_t bytes, void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OGN_H_ */
