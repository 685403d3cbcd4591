// CSR SpMM (torch_sparse semantics): the CSR engine in column-gather mode.
#include "csr_engine.h"

#include <mutex>
#include <string>

using namespace ogn;
using namespace ogn::eng;

// Engine workspace of ogn_spmm_csr_noalloc: a file-scope device array, one
// copy per GPU.  Host code never passes `scratch` itself to a kernel (in
// host code the name is a stand-in, not a device address); it passes the
// address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[OGN_SPMM_NOALLOC_SCRATCH_BYTES];

namespace {
bool is_aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// Device address of the current device's `scratch`, looked up once per
// device (with that device current) and kept.
int scratch_address(void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(OGN_EHIP, std::string("ogn_spmm_csr_noalloc: hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(OGN_EUNSUPPORTED, "ogn_spmm_csr_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(OGN_EHIP, std::string("ogn_spmm_csr_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return OGN_OK;
}
}  // namespace

extern "C" {

size_t ogn_spmm_csr_workspace_size(int64_t m, int64_t nnz, int64_t k, int64_t batch, int in_dtype,
                                   int reduce) {
  (void)m;
  if (nnz < 0 || k <= 0 || batch <= 0) return 0;
  const int rk = (reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX) ? RK_MINMAX : RK_SUM;
  const Plan pa = make_plan(nnz, k, in_dtype, true, true);
  const Plan pu = make_plan(nnz, k, in_dtype, false, true);
  return std::max(workspace_layout(pa, k, batch, 1, rk).total, workspace_layout(pu, k, batch, 1, rk).total);
}

static int spmm_impl(const void* rowptr, const void* col, int index_dtype, const void* value, int64_t value_width,
                     const void* mat, int in_dtype, int64_t batch, int64_t m, int64_t n, int64_t k, int64_t nnz,
                     void* out, int out_dtype, int64_t* arg, int reduce, int message_op, int semantics,
                     void* workspace, size_t workspace_bytes, void* stream);

int ogn_spmm_csr(const void* rowptr, const void* col, int index_dtype, const void* value,
                 int64_t value_width, const void* mat, int in_dtype, int64_t batch, int64_t m,
                 int64_t n, int64_t k, int64_t nnz, void* out, int out_dtype, int64_t* arg,
                 int reduce, void* workspace, size_t workspace_bytes, void* stream) {
  return spmm_impl(rowptr, col, index_dtype, value, value_width, mat, in_dtype, batch, m, n, k, nnz, out,
                   out_dtype, arg, reduce, OGN_MSG_MUL, OGN_SPMM_TORCH_SPARSE, workspace, workspace_bytes,
                   stream);
}

int ogn_spmm_csr_ex(const void* rowptr, const void* col, int index_dtype, const void* value,
                    int64_t value_width, const void* mat, int in_dtype, int64_t batch, int64_t m,
                    int64_t n, int64_t k, int64_t nnz, void* out, int out_dtype, int64_t* arg,
                    int reduce, int message_op, int semantics, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (message_op < OGN_MSG_MUL || message_op > OGN_MSG_DIV)
    return fail(OGN_EINVAL, "ogn_spmm_csr_ex: unknown message op");
  if (semantics != OGN_SPMM_TORCH_SPARSE && semantics != OGN_SPMM_DGL)
    return fail(OGN_EINVAL, "ogn_spmm_csr_ex: unknown semantics");
  return spmm_impl(rowptr, col, index_dtype, value, value_width, mat, in_dtype, batch, m, n, k, nnz, out,
                   out_dtype, arg, reduce, message_op, semantics, workspace, workspace_bytes, stream);
}

int ogn_spmm_csr_noalloc(const void* rowptr, const void* col, int index_dtype, const void* value,
                         int64_t value_width, const void* mat, int in_dtype, int64_t batch, int64_t m,
                         int64_t n, int64_t k, int64_t nnz, void* out, int out_dtype, int64_t* arg,
                         int reduce, void* stream) {
  const size_t need = ogn_spmm_csr_workspace_size(m, nnz, k, batch, in_dtype, reduce);
  if (need > OGN_SPMM_NOALLOC_SCRATCH_BYTES)
    return fail(OGN_EINVAL, "ogn_spmm_csr_noalloc: this call needs " + std::to_string(need) +
                                " bytes of scratch, above the maximum of " +
                                std::to_string(OGN_SPMM_NOALLOC_SCRATCH_BYTES) +
                                "; use ogn_spmm_csr with a caller workspace");
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != OGN_OK) return rc;
  return spmm_impl(rowptr, col, index_dtype, value, value_width, mat, in_dtype, batch, m, n, k, nnz, out,
                   out_dtype, arg, reduce, OGN_MSG_MUL, OGN_SPMM_TORCH_SPARSE, ws, OGN_SPMM_NOALLOC_SCRATCH_BYTES,
                   stream);
}

}  // extern "C"

static int spmm_impl(const void* rowptr, const void* col, int index_dtype, const void* value,
                 int64_t value_width, const void* mat, int in_dtype, int64_t batch, int64_t m,
                 int64_t n, int64_t k, int64_t nnz, void* out, int out_dtype, int64_t* arg,
                 int reduce, int message_op, int semantics, void* workspace, size_t workspace_bytes,
                 void* stream) {
  if (m < 0 || n < 0 || k < 0 || nnz < 0 || batch < 0)
    return fail(OGN_EINVAL, "ogn_spmm_csr: negative size");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_spmm_csr: index dtype must be int32 or int64");
  // Input -> output dtype table of the reference (torch_sparse_spmm.cpp:88-90):
  // f32 -> f32; f16 -> f32|f16; bf16 -> f32|bf16; int8 -> f32|int32.
  if (in_dtype != OGN_F32 && in_dtype != OGN_F16 && in_dtype != OGN_BF16 && in_dtype != OGN_I8)
    return fail(OGN_EUNSUPPORTED, "ogn_spmm_csr: mat dtype must be float32, float16, bfloat16 or int8");
  if (!(out_dtype == OGN_F32 || (in_dtype == OGN_I8 ? out_dtype == OGN_I32 : out_dtype == in_dtype)))
    return fail(OGN_EUNSUPPORTED, "ogn_spmm_csr: unsupported input/output dtype combination");
  if (in_dtype == OGN_I8 && (message_op != OGN_MSG_MUL || semantics != OGN_SPMM_TORCH_SPARSE))
    return fail(OGN_EUNSUPPORTED, "ogn_spmm_csr: int8 supports torch_sparse x * w messages only");
  if (reduce < OGN_REDUCE_SUM || reduce > OGN_REDUCE_MAX)
    return fail(OGN_EINVAL, "ogn_spmm_csr: reduce must be sum/mean/min/max");
  const bool mm = reduce >= OGN_REDUCE_MIN;
  if (m == 0 || k == 0 || batch == 0) return OGN_OK;
  if (!rowptr || !out || (mm && !arg && semantics == OGN_SPMM_TORCH_SPARSE))
    return fail(OGN_EINVAL, "ogn_spmm_csr: null pointer");
  if (nnz > 0 && (!col || !mat || n == 0))
    return fail(OGN_EINVAL, "ogn_spmm_csr: nnz > 0 needs col, mat and n > 0");
  if (value && value_width != 1 && value_width != k)
    return fail(OGN_EINVAL, "ogn_spmm_csr: value width must be 1 or k");

  const bool aligned = is_aligned(mat, 16) && is_aligned(out, 16) &&
                       (!value || value_width == 1 || is_aligned(value, 16));
  const Plan pl = make_plan(nnz, k, in_dtype, aligned, true);
  Params p{};
  p.ptr = rowptr;
  p.ptr_bstride = 0;
  p.col = col;
  p.val = value;
  p.val_mode = value == nullptr ? 0 : (value_width == 1 ? 1 : 2);
  p.src = mat;
  p.src_dt = in_dtype;
  p.src_bstride = n * k;
  p.out = out;
  p.out_dt = out_dtype;
  p.out_bstride = m * k;
  p.arg = arg;
  p.m = m;
  p.n = std::max<int64_t>(n, 1);
  p.k = k;
  p.nnz_bound = nnz;
  p.reduce = reduce;
  p.val_op = message_op;
  p.mm_mode = semantics == OGN_SPMM_DGL ? MM_NANPROP : MM_SPMM;
  p.seed_mode = SEED_NONE;
  p.arg_empty = nnz;
  return run(pl, p, in_dtype, index_dtype, true, mm ? RK_MINMAX : RK_SUM, batch, workspace,
             workspace_bytes, static_cast<hipStream_t>(stream), "spmm");
}


