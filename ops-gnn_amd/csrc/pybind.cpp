// ops_gnn._pybind -- the PyTorch-ROCm extension over the C ABI (include/ogn.h).
//
// Replaces the reference's pybind module (reference csrc/pybind.cpp:92-349):
// tensor in, tensor out, outputs allocated with torch's caching allocator,
// every launch on torch's current HIP stream of the operand's device, taken
// after the contiguity copies (reference torch_sparse_spmm.cpp:127-129).
// Every binding releases the GIL while it runs (py::call_guard).  The module holds no state:
// proof caches stay in the Python layer.  Host code only -- every kernel is
// in libogn_hip.so.
#include <torch/extension.h>

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <optional>
#include <tuple>

#include "../../include/ogn.h"

namespace {

using at::Tensor;

void* stream_of(const Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void ok(int rc, const char* what) {
  TORCH_CHECK(rc == OGN_OK, what, ": ", ogn_last_error());
}

void on_gpu(const Tensor& t, const char* name) {
  TORCH_CHECK(t.defined() && t.is_cuda(), name, " must be a GPU tensor");
}

int index_code(const Tensor& t) {
  TORCH_CHECK(t.scalar_type() == at::kLong || t.scalar_type() == at::kInt,
              "index tensors must be int32 or int64");
  return t.scalar_type() == at::kLong ? OGN_I64 : OGN_I32;
}

// Output-type codes of the reference (python/ops_gnn/torch_sparse_spmm.py:28):
// float32 0, float16 1, bfloat16 2, int8 3, int32 4 -- the same numbers as
// the library's ogn_dtype codes.
int input_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return OGN_F32;
    case at::kHalf: return OGN_F16;
    case at::kBFloat16: return OGN_BF16;
    case at::kChar: return OGN_I8;
    default: TORCH_CHECK(false, "mat must be float32, float16, bfloat16 or int8");
  }
  return -1;
}

at::ScalarType output_type(int64_t code) {
  switch (code) {
    case OGN_F32: return at::kFloat;
    case OGN_F16: return at::kHalf;
    case OGN_BF16: return at::kBFloat16;
    case OGN_I32: return at::kInt;
    default: TORCH_CHECK(false, "unsupported input/output dtype combination");
  }
  return at::kFloat;
}

Tensor workspace(size_t bytes, const Tensor& like) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

int64_t trailing_width(const Tensor& v) {
  int64_t w = 1;
  for (int64_t i = 1; i < v.dim(); ++i) w *= v.size(i);
  return w;
}

// ------------------------------------------------------------ torch_sparse_spmm
// forward(ptr, col, value, mat, reduce, outtype) -> (out, arg); reference
// TorchSparseSpmmForward (csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:97-135).
std::tuple<Tensor, Tensor> spmm_forward(Tensor ptr, Tensor col, std::optional<Tensor> value, Tensor mat,
                                        int64_t reduce, int64_t outtype) {
  on_gpu(ptr, "ptr");
  on_gpu(col, "col");
  on_gpu(mat, "mat");
  TORCH_CHECK(ptr.dim() == 1 && col.dim() == 1 && ptr.numel() >= 1, "ptr and col must be 1-D, ptr nonempty");
  TORCH_CHECK(mat.dim() >= 2, "mat must be [..., N, K]");
  TORCH_CHECK(reduce >= OGN_REDUCE_SUM && reduce <= OGN_REDUCE_MAX, "reduce must be 0..3 (sum/mean/min/max)");
  const int in = input_code(mat.scalar_type());
  const at::ScalarType ot = output_type(outtype);
  const bool allowed = outtype == OGN_F32 || (in == OGN_I8 ? outtype == OGN_I32 : outtype == in);
  TORCH_CHECK(allowed, "unsupported input/output dtype combination");
  const int64_t nnz = col.numel();
  int64_t width = 1;
  if (value.has_value()) {
    on_gpu(*value, "value");
    TORCH_CHECK(value->scalar_type() == mat.scalar_type(), "value dtype must match mat dtype");
    TORCH_CHECK(value->dim() >= 1 && value->size(0) == nnz, "value length must equal E");
    width = trailing_width(*value);
  }
  const int64_t n = mat.size(-2), k = mat.size(-1), m = ptr.numel() - 1;
  TORCH_CHECK(width == 1 || width == k, "value must contain 1 or K weights per edge");
  c10::DeviceGuard guard(mat.device());
  ptr = ptr.contiguous();
  col = col.scalar_type() == ptr.scalar_type() ? col.contiguous() : col.to(ptr.scalar_type()).contiguous();
  mat = mat.contiguous();
  Tensor v = value.has_value() ? value->contiguous() : Tensor();
  std::vector<int64_t> shape = mat.sizes().vec();
  shape[shape.size() - 2] = m;
  const int64_t batch = mat.numel() / std::max<int64_t>(n * k, 1);
  Tensor out = at::empty(shape, mat.options().dtype(ot));
  const bool minmax = reduce >= OGN_REDUCE_MIN;
  Tensor arg = at::empty(minmax ? shape : std::vector<int64_t>{0}, col.options().dtype(at::kLong));
  if (out.numel() == 0) return {out, arg};
  const size_t ws_bytes = ogn_spmm_csr_workspace_size(m, nnz, k, batch, in, (int)reduce);
  Tensor ws = workspace(ws_bytes, mat);
  ok(ogn_spmm_csr(ptr.data_ptr(), col.data_ptr(), index_code(ptr), v.defined() ? v.data_ptr() : nullptr, width,
                  mat.data_ptr(), in, batch, m, n, k, nnz, out.data_ptr(), (int)outtype,
                  minmax ? arg.data_ptr<int64_t>() : nullptr, (int)reduce, ws.data_ptr(), ws_bytes, stream_of(mat)),
     "torch_sparse_spmm.forward");
  return {out, arg};
}

// validate(ptr, col, n) -> int32 [1] status (0 valid, 1 bad rowptr, 2 column
// out of range); reference TorchSparseSpmmValidate (torch_sparse_spmm.cpp:136-147).
Tensor spmm_validate(Tensor ptr, Tensor col, int64_t n) {
  on_gpu(ptr, "ptr");
  on_gpu(col, "col");
  TORCH_CHECK(ptr.dim() == 1 && col.dim() == 1, "ptr and col must be 1-D");
  TORCH_CHECK(n >= 0, "N must be nonnegative");
  c10::DeviceGuard guard(ptr.device());
  Tensor status = at::empty({1}, ptr.options().dtype(at::kInt));
  if (ptr.numel() == 0) return status.fill_(1);
  ptr = ptr.contiguous();
  col = col.scalar_type() == ptr.scalar_type() ? col.contiguous() : col.to(ptr.scalar_type()).contiguous();
  ok(ogn_validate_csr(ptr.data_ptr(), col.data_ptr(), index_code(ptr), ptr.numel() - 1, col.numel(), n,
                      status.data_ptr<int32_t>(), stream_of(ptr)),
     "torch_sparse_spmm.validate");
  return status;
}

// value_backward(ptr, col, mat, grad, reduce, width) -> float32 [E] or [E, K]:
// dv[e] = sum_b <grad[b, row(e)], mat[b, col(e)]> (/ deg(row) for mean), or
// the per-feature products for K-wide weights.  Reference
// TorchSparseSpmmValueGrad (torch_sparse_spmm.cpp:148-169) and ValueGradCompute
// (op_kernel/arch35/torch_sparse_spmm_kernel.h:326-395); here one SDDMM per
// batch (dot for width 1, mul for width K).
Tensor spmm_value_backward(Tensor ptr, Tensor col, Tensor mat, Tensor grad, int64_t reduce, int64_t width) {
  on_gpu(ptr, "ptr");
  on_gpu(col, "col");
  on_gpu(mat, "mat");
  on_gpu(grad, "grad");
  TORCH_CHECK(reduce == OGN_REDUCE_SUM || reduce == OGN_REDUCE_MEAN, "value backward supports sum/mean");
  TORCH_CHECK(mat.is_floating_point() && mat.dim() >= 2, "mat must be floating [..., N, K]");
  const int64_t n = mat.size(-2), k = mat.size(-1), m = ptr.numel() - 1, nnz = col.numel();
  TORCH_CHECK(width == 1 || width == k, "value width must be 1 or K");
  std::vector<int64_t> expect = mat.sizes().vec();
  expect[expect.size() - 2] = m;
  TORCH_CHECK(grad.is_floating_point() && grad.sizes().vec() == expect && grad.device() == mat.device(),
              "grad must be floating [..., M, K] on the same GPU as mat");
  c10::DeviceGuard guard(mat.device());
  ptr = ptr.contiguous();
  col = col.scalar_type() == ptr.scalar_type() ? col.contiguous() : col.to(ptr.scalar_type()).contiguous();
  Tensor g = grad.to(at::kFloat).reshape({-1, m, k});
  if (reduce == OGN_REDUCE_MEAN) {
    Tensor deg = (ptr.slice(0, 1) - ptr.slice(0, 0, m)).clamp_min(1).to(at::kFloat);
    g = g / deg.reshape({1, m, 1});
  }
  g = g.contiguous();
  Tensor x = mat.to(at::kFloat).reshape({-1, n, k}).contiguous();
  Tensor dv = width == 1 ? at::zeros({nnz}, g.options()) : at::zeros({nnz, k}, g.options());
  if (nnz == 0 || m == 0) return dv;
  Tensor part = at::empty_like(dv);
  const int op = width == 1 ? OGN_SDDMM_DOT : OGN_SDDMM_MUL;
  void* s = stream_of(mat);
  const size_t ws_bytes = ogn_sddmm_csr_workspace_size(nnz, k, OGN_F32);
  Tensor ws = workspace(ws_bytes, mat);
  for (int64_t b = 0; b < g.size(0); ++b) {
    Tensor dst = b == 0 ? dv : part;
    ok(ogn_sddmm_csr(ptr.data_ptr(), col.data_ptr(), index_code(ptr), m, nnz, g[b].data_ptr(), m, 0,
                     x[b].data_ptr(), n, 2, k, OGN_F32, op, dst.data_ptr(), ws.data_ptr(), ws_bytes, s),
       "torch_sparse_spmm.value_backward");
    if (b > 0) dv.add_(part);
  }
  return dv;
}

// convert(src, output, to_ptr): to_ptr -> ind2ptr(src, output - 1) (output =
// M + 1 pointer entries); else ptr2ind(src, output) (output = E).  Reference
// TorchSparseSpmmConvert (torch_sparse_spmm.cpp:170-184).
Tensor spmm_convert(Tensor src, int64_t output, bool to_ptr) {
  on_gpu(src, "src");
  TORCH_CHECK(src.dim() == 1, "convert: src must be 1-D");
  TORCH_CHECK(output >= (to_ptr ? 1 : 0), "convert: output length out of range");
  c10::DeviceGuard guard(src.device());
  src = src.contiguous();
  Tensor out = at::empty({output}, src.options().dtype(at::kLong));
  void* s = stream_of(src);
  if (to_ptr) {
    if (src.numel() == 0) return out.zero_();
    ok(ogn_ind2ptr(src.data_ptr(), index_code(src), src.numel(), output - 1, out.data_ptr<int64_t>(), s),
       "torch_sparse_spmm.convert");
  } else if (output > 0) {
    TORCH_CHECK(src.numel() >= 1, "convert: ptr must be nonempty");
    ok(ogn_ptr2ind(src.data_ptr(), index_code(src), src.numel() - 1, output, out.data_ptr<int64_t>(), s),
       "torch_sparse_spmm.convert");
  }
  return out;
}

// permute_values(value, perm) -> value[perm] along dim 0 (raw row copies, any
// trailing shape).  Reference TorchSparseSpmmPermuteValues (torch_sparse_spmm.cpp:185-209);
// here the gather_coo row copy.
Tensor spmm_permute_values(Tensor value, Tensor perm) {
  on_gpu(value, "value");
  on_gpu(perm, "perm");
  TORCH_CHECK(value.device() == perm.device() && value.dim() >= 1 && perm.dim() == 1 &&
                  perm.scalar_type() == at::kLong && perm.numel() == value.size(0),
              "invalid value permutation metadata");
  input_code(value.scalar_type());  // the edge-value dtypes of SpMM
  c10::DeviceGuard guard(value.device());
  value = value.contiguous();
  perm = perm.contiguous();
  Tensor out = at::empty_like(value, at::MemoryFormat::Contiguous);
  if (out.numel() == 0) return out;
  const int64_t row_bytes = (int64_t)value.element_size() * trailing_width(value);
  ok(ogn_gather_coo(perm.data_ptr<int64_t>(), value.data_ptr(), 1, value.size(0), perm.numel(), row_bytes,
                    out.data_ptr(), stream_of(value)),
     "torch_sparse_spmm.permute_values");
  return out;
}

// tensor_version(t) -> the autograd version counter, or None for inference
// tensors (which carry none and must never enter a mutation-keyed cache).
// Reference TorchSparseSpmmTensorVersion (torch_sparse_spmm.cpp:210-217).
std::optional<int64_t> tensor_version(const Tensor& t) {
  if (t.is_inference()) return std::nullopt;
  return (int64_t)t._version();
}

// ------------------------------------------------------------ index conversion
Tensor ind2ptr(Tensor ind, int64_t rows) {
  TORCH_CHECK(rows >= 0, "ind2ptr: M must be non-negative");
  return spmm_convert(std::move(ind), rows + 1, true);
}

Tensor ptr2ind(Tensor ptr, int64_t edges) {
  TORCH_CHECK(edges >= 0, "ptr2ind: E must be non-negative");
  return spmm_convert(std::move(ptr), edges, false);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "ops_gnn: MI355X (gfx950) extension over libogn_hip.so";
  m.attr("arch") = ogn_arch();
  m.attr("abi_version") = ogn_abi_version();
  auto ts = m.def_submodule("torch_sparse_spmm", "torch_sparse SpMM on MI355X");
  ts.def("forward", &spmm_forward, py::arg("ptr"), py::arg("col"), py::arg("value"), py::arg("mat"),
         py::arg("reduce"), py::arg("outtype"), py::call_guard<py::gil_scoped_release>());
  ts.def("validate", &spmm_validate, py::arg("ptr"), py::arg("col"), py::arg("n"),
         py::call_guard<py::gil_scoped_release>());
  ts.def("value_backward", &spmm_value_backward, py::arg("ptr"), py::arg("col"), py::arg("mat"), py::arg("grad"),
         py::arg("reduce"), py::arg("width"), py::call_guard<py::gil_scoped_release>());
  ts.def("convert", &spmm_convert, py::arg("src"), py::arg("output"), py::arg("to_ptr"),
         py::call_guard<py::gil_scoped_release>());
  ts.def("permute_values", &spmm_permute_values, py::arg("value"), py::arg("perm"),
         py::call_guard<py::gil_scoped_release>());
  ts.def("tensor_version", &tensor_version, py::arg("tensor"));
  m.def("ind2ptr", &ind2ptr, py::arg("ind"), py::arg("M"),
        "sorted row indices -> CSR row pointer (torch_sparse.ind2ptr)", py::call_guard<py::gil_scoped_release>());
  m.def("ptr2ind", &ptr2ind, py::arg("ptr"), py::arg("E"),
        "CSR row pointer -> row index of every edge (torch_sparse.ptr2ind)", py::call_guard<py::gil_scoped_release>());
}
