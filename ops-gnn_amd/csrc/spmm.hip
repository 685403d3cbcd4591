// CSR SpMM (torch_sparse semantics) for gfx950.
//
// Schedule: nnz-split.  The edge list [0, nnz) is cut into fixed chunks of C
// edges and one wavefront owns one chunk, so every wave does the same amount
// of gather work whatever the row-length distribution (power-law hub rows of
// 20 000 edges are spread over many waves, runs of short rows share one).
//
// Inside a wave the 64 lanes are split into S = 64 / G sub-groups of G lanes;
// a sub-group covers one feature row of `mat` with one 16-byte load per lane
// (G = K * sizeof(T) / 16), so a step gathers S edges at once and U steps are
// issued before any is consumed (S * U feature rows in flight per wave).
// Column indices and edge weights are staged with one coalesced load per 64
// edges and handed to the sub-groups with ds_bpermute; row ends come from a
// 64-row window of rowptr held one entry per lane (v_readlane).
//
// Ownership: a row is written by the chunk holding its last edge (empty rows
// by the chunk where their position falls).  A row that crosses a chunk
// boundary leaves a partial record: "tail" in each chunk it leaves, "head" in
// the chunk where it ends.  A fix-up kernel folds tail[c1..c2-1] + head[c2]
// in chunk order and finalises the row, so results are deterministic and no
// atomics are used.
#include "spmm_kernels.h"

#include <algorithm>
#include <cstdlib>
#include <string>

namespace ogn {
namespace spmm {
namespace {

Plan make_plan(int64_t nnz, int64_t k, int in_dtype, bool aligned) {
  Plan pl{};
  const int esz = dtype_size(in_dtype);
  const int vec = 16 / esz;
  const int64_t kv = k / vec;
  if (aligned && k % vec == 0 && kv <= 64 && (kv & (kv - 1)) == 0) {
    pl.vec = true;
    pl.g = (int)kv;
    pl.tiles = 1;
  } else if (aligned && k % vec == 0 && kv % 64 == 0) {
    pl.vec = true;
    pl.g = 64;
    pl.tiles = kv / 64;
  } else {
    pl.vec = false;
    pl.g = 64;
    pl.tiles = (k + 63) / 64;
  }
  // ~128 KiB of feature gathers per wave, in whole 64-edge windows.
  const int64_t row_bytes = std::max<int64_t>(1, std::min<int64_t>(k, 64 * vec) * esz);
  int64_t chunk = (131072 / row_bytes + 63) / 64 * 64;
  if (const char* env = std::getenv("OGN_SPMM_CHUNK")) {
    const long v = std::atol(env);
    if (v >= 64) chunk = v / 64 * 64;
  }
  pl.chunk = std::min<int64_t>(std::max<int64_t>(chunk, 64), 8192);
  pl.nchunks = std::max<int64_t>(1, (nnz + pl.chunk - 1) / pl.chunk);
  return pl;
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

struct WsLayout {
  size_t chunk_row, head, tail, arg_head, arg_tail, total;
};

WsLayout ws_layout(const Plan& pl, int64_t k, int64_t batch, bool mm) {
  WsLayout w{};
  const size_t rec = (size_t)pl.nchunks * batch * k;
  w.chunk_row = 0;
  w.head = align256(sizeof(int64_t) * pl.nchunks);
  const size_t vbytes = align256(rec * (mm ? sizeof(double) : sizeof(float)));
  w.tail = w.head + vbytes;
  w.arg_head = w.tail + vbytes;
  const size_t abytes = mm ? align256(rec * sizeof(int64_t)) : 0;
  w.arg_tail = w.arg_head + abytes;
  w.total = w.arg_tail + abytes;
  return w;
}

bool is_aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace
}  // namespace spmm
}  // namespace ogn

using namespace ogn;
using namespace ogn::spmm;

extern "C" {

size_t ogn_spmm_csr_workspace_size(int64_t m, int64_t nnz, int64_t k, int64_t batch, int in_dtype,
                                   int reduce) {
  (void)m;
  if (nnz < 0 || k <= 0 || batch <= 0) return 0;
  const Plan pl = make_plan(nnz, k, in_dtype, true);
  const Plan ps = make_plan(nnz, k, in_dtype, false);
  const bool mm = reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX;
  return std::max(ws_layout(pl, k, batch, mm).total, ws_layout(ps, k, batch, mm).total);
}

int ogn_spmm_csr(const void* rowptr, const void* col, int index_dtype, const void* value,
                 int64_t value_width, const void* mat, int in_dtype, int64_t batch, int64_t m,
                 int64_t n, int64_t k, int64_t nnz, void* out, int out_dtype, int64_t* arg,
                 int reduce, void* workspace, size_t workspace_bytes, void* stream) {
  if (m < 0 || n < 0 || k < 0 || nnz < 0 || batch < 0)
    return fail(OGN_EINVAL, "ogn_spmm_csr: negative size");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_spmm_csr: index dtype must be int32 or int64");
  if (in_dtype != OGN_F32 && in_dtype != OGN_F16 && in_dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_spmm_csr: mat dtype must be float32, float16 or bfloat16");
  if (out_dtype != OGN_F32 && out_dtype != OGN_F16 && out_dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_spmm_csr: out dtype must be float32, float16 or bfloat16");
  if (reduce < OGN_REDUCE_SUM || reduce > OGN_REDUCE_MAX)
    return fail(OGN_EINVAL, "ogn_spmm_csr: reduce must be sum/mean/min/max");
  const bool mm = reduce >= OGN_REDUCE_MIN;
  if (m == 0 || k == 0 || batch == 0) return OGN_OK;
  if (!rowptr || !out || (mm && !arg)) return fail(OGN_EINVAL, "ogn_spmm_csr: null pointer");
  if (nnz > 0 && (!col || !mat || n == 0))
    return fail(OGN_EINVAL, "ogn_spmm_csr: nnz > 0 needs col, mat and n > 0");
  if (value && value_width != 1 && value_width != k)
    return fail(OGN_EINVAL, "ogn_spmm_csr: value width must be 1 or k");
  if (batch > 65535) return fail(OGN_EUNSUPPORTED, "ogn_spmm_csr: batch > 65535");

  const bool aligned = is_aligned(mat, 16) && is_aligned(out, 16) &&
                       (!value || value_width == 1 || is_aligned(value, 16));
  const Plan pl = make_plan(nnz, k, in_dtype, aligned);
  if (pl.tiles > 65535) return fail(OGN_EUNSUPPORTED, "ogn_spmm_csr: k too large");
  const WsLayout wl = ws_layout(pl, k, batch, mm);
  if (!workspace || workspace_bytes < wl.total)
    return fail(OGN_EINVAL, "ogn_spmm_csr: workspace too small (need " +
                                std::to_string(wl.total) + " bytes)");
  char* ws = static_cast<char*>(workspace);
  SpmmParams p{};
  p.ptr = rowptr;
  p.col = col;
  p.val = value;
  p.mat = mat;
  p.out = out;
  p.arg = arg;
  p.chunk_row = reinterpret_cast<const int64_t*>(ws + wl.chunk_row);
  if (mm) {
    p.mm_head = reinterpret_cast<double*>(ws + wl.head);
    p.mm_tail = reinterpret_cast<double*>(ws + wl.tail);
    p.arg_head = reinterpret_cast<int64_t*>(ws + wl.arg_head);
    p.arg_tail = reinterpret_cast<int64_t*>(ws + wl.arg_tail);
  } else {
    p.sum_head = reinterpret_cast<float*>(ws + wl.head);
    p.sum_tail = reinterpret_cast<float*>(ws + wl.tail);
  }
  p.m = m;
  p.n = std::max<int64_t>(n, 1);
  p.k = k;
  p.nnz = nnz;
  p.chunk = pl.chunk;
  p.nchunks = pl.nchunks;
  p.val_mode = value == nullptr ? 0 : (value_width == 1 ? 1 : 2);
  p.out_dt = out_dtype;
  p.reduce = reduce;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool i64 = index_dtype == OGN_I64;
  if (nnz > 0) {
    TimedLaunch t("spmm_chunk_rows", s);
    const dim3 g((unsigned)((m + 255) / 256));
    if (i64)
      hipLaunchKernelGGL(chunk_rows_kernel<int64_t>, g, dim3(256), 0, s,
                         static_cast<const int64_t*>(rowptr), m, pl.chunk, pl.nchunks,
                         reinterpret_cast<int64_t*>(ws + wl.chunk_row));
    else
      hipLaunchKernelGGL(chunk_rows_kernel<int32_t>, g, dim3(256), 0, s,
                         static_cast<const int32_t*>(rowptr), m, pl.chunk, pl.nchunks,
                         reinterpret_cast<int64_t*>(ws + wl.chunk_row));
  }
  const dim3 grid((unsigned)((pl.nchunks + kWavesPerBlock - 1) / kWavesPerBlock),
                  (unsigned)pl.tiles, (unsigned)batch);
  {
    TimedLaunch t("spmm_main", s);
    switch (in_dtype) {
    case OGN_F32: launch_f32(pl, mm, grid, s, p, i64); break;
    case OGN_F16: launch_f16(pl, mm, grid, s, p, i64); break;
    default: launch_bf16(pl, mm, grid, s, p, i64); break;
    }
  }
  if (pl.nchunks > 1) {
    TimedLaunch t("spmm_fixup", s);
    const dim3 fg((unsigned)((pl.nchunks + kWavesPerBlock - 1) / kWavesPerBlock), 1, (unsigned)batch);
    if (i64) {
      if (mm) hipLaunchKernelGGL((spmm_fixup_kernel<int64_t, true>), fg, dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL((spmm_fixup_kernel<int64_t, false>), fg, dim3(kBlock), 0, s, p);
    } else {
      if (mm) hipLaunchKernelGGL((spmm_fixup_kernel<int32_t, true>), fg, dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL((spmm_fixup_kernel<int32_t, false>), fg, dim3(kBlock), 0, s, p);
    }
  }
  return check_launch("ogn_spmm_csr");
}

}  // extern "C"
