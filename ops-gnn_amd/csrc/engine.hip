// Host side of the CSR reduction engine: launch geometry, workspace layout
// and the three-pass launch sequence (chunk rows, main, fix-up).
#include "csr_engine.h"

#include <cstdlib>
#include <mutex>
#include <string>
#include <vector>

namespace ogn {
namespace eng {

Plan make_plan(int64_t nnz_bound, int64_t k, int in_dtype, bool aligned, bool gather) {
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
  } else if (k == 1) {
    pl.vec = false;  // one feature: 64 positions per step, one per lane
    pl.g = 1;
    pl.tiles = 1;
  } else {
    pl.vec = false;
    pl.g = 64;
    pl.tiles = (k + 63) / 64;
  }
  // Feature traffic per wave, in whole 64-position windows: 48 KiB in
  // contiguous mode (config 5 scatter, wall ms, at 320 / 384 / 448 / 512
  // positions: sum 1.166 / 1.168 / 1.176 / 1.184, max 1.315 / 1.314 / 1.315 /
  // 1.329, logsumexp 1.198 / 1.191 / 1.202 / 1.221), 256 KiB in
  // gather mode, where halving the chunk count halves the rows that cross a
  // chunk boundary and so the fix-up pass (config 3 SpMM sum step 5.79 ->
  // 5.70 ms, max 7.27 -> 6.96 ms).
  const int64_t row_bytes = std::max<int64_t>(1, std::min<int64_t>(k, 64 * vec) * esz);
  int64_t wave_bytes = gather ? 262144 : 49152;
  if (const char* env = std::getenv("OGN_ENGINE_WAVE_KIB")) {
    const long v = std::atol(env);
    if (v >= 16) wave_bytes = (int64_t)v * 1024;
  }
  int64_t chunk = (wave_bytes / row_bytes + 63) / 64 * 64;
  if (const char* env = std::getenv("OGN_ENGINE_CHUNK")) {
    const long v = std::atol(env);
    if (v >= 64) chunk = v / 64 * 64;
  }
  // Small problems: shrink chunks until there are about 8K wavefronts (8 per
  // SIMD), so latency is hidden (floor 128 positions: smaller chunks cost
  // more in row fix-ups than they gain).
  const int64_t waves_floor = ((nnz_bound / 8192) / 64) * 64;
  if (!std::getenv("OGN_ENGINE_CHUNK")) {
    chunk = std::min<int64_t>(chunk, std::max<int64_t>(waves_floor, 128));
    // Contiguous mode, fewer than two rounds of resident waves (4096 = 256
    // CUs x 16): one round instead -- no partly filled second round, and
    // half the rows crossing chunk ends (config 2: 7812 waves of 128
    // positions -> 3906 of 256; segment max 140 -> 131 us and 150 -> 145 us
    // on two boxes, sum and logsumexp within 1 %).
    constexpr int64_t kRound = 4096;
    if (!gather && nnz_bound > 0 && (nnz_bound + chunk - 1) / chunk < 2 * kRound)
      chunk = std::max<int64_t>(chunk, ((nnz_bound + kRound - 1) / kRound + 63) / 64 * 64);
  }
  pl.chunk = std::min<int64_t>(std::max<int64_t>(chunk, 64), 8192);
  pl.nchunks = std::max<int64_t>(1, (nnz_bound + pl.chunk - 1) / pl.chunk);
  return pl;
}

static size_t align256(size_t v) { return (v + 255) / 256 * 256; }

Workspace workspace_layout(const Plan& pl, int64_t k, int64_t batch, int64_t ptr_batches, int rk) {
  Workspace w{};
  const size_t rec = (size_t)pl.nchunks * batch * k;
  w.chunk_row = 0;
  w.fix = align256(sizeof(int64_t) * pl.nchunks * ptr_batches);
  w.head = w.fix + align256(sizeof(longlong4) * pl.nchunks * ptr_batches);
  const size_t vsz = rk == RK_SUM ? sizeof(float) : (rk == RK_LSE ? sizeof(float2) : sizeof(double));
  const size_t vbytes = align256(rec * vsz);
  w.tail = w.head + vbytes;
  w.arg_head = w.tail + vbytes;
  const size_t abytes = rk == RK_MINMAX ? align256(rec * sizeof(int64_t)) : 0;
  w.arg_tail = w.arg_head + abytes;
  w.total = w.arg_tail + abytes;
  return w;
}

// Layouts kept in caller workspaces (LAYOUT_KEEP / LAYOUT_REUSE, and the
// long-row list of the grouped softmax): which pointer array and plan each
// workspace's layout was computed for.  A small list (most recent last),
// bounded.
namespace {
std::mutex g_kept_mu;
std::vector<KeptKey> g_kept;
constexpr size_t kKeptMax = 64;
}  // namespace

bool kept_layout_find(const KeptKey& k, int64_t* payload) {
  std::lock_guard<std::mutex> lock(g_kept_mu);
  for (const KeptKey& e : g_kept) {
    if (e.same(k)) {
      if (payload)
        for (int i = 0; i < 8; ++i) payload[i] = e.payload[i];
      return true;
    }
  }
  return false;
}

bool kept_layout_match(const KeptKey& k) { return kept_layout_find(k, nullptr); }

void kept_layout_store(const KeptKey& k) {
  std::lock_guard<std::mutex> lock(g_kept_mu);
  for (size_t i = 0; i < g_kept.size(); ++i) {
    if (g_kept[i].ws == k.ws) {
      g_kept.erase(g_kept.begin() + (std::ptrdiff_t)i);
      break;
    }
  }
  if (g_kept.size() >= kKeptMax) g_kept.erase(g_kept.begin());
  g_kept.push_back(k);
}

int run(const Plan& pl, Params& p, int in_dtype, int index_dtype, bool gather, int rk, int64_t batch,
        void* workspace, size_t workspace_bytes, hipStream_t s, const char* name, int layout) {
  const int64_t ptr_batches = p.ptr_bstride ? batch : 1;
  const Workspace wl = workspace_layout(pl, p.k, batch, ptr_batches, rk);
  if (!workspace || workspace_bytes < wl.total)
    return fail(OGN_EINVAL, std::string(name) + ": workspace too small (need " +
                                std::to_string(wl.total) + " bytes)");
  if (batch > 65535 || pl.tiles > 65535)
    return fail(OGN_EUNSUPPORTED, std::string(name) + ": batch or feature tiles exceed 65535");
  char* ws = static_cast<char*>(workspace);
  p.chunk_row = reinterpret_cast<int64_t*>(ws + wl.chunk_row);
  p.fix = reinterpret_cast<longlong4*>(ws + wl.fix);
  p.rec_head = ws + wl.head;
  p.rec_tail = ws + wl.tail;
  p.arg_head = rk == RK_MINMAX ? reinterpret_cast<int64_t*>(ws + wl.arg_head) : nullptr;
  p.arg_tail = rk == RK_MINMAX ? reinterpret_cast<int64_t*>(ws + wl.arg_tail) : nullptr;
  p.chunk = pl.chunk;
  p.nchunks = pl.nchunks;
  const bool i64 = index_dtype == OGN_I64;
  const std::string n(name);
  // contiguous mode, fast variants: chunks of short rows take short_chunk
  p.short_rows = !gather && in_dtype != OGN_I8 && variant_of(rk, false, p) != V_GENERIC &&
                 !std::getenv("OGN_ENGINE_NO_SHORT");
  if (p.short_rows && !std::getenv("OGN_ENGINE_NO_STAGE")) p.short_rows = 2;
  // Contiguous fast variants read a source larger than the 256 MiB
  // last-level cache with non-temporal loads (each packet is read once per
  // call), a smaller one with plain loads, which leave it cached for the next
  // call: config 2 (544 MB) segment sum 119 -> 108 us non-temporal; 64 / 128
  // / 192 MB sources 26 / 31 / 40 us plain against 31 / 34 / 43 us.
  // OGN_ENGINE_NT=0 / 1 forces either, for A/B measurement.
  const double src_bytes = (double)batch * (double)p.nnz_bound * (double)p.k * (double)dtype_size(in_dtype);
  bool nt = src_bytes > 256.0 * 1024 * 1024;
  if (const char* env = std::getenv("OGN_ENGINE_NT")) nt = std::atoi(env) != 0;
  p.src_nt = !gather && in_dtype != OGN_I8 && nt && variant_of(rk, false, p) != V_GENERIC;
  // extremum positions of outputs larger than that cache: non-temporal
  const double out_bytes = (double)batch * (double)p.m * (double)p.k * (double)(dtype_size(p.out_dt) + 8);
  p.out_nt = rk == RK_MINMAX && out_bytes > 256.0 * 1024 * 1024;
  const KeptKey kl{workspace, p.ptr, {0, p.ptr_bstride, ptr_batches, p.m, p.nnz_bound, pl.chunk, pl.nchunks,
                                       index_dtype}, {}};
  if (!(layout & LAYOUT_REUSE) || !kept_layout_match(kl)) {
    TimedLaunch t((n + "_chunk_rows").c_str(), s);
    const dim3 g((unsigned)((pl.nchunks + 255) / 256), (unsigned)ptr_batches);
    if (i64) hipLaunchKernelGGL(chunk_rows_kernel<int64_t>, g, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(chunk_rows_kernel<int32_t>, g, dim3(256), 0, s, p);
    if (layout & (LAYOUT_KEEP | LAYOUT_REUSE)) kept_layout_store(kl);
  }
  const dim3 grid((unsigned)((pl.nchunks + kWavesPerBlock - 1) / kWavesPerBlock), (unsigned)pl.tiles,
                  (unsigned)batch);
  {
    TimedLaunch t((n + "_main").c_str(), s);
    switch (in_dtype) {
      case OGN_F32:
        gather ? launch_gather_f32(pl, rk, i64, grid, s, p)
               : (p.src_nt ? launch_contig_f32_nt : launch_contig_f32)(pl, rk, i64, grid, s, p);
        break;
      case OGN_F16:
        gather ? launch_gather_f16(pl, rk, i64, grid, s, p)
               : (p.src_nt ? launch_contig_f16_nt : launch_contig_f16)(pl, rk, i64, grid, s, p);
        break;
      case OGN_I8:
        launch_gather_i8(pl, rk, i64, grid, s, p);  // gather mode only (torch_sparse int8 SpMM)
        break;
      default:
        gather ? launch_gather_bf16(pl, rk, i64, grid, s, p)
               : (p.src_nt ? launch_contig_bf16_nt : launch_contig_bf16)(pl, rk, i64, grid, s, p);
        break;
    }
  }
  // a row longer than 64 * chunk positions can span more than kLongSpan
  // chunks; with every row at most kShortRowsMax <= 64 * chunk, none does
  static_assert(kShortRowsMax <= kLongSpan * 64, "the shortest chunk is 64 positions");
  if (pl.nchunks > kLongSpan + 1 && !(layout & LAYOUT_SHORT_ROWS)) {
    // rows spanning more than kLongSpan chunks: fold their interior records
    // in runs of kPiece first
    TimedLaunch t((n + "_prefold").c_str(), s);
    const int64_t groups = (pl.nchunks + kPiece - 1) / kPiece;
    const dim3 pg((unsigned)((groups + kWavesPerBlock - 1) / kWavesPerBlock), 1, (unsigned)batch);
    const bool f32mm = rk == RK_MINMAX && in_dtype == OGN_F32;
#define OGN_PRE(IDX)                                                                          \
  switch (rk) {                                                                               \
    case RK_MINMAX:                                                                           \
      if (f32mm) hipLaunchKernelGGL((prefold_kernel<IDX, RK_MINMAX, true>), pg, dim3(kBlock), 0, s, p); \
      else hipLaunchKernelGGL((prefold_kernel<IDX, RK_MINMAX, false>), pg, dim3(kBlock), 0, s, p);     \
      break;                                                                                  \
    case RK_LSE: hipLaunchKernelGGL((prefold_kernel<IDX, RK_LSE, false>), pg, dim3(kBlock), 0, s, p); break; \
    default: hipLaunchKernelGGL((prefold_kernel<IDX, RK_SUM, false>), pg, dim3(kBlock), 0, s, p); break;     \
  }
    if (in_dtype == OGN_I8 && rk == RK_SUM) {
      if (i64) hipLaunchKernelGGL((prefold_kernel<int64_t, RK_SUM, false, true>), pg, dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL((prefold_kernel<int32_t, RK_SUM, false, true>), pg, dim3(kBlock), 0, s, p);
    } else if (i64) {
      OGN_PRE(int64_t)
    } else {
      OGN_PRE(int32_t)
    }
#undef OGN_PRE
  }
  if (pl.nchunks > 1) {
    TimedLaunch t((n + "_fixup").c_str(), s);
    const dim3 fg((unsigned)((pl.nchunks + kWavesPerBlock - 1) / kWavesPerBlock), 1, (unsigned)batch);
    const bool f32mm = rk == RK_MINMAX && in_dtype == OGN_F32;
#define OGN_FIX(IDX)                                                                          \
  switch (rk) {                                                                               \
    case RK_MINMAX:                                                                           \
      if (f32mm) hipLaunchKernelGGL((fixup_kernel<IDX, RK_MINMAX, true>), fg, dim3(kBlock), 0, s, p); \
      else hipLaunchKernelGGL((fixup_kernel<IDX, RK_MINMAX, false>), fg, dim3(kBlock), 0, s, p);     \
      break;                                                                                  \
    case RK_LSE: hipLaunchKernelGGL((fixup_kernel<IDX, RK_LSE, false>), fg, dim3(kBlock), 0, s, p); break; \
    default: hipLaunchKernelGGL((fixup_kernel<IDX, RK_SUM, false>), fg, dim3(kBlock), 0, s, p); break;     \
  }
    if (in_dtype == OGN_I8 && rk == RK_SUM) {
      if (i64) hipLaunchKernelGGL((fixup_kernel<int64_t, RK_SUM, false, true>), fg, dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL((fixup_kernel<int32_t, RK_SUM, false, true>), fg, dim3(kBlock), 0, s, p);
    } else if (i64) {
      OGN_FIX(int64_t)
    } else {
      OGN_FIX(int32_t)
    }
#undef OGN_FIX
  }
  return check_launch(name);
}

}  // namespace eng
}  // namespace ogn
