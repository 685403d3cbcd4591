// Library-wide pieces of the C ABI: error channel, identification, CSR
// validation.
#include "ogn_device.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <vector>

namespace ogn {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(OGN_EHIP, std::string(what) + ": kernel launch failed: " + hipGetErrorString(e));
  return OGN_OK;
}

// ---------------------------------------------------------------- kernel timing
// Opt-in per-kernel timing: while enabled, every library launch wrapped in a
// TimedLaunch records a pair of HIP events on its stream.  Reading the totals
// synchronises on those events only.
namespace {
struct TimingRecord {
  std::string name;
  hipEvent_t start, stop;
};
std::mutex g_timing_mu;
bool g_timing_on = false;
std::vector<TimingRecord> g_records;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void recycle_records() {
  for (auto& r : g_records) {
    g_event_pool.push_back(r.start);
    g_event_pool.push_back(r.stop);
  }
  g_records.clear();
}
}  // namespace

TimedLaunch::TimedLaunch(const char* name, hipStream_t stream) : stream_(stream) {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  if (!g_timing_on) return;
  start_ = take_event();
  stop_ = take_event();
  if (!start_ || !stop_) return;
  name_ = name;
  active_ = hipEventRecord(start_, stream_) == hipSuccess;
}

TimedLaunch::~TimedLaunch() {
  if (!active_) return;
  if (hipEventRecord(stop_, stream_) != hipSuccess) return;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_records.push_back({name_, start_, stop_});
}

namespace {

__global__ void fill_i32(int32_t* p, int32_t v) { *p = v; }

// One pass over rowptr and col; any violation raises the status with an
// atomic max (status codes: 1 bad rowptr, 2 column out of range).
template <typename IDX>
__global__ __launch_bounds__(256) void validate_csr_kernel(const IDX* __restrict__ ptr,
                                                           const IDX* __restrict__ col,
                                                           int64_t m, int64_t nnz, int64_t n,
                                                           int32_t* status) {
  int32_t bad = 0;
  const int64_t total = col ? std::max(m + 1, nnz) : m + 1;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    if (i <= m) {
      const int64_t v = ptr[i];
      if (v < 0 || v > nnz) bad = max(bad, 1);
      if (i == 0 && v != 0) bad = max(bad, 1);
      if (i == m && v != nnz) bad = max(bad, 1);
      if (i < m && (int64_t)ptr[i + 1] < v) bad = max(bad, 1);
    }
    if (col != nullptr && i < nnz) {
      const int64_t cidx = col[i];
      if (cidx < 0 || cidx >= n) bad = max(bad, 2);
    }
  }
  if (bad) atomicMax(status, bad);
}

}  // namespace
}  // namespace ogn

using namespace ogn;

extern "C" {

const char* ogn_last_error(void) { return g_last_error.c_str(); }

int ogn_timing_enable(int on) {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timing_on = on != 0;
  recycle_records();
  return OGN_OK;
}

int ogn_timing_query(const char* kernel, double* total_ms, int64_t* launches) {
  if (!kernel || !total_ms || !launches) return fail(OGN_EINVAL, "ogn_timing_query: null pointer");
  std::lock_guard<std::mutex> lk(g_timing_mu);
  double acc = 0.0;
  int64_t count = 0;
  for (auto& r : g_records) {
    if (r.name != kernel) continue;
    if (hipEventSynchronize(r.stop) != hipSuccess)
      return fail(OGN_EHIP, "ogn_timing_query: event synchronisation failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess)
      return fail(OGN_EHIP, "ogn_timing_query: elapsed-time query failed");
    acc += ms;
    ++count;
  }
  *total_ms = acc;
  *launches = count;
  return OGN_OK;
}
const char* ogn_arch(void) { return "gfx950"; }
int ogn_abi_version(void) { return 3; }

int ogn_validate_csr(const void* rowptr, const void* col, int index_dtype, int64_t m,
                     int64_t nnz, int64_t n, int32_t* status, void* stream) {
  if (!rowptr || !status) return fail(OGN_EINVAL, "ogn_validate_csr: null pointer");
  if (m < 0 || nnz < 0 || n < 0) return fail(OGN_EINVAL, "ogn_validate_csr: negative size");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_validate_csr: index dtype must be int32 or int64");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_i32, dim3(1), dim3(1), 0, s, status, 0);
  const int64_t total = col ? std::max(m + 1, nnz) : m + 1;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
  if (index_dtype == OGN_I64)
    hipLaunchKernelGGL(validate_csr_kernel<int64_t>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const int64_t*>(rowptr), static_cast<const int64_t*>(col),
                       m, nnz, n, status);
  else
    hipLaunchKernelGGL(validate_csr_kernel<int32_t>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const int32_t*>(rowptr), static_cast<const int32_t*>(col),
                       m, nnz, n, status);
  return check_launch("ogn_validate_csr");
}

}  // extern "C"
