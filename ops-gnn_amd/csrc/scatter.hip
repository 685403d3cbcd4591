// Unsorted-index scatter and the grouped-softmax passes for gfx950.
//
// scatter (torch_scatter rules) with an arbitrary index: one thread per src
// element, fp32 accumulators in a workspace, hardware float atomics for
// sum/mean, a compare-and-swap loop for prod, and an order-preserving
// integer encoding of floats for min/max (atomic min/max on the key, then a
// second pass records the largest position holding the winning value, which
// is the "later writer wins" tie rule).  A finishing pass converts to the
// output dtype.  Sum/mean/prod of floats are order-nondeterministic here (as
// in any atomic scatter); the sorted-index path (segment engine) is exact.
//
// grouped softmax: per-(batch, group, feature) statistics m = max and
// s = sum(exp(x - clamp(m))) -- from the segment engine when the index is
// sorted, from atomics otherwise -- then one elementwise pass produces
// softmax / log_softmax, or one pass over the groups produces logsumexp.
#include "ogn_device.h"
#include "typed.h"

#include <algorithm>
#include <string>

namespace ogn {
namespace {

constexpr float kFltMax = 3.402823466e38f;

__device__ __forceinline__ uint32_t key_of(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float float_of(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
__device__ __forceinline__ float clampm(float m) { return fminf(fmaxf(m, -kFltMax), kFltMax); }

struct ScatterArgs {
  const void* src;
  int dt;
  const int64_t* index;
  int64_t isb, isl, isf;  // index strides over (before, len, after)
  int64_t before, len, after, size;
  void* out;
  int64_t* arg;
  float* acc;       // [before, size, after] fp32 accumulators (sum/mean/prod)
  uint32_t* key;    // [before, size, after] min/max keys
  int32_t* count;   // [before, size, after] mean counts
  int reduce;
  int has_out;
  float limit;
  Split3 sp;  // index split of [before, len, after]
};

__global__ __launch_bounds__(256) void scatter_init_kernel(ScatterArgs a) {
  const int64_t total = a.before * a.size * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const float seed = a.has_out ? load_float(a.out, a.dt, i) : 0.f;
    if (a.reduce == OGN_REDUCE_MIN || a.reduce == OGN_REDUCE_MAX) {
      const bool is_min = a.reduce == OGN_REDUCE_MIN;
      const float s0 = a.has_out ? seed : (is_min ? a.limit : -a.limit);
      a.key[i] = key_of(s0 != s0 ? (is_min ? kFltMax : -kFltMax) : s0);
      a.arg[i] = -1;  // no position taken yet
    } else {
      a.acc[i] = a.has_out ? seed : (a.reduce == OGN_REDUCE_PROD ? 1.f : 0.f);
      if (a.count) a.count[i] = 0;
    }
  }
}

__device__ __forceinline__ void atomic_mul(float* p, float v) {
  unsigned int* u = reinterpret_cast<unsigned int*>(p);
  unsigned int old = __atomic_load_n(u, __ATOMIC_RELAXED);
  while (true) {
    const unsigned int want = __float_as_uint(__uint_as_float(old) * v);
    if (__atomic_compare_exchange_n(u, &old, want, false, __ATOMIC_RELAXED, __ATOMIC_RELAXED)) break;
  }
}

__global__ __launch_bounds__(256) void scatter_main_kernel(ScatterArgs a) {
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t b, l, f;
    split3(i, a.sp, b, l, f);
    const int64_t t = a.index[b * a.isb + l * a.isl + f * a.isf];
    if (t < 0 || t >= a.size) continue;
    const float x = load_float(a.src, a.dt, i);
    const int64_t o = (b * a.size + t) * a.after + f;
    switch (a.reduce) {
      case OGN_REDUCE_MIN:
        if (!(x != x)) atomicMin(&a.key[o], key_of(x));
        break;
      case OGN_REDUCE_MAX:
        if (!(x != x)) atomicMax(&a.key[o], key_of(x));
        break;
      case OGN_REDUCE_PROD:
        atomic_mul(&a.acc[o], x);
        break;
      default:
        atomicAdd(&a.acc[o], x);
        if (a.count) atomicAdd(&a.count[o], 1);
        break;
    }
  }
}

// Largest position whose value equals the final extremum (later writer wins).
__global__ __launch_bounds__(256) void scatter_arg_kernel(ScatterArgs a) {
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t b, l, f;
    split3(i, a.sp, b, l, f);
    const int64_t t = a.index[b * a.isb + l * a.isl + f * a.isf];
    if (t < 0 || t >= a.size) continue;
    const float x = load_float(a.src, a.dt, i);
    if (x != x) continue;
    const int64_t o = (b * a.size + t) * a.after + f;
    if (float_of(a.key[o]) == x) atomicMax(reinterpret_cast<long long*>(&a.arg[o]), (long long)l);
  }
}

__global__ __launch_bounds__(256) void scatter_finish_kernel(ScatterArgs a) {
  const int64_t total = a.before * a.size * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    float v;
    if (a.reduce == OGN_REDUCE_MIN || a.reduce == OGN_REDUCE_MAX) {
      const float seed = a.has_out ? load_float(a.out, a.dt, i) : 0.f;
      int64_t where = a.arg[i] < 0 ? a.len : a.arg[i];
      if (a.has_out && seed != seed) {
        v = seed;  // a NaN start value is never replaced
        where = a.len;
      } else if (where == a.len) {
        v = seed;
      } else {
        const int64_t f = i % a.after;
        const int64_t b = i / (a.after * a.size);
        v = load_float(a.src, a.dt, (b * a.len + where) * a.after + f);
      }
      a.arg[i] = where;
    } else {
      v = a.acc[i];
      if (a.reduce == OGN_REDUCE_MEAN) {
        const int32_t c = a.count[i];
        if (c > 0) v = v / (float)c;
      }
    }
    store_floats<1>(a.out, a.dt, i, &v);
  }
}

// ------------------------------------------------------------------ grouped softmax
struct GroupArgs {
  const void* src;
  int dt;
  const void* index;  // [len] int32 or int64
  int idx64;
  int64_t before, len, after, groups;
  float* m;  // [before, groups, after]
  float* s;
  uint32_t* key;
  void* out;
  int mode;  // 0 softmax, 1 log_softmax
  Split3 sp;
};

__device__ __forceinline__ int64_t group_of(const GroupArgs& a, int64_t l) {
  return a.idx64 ? static_cast<const int64_t*>(a.index)[l] : (int64_t) static_cast<const int32_t*>(a.index)[l];
}

__global__ __launch_bounds__(256) void group_init_kernel(GroupArgs a) {
  const int64_t total = a.before * a.groups * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    a.key[i] = key_of(-__builtin_inff());
    a.s[i] = 0.f;
  }
}

__global__ __launch_bounds__(256) void group_max_kernel(GroupArgs a) {
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t b, l, f;
    split3(i, a.sp, b, l, f);
    const int64_t g = group_of(a, l);
    if (g < 0 || g >= a.groups) continue;
    const float x = load_float(a.src, a.dt, i);
    if (!(x != x)) atomicMax(&a.key[(b * a.groups + g) * a.after + f], key_of(x));
  }
}

__global__ __launch_bounds__(256) void group_sum_kernel(GroupArgs a) {
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t b, l, f;
    split3(i, a.sp, b, l, f);
    const int64_t g = group_of(a, l);
    if (g < 0 || g >= a.groups) continue;
    const int64_t o = (b * a.groups + g) * a.after + f;
    const float x = load_float(a.src, a.dt, i);
    atomicAdd(&a.s[o], fast_exp(x - clampm(float_of(a.key[o]))));
  }
}

__global__ __launch_bounds__(256) void group_keys_to_max_kernel(GroupArgs a) {
  const int64_t total = a.before * a.groups * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride)
    a.m[i] = float_of(a.key[i]);
}

// softmax: exp(x - clamp(m)) / s;  log_softmax: (x - clamp(m)) - log(s).
// A group holding +inf (m = +inf) is NaN throughout, as torch.softmax gives.
__device__ __forceinline__ float group_apply_one(const GroupArgs& a, float x, float m, float s) {
  const float d = x - clampm(m);
  float v = a.mode == 0 ? fast_exp(d) / s : d - logf(s);
  if (m == __builtin_inff()) v = __builtin_nanf("");
  return v;
}

__global__ __launch_bounds__(256) void group_apply_kernel(GroupArgs a) {
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t b, l, f;
    split3(i, a.sp, b, l, f);
    const int64_t g = group_of(a, l);
    float v = 0.f;
    if (g >= 0 && g < a.groups) {
      const int64_t o = (b * a.groups + g) * a.after + f;
      v = group_apply_one(a, load_float(a.src, a.dt, i), a.m[o], a.s[o]);
    }
    store_floats<1>(a.out, a.dt, i, &v);
  }
}

// One position per element (after == 1, the per-edge score layout): each
// thread takes one 16-byte packet of consecutive positions, their groups
// from the index and m / s per position (neighbouring positions usually
// share a group, so those reads hit the cache).
template <int DT>
__global__ __launch_bounds__(256) void group_apply_rows_kernel(GroupArgs a) {
  using E = Elem<DT>;
  constexpr int NE = E::VEC;
  const int64_t packets = a.before * a.len / NE;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const typename E::S* __restrict__ src = static_cast<const typename E::S*>(a.src);
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < packets; p += stride) {
    const int64_t i0 = p * NE;
    const int64_t b = fdiv(i0, a.sp.len);
    const int64_t l0 = i0 - b * a.len;
    float x[NE], v[NE];
    E::unpack(load16(src + i0), x);
    int64_t g[NE];
    if (a.idx64) {
      const int64_t* ix = static_cast<const int64_t*>(a.index) + l0;
#pragma unroll
      for (int j = 0; j < NE; j += 2) {
        const longlong2 q = *reinterpret_cast<const longlong2*>(ix + j);
        g[j] = q.x;
        g[j + 1] = q.y;
      }
    } else {
      const int32_t* ix = static_cast<const int32_t*>(a.index) + l0;
#pragma unroll
      for (int j = 0; j < NE; j += 4) {
        const int4 q = *reinterpret_cast<const int4*>(ix + j);
        g[j] = q.x;
        g[j + 1] = q.y;
        g[j + 2] = q.z;
        g[j + 3] = q.w;
      }
    }
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      if (g[j] >= 0 && g[j] < a.groups) {
        const int64_t o = b * a.groups + g[j];
        v[j] = group_apply_one(a, x[j], a.m[o], a.s[o]);
      } else {
        v[j] = 0.f;
      }
    }
    store_floats<NE>(a.out, DT, i0, v);
  }
}

// The same, one 16-byte packet of src / out per thread (4 fp32 or 8 fp16 /
// bf16 features of one position) when after is a multiple of the packet:
// the index and the (b, l) split are read once per packet and m / s come in
// 16-byte loads.
template <int DT>
__global__ __launch_bounds__(256) void group_apply_vec_kernel(GroupArgs a) {
  using E = Elem<DT>;
  constexpr int NE = E::VEC;
  const int64_t packets = a.before * a.len * a.after / NE;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const typename E::S* __restrict__ src = static_cast<const typename E::S*>(a.src);
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < packets; p += stride) {
    const int64_t i0 = p * NE;
    int64_t b, l, f;
    split3(i0, a.sp, b, l, f);
    const int64_t g = group_of(a, l);
    float v[NE];
    if (g >= 0 && g < a.groups) {
      float x[NE];
      E::unpack(load16(src + i0), x);
      const int64_t o = (b * a.groups + g) * a.after + f;
#pragma unroll
      for (int j = 0; j < NE; j += 4) {
        const float4 m4 = *reinterpret_cast<const float4*>(a.m + o + j);
        const float4 s4 = *reinterpret_cast<const float4*>(a.s + o + j);
        v[j] = group_apply_one(a, x[j], m4.x, s4.x);
        v[j + 1] = group_apply_one(a, x[j + 1], m4.y, s4.y);
        v[j + 2] = group_apply_one(a, x[j + 2], m4.z, s4.z);
        v[j + 3] = group_apply_one(a, x[j + 3], m4.w, s4.w);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NE; ++j) v[j] = 0.f;
    }
    store_floats<NE>(a.out, DT, i0, v);
  }
}

__global__ __launch_bounds__(256) void group_lse_kernel(GroupArgs a) {
  const int64_t total = a.before * a.groups * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const float v = clampm(a.m[i]) + logf(a.s[i]);
    store_floats<1>(a.out, a.dt, i, &v);
  }
}

// ------------------------------------------------------------------ grouped softmax backward
// softmax:     grad_src = out * (g - T[group]),        T = sum over the group of out * g
// log_softmax: grad_src = g - exp(out) * T[group],     T = sum over the group of g
// logsumexp:   grad_src = g_red[group] * exp(x - out_red[group])   (no group sum)
// Positions whose index is outside [0, groups) get 0.
struct GroupBwdArgs {
  const void* saved;  // softmax / log_softmax: forward output; logsumexp: src
  const void* grad;   // grad of the forward output (same shape as saved; [b, groups, f] for logsumexp)
  const void* red;    // logsumexp: the forward output [b, groups, f]
  int dt;
  const void* index;
  int idx64;
  int64_t before, len, after, groups;
  float* total;  // [b, groups, f] fp32 group sums (zeroed by the caller of the sum pass)
  void* grad_src;
  int mode;  // 0 softmax, 1 log_softmax, 2 logsumexp
  Split3 sp;
};

__device__ __forceinline__ int64_t bwd_group_of(const GroupBwdArgs& a, int64_t l) {
  return a.idx64 ? static_cast<const int64_t*>(a.index)[l] : (int64_t) static_cast<const int32_t*>(a.index)[l];
}

__global__ __launch_bounds__(256) void group_zero_kernel(float* t, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) t[i] = 0.f;
}

// Group sums with one atomic per run of equal targets inside a wavefront:
// a segmented inclusive scan over the 64 lanes (runs are found from the
// neighbour's target, so any index order is correct) leaves each run's sum
// in its last lane.  With a sorted index and after == 1 a wave issues about
// one atomic per group it touches instead of one per element.
__global__ __launch_bounds__(256) void group_bwd_sum_kernel(GroupBwdArgs a) {
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int lane = lane_id();
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~(kWave - 1)); base < total;
       base += stride) {
    const int64_t i = base + lane;
    int64_t key = -1;
    float v = 0.f;
    if (i < total) {
      int64_t b, l, f;
      split3(i, a.sp, b, l, f);
      const int64_t g = bwd_group_of(a, l);
      if (g >= 0 && g < a.groups) {
        key = (b * a.groups + g) * a.after + f;
        const float gv = load_float(a.grad, a.dt, i);
        v = a.mode == 0 ? load_float(a.saved, a.dt, i) * gv : gv;
      }
    }
    const int64_t prev = shfl64(key, lane > 0 ? lane - 1 : 0);
    const int head = (lane == 0 || prev != key) ? lane : 0;
    // start lane of this lane's run = max of the head marks up to this lane
    int start = head;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int o = shfl32(start, lane >= off ? lane - off : lane);
      if (lane >= off) start = start > o ? start : o;
    }
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const float o = shflf(v, lane >= off ? lane - off : lane);
      if (lane - off >= start) v += o;
    }
    const int64_t next = shfl64(key, lane < kWave - 1 ? lane + 1 : lane);
    const bool tail = lane == kWave - 1 || next != key;
    if (tail && key >= 0) atomicAdd(&a.total[key], v);
  }
}

// The per-position terms the backward sums per group, in fp32: out * grad
// (softmax, mode 0) or grad (log_softmax, mode 1).
__global__ __launch_bounds__(256) void group_bwd_messages_kernel(const void* saved, const void* grad, int dt, int64_t n,
                                                                 int mode, float* __restrict__ msg) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gv = load_float(grad, dt, i);
    msg[i] = mode == 0 ? load_float(saved, dt, i) * gv : gv;
  }
}

// The same in 16-byte packets (n a multiple of the packet, aligned buffers).
template <int DT>
__global__ __launch_bounds__(256) void group_bwd_messages_vec_kernel(const void* saved, const void* grad, int64_t n,
                                                                     int mode, float* __restrict__ msg) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr int NE = E::VEC;
  const S_t* __restrict__ sv = static_cast<const S_t*>(saved);
  const S_t* __restrict__ gr = static_cast<const S_t*>(grad);
  const int64_t packets = n / NE;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < packets; p += stride) {
    const int64_t i0 = p * NE;
    float g[NE];
    E::unpack(load16(gr + i0), g);
    if (mode == 0) {
      float y[NE];
      E::unpack(load16(sv + i0), y);
#pragma unroll
      for (int i = 0; i < NE; ++i) g[i] = y[i] * g[i];
    }
    store_floats<NE>(msg, OGN_F32, i0, g);
  }
}

__global__ __launch_bounds__(256) void group_bwd_apply_kernel(GroupBwdArgs a) {
  const int64_t total = a.before * a.len * a.after;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t b, l, f;
    split3(i, a.sp, b, l, f);
    const int64_t g = bwd_group_of(a, l);
    float v = 0.f;
    if (g >= 0 && g < a.groups) {
      const int64_t o = (b * a.groups + g) * a.after + f;
      if (a.mode == 2) {
        const float x = load_float(a.saved, a.dt, i);
        v = load_float(a.grad, a.dt, o) * expf(x - load_float(a.red, a.dt, o));
      } else {
        const float y = load_float(a.saved, a.dt, i);
        const float gv = load_float(a.grad, a.dt, i);
        v = a.mode == 0 ? y * (gv - a.total[o]) : gv - expf(y) * a.total[o];
      }
    }
    store_floats<1>(a.grad_src, a.dt, i, &v);
  }
}

// The same, one 16-byte packet of saved / grad / grad_src per thread (4 fp32
// or 8 fp16 / bf16 features of one position) when after is a multiple of
// the packet: the index and the (b, l) split are read once per packet, the
// group values in 16-byte loads.  Same arithmetic per element as above.
template <int DT>
__global__ __launch_bounds__(256) void group_bwd_apply_vec_kernel(GroupBwdArgs a) {
  using E = Elem<DT>;
  using S_t = typename E::S;
  constexpr int NE = E::VEC;
  const int64_t packets = a.before * a.len * a.after / NE;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const S_t* __restrict__ saved = static_cast<const S_t*>(a.saved);
  const S_t* __restrict__ grad = static_cast<const S_t*>(a.grad);
  const S_t* __restrict__ red = static_cast<const S_t*>(a.red);
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < packets; p += stride) {
    const int64_t i0 = p * NE;
    int64_t b, l, f;
    split3(i0, a.sp, b, l, f);
    const int64_t g = bwd_group_of(a, l);
    float v[NE];
    if (g >= 0 && g < a.groups) {
      const int64_t o = (b * a.groups + g) * a.after + f;
      float x[NE];
      E::unpack(load16(saved + i0), x);
      if (a.mode == 2) {
        float go[NE], ro[NE];
        E::unpack(load16(grad + o), go);
        E::unpack(load16(red + o), ro);
#pragma unroll
        for (int i = 0; i < NE; ++i) v[i] = go[i] * expf(x[i] - ro[i]);
      } else {
        float gv[NE], t[NE];
        E::unpack(load16(grad + i0), gv);
#pragma unroll
        for (int j = 0; j < NE; j += 4) {
          const float4 t4 = *reinterpret_cast<const float4*>(a.total + o + j);
          t[j] = t4.x;
          t[j + 1] = t4.y;
          t[j + 2] = t4.z;
          t[j + 3] = t4.w;
        }
#pragma unroll
        for (int i = 0; i < NE; ++i) v[i] = a.mode == 0 ? x[i] * (gv[i] - t[i]) : gv[i] - expf(x[i]) * t[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < NE; ++i) v[i] = 0.f;
    }
    store_floats<NE>(a.grad_src, DT, i0, v);
  }
}

unsigned grid_for(int64_t total) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((total + 255) / 256, 65536));
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace
}  // namespace ogn

using namespace ogn;

extern "C" {

size_t ogn_scatter_atomic_workspace_size(int64_t before, int64_t size, int64_t after, int reduce) {
  const size_t cells = (size_t)std::max<int64_t>(before, 0) * std::max<int64_t>(size, 0) * std::max<int64_t>(after, 0);
  // sized for the widest accumulator (8 bytes: integer and float64 dtypes)
  return std::max(align256(cells * 4) + (reduce == OGN_REDUCE_MEAN ? align256(cells * 4) : 0) + 256,
                  exact_scatter_workspace_size((int64_t)cells, reduce));
}

int ogn_scatter_atomic(const void* src, int dtype, const int64_t* index, int64_t index_stride_before,
                       int64_t index_stride_len, int64_t index_stride_after, int64_t before, int64_t len,
                       int64_t after, int64_t size, void* out, int64_t* arg, int reduce, int has_out,
                       void* workspace, size_t workspace_bytes, void* stream) {
  if (before < 0 || len < 0 || after < 0 || size < 0) return fail(OGN_EINVAL, "ogn_scatter_atomic: negative size");
  const bool exact = is_exact_dtype(dtype);
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16 && !exact)
    return fail(OGN_EUNSUPPORTED, "ogn_scatter_atomic: unsupported dtype");
  if (reduce < OGN_REDUCE_SUM || reduce > OGN_REDUCE_PROD)
    return fail(OGN_EINVAL, "ogn_scatter_atomic: reduce must be sum/mean/min/max/prod");
  const int64_t cells = before * size * after;
  if (cells == 0) return OGN_OK;
  if (!out || (len > 0 && (!src || !index))) return fail(OGN_EINVAL, "ogn_scatter_atomic: null pointer");
  if ((reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX) && !arg)
    return fail(OGN_EINVAL, "ogn_scatter_atomic: min/max need an arg buffer");
  if (!workspace || workspace_bytes < ogn_scatter_atomic_workspace_size(before, size, after, reduce))
    return fail(OGN_EINVAL, "ogn_scatter_atomic: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (exact)
    return exact_scatter_atomic(src, dtype, index, index_stride_before, index_stride_len, index_stride_after, before,
                                len, after, size, out, arg, reduce, has_out, workspace, s);
  ScatterArgs a{};
  a.src = src;
  a.dt = dtype;
  a.index = index;
  a.isb = index_stride_before;
  a.isl = index_stride_len;
  a.isf = index_stride_after;
  a.before = before;
  a.len = len;
  a.after = after;
  a.sp = make_split3(len, after);
  a.size = size;
  a.out = out;
  a.arg = (reduce == OGN_REDUCE_MIN || reduce == OGN_REDUCE_MAX) ? arg : nullptr;
  char* ws = static_cast<char*>(workspace);
  a.acc = reinterpret_cast<float*>(ws);
  a.key = reinterpret_cast<uint32_t*>(ws);
  a.count = reduce == OGN_REDUCE_MEAN ? reinterpret_cast<int32_t*>(ws + align256(cells * 4)) : nullptr;
  a.reduce = reduce;
  a.has_out = has_out;
  a.limit = dtype == OGN_F32 ? 3.4028234663852886e38f : (dtype == OGN_F16 ? 65504.f : 3.3895313892515355e38f);
  {
    TimedLaunch t("scatter_init", s);
    hipLaunchKernelGGL(scatter_init_kernel, dim3(grid_for(cells)), dim3(256), 0, s, a);
  }
  const int64_t total = before * len * after;
  if (total > 0) {
    TimedLaunch t("scatter_main", s);
    hipLaunchKernelGGL(scatter_main_kernel, dim3(grid_for(total)), dim3(256), 0, s, a);
  }
  if (a.arg != nullptr && total > 0) {
    TimedLaunch t("scatter_arg", s);
    hipLaunchKernelGGL(scatter_arg_kernel, dim3(grid_for(total)), dim3(256), 0, s, a);
  }
  {
    TimedLaunch t("scatter_finish", s);
    hipLaunchKernelGGL(scatter_finish_kernel, dim3(grid_for(cells)), dim3(256), 0, s, a);
  }
  return check_launch("ogn_scatter_atomic");
}

int ogn_group_stats_atomic(const void* src, int dtype, const void* index, int index_dtype, int64_t before,
                           int64_t len, int64_t after, int64_t groups, float* m, float* s_out, uint32_t* scratch_key,
                           void* stream) {
  if (before < 0 || len < 0 || after < 0 || groups < 0)
    return fail(OGN_EINVAL, "ogn_group_stats_atomic: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_group_stats_atomic: dtype must be float32, float16 or bfloat16");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_group_stats_atomic: index dtype must be int32 or int64");
  const int64_t cells = before * groups * after;
  if (cells == 0) return OGN_OK;
  if (!m || !s_out || !scratch_key || (len > 0 && (!src || !index)))
    return fail(OGN_EINVAL, "ogn_group_stats_atomic: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  GroupArgs a{};
  a.src = src;
  a.dt = dtype;
  a.index = index;
  a.idx64 = index_dtype == OGN_I64;
  a.before = before;
  a.len = len;
  a.after = after;
  a.sp = make_split3(len, after);
  a.groups = groups;
  a.m = m;
  a.s = s_out;
  a.key = scratch_key;
  const int64_t total = before * len * after;
  TimedLaunch t("group_stats", st);
  hipLaunchKernelGGL(group_init_kernel, dim3(grid_for(cells)), dim3(256), 0, st, a);
  if (total > 0) hipLaunchKernelGGL(group_max_kernel, dim3(grid_for(total)), dim3(256), 0, st, a);
  if (total > 0) hipLaunchKernelGGL(group_sum_kernel, dim3(grid_for(total)), dim3(256), 0, st, a);
  hipLaunchKernelGGL(group_keys_to_max_kernel, dim3(grid_for(cells)), dim3(256), 0, st, a);
  return check_launch("ogn_group_stats_atomic");
}

int ogn_group_softmax_apply(const void* src, int dtype, const void* index, int index_dtype, int64_t before,
                            int64_t len, int64_t after, int64_t groups, const float* m, const float* s,
                            void* out, int log_softmax, void* stream) {
  if (before < 0 || len < 0 || after < 0 || groups < 0)
    return fail(OGN_EINVAL, "ogn_group_softmax_apply: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_group_softmax_apply: dtype must be float32, float16 or bfloat16");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_group_softmax_apply: index dtype must be int32 or int64");
  const int64_t total = before * len * after;
  if (total == 0) return OGN_OK;
  if (!src || !index || !out || (groups > 0 && (!m || !s)))
    return fail(OGN_EINVAL, "ogn_group_softmax_apply: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  GroupArgs a{};
  a.src = src;
  a.dt = dtype;
  a.index = index;
  a.idx64 = index_dtype == OGN_I64;
  a.before = before;
  a.len = len;
  a.after = after;
  a.sp = make_split3(len, after);
  a.groups = groups;
  a.m = const_cast<float*>(m);
  a.s = const_cast<float*>(s);
  a.out = out;
  a.mode = log_softmax ? 1 : 0;
  TimedLaunch t("group_apply", st);
  const int ne = 16 / dtype_size(dtype);
  const bool vec = after % ne == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)out % 16 == 0 &&
                   (uintptr_t)m % 16 == 0 && (uintptr_t)s % 16 == 0;
  const bool rows_vec = after == 1 && len % ne == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)out % 16 == 0 &&
                        (uintptr_t)index % 16 == 0;
  if (rows_vec) {
    const dim3 g(grid_for(total / ne));
    if (dtype == OGN_F32) hipLaunchKernelGGL(group_apply_rows_kernel<OGN_F32>, g, dim3(256), 0, st, a);
    else if (dtype == OGN_F16) hipLaunchKernelGGL(group_apply_rows_kernel<OGN_F16>, g, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(group_apply_rows_kernel<OGN_BF16>, g, dim3(256), 0, st, a);
  } else if (vec) {
    const dim3 g(grid_for(total / ne));
    if (dtype == OGN_F32) hipLaunchKernelGGL(group_apply_vec_kernel<OGN_F32>, g, dim3(256), 0, st, a);
    else if (dtype == OGN_F16) hipLaunchKernelGGL(group_apply_vec_kernel<OGN_F16>, g, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(group_apply_vec_kernel<OGN_BF16>, g, dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL(group_apply_kernel, dim3(grid_for(total)), dim3(256), 0, st, a);
  }
  return check_launch("ogn_group_softmax_apply");
}

int ogn_group_lse_from_stats(const float* m, const float* s, int64_t cells, void* out, int dtype, void* stream) {
  if (cells < 0) return fail(OGN_EINVAL, "ogn_group_lse_from_stats: negative size");
  if (cells == 0) return OGN_OK;
  if (!m || !s || !out) return fail(OGN_EINVAL, "ogn_group_lse_from_stats: null pointer");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_group_lse_from_stats: dtype must be float32, float16 or bfloat16");
  hipStream_t st = static_cast<hipStream_t>(stream);
  GroupArgs a{};
  a.before = 1;
  a.groups = cells;
  a.after = 1;
  a.m = const_cast<float*>(m);
  a.s = const_cast<float*>(s);
  a.out = out;
  a.dt = dtype;
  TimedLaunch t("group_lse", st);
  hipLaunchKernelGGL(group_lse_kernel, dim3(grid_for(cells)), dim3(256), 0, st, a);
  return check_launch("ogn_group_lse_from_stats");
}

int ogn_group_bwd_messages(const void* saved, const void* grad, int dtype, int64_t n, int mode, float* msg,
                           void* stream) {
  if (n < 0) return fail(OGN_EINVAL, "ogn_group_bwd_messages: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_group_bwd_messages: dtype must be float32, float16 or bfloat16");
  if (mode != 0 && mode != 1) return fail(OGN_EINVAL, "ogn_group_bwd_messages: mode must be 0 or 1");
  if (n == 0) return OGN_OK;
  if (!grad || !msg || (mode == 0 && !saved)) return fail(OGN_EINVAL, "ogn_group_bwd_messages: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  TimedLaunch t("group_bwd_messages", st);
  const int ne = 16 / dtype_size(dtype);
  auto al = [](const void* q) { return (uintptr_t)q % 16 == 0; };
  if (n % ne == 0 && al(grad) && al(msg) && (mode == 1 || al(saved))) {
    const dim3 g(grid_for(n / ne));
    if (dtype == OGN_F32) hipLaunchKernelGGL(group_bwd_messages_vec_kernel<OGN_F32>, g, dim3(256), 0, st, saved, grad, n, mode, msg);
    else if (dtype == OGN_F16) hipLaunchKernelGGL(group_bwd_messages_vec_kernel<OGN_F16>, g, dim3(256), 0, st, saved, grad, n, mode, msg);
    else hipLaunchKernelGGL(group_bwd_messages_vec_kernel<OGN_BF16>, g, dim3(256), 0, st, saved, grad, n, mode, msg);
  } else {
    hipLaunchKernelGGL(group_bwd_messages_kernel, dim3(grid_for(n)), dim3(256), 0, st, saved, grad, dtype, n, mode, msg);
  }
  return check_launch("ogn_group_bwd_messages");
}

int ogn_group_softmax_backward(const void* saved, const void* grad, const void* reduced, int dtype,
                               const void* index, int index_dtype, int64_t before, int64_t len, int64_t after,
                               int64_t groups, int mode, void* grad_src, float* workspace, size_t workspace_bytes,
                               void* stream) {
  if (before < 0 || len < 0 || after < 0 || groups < 0)
    return fail(OGN_EINVAL, "ogn_group_softmax_backward: negative size");
  if (dtype != OGN_F32 && dtype != OGN_F16 && dtype != OGN_BF16)
    return fail(OGN_EUNSUPPORTED, "ogn_group_softmax_backward: dtype must be float32, float16 or bfloat16");
  if (index_dtype != OGN_I32 && index_dtype != OGN_I64)
    return fail(OGN_EINVAL, "ogn_group_softmax_backward: index dtype must be int32 or int64");
  const bool given = (mode & OGN_GROUP_BWD_TOTALS_GIVEN) != 0;
  mode &= ~OGN_GROUP_BWD_TOTALS_GIVEN;
  if (mode < 0 || mode > 2) return fail(OGN_EINVAL, "ogn_group_softmax_backward: mode must be 0, 1 or 2");
  const int64_t total = before * len * after;
  if (total == 0) return OGN_OK;
  const int64_t cells = before * groups * after;
  if (!saved || !grad || !index || !grad_src || (mode == 2 && !reduced))
    return fail(OGN_EINVAL, "ogn_group_softmax_backward: null pointer");
  if (mode != 2 && cells > 0 && (!workspace || workspace_bytes < (size_t)cells * sizeof(float)))
    return fail(OGN_EINVAL, "ogn_group_softmax_backward: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  GroupBwdArgs a{};
  a.saved = saved;
  a.grad = grad;
  a.red = reduced;
  a.dt = dtype;
  a.index = index;
  a.idx64 = index_dtype == OGN_I64;
  a.before = before;
  a.len = len;
  a.after = after;
  a.sp = make_split3(len, after);
  a.groups = groups;
  a.total = workspace;
  a.grad_src = grad_src;
  a.mode = mode;
  if (mode != 2 && cells > 0 && !given) {
    TimedLaunch t("group_bwd_sum", st);
    hipLaunchKernelGGL(group_zero_kernel, dim3(grid_for(cells)), dim3(256), 0, st, workspace, cells);
    hipLaunchKernelGGL(group_bwd_sum_kernel, dim3(grid_for(total)), dim3(256), 0, st, a);
  }
  {
    TimedLaunch t("group_bwd_apply", st);
    const bool vdt = dtype == OGN_F32 || dtype == OGN_F16 || dtype == OGN_BF16;
    const int ne = vdt ? 16 / dtype_size(dtype) : 1;
    auto al = [](const void* q) { return (uintptr_t)q % 16 == 0; };
    const bool vec = vdt && after % ne == 0 && al(saved) && al(grad) && al(grad_src) &&
                     (mode == 2 ? al(reduced) : al(workspace));
    const dim3 g(grid_for(vec ? total / ne : total));
    if (vec && dtype == OGN_F32) hipLaunchKernelGGL(group_bwd_apply_vec_kernel<OGN_F32>, g, dim3(256), 0, st, a);
    else if (vec && dtype == OGN_F16) hipLaunchKernelGGL(group_bwd_apply_vec_kernel<OGN_F16>, g, dim3(256), 0, st, a);
    else if (vec) hipLaunchKernelGGL(group_bwd_apply_vec_kernel<OGN_BF16>, g, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(group_bwd_apply_kernel, g, dim3(256), 0, st, a);
  }
  return check_launch("ogn_group_softmax_backward");
}

}  // extern "C"
