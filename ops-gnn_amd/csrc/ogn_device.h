// Device-side helpers shared by every ops-gnn gfx950 kernel: element codecs,
// 16-byte packet loads/stores, wavefront cross-lane primitives and the
// thread-local error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/ogn.h"

namespace ogn {

constexpr int kWave = 64;

// ---------------------------------------------------------------- errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// RAII bracket of one kernel launch for the opt-in timer (ogn_timing_enable).
class TimedLaunch {
 public:
  TimedLaunch(const char* name, hipStream_t stream);
  ~TimedLaunch();
  TimedLaunch(const TimedLaunch&) = delete;
  TimedLaunch& operator=(const TimedLaunch&) = delete;

 private:
  hipStream_t stream_;
  hipEvent_t start_ = nullptr, stop_ = nullptr;
  std::string name_;
  bool active_ = false;
};

// ---------------------------------------------------------------- exponential
// e^x through the hardware base-2 exponential (v_exp_f32): exp2(x * log2 e).
// The rounded product adds a relative error of about |x| * 2^-24 to the
// ~1 ulp of exp2, so terms far below the largest one (|x| large) carry a
// larger relative but negligible absolute error -- the regime of log-sum-exp
// and softmax, where every term is exp(x - max) <= 1.  exp2(+-inf) and NaN
// behave as IEEE.
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// ---------------------------------------------------------------- invariant division
// n / d for 0 <= n < 2^63 and a divisor d >= 1 fixed at launch:
// q = (umulhi(n, m) + n) >> l with l = ceil(log2 d) and
// m = floor(2^64 (2^l - d) / d) + 1 (T. Granlund, P. Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994, section 4).  Replaces
// the software 64-bit division in per-element index arithmetic.
struct FastDiv {
  uint64_t d;
  uint64_t m;
  int l;
};

inline FastDiv make_fastdiv(int64_t d) {
  FastDiv f{};
  f.d = (uint64_t)(d < 1 ? 1 : d);
  f.l = 0;
  while ((1ull << f.l) < f.d) ++f.l;
  const unsigned __int128 one = 1;
  f.m = (uint64_t)(((one << 64) * ((one << f.l) - f.d)) / f.d + 1);
  return f;
}

__device__ __forceinline__ int64_t fdiv(int64_t n, const FastDiv& f) {
  const uint64_t hi = __umul64hi((uint64_t)n, f.m);
  return (int64_t)((hi + (uint64_t)n) >> f.l);
}

// i = (b * len + l) * after + k  ->  (b, l, k) for a [before, len, after] tensor.
struct Split3 {
  FastDiv after, len;
};

inline Split3 make_split3(int64_t len, int64_t after) { return Split3{make_fastdiv(after), make_fastdiv(len)}; }

__device__ __forceinline__ void split3(int64_t i, const Split3& s, int64_t& b, int64_t& l, int64_t& k) {
  const int64_t t = fdiv(i, s.after);
  k = i - t * (int64_t)s.after.d;
  b = fdiv(t, s.len);
  l = t - b * (int64_t)s.len.d;
}

// ---------------------------------------------------------------- codecs
// bf16 <-> fp32: a bf16 is the high half of an fp32; narrowing rounds to
// nearest-even on the 16 discarded bits and keeps NaNs quiet.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)b);
  return (float)h;
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

// Element traits for the floating storage types.  VEC = elements in 16 B.
template <int DT> struct Elem;
template <> struct Elem<OGN_F32> {
  using S = float;
  static constexpr int VEC = 4;
  __device__ static __forceinline__ float load1(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
  }
  __device__ static __forceinline__ void unpack(const uint4& v, float* x) {
    x[0] = __uint_as_float(v.x); x[1] = __uint_as_float(v.y);
    x[2] = __uint_as_float(v.z); x[3] = __uint_as_float(v.w);
  }
};
template <> struct Elem<OGN_F16> {
  using S = uint16_t;
  static constexpr int VEC = 8;
  __device__ static __forceinline__ float load1(const void* p, int64_t i) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ static __forceinline__ void unpack(const uint4& v, float* x) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
      x[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  }
};
template <> struct Elem<OGN_BF16> {
  using S = uint16_t;
  static constexpr int VEC = 8;
  __device__ static __forceinline__ float load1(const void* p, int64_t i) {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ static __forceinline__ void unpack(const uint4& v, float* x) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};

// int8 features (torch_sparse SpMM int8 -> int32): values widen to float
// exactly; products of two int8 values (|x w| <= 2^14) are exact in fp32.
template <> struct Elem<OGN_I8> {
  using S = int8_t;
  static constexpr int VEC = 16;
  __device__ static __forceinline__ float load1(const void* p, int64_t i) {
    return (float)static_cast<const int8_t*>(p)[i];
  }
  __device__ static __forceinline__ void unpack(const uint4& v, float* x) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * i + j] = (float)(int8_t)((w[i] >> (8 * j)) & 0xffu);
    }
  }
};

__host__ __device__ constexpr int dtype_size(int dt) {
  return dt == OGN_F32 || dt == OGN_I32 ? 4
       : dt == OGN_I64 || dt == OGN_F64 ? 8
       : dt == OGN_I8 || dt == OGN_U8 ? 1 : 2;
}

// Store n consecutive fp32 values into an output of runtime dtype `dt`
// (fp32/fp16/bf16) at element offset `off`.  `aligned` promises that the
// address is n*size aligned so that one wide store can be used.
// NT = non-temporal stores (streaming outputs that are not read back soon).
template <int N, bool NT = false>
__device__ __forceinline__ void store_floats(void* out, int dt, int64_t off,
                                             const float* v) {
  if (dt == OGN_I32) {
    int32_t* p = static_cast<int32_t*>(out) + off;
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = (int32_t)v[i];
    return;
  }
  if (dt == OGN_F32) {
    float* p = static_cast<float*>(out) + off;
    if constexpr (N % 4 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 4) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const f32x4 q = {v[i], v[i + 1], v[i + 2], v[i + 3]};
        if constexpr (NT) __builtin_nontemporal_store(q, reinterpret_cast<f32x4*>(p + i));
        else *reinterpret_cast<f32x4*>(p + i) = q;
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) p[i] = v[i];
    }
  } else {
    uint16_t* p = static_cast<uint16_t*>(out) + off;
    uint16_t h[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
      h[i] = dt == OGN_F16 ? f32_to_f16_bits(v[i]) : f32_to_bf16_bits(v[i]);
    if constexpr (N % 8 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 8) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 q = {h[i] | ((uint32_t)h[i + 1] << 16), h[i + 2] | ((uint32_t)h[i + 3] << 16),
                         h[i + 4] | ((uint32_t)h[i + 5] << 16), h[i + 6] | ((uint32_t)h[i + 7] << 16)};
        if constexpr (NT) __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(p + i));
        else *reinterpret_cast<u32x4*>(p + i) = q;
      }
    } else if constexpr (N % 4 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 4)
        *reinterpret_cast<uint2*>(p + i) = make_uint2(
            h[i] | ((uint32_t)h[i + 1] << 16), h[i + 2] | ((uint32_t)h[i + 3] << 16));
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) p[i] = h[i];
    }
  }
}

__device__ __forceinline__ float load_float(const void* p, int dt, int64_t i) {
  switch (dt) {
    case OGN_F16: return Elem<OGN_F16>::load1(p, i);
    case OGN_BF16: return Elem<OGN_BF16>::load1(p, i);
    default: return Elem<OGN_F32>::load1(p, i);
  }
}

// ---------------------------------------------------------------- lanes
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Wave-uniform broadcast of lane `src` (src must be wave-uniform).
__device__ __forceinline__ int64_t readlane64(int64_t v, int src) {
  const int lo = __builtin_amdgcn_readlane((int)(uint32_t)v, src);
  const int hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), src);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ int32_t readlane64(int32_t v, int src) {
  return __builtin_amdgcn_readlane(v, src);
}

// Per-lane gather from another lane (ds_bpermute); all lanes must be active.
__device__ __forceinline__ int32_t shfl32(int32_t v, int src) {
  return __builtin_amdgcn_ds_bpermute(src << 2, v);
}
__device__ __forceinline__ float shflf(float v, int src) {
  return __int_as_float(shfl32(__float_as_int(v), src));
}
__device__ __forceinline__ int64_t shfl64(int64_t v, int src) {
  const int lo = shfl32((int32_t)(uint32_t)v, src);
  const int hi = shfl32((int32_t)(uint32_t)((uint64_t)v >> 32), src);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ int32_t shfl64(int32_t v, int src) { return shfl32(v, src); }
__device__ __forceinline__ double shfld(double v, int src) {
  return __longlong_as_double(shfl64((int64_t)__double_as_longlong(v), src));
}

// Value of lane (lane ^ OFF), OFF a power of two below 64: ds_swizzle in
// xor mode (no address register) within 32-lane halves, ds_bpermute across
// them.
template <int OFF>
__device__ __forceinline__ int32_t xor_shfl32(int32_t v) {
  static_assert(OFF >= 1 && OFF <= 32 && (OFF & (OFF - 1)) == 0, "OFF must be a power of two <= 32");
  if constexpr (OFF == 32) {
    return __builtin_amdgcn_ds_bpermute((int)((threadIdx.x ^ 32) & 63) << 2, v);
  } else {
    return __builtin_amdgcn_ds_swizzle(v, (OFF << 10) | 0x1f);
  }
}
template <int OFF>
__device__ __forceinline__ float xor_shfl(float v) {
  return __int_as_float(xor_shfl32<OFF>(__float_as_int(v)));
}
template <int OFF>
__device__ __forceinline__ int32_t xor_shfl(int32_t v) {
  return xor_shfl32<OFF>(v);
}
template <int OFF>
__device__ __forceinline__ double xor_shfl(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)xor_shfl32<OFF>((int32_t)(uint32_t)u);
  const uint32_t hi = (uint32_t)xor_shfl32<OFF>((int32_t)(uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// This wavefront's index in its block, as a wave-uniform (scalar) value:
// the compiler does not know that threadIdx.x >> 6 is uniform, and code
// indexed by it otherwise runs as vector code with serialised scalar loads.
__device__ __forceinline__ int wave_in_block() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__device__ __forceinline__ uint4 load16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
// A 16-byte packet read exactly once (the contiguous source of a segment
// reduction): a non-temporal load, which streams past the caches.  Reading
// 544 MB in 136 KB per-wave chunks of 512-byte rows on one MI355X: 91.6 us
// with plain loads, 81.4 us non-temporal.
template <bool NT>
__device__ __forceinline__ uint4 load16_once(const void* p) {
  if constexpr (NT) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return load16(p);
  }
}
template <typename T>
__device__ __forceinline__ T load_stream(const T* p) {
  return __builtin_nontemporal_load(p);
}

}  // namespace ogn
