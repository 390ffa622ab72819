// Internal helpers shared by the gfx950 kernels of libwide_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <initializer_list>
#include <type_traits>

#include "wc_abi.h"

namespace wc {

// ---------------------------------------------------------------------------
// error reporting (host side)
// ---------------------------------------------------------------------------
int32_t set_error(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Checks the launch status of the last kernel on this thread; returns 0 or the
// hipError_t (recorded in wc_last_error).
int32_t check_launch(const char* what);

#define WC_REQUIRE(cond, code, ...)                 \
  do {                                              \
    if (!(cond)) return ::wc::set_error((code), __VA_ARGS__); \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// elements * element size as unsigned bytes, for alignment tests of caller strides: the value
// mod 16 is exact however large the stride (unsigned arithmetic wraps by definition)
inline uint64_t ubytes(int64_t elems, int es) { return static_cast<uint64_t>(elems) * static_cast<uint64_t>(es); }

// every value within int32 range: checked before sizes enter derived arithmetic
inline bool fits_i32(std::initializer_list<int64_t> f) {
  for (int64_t x : f)
    if (x < -0x7fffffffll || x > 0x7fffffffll) return false;
  return true;
}

// product of sizes known to be >= 0, saturated at INT64_MAX: a limit check on it fails for
// sizes whose product does not fit instead of comparing a wrapped value
inline int64_t mul_sat(std::initializer_list<int64_t> f) {
  int64_t r = 1;
  for (int64_t x : f)
    if (__builtin_mul_overflow(r, x, &r)) return INT64_MAX;
  return r;
}

inline int dtype_size(int32_t dt) {
  switch (dt) {
    case WC_F32: return 4;
    case WC_BF16: return 2;
    case WC_F16: return 2;
    default: return 0;
  }
}

inline const char* dtype_name(int32_t dt) {
  switch (dt) {
    case WC_F32: return "f32";
    case WC_BF16: return "bf16";
    case WC_F16: return "f16";
    default: return "?";
  }
}

inline bool aligned(const void* p, int64_t a) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(a)) == 0;
}

// ---------------------------------------------------------------------------
// device-side element conversions
// ---------------------------------------------------------------------------
typedef __bf16 bf16;
typedef _Float16 f16;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<bf16>(bf16 v) { return static_cast<float>(v); }
template <> __device__ __forceinline__ float to_f32<f16>(f16 v) { return static_cast<float>(v); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
// round-to-nearest-even, as torch's float -> bfloat16 / half casts
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return static_cast<bf16>(v); }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// two floats -> two round-to-nearest-even bf16 in one dword (v_cvt_pk_bf16_f32), low half first
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// v_mfma_f32_16x16x32 on 16-bit operands carried as raw 16-byte fragments: the bf16 or
// the fp16 instruction by the element type T
template <typename T>
__device__ __forceinline__ f32x4 mma16(bf16x8 a, bf16x8 b, f32x4 c) {
  if constexpr (std::is_same<T, f16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// the low / high bf16 of a dword as a float (exact)
__device__ __forceinline__ float bf16_lo(uint32_t v) { return __builtin_bit_cast(float, v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __builtin_bit_cast(float, v & 0xffff0000u); }

// wave64 reductions (all lanes receive the result)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// reduction over groups of `width` adjacent lanes (width a power of two <= 64)
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------------------
// unsigned 32-bit division by a run-time constant (multiply-high + shift),
// valid for dividends < 2^31.  q = (umulhi(x, mul) + x) >> shift.
// ---------------------------------------------------------------------------
struct FastDiv {
  uint32_t d, mul, shift;
};

// d > 0 (entry points reject zero divisors; d == 0 gives a divisor that divides nothing
// rather than a host division by zero)
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  if (d == 0) {
    f.mul = 0;
    f.shift = 0;
    return f;
  }
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.shift = s;
  f.mul = static_cast<uint32_t>(((1ull << 32) * ((1ull << s) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t x, const FastDiv& f) {
  return static_cast<uint32_t>((static_cast<uint64_t>(__umulhi(x, f.mul)) + x) >> f.shift);
}

// Compute units of the current device (cached per device id); 0 if the query fails.
inline int device_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 0;
    cache[dev] = v;
  }
  return cache[dev];
}

// Largest power-of-two byte width <= 16 dividing every given value.
inline int common_vec_bytes(std::initializer_list<uint64_t> vals) {
  int v = 16;
  for (uint64_t x : vals)
    while (v > 1 && (x % static_cast<uint64_t>(v)) != 0) v >>= 1;
  return v;
}

}  // namespace wc
