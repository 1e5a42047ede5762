// Shared host/device helpers for the mvattn kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mvattn.h"

namespace mv {

// ---------------------------------------------------------------- errors --

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks the launch status of the kernels just enqueued.
int check_launch(const char* what);

// ------------------------------------------------------------- dtypes ----

// Storage types: 16-bit floats are moved around as raw uint16_t; only the
// conversions below interpret them.
template <int DTYPE> struct Elem;
template <> struct Elem<MV_DTYPE_F32> { using raw = float; static constexpr int bytes = 4; };
template <> struct Elem<MV_DTYPE_F16> { using raw = uint16_t; static constexpr int bytes = 2; };
template <> struct Elem<MV_DTYPE_BF16> { using raw = uint16_t; static constexpr int bytes = 2; };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, x));
}
// Round-to-nearest-even conversions (hardware v_cvt on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

template <int DTYPE> __device__ __forceinline__ float to_f32(typename Elem<DTYPE>::raw x);
template <> __device__ __forceinline__ float to_f32<MV_DTYPE_F32>(float x) { return x; }
template <> __device__ __forceinline__ float to_f32<MV_DTYPE_F16>(uint16_t x) { return f16_to_f32(x); }
template <> __device__ __forceinline__ float to_f32<MV_DTYPE_BF16>(uint16_t x) { return bf16_to_f32(x); }

template <int DTYPE> __device__ __forceinline__ typename Elem<DTYPE>::raw from_f32(float x);
template <> __device__ __forceinline__ float from_f32<MV_DTYPE_F32>(float x) { return x; }
template <> __device__ __forceinline__ uint16_t from_f32<MV_DTYPE_F16>(float x) { return f32_to_f16(x); }
template <> __device__ __forceinline__ uint16_t from_f32<MV_DTYPE_BF16>(float x) { return f32_to_bf16(x); }

// ------------------------------------------------------------- misc ------

__host__ __device__ constexpr int ilog2_exact(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

inline int dtype_bytes(int dtype) {
  return dtype == MV_DTYPE_F32 ? 4 : (dtype == MV_DTYPE_F16 || dtype == MV_DTYPE_BF16) ? 2 : 0;
}

}  // namespace mv
