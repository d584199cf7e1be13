// Scalar conversions shared by the kernels.  Rounding is IEEE round-to-nearest-
// even everywhere, matching torch's CPU casts that the reference tests compare with.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asc {

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// v_cvt_pk_bf16_f32 on gfx950: IEEE round-to-nearest-even, NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  _Float16 v = static_cast<_Float16>(f);  // v_cvt_f16_f32 rounds to nearest even
  return __builtin_bit_cast(uint16_t, v);
}

// Forces `v` to be rounded to fp32 and held in a register.  Without it the
// compiler may fuse a following fp32 -> fp16 conversion into the producing
// multiply (v_fma_mixlo_f16), rounding the exact product once instead of
// rounding to fp32 first -- a different result in rare ties.
__device__ __forceinline__ float materialize(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

}  // namespace asc
