// Device code of the elementwise asc2 kernels beside vadd:
//   leaky_relu_kernel  python/test/asc2/kernels/test_leaky_relu.py:16-26
//                      out = where(x >= 0, x, x * alpha)
//   vmuladd_kernel     python/test/asc2/kernels/test_vmuladd.py:16-31
//                      out = x * y + z (multiply and add rounded separately)
//   gelu_kernel        python/test/asc2/kernels/test_gelu.py:19-33
//                      grid-stride rows, tanh-form or erf-form GELU
// Shared by the library (elementwise.hip, launched through asc_leaky_relu /
// asc_vmuladd / asc_gelu_rows_f32) and the standalone gfx950 code object
// (co/asc2_elementwise.hip, loaded with hipModuleLoad by the asc2 launch path),
// so both launch paths run the same instructions.  Both build it with
// -ffp-contract=off: no multiply-add is fused.
//
// leaky_relu and vmuladd stream like vadd: HBM-bound, 16-byte non-temporal
// vectors, four per thread per operand, the physical grid sized by the covered
// length (the logical grid only decides how far the writes reach:
// [0, min(size, grid * tile_per_block * tile_size))).  Unaligned buffers and
// the sub-vector tail take an element-wise body with the same arithmetic.
#pragma once

#include <math.h>

#include "common.h"
#include "numeric.h"

namespace asc {
namespace elementwise {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int kScalarMaxBlocks = 4096;  // the element-wise body is grid-stride
constexpr int kGeluMaxBlocks = 8192;    // gelu rows are grid-stride as well

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---- element types: storage T, conversion to and from fp32 (RNE)
struct F32 {
  using T = float;
  __device__ static float in(float v) { return v; }
  __device__ static float out(float v) { return v; }
};
struct F16 {
  using T = uint16_t;
  __device__ static float in(uint16_t v) { return asc::f16_to_f32(v); }
  __device__ static uint16_t out(float v) { return asc::f32_to_f16_rne(v); }
};
struct BF16 {
  using T = uint16_t;
  __device__ static float in(uint16_t v) { return asc::bf16_to_f32(v); }
  __device__ static uint16_t out(float v) { return asc::f32_to_bf16_rne(v); }
};

// where(x >= 0, x, x * alpha): the product is formed in fp32 and rounded once
// to the element type (exact before rounding for 16-bit inputs and a 16-bit
// alpha); a non-negative x (including -0) passes through unchanged.
template <class E>
struct LeakyRelu {
  using T = typename E::T;
  static constexpr int kIn = 1;
  float alpha;
  __device__ T operator()(T x) const {
    const float xf = E::in(x);
    return xf >= 0.f ? x : E::out(xf * alpha);
  }
};

// x * y + z with the product rounded to the element type before the add.
template <class E>
struct MulAdd {
  using T = typename E::T;
  static constexpr int kIn = 3;
  __device__ T operator()(T x, T y, T z) const {
    const T p = E::out(E::in(x) * E::in(y));
    return E::out(E::in(p) + E::in(z));
  }
};

template <class Op>
__device__ __forceinline__ u32x4 apply_vec(const Op& op, u32x4 a, u32x4 b, u32x4 c) {
  using T = typename Op::T;
  constexpr int kN = 16 / sizeof(T);
  T ea[kN], eb[kN], ec[kN], eo[kN];
  __builtin_memcpy(ea, &a, 16);
  __builtin_memcpy(eb, &b, 16);
  __builtin_memcpy(ec, &c, 16);
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    if constexpr (Op::kIn == 1) {
      eo[i] = op(ea[i]);
    } else {
      eo[i] = op(ea[i], eb[i], ec[i]);
    }
  }
  u32x4 o;
  __builtin_memcpy(&o, eo, 16);
  return o;
}

// out[v] = op(in0[v], in1[v], in2[v]) for 16-byte vectors v < n_vec (unused
// inputs are not read); a workgroup of kThreads covers kThreads * kUnroll vectors.
template <class Op>
__device__ __forceinline__ void map_vec_body(const Op& op, const u32x4* __restrict__ in0,
                                             const u32x4* __restrict__ in1, const u32x4* __restrict__ in2,
                                             u32x4* __restrict__ out, int64_t n_vec) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  if (base + (kUnroll - 1) * kThreads < n_vec) {
    u32x4 a[kUnroll], b[kUnroll], c[kUnroll];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) a[j] = __builtin_nontemporal_load(in0 + base + j * kThreads);
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      b[j] = Op::kIn > 1 ? __builtin_nontemporal_load(in1 + base + j * kThreads) : zero;
      c[j] = Op::kIn > 2 ? __builtin_nontemporal_load(in2 + base + j * kThreads) : zero;
    }
#pragma unroll
    for (int j = 0; j < kUnroll; ++j)
      __builtin_nontemporal_store(apply_vec(op, a[j], b[j], c[j]), out + base + j * kThreads);
  } else {
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int64_t v = base + j * kThreads;
      if (v < n_vec) {
        out[v] = apply_vec(op, in0[v], Op::kIn > 1 ? in1[v] : zero, Op::kIn > 2 ? in2[v] : zero);
      }
    }
  }
}

// Element-wise body for [begin, end), grid-stride.
template <class Op>
__device__ __forceinline__ void map_scalar_body(const Op& op, const typename Op::T* __restrict__ in0,
                                                const typename Op::T* __restrict__ in1,
                                                const typename Op::T* __restrict__ in2,
                                                typename Op::T* __restrict__ out, int64_t begin, int64_t end) {
  for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < end;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    if constexpr (Op::kIn == 1) {
      out[i] = op(in0[i]);
    } else {
      out[i] = op(in0[i], in1[i], in2[i]);
    }
  }
}

// ---- GELU (fp32 rows).  The constants and the operation order are those of
// the reference kernel body: tanh form via x - x / (exp(p) + 1) with
// p = x * (x*x*k2 + k1), k1 = 2*sqrt(2/pi), k2 = k1 * 0.044715; erf form
// x * (erf(x * sqrt(0.5)) + 1) * 0.5.  Accurate libm expf / erff, true division.
__device__ __forceinline__ float gelu_tanh(float x, float k1, float k2) {
  const float p = x * ((x * x) * k2 + k1);
  return x - x / (expf(p) + 1.0f);
}
__device__ __forceinline__ float gelu_erf(float x, float k) { return x * (erff(x * k) + 1.0f) * 0.5f; }

// Rows b, b + gridDim.x, ... of a [rows, cols] fp32 matrix (cols = row stride):
// the first len columns of each.  vec_ok: x and out 16-byte aligned, cols % 4 == 0.
__device__ __forceinline__ void gelu_rows_body(const float* __restrict__ x, float* __restrict__ out, int64_t rows,
                                               int64_t cols, int32_t len, int32_t approximate, int32_t vec_ok) {
  const float s = sqrtf(static_cast<float>(2.0 / 3.141592653589793238462643383279502884));
  const float k1 = 2.0f * s;
  const float k2 = 2.0f * s * 0.044715f;
  const float k = sqrtf(0.5f);
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const float* xr = x + r * cols;
    float* orow = out + r * cols;
    const int n4 = vec_ok ? len / 4 : 0;
    for (int q = threadIdx.x; q < n4; q += kThreads) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr) + q);
      float e[4];
      __builtin_memcpy(e, &v, 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = approximate ? gelu_tanh(e[i], k1, k2) : gelu_erf(e[i], k);
      u32x4 o;
      __builtin_memcpy(&o, e, 16);
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(orow) + q);
    }
    for (int c = n4 * 4 + threadIdx.x; c < len; c += kThreads) {
      orow[c] = approximate ? gelu_tanh(xr[c], k1, k2) : gelu_erf(xr[c], k);
    }
  }
}

}  // namespace elementwise
}  // namespace asc

// Defines the elementwise kernels as PREFIX##<name> with the given linkage
// specifier (the library's are internal, the code object's have C names for
// hipModuleGetFunction):
//   leaky_relu_vec_<dt>(const u32x4* x, u32x4* out, int64_t n_vec, float alpha)
//   leaky_relu_elem_<dt>(const T* x, T* out, int64_t begin, int64_t end, float alpha)
//   vmuladd_vec_<dt>(const u32x4* x, const u32x4* y, const u32x4* z, u32x4* out, int64_t n_vec)
//   vmuladd_elem_<dt>(const T* x, const T* y, const T* z, T* out, int64_t begin, int64_t end)
//   gelu_rows_f32(const float* x, float* out, int64_t rows, int64_t cols, int32_t len,
//                 int32_t approximate, int32_t vec_ok)
// for dt in f32, f16, bf16.  Vector kernels: grid ceil(n_vec / (kThreads * kUnroll));
// element kernels: any grid (grid-stride); all kThreads threads.
#define ASC_ELEMENTWISE_TYPED_KERNELS(LINKAGE, PREFIX, DT, E)                                                      \
  LINKAGE __global__ void __launch_bounds__(asc::elementwise::kThreads)                                            \
      PREFIX##leaky_relu_vec_##DT(const asc::elementwise::u32x4* __restrict__ x,                                   \
                                  asc::elementwise::u32x4* __restrict__ out, int64_t n_vec, float alpha) {         \
    asc::elementwise::map_vec_body(asc::elementwise::LeakyRelu<asc::elementwise::E>{alpha}, x, x, x, out, n_vec);  \
  }                                                                                                                \
  LINKAGE __global__ void __launch_bounds__(asc::elementwise::kThreads)                                            \
      PREFIX##leaky_relu_elem_##DT(const asc::elementwise::E::T* __restrict__ x,                                   \
                                   asc::elementwise::E::T* __restrict__ out, int64_t begin, int64_t end,           \
                                   float alpha) {                                                                  \
    asc::elementwise::map_scalar_body(asc::elementwise::LeakyRelu<asc::elementwise::E>{alpha}, x, x, x, out,      \
                                      begin, end);                                                                 \
  }                                                                                                                \
  LINKAGE __global__ void __launch_bounds__(asc::elementwise::kThreads)                                            \
      PREFIX##vmuladd_vec_##DT(const asc::elementwise::u32x4* __restrict__ x,                                      \
                               const asc::elementwise::u32x4* __restrict__ y,                                      \
                               const asc::elementwise::u32x4* __restrict__ z,                                      \
                               asc::elementwise::u32x4* __restrict__ out, int64_t n_vec) {                         \
    asc::elementwise::map_vec_body(asc::elementwise::MulAdd<asc::elementwise::E>{}, x, y, z, out, n_vec);          \
  }                                                                                                                \
  LINKAGE __global__ void __launch_bounds__(asc::elementwise::kThreads)                                            \
      PREFIX##vmuladd_elem_##DT(const asc::elementwise::E::T* __restrict__ x,                                      \
                                const asc::elementwise::E::T* __restrict__ y,                                      \
                                const asc::elementwise::E::T* __restrict__ z,                                      \
                                asc::elementwise::E::T* __restrict__ out, int64_t begin, int64_t end) {            \
    asc::elementwise::map_scalar_body(asc::elementwise::MulAdd<asc::elementwise::E>{}, x, y, z, out, begin, end);  \
  }

#define ASC_ELEMENTWISE_KERNELS(LINKAGE, PREFIX)                                                                   \
  ASC_ELEMENTWISE_TYPED_KERNELS(LINKAGE, PREFIX, f32, F32)                                                         \
  ASC_ELEMENTWISE_TYPED_KERNELS(LINKAGE, PREFIX, f16, F16)                                                         \
  ASC_ELEMENTWISE_TYPED_KERNELS(LINKAGE, PREFIX, bf16, BF16)                                                       \
  LINKAGE __global__ void __launch_bounds__(asc::elementwise::kThreads)                                            \
      PREFIX##gelu_rows_f32(const float* __restrict__ x, float* __restrict__ out, int64_t rows, int64_t cols,      \
                            int32_t len, int32_t approximate, int32_t vec_ok) {                                    \
    asc::elementwise::gelu_rows_body(x, out, rows, cols, len, approximate, vec_ok);                                \
  }
