// Elementwise asc2 kernels beside vadd:
//   leaky_relu_kernel  python/test/asc2/kernels/test_leaky_relu.py:16-26
//                      out = where(x >= 0, x, x * alpha)
//   vmuladd_kernel     python/test/asc2/kernels/test_vmuladd.py:16-31
//                      out = x * y + z (multiply and add rounded separately)
//   gelu_kernel        python/test/asc2/kernels/test_gelu.py:19-33
//                      grid-stride rows, tanh-form or erf-form GELU
//
// leaky_relu and vmuladd stream like vadd: HBM-bound, 16-byte non-temporal
// vectors, four per thread per operand, the physical grid sized by the covered
// length (the logical grid only decides how far the writes reach:
// [0, min(size, grid * tile_per_block * tile_size))).  Unaligned buffers and
// the sub-vector tail take an element-wise kernel with the same arithmetic.
// Compiled with -ffp-contract=off: no multiply-add is fused.
#include <math.h>

#include "common.h"
#include "numeric.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

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
// inputs are not read).
template <class Op>
__global__ void __launch_bounds__(kThreads) map_vec_kernel(Op op, const u32x4* __restrict__ in0,
                                                           const u32x4* __restrict__ in1,
                                                           const u32x4* __restrict__ in2, u32x4* __restrict__ out,
                                                           int64_t n_vec) {
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

// Element-wise path for [begin, end).
template <class Op>
__global__ void __launch_bounds__(kThreads) map_scalar_kernel(Op op, const typename Op::T* __restrict__ in0,
                                                              const typename Op::T* __restrict__ in1,
                                                              const typename Op::T* __restrict__ in2,
                                                              typename Op::T* __restrict__ out, int64_t begin,
                                                              int64_t end) {
  for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < end;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    if constexpr (Op::kIn == 1) {
      out[i] = op(in0[i]);
    } else {
      out[i] = op(in0[i], in1[i], in2[i]);
    }
  }
}

template <class Op>
int32_t launch_map(const Op& op, const void* in0v, const void* in1v, const void* in2v, void* outv, int64_t covered,
                   hipStream_t stream, const char* who) {
  using T = typename Op::T;
  const T* in0 = static_cast<const T*>(in0v);
  const T* in1 = static_cast<const T*>(in1v);
  const T* in2 = static_cast<const T*>(in2v);
  T* out = static_cast<T*>(outv);
  constexpr int64_t kPerVec = 16 / sizeof(T);
  int64_t done = 0;
  const bool aligned = asc::aligned16(in0) && asc::aligned16(out) && (Op::kIn < 2 || asc::aligned16(in1)) &&
                       (Op::kIn < 3 || asc::aligned16(in2));
  if (aligned) {
    const int64_t n_vec = covered / kPerVec;
    if (n_vec > 0) {
      const int64_t blocks = asc::ceil_div(n_vec, kThreads * kUnroll);
      hipLaunchKernelGGL(map_vec_kernel<Op>, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream, op,
                         reinterpret_cast<const u32x4*>(in0), reinterpret_cast<const u32x4*>(in1),
                         reinterpret_cast<const u32x4*>(in2), reinterpret_cast<u32x4*>(out), n_vec);
      const int32_t rc = asc::check_launch(who);
      if (rc != ASC_OK) return rc;
    }
    done = n_vec * kPerVec;
  }
  if (done < covered) {
    const int64_t rest = covered - done;
    const int64_t blocks = asc::ceil_div(rest, kThreads) < 4096 ? asc::ceil_div(rest, kThreads) : 4096;
    hipLaunchKernelGGL(map_scalar_kernel<Op>, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream, op,
                       in0, in1, in2, out, done, covered);
    return asc::check_launch(who);
  }
  return ASC_OK;
}

// Coverage of the reference's tiled elementwise kernel bodies.
int64_t covered_elements(int64_t size, int32_t tile_size, int32_t tile_per_block, int32_t grid) {
  const int64_t reach = static_cast<int64_t>(grid) * tile_per_block * tile_size;
  return reach < size ? reach : size;
}

// ---- GELU (fp32 rows).  The constants and the operation order are those of
// the reference kernel body: tanh form via x - x / (exp(p) + 1) with
// p = x * (x*x*k2 + k1), k1 = 2*sqrt(2/pi), k2 = k1 * 0.044715; erf form
// x * (erf(x * sqrt(0.5)) + 1) * 0.5.  Accurate libm expf / erff, true division.
struct GeluArgs {
  const float* x;
  float* out;
  int64_t rows, cols;  // cols = row stride
  int32_t len;         // columns processed per row (tile_size)
  int32_t approximate;
  bool vec_ok;
};

__device__ __forceinline__ float gelu_tanh(float x, float k1, float k2) {
  const float p = x * ((x * x) * k2 + k1);
  return x - x / (expf(p) + 1.0f);
}
__device__ __forceinline__ float gelu_erf(float x, float k) { return x * (erff(x * k) + 1.0f) * 0.5f; }

__global__ void __launch_bounds__(kThreads) gelu_rows_kernel(GeluArgs p) {
  const float s = sqrtf(static_cast<float>(2.0 / 3.141592653589793238462643383279502884));
  const float k1 = 2.0f * s;
  const float k2 = 2.0f * s * 0.044715f;
  const float k = sqrtf(0.5f);
  // one row per block-iteration: rows b, b + gridDim.x, ... (all rows covered)
  for (int64_t r = blockIdx.x; r < p.rows; r += gridDim.x) {
    const float* xr = p.x + r * p.cols;
    float* orow = p.out + r * p.cols;
    const int n4 = p.vec_ok ? p.len / 4 : 0;
    for (int q = threadIdx.x; q < n4; q += kThreads) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr) + q);
      float e[4];
      __builtin_memcpy(e, &v, 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = p.approximate ? gelu_tanh(e[i], k1, k2) : gelu_erf(e[i], k);
      u32x4 o;
      __builtin_memcpy(&o, e, 16);
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(orow) + q);
    }
    for (int c = n4 * 4 + threadIdx.x; c < p.len; c += kThreads) {
      orow[c] = p.approximate ? gelu_tanh(xr[c], k1, k2) : gelu_erf(xr[c], k);
    }
  }
}

}  // namespace

extern "C" int32_t asc_leaky_relu(int32_t dtype, const void* x, float alpha, void* out, int64_t size,
                                  int32_t tile_size, int32_t tile_per_block, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(size >= 0, ASC_ERR_INVALID_ARG, "asc_leaky_relu: size must be >= 0, got %lld", (long long)size);
  ASC_REQUIRE(tile_size > 0 && tile_per_block >= 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_leaky_relu: need tile_size > 0, tile_per_block >= 0, grid > 0 (got %d, %d, %d)", tile_size,
              tile_per_block, grid);
  const int64_t covered = covered_elements(size, tile_size, tile_per_block, grid);
  if (covered == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "asc_leaky_relu: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case ASC_DT_FLOAT32: return launch_map(LeakyRelu<F32>{alpha}, x, nullptr, nullptr, out, covered, s, "asc_leaky_relu");
    case ASC_DT_FLOAT16: return launch_map(LeakyRelu<F16>{alpha}, x, nullptr, nullptr, out, covered, s, "asc_leaky_relu");
    case ASC_DT_BFLOAT16:
      return launch_map(LeakyRelu<BF16>{alpha}, x, nullptr, nullptr, out, covered, s, "asc_leaky_relu");
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_leaky_relu: unsupported dtype code %d", dtype);
  }
}

extern "C" int32_t asc_vmuladd(int32_t dtype, const void* x, const void* y, const void* z, void* out, int64_t size,
                               int32_t tile_size, int32_t tile_per_block, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(size >= 0, ASC_ERR_INVALID_ARG, "asc_vmuladd: size must be >= 0, got %lld", (long long)size);
  ASC_REQUIRE(tile_size > 0 && tile_per_block >= 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_vmuladd: need tile_size > 0, tile_per_block >= 0, grid > 0 (got %d, %d, %d)", tile_size,
              tile_per_block, grid);
  const int64_t covered = covered_elements(size, tile_size, tile_per_block, grid);
  if (covered == 0) return ASC_OK;
  ASC_REQUIRE(x && y && z && out, ASC_ERR_INVALID_ARG, "asc_vmuladd: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case ASC_DT_FLOAT32: return launch_map(MulAdd<F32>{}, x, y, z, out, covered, s, "asc_vmuladd");
    case ASC_DT_FLOAT16: return launch_map(MulAdd<F16>{}, x, y, z, out, covered, s, "asc_vmuladd");
    case ASC_DT_BFLOAT16: return launch_map(MulAdd<BF16>{}, x, y, z, out, covered, s, "asc_vmuladd");
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_vmuladd: unsupported dtype code %d", dtype);
  }
}

extern "C" int32_t asc_gelu_rows_f32(const float* x, float* out, int64_t num_rows, int64_t num_cols,
                                     int32_t tile_size, int32_t approximate, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(num_rows >= 0 && num_cols >= 0, ASC_ERR_INVALID_ARG, "asc_gelu_rows_f32: negative shape");
  ASC_REQUIRE(tile_size > 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_gelu_rows_f32: need tile_size > 0 and grid > 0 (got %d, %d)", tile_size, grid);
  // A tile wider than the row: the load pads with zeros and gelu is element-wise, so the
  // row's own columns are all that is computed and written (the reference's tile store
  // would also spill the padding's gelu(0) = 0 into the next row).
  if (tile_size > num_cols) tile_size = static_cast<int32_t>(num_cols);
  if (num_rows == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "asc_gelu_rows_f32: null buffer");
  GeluArgs p{x, out, num_rows, num_cols, tile_size, approximate ? 1 : 0,
             asc::aligned16(x) && asc::aligned16(out) && (num_cols % 4) == 0};
  // Rows b, b+grid, ... for b < grid cover every row exactly once; the physical
  // grid is the library's (rows are independent).
  const int64_t blocks = num_rows < 8192 ? num_rows : 8192;
  hipLaunchKernelGGL(gelu_rows_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), p);
  return asc::check_launch("asc_gelu_rows_f32");
}
