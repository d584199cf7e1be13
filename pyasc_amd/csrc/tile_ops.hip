// Element-wise asc2 tile operations, as the reference's operation tests use them:
//   unary   python/test/asc2/operations/test_unary_ops.py:35-40   z = op(x)       (fp32)
//   binary  python/test/asc2/operations/test_binary_ops.py:24-38  z = op(x, y), either operand may be a scalar
//   where   python/test/asc2/operations/test_where.py:18-27, 48-55
//           z = where(cmp(x, y), x, y)  or  z = where(cmp(x, s), 0, 1)
//   rect    python/test/asc2/operations/test_memory_ops.py:58-92   z[tile] = x[tile] + y[tile]
//   rows    python/test/asc2/operations/test_shape_ops.py:47-55    broadcast_to / reshape data movement
//   atomic  python/test/asc2/operations/test_atomic_ops.py:33-40   z[j] = op(z[j], x[b, j] + c), atomically
//   fill    python/test/asc2/operations/test_shape_ops.py:64-78    z = full([1], c).broadcast_to(shape)
//   axpy, transpose: asc1 vector intrinsics of python/test/generalization/basic/
//
// Semantics follow the op definitions (python/asc/language/tile/binary_ops.py,
// unary_ops.py; dtype inference utils.py:73-94): a scalar operand takes the
// tile's dtype; integer add/sub/mul wrap (arith.addi/subi/muli), integer div
// truncates (arith.divsi), max/min are signed for integers and NaN-propagating
// for floats (arith.maximumf/minimumf: -0 < +0), shifts are shli / shrsi
// (arithmetic) by a non-negative amount below the bit width.  16-bit float
// elements are computed in fp32 and rounded once (RNE) to the element type.
// Integer division by zero yields 0 (arith.divsi leaves it undefined).  A
// scalar operand of a 16-bit float tile is rounded to fp32 on the host, then to
// the element type (exact for values that come from such a tile).
//
// One grid-stride kernel per (element type, operation family); the op code is a
// kernel argument (uniform branch).  These are HBM-bound streams; the reference
// tests run them on 32 elements.
#include <math.h>

#include "common.h"
#include "numeric.h"

namespace {

constexpr int kThreads = 256;

struct F32 {
  using T = float;
  static constexpr bool kFloat = true;
  __device__ static float in(float v) { return v; }
  __device__ static float out(float v) { return v; }
};
struct F16 {
  using T = uint16_t;
  static constexpr bool kFloat = true;
  __device__ static float in(uint16_t v) { return asc::f16_to_f32(v); }
  __device__ static uint16_t out(float v) { return asc::f32_to_f16_rne(v); }
};
struct BF16 {
  using T = uint16_t;
  static constexpr bool kFloat = true;
  __device__ static float in(uint16_t v) { return asc::bf16_to_f32(v); }
  __device__ static uint16_t out(float v) { return asc::f32_to_bf16_rne(v); }
};
struct I32 {
  using T = int32_t;
  using U = uint32_t;
  static constexpr bool kFloat = false;
  static constexpr int kBits = 32;
};
struct I16 {
  using T = int16_t;
  using U = uint16_t;
  static constexpr bool kFloat = false;
  static constexpr int kBits = 16;
};

// ---- unary (fp32): op codes of ASC_UNARY_* in asc_hip.h
__device__ __forceinline__ float unary_f32(int op, float x) {
  switch (op) {
    case 0: return fabsf(x);
    case 1: return ceilf(x);
    case 2: return cosf(x);
    case 3: return coshf(x);
    case 4: return erff(x);
    case 5: return expf(x);
    case 6: return exp2f(x);
    case 7: return floorf(x);
    case 8: return logf(x);
    case 9: return log2f(x);
    case 10: return -x;
    case 11: return x < 0.f ? 0.f : x;  // relu: negative -> +0; -0 and NaN pass through
    case 12: return 1.0f / sqrtf(x);
    case 13: return sinf(x);
    case 14: return sinhf(x);
    case 15: return sqrtf(x);
    case 16: return tanf(x);
    default: return tanhf(x);
  }
}

// fp32 elements directly; 16-bit float elements widen to fp32, take the fp32 op and
// round once (RNE) to the element type.
template <class E>
__global__ void __launch_bounds__(kThreads) unary_kernel(int op, const typename E::T* __restrict__ x,
                                                         typename E::T* __restrict__ out, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    out[i] = E::out(unary_f32(op, E::in(x[i])));
}

// ---- binary: op codes of ASC_BIN_* in asc_hip.h
// IEEE 754-2019 maximum / minimum (arith.maximumf / minimumf): NaN propagates,
// -0 orders below +0.
__device__ __forceinline__ float max_f(float x, float y) {
  if (x != x) return x;
  if (y != y) return y;
  if (x == y) return __builtin_signbit(x) ? y : x;
  return x > y ? x : y;
}
__device__ __forceinline__ float min_f(float x, float y) {
  if (x != x) return x;
  if (y != y) return y;
  if (x == y) return __builtin_signbit(x) ? x : y;
  return x < y ? x : y;
}

template <class E>
__device__ __forceinline__ typename E::T binary_op(int op, typename E::T a, typename E::T b) {
  if constexpr (E::kFloat) {
    const float x = E::in(a), y = E::in(b);
    float r;
    switch (op) {
      case 0: r = x + y; break;
      case 1: r = x - y; break;
      case 2: r = x * y; break;
      case 3: r = x / y; break;
      case 4: r = max_f(x, y); break;
      default: r = min_f(x, y); break;
    }
    return E::out(r);
  } else {
    using T = typename E::T;
    using U = typename E::U;
    const U ua = static_cast<U>(a), ub = static_cast<U>(b);
    switch (op) {
      case 0: return static_cast<T>(static_cast<U>(ua + ub));
      case 1: return static_cast<T>(static_cast<U>(ua - ub));
      case 2: return static_cast<T>(static_cast<U>(ua * ub));
      case 3:
        if (b == 0) return T(0);
        if (b == T(-1)) return static_cast<T>(static_cast<U>(U(0) - ua));  // wraps for the minimum value
        return static_cast<T>(a / b);
      case 4: return a > b ? a : b;
      case 5: return a < b ? a : b;
      case 6: return static_cast<T>(static_cast<U>(ua << static_cast<int>(b)));
      default: return static_cast<T>(a >> static_cast<int>(b));
    }
  }
}

// A scalar operand travels as fp32 (float elements) or int64 (integer
// elements) and is rounded (RNE) or wrapped to the element type here.
template <class E>
__device__ __forceinline__ typename E::T element_of(float v_f, int64_t v_i) {
  if constexpr (E::kFloat) {
    return E::out(v_f);
  } else {
    return static_cast<typename E::T>(static_cast<typename E::U>(static_cast<uint64_t>(v_i)));
  }
}

// mode 0: x, y vectors; 1: y is the scalar s; 2: x is the scalar s
template <class E>
__global__ void __launch_bounds__(kThreads) binary_kernel(int op, int mode, const typename E::T* __restrict__ x,
                                                          const typename E::T* __restrict__ y,
                                                          typename E::T* __restrict__ out, float s_f, int64_t s_i,
                                                          int64_t n) {
  const typename E::T s = element_of<E>(s_f, s_i);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const typename E::T a = mode == 2 ? s : x[i];
    const typename E::T b = mode == 1 ? s : y[i];
    out[i] = binary_op<E>(op, a, b);
  }
}

// ---- compare + where: cmp codes of ASC_CMP_* in asc_hip.h
template <class E>
__device__ __forceinline__ bool compare(int cmp, typename E::T a, typename E::T b) {
  if constexpr (E::kFloat) {
    const float x = E::in(a), y = E::in(b);
    switch (cmp) {
      case 0: return x == y;
      case 1: return x != y;
      case 2: return x > y;
      case 3: return x >= y;
      case 4: return x < y;
      default: return x <= y;
    }
  } else {
    switch (cmp) {
      case 0: return a == b;
      case 1: return a != b;
      case 2: return a > b;
      case 3: return a >= b;
      case 4: return a < b;
      default: return a <= b;
    }
  }
}

// mode 0: out = cmp(x, y) ? x : y; mode 1: out = cmp(x, s) ? t : f
template <class E>
__global__ void __launch_bounds__(kThreads) where_kernel(int cmp, int mode, const typename E::T* __restrict__ x,
                                                         const typename E::T* __restrict__ y,
                                                         typename E::T* __restrict__ out, float s_f, int64_t s_i,
                                                         float t_f, float f_f, int64_t n) {
  const typename E::T s = element_of<E>(s_f, s_i);
  const typename E::T t = element_of<E>(t_f, static_cast<int64_t>(t_f));
  const typename E::T f = element_of<E>(f_f, static_cast<int64_t>(f_f));
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const typename E::T a = x[i];
    if (mode == 0) {
      const typename E::T b = y[i];
      out[i] = compare<E>(cmp, a, b) ? a : b;
    } else {
      out[i] = compare<E>(cmp, a, s) ? t : f;
    }
  }
}

// ---- a binary op over a rectangle of a row-major [rows, cols] tensor:
// z[r0+i, c0+j] = op(x[..], y[..]) for i < h, j < w (the tile load / add / store of
// python/test/asc2/operations/test_memory_ops.py's kernels).
template <class E>
__global__ void __launch_bounds__(kThreads) rect_binary_kernel(int op, const typename E::T* __restrict__ x,
                                                               const typename E::T* __restrict__ y,
                                                               typename E::T* __restrict__ z, int64_t cols,
                                                               int64_t r0, int64_t c0, int64_t h, int64_t w) {
  const int64_t n = h * w;
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k < n;
       k += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t i = k / w, j = k - (k / w) * w;
    const int64_t off = (r0 + i) * cols + c0 + j;
    z[off] = binary_op<E>(op, x[off], y[off]);
  }
}

// ---- row broadcast: z[r, c] = x[c] for r < rows (broadcast_to from [1, cols]; with
// rows = 1 a plain copy, the data movement of reshape / ravel / squeeze / expand_dims).
template <class T>
__global__ void __launch_bounds__(kThreads) broadcast_rows_kernel(const T* __restrict__ x, T* __restrict__ z,
                                                                  int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k < n;
       k += static_cast<int64_t>(gridDim.x) * kThreads)
    z[k] = x[k % cols];
}

// ---- atomic combine.  An asc2 atomic op is a store in atomic mode
// (python/asc/language/tile/atomic_ops.py:19-33, lowered to a store bracketed by
// SetAtomicAdd/Max/Min ... SetAtomicNone in lib/Conversion/LowerToAsc/LowerAtomic.cpp:44-70):
// every element of the tile is combined into the destination.  Here tile b of x (tile_len
// elements), plus the scalar c in the element type, is combined into z[0, tile_len) for
// b < n_tiles, the body of the reference test with one workgroup range per tile.
// 32-bit integers use the hardware atomics (relaxed, device scope), fp32 add the hardware
// float add; fp32 max/min and every 16-bit element type run a compare-and-swap loop on the
// enclosing aligned 32-bit word (the other half is written back unchanged, and a concurrent
// change to it makes the swap fail and retry).  The combine of each element is the binary
// op of the element type (rounded once for 16-bit floats; IEEE maximum/minimum).
template <class E>
__device__ __forceinline__ void atomic_combine(int op, typename E::T* p, typename E::T v) {
  using T = typename E::T;
  if constexpr (sizeof(T) == 4 && !E::kFloat) {
    if (op == 0)
      __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else if (op == 4)
      __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      __hip_atomic_fetch_min(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if constexpr (sizeof(T) == 4) {
    if (op == 0) {
      __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    uint32_t* w = reinterpret_cast<uint32_t*>(p);
    uint32_t old = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
      const uint32_t nw = __float_as_uint(binary_op<E>(op, __uint_as_float(old), v));
      if (nw == old) return;
      if (__hip_atomic_compare_exchange_strong(w, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        return;
    }
  } else {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    uint32_t* w = reinterpret_cast<uint32_t*>(a & ~uintptr_t(3));
    const int shift = (a & 2) ? 16 : 0;
    uint32_t old = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
      const T cur = static_cast<T>(static_cast<uint16_t>(old >> shift));
      const uint16_t r = static_cast<uint16_t>(binary_op<E>(op, cur, v));
      const uint32_t nw = (old & ~(0xffffu << shift)) | (static_cast<uint32_t>(r) << shift);
      if (nw == old) return;
      if (__hip_atomic_compare_exchange_strong(w, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        return;
    }
  }
}

template <class E>
__global__ void __launch_bounds__(kThreads) atomic_tiles_kernel(int op, const typename E::T* __restrict__ x,
                                                                typename E::T* z, int64_t tile_len, int64_t n,
                                                                float c_f, int64_t c_i) {
  const typename E::T c = element_of<E>(c_f, c_i);
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k < n;
       k += static_cast<int64_t>(gridDim.x) * kThreads)
    atomic_combine<E>(op, z + (k - (k / tile_len) * tile_len), binary_op<E>(0, x[k], c));
}

// ---- axpy (python/asc/language/basic/vec_ternary_scalar.py, asc.axpy; the kernel of
// python/test/generalization/basic/test_axpy.py): dst[i] = src[i] * s + dst[i], with s
// in the element type (Axpy's scalar has the source type), computed in fp32 and
// rounded once to the element type (-ffp-contract=off: product and sum each rounded
// in fp32).
template <class E>
__global__ void __launch_bounds__(kThreads) axpy_kernel(const typename E::T* __restrict__ src,
                                                        typename E::T* __restrict__ dst, float s_f, int64_t n) {
  const float s = E::in(element_of<E>(s_f, 0));
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    dst[i] = E::out(E::in(src[i]) * s + E::in(dst[i]));
}

// ---- batched transpose: z[b, c, r] = x[b, r, c] for [batch, rows, cols] row-major
// (asc.transpose of a 16x16 tile of 2-byte elements, python/test/generalization/basic/
// test_transpose.py, is batch = tiles, rows = cols = 16).
template <class T>
__global__ void __launch_bounds__(kThreads) transpose_kernel(const T* __restrict__ x, T* __restrict__ z,
                                                             int64_t rows, int64_t cols, int64_t n) {
  const int64_t rc = rows * cols;
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k < n;
       k += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t b = k / rc, rem = k - b * rc;
    const int64_t r = rem / cols, c = rem - r * cols;
    z[b * rc + c * rows + r] = x[k];
  }
}

// ---- quantization to int8 (asc.adv.quant, python/asc/language/adv/quantization.py:18-36;
// the kernel of python/test/generalization/adv/test_quant.py):
// dst = saturate_int8(rint(src * scale + offset)) with scale and offset materialized in the
// source dtype (quantization.py:28-29), the multiply and the add each rounded to that
// dtype, rint rounding half to even, results clamped to [-128, 127], NaN giving 0.
template <class E>
__global__ void __launch_bounds__(kThreads) quant_i8_kernel(const typename E::T* __restrict__ src,
                                                            int8_t* __restrict__ dst, float scale_f, float offset_f,
                                                            int64_t n) {
  const float sc = E::in(element_of<E>(scale_f, 0)), of = E::in(element_of<E>(offset_f, 0));
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const float v = E::in(E::out(E::in(E::out(E::in(src[i]) * sc)) + of));
    const float r = fminf(fmaxf(rintf(v), -128.0f), 127.0f);
    dst[i] = v != v ? int8_t(0) : static_cast<int8_t>(r);
  }
}

// ---- fill: every element of z takes the scalar c converted to the element type
template <class E>
__global__ void __launch_bounds__(kThreads) fill_kernel(typename E::T* __restrict__ z, int64_t n, float c_f,
                                                        int64_t c_i) {
  const typename E::T c = element_of<E>(c_f, c_i);
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k < n;
       k += static_cast<int64_t>(gridDim.x) * kThreads)
    z[k] = c;
}

uint32_t grid_for(int64_t n) {
  const int64_t blocks = asc::ceil_div(n, kThreads);
  return static_cast<uint32_t>(blocks < 8192 ? blocks : 8192);
}

template <class E>
int32_t launch_binary(int op, int mode, const void* x, const void* y, void* out, int64_t n, double s_f, int64_t s_i,
                      hipStream_t stream) {
  using T = typename E::T;
  hipLaunchKernelGGL(binary_kernel<E>, dim3(grid_for(n)), dim3(kThreads), 0, stream, op, mode,
                     static_cast<const T*>(x), static_cast<const T*>(y), static_cast<T*>(out),
                     static_cast<float>(s_f), s_i, n);
  return asc::check_launch("asc_binary");
}

template <class E>
int32_t launch_where(int cmp, int mode, const void* x, const void* y, void* out, int64_t n, double s_f, int64_t s_i,
                     double t, double f, hipStream_t stream) {
  using T = typename E::T;
  hipLaunchKernelGGL(where_kernel<E>, dim3(grid_for(n)), dim3(kThreads), 0, stream, cmp, mode,
                     static_cast<const T*>(x), static_cast<const T*>(y), static_cast<T*>(out),
                     static_cast<float>(s_f), s_i, static_cast<float>(t), static_cast<float>(f), n);
  return asc::check_launch("asc_where_cmp");
}

}  // namespace

extern "C" int32_t asc_unary(int32_t op, int32_t dtype, const void* x, void* out, int64_t n,
                             asc_stream_t stream) {
  ASC_REQUIRE(op >= 0 && op <= 17, ASC_ERR_INVALID_ARG, "asc_unary: unknown op code %d", op);
  ASC_REQUIRE(n >= 0, ASC_ERR_INVALID_ARG, "asc_unary: negative length");
  if (n == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "asc_unary: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n));
  switch (dtype) {
    case ASC_DT_FLOAT32:
      hipLaunchKernelGGL(unary_kernel<F32>, grid, dim3(kThreads), 0, s, op, static_cast<const float*>(x),
                         static_cast<float*>(out), n);
      break;
    case ASC_DT_FLOAT16:
      hipLaunchKernelGGL(unary_kernel<F16>, grid, dim3(kThreads), 0, s, op, static_cast<const uint16_t*>(x),
                         static_cast<uint16_t*>(out), n);
      break;
    case ASC_DT_BFLOAT16:
      hipLaunchKernelGGL(unary_kernel<BF16>, grid, dim3(kThreads), 0, s, op, static_cast<const uint16_t*>(x),
                         static_cast<uint16_t*>(out), n);
      break;
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_unary: unsupported dtype code %d", dtype);
  }
  return asc::check_launch("asc_unary");
}

extern "C" int32_t asc_unary_f32(int32_t op, const float* x, float* out, int64_t n, asc_stream_t stream) {
  return asc_unary(op, ASC_DT_FLOAT32, x, out, n, stream);
}

extern "C" int32_t asc_axpy(int32_t dtype, const void* src, void* dst, double scalar, int64_t n,
                            asc_stream_t stream) {
  ASC_REQUIRE(n >= 0, ASC_ERR_INVALID_ARG, "asc_axpy: negative length");
  if (n == 0) return ASC_OK;
  ASC_REQUIRE(src && dst, ASC_ERR_INVALID_ARG, "asc_axpy: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n));
  switch (dtype) {
    case ASC_DT_FLOAT32:
      hipLaunchKernelGGL(axpy_kernel<F32>, grid, dim3(kThreads), 0, s, static_cast<const float*>(src),
                         static_cast<float*>(dst), static_cast<float>(scalar), n);
      break;
    case ASC_DT_FLOAT16:
      hipLaunchKernelGGL(axpy_kernel<F16>, grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(src),
                         static_cast<uint16_t*>(dst), static_cast<float>(scalar), n);
      break;
    case ASC_DT_BFLOAT16:
      hipLaunchKernelGGL(axpy_kernel<BF16>, grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(src),
                         static_cast<uint16_t*>(dst), static_cast<float>(scalar), n);
      break;
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_axpy: unsupported dtype code %d", dtype);
  }
  return asc::check_launch("asc_axpy");
}

extern "C" int32_t asc_transpose_batched(int32_t elem_bytes, const void* x, void* z, int64_t batch, int64_t rows,
                                         int64_t cols, asc_stream_t stream) {
  ASC_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0, ASC_ERR_INVALID_ARG, "asc_transpose_batched: negative shape");
  ASC_REQUIRE(rows == 0 || cols == 0 || batch <= INT64_MAX / rows / cols, ASC_ERR_INVALID_ARG,
              "asc_transpose_batched: size overflows");
  const int64_t n = batch * rows * cols;
  if (n == 0) return ASC_OK;
  ASC_REQUIRE(x && z && x != z, ASC_ERR_INVALID_ARG, "asc_transpose_batched: null or aliased buffers");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n));
  switch (elem_bytes) {
    case 2:
      hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(x),
                         static_cast<uint16_t*>(z), rows, cols, n);
      break;
    case 4:
      hipLaunchKernelGGL(transpose_kernel<uint32_t>, grid, dim3(kThreads), 0, s, static_cast<const uint32_t*>(x),
                         static_cast<uint32_t*>(z), rows, cols, n);
      break;
    default:
      return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_transpose_batched: element size %d not supported", elem_bytes);
  }
  return asc::check_launch("asc_transpose_batched");
}

extern "C" int32_t asc_binary(int32_t op, int32_t dtype, const void* x, const void* y, void* out, int64_t n,
                              int32_t mode, double scalar_f, int64_t scalar_i, asc_stream_t stream) {
  ASC_REQUIRE(op >= 0 && op <= 7, ASC_ERR_INVALID_ARG, "asc_binary: unknown op code %d", op);
  ASC_REQUIRE(mode >= 0 && mode <= 2, ASC_ERR_INVALID_ARG, "asc_binary: unknown operand mode %d", mode);
  ASC_REQUIRE(n >= 0, ASC_ERR_INVALID_ARG, "asc_binary: negative length");
  const bool is_int = dtype == ASC_DT_INT32 || dtype == ASC_DT_INT16;
  ASC_REQUIRE(op < 6 || is_int, ASC_ERR_UNSUPPORTED, "asc_binary: shifts need an integer dtype");
  if (op >= 6) {
    const int bits = dtype == ASC_DT_INT32 ? 32 : 16;
    ASC_REQUIRE(mode == 1 && scalar_i >= 0 && scalar_i < bits, ASC_ERR_INVALID_ARG,
                "asc_binary: a shift takes a scalar amount in [0, %d), got mode %d amount %lld", bits, mode,
                (long long)scalar_i);
  }
  if (n == 0) return ASC_OK;
  ASC_REQUIRE(out && (mode == 2 || x) && (mode == 1 || y), ASC_ERR_INVALID_ARG, "asc_binary: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case ASC_DT_FLOAT32: return launch_binary<F32>(op, mode, x, y, out, n, scalar_f, scalar_i, s);
    case ASC_DT_FLOAT16: return launch_binary<F16>(op, mode, x, y, out, n, scalar_f, scalar_i, s);
    case ASC_DT_BFLOAT16: return launch_binary<BF16>(op, mode, x, y, out, n, scalar_f, scalar_i, s);
    case ASC_DT_INT32: return launch_binary<I32>(op, mode, x, y, out, n, scalar_f, scalar_i, s);
    case ASC_DT_INT16: return launch_binary<I16>(op, mode, x, y, out, n, scalar_f, scalar_i, s);
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_binary: unsupported dtype code %d", dtype);
  }
}

extern "C" int32_t asc_where_cmp(int32_t cmp, int32_t dtype, const void* x, const void* y, void* out, int64_t n,
                                 int32_t mode, double scalar_f, int64_t scalar_i, double true_value,
                                 double false_value, asc_stream_t stream) {
  ASC_REQUIRE(cmp >= 0 && cmp <= 5, ASC_ERR_INVALID_ARG, "asc_where_cmp: unknown comparison code %d", cmp);
  ASC_REQUIRE(mode == 0 || mode == 1, ASC_ERR_INVALID_ARG, "asc_where_cmp: unknown operand mode %d", mode);
  ASC_REQUIRE(n >= 0, ASC_ERR_INVALID_ARG, "asc_where_cmp: negative length");
  if (n == 0) return ASC_OK;
  ASC_REQUIRE(x && out && (mode == 1 || y), ASC_ERR_INVALID_ARG, "asc_where_cmp: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case ASC_DT_FLOAT32:
      return launch_where<F32>(cmp, mode, x, y, out, n, scalar_f, scalar_i, true_value, false_value, s);
    case ASC_DT_FLOAT16:
      return launch_where<F16>(cmp, mode, x, y, out, n, scalar_f, scalar_i, true_value, false_value, s);
    case ASC_DT_BFLOAT16:
      return launch_where<BF16>(cmp, mode, x, y, out, n, scalar_f, scalar_i, true_value, false_value, s);
    case ASC_DT_INT32:
      return launch_where<I32>(cmp, mode, x, y, out, n, scalar_f, scalar_i, true_value, false_value, s);
    case ASC_DT_INT16:
      return launch_where<I16>(cmp, mode, x, y, out, n, scalar_f, scalar_i, true_value, false_value, s);
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_where_cmp: unsupported dtype code %d", dtype);
  }
}

extern "C" int32_t asc_rect_binary(int32_t op, int32_t dtype, const void* x, const void* y, void* z, int64_t rows,
                                   int64_t cols, int64_t r0, int64_t c0, int64_t h, int64_t w,
                                   asc_stream_t stream) {
  ASC_REQUIRE(op >= 0 && op <= 5, ASC_ERR_INVALID_ARG, "asc_rect_binary: op code %d is not element-wise", op);
  ASC_REQUIRE(rows >= 0 && cols >= 0 && h >= 0 && w >= 0, ASC_ERR_INVALID_ARG, "asc_rect_binary: negative shape");
  ASC_REQUIRE(r0 >= 0 && c0 >= 0, ASC_ERR_INVALID_ARG, "asc_rect_binary: negative offset");
  // the store clips at the tensor bounds
  if (r0 + h > rows) h = rows > r0 ? rows - r0 : 0;
  if (c0 + w > cols) w = cols > c0 ? cols - c0 : 0;
  if (h == 0 || w == 0) return ASC_OK;
  ASC_REQUIRE(x && y && z, ASC_ERR_INVALID_ARG, "asc_rect_binary: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(h * w));
#define ASC_RECT(E)                                                                                              \
  hipLaunchKernelGGL(rect_binary_kernel<E>, grid, dim3(kThreads), 0, s, op, static_cast<const E::T*>(x),         \
                     static_cast<const E::T*>(y), static_cast<E::T*>(z), cols, r0, c0, h, w);                    \
  return asc::check_launch("asc_rect_binary")
  switch (dtype) {
    case ASC_DT_FLOAT32: ASC_RECT(F32);
    case ASC_DT_FLOAT16: ASC_RECT(F16);
    case ASC_DT_BFLOAT16: ASC_RECT(BF16);
    case ASC_DT_INT32: ASC_RECT(I32);
    case ASC_DT_INT16: ASC_RECT(I16);
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_rect_binary: unsupported dtype code %d", dtype);
  }
#undef ASC_RECT
}

extern "C" int32_t asc_broadcast_rows(int32_t elem_bytes, const void* x, void* z, int64_t rows, int64_t cols,
                                      asc_stream_t stream) {
  ASC_REQUIRE(rows >= 0 && cols >= 0, ASC_ERR_INVALID_ARG, "asc_broadcast_rows: negative shape");
  if (rows == 0 || cols == 0) return ASC_OK;
  ASC_REQUIRE(x && z, ASC_ERR_INVALID_ARG, "asc_broadcast_rows: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(rows * cols));
  switch (elem_bytes) {
    case 1:
      hipLaunchKernelGGL(broadcast_rows_kernel<uint8_t>, grid, dim3(kThreads), 0, s, static_cast<const uint8_t*>(x),
                         static_cast<uint8_t*>(z), rows, cols);
      break;
    case 2:
      hipLaunchKernelGGL(broadcast_rows_kernel<uint16_t>, grid, dim3(kThreads), 0, s,
                         static_cast<const uint16_t*>(x), static_cast<uint16_t*>(z), rows, cols);
      break;
    case 4:
      hipLaunchKernelGGL(broadcast_rows_kernel<uint32_t>, grid, dim3(kThreads), 0, s,
                         static_cast<const uint32_t*>(x), static_cast<uint32_t*>(z), rows, cols);
      break;
    case 8:
      hipLaunchKernelGGL(broadcast_rows_kernel<uint64_t>, grid, dim3(kThreads), 0, s,
                         static_cast<const uint64_t*>(x), static_cast<uint64_t*>(z), rows, cols);
      break;
    default:
      return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_broadcast_rows: element size %d not supported", elem_bytes);
  }
  return asc::check_launch("asc_broadcast_rows");
}

extern "C" int32_t asc_atomic_tiles(int32_t op, int32_t dtype, const void* x, void* z, int64_t n_tiles,
                                    int64_t tile_len, double c_f, int64_t c_i, asc_stream_t stream) {
  ASC_REQUIRE(op == ASC_BIN_ADD || op == ASC_BIN_MAXIMUM || op == ASC_BIN_MINIMUM, ASC_ERR_INVALID_ARG,
              "asc_atomic_tiles: op code %d is not add / maximum / minimum", op);
  ASC_REQUIRE(n_tiles >= 0 && tile_len >= 0, ASC_ERR_INVALID_ARG, "asc_atomic_tiles: negative shape");
  if (n_tiles == 0 || tile_len == 0) return ASC_OK;
  ASC_REQUIRE(n_tiles <= INT64_MAX / tile_len, ASC_ERR_INVALID_ARG, "asc_atomic_tiles: size overflows");
  ASC_REQUIRE(x && z, ASC_ERR_INVALID_ARG, "asc_atomic_tiles: null buffer");
  const int64_t n = n_tiles * tile_len;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n));
#define ASC_ATOMIC(E)                                                                                            \
  hipLaunchKernelGGL(atomic_tiles_kernel<E>, grid, dim3(kThreads), 0, s, op, static_cast<const E::T*>(x),        \
                     static_cast<E::T*>(z), tile_len, n, static_cast<float>(c_f), c_i);                          \
  return asc::check_launch("asc_atomic_tiles")
  switch (dtype) {
    case ASC_DT_FLOAT32: ASC_ATOMIC(F32);
    case ASC_DT_FLOAT16: ASC_ATOMIC(F16);
    case ASC_DT_BFLOAT16: ASC_ATOMIC(BF16);
    case ASC_DT_INT32: ASC_ATOMIC(I32);
    case ASC_DT_INT16: ASC_ATOMIC(I16);
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_atomic_tiles: unsupported dtype code %d", dtype);
  }
#undef ASC_ATOMIC
}

extern "C" int32_t asc_fill(int32_t dtype, void* z, int64_t n, double c_f, int64_t c_i, asc_stream_t stream) {
  ASC_REQUIRE(n >= 0, ASC_ERR_INVALID_ARG, "asc_fill: negative length");
  if (n == 0) return ASC_OK;
  ASC_REQUIRE(z, ASC_ERR_INVALID_ARG, "asc_fill: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n));
#define ASC_FILL(E)                                                                                              \
  hipLaunchKernelGGL(fill_kernel<E>, grid, dim3(kThreads), 0, s, static_cast<E::T*>(z), n,                       \
                     static_cast<float>(c_f), c_i);                                                              \
  return asc::check_launch("asc_fill")
  switch (dtype) {
    case ASC_DT_FLOAT32: ASC_FILL(F32);
    case ASC_DT_FLOAT16: ASC_FILL(F16);
    case ASC_DT_BFLOAT16: ASC_FILL(BF16);
    case ASC_DT_INT32: ASC_FILL(I32);
    case ASC_DT_INT16: ASC_FILL(I16);
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_fill: unsupported dtype code %d", dtype);
  }
#undef ASC_FILL
}

extern "C" int32_t asc_quant_i8(int32_t dtype, const void* src, int8_t* dst, double scale, double offset, int64_t n,
                                asc_stream_t stream) {
  ASC_REQUIRE(n >= 0, ASC_ERR_INVALID_ARG, "asc_quant_i8: negative length");
  if (n == 0) return ASC_OK;
  ASC_REQUIRE(src && dst, ASC_ERR_INVALID_ARG, "asc_quant_i8: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n));
  switch (dtype) {
    case ASC_DT_FLOAT32:
      hipLaunchKernelGGL(quant_i8_kernel<F32>, grid, dim3(kThreads), 0, s, static_cast<const float*>(src), dst,
                         static_cast<float>(scale), static_cast<float>(offset), n);
      break;
    case ASC_DT_FLOAT16:
      hipLaunchKernelGGL(quant_i8_kernel<F16>, grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(src), dst,
                         static_cast<float>(scale), static_cast<float>(offset), n);
      break;
    case ASC_DT_BFLOAT16:
      hipLaunchKernelGGL(quant_i8_kernel<BF16>, grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(src), dst,
                         static_cast<float>(scale), static_cast<float>(offset), n);
      break;
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_quant_i8: unsupported dtype code %d", dtype);
  }
  return asc::check_launch("asc_quant_i8");
}
