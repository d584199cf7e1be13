// Row softmax device code: the element math and the row bodies of the two asc2
// softmax kernels
//   test_softmax.py:16-27        grid-stride rows, one [1, tile_size] tile per row
//   test_softmax_fused.py:16-24  contiguous row blocks through asc2.softmax
// (python/test/asc2/kernels/).  Both reduce to: for each covered row r,
// out[r, :L] = exp(x - max) / sum(exp(x - max)) over the row's first L columns
// (row stride S).  Shared by the library (softmax.hip, launched through
// asc_softmax_*) and the standalone gfx950 code object (co/asc2_softmax.hip,
// loaded with hipModuleLoad by the asc2 launch path), so both launch paths run
// the same instructions.
//
// Every body takes the same six arguments,
//   (x, out, rows, stride, len, flag)
// where flag is "rows start 16-byte aligned" for the register-resident and f16
// bodies and the pad count (tile - num_cols) for the padded bodies.
//
// HBM-bound (one read + one write of every element).  Rows up to 8192 columns
// stay in registers: a wave per row (two rows per wave) up to 512 columns, a
// 128- or 256-thread block per row above (asc_softmax_plan picks the body).  Max,
// min and sum reduce in-thread, then across the wave with DPP and permlane
// swaps (no LDS round trips), then across waves through LDS.  x - max is
// rounded to fp32 as in the reference (test_softmax.py:22-24); exp of it is
// accurate to ~2 ulp (the row's min picks a shorter exp when no result can fall
// below 2^-126) and the normalisation multiplies by one correctly rounded
// reciprocal per row, which stays within 2 ulp of the reference's true division
// (DivL2, lib/Conversion/LowerToAsc/LowerArithBinary.cpp:116).
#pragma once

#include <math.h>

#include "common.h"
#include "rows.h"

namespace asc {
namespace softmax {

using asc::rows::load_row;
using asc::rows::load_vec;
using asc::rows::RowView;
using asc::rows::store_row;
using asc::rows::store_vec;

// softmax rows are padded with -inf (no effect on max, sum or the exp path)
constexpr float kPad = -INFINITY;

constexpr float kL2E = 1.44269504088896340736f;   // log2(e) rounded to fp32
constexpr float kL2ELo = 1.925963033500011e-08f;  // log2(e) - kL2E
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kMinNormalLog2 = -126.0f;

// Normalises the row in registers and stores it.
template <int N, int kStride>
__device__ __forceinline__ void store_scaled(float4 (&v)[N], float* row, int q0, int len, bool vec_ok, float rs) {
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = make_float4(v[j].x * rs, v[j].y * rs, v[j].z * rs, v[j].w * rs);
  store_row<N, kStride>(v, row, q0, len, vec_ok);
}

// exp(y) for finite y <= 0 with y*log2(e) >= -126 (the caller checks the row's
// range), within ~2 ulp: t = y*log2(e) rounded, v_exp_f32 of t, and a
// first-order correction by the rounding residual, taken from a two-term split
// of log2(e) (Cody-Waite).
__device__ __forceinline__ float exp_plain(float y) {
  const float t = y * kL2E;
  const float err = fmaf(y, kL2ELo, fmaf(y, kL2E, -t));
  const float e = __builtin_amdgcn_exp2f(t);
  return fmaf(e, err * kLn2, e);
}

// exp(y) for any y <= 0 (-inf gives 0, NaN stays NaN).  v_exp_f32 flushes
// results below 2^-126, so those are evaluated 64 octaves up (t + 64 is exact
// for t <= -126) and scaled back by an exact power of two, which rounds once
// into the denormal range.
__device__ __forceinline__ float exp_nonpos(float y) {
  const float t = y * kL2E;
  const float yc = fmaxf(y, -104.0f);  // keeps the residual finite for y = -inf
  const float err = fmaf(yc, kL2ELo, fmaf(yc, kL2E, -(yc * kL2E)));
  const bool tiny = t < kMinNormalLog2;
  const float e = __builtin_amdgcn_exp2f(tiny ? t + 64.0f : t);
  const float r = fmaf(e, err * kLn2, e);
  return tiny ? r * 0x1p-64f : r;
}

// True when every exp(x - m) of a row with maximum m and minimum mn is a
// normal number reached by exp_plain: RN(RN(mn - m) * log2 e) >= -126 bounds
// RN(RN(x - m) * log2 e) for every x of the row (rounding is monotonic).
// mn = -inf (a -inf element or padding) selects the general path.
__device__ __forceinline__ bool plain_range(float m, float mn) { return (mn - m) * kL2E >= kMinNormalLog2; }

// exp(v - m) per lane of a vector
template <bool kPlain>
__device__ __forceinline__ float4 exp_shift(float4 v, float m) {
  float4 r;
  if constexpr (kPlain) {
    r.x = exp_plain(v.x - m);
    r.y = exp_plain(v.y - m);
    r.z = exp_plain(v.z - m);
    r.w = exp_plain(v.w - m);
  } else {
    r.x = exp_nonpos(v.x - m);
    r.y = exp_nonpos(v.y - m);
    r.z = exp_nonpos(v.z - m);
    r.w = exp_nonpos(v.w - m);
  }
  return r;
}

__device__ __forceinline__ float max4(float4 v) { return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)); }
__device__ __forceinline__ float min4(float4 v) { return fminf(fminf(v.x, v.y), fminf(v.z, v.w)); }

// Replaces the vectors of one row by exp(v - m) and returns their sum.  One
// vector at a time (scheduling fence): with many waves per SIMD resident,
// overlapping the exps of several vectors buys nothing and its temporaries
// would cost occupancy.
template <int N>
__device__ __forceinline__ float exp_row(float4 (&v)[N], float m, float mn) {
  float s = 0.f;
  if (plain_range(m, mn)) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      v[j] = exp_shift<true>(v[j], m);
      s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      v[j] = exp_shift<false>(v[j], m);
      s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  return s;
}

__device__ __forceinline__ RowView row_view(const void* x, void* out, int64_t rows, int64_t stride, int32_t len,
                                            int32_t vec_ok) {
  return RowView{static_cast<const float*>(x), static_cast<float*>(out), rows, stride, len, vec_ok != 0};
}

// One wave per row; each lane holds VPL float4 vectors of each of kRows rows
// (all rows' loads are issued before any reduction, so more bytes are in flight).
// 256-thread blocks, four waves: block b covers rows [8b, 8b + 8) for kRows = 2.
template <int VPL, int kRows>
__device__ __forceinline__ void wave_body(const void* x, void* out, int64_t rows, int64_t stride, int32_t len,
                                          int32_t vec_ok) {
  const RowView p = row_view(x, out, rows, stride, len, vec_ok);
  const int lane = threadIdx.x & 63;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * kRows;
  float4 v[kRows][VPL];
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    if (r0 + k >= p.rows) continue;
    load_row<VPL, 64>(v[k], p.x + (r0 + k) * p.stride, lane, p.len, p.vec_ok, kPad);
  }
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    if (r0 + k >= p.rows) continue;
    float m = -INFINITY, mn = INFINITY;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      m = fmaxf(m, max4(v[k][j]));
      mn = fminf(mn, min4(v[k][j]));
    }
    m = asc::wave_max(m);
    mn = asc::wave_min(mn);
    const float rs = 1.0f / asc::wave_sum(exp_row(v[k], m, mn));
    store_scaled<VPL, 64>(v[k], p.out + (r0 + k) * p.stride, lane, p.len, p.vec_ok, rs);
  }
}

// One kThreads-thread block per row (block b is row b); each thread holds VPT
// float4 vectors.  The cross-wave max/min and sum go through LDS, one barrier each.
template <int VPT, int kThreads>
__device__ __forceinline__ void block_body(const void* x, void* out, int64_t rows, int64_t stride, int32_t len,
                                           int32_t vec_ok) {
  const RowView p = row_view(x, out, rows, stride, len, vec_ok);
  constexpr int kWaves = kThreads / 64;
  __shared__ float red[3][kWaves];  // max, min, sum per wave
  const int t = threadIdx.x;
  const int64_t r = blockIdx.x;
  float4 v[VPT];
  load_row<VPT, kThreads>(v, p.x + r * p.stride, t, p.len, p.vec_ok, kPad);
  float m = -INFINITY, mn = INFINITY;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    m = fmaxf(m, max4(v[j]));
    mn = fminf(mn, min4(v[j]));
  }
  m = asc::wave_max(m);
  mn = asc::wave_min(mn);
  if ((t & 63) == 0) {
    red[0][t >> 6] = m;
    red[1][t >> 6] = mn;
  }
  __syncthreads();
  m = red[0][0];
  mn = red[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    m = fmaxf(m, red[0][w]);
    mn = fminf(mn, red[1][w]);
  }
  const float s = asc::wave_sum(exp_row(v, m, mn));
  if ((t & 63) == 0) red[2][t >> 6] = s;
  __syncthreads();
  float sum = red[2][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) sum += red[2][w];
  store_scaled<VPT, kThreads>(v, p.out + r * p.stride, t, p.len, p.vec_ok, 1.0f / sum);
}

// Rows longer than the register-resident bodies: three passes over the row,
// one 256-thread block per row.
__device__ __forceinline__ void long_body(const void* x, void* out, int64_t rows, int64_t stride, int32_t len,
                                          int32_t vec_ok) {
  const RowView p = row_view(x, out, rows, stride, len, vec_ok);
  constexpr int kWaves = 256 / 64;
  __shared__ float red[3][kWaves];
  const int t = threadIdx.x;
  const int64_t r = blockIdx.x;
  const float* row = p.x + r * p.stride;
  const int nvec = (p.len + 3) / 4;
  float m = -INFINITY, mn = INFINITY;
  for (int q = t; q < nvec; q += 256) {
    const float4 v = load_vec(row, q, p.len, p.vec_ok, kPad);
    m = fmaxf(m, max4(v));
    mn = fminf(mn, min4(v));
  }
  m = asc::wave_max(m);
  mn = asc::wave_min(mn);
  if ((t & 63) == 0) {
    red[0][t >> 6] = m;
    red[1][t >> 6] = mn;
  }
  __syncthreads();
  m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  mn = fminf(fminf(red[1][0], red[1][1]), fminf(red[1][2], red[1][3]));
  float s = 0.f;
  for (int q = t; q < nvec; q += 256) {
    float4 v[1] = {load_vec(row, q, p.len, p.vec_ok, kPad)};
    s += exp_row(v, m, mn);
  }
  s = asc::wave_sum(s);
  if ((t & 63) == 0) red[2][t >> 6] = s;
  __syncthreads();
  const float rs = 1.0f / ((red[2][0] + red[2][1]) + (red[2][2] + red[2][3]));
  float* orow = p.out + r * p.stride;
  for (int q = t; q < nvec; q += 256) {
    float4 v[1] = {load_vec(row, q, p.len, p.vec_ok, kPad)};
    exp_row(v, m, mn);
    store_vec(orow, q, p.len, p.vec_ok, make_float4(v[0].x * rs, v[0].y * rs, v[0].z * rs, v[0].w * rs));
  }
}

// ---- float16 rows (asc2.softmax on an f16 tile, python/asc/language/tile/unary_ops.py:213-222;
// python/test/asc2/operations/test_softmax.py).  fp32 statistics: x - max rounded
// to fp32, libm expf, one reciprocal of the sum, then one RNE rounding of each
// output to fp16.  256-thread workgroups over rows b, b + gridDim.x, ..., three
// passes over the row (max, sum, normalise + store); 16-byte vectors of 8 halves
// when vec_ok (16-byte aligned rows and len % 8 == 0).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_at(const uint16_t* p, int i) {
  return static_cast<float>(__builtin_bit_cast(_Float16, p[i]));
}
__device__ __forceinline__ void halves8(u32x4_t v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v[i] & 0xffffu)));
    f[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v[i] >> 16)));
  }
}
__device__ __forceinline__ uint16_t to_half(float v) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

__device__ __forceinline__ void f16_body(const void* xv, void* outv, int64_t rows, int64_t stride, int32_t len,
                                         int32_t vec_ok) {
  __shared__ float red[2][4];
  const uint16_t* x = static_cast<const uint16_t*>(xv);
  uint16_t* out = static_cast<uint16_t*>(outv);
  const int t = threadIdx.x;
  const int nvec = vec_ok ? len / 8 : 0;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const uint16_t* row = x + r * stride;
    uint16_t* orow = out + r * stride;
    float m = -INFINITY;
    for (int q = t; q < nvec; q += 256) {
      float f[8];
      halves8(reinterpret_cast<const u32x4_t*>(row)[q], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, f[i]);
    }
    for (int c = nvec * 8 + t; c < len; c += 256) m = fmaxf(m, half_at(row, c));
    m = asc::wave_max(m);
    __syncthreads();
    if ((t & 63) == 0) red[0][t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float s = 0.f;
    for (int q = t; q < nvec; q += 256) {
      float f[8];
      halves8(reinterpret_cast<const u32x4_t*>(row)[q], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) s += expf(f[i] - m);
    }
    for (int c = nvec * 8 + t; c < len; c += 256) s += expf(half_at(row, c) - m);
    s = asc::wave_sum(s);
    if ((t & 63) == 0) red[1][t >> 6] = s;
    __syncthreads();
    const float rs = 1.0f / ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3]));
    for (int q = t; q < nvec; q += 256) {
      float f[8];
      halves8(reinterpret_cast<const u32x4_t*>(row)[q], f);
      u32x4_t o;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] = static_cast<uint32_t>(to_half(expf(f[2 * i] - m) * rs)) |
               (static_cast<uint32_t>(to_half(expf(f[2 * i + 1] - m) * rs)) << 16);
      reinterpret_cast<u32x4_t*>(orow)[q] = o;
    }
    for (int c = nvec * 8 + t; c < len; c += 256) orow[c] = to_half(expf(half_at(row, c) - m) * rs);
  }
}

// ---- tiles wider than the row (test_softmax.py's softmax_kernel with tile_size >
// num_cols).  The reference's load right-pads the [1, tile] tile with the pad value 0
// (lib/Conversion/LowerToAsc/LowerAscTileDataTransfer.cpp:181-222) and its reductions
// count the whole tile (lib/Conversion/LowerToAsc/LowerAscTile.cpp:428-459), so each
// row's statistics include pad = tile - num_cols zeros:
//   m = max(max_j x_j, 0),  s = sum_j exp(x_j - m) + pad * exp(-m),  out_j = exp(x_j - m) / s.
// Its store then writes the whole tile from the row's start, spilling pad values
// into the next row, where they race with that row's own store whenever the two rows
// run on different blocks; here every row writes its own num_cols values only (what
// running the rows in order on one block leaves).  256-thread workgroups over rows
// b, b + gridDim.x, ..., three passes (rows are contiguous: stride = len = num_cols);
// not a tuned path.
template <bool kHalf>
__device__ __forceinline__ float padded_at(const void* row, int64_t c) {
  if constexpr (kHalf) return half_at(static_cast<const uint16_t*>(row), static_cast<int>(c));
  else return static_cast<const float*>(row)[c];
}

template <bool kHalf>
__device__ __forceinline__ void padded_body(const void* x, void* out, int64_t rows, int64_t stride, int32_t len,
                                            int32_t pad) {
  __shared__ float red[2][4];
  const int t = threadIdx.x;
  constexpr int64_t kES = kHalf ? 2 : 4;
  const int64_t cols = len;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const void* row = static_cast<const uint8_t*>(x) + r * stride * kES;
    float m = pad > 0 ? 0.0f : -INFINITY;  // the padding zeros take part in the maximum
    for (int64_t c = t; c < cols; c += 256) m = fmaxf(m, padded_at<kHalf>(row, c));
    m = asc::wave_max(m);
    __syncthreads();
    if ((t & 63) == 0) red[0][t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float s = 0.f;
    for (int64_t c = t; c < cols; c += 256) s += exp_nonpos(padded_at<kHalf>(row, c) - m);
    s = asc::wave_sum(s);
    if ((t & 63) == 0) red[1][t >> 6] = s;
    __syncthreads();
    s = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    s += static_cast<float>(pad) * exp_nonpos(0.0f - m);
    const float rs = 1.0f / s;
    for (int64_t c = t; c < cols; c += 256) {
      const float v = exp_nonpos(padded_at<kHalf>(row, c) - m) * rs;
      if constexpr (kHalf) static_cast<uint16_t*>(out)[r * stride + c] = to_half(v);
      else static_cast<float*>(out)[r * stride + c] = v;
    }
  }
}

}  // namespace softmax
}  // namespace asc

// Defines the softmax kernels, one per body, as `PREFIX##<body name>` with the
// given linkage specifier (the library's are internal, the code object's have C
// names for hipModuleGetFunction).  The names and their order are those of
// asc_softmax_plan's kernel table.
#define ASC_SOFTMAX_KERNEL(LINKAGE, NAME, THREADS, BODY)                                                            \
  LINKAGE __global__ void __launch_bounds__(THREADS)                                                               \
      NAME(const void* __restrict__ x, void* __restrict__ out, int64_t rows, int64_t stride, int32_t len,          \
           int32_t flag) {                                                                                         \
    BODY(x, out, rows, stride, len, flag);                                                                         \
  }

#define ASC_SOFTMAX_KERNELS(LINKAGE, PREFIX)                                                                       \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##wave_1x2, 256, (asc::softmax::wave_body<1, 2>))                              \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##wave_2x2, 256, (asc::softmax::wave_body<2, 2>))                              \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##block_2x128, 128, (asc::softmax::block_body<2, 128>))                        \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##block_2x256, 256, (asc::softmax::block_body<2, 256>))                        \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##block_2x512, 512, (asc::softmax::block_body<2, 512>))                        \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##block_8x256, 256, (asc::softmax::block_body<8, 256>))                        \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##long, 256, asc::softmax::long_body)                                          \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##f16, 256, asc::softmax::f16_body)                                            \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##padded_f32, 256, asc::softmax::padded_body<false>)                           \
  ASC_SOFTMAX_KERNEL(LINKAGE, PREFIX##padded_f16, 256, asc::softmax::padded_body<true>)
