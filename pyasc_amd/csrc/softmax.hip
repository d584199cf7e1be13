// Row softmax for the two asc2 softmax kernels:
//   test_softmax.py:16-27        grid-stride rows, one [1, tile_size] tile per row
//   test_softmax_fused.py:16-24  contiguous row blocks through asc2.softmax
// Both reduce to: for each covered row r, out[r, :L] = exp(x - max) / sum(exp(x - max))
// over the row's first L columns (row stride S).
//
// HBM-bound (one read + one write of every element).  Rows up to 8192 columns
// stay in registers: a wave per row (two rows per wave) up to 512 columns, a
// 128- or 256-thread block per row above (see launch_rows).  Max, min and sum reduce in-thread,
// then across the wave with DPP and permlane swaps (no LDS round trips), then
// across waves through LDS.  x - max is rounded to fp32 as in the reference
// (test_softmax.py:22-24); exp of it is accurate to ~2 ulp (the row's min picks
// a shorter exp when no result can fall below 2^-126) and the
// normalisation multiplies by one correctly rounded reciprocal per row, which
// stays within 2 ulp of the reference's true division (DivL2,
// lib/Conversion/LowerToAsc/LowerArithBinary.cpp:116).
#include <math.h>

#include "common.h"
#include "rows.h"

namespace {

using asc::rows::f32x4;
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

// One wave per row; each lane holds VPL float4 vectors of each of kRows rows
// (all rows' loads are issued before any reduction, so more bytes are in flight).
template <int VPL, int kRows>
__global__ void __launch_bounds__(256) softmax_wave_kernel(RowView p) {
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

// One kThreads-thread block per row; each thread holds VPT float4 vectors.
// The cross-wave max/min and sum go through LDS, one barrier each.
template <int VPT, int kThreads>
__global__ void __launch_bounds__(kThreads) softmax_block_kernel(RowView p) {
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

// Rows longer than the register-resident variants: three passes over the row.
__global__ void __launch_bounds__(256) softmax_long_kernel(RowView p) {
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

int32_t launch_rows(const RowView& p, hipStream_t stream, const char* who) {
  if (p.rows == 0 || p.len == 0) return ASC_OK;
  const int64_t L = p.len;
  const dim3 block(256);
  // 2 rows per wave (measured faster at 1024 columns than 1)
  const dim3 wave_grid(static_cast<uint32_t>(asc::ceil_div(p.rows, 8)));
  if (L <= 256) {
    hipLaunchKernelGGL((softmax_wave_kernel<1, 2>), wave_grid, block, 0, stream, p);
  } else if (L <= 512) {
    hipLaunchKernelGGL((softmax_wave_kernel<2, 2>), wave_grid, block, 0, stream, p);
  } else if (L <= 1024) {
    // Above 512 columns a row takes several waves with 2-4 vectors per lane:
    // more, shorter waves than one wave per row, and each wave's loads, cross-wave
    // reductions and stores finish sooner (fp32 rows, 64 MiB in and out, same
    // box: 1024 columns 5500-5560 GB/s with one wave per two rows, 5950 here;
    // 2048: 5680 with two waves per row, 5870 with four; 4096: 5560-5590 with
    // two waves per row, 5740-5780 with four, beside a 5840-5850 GB/s copy).
    hipLaunchKernelGGL((softmax_block_kernel<2, 128>), dim3(static_cast<uint32_t>(p.rows)), dim3(128), 0, stream, p);
  } else if (L <= 2048) {
    hipLaunchKernelGGL((softmax_block_kernel<2, 256>), dim3(static_cast<uint32_t>(p.rows)), block, 0, stream, p);
  } else if (L <= 4096) {
    hipLaunchKernelGGL((softmax_block_kernel<4, 256>), dim3(static_cast<uint32_t>(p.rows)), block, 0, stream, p);
  } else if (L <= 8192) {
    hipLaunchKernelGGL((softmax_block_kernel<8, 256>), dim3(static_cast<uint32_t>(p.rows)), block, 0, stream, p);
  } else {
    hipLaunchKernelGGL(softmax_long_kernel, dim3(static_cast<uint32_t>(p.rows)), block, 0, stream, p);
  }
  return asc::check_launch(who);
}

bool rows_aligned(const float* x, const float* out, int64_t stride) {
  return asc::aligned16(x) && asc::aligned16(out) && (stride % 4) == 0;
}

// ---- float16 rows (asc2.softmax on an f16 tile, python/asc/language/tile/unary_ops.py:213-222;
// python/test/asc2/operations/test_softmax.py).  fp32 statistics: x - max rounded
// to fp32, libm expf, one reciprocal of the sum, then one RNE rounding of each
// output to fp16.  One 256-thread workgroup per row, three passes over the row
// (max, sum, normalise + store); 16-byte vectors of 8 halves when aligned.
struct RowView16 {
  const uint16_t* x;
  uint16_t* out;
  int64_t rows, stride;
  int32_t len;
  bool vec_ok;  // 16-byte aligned rows and len % 8 == 0
};

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

__global__ void __launch_bounds__(256) softmax_f16_kernel(RowView16 p) {
  __shared__ float red[2][4];
  const int t = threadIdx.x;
  const int nvec = p.vec_ok ? p.len / 8 : 0;
  for (int64_t r = blockIdx.x; r < p.rows; r += gridDim.x) {
    const uint16_t* row = p.x + r * p.stride;
    uint16_t* orow = p.out + r * p.stride;
    float m = -INFINITY;
    for (int q = t; q < nvec; q += 256) {
      float f[8];
      halves8(reinterpret_cast<const u32x4_t*>(row)[q], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, f[i]);
    }
    for (int c = nvec * 8 + t; c < p.len; c += 256) m = fmaxf(m, half_at(row, c));
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
    for (int c = nvec * 8 + t; c < p.len; c += 256) s += expf(half_at(row, c) - m);
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
    for (int c = nvec * 8 + t; c < p.len; c += 256) orow[c] = to_half(expf(half_at(row, c) - m) * rs);
  }
}

int32_t launch_rows_f16(const RowView16& p, hipStream_t stream, const char* who) {
  if (p.rows == 0 || p.len == 0) return ASC_OK;
  const int64_t blocks = p.rows < 65536 ? p.rows : 65536;
  hipLaunchKernelGGL(softmax_f16_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, p);
  return asc::check_launch(who);
}

bool rows_aligned16(const void* x, const void* out, int64_t stride, int64_t len) {
  return asc::aligned16(x) && asc::aligned16(out) && (stride % 8) == 0 && (len % 8) == 0;
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
// running the rows in order on one block leaves).  One 256-thread workgroup per row
// (grid-stride), three passes; not a tuned path.
template <bool kHalf>
__device__ __forceinline__ float padded_at(const void* row, int64_t c) {
  if constexpr (kHalf) return half_at(static_cast<const uint16_t*>(row), static_cast<int>(c));
  else return static_cast<const float*>(row)[c];
}

template <bool kHalf>
__global__ void __launch_bounds__(256) softmax_padded_kernel(const void* x, void* out, int64_t rows, int64_t cols,
                                                             int32_t pad) {
  __shared__ float red[2][4];
  const int t = threadIdx.x;
  constexpr int64_t kES = kHalf ? 2 : 4;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const void* row = static_cast<const uint8_t*>(x) + r * cols * kES;
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
      if constexpr (kHalf) static_cast<uint16_t*>(out)[r * cols + c] = to_half(v);
      else static_cast<float*>(out)[r * cols + c] = v;
    }
  }
}

template <bool kHalf>
int32_t launch_padded(const void* x, void* out, int64_t rows, int64_t cols, int32_t tile, hipStream_t stream,
                      const char* who) {
  if (rows == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "%s: null buffer", who);
  const int64_t blocks = rows < 65536 ? rows : 65536;
  hipLaunchKernelGGL((softmax_padded_kernel<kHalf>), dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, x,
                     out, rows, cols, static_cast<int32_t>(tile - cols));
  return asc::check_launch(who);
}

}  // namespace

extern "C" int32_t asc_softmax_rows_f32(const float* x, float* out, int64_t num_rows, int64_t num_cols,
                                        int32_t tile_size, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(num_rows >= 0 && num_cols >= 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_rows_f32: negative shape (%lld, %lld)", (long long)num_rows, (long long)num_cols);
  ASC_REQUIRE(tile_size > 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_rows_f32: need tile_size > 0 and grid > 0 (got %d, %d)", tile_size, grid);
  if (tile_size > num_cols) {
    return launch_padded<false>(x, out, num_rows, num_cols, tile_size, static_cast<hipStream_t>(stream),
                                "asc_softmax_rows_f32");
  }
  if (num_rows == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "asc_softmax_rows_f32: null buffer");
  // Rows b, b+grid, ... for b < grid cover every row exactly once.
  RowView p{x, out, num_rows, num_cols, tile_size, rows_aligned(x, out, num_cols)};
  return launch_rows(p, static_cast<hipStream_t>(stream), "asc_softmax_rows_f32");
}

extern "C" int32_t asc_softmax_blocks_f32(const float* x, float* out, int64_t num_rows, int64_t num_cols,
                                          int32_t block_size, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(num_rows >= 0 && num_cols >= 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_blocks_f32: negative shape (%lld, %lld)", (long long)num_rows, (long long)num_cols);
  ASC_REQUIRE(block_size > 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_blocks_f32: need block_size > 0 and grid > 0 (got %d, %d)", block_size, grid);
  ASC_REQUIRE(num_cols <= INT32_MAX, ASC_ERR_UNSUPPORTED, "asc_softmax_blocks_f32: num_cols too large");
  const int64_t reach = static_cast<int64_t>(grid) * block_size;
  const int64_t rows = reach < num_rows ? reach : num_rows;
  if (rows == 0 || num_cols == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "asc_softmax_blocks_f32: null buffer");
  RowView p{x, out, rows, num_cols, static_cast<int32_t>(num_cols), rows_aligned(x, out, num_cols)};
  return launch_rows(p, static_cast<hipStream_t>(stream), "asc_softmax_blocks_f32");
}

extern "C" int32_t asc_softmax_rows_f16(const void* x, void* out, int64_t num_rows, int64_t num_cols,
                                        int32_t tile_size, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(num_rows >= 0 && num_cols >= 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_rows_f16: negative shape (%lld, %lld)", (long long)num_rows, (long long)num_cols);
  ASC_REQUIRE(tile_size > 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_rows_f16: need tile_size > 0 and grid > 0 (got %d, %d)", tile_size, grid);
  if (tile_size > num_cols) {
    return launch_padded<true>(x, out, num_rows, num_cols, tile_size, static_cast<hipStream_t>(stream),
                               "asc_softmax_rows_f16");
  }
  if (num_rows == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "asc_softmax_rows_f16: null buffer");
  RowView16 p{static_cast<const uint16_t*>(x), static_cast<uint16_t*>(out), num_rows, num_cols, tile_size,
              rows_aligned16(x, out, num_cols, tile_size)};
  return launch_rows_f16(p, static_cast<hipStream_t>(stream), "asc_softmax_rows_f16");
}

extern "C" int32_t asc_softmax_blocks_f16(const void* x, void* out, int64_t num_rows, int64_t num_cols,
                                          int32_t block_size, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(num_rows >= 0 && num_cols >= 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_blocks_f16: negative shape (%lld, %lld)", (long long)num_rows, (long long)num_cols);
  ASC_REQUIRE(block_size > 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_blocks_f16: need block_size > 0 and grid > 0 (got %d, %d)", block_size, grid);
  ASC_REQUIRE(num_cols <= INT32_MAX, ASC_ERR_UNSUPPORTED, "asc_softmax_blocks_f16: num_cols too large");
  const int64_t reach = static_cast<int64_t>(grid) * block_size;
  const int64_t rows = reach < num_rows ? reach : num_rows;
  if (rows == 0 || num_cols == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "asc_softmax_blocks_f16: null buffer");
  RowView16 p{static_cast<const uint16_t*>(x), static_cast<uint16_t*>(out), rows, num_cols,
              static_cast<int32_t>(num_cols), rows_aligned16(x, out, num_cols, num_cols)};
  return launch_rows_f16(p, static_cast<hipStream_t>(stream), "asc_softmax_blocks_f16");
}
