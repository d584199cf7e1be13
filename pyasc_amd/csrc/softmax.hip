// Row softmax for the two asc2 softmax kernels:
//   test_softmax.py:16-27        grid-stride rows, one [1, tile_size] tile per row
//   test_softmax_fused.py:16-24  contiguous row blocks through asc2.softmax
// Both reduce to: for each covered row r, out[r, :L] = exp(x - max) / sum(exp(x - max))
// over the row's first L columns (row stride S).
//
// HBM-bound (one read + one write of every element).  Rows up to 8192 columns
// stay in registers: a wave per row up to 1024 columns, a 256-thread block per
// row above that (measured faster at 4096 columns than a wave per row).  Max and sum reduce in-thread, then by wave butterfly
// (__shfl_xor), then across waves through LDS.  exp is the accurate libm expf
// and the normalisation is a true division, as the reference's DivL2
// (lib/Conversion/LowerToAsc/LowerArithBinary.cpp:116).
#include <math.h>

#include "common.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct RowView {
  const float* x;
  float* out;
  int64_t rows;    // covered rows [0, rows)
  int64_t stride;  // elements between row starts
  int32_t len;     // columns processed per row
  bool vec_ok;     // rows start 16-byte aligned
};

// Loads vector q (elements 4q..4q+3) of a row, padding with -inf past `len`.
__device__ __forceinline__ float4 load_vec(const float* row, int q, int len, bool vec_ok) {
  const int e = q * 4;
  if (vec_ok && e + 3 < len) {
    // streamed once: non-temporal so the rows do not displace other cached data
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row + e));
    return make_float4(v.x, v.y, v.z, v.w);
  }
  float4 v;
  v.x = e + 0 < len ? row[e + 0] : -INFINITY;
  v.y = e + 1 < len ? row[e + 1] : -INFINITY;
  v.z = e + 2 < len ? row[e + 2] : -INFINITY;
  v.w = e + 3 < len ? row[e + 3] : -INFINITY;
  return v;
}

__device__ __forceinline__ void store_vec(float* row, int q, int len, bool vec_ok, float4 v) {
  const int e = q * 4;
  if (vec_ok && e + 3 < len) {
    __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4*>(row + e));
    return;
  }
  if (e + 0 < len) row[e + 0] = v.x;
  if (e + 1 < len) row[e + 1] = v.y;
  if (e + 2 < len) row[e + 2] = v.z;
  if (e + 3 < len) row[e + 3] = v.w;
}

// exp(v - m) with masked (-inf) lanes giving exactly 0.
__device__ __forceinline__ float4 exp_shift(float4 v, float m) {
  float4 r;
  r.x = expf(v.x - m);
  r.y = expf(v.y - m);
  r.z = expf(v.z - m);
  r.w = expf(v.w - m);
  return r;
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
    const float* row = p.x + (r0 + k) * p.stride;
#pragma unroll
    for (int j = 0; j < VPL; ++j) v[k][j] = load_vec(row, lane + 64 * j, p.len, p.vec_ok);
  }
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    if (r0 + k >= p.rows) continue;
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPL; ++j) m = fmaxf(m, fmaxf(fmaxf(v[k][j].x, v[k][j].y), fmaxf(v[k][j].z, v[k][j].w)));
    m = asc::wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      v[k][j] = exp_shift(v[k][j], m);
      s += (v[k][j].x + v[k][j].y) + (v[k][j].z + v[k][j].w);
    }
    s = asc::wave_sum(s);
    float* orow = p.out + (r0 + k) * p.stride;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float4 o = make_float4(v[k][j].x / s, v[k][j].y / s, v[k][j].z / s, v[k][j].w / s);
      store_vec(orow, lane + 64 * j, p.len, p.vec_ok, o);
    }
  }
}

// One 256-thread block per kRows rows; each thread holds VPT float4 vectors of
// each row.  All rows are loaded first; the cross-wave max and sum of all rows
// share one barrier each.
template <int VPT, int kRows>
__global__ void __launch_bounds__(256) softmax_block_kernel(RowView p) {
  constexpr int kWaves = 256 / 64;
  __shared__ float red[2][kRows][kWaves];
  const int t = threadIdx.x;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows;
  float4 v[kRows][VPT];
  float m[kRows], s[kRows];
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    const bool live = r0 + k < p.rows;
    const float* row = p.x + (live ? r0 + k : r0) * p.stride;
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[k][j] = load_vec(row, t + 256 * j, live ? p.len : 0, p.vec_ok);
  }
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    m[k] = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPT; ++j)
      m[k] = fmaxf(m[k], fmaxf(fmaxf(v[k][j].x, v[k][j].y), fmaxf(v[k][j].z, v[k][j].w)));
    m[k] = asc::wave_max(m[k]);
    if ((t & 63) == 0) red[0][k][t >> 6] = m[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    m[k] = fmaxf(fmaxf(red[0][k][0], red[0][k][1]), fmaxf(red[0][k][2], red[0][k][3]));
    s[k] = 0.f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      v[k][j] = exp_shift(v[k][j], m[k]);
      s[k] += (v[k][j].x + v[k][j].y) + (v[k][j].z + v[k][j].w);
    }
    s[k] = asc::wave_sum(s[k]);
    if ((t & 63) == 0) red[1][k][t >> 6] = s[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    if (r0 + k >= p.rows) continue;
    const float sum = (red[1][k][0] + red[1][k][1]) + (red[1][k][2] + red[1][k][3]);
    float* orow = p.out + (r0 + k) * p.stride;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      float4 o = make_float4(v[k][j].x / sum, v[k][j].y / sum, v[k][j].z / sum, v[k][j].w / sum);
      store_vec(orow, t + 256 * j, p.len, p.vec_ok, o);
    }
  }
}

// Rows longer than the register-resident variants: three passes over the row.
__global__ void __launch_bounds__(256) softmax_long_kernel(RowView p) {
  constexpr int kWaves = 256 / 64;
  __shared__ float red[2][kWaves];
  const int t = threadIdx.x;
  const int64_t r = blockIdx.x;
  const float* row = p.x + r * p.stride;
  const int nvec = (p.len + 3) / 4;
  float m = -INFINITY;
  for (int q = t; q < nvec; q += 256) {
    float4 v = load_vec(row, q, p.len, p.vec_ok);
    m = fmaxf(m, fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
  }
  m = asc::wave_max(m);
  if ((t & 63) == 0) red[0][t >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  float s = 0.f;
  for (int q = t; q < nvec; q += 256) {
    float4 v = exp_shift(load_vec(row, q, p.len, p.vec_ok), m);
    s += (v.x + v.y) + (v.z + v.w);
  }
  s = asc::wave_sum(s);
  if ((t & 63) == 0) red[1][t >> 6] = s;
  __syncthreads();
  s = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  float* orow = p.out + r * p.stride;
  for (int q = t; q < nvec; q += 256) {
    float4 v = exp_shift(load_vec(row, q, p.len, p.vec_ok), m);
    store_vec(orow, q, p.len, p.vec_ok, make_float4(v.x / s, v.y / s, v.z / s, v.w / s));
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
    hipLaunchKernelGGL((softmax_wave_kernel<4, 2>), wave_grid, block, 0, stream, p);
  } else if (L <= 2048) {
    hipLaunchKernelGGL((softmax_block_kernel<2, 1>), dim3(static_cast<uint32_t>(p.rows)), block, 0, stream, p);
  } else if (L <= 4096) {
    // one row per block measured fastest here (2 rows per block, or persistent
    // blocks streaming rows, lose occupancy or add a launch round)
    hipLaunchKernelGGL((softmax_block_kernel<4, 1>), dim3(static_cast<uint32_t>(p.rows)), block, 0, stream, p);
  } else if (L <= 8192) {
    hipLaunchKernelGGL((softmax_block_kernel<8, 1>), dim3(static_cast<uint32_t>(p.rows)), block, 0, stream, p);
  } else {
    hipLaunchKernelGGL(softmax_long_kernel, dim3(static_cast<uint32_t>(p.rows)), block, 0, stream, p);
  }
  return asc::check_launch(who);
}

bool rows_aligned(const float* x, const float* out, int64_t stride) {
  return asc::aligned16(x) && asc::aligned16(out) && (stride % 4) == 0;
}

}  // namespace

extern "C" int32_t asc_softmax_rows_f32(const float* x, float* out, int64_t num_rows, int64_t num_cols,
                                        int32_t tile_size, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(num_rows >= 0 && num_cols >= 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_rows_f32: negative shape (%lld, %lld)", (long long)num_rows, (long long)num_cols);
  ASC_REQUIRE(tile_size > 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_softmax_rows_f32: need tile_size > 0 and grid > 0 (got %d, %d)", tile_size, grid);
  ASC_REQUIRE(tile_size <= num_cols, ASC_ERR_UNSUPPORTED,
              "asc_softmax_rows_f32: tile_size %d > num_cols %lld (the reference's padded reduction and "
              "row-spilling store are not reproduced)",
              tile_size, (long long)num_cols);
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
