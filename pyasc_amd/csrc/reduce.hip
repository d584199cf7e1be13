// Row reductions and RMS norm.
//
// asc_reduce_f32 covers the reference's reduction tests
// (python/test/asc2/operations/test_reduce_ops.py): asc2.reduce_{sum,max,min,prod}
// (python/asc/language/tile/reduction_ops.py:61-126) of a 2-D fp32 tile along
// dim 1 (one result per row), dim 0 (one per column) or over all elements
// (the scalar broadcast into an output by asc2.full).  fp32 accumulation; max
// and min return the larger / smaller non-NaN operand (IEEE maxNum / minNum).
//   dim 1: a wave per row, 16-byte loads, in-lane accumulation, DPP/permlane
//          combine (HBM-bound: 4 B per element).
//   dim 0: a thread per column walking the rows (coalesced across threads).
//   all:   one 1024-thread block.
//
// asc_rms_norm covers asc2.rms_norm (python/asc/language/tile/unary_ops.py:225-237,
// AscendC RmsNorm): y = x * rsqrt(mean(x^2) + eps) * gamma along the last dim,
// fp32 or fp16 rows computed in fp32 (a block per row, the row held in
// registers up to 8192 fp32 / 16384 fp16 columns, two 16-byte vectors per lane
// from 1024 fp32 / 2048 fp16 columns up).
#include <math.h>

#include "common.h"
#include "numeric.h"
#include "rows.h"

namespace {

enum ReduceOp { kSum = 0, kMax = 1, kMin = 2, kProd = 3 };

template <int kOp>
__device__ __forceinline__ float identity() {
  return kOp == kSum ? 0.0f : kOp == kMax ? -INFINITY : kOp == kMin ? INFINITY : 1.0f;
}

template <int kOp>
__device__ __forceinline__ float combine(float a, float b) {
  if constexpr (kOp == kSum) return a + b;
  if constexpr (kOp == kMax) return fmaxf(a, b);
  if constexpr (kOp == kMin) return fminf(a, b);
  return a * b;
}

// Wave-wide combine; every lane ends with the same value (see asc::wave_sum).
template <int kOp>
__device__ __forceinline__ float wave_combine(float v) {
  v = combine<kOp>(v, asc::dpp_mov<asc::kDppQuadXor1>(v));
  v = combine<kOp>(v, asc::dpp_mov<asc::kDppQuadXor2>(v));
  v = combine<kOp>(v, asc::dpp_mov<asc::kDppRowHalfMirror>(v));
  v = combine<kOp>(v, asc::dpp_mov<asc::kDppRowMirror>(v));
  v = combine<kOp>(v, asc::lane_xor16(v));
  return combine<kOp>(v, asc::lane_xor32(v));
}

struct ReduceArgs {
  const float* x;
  float* out;
  int64_t rows, cols;
  int64_t out_count;  // "all": number of output elements receiving the result
  bool vec_ok;
};

// dim 1: rows 4*blockIdx.x + wave; four independent vector loads per lane in
// flight, then the in-lane partials are combined in a fixed order.
template <int kOp>
__global__ void __launch_bounds__(256) reduce_rows_kernel(ReduceArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= p.rows) return;
  const float* row = p.x + r * p.cols;
  const int len = static_cast<int>(p.cols);
  float acc[4] = {identity<kOp>(), identity<kOp>(), identity<kOp>(), identity<kOp>()};
  const int nvec = len / 4;
  int q = lane;
  if (p.vec_ok) {
    for (; q + 192 < nvec; q += 256) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = asc::rows::load_vec(row, q + 64 * u, len, true, identity<kOp>());
#pragma unroll
      for (int u = 0; u < 4; ++u)
        acc[u] = combine<kOp>(acc[u], combine<kOp>(combine<kOp>(v[u].x, v[u].y), combine<kOp>(v[u].z, v[u].w)));
    }
  }
  // remaining vectors (and every element when the row is not 16-byte aligned)
  for (int e = q * 4; e < len; e += 256) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (e + i < len) acc[i] = combine<kOp>(acc[i], row[e + i]);
  }
  const float t = combine<kOp>(combine<kOp>(acc[0], acc[1]), combine<kOp>(acc[2], acc[3]));
  const float total = wave_combine<kOp>(t);
  if (lane == 0) p.out[r] = total;
}

// dim 0: thread per column, rows in order.
template <int kOp>
__global__ void __launch_bounds__(256) reduce_cols_kernel(ReduceArgs p) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= p.cols) return;
  float acc = identity<kOp>();
  for (int64_t r = 0; r < p.rows; ++r) acc = combine<kOp>(acc, p.x[r * p.cols + c]);
  p.out[c] = acc;
}

// all elements: one block; the result is written to out[0 .. out_count).
template <int kOp>
__global__ void __launch_bounds__(1024) reduce_all_kernel(ReduceArgs p) {
  __shared__ float part[16];
  const int64_t n = p.rows * p.cols;
  float acc = identity<kOp>();
  for (int64_t i = threadIdx.x; i < n; i += 1024) acc = combine<kOp>(acc, p.x[i]);
  acc = wave_combine<kOp>(acc);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  float total = part[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) total = combine<kOp>(total, part[w]);
  for (int64_t i = threadIdx.x; i < p.out_count; i += 1024) p.out[i] = total;
}

template <int kOp>
int32_t launch_reduce(const ReduceArgs& p, int dim, hipStream_t s) {
  if (dim == 1) {
    // four rows per 256-thread workgroup; one dispatch covers fewer than 2^32 threads
    const int64_t blocks = asc::ceil_div(p.rows, 4);
    ASC_REQUIRE(blocks * 256 < (int64_t{1} << 32), ASC_ERR_UNSUPPORTED, "asc_reduce_f32: %lld rows exceed one launch",
                static_cast<long long>(p.rows));
    hipLaunchKernelGGL(reduce_rows_kernel<kOp>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, p);
  } else if (dim == 0) {
    hipLaunchKernelGGL(reduce_cols_kernel<kOp>, dim3(static_cast<uint32_t>(asc::ceil_div(p.cols, 256))), dim3(256),
                       0, s, p);
  } else {
    hipLaunchKernelGGL(reduce_all_kernel<kOp>, dim3(1), dim3(1024), 0, s, p);
  }
  return asc::check_launch("asc_reduce_f32");
}

// ---- RMS norm

struct F32E {
  using T = float;
  static constexpr int kPerVec = 4;
};
struct F16E {
  using T = uint16_t;
  static constexpr int kPerVec = 8;
};

struct RmsArgs {
  const void* x;
  const float* gamma;
  void* out;
  int64_t rows, stride;  // stride = num_cols (elements between row starts)
  int32_t len;           // columns normalised per row
  float eps;
  bool vec_ok;
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte vector q of a row as fp32 values (0 past len).
template <class E>
__device__ __forceinline__ void load_elems(const typename E::T* row, int q, int len, bool full, float (&v)[E::kPerVec]) {
  constexpr int kP = E::kPerVec;
  const int e = q * kP;
  if (full) {
    const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row) + q);
    typename E::T t[kP];
    __builtin_memcpy(t, &raw, 16);
#pragma unroll
    for (int i = 0; i < kP; ++i) {
      if constexpr (sizeof(typename E::T) == 4) v[i] = t[i];
      else v[i] = asc::f16_to_f32(t[i]);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < kP; ++i) {
    float f = 0.0f;
    if (e + i < len) {
      if constexpr (sizeof(typename E::T) == 4) f = row[e + i];
      else f = asc::f16_to_f32(row[e + i]);
    }
    v[i] = f;
  }
}

template <class E>
__device__ __forceinline__ void store_elems(typename E::T* row, int q, int len, bool full,
                                            const float (&v)[E::kPerVec]) {
  constexpr int kP = E::kPerVec;
  typename E::T t[kP];
#pragma unroll
  for (int i = 0; i < kP; ++i) {
    if constexpr (sizeof(typename E::T) == 4) t[i] = v[i];
    else t[i] = asc::f32_to_f16_rne(v[i]);
  }
  if (full) {
    u32x4 raw;
    __builtin_memcpy(&raw, t, 16);
    __builtin_nontemporal_store(raw, reinterpret_cast<u32x4*>(row) + q);
    return;
  }
  const int e = q * kP;
#pragma unroll
  for (int i = 0; i < kP; ++i)
    if (e + i < len) row[e + i] = t[i];
}

// y = (x * inv_rms) * gamma, inv_rms = 1 / sqrt(sum(x^2) / len + eps)
// (correctly rounded division and square root).  kThreads threads per row,
// VPT 16-byte vectors per thread; gamma is read as 16-byte vectors too.
template <class E, int VPT, int kThreads>
__global__ void __launch_bounds__(kThreads) rms_norm_kernel(RmsArgs p) {
  using T = typename E::T;
  constexpr int kP = E::kPerVec;
  constexpr int kWaves = kThreads / 64;
  __shared__ float red[kWaves];
  const int t = threadIdx.x;
  const int64_t r = blockIdx.x;
  const T* xr = static_cast<const T*>(p.x) + r * p.stride;
  T* orow = static_cast<T*>(p.out) + r * p.stride;
  float v[VPT][kP];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    // uniform test: vector j is inside the row for every thread
    const bool full = p.vec_ok && kThreads * (j + 1) * kP <= p.len;
    load_elems<E>(xr, t + kThreads * j, p.len, full, v[j]);
  }
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < VPT; ++j)
#pragma unroll
    for (int i = 0; i < kP; ++i) ss += v[j][i] * v[j][i];
  ss = asc::wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  float total = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) total += red[w];
  const float inv = 1.0f / sqrtf(total / static_cast<float>(p.len) + p.eps);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int q = t + kThreads * j;
    const bool full = p.vec_ok && kThreads * (j + 1) * kP <= p.len;
    float gm[kP];
    if (full) {
#pragma unroll
      for (int h = 0; h < kP / 4; ++h) {
        const u32x4 g4 = *reinterpret_cast<const u32x4*>(p.gamma + q * kP + 4 * h);
        __builtin_memcpy(gm + 4 * h, &g4, 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kP; ++i) gm[i] = q * kP + i < p.len ? p.gamma[q * kP + i] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kP; ++i) v[j][i] = (v[j][i] * inv) * gm[i];
    store_elems<E>(orow, q, p.len, full, v[j]);
  }
}

// Rows longer than the register-resident variant: two passes over the row.
template <class E>
__global__ void __launch_bounds__(256) rms_norm_long_kernel(RmsArgs p) {
  using T = typename E::T;
  __shared__ float red[4];
  const int t = threadIdx.x;
  const int64_t r = blockIdx.x;
  const T* xr = static_cast<const T*>(p.x) + r * p.stride;
  T* orow = static_cast<T*>(p.out) + r * p.stride;
  auto at = [&](int c) -> float {
    if constexpr (sizeof(T) == 4) return xr[c];
    else return asc::f16_to_f32(xr[c]);
  };
  float ss = 0.0f;
  for (int c = t; c < p.len; c += 256) {
    const float x = at(c);
    ss += x * x;
  }
  ss = asc::wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(total / static_cast<float>(p.len) + p.eps);
  for (int c = t; c < p.len; c += 256) {
    const float y = (at(c) * inv) * p.gamma[c];
    if constexpr (sizeof(T) == 4) orow[c] = y;
    else orow[c] = asc::f32_to_f16_rne(y);
  }
}

template <class E>
int32_t launch_rms(const RmsArgs& p, hipStream_t s) {
  constexpr int kP = E::kPerVec;
  // One workgroup per row, two 16-byte vectors per lane above 256 vectors per row:
  // more, shorter waves per row finish each row's loads, reduction and stores sooner
  // (4096 fp32 columns, 64 MiB in and out, same box: 5480-5530 GB/s with 128 threads
  // x 8 vectors, 5730-5740 with 512 x 2, 5040 with 1024 x 1; 2048 columns: 5500-5550
  // with 128 x 4, 5650-5680 with 256 x 2; 8192: 5370 with 256 x 8, 5510 with 512 x 4,
  // 5560-5570 with 1024 x 2).  Two passes over longer rows.
  const int64_t vecs = (static_cast<int64_t>(p.len) + kP - 1) / kP;
  const int64_t threads = vecs <= 256 ? 128 : vecs <= 512 ? 256 : vecs <= 1024 ? 512 : vecs <= 2048 ? 1024 : 256;
  // one dispatch covers fewer than 2^32 threads
  ASC_REQUIRE(p.rows * threads < (int64_t{1} << 32), ASC_ERR_UNSUPPORTED, "asc_rms_norm: %lld rows exceed one launch",
              static_cast<long long>(p.rows));
  const dim3 grid(static_cast<uint32_t>(p.rows));
  if (vecs <= 128) {
    hipLaunchKernelGGL((rms_norm_kernel<E, 1, 128>), grid, dim3(128), 0, s, p);
  } else if (vecs <= 256) {
    hipLaunchKernelGGL((rms_norm_kernel<E, 2, 128>), grid, dim3(128), 0, s, p);
  } else if (vecs <= 512) {
    hipLaunchKernelGGL((rms_norm_kernel<E, 2, 256>), grid, dim3(256), 0, s, p);
  } else if (vecs <= 1024) {
    hipLaunchKernelGGL((rms_norm_kernel<E, 2, 512>), grid, dim3(512), 0, s, p);
  } else if (vecs <= 2048) {
    hipLaunchKernelGGL((rms_norm_kernel<E, 2, 1024>), grid, dim3(1024), 0, s, p);
  } else {
    hipLaunchKernelGGL(rms_norm_long_kernel<E>, grid, dim3(256), 0, s, p);
  }
  return asc::check_launch("asc_rms_norm");
}

}  // namespace

extern "C" int32_t asc_reduce_f32(int32_t op, const float* x, float* out, int64_t rows, int64_t cols, int32_t dim,
                                  int64_t out_count, asc_stream_t stream) {
  ASC_REQUIRE(op >= kSum && op <= kProd, ASC_ERR_INVALID_ARG, "asc_reduce_f32: op must be 0..3, got %d", op);
  ASC_REQUIRE(dim == 0 || dim == 1 || dim == -1, ASC_ERR_INVALID_ARG,
              "asc_reduce_f32: dim must be 0, 1 or -1 (all), got %d", dim);
  ASC_REQUIRE(rows >= 0 && cols >= 0 && out_count >= 0, ASC_ERR_INVALID_ARG, "asc_reduce_f32: negative size");
  ASC_REQUIRE(cols < (int64_t{1} << 31), ASC_ERR_UNSUPPORTED, "asc_reduce_f32: cols too large");
  const int64_t results = dim == 1 ? rows : dim == 0 ? cols : out_count;
  if (results == 0) return ASC_OK;
  ASC_REQUIRE(rows > 0 && cols > 0, ASC_ERR_INVALID_ARG, "asc_reduce_f32: empty input");
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "asc_reduce_f32: null buffer");
  ReduceArgs p{x, out, rows, cols, out_count, asc::aligned16(x) && (cols % 4) == 0};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (op) {
    case kSum: return launch_reduce<kSum>(p, dim, s);
    case kMax: return launch_reduce<kMax>(p, dim, s);
    case kMin: return launch_reduce<kMin>(p, dim, s);
    default: return launch_reduce<kProd>(p, dim, s);
  }
}

extern "C" int32_t asc_rms_norm(int32_t dtype, const void* x, const float* gamma, void* out, int64_t num_rows,
                                int64_t num_cols, int32_t tile_size, float epsilon, asc_stream_t stream) {
  ASC_REQUIRE(num_rows >= 0 && num_cols >= 0, ASC_ERR_INVALID_ARG, "asc_rms_norm: negative shape");
  ASC_REQUIRE(tile_size > 0 && tile_size <= num_cols, ASC_ERR_INVALID_ARG,
              "asc_rms_norm: need 0 < tile_size <= num_cols (got %d, %lld)", tile_size, (long long)num_cols);
  ASC_REQUIRE(dtype == ASC_DT_FLOAT32 || dtype == ASC_DT_FLOAT16, ASC_ERR_UNSUPPORTED,
              "asc_rms_norm: dtype %d not supported (float32, float16)", dtype);
  if (num_rows == 0) return ASC_OK;
  ASC_REQUIRE(x && gamma && out, ASC_ERR_INVALID_ARG, "asc_rms_norm: null buffer");
  const int64_t es = dtype == ASC_DT_FLOAT32 ? 4 : 2;
  RmsArgs p{x, gamma, out, num_rows, num_cols, tile_size, epsilon,
            asc::aligned16(x) && asc::aligned16(out) && asc::aligned16(gamma) && (num_cols * es) % 16 == 0};
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == ASC_DT_FLOAT32 ? launch_rms<F32E>(p, s) : launch_rms<F16E>(p, s);
}
