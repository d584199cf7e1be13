// Elementwise vadd for asc2 vadd_kernel (python/test/asc2/kernels/test_vadd.py:16-28),
// launched through asc_vadd; the device bodies are in vadd_kernels.h.
#include "vadd_kernels.h"

namespace {

using asc::vadd::AddBF16;
using asc::vadd::AddF16;
using asc::vadd::AddF32;
using asc::vadd::AddI32;
using asc::vadd::kThreads;
using asc::vadd::kUnroll;
using asc::vadd::u32x4;

template <typename Op>
__global__ void __launch_bounds__(kThreads) vadd_vec_kernel(const u32x4* __restrict__ x, const u32x4* __restrict__ y,
                                                            u32x4* __restrict__ out, int64_t n_vec) {
  asc::vadd::vec_body<Op>(x, y, out, n_vec);
}

template <typename Op>
__global__ void __launch_bounds__(kThreads) vadd_scalar_kernel(const typename Op::T* __restrict__ x,
                                                               const typename Op::T* __restrict__ y,
                                                               typename Op::T* __restrict__ out, int64_t begin,
                                                               int64_t end) {
  asc::vadd::scalar_body<Op>(x, y, out, begin, end);
}

template <typename Op>
int32_t launch(const void* xv, const void* yv, void* outv, int64_t covered, hipStream_t stream) {
  using T = typename Op::T;
  const T* x = static_cast<const T*>(xv);
  const T* y = static_cast<const T*>(yv);
  T* out = static_cast<T*>(outv);
  constexpr int64_t kPerVec = 16 / sizeof(T);
  int64_t done = 0;
  if (asc::aligned16(x) && asc::aligned16(y) && asc::aligned16(out)) {
    const int64_t n_vec = covered / kPerVec;
    if (n_vec > 0) {
      hipLaunchKernelGGL(vadd_vec_kernel<Op>, dim3(static_cast<uint32_t>(asc::vadd::vec_blocks(n_vec))),
                         dim3(kThreads), 0, stream, reinterpret_cast<const u32x4*>(x),
                         reinterpret_cast<const u32x4*>(y), reinterpret_cast<u32x4*>(out), n_vec);
      int32_t rc = asc::check_launch("asc_vadd");
      if (rc != ASC_OK) return rc;
    }
    done = n_vec * kPerVec;
  }
  if (done < covered) {
    hipLaunchKernelGGL(vadd_scalar_kernel<Op>, dim3(static_cast<uint32_t>(asc::vadd::scalar_blocks(covered - done))),
                       dim3(kThreads), 0, stream, x, y, out, done, covered);
    return asc::check_launch("asc_vadd");
  }
  return ASC_OK;
}

// dst[v] = src[v] for 16-byte vectors v < n_vec: the same streaming shape as
// vadd_vec_kernel (4 non-temporal vectors per thread in flight) with one operand,
// the bandwidth reference the streaming kernels are compared with.
__global__ void __launch_bounds__(kThreads) copy_vec_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                            int64_t n_vec) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
  if (base + (kUnroll - 1) * kThreads < n_vec) {
    u32x4 a[kUnroll];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) a[j] = __builtin_nontemporal_load(src + base + j * kThreads);
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) __builtin_nontemporal_store(a[j], dst + base + j * kThreads);
  } else {
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int64_t v = base + j * kThreads;
      if (v < n_vec) dst[v] = src[v];
    }
  }
}

}  // namespace

extern "C" int32_t asc_copy_bytes(const void* src, void* dst, int64_t n_bytes, asc_stream_t stream) {
  ASC_REQUIRE(n_bytes >= 0, ASC_ERR_INVALID_ARG, "asc_copy_bytes: negative size");
  if (n_bytes == 0) return ASC_OK;
  ASC_REQUIRE(src && dst, ASC_ERR_INVALID_ARG, "asc_copy_bytes: null buffer");
  ASC_REQUIRE(asc::aligned16(src) && asc::aligned16(dst) && n_bytes % 16 == 0, ASC_ERR_ALIGNMENT,
              "asc_copy_bytes: buffers and size must be multiples of 16 bytes");
  const int64_t n_vec = n_bytes / 16;
  const int64_t blocks = asc::ceil_div(n_vec, kThreads * kUnroll);
  ASC_REQUIRE(blocks <= (int64_t{1} << 31) - 1, ASC_ERR_UNSUPPORTED, "asc_copy_bytes: size too large");
  hipLaunchKernelGGL(copy_vec_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src), static_cast<u32x4*>(dst),
                     n_vec);
  return asc::check_launch("asc_copy_bytes");
}

extern "C" int32_t asc_vadd(int32_t dtype, const void* x, const void* y, void* out, int64_t size, int32_t tile_size,
                            int32_t tile_per_block, int32_t grid, asc_stream_t stream) {
  ASC_REQUIRE(size >= 0, ASC_ERR_INVALID_ARG, "asc_vadd: size must be >= 0, got %lld", (long long)size);
  ASC_REQUIRE(tile_size > 0 && tile_per_block >= 0 && grid > 0, ASC_ERR_INVALID_ARG,
              "asc_vadd: need tile_size > 0, tile_per_block >= 0, grid > 0 (got %d, %d, %d)", tile_size,
              tile_per_block, grid);
  // Coverage of the reference kernel body: grid*tpb tiles of tile_size, clipped at size.
  const int64_t reach = static_cast<int64_t>(grid) * tile_per_block * tile_size;
  const int64_t covered = reach < size ? reach : size;
  if (covered == 0) return ASC_OK;
  ASC_REQUIRE(x && y && out, ASC_ERR_INVALID_ARG, "asc_vadd: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case ASC_DT_FLOAT32: return launch<AddF32>(x, y, out, covered, s);
    case ASC_DT_INT32: return launch<AddI32>(x, y, out, covered, s);
    case ASC_DT_FLOAT16: return launch<AddF16>(x, y, out, covered, s);
    case ASC_DT_BFLOAT16: return launch<AddBF16>(x, y, out, covered, s);
    default: return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_vadd: unsupported dtype code %d", dtype);
  }
}
