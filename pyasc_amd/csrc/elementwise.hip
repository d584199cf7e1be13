// Elementwise asc2 kernels beside vadd (leaky_relu, vmuladd, gelu): the host
// side of the library -- argument checks, coverage and launch geometry -- over
// the device bodies of elementwise_kernels.h.
//   leaky_relu_kernel  python/test/asc2/kernels/test_leaky_relu.py:16-26
//   vmuladd_kernel     python/test/asc2/kernels/test_vmuladd.py:16-31
//   gelu_kernel        python/test/asc2/kernels/test_gelu.py:19-33
// Compiled with -ffp-contract=off: no multiply-add is fused.
#include "elementwise_kernels.h"

namespace {

using asc::elementwise::kThreads;
using asc::elementwise::kUnroll;
using asc::elementwise::u32x4;

ASC_ELEMENTWISE_KERNELS(, ew_)

// Streams [0, covered) through a vector kernel (16-byte vectors, when every buffer is
// 16-byte aligned) and an element kernel (the rest).  launch_vec(grid, n_vec) and
// launch_elem(grid, begin, end) issue the two kernels.
template <class T, class VecLaunch, class ElemLaunch>
int32_t stream(bool aligned, int64_t covered, VecLaunch launch_vec, ElemLaunch launch_elem, const char* who) {
  constexpr int64_t kPerVec = 16 / sizeof(T);
  int64_t done = 0;
  if (aligned) {
    const int64_t n_vec = covered / kPerVec;
    if (n_vec > 0) {
      launch_vec(dim3(static_cast<uint32_t>(asc::ceil_div(n_vec, kThreads * kUnroll))), n_vec);
      const int32_t rc = asc::check_launch(who);
      if (rc != ASC_OK) return rc;
    }
    done = n_vec * kPerVec;
  }
  if (done < covered) {
    const int64_t blocks = asc::ceil_div(covered - done, kThreads);
    const int64_t grid = blocks < asc::elementwise::kScalarMaxBlocks ? blocks : asc::elementwise::kScalarMaxBlocks;
    launch_elem(dim3(static_cast<uint32_t>(grid)), done, covered);
    return asc::check_launch(who);
  }
  return ASC_OK;
}

template <class T>
int32_t leaky_relu(void (*vec)(const u32x4*, u32x4*, int64_t, float),
                   void (*elem)(const T*, T*, int64_t, int64_t, float), const void* x, float alpha, void* out,
                   int64_t covered, hipStream_t s) {
  const bool aligned = asc::aligned16(x) && asc::aligned16(out);
  return stream<T>(
      aligned, covered,
      [&](dim3 grid, int64_t n_vec) {
        hipLaunchKernelGGL(vec, grid, dim3(kThreads), 0, s, static_cast<const u32x4*>(x), static_cast<u32x4*>(out),
                           n_vec, alpha);
      },
      [&](dim3 grid, int64_t begin, int64_t end) {
        hipLaunchKernelGGL(elem, grid, dim3(kThreads), 0, s, static_cast<const T*>(x), static_cast<T*>(out), begin,
                           end, alpha);
      },
      "asc_leaky_relu");
}

template <class T>
int32_t muladd(void (*vec)(const u32x4*, const u32x4*, const u32x4*, u32x4*, int64_t),
               void (*elem)(const T*, const T*, const T*, T*, int64_t, int64_t), const void* x, const void* y,
               const void* z, void* out, int64_t covered, hipStream_t s) {
  const bool aligned = asc::aligned16(x) && asc::aligned16(y) && asc::aligned16(z) && asc::aligned16(out);
  return stream<T>(
      aligned, covered,
      [&](dim3 grid, int64_t n_vec) {
        hipLaunchKernelGGL(vec, grid, dim3(kThreads), 0, s, static_cast<const u32x4*>(x),
                           static_cast<const u32x4*>(y), static_cast<const u32x4*>(z), static_cast<u32x4*>(out),
                           n_vec);
      },
      [&](dim3 grid, int64_t begin, int64_t end) {
        hipLaunchKernelGGL(elem, grid, dim3(kThreads), 0, s, static_cast<const T*>(x), static_cast<const T*>(y),
                           static_cast<const T*>(z), static_cast<T*>(out), begin, end);
      },
      "asc_vmuladd");
}

// Coverage of the reference's tiled elementwise kernel bodies.
int64_t covered_elements(int64_t size, int32_t tile_size, int32_t tile_per_block, int32_t grid) {
  const int64_t reach = static_cast<int64_t>(grid) * tile_per_block * tile_size;
  return reach < size ? reach : size;
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
    case ASC_DT_FLOAT32:
      return leaky_relu<float>(ew_leaky_relu_vec_f32, ew_leaky_relu_elem_f32, x, alpha, out, covered, s);
    case ASC_DT_FLOAT16:
      return leaky_relu<uint16_t>(ew_leaky_relu_vec_f16, ew_leaky_relu_elem_f16, x, alpha, out, covered, s);
    case ASC_DT_BFLOAT16:
      return leaky_relu<uint16_t>(ew_leaky_relu_vec_bf16, ew_leaky_relu_elem_bf16, x, alpha, out, covered, s);
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
    case ASC_DT_FLOAT32: return muladd<float>(ew_vmuladd_vec_f32, ew_vmuladd_elem_f32, x, y, z, out, covered, s);
    case ASC_DT_FLOAT16: return muladd<uint16_t>(ew_vmuladd_vec_f16, ew_vmuladd_elem_f16, x, y, z, out, covered, s);
    case ASC_DT_BFLOAT16:
      return muladd<uint16_t>(ew_vmuladd_vec_bf16, ew_vmuladd_elem_bf16, x, y, z, out, covered, s);
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
  const int32_t vec_ok = asc::aligned16(x) && asc::aligned16(out) && (num_cols % 4) == 0;
  // Rows b, b+grid, ... for b < grid cover every row exactly once; the physical
  // grid is the library's (rows are independent).
  const int64_t max_blocks = asc::elementwise::kGeluMaxBlocks;
  const int64_t blocks = num_rows < max_blocks ? num_rows : max_blocks;
  hipLaunchKernelGGL(ew_gelu_rows_f32, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), x, out, num_rows, num_cols, tile_size, approximate ? 1 : 0,
                     vec_ok);
  return asc::check_launch("asc_gelu_rows_f32");
}
