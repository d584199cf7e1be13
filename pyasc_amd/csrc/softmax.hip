// Row softmax for the two asc2 softmax kernels (python/test/asc2/kernels/):
//   test_softmax.py:16-27        grid-stride rows, one [1, tile_size] tile per row
//   test_softmax_fused.py:16-24  contiguous row blocks through asc2.softmax
// The device bodies are in softmax_kernels.h.  This file holds the launch plan
// (asc_softmax_plan: which body, its grid and block, its six arguments), which
// the library's entry points and the asc2 code-object launch path share, and
// the library's own instances of the kernels.
#include "softmax_kernels.h"

namespace {

ASC_SOFTMAX_KERNELS(, softmax_)

enum Kernel : int32_t {
  kWave1x2,
  kWave2x2,
  kBlock2x128,
  kBlock2x256,
  kBlock2x512,
  kBlock8x256,
  kLong,
  kF16,
  kPaddedF32,
  kPaddedF16,
  kNumKernels
};

using KernelFn = void (*)(const void*, void*, int64_t, int64_t, int32_t, int32_t);

// The library's kernels and the code object's names for the same bodies
// (co/asc2_softmax.hip), in Kernel order.
const KernelFn kKernels[kNumKernels] = {softmax_wave_1x2,    softmax_wave_2x2,    softmax_block_2x128,
                                        softmax_block_2x256, softmax_block_2x512, softmax_block_8x256,
                                        softmax_long,        softmax_f16,         softmax_padded_f32,
                                        softmax_padded_f16};
const char* const kCodeObjectNames[kNumKernels] = {
    "asc2_softmax_wave_1x2",    "asc2_softmax_wave_2x2",    "asc2_softmax_block_2x128", "asc2_softmax_block_2x256",
    "asc2_softmax_block_2x512", "asc2_softmax_block_8x256", "asc2_softmax_long",        "asc2_softmax_f16",
    "asc2_softmax_padded_f32",  "asc2_softmax_padded_f16"};

struct Plan {
  Kernel kernel = kNumKernels;
  int64_t grid = 0;  // 0: nothing to launch
  int32_t block = 0;
  const void* x = nullptr;
  void* out = nullptr;
  int64_t rows = 0, stride = 0;
  int32_t len = 0, flag = 0;
};

// Row-resident fp32 body for rows of `len` columns.  Above 512 columns a row takes
// several waves with 2 vectors per lane (8 at 8192 columns): more, shorter waves than
// one wave per row, and each wave's loads, cross-wave reductions and stores finish
// sooner (fp32 rows, 64 MiB in and out, same box: 1024 columns 5500-5560 GB/s with
// one wave per two rows, 5950 with block_2x128, 5500 with block_1x256; 2048: 5680 with
// two waves per row, 5870-5970 with four, 5210-5360 with eight; 4096: 5560-5590 with
// two waves per row, 5690-5740 with four (4 vectors), 5890-5900 with eight
// (block_2x512), 5200-5260 with sixteen; 8192: 5650-5670 with four waves of 8
// vectors, 5580-5610 with eight, 5480-5510 with sixteen; a plain copy of the same
// bytes 5840-5850).  Up to 512 columns a wave takes two rows (measured faster at
// 1024 columns than one).
void plan_f32_rows(Plan& p) {
  const int64_t L = p.len;
  p.block = 256;
  if (L <= 512) {
    p.kernel = L <= 256 ? kWave1x2 : kWave2x2;
    p.grid = asc::ceil_div(p.rows, 8);
    return;
  }
  p.grid = p.rows;  // one block per row
  if (L <= 1024) {
    p.kernel = kBlock2x128;
    p.block = 128;
  } else if (L <= 2048) {
    p.kernel = kBlock2x256;
  } else if (L <= 4096) {
    p.kernel = kBlock2x512;
    p.block = 512;
  } else if (L <= 8192) {
    p.kernel = kBlock8x256;
  } else {
    p.kernel = kLong;
  }
}

bool vec_ok_f32(const void* x, const void* out, int64_t stride) {
  return asc::aligned16(x) && asc::aligned16(out) && (stride % 4) == 0;
}
bool vec_ok_f16(const void* x, const void* out, int64_t stride, int64_t len) {
  return asc::aligned16(x) && asc::aligned16(out) && (stride % 8) == 0 && (len % 8) == 0;
}

// The launch of asc_softmax_{rows,blocks}_{f32,f16}: `size` is tile_size (rows) or
// block_size (blocks).  Errors are reported under `who`.
int32_t make_plan(bool half, bool fused, const void* x, const void* out, int64_t num_rows, int64_t num_cols,
                  int32_t size, int32_t grid, const char* who, Plan& p) {
  ASC_REQUIRE(num_rows >= 0 && num_cols >= 0, ASC_ERR_INVALID_ARG, "%s: negative shape (%lld, %lld)", who,
              (long long)num_rows, (long long)num_cols);
  ASC_REQUIRE(size > 0 && grid > 0, ASC_ERR_INVALID_ARG, "%s: need %s > 0 and grid > 0 (got %d, %d)", who,
              fused ? "block_size" : "tile_size", size, grid);
  p = Plan{};
  p.x = x;
  p.out = const_cast<void*>(out);
  p.stride = num_cols;
  if (fused) {
    ASC_REQUIRE(num_cols <= INT32_MAX, ASC_ERR_UNSUPPORTED, "%s: num_cols too large", who);
    // rows [0, min(num_rows, grid * block_size)): block b covers [b * block_size, (b + 1) * block_size)
    const int64_t reach = static_cast<int64_t>(grid) * size;
    p.rows = reach < num_rows ? reach : num_rows;
    p.len = static_cast<int32_t>(num_cols);
  } else {
    // rows b, b + grid, ... for b < grid cover every row exactly once
    p.rows = num_rows;
    p.len = size;
    if (size > num_cols) {  // tiles wider than the row: the padded bodies
      if (p.rows == 0) return ASC_OK;
      ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "%s: null buffer", who);
      p.kernel = half ? kPaddedF16 : kPaddedF32;
      p.len = static_cast<int32_t>(num_cols);
      p.flag = size - static_cast<int32_t>(num_cols);
      p.grid = p.rows < 65536 ? p.rows : 65536;
      p.block = 256;
      return ASC_OK;
    }
  }
  if (p.rows == 0 || p.len == 0) return ASC_OK;
  ASC_REQUIRE(x && out, ASC_ERR_INVALID_ARG, "%s: null buffer", who);
  if (half) {
    p.kernel = kF16;
    p.flag = vec_ok_f16(x, out, p.stride, p.len);
    p.grid = p.rows < 65536 ? p.rows : 65536;
    p.block = 256;
  } else {
    p.flag = vec_ok_f32(x, out, p.stride);
    plan_f32_rows(p);
  }
  // hipLaunchKernel takes the grid in threads as a 32-bit count
  ASC_REQUIRE(p.grid * p.block <= static_cast<int64_t>(UINT32_MAX), ASC_ERR_UNSUPPORTED,
              "%s: %lld rows exceed one launch", who, (long long)p.rows);
  return ASC_OK;
}

int32_t launch(const Plan& p, asc_stream_t stream, const char* who) {
  if (p.grid == 0) return ASC_OK;
  hipLaunchKernelGGL(kKernels[p.kernel], dim3(static_cast<uint32_t>(p.grid)), dim3(p.block), 0,
                     static_cast<hipStream_t>(stream), p.x, p.out, p.rows, p.stride, p.len, p.flag);
  return asc::check_launch(who);
}

int32_t plan_and_launch(bool half, bool fused, const void* x, void* out, int64_t num_rows, int64_t num_cols,
                        int32_t size, int32_t grid, asc_stream_t stream, const char* who) {
  Plan p;
  const int32_t rc = make_plan(half, fused, x, out, num_rows, num_cols, size, grid, who, p);
  return rc != ASC_OK ? rc : launch(p, stream, who);
}

}  // namespace

extern "C" int32_t asc_softmax_rows_f32(const float* x, float* out, int64_t num_rows, int64_t num_cols,
                                        int32_t tile_size, int32_t grid, asc_stream_t stream) {
  return plan_and_launch(false, false, x, out, num_rows, num_cols, tile_size, grid, stream, "asc_softmax_rows_f32");
}

extern "C" int32_t asc_softmax_blocks_f32(const float* x, float* out, int64_t num_rows, int64_t num_cols,
                                          int32_t block_size, int32_t grid, asc_stream_t stream) {
  return plan_and_launch(false, true, x, out, num_rows, num_cols, block_size, grid, stream,
                         "asc_softmax_blocks_f32");
}

extern "C" int32_t asc_softmax_rows_f16(const void* x, void* out, int64_t num_rows, int64_t num_cols,
                                        int32_t tile_size, int32_t grid, asc_stream_t stream) {
  return plan_and_launch(true, false, x, out, num_rows, num_cols, tile_size, grid, stream, "asc_softmax_rows_f16");
}

extern "C" int32_t asc_softmax_blocks_f16(const void* x, void* out, int64_t num_rows, int64_t num_cols,
                                          int32_t block_size, int32_t grid, asc_stream_t stream) {
  return plan_and_launch(true, true, x, out, num_rows, num_cols, block_size, grid, stream,
                         "asc_softmax_blocks_f16");
}

extern "C" int32_t asc_softmax_plan(int32_t dtype, int32_t fused, const void* x, const void* out, int64_t num_rows,
                                    int64_t num_cols, int32_t size, int32_t grid, asc_softmax_plan_t* plan) {
  ASC_REQUIRE(plan, ASC_ERR_INVALID_ARG, "asc_softmax_plan: null plan");
  ASC_REQUIRE(dtype == ASC_DT_FLOAT32 || dtype == ASC_DT_FLOAT16, ASC_ERR_UNSUPPORTED,
              "asc_softmax_plan: unsupported dtype code %d", dtype);
  const bool half = dtype == ASC_DT_FLOAT16;
  const char* who = fused ? (half ? "asc_softmax_blocks_f16" : "asc_softmax_blocks_f32")
                          : (half ? "asc_softmax_rows_f16" : "asc_softmax_rows_f32");
  Plan p;
  const int32_t rc = make_plan(half, fused != 0, x, out, num_rows, num_cols, size, grid, who, p);
  if (rc != ASC_OK) return rc;
  *plan = asc_softmax_plan_t{};
  if (p.grid == 0) return ASC_OK;
  __builtin_strncpy(plan->kernel, kCodeObjectNames[p.kernel], sizeof(plan->kernel) - 1);
  plan->grid = static_cast<uint32_t>(p.grid);
  plan->block = static_cast<uint32_t>(p.block);
  plan->rows = p.rows;
  plan->stride = p.stride;
  plan->len = p.len;
  plan->flag = p.flag;
  return ASC_OK;
}
