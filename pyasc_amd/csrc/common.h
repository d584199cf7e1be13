// Shared helpers for the libasc_hip.so kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "asc_hip.h"

namespace asc {

// Records a formatted message as the thread's last error and returns `code`.
int32_t set_error(int32_t code, const char* fmt, ...);
// Converts the launch status of the last kernel into an ASC return code.
int32_t check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

constexpr int kWave = 64;

// Butterfly reductions across the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

}  // namespace asc

#define ASC_REQUIRE(cond, code, ...) \
  do {                               \
    if (!(cond)) return ::asc::set_error((code), __VA_ARGS__); \
  } while (0)
