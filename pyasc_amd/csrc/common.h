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

// Cross-lane helpers for one wavefront.  Lane l^1 and l^2 come from DPP quad
// permutations, l^(7-i) / l^(15-i) patterns from the row (half-)mirrors, l^16
// and l^32 from the gfx950 permlane swaps (each swap returns the partner's
// value in one result and the lane's own in the other; the lane half picks).
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}
__device__ __forceinline__ float lane_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// Reductions across the 64 lanes of a wavefront.  Every step combines a lane
// with a partner holding the same partial result over the complementary lane
// set, so all lanes end with the bit-identical total (IEEE add and max are
// commutative).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_mov<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_mov<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_mov<kDppRowMirror>(v));
  v = fmaxf(v, lane_xor16(v));
  return fmaxf(v, lane_xor32(v));
}

__device__ __forceinline__ float wave_min(float v) {
  v = fminf(v, dpp_mov<kDppQuadXor1>(v));
  v = fminf(v, dpp_mov<kDppQuadXor2>(v));
  v = fminf(v, dpp_mov<kDppRowHalfMirror>(v));
  v = fminf(v, dpp_mov<kDppRowMirror>(v));
  v = fminf(v, lane_xor16(v));
  return fminf(v, lane_xor32(v));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<kDppQuadXor1>(v);
  v += dpp_mov<kDppQuadXor2>(v);
  v += dpp_mov<kDppRowHalfMirror>(v);
  v += dpp_mov<kDppRowMirror>(v);
  v += lane_xor16(v);
  return v + lane_xor32(v);
}

}  // namespace asc

#define ASC_REQUIRE(cond, code, ...) \
  do {                               \
    if (!(cond)) return ::asc::set_error((code), __VA_ARGS__); \
  } while (0)
