// int8 GEMM with exact int32 accumulation and the per-output-channel fp16
// dequant of the reference's DEQF16 fixpipe mode: the device code, shared by the
// library (matmul_i8.hip, launched through asc_matmul_i8_*) and the standalone
// gfx950 code object (co/asc2_matmul_i8.hip, loaded with hipModuleLoad by the
// asc2 launch path)
// (python/test/generalization/adv/test_matmul_quant.py:23-51,94-106;
//  lib/Conversion/LowerToAsc/LowerAscTileDataTransfer.cpp:116-117).
//
// Same structure as the fp16/bf16 kernel on v_mfma_i32_32x32x32_i8: 256x256
// output tile; tile-aligned shapes take the direct-to-LDS loop of
// gemm_direct.h (8 waves of 128x64, 64-byte k-tiles, B read with
// ds_read_b64_tr_b8), others the register-staged loop of gemm_core.h (4 waves
// of 128x128, B transposed in registers as 16(k) x 8(n) byte blocks).  The epilogue either stores the int32
// accumulators or out = fp16_rne(fp32_rne(acc) * s[n]) with s[n] the fp32
// scale (optionally with its low 13 mantissa bits cleared, the reference
// golden's trunc-19 form).
#pragma once

#include "common.h"
#include "gemm_common.h"
#include "gemm_core.h"
#include "gemm_direct.h"
#include "numeric.h"

namespace asc {
namespace i8 {

using asc::gemm::u32x2;
using asc::gemm::u32x4;
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = asc::gemm::kTileM;
constexpr int BN = asc::gemm::kTileN;
constexpr int BK = 128;  // int8 elements per LDS row = 128 bytes
constexpr int kThreads = asc::gemm::kGemmThreads;
constexpr int kStageBytes = asc::gemm::kStageBytes;

struct I8Args {
  const int8_t* a;
  const int8_t* b;
  const float* scale;
  void* c;
  int M, N, K;
  int trunc19;
  int tiles_m, tiles_n;
};

template <bool kChecked>
__device__ __forceinline__ u32x4 load16(const int8_t* base, int64_t ld, int row, int col, int rows, int cols,
                                        bool vec_ok) {
  const int8_t* p = base + row * ld + col;
  if (!kChecked) return *reinterpret_cast<const u32x4*>(p);
  if (row < rows && vec_ok && col + 15 < cols) return *reinterpret_cast<const u32x4*>(p);
  uint8_t e[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) e[i] = (row < rows && col + i < cols) ? static_cast<uint8_t>(p[i]) : uint8_t(0);
  u32x4 v;
  __builtin_memcpy(&v, e, 16);
  return v;
}

template <bool kChecked>
__device__ __forceinline__ u32x2 load8(const int8_t* base, int64_t ld, int row, int col, int rows, int cols,
                                       bool vec_ok) {
  const int8_t* p = base + row * ld + col;
  if (!kChecked) return *reinterpret_cast<const u32x2*>(p);
  if (row < rows && vec_ok && col + 7 < cols) return *reinterpret_cast<const u32x2*>(p);
  uint8_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = (row < rows && col + i < cols) ? static_cast<uint8_t>(p[i]) : uint8_t(0);
  u32x2 v;
  __builtin_memcpy(&v, e, 8);
  return v;
}

struct TrI8 {
  using Elem = int8_t;
  using Acc = i32x16;
  using BReg = u32x2;
  static constexpr int kBK = BK;
  static constexpr int kBRows = 16;
  template <bool kChecked>
  __device__ __forceinline__ static u32x4 load_a(const int8_t* base, int64_t ld, int row, int col, int rows, int cols,
                                                 bool vec_ok) {
    return load16<kChecked>(base, ld, row, col, rows, cols, vec_ok);
  }
  template <bool kChecked>
  __device__ __forceinline__ static u32x2 load_b(const int8_t* base, int64_t ld, int row, int col, int rows, int cols,
                                                 bool vec_ok) {
    return load8<kChecked>(base, ld, row, col, rows, cols, vec_ok);
  }
  __device__ __forceinline__ static void transpose_b(const u32x2 (&in)[16], u32x4 (&out)[8]) {
    asc::gemm::transpose16x8_b8(in, out);
  }
  __device__ __forceinline__ static i32x16 mfma(u32x4 a, u32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                                 0);
  }
};

// Waves across the 256 columns of the fast path's tile: 2 (one wave per SIMD,
// 128x128 accumulators each) or 4 (two waves per SIMD, 128x64 each).
constexpr int kFastWavesN = 4;
using FastLoop = asc::gemm::GemmDirectLoop<TrI8, kFastWavesN>;
constexpr int kFastThreads = FastLoop::kThreads;

// fp32 scale of column n (optionally with its low 13 mantissa bits cleared)
__device__ __forceinline__ float load_scale(const I8Args& p, int n) {
  float s = p.scale[n];
  if (p.trunc19) s = __uint_as_float(__float_as_uint(s) & 0xFFFFE000u);
  return s;
}

// kMode: 0 = int32 accumulators, 1 = fp16 dequant
// The output tile of one workgroup (tile index = block index).
template <bool kChecked, int kMode>
__device__ __forceinline__ void gemm_i8_body(const I8Args& p) {
  int tm, tn;
  asc::gemm::tile_coords(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, asc::gemm::kGroupM, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63;
  if constexpr (!kChecked) {
    // the LDS stages as distinct objects (see gemm_direct.h)
    __shared__ __attribute__((aligned(16))) uint8_t lds0[asc::gemm::kDirectStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds1[asc::gemm::kDirectStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds2[asc::gemm::kDirectStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds3[asc::gemm::kDirectStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds4[asc::gemm::kDirectStageBytes];
    static_assert(asc::gemm::kDirectStages == 5, "one __shared__ stage object per ring stage");
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);  // wave-uniform (SGPR)
    FastLoop L;
    L.a = p.a;
    L.b = p.b;
    L.m0 = m0;
    L.n0 = n0;
    L.lane = lane;
    L.wave = wave;
    L.wm = wave / kFastWavesN;
    L.wn = wave % kFastWavesN;
    L.lds[0] = lds0;
    L.lds[1] = lds1;
    L.lds[2] = lds2;
    L.lds[3] = lds3;
    L.lds[4] = lds4;
    L.init(p.K, p.N);
    i32x16 acc[4][FastLoop::kJ];
    L.run(p.K, acc);
    // Epilogue: the whole tile is in bounds and C's rows are 16-byte aligned, so the
    // results leave through quad-transposed wide stores.
    const int n_base = n0 + L.wn * 32 * FastLoop::kJ;
    float scale_n[FastLoop::kJ];
#pragma unroll
    for (int j = 0; j < FastLoop::kJ; ++j) scale_n[j] = kMode == 1 ? load_scale(p, n_base + j * 32 + (lane & 31)) : 0.f;
    const auto conv = [&](int j, int32_t x) -> uint32_t {
      if constexpr (kMode == 0) return static_cast<uint32_t>(x);
      else return asc::f32_to_f16_rne(asc::materialize(static_cast<float>(x) * scale_n[j]));
    };
    asc::gemm::store_wave_tile<kMode == 0 ? 4 : 2, FastLoop::kJ>(acc, conv, p.c, p.N, m0 + L.wm * 128, n_base, lane);
  } else {
    const int wm = (threadIdx.x >> 6) >> 1, wn = (threadIdx.x >> 6) & 1;
    i32x16 acc[4][4];
    __shared__ __attribute__((aligned(16))) uint8_t lds0[asc::gemm::kStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds1[asc::gemm::kStageBytes];
    asc::gemm::GemmMainLoop<TrI8, true> L;
    L.a = p.a;
    L.b = p.b;
    L.s = asc::gemm::GemmShape{p.M, p.N, p.K, p.K, p.N, p.tiles_m, p.tiles_n};
    L.m0 = m0;
    L.n0 = n0;
    L.tid = threadIdx.x;
    L.lane = lane;
    L.wm = wm;
    L.wn = wn;
    L.a_vec = ((reinterpret_cast<uintptr_t>(p.a) | static_cast<uintptr_t>(p.K)) & 15) == 0;
    L.b_vec = ((reinterpret_cast<uintptr_t>(p.b) | static_cast<uintptr_t>(p.N)) & 7) == 0;
    L.lds[0] = lds0;
    L.lds[1] = lds1;
    L.run(acc);
    // Epilogue: lane holds column lane%32 of each 32x32 block, register r row
    // 8*(r/4) + 4*(lane/32) + r%4.
    const int col_in = lane & 31;
    const int row_q = (lane >> 5) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 128 + j * 32 + col_in;
      const float s = (kMode == 1 && n < p.N) ? load_scale(p, n) : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * 128 + i * 32 + (r >> 2) * 8 + row_q + (r & 3);
          if (m >= p.M || n >= p.N) continue;
          const int64_t off = static_cast<int64_t>(m) * p.N + n;
          if constexpr (kMode == 0) {
            static_cast<int32_t*>(p.c)[off] = acc[i][j][r];
          } else {
            const float v = asc::materialize(static_cast<float>(acc[i][j][r]) * s);
            static_cast<uint16_t*>(p.c)[off] = asc::f32_to_f16_rne(v);
          }
        }
      }
    }
  }
}

}  // namespace i8
}  // namespace asc

// Defines the int8 kernels as PREFIX##{fast,checked}_{i32,f16} (the direct-to-LDS
// loop for tile-aligned shapes, or the bounds-checked one; int32 accumulators or the
// fp16 dequant), each taking one asc::i8::I8Args by value.
#define ASC_I8_KERNEL(LINKAGE, NAME, CHECKED, MODE)                                                                \
  LINKAGE __global__ void __launch_bounds__(CHECKED ? asc::i8::kThreads : asc::i8::kFastThreads, 1)               \
      NAME(asc::i8::I8Args p) {                                                                                    \
    asc::i8::gemm_i8_body<CHECKED, MODE>(p);                                                                       \
  }
#define ASC_I8_KERNELS(LINKAGE, PREFIX)                 \
  ASC_I8_KERNEL(LINKAGE, PREFIX##fast_i32, false, 0)    \
  ASC_I8_KERNEL(LINKAGE, PREFIX##fast_f16, false, 1)    \
  ASC_I8_KERNEL(LINKAGE, PREFIX##checked_i32, true, 0)  \
  ASC_I8_KERNEL(LINKAGE, PREFIX##checked_f16, true, 1)
