// Dense matmul C = epilogue(A . B) for the asc2 cube path: the device code, shared
// by the library (matmul.hip, launched through asc_matmul / asc_matmul_bias_act) and
// the standalone gfx950 code object (co/asc2_matmul.hip, loaded with hipModuleLoad
// by the asc2 launch path)
// (python/asc/language/tile/binary_ops.py:180-221; kernels in
// python/test/asc2/kernels/test_matmul_{mnblock,tiled,fixpipe,l0c_to_l1}.py).
//
// fp16/bf16 inputs run on MFMA (v_mfma_f32_32x32x16_{bf16,f16}) with fp32
// accumulation and a 256x256 output tile per workgroup:
//   - tile-aligned shapes (M, N multiples of 256, K of 32, offsets within
//     32 bits): the direct-to-LDS loop of gemm_direct.h with 8 waves in 2x4,
//     each 128x64 = 4x2 MFMA blocks, two waves per SIMD -- operands go from HBM
//     straight into five 32 KiB LDS stages, B stays row-major and its
//     K-contiguous MFMA operand comes from LDS transpose reads;
//   - other shapes: the register-staged loop of gemm_core.h (4 waves in 2x2,
//     each 128x128) with bounds-checked loads (zero fill), B transposed in
//     registers, masked stores;
//   - XCD-aware, grouped tile order (gemm_common.h).
// The epilogue applies the fixpipe relu and the RNE cast to fp16/bf16, or
// stores fp32 as is.
//
// fp32 inputs (test_matmul_fixpipe.py's float32 case; the asc1 kernels of
// python/test/kernels/test_matmul.py, test_matmul_torch.py) run on
// v_mfma_f32_16x16x4_f32 up to 2048x2048 outputs, and on a plain LDS-tiled FMA
// kernel beyond that.
#pragma once

#include "common.h"
#include "gemm_common.h"
#include "gemm_core.h"
#include "gemm_direct.h"
#include "numeric.h"

namespace asc {
namespace mm {

using asc::gemm::u32x4;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = asc::gemm::kTileM;
constexpr int BN = asc::gemm::kTileN;
constexpr int BK = 64;  // 16-bit elements per LDS row = 128 bytes
constexpr int kThreads = asc::gemm::kGemmThreads;
constexpr int kStageBytes = asc::gemm::kStageBytes;

enum OutKind { kOutF32 = 0, kOutF16 = 1, kOutBF16 = 2 };

// Epilogue on the fp32 accumulator, before the output cast: optional
// per-column bias (fp32 add), then an activation -- 0 none, 1 relu (fixpipe
// relu), 2 leaky relu v >= 0 ? v : v * alpha.
struct Epilogue {
  const float* bias;  // [N] or null
  int act;
  float alpha;
  __device__ __forceinline__ float operator()(float v, float bias_n) const {
    if (bias != nullptr) v += bias_n;
    if (act == 1) {
      v = fmaxf(v, 0.0f);
    } else if (act == 2) {
      v = v >= 0.0f ? v : v * alpha;
    }
    return v;
  }
  __device__ __forceinline__ float bias_at(int n) const { return bias != nullptr ? bias[n] : 0.0f; }
};

// The arguments of every matmul kernel (fp32 kernels read a and b as float).
struct GemmArgs {
  const void* a;
  const void* b;
  void* c;
  int M, N, K;
  int64_t lda, ldb, ldc;
  Epilogue epi;
  int tiles_m, tiles_n;
};

// 8 consecutive 16-bit elements of row `row`, columns col..col+7 of a row-major
// [rows x cols] matrix; out-of-range elements read as 0.
template <bool kChecked>
__device__ __forceinline__ u32x4 load_chunk(const uint16_t* base, int64_t ld, int row, int col, int rows, int cols,
                                            bool vec_ok) {
  const uint16_t* p = base + row * ld + col;
  if (!kChecked) return *reinterpret_cast<const u32x4*>(p);
  if (row < rows && vec_ok && col + 7 < cols) return *reinterpret_cast<const u32x4*>(p);
  uint16_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = (row < rows && col + i < cols) ? p[i] : uint16_t(0);
  u32x4 v;
  __builtin_memcpy(&v, e, 16);
  return v;
}

template <bool kBf16>
struct Tr16 {
  using Elem = uint16_t;
  using Acc = f32x16;
  using BReg = u32x4;
  static constexpr int kBK = BK;
  static constexpr int kBRows = 8;
  template <bool kChecked>
  __device__ __forceinline__ static u32x4 load_a(const uint16_t* base, int64_t ld, int row, int col, int rows,
                                                 int cols, bool vec_ok) {
    return load_chunk<kChecked>(base, ld, row, col, rows, cols, vec_ok);
  }
  template <bool kChecked>
  __device__ __forceinline__ static u32x4 load_b(const uint16_t* base, int64_t ld, int row, int col, int rows,
                                                 int cols, bool vec_ok) {
    return load_chunk<kChecked>(base, ld, row, col, rows, cols, vec_ok);
  }
  __device__ __forceinline__ static void transpose_b(const u32x4 (&in)[8], u32x4 (&out)[8]) {
    asc::gemm::transpose8x8_b16(in, out);
  }
  __device__ __forceinline__ static f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (kBf16) {
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                     c, 0, 0, 0);
    } else {
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                    0, 0, 0);
    }
  }
};

// Waves across the 256 columns of the fast path's tile: 2 (one wave per SIMD,
// 128x128 accumulators each) or 4 (two waves per SIMD, 128x64 each).
constexpr int kFastWavesN = 4;
using FastLoopBf16 = asc::gemm::GemmDirectLoop<Tr16<true>, kFastWavesN>;
constexpr int kFastThreads = FastLoopBf16::kThreads;

// The output tile of one workgroup (tile index = block index): fp16 / bf16 inputs.
template <bool kBf16, bool kChecked, int kOut>
__device__ __forceinline__ void gemm_mfma_body(const GemmArgs& p) {
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
    using Loop = asc::gemm::GemmDirectLoop<Tr16<kBf16>, kFastWavesN>;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);  // wave-uniform (SGPR)
    Loop L;
    L.a = static_cast<const uint16_t*>(p.a);
    L.b = static_cast<const uint16_t*>(p.b);
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
    L.init(p.lda, p.ldb);
    f32x16 acc[4][Loop::kJ];
    L.run(p.K, acc);
    // Epilogue: the whole tile is in bounds and C's rows are 16-byte aligned, so the
    // results leave through quad-transposed wide stores.
    const int n_base = n0 + L.wn * 32 * Loop::kJ;
    float bias_n[Loop::kJ];
#pragma unroll
    for (int j = 0; j < Loop::kJ; ++j) bias_n[j] = p.epi.bias_at(n_base + j * 32 + (lane & 31));
    const auto conv = [&](int j, float x) -> uint32_t {
      const float v = p.epi(x, bias_n[j]);
      if constexpr (kOut == kOutF32) return __float_as_uint(v);
      else if constexpr (kOut == kOutF16) return asc::f32_to_f16_rne(v);
      else return asc::f32_to_bf16_rne(v);
    };
    asc::gemm::store_wave_tile<kOut == kOutF32 ? 4 : 2, Loop::kJ>(acc, conv, p.c, p.ldc, m0 + L.wm * 128, n_base,
                                                                   lane);
  } else {
    const int wm = (threadIdx.x >> 6) >> 1, wn = (threadIdx.x >> 6) & 1;
    f32x16 acc[4][4];
    __shared__ __attribute__((aligned(16))) uint8_t lds0[asc::gemm::kStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds1[asc::gemm::kStageBytes];
    asc::gemm::GemmMainLoop<Tr16<kBf16>, true> L;
    L.a = static_cast<const uint16_t*>(p.a);
    L.b = static_cast<const uint16_t*>(p.b);
    L.s = asc::gemm::GemmShape{p.M, p.N, p.K, p.lda, p.ldb, p.tiles_m, p.tiles_n};
    L.m0 = m0;
    L.n0 = n0;
    L.tid = threadIdx.x;
    L.lane = lane;
    L.wm = wm;
    L.wn = wn;
    // vector loads need 16-byte aligned chunks
    L.a_vec = ((reinterpret_cast<uintptr_t>(p.a) | (p.lda * 2)) & 15) == 0;
    L.b_vec = ((reinterpret_cast<uintptr_t>(p.b) | (p.ldb * 2)) & 15) == 0;
    L.lds[0] = lds0;
    L.lds[1] = lds1;
    L.run(acc);
    // Epilogue.  MFMA 32x32 result layout: lane holds column lane%32 of the block,
    // register r holds row 8*(r/4) + 4*(lane/32) + r%4.
    const int col_in = lane & 31;
    const int row_q = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 128 + j * 32 + col_in;
        const float bias_n = n < p.N ? p.epi.bias_at(n) : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * 128 + i * 32 + (r >> 2) * 8 + row_q + (r & 3);
          if (m >= p.M || n >= p.N) continue;
          const float v = p.epi(acc[i][j][r], bias_n);
          const int64_t off = static_cast<int64_t>(m) * p.ldc + n;
          if constexpr (kOut == kOutF32) {
            static_cast<float*>(p.c)[off] = v;
          } else if constexpr (kOut == kOutF16) {
            static_cast<uint16_t*>(p.c)[off] = asc::f32_to_f16_rne(v);
          } else {
            static_cast<uint16_t*>(p.c)[off] = asc::f32_to_bf16_rne(v);
          }
        }
      }
    }
  }
}

// ---- fp32 inputs, small outputs: v_mfma_f32_16x16x4_f32.  A 256-thread workgroup
// owns one 16x16 output block and splits K over its four waves: wave w takes the
// 16-value k-groups w, w+4, ...; the four partial blocks meet in LDS and wave 0 sums
// them in wave order, then runs the epilogue.  Operands come from global memory (L2)
// straight into registers.  Lane l holds row l%16 of A and column l%16 of B; in
// k-group g, MFMA step j uses k = 16g + 4*(l/16) + j in both operands, so the four
// steps of a group cover its 16 values once (the order of k within a sum is free).
// D layout: lane l holds rows 4*(l/16) + r (r = 0..3) of column l%16.
// Out-of-range rows, columns and k read a clamped in-bounds address and use 0.
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kF32MfmaMaxBlocks = 16384;  // 16x16 output blocks: up to 2048 x 2048 outputs

// Block b covers output block (b / ceil(N/16), b % ceil(N/16)).
template <int kOut>
__device__ __forceinline__ void gemm_f32_mfma_body(const GemmArgs& p) {
  const float* __restrict__ a = static_cast<const float*>(p.a);
  const float* __restrict__ b = static_cast<const float*>(p.b);
  void* c = p.c;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb, ldc = p.ldc;
  const Epilogue& epi = p.epi;
  __shared__ f32x4 partial[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gx = (N + 15) / 16;
  const int m0 = static_cast<int>(blockIdx.x) / gx * 16, n0 = static_cast<int>(blockIdx.x) % gx * 16;
  const int r = lane & 15, q = lane >> 4;
  const bool a_ok = m0 + r < M, b_ok = n0 + r < N;
  const float* arow = a + static_cast<int64_t>(a_ok ? m0 + r : 0) * lda;
  const float* bcol = b + (b_ok ? n0 + r : 0);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int groups = (K + 15) / 16;
  for (int g = wave; g < groups; g += 4) {
    const int kb = 16 * g + 4 * q;
    float av[4], bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool k_ok = kb + j < K;
      const int k = k_ok ? kb + j : 0;
      av[j] = a_ok && k_ok ? arow[k] : 0.f;
      bv[j] = b_ok && k_ok ? bcol[static_cast<int64_t>(k) * ldb] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv[j], acc, 0, 0, 0);
  }
  partial[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  acc = partial[0][lane];
#pragma unroll
  for (int w = 1; w < 4; ++w) acc += partial[w][lane];
  const int n = n0 + r;
  if (n >= N) return;
  const float bias_n = epi.bias_at(n);
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int m = m0 + 4 * q + rr;
    if (m >= M) continue;
    const float v = epi(acc[rr], bias_n);
    const int64_t off = static_cast<int64_t>(m) * ldc + n;
    if constexpr (kOut == kOutF32) static_cast<float*>(c)[off] = v;
    else if constexpr (kOut == kOutF16) static_cast<uint16_t*>(c)[off] = asc::f32_to_f16_rne(v);
    else static_cast<uint16_t*>(c)[off] = asc::f32_to_bf16_rne(v);
  }
}

// ---- fp32 inputs, large outputs: LDS-tiled FMA kernel (64x64 tile, 256 threads, 4x4 per thread)
// Block b covers output tile (b / ceil(N/64), b % ceil(N/64)).
template <int kOut>
__device__ __forceinline__ void gemm_f32_fma_body(const GemmArgs& p) {
  const float* __restrict__ a = static_cast<const float*>(p.a);
  const float* __restrict__ b = static_cast<const float*>(p.b);
  void* c = p.c;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb, ldc = p.ldc;
  const Epilogue& epi = p.epi;
  __shared__ float as[16][64 + 1];
  __shared__ float bs[16][64 + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int gx = (N + 63) / 64;
  const int m0 = static_cast<int>(blockIdx.x) / gx * 64, n0 = static_cast<int>(blockIdx.x) % gx * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = threadIdx.x; i < 16 * 64; i += 256) {
      const int kk = i & 15, mm = i >> 4;
      as[kk][mm] = (m0 + mm < M && k0 + kk < K) ? a[(m0 + mm) * lda + k0 + kk] : 0.f;
      const int nn = i & 63, kb = i >> 6;
      bs[kb][nn] = (n0 + nn < N && k0 + kb < K) ? b[(k0 + kb) * ldb + n0 + nn] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(as[kk][ty * 4 + i], bs[kk][tx * 4 + j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m >= M || n >= N) continue;
      const float v = epi(acc[i][j], epi.bias_at(n));
      const int64_t off = static_cast<int64_t>(m) * ldc + n;
      if constexpr (kOut == kOutF32) static_cast<float*>(c)[off] = v;
      else if constexpr (kOut == kOutF16) static_cast<uint16_t*>(c)[off] = asc::f32_to_f16_rne(v);
      else static_cast<uint16_t*>(c)[off] = asc::f32_to_bf16_rne(v);
    }
  }
}

}  // namespace mm
}  // namespace asc

// Defines the matmul kernels with the given linkage specifier, each taking one
// asc::mm::GemmArgs by value:
//   PREFIX##mfma_{bf16,f16}_{fast,checked}_{f32,f16,bf16}  16-bit inputs, output dtype
//   PREFIX##f32_mfma_{f32,f16,bf16}                          fp32 inputs, 16x16 blocks
//   PREFIX##f32_fma_{f32,f16,bf16}                           fp32 inputs, 64x64 tiles
#define ASC_MM_MFMA_KERNEL(LINKAGE, NAME, BF16, CHECKED, OUT)                                                      \
  LINKAGE __global__ void __launch_bounds__(CHECKED ? asc::mm::kThreads : asc::mm::kFastThreads, 1)               \
      NAME(asc::mm::GemmArgs p) {                                                                                  \
    asc::mm::gemm_mfma_body<BF16, CHECKED, OUT>(p);                                                                \
  }
#define ASC_MM_F32_KERNEL(LINKAGE, NAME, BODY, OUT)                                                                \
  LINKAGE __global__ void __launch_bounds__(256) NAME(asc::mm::GemmArgs p) { asc::mm::BODY<OUT>(p); }
#define ASC_MM_KERNELS_OUT(LINKAGE, PREFIX, SFX, OUT)                                                              \
  ASC_MM_MFMA_KERNEL(LINKAGE, PREFIX##mfma_bf16_fast_##SFX, true, false, OUT)                                      \
  ASC_MM_MFMA_KERNEL(LINKAGE, PREFIX##mfma_bf16_checked_##SFX, true, true, OUT)                                    \
  ASC_MM_MFMA_KERNEL(LINKAGE, PREFIX##mfma_f16_fast_##SFX, false, false, OUT)                                      \
  ASC_MM_MFMA_KERNEL(LINKAGE, PREFIX##mfma_f16_checked_##SFX, false, true, OUT)                                    \
  ASC_MM_F32_KERNEL(LINKAGE, PREFIX##f32_mfma_##SFX, gemm_f32_mfma_body, OUT)                                      \
  ASC_MM_F32_KERNEL(LINKAGE, PREFIX##f32_fma_##SFX, gemm_f32_fma_body, OUT)
#define ASC_MM_KERNELS(LINKAGE, PREFIX)                                                                            \
  ASC_MM_KERNELS_OUT(LINKAGE, PREFIX, f32, asc::mm::kOutF32)                                                       \
  ASC_MM_KERNELS_OUT(LINKAGE, PREFIX, f16, asc::mm::kOutF16)                                                       \
  ASC_MM_KERNELS_OUT(LINKAGE, PREFIX, bf16, asc::mm::kOutBF16)
