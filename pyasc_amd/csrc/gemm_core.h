// Software-pipelined MFMA GEMM main loop shared by the fp16/bf16 and int8
// kernels (matmul.hip, matmul_i8.hip).
//
//   - 256x256 output tile per 256-thread workgroup; 4 waves in 2x2, each wave
//     128x128 = 4x4 blocks of 32x32 MFMA accumulators (256 AGPRs).
//   - Two LDS stages of 64 KiB (A and B tiles, 128-byte K-contiguous rows,
//     XOR-swizzled 16-byte chunks).  One k-tile = 4 MFMA k-steps of 16 bytes
//     per lane half.
//   - Per k-tile: global loads for the k-tile two ahead are issued during
//     k-step 0 (two register staging sets), the operand fragments of k-step
//     s+1 are read from LDS while the MFMAs of k-step s run, and the next tile
//     is transposed/written into the other LDS stage during k-step 3.
//     sched_barrier fences between the k-steps keep that order, so neither
//     LDS nor HBM latency is serialised in front of the MFMAs.
//   - The loop body is branch-free on the unchecked path: the last iterations
//     re-fetch the last tile and write it into the unused stage.
#pragma once

#include "gemm_common.h"

namespace asc {
namespace gemm {

constexpr int kTileM = 256;
constexpr int kTileN = 256;
constexpr int kGemmThreads = 256;
constexpr int kStageBytes = (kTileM + kTileN) * 128;
constexpr int kGroupM = 8;

struct GemmShape {
  int M, N, K;
  int64_t lda, ldb;  // elements (16-bit) or bytes (int8)
  int tiles_m, tiles_n;
};

// Traits provide: Elem (storage type), Acc (accumulator vector), kBK (K elements
// per k-tile = 128 bytes), kBRows (B rows per lane per k-tile), BReg (one B row
// fragment), load_a / load_b (global), transpose_b, mfma.
template <class Tr, bool kChecked>
struct GemmMainLoop {
  using Elem = typename Tr::Elem;
  using Acc = typename Tr::Acc;
  using BReg = typename Tr::BReg;
  static constexpr int kBK = Tr::kBK;
  static constexpr int kBRows = Tr::kBRows;  // rows of the per-lane B block (k direction)

  const Elem* a;
  const Elem* b;
  GemmShape s;
  int m0, n0;
  int tid, lane, wm, wn;
  bool a_vec, b_vec;
  uint8_t* lds[2];  // the two LDS stages
  // Unchecked path: buffer loads with one per-lane VGPR offset per operand and
  // wave-uniform (SGPR) offsets for the row/k advance, instead of a 64-bit
  // address per load.  Descriptors cover the block's A panel and B columns.
  __amdgpu_buffer_rsrc_t rsrc_a, rsrc_b;
  int voff_a, voff_b;
  int lda_bytes, ldb_bytes;

  __device__ __forceinline__ void init_buffers() {
    constexpr int es = sizeof(Elem);
    lda_bytes = static_cast<int>(s.lda) * es;
    ldb_bytes = static_cast<int>(s.ldb) * es;
    const Elem* a_panel = a + static_cast<int64_t>(m0) * s.lda;
    const Elem* b_cols = b + n0;
    rsrc_a = __builtin_amdgcn_make_buffer_rsrc(const_cast<Elem*>(a_panel), static_cast<short>(0), 0x7fffffff,
                                               0x00020000);
    rsrc_b = __builtin_amdgcn_make_buffer_rsrc(const_cast<Elem*>(b_cols), static_cast<short>(0), 0x7fffffff,
                                               0x00020000);
    voff_a = (tid >> 3) * lda_bytes + (tid & 7) * 16;
    voff_b = (tid >> 5) * kBRows * ldb_bytes + (tid & 31) * 8 * es;
  }

  // Global-load staging registers: one k-tile of A (8 x 16 bytes) and B
  // (kBRows rows) per lane.  Two sets so that loads run two k-tiles ahead.
  struct Stage {
    u32x4 ra[8];
    BReg rb[kBRows];
  };

  __device__ __forceinline__ void fetch(int k0, Stage& st) {
    if constexpr (!kChecked) {
      const int kb = k0 * static_cast<int>(sizeof(Elem));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        st.ra[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, voff_a, 32 * i * lda_bytes + kb, 0);
      }
#pragma unroll
      for (int r = 0; r < kBRows; ++r) {
        if constexpr (sizeof(BReg) == 16) {
          st.rb[r] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_b, voff_b, (k0 + r) * ldb_bytes, 0);
        } else {
          st.rb[r] = __builtin_amdgcn_raw_buffer_load_b64(rsrc_b, voff_b, (k0 + r) * ldb_bytes, 0);
        }
      }
      return;
    }
    // A: chunk c = tid + 256*i -> row c/8, 16-byte chunk c%8 of the 128-byte k row
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = tid + kGemmThreads * i;
      st.ra[i] = Tr::template load_a<kChecked>(a, s.lda, m0 + (c >> 3), k0 + (c & 7) * (16 / sizeof(Elem)), s.M,
                                               s.K, a_vec);
    }
    // B: lane block = kBRows k-rows x 8 columns; n-chunk tid%32, k-group tid/32
    const int nc = tid & 31, kg = tid >> 5;
#pragma unroll
    for (int r = 0; r < kBRows; ++r) {
      st.rb[r] = Tr::template load_b<kChecked>(b, s.ldb, k0 + kg * kBRows + r, n0 + nc * 8, s.K, s.N, b_vec);
    }
  }

  __device__ __forceinline__ void stash(int stage, const Stage& st) {
    uint8_t* as = lds[stage];
    uint8_t* bs = as + kTileM * 128;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = tid + kGemmThreads * i;
      *reinterpret_cast<u32x4*>(as + lds_offset(c >> 3, c & 7)) = st.ra[i];
    }
    u32x4 tb[8];
    Tr::transpose_b(st.rb, tb);
    const int nc = tid & 31, kg = tid >> 5;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      *reinterpret_cast<u32x4*>(bs + lds_offset(nc * 8 + e, kg)) = tb[e];
    }
  }

  __device__ __forceinline__ void read_frags(int stage, int step, u32x4 (&fa)[4], u32x4 (&fb)[4]) const {
    const uint8_t* as = lds[stage];
    const uint8_t* bs = as + kTileM * 128;
    const int chunk = step * 2 + (lane >> 5);
    const int arow = wm * 128 + (lane & 31);
    const int brow = wn * 128 + (lane & 31);
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[i] = *reinterpret_cast<const u32x4*>(as + lds_offset(arow + i * 32, chunk));
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const u32x4*>(bs + lds_offset(brow + j * 32, chunk));
  }

  __device__ __forceinline__ static void mma(Acc (&acc)[4][4], const u32x4 (&fa)[4], const u32x4 (&fb)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = Tr::mfma(fa[i], fb[j], acc[i][j]);
  }

  // One k-tile.  LDS stage `kStage` holds tile kt; `held` holds tile kt+1 (loaded
  // one iteration earlier) and is written to the other stage in k-step 3;
  // `spare` receives tile kt+2.  Phases are fenced with sched_barrier so each
  // load stays one phase ahead of the MFMAs that consume it.
  template <int kStage>
  __device__ __forceinline__ void iteration(int kt, int k_tiles, Acc (&acc)[4][4], Stage& held, Stage& spare,
                                            u32x4 (&fa0)[4], u32x4 (&fb0)[4], u32x4 (&fa1)[4], u32x4 (&fb1)[4]) {
    const int ahead = kt + 2 < k_tiles ? kt + 2 : k_tiles - 1;
    // k-step 0: global loads of tile kt+2, LDS reads of k-step 1
    fetch(ahead * kBK, spare);
    read_frags(kStage, 1, fa1, fb1);
    mma(acc, fa0, fb0);
    __builtin_amdgcn_sched_barrier(0);
    // k-step 1
    read_frags(kStage, 2, fa0, fb0);
    mma(acc, fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    // k-step 2
    read_frags(kStage, 3, fa1, fb1);
    mma(acc, fa0, fb0);
    __builtin_amdgcn_sched_barrier(0);
    // k-step 3: transpose + store tile kt+1 into the other stage
    stash(kStage ^ 1, held);
    mma(acc, fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    read_frags(kStage ^ 1, 0, fa0, fb0);
  }

  __device__ __forceinline__ void run(Acc (&acc)[4][4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = Acc{};

    const int k_tiles = (s.K + kBK - 1) / kBK;
    if constexpr (!kChecked) init_buffers();
    Stage sa, sb;
    fetch(0, sa);
    fetch((k_tiles > 1 ? 1 : 0) * kBK, sb);
    stash(0, sa);
    __syncthreads();
    u32x4 fa0[4], fb0[4], fa1[4], fb1[4];
    read_frags(0, 0, fa0, fb0);

    // unrolled by two so that the staging sets and LDS stages are compile-time
    int kt = 0;
    for (; kt + 1 < k_tiles; kt += 2) {
      iteration<0>(kt, k_tiles, acc, sb, sa, fa0, fb0, fa1, fb1);
      iteration<1>(kt + 1, k_tiles, acc, sa, sb, fa0, fb0, fa1, fb1);
    }
    if (kt < k_tiles) iteration<0>(kt, k_tiles, acc, sb, sa, fa0, fb0, fa1, fb1);
  }
};

}  // namespace gemm
}  // namespace asc
