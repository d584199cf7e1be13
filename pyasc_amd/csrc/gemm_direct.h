// Direct-to-LDS MFMA GEMM main loop for tile-aligned shapes (the fast path of
// matmul.hip and matmul_i8.hip; ragged shapes use gemm_core.h).
//
//   - 256x256 output tile per workgroup of 2 x kWavesN waves: with kWavesN = 2
//     each wave owns 128x128 = 4x4 blocks of 32x32 MFMA accumulators (256
//     AGPRs, one wave per SIMD); with kWavesN = 4 each owns 128x64 = 4x2 blocks
//     (128 AGPRs), two waves per SIMD whose stalls the other covers.
//   - A k-tile is 64 bytes of K (32 fp16/bf16 or 64 int8 elements): 2 MFMA
//     k-steps.  Operands go from HBM straight into LDS (buffer_load ... lds,
//     16 bytes per lane, 1 KiB per wave instruction): no staging registers, no
//     ds_write.  Five LDS stages of 32 KiB (A 16 KiB + B 16 KiB, 160 KiB: all
//     of the CU's LDS); the loads of k-tile kt+4 are issued while k-tile kt is
//     computed, so each tile has three to four tiles of MFMA work to arrive
//     (a fifth stage measured -8% loop time on the 4096x11008x4096 int8 shape
//     and no change on power-of-two shapes).
//   - One s_barrier per k-tile with no drain: before it a wave only waits for
//     its own loads of tile kt+2 (vmcnt counts the two newer tiles), and the
//     first operand fragments of tile kt+1 are already read.
//   - A tile: 256 rows x 64 bytes (K contiguous); 16-byte chunks swizzled by
//     gA(row) = (row >> 2) & 3; MFMA operands are ds_read_b128.
//   - B tile: kBK rows (K) x 256 columns, row-major as in HBM (N contiguous);
//     the K-contiguous MFMA operand is read with the gfx950 LDS transpose
//     reads (ds_read_b64_tr_b16 / ds_read_b64_tr_b8).  16-byte chunks are
//     swizzled per row so those reads are conflict-free (tables found by
//     enumerating bank models, confirmed with SQ_LDS_BANK_CONFLICT = 0 on the
//     device).
//   - Lane layouts of the transpose reads (measured on the device): in each
//     16-lane group, b16: lane i receives element i%4 of lane 4j + i/4's 8-byte
//     read (j = 0..3); b8: lane i receives byte i%8 of lane 2j + i/8's read
//     (j = 0..7).
//   - The stages are distinct __shared__ objects and every access names its
//     stage at compile time (the loop is unrolled by the stage count), so the
//     compiler can tell that loads into one stage do not alias reads of another.
#pragma once

#include <utility>

#include "gemm_common.h"

namespace asc {
namespace gemm {

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((vector_size(8)));

constexpr int kDirectStages = 5;
constexpr int kDirectStageBytes = 32768;

template <class Tr, int kWavesN = 2>
struct GemmDirectLoop {
  using Elem = typename Tr::Elem;
  using Acc = typename Tr::Acc;
  static constexpr int kES = sizeof(Elem);
  static constexpr int kBK = 64 / kES;          // K elements per k-tile (64 bytes)
  static constexpr int kBRowBytes = 256 * kES;  // one B tile row (256 columns)
  static constexpr int kBRowsPerLoad = 1024 / kBRowBytes;
  static constexpr int kBOff = 16384;
  static constexpr int kWaves = 2 * kWavesN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kJ = 8 / kWavesN;           // 32-column MFMA blocks per wave
  static constexpr int kLoads = 16 / kWaves;       // 1 KiB load instructions per wave per operand and k-tile
  // loads a wave may leave in flight at a k-tile's barrier: tiles kt+3 .. kt+S-1
  static constexpr int kInFlight = 2 * kLoads * (kDirectStages - 3);
  static constexpr int kMfmaPerStep = 4 * kJ;
  static constexpr int kDsPerStep = 4 + 2 * kJ;
  static_assert(kWavesN == 2 || kWavesN == 4, "2x2 or 2x4 waves");

  // A chunk swizzle (4 chunks per 64-byte row).  Chosen by measurement
  // (SQ_LDS_BANK_CONFLICT on the operand-read pattern): (row >> 2) & 3 reads
  // conflict-free, ((row >> 1) ^ (row >> 3)) & 3 costs 4 conflict cycles per read.
  __device__ __forceinline__ static int ga(int row) { return (row >> 2) & 3; }
  // B chunk swizzle: position p of row r holds logical chunk p ^ fb(r)
  __device__ __forceinline__ static int fb(int row) {
    if constexpr (kES == 2) return (0xCA60u >> (4 * (row & 3))) & 15;   // {0, 6, 10, 12}
    else return (0xE5CB2097u >> (4 * (row & 7))) & 15;                  // {7, 9, 0, 2, 11, 12, 5, 14}
  }

  const Elem* a;
  const Elem* b;
  int m0, n0;
  int lane, wave, wm, wn;
  int lda_bytes, ldb_bytes;
  uint8_t* lds[kDirectStages];
  __amdgpu_buffer_rsrc_t rsrc_a, rsrc_b;
  int voff_a[4];       // per A load instruction (the first kLoads are used)
  int voff_b[2];       // per parity of the B load instruction

  __device__ __forceinline__ void init(int64_t lda, int64_t ldb) {
    lda_bytes = static_cast<int>(lda) * kES;
    ldb_bytes = static_cast<int>(ldb) * kES;
    const Elem* a_panel = a + static_cast<int64_t>(m0) * lda;
    const Elem* b_cols = b + n0;
    rsrc_a = __builtin_amdgcn_make_buffer_rsrc(const_cast<Elem*>(a_panel), static_cast<short>(0), 0x7fffffff,
                                               0x00020000);
    rsrc_b = __builtin_amdgcn_make_buffer_rsrc(const_cast<Elem*>(b_cols), static_cast<short>(0), 0x7fffffff,
                                               0x00020000);
    // A: instruction i of wave w loads rows 16R .. 16R+15, R = kLoads*w + i; lane l ->
    // row 16R + l/4, LDS position l%4 holding logical chunk (l%4) ^ ga(row).
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int R = wave * kLoads + i;
      const int row = 16 * R + (lane >> 2);
      const int c = (lane & 3) ^ ga(row);
      voff_a[i] = (lane >> 2) * lda_bytes + c * 16;
    }
    // B: instruction R loads rows kBRowsPerLoad*R + lane / (64 / kBRowsPerLoad);
    // the row's swizzle only depends on R's parity.
    constexpr int kLanesPerRow = 64 / kBRowsPerLoad;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int rr = lane / kLanesPerRow;
      const int row = kBRowsPerLoad * par + rr;
      const int c = (lane % kLanesPerRow) ^ fb(row);
      voff_b[par] = rr * ldb_bytes + c * 16;
    }
  }

  template <int kS>
  __device__ __forceinline__ void issue_loads(int k0) {
    uint8_t* base = lds[kS];
    const int kb = k0 * kES;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int R = wave * kLoads + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (__attribute__((address_space(3))) void*)(base + R * 1024),
                                               16, voff_a[i], 16 * R * lda_bytes + kb, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int R = wave * kLoads + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_b,
                                               (__attribute__((address_space(3))) void*)(base + kBOff + R * 1024), 16,
                                               voff_b[i & 1], (k0 + kBRowsPerLoad * R) * ldb_bytes, 0, 0);
    }
  }

  // byte offset of element (row, col) in the swizzled B tile
  __device__ __forceinline__ static int b_off(int row, int col) {
    const int byte = col * kES;
    return row * kBRowBytes + (((byte >> 4) ^ fb(row)) << 4) + (byte & 15);
  }

  template <int kS>
  __device__ __forceinline__ void read_frags(int step, u32x4 (&fa)[4], u32x4 (&fbv)[kJ]) const {
    const uint8_t* as = lds[kS];
    const uint8_t* bs = as + kBOff;
    const int h = lane >> 5;
    const int chunk = step * 2 + h;
    const int arow = wm * 128 + (lane & 31);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = arow + i * 32;
      fa[i] = *reinterpret_cast<const u32x4*>(as + row * 64 + ((chunk ^ ga(row)) << 4));
    }
    const int g = (lane >> 4) & 1, t = lane & 15;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int nb = wn * (32 * kJ) + j * 32 + 16 * g;
      if constexpr (kES == 2) {
        // k = 16*step + 8h + e; read e = 0..3 then 4..7; lane 4jj+q -> row +jj, col +4q
        const int row = step * 16 + 8 * h + (t >> 2);
        const int col = nb + 4 * (t & 3);
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4_t*)(bs + b_off(row, col)));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4_t*)(bs + b_off(row + 4, col)));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        fbv[j] = u32x4{l2[0], l2[1], h2[0], h2[1]};
      } else {
        // k = 32*step + 16h + e; read e = 0..7 then 8..15; lane 2jj+sub -> row +jj, col +8sub
        const int row = step * 32 + 16 * h + (t >> 1);
        const int col = nb + 8 * (t & 1);
        const i32x2_t lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) i32x2_t*)(bs + b_off(row, col)));
        const i32x2_t hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) i32x2_t*)(bs + b_off(row + 8, col)));
        fbv[j] = u32x4{static_cast<uint32_t>(lo[0]), static_cast<uint32_t>(lo[1]), static_cast<uint32_t>(hi[0]),
                       static_cast<uint32_t>(hi[1])};
      }
    }
  }

  __device__ __forceinline__ static void mma(Acc (&acc)[4][kJ], const u32x4 (&fa)[4], const u32x4 (&fbv)[kJ]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < kJ; ++j) acc[i][j] = Tr::mfma(fa[i], fbv[j], acc[i][j]);
  }

  // Workgroup barrier that does not wait for outstanding loads (unlike
  // __syncthreads, whose fence drains vmcnt).
  __device__ __forceinline__ static void barrier() { asm volatile("s_barrier" ::: "memory"); }

  // k-tile kt, held in stage kS.  On entry the k-step-0 fragments of tile kt
  // are in fa0/fb0, and tiles kt and kt+1 are visible in LDS.
  template <int kS>
  __device__ __forceinline__ void iteration(int kt, int k_tiles, Acc (&acc)[4][kJ], u32x4 (&fa0)[4],
                                            u32x4 (&fb0)[kJ], u32x4 (&fa1)[4], u32x4 (&fb1)[kJ]) {
    constexpr int kAheadTiles = kDirectStages - 1;
    constexpr int kNext = (kS + 1) % kDirectStages;
    constexpr int kAhead = (kS + kAheadTiles) % kDirectStages;  // the stage tile kt-1 has left
    constexpr int kVmem = 2 * kLoads;
    // k-step 0: tile kt+4's loads (clamped: the tail re-loads the last tile
    // into a free stage) and k-step 1's operand reads, one per MFMA.
    issue_loads<kAhead>((kt + kAheadTiles < k_tiles ? kt + kAheadTiles : k_tiles - 1) * kBK);
    read_frags<kS>(1, fa1, fb1);
    mma(acc, fa0, fb0);
#pragma unroll
    for (int i = 0; i < kVmem; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read (LDS DMA)
    }
#pragma unroll
    for (int i = 0; i < kDsPerStep - kVmem; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (kMfmaPerStep > kDsPerStep) __builtin_amdgcn_sched_group_barrier(0x008, kMfmaPerStep - kDsPerStep, 0);
    // k-step 1: the next tile's k-step-0 operands, one read per MFMA
    read_frags<kNext>(0, fa0, fb0);
    mma(acc, fa1, fb1);
#pragma unroll
    for (int i = 0; i < kDsPerStep; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
    }
    if constexpr (kMfmaPerStep > kDsPerStep) __builtin_amdgcn_sched_group_barrier(0x008, kMfmaPerStep - kDsPerStep, 1);
    // own loads of tile kt+2 done (only the newer tiles' may still run), and
    // this wave's reads of stage kS complete before anyone reloads it
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"i"(kInFlight) : "memory");
    barrier();
  }

  // One pass over the ring: k-tiles kt .. kt+kDirectStages-1 in stages 0 ..
  template <int... kS>
  __device__ __forceinline__ void ring(std::integer_sequence<int, kS...>, int kt, int k_tiles, Acc (&acc)[4][kJ],
                                       u32x4 (&fa0)[4], u32x4 (&fb0)[kJ], u32x4 (&fa1)[4], u32x4 (&fb1)[kJ]) {
    (iteration<kS>(kt + kS, k_tiles, acc, fa0, fb0, fa1, fb1), ...);
  }
  // The last k_tiles - kt (< kDirectStages) tiles, from stage 0.
  template <int... kS>
  __device__ __forceinline__ void ring_tail(std::integer_sequence<int, kS...>, int kt, int k_tiles,
                                            Acc (&acc)[4][kJ], u32x4 (&fa0)[4], u32x4 (&fb0)[kJ], u32x4 (&fa1)[4],
                                            u32x4 (&fb1)[kJ]) {
    ((kt + kS < k_tiles ? iteration<kS>(kt + kS, k_tiles, acc, fa0, fb0, fa1, fb1) : void()), ...);
  }

  template <int... kS>
  __device__ __forceinline__ void prologue(std::integer_sequence<int, kS...>, int k_tiles) {
    (issue_loads<kS>((kS < k_tiles ? kS : k_tiles - 1) * kBK), ...);
  }

  __device__ __forceinline__ void run(int K, Acc (&acc)[4][kJ]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < kJ; ++j) acc[i][j] = Acc{};
    const int k_tiles = K / kBK;
    // tiles 0 .. kDirectStages-2 (clamped like the loop's), then wait for 0 and 1
    prologue(std::make_integer_sequence<int, kDirectStages - 1>(), k_tiles);
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"(kInFlight) : "memory");
    barrier();
    u32x4 fa0[4], fb0[kJ], fa1[4], fb1[kJ];
    read_frags<0>(0, fa0, fb0);
    int kt = 0;
    for (; kt + kDirectStages <= k_tiles; kt += kDirectStages)
      ring(std::make_integer_sequence<int, kDirectStages>(), kt, k_tiles, acc, fa0, fb0, fa1, fb1);
    ring_tail(std::make_integer_sequence<int, kDirectStages - 1>(), kt, k_tiles, acc, fa0, fb0, fa1, fb1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load may outlive the kernel
  }
};

}  // namespace gemm
}  // namespace asc
