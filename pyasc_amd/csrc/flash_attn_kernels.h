// Flash-attention forward, bf16 in/out, fp32 online-softmax statistics: the device
// code, shared by the library (flash_attn.hip, launched through
// asc_flash_attention_fwd_bf16) and the standalone gfx950 code object
// (co/asc2_flash_attention.hip, loaded with hipModuleLoad by the asc2 launch path).
// The reference has no attention kernel; this is the build's asc2-style
// flash_attention_fwd_kernel (BASELINE config: batch 4, 32 heads, seq 4096,
// head_dim 128, scale 1/sqrt(128), causal and non-causal).
//
// Design (gfx950, wave64, MFMA 32x32x16 bf16):
//  - A wave owns 32 queries of one (batch, head); a workgroup has 4 waves
//    (128 queries; head_dim 64) or 8 waves (256 queries; head_dim 128).  Keys/values stream through LDS in tiles of 64,
//    K and V each in a ring of three stages filled by direct-to-LDS loads.
//  - Each wave computes S^T = K Q^T (keys x queries) instead of S = Q K^T:
//    in the MFMA result layout a lane then holds ONE query column and 16 keys
//    per 32x32 block, so the online-softmax max/sum of a query live in two
//    lanes (lane and lane^32) -- one cross-lane shuffle per statistic.
//  - O^T = V^T P^T: P^T is the B operand straight from the S^T registers (no
//    data movement; A and B agree on which key each operand slot holds), V^T is
//    read from the row-major V tile with ds_read_b64_tr_b16 (gfx950 LDS
//    transpose read).  Q^T stays in registers for the whole kernel.
//  - Online softmax in the exp2 domain: scale*log2(e) and the shift by the
//    reference point fold into one FMA before exp2; the reference point is not
//    moved per tile but only when a lane's probability sum over a tile exceeds
//    kTileSumLimit, and then to the tile max (exact arithmetic either way, O
//    and l are rescaled rarely); causal tiles above the diagonal are skipped and
//    the diagonal tile is masked; heavy (late) query blocks are scheduled first.
//  - The clean step computes tile j's probabilities between the S^T MFMAs of
//    tile j+1, so one wave's exp2 work and MFMAs overlap.
// LDS tiles use XOR-swizzled 16-byte chunks so that both the MFMA operand
// reads and the transpose reads are free of bank conflicts.
#pragma once

#include <math.h>

#include "common.h"
#include "numeric.h"

namespace asc {
namespace fa {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BKV = 64;  // keys per LDS tile

struct FaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t heads_total;  // batch * heads
  int seq;
  int n_qblocks;
  int head_group;  // heads whose query blocks an XCD interleaves (see the block order)
  float scale_log2;  // sm_scale * log2(e)
  int causal;
};

// K tile rows (D/8 chunks of 16 bytes): chunk position = c ^ kswz(row) makes
// 16 consecutive rows reading the same chunk hit 16 distinct bank groups.
template <int D>
__device__ __forceinline__ int kswz(int row) {
  return D == 128 ? (row & 15) : ((row >> 1) & 7);
}
// V tile rows: the transpose read touches 4 consecutive rows x 64 bytes; the
// swizzle spreads those rows over distinct 64-byte bank quadrants.
template <int D>
__device__ __forceinline__ int vswz(int row) {
  return D == 128 ? ((row & 3) << 2) : (((row >> 1) & 1) << 2);
}

template <int D>
__device__ __forceinline__ uint32_t k_off(int row, int chunk) {
  return static_cast<uint32_t>(row * (D * 2) + ((chunk ^ kswz<D>(row)) << 4));
}
template <int D>
__device__ __forceinline__ uint32_t v_off(int row, int col) {
  return static_cast<uint32_t>(row * (D * 2) + (((col >> 3) ^ vswz<D>(row)) << 4) + ((col & 7) << 1));
}

__device__ __forceinline__ f32x16 mfma_bf16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 pair, RNE (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)p));
}

// MFMA operand reads from LDS are inline asm.  The compiler cannot prove that a
// read of one ring stage does not alias the buffer_load ... lds still streaming
// into the other stage, so with plain loads it inserts an s_waitcnt vmcnt for
// that DMA in the middle of the step.  The kernel orders DMA and reads itself
// (every stage is refilled only after the workgroup barrier that follows its
// last read, and each step ends with vmcnt(0) + barrier before the stage it
// filled is read); the asm reads carry explicit lgkmcnt waits, tied to the
// registers they produce so that the consuming MFMA cannot move above them.
// LDS reads complete in order, so lgkmcnt(n) after a group of reads makes all
// but the newest n of them available.
// (`off` must fold to a constant once the calling loops are unrolled.)
__device__ __forceinline__ u32x4 lds_read_b128(uint32_t addr, int off) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off));
  return r;
}
__device__ __forceinline__ u32x2 lds_read_tr16_b64(uint32_t addr, int off) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off));
  return r;
}
__device__ __forceinline__ void lds_wait(u32x4& r, int n) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(n));
}
__device__ __forceinline__ void lds_wait(u32x4 (&r)[4], int n) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]) : "i"(n));
}

// Value of lane l^32 (v_permlane32_swap: lanes 32..63 of the first operand trade
// places with lanes 0..31 of the second; the lane half picks the result that
// holds the partner's value).
__device__ __forceinline__ float other_half(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

// Largest sum of one lane's unnormalised probabilities over a key tile (32
// values) before the reference point is moved: bounds every exp2 value by 2^16.
constexpr float kTileSumLimit = 65536.0f;

// Per-wave state of the attention kernel.  A wave owns QB blocks of 32 queries
// (32*QB queries); a workgroup of kWaves waves owns 32*QB*kWaves.  Every K or V
// operand a wave reads from LDS feeds QB MFMAs, one per query block, so LDS
// read traffic per MFMA falls as 1/QB.
template <int D, int kWaves, int QB>
struct FaState {
  static constexpr int kQ = 32 * QB;              // queries per wave
  static constexpr int kChunks = D / 8;           // 16-byte chunks per row
  static constexpr int kTileBytes = BKV * D * 2;  // one K or V tile
  static constexpr int kKSteps = D / 16;          // MFMA k-steps over head_dim
  static constexpr int kDBlocks = D / 32;         // 32-wide d blocks of O^T
  static constexpr int kRowsPerLoad = 1024 / (D * 2);     // tile rows per 1 KiB wave load
  static constexpr int kLoadsPerWave = BKV / kRowsPerLoad / kWaves;  // per tile

  int lane, wave, col, h;
  int q0, S, causal;
  int qw0;  // first query of this wave: q0 + wave * kQ
  float scale_log2;
  __amdgpu_buffer_rsrc_t rsrc_k, rsrc_v;
  int voff_k[4], voff_v;  // voff_k[i]: this wave's i-th K load (kLoadsPerWave <= 4)
  // Per-lane LDS read offsets, loop-invariant: the K swizzle of row kb*32+col
  // equals that of row col, and the V swizzle of row r0+j (r0 % 4 == 0) equals
  // that of row j, so every other term of a read address is an immediate.
  uint32_t kaddr[kKSteps];   // K row col, chunk 2*kk+h
  uint32_t vaddr[kDBlocks];  // V transpose read of d block db, rows 4h+j
  u32x4 qreg[QB][kKSteps];
  f32x16 acc_o[QB][kDBlocks];
  float m_run[QB];   // reference point of the scaled scores (log2 domain), <= running max
  float l_part[QB];  // this lane half's share of the running sum of exp2(s*scale_log2 - m_run)

  // query of this lane in query block qb
  __device__ __forceinline__ int my_q(int qb) const { return qw0 + qb * 32 + col; }

  // K/V tile rows go straight from HBM into LDS (buffer_load ... lds, 1 KiB per
  // wave instruction, lane l -> row kRowsPerLoad*R + l/(64/kRowsPerLoad)).  The
  // lane loads the logical chunk that the row's swizzle puts at its position;
  // keys >= S read as zero through the descriptor's byte bound.
  __device__ __forceinline__ void init_loads(const uint16_t* Kh, const uint16_t* Vh) {
    const int bytes = S * D * 2;
    rsrc_k = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Kh), static_cast<short>(0), bytes, 0x00020000);
    rsrc_v = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Vh), static_cast<short>(0), bytes, 0x00020000);
    constexpr int kLanesPerRow = 64 / kRowsPerLoad;
    const int rr = lane / kLanesPerRow, pos = lane % kLanesPerRow;
    static_assert(kLoadsPerWave >= 1 && kLoadsPerWave <= 4, "K load offsets");
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) {
      // the K swizzle depends on (row mod 16) = kRowsPerLoad*(R mod 4) + rr; indexing
      // by the load number keeps the array in registers whatever the wave count
      const int R = wave * kLoadsPerWave + i;
      const int row = kRowsPerLoad * (R & 3) + rr;
      voff_k[i] = rr * (D * 2) + ((pos ^ kswz<D>(row)) << 4);
    }
    voff_v = rr * (D * 2) + ((pos ^ vswz<D>(rr)) << 4);
#pragma unroll
    for (int kk = 0; kk < kKSteps; ++kk) kaddr[kk] = k_off<D>(col, kk * 2 + h);
    // ds_read_b64_tr_b16: in each 16-lane group, lane 4j+q addresses row
    // (rowstart + j), columns 4q..4q+3 of the group's 16 columns; lane i of the
    // group receives column i, rows rowstart..+3.
    const int g_lane = lane & 15;
    const int tr_col = ((lane >> 4) & 1) * 16 + (g_lane & 3) * 4;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) vaddr[db] = v_off<D>(h * 4 + (g_lane >> 2), db * 32 + tr_col);
  }

  // Keys k0 .. k0+63 of K (kIsV false) or V into one LDS stage.
  template <bool kIsV>
  __device__ __forceinline__ void load_tile(uint8_t* dst, int k0) const {
    // The LDS destination (M0) of each load is formed here, from an opaque copy
    // of the wave's offset: left to itself the compiler keeps one SGPR per stage
    // and load for the whole kernel and spills them.
    int wave_lds = wave * (kLoadsPerWave * 1024);
    asm volatile("" : "+s"(wave_lds));
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) {
      const int R = wave * kLoadsPerWave + i;
      // the row offset goes into the per-lane offset, not the SGPR offset: the
      // buffer range check (keys >= S read as zero) only covers the former
      const int roff = (k0 + kRowsPerLoad * R) * (D * 2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(kIsV ? rsrc_v : rsrc_k,
                                               (__attribute__((address_space(3))) void*)(dst + wave_lds + i * 1024),
                                               16, (kIsV ? voff_v : voff_k[i]) + roff, 0, 0, 0);
    }
  }

  // causal: a wave whose queries all precede the tile skips it
  __device__ __forceinline__ bool active(int k0) const { return !(causal && k0 > qw0 + kQ - 1); }

  // S^T = K Q^T for keys k0 .. k0+63 (two 32-key blocks) and each query block.
  // Register r of s[qb][kb] then holds key k0 + 32*kb + 8*(r/4) + 4*h + r%4 for
  // query my_q(qb).  A window of kWin K operand reads is in flight: read r+kWin
  // goes out once the MFMAs of read r have been issued (they have read their
  // operands by then).
  __device__ __forceinline__ void scores(const uint8_t* ks_, f32x16 (&s)[QB][2]) const {
    const uint32_t base = lds_addr(ks_);
    constexpr int kWin = 4;
    constexpr int kReads = 2 * kKSteps;
    u32x4 a[kReads];
#pragma unroll
    for (int r = 0; r < kWin; ++r) a[r] = lds_read_b128(base + kaddr[r % kKSteps], (r / kKSteps) * 32 * (D * 2));
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      s[qb][0] = f32x16{};
      s[qb][1] = f32x16{};
    }
#pragma unroll
    for (int r = 0; r < kReads; ++r) {
      lds_wait(a[r], r + kWin <= kReads ? kWin - 1 : kReads - 1 - r);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        s[qb][r / kKSteps] = mfma_bf16(a[r], qreg[qb][r % kKSteps], s[qb][r / kKSteps]);
      }
      if (r + kWin < kReads) {
        a[r + kWin] = lds_read_b128(base + kaddr[(r + kWin) % kKSteps], ((r + kWin) / kKSteps) * 32 * (D * 2));
      }
    }
  }

  // Probability iteration i (0..15) of query block qb: the two values of registers
  // 8u + 2w and 8u + 2w + 1 of score block kb (i = 8kb + 4u + w), as in probs.
  __device__ __forceinline__ void prob_pair(int qb, int i, const f32x16 (&sp)[2], float neg_m, u32x4 (&pb)[2][2],
                                            float& rs) const {
    const int kb = i >> 3, u = (i >> 2) & 1, w = i & 3;
    const float e0 = __builtin_amdgcn_exp2f(fmaf(sp[kb][8 * u + 2 * w], scale_log2, neg_m));
    const float e1 = __builtin_amdgcn_exp2f(fmaf(sp[kb][8 * u + 2 * w + 1], scale_log2, neg_m));
    rs += e0;
    rs += e1;
    pb[kb][u][w] = pack_bf16(e0, e1);
  }

  // The clean step's two streams in one: S^T = K Q^T of the next tile (into s, as
  // scores) and the probabilities of this tile (from sp, as probs, sums into rs), with
  // the probability iterations spread between the MFMAs (kPer after each K operand's
  // MFMAs).  Each chunk (operand wait, MFMAs, exp2 work, next operand read) is pinned
  // with a scheduling barrier, so the wave issues its exp2 work while its MFMAs run
  // instead of before them.  Values and summation order are those of probs and scores.
  __device__ __forceinline__ void scores_probs(const uint8_t* ks_, f32x16 (&s)[QB][2], const f32x16 (&sp)[QB][2],
                                               u32x4 (&pb)[QB][2][2], float (&rs)[QB]) const {
    const uint32_t base = lds_addr(ks_);
    constexpr int kWin = 4;
    constexpr int kReads = 2 * kKSteps;
    constexpr int kIters = 16 * QB;
    static_assert(kIters % kReads == 0, "probability iterations per K operand");
    constexpr int kPer = kIters / kReads;
    float neg_m[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      neg_m[qb] = m_run[qb] == -INFINITY ? 0.f : -m_run[qb];
      rs[qb] = 0.f;
      s[qb][0] = f32x16{};
      s[qb][1] = f32x16{};
    }
    u32x4 a[kReads];
#pragma unroll
    for (int r = 0; r < kWin; ++r) a[r] = lds_read_b128(base + kaddr[r % kKSteps], (r / kKSteps) * 32 * (D * 2));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < kReads; ++r) {
      lds_wait(a[r], r + kWin <= kReads ? kWin - 1 : kReads - 1 - r);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        s[qb][r / kKSteps] = mfma_bf16(a[r], qreg[qb][r % kKSteps], s[qb][r / kKSteps]);
      }
#pragma unroll
      for (int t = 0; t < kPer; ++t) {
        const int it = r * kPer + t;
        prob_pair(it / 16, it % 16, sp[it / 16], neg_m[it / 16], pb[it / 16], rs[it / 16]);
      }
      if (r + kWin < kReads) {
        a[r + kWin] = lds_read_b128(base + kaddr[(r + kWin) % kKSteps], ((r + kWin) / kKSteps) * 32 * (D * 2));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Keys >= S and (causal) keys after the query score -inf.
  __device__ __forceinline__ void mask(f32x16 (&s)[QB][2], int k0) const {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const bool need_mask = (k0 + BKV > S) || (causal && k0 + BKV - 1 > qw0 + qb * 32);
      if (need_mask) {
        const int q = my_q(qb);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + kb * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
            if (key >= S || (causal && key > q)) s[qb][kb][r] = -INFINITY;
          }
        }
      }
    }
  }

  // Tile max of the raw scores of one query block over both lane halves, times
  // scale_log2 (sm_scale > 0, so the max of the scaled scores is the scaled max).
  __device__ __forceinline__ float tile_max(const f32x16 (&s)[2]) const {
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    return fmaxf(mt, other_half(mt)) * scale_log2;
  }

  // The reference point of query block qb moves up to the tile max mt wherever
  // that exceeds it: on the first tile, and on the rare tile whose
  // probabilities relative to the current reference point come out too large
  // (see fa_step).  O and l are rescaled by the same factor.
  __device__ __forceinline__ void raise(int qb, float mt) {
    const bool upd = mt > m_run[qb];
    const float alpha = upd ? __builtin_amdgcn_exp2f(m_run[qb] - mt) : 1.0f;
    if (upd) m_run[qb] = mt;
    l_part[qb] *= alpha;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) acc_o[qb][db] *= alpha;
  }

  // P^T operands of query block qb: exp2(s * scale_log2 - m_run) rounded to
  // bf16.  Block kb, step u uses registers 8u..8u+7, i.e. keys 32kb + 16u + 4h +
  // {0..3} and 32kb + 16u + 8 + 4h + {0..3}.  Returns this lane's sum of the
  // tile's probabilities (fp32, before rounding).
  __device__ __forceinline__ float probs(int qb, const f32x16 (&s)[2], u32x4 (&pb)[2][2]) const {
    const float neg_m = m_run[qb] == -INFINITY ? 0.f : -m_run[qb];
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float e0 = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * u + 2 * w], scale_log2, neg_m));
          const float e1 = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * u + 2 * w + 1], scale_log2, neg_m));
          rs += e0;
          rs += e1;
          pb[kb][u][w] = pack_bf16(e0, e1);
        }
    return rs;
  }

  // V^T operand r of the tile (d block r / 4, keys 16 * (r % 4) .. +15): the
  // tile rows 16 * (r % 4) + {0, 8}, two transpose reads.
  __device__ __forceinline__ u32x4 vt_read(uint32_t base, int r) const {
    const int db = r / 4, row = (r % 4) * 16;
    const u32x2 lo = lds_read_tr16_b64(base + vaddr[db], row * (D * 2));
    const u32x2 hi = lds_read_tr16_b64(base + vaddr[db], (row + 8) * (D * 2));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  }

  // O^T += V^T P^T for every query block; V^T comes from transpose reads of the
  // row-major V tile, a window of kWin operands in flight: operand r+kWin is
  // read once the MFMAs of operand r have been issued.
  __device__ __forceinline__ void pv(const uint8_t* vs_, const u32x4 (&pb)[QB][2][2]) {
    const uint32_t base = lds_addr(vs_);
    constexpr int kWin = 4;
    constexpr int kOps = 4 * kDBlocks;
    u32x4 a[kOps];
#pragma unroll
    for (int r = 0; r < kWin; ++r) a[r] = vt_read(base, r);
#pragma unroll
    for (int r = 0; r < kOps; ++r) {
      lds_wait(a[r], 2 * (r + kWin <= kOps ? kWin - 1 : kOps - 1 - r));
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        acc_o[qb][r / 4] = mfma_bf16(a[r], pb[qb][(r % 4) >> 1][r & 1], acc_o[qb][r / 4]);
      }
      if (r + kWin < kOps) a[r + kWin] = vt_read(base, r + kWin);
    }
  }
};

// One pipeline step for key tile j.  K and V each stream through a ring of
// three LDS stages, tile t in stage t % 3.  On entry LDS holds K_{j+1} and V_j,
// and sc holds the masked scores of tile j; K_{j+2} and V_{j+1} may still be in
// flight.  The step requests V_{j+2} and K_{j+3} into the stages read in the
// previous step, overlaps the exp2 of tile j with the S^T MFMAs of tile j+1
// (into sn), and multiplies P_j V_j.  At its end every wave waits for its loads
// of the previous step (those of this step stay in flight for a whole step
// more) and its LDS reads, and the workgroup meets.
// The reference point m_run is not moved per tile: the probabilities of tile j
// are taken against the current one, and only when a lane's sum over the tile
// exceeds kTileSumLimit (a score above the reference point by more than about
// 11 in log2 units) does the wave take the tile max, move the reference point
// and take them again.  kGuard false (a clean step): tiles j+1 .. j+3 exist,
// every wave is active for tiles j and j+1, and tile j+1 needs no mask -- the
// caller guarantees it.  `ring` is the LDS ring base (K stages 0-2, V stages
// 3-5), `c` = j % 3.
template <int D, int kWaves, int QB, bool kGuard>
__device__ __forceinline__ void fa_step(FaState<D, kWaves, QB>& st, int j, int n_tiles, uint8_t* ring, int c,
                                        f32x16 (&sc)[QB][2], f32x16 (&sn)[QB][2]) {
  using St = FaState<D, kWaves, QB>;
  constexpr int T = St::kTileBytes;
  constexpr int L = St::kLoadsPerWave;
  const int c1 = c == 2 ? 0 : c + 1;  // (j + 1) % 3
  const int c2 = c == 0 ? 2 : c - 1;  // (j + 2) % 3
  const int k1 = (j + 1) * BKV;
  const bool has_next = !kGuard || j + 1 < n_tiles;
  const bool act = !kGuard || st.active(j * BKV);
  const bool act_next = !kGuard || (has_next && st.active(k1));
  const bool load_v = !kGuard || j + 2 < n_tiles;
  const bool load_k = !kGuard || j + 3 < n_tiles;
  if (load_v) st.template load_tile<true>(ring + (3 + c2) * T, k1 + BKV);
  if (load_k) st.template load_tile<false>(ring + c * T, k1 + 2 * BKV);
  u32x4 pb[QB][2][2];
  float rs[QB];
  if constexpr (!kGuard) {
    st.scores_probs(ring + c1 * T, sn, sc, pb, rs);  // both streams, interleaved
  } else if (act_next) {  // a wave active for tile j+1 is active for tile j
    st.scores_probs(ring + c1 * T, sn, sc, pb, rs);
    st.mask(sn, k1);
  } else if (act) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) rs[qb] = st.probs(qb, sc[qb], pb[qb]);
  }
  if (act) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (__builtin_amdgcn_ballot_w64(rs[qb] > kTileSumLimit) != 0) {
        st.raise(qb, st.tile_max(sc[qb]));
        rs[qb] = st.probs(qb, sc[qb], pb[qb]);
      }
      st.l_part[qb] += rs[qb];
    }
    st.pv(ring + (3 + c) * T, pb);
  }
  if (load_v && load_k) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * L) : "memory");
  } else if (load_v || load_k) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(L) : "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  }
  asm volatile("s_barrier" ::: "memory");
}

// Configurations.  head_dim 128: one workgroup of 8 waves (256 queries) per CU,
// each K/V tile streamed once for 256 queries; the two waves of a SIMD belong
// to one workgroup and would run their exp2 and MFMA phases in lockstep, so
// waves 0-3 run at raised priority and their SIMD partners fill in behind them.
// (4 waves of 64 queries each, QB = 2, halve the LDS reads per MFMA but leave
// one wave per SIMD with nothing to overlap its MFMAs with: 1025 against 950 us
// at the bench shape, measured with the rare rescale path left out -- with it
// the kernel does not fit the register file.)  head_dim 64: 4 waves of 32 queries, two workgroups per
// CU, whose waves share each SIMD and drift apart.
template <int D>
struct FaConfig;
template <>
struct FaConfig<128> {
  static constexpr int kWaves = 8, QB = 1, kWgPerCu = 1;
};
template <>
struct FaConfig<64> {
  static constexpr int kWaves = 4, QB = 1, kWgPerCu = 2;
};

// The attention of one workgroup: query block and (batch, head) from the block index.
template <int D>
__device__ __forceinline__ void fa_fwd_body(const FaArgs& p) {
  constexpr int kWaves = FaConfig<D>::kWaves;
  constexpr int QB = FaConfig<D>::QB;
  using St = FaState<D, kWaves, QB>;
  constexpr int kTileBytes = St::kTileBytes;
  constexpr int kChunks = St::kChunks;
  constexpr int kKSteps = St::kKSteps;
  constexpr int kDBlocks = St::kDBlocks;
  constexpr int kThreads = kWaves * 64;
  constexpr int BQ = St::kQ * kWaves;  // queries per workgroup
  // K ring (stages 0-2) and V ring (stages 3-5).  LDS reads of the rings are
  // inline asm with explicit waits, so no compiler alias analysis between DMA
  // and reads is involved.
  __shared__ __attribute__((aligned(16))) uint8_t ring[6 * kTileBytes];

  St st;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  if (kWaves == 8 && (tid >> 6) < 4) __builtin_amdgcn_s_setprio(1);
  st.lane = lane;
  st.wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  st.col = lane & 31;  // query column within a query block
  st.h = lane >> 5;    // lane half
  const int wave = st.wave, col = st.col, h = st.h;

  // Block order.  Workgroup b runs on XCD b % 8, and each XCD starts its
  // workgroups in order of b / 8.  When the (batch, head) count divides by 8,
  // XCD x takes heads x, x+8, x+16, ... in groups of head_group heads and runs
  // the query blocks of one group back to back, interleaving the group's heads
  // block by block.  The workgroups resident on an XCD at once then stream the
  // same few heads' K/V through that XCD's L2 (fetched from HBM about once per
  // head, instead of once per round of resident query blocks).  Non-causal
  // blocks are all alike and use groups of one head.  Causal blocks run heavy
  // (late) query blocks first, and the host sizes the group so that one group's
  // blocks fill the workgroup slots of the XCD twice over: the heaviest blocks of
  // a group then start together and the lightest end the XCD's run, instead of
  // the last head's heavy blocks starting behind the previous head's light ones.
  // Otherwise: query-block major (heavy first over all heads when causal).
  const int64_t bid = blockIdx.x;
  int64_t bh;
  int qblk;
  if (p.heads_total % 8 == 0) {
    const int64_t slot = bid >> 3;  // < heads_total / 8 * n_qblocks
    const int64_t per_group = static_cast<int64_t>(p.head_group) * p.n_qblocks;
    const int64_t grp = slot / per_group;
    const int64_t r = slot - grp * per_group;
    const int64_t g0 = grp * p.head_group;
    const int64_t heads_left = (p.heads_total >> 3) - g0;  // >= 1; the last group may be partial
    const int64_t gsz = heads_left < p.head_group ? heads_left : p.head_group;
    bh = (bid & 7) + 8 * (g0 + r % gsz);
    qblk = static_cast<int>(r / gsz);
  } else {
    bh = bid % p.heads_total;
    qblk = static_cast<int>(bid / p.heads_total);
  }
  if (p.causal) qblk = p.n_qblocks - 1 - qblk;
  const int q0 = qblk * BQ;
  const int S = p.seq;
  const int64_t head_off = bh * static_cast<int64_t>(S) * D;
  const uint16_t* Qh = p.q + head_off;
  st.q0 = q0;
  st.S = S;
  st.causal = p.causal;
  st.scale_log2 = p.scale_log2;
  st.qw0 = q0 + wave * St::kQ;

  // Q^T operand of query block qb: lane (query col, half h) holds
  // Q[my_q(qb)][16*ks + 8h .. +8]
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int q = st.my_q(qb);
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
      if (q < S) {
        st.qreg[qb][ks] = *reinterpret_cast<const u32x4*>(Qh + static_cast<int64_t>(q) * D + ks * 16 + h * 8);
      } else {
        st.qreg[qb][ks] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < kDBlocks; ++i) st.acc_o[qb][i] = f32x16{};
    st.m_run[qb] = -INFINITY;
    st.l_part[qb] = 0.f;
  }

  int kv_end = S;
  if (p.causal) kv_end = min(S, q0 + BQ);
  const int n_tiles = (kv_end + BKV - 1) / BKV;

  // K_0, V_0 and K_1 are needed first; V_1 and K_2 (step 1) may land later
  st.init_loads(p.k + head_off, p.v + head_off);
  constexpr int L = St::kLoadsPerWave;
  st.template load_tile<false>(ring, 0);
  st.template load_tile<true>(ring + 3 * kTileBytes, 0);
  if (n_tiles > 1) {
    st.template load_tile<false>(ring + kTileBytes, BKV);
    st.template load_tile<true>(ring + 4 * kTileBytes, BKV);
  }
  if (n_tiles > 2) {
    st.template load_tile<false>(ring + 2 * kTileBytes, 2 * BKV);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * L) : "memory");
  } else if (n_tiles > 1) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L) : "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  asm volatile("s_barrier" ::: "memory");
  f32x16 sa[QB][2], sb[QB][2];
  st.scores(ring, sa);  // tile 0 is active for every wave
  // step 0 refills stage 0 with K_3: every wave must be done reading K_0
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  asm volatile("s_barrier" ::: "memory");
  st.mask(sa, 0);
  // Key 0 is never masked, so the reference points are finite from here on.
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) st.raise(qb, st.tile_max(sa[qb]));
  // Clean tiles need no mask and are active for every wave: all their keys are
  // < S and, for causal, precede the block's first query q0.  Step j is clean
  // when tile j+1 is and tiles up to j+3 exist; the clean steps run as pairs,
  // the rest (at most seven: n_tiles - n_clean <= 4 for BQ = 256) guarded.
  // c = j % 3 is the ring stage of tile j.
  const int n_clean = p.causal ? min(q0 / BKV, S / BKV) : S / BKV;
  int j = 0, c = 0;
  for (; j + 4 < n_clean; j += 2) {
    fa_step<D, kWaves, QB, false>(st, j, n_tiles, ring, c, sa, sb);
    c = c == 2 ? 0 : c + 1;
    fa_step<D, kWaves, QB, false>(st, j + 1, n_tiles, ring, c, sb, sa);
    c = c == 2 ? 0 : c + 1;
  }
  for (; j < n_tiles; j += 2) {
    fa_step<D, kWaves, QB, true>(st, j, n_tiles, ring, c, sa, sb);
    c = c == 2 ? 0 : c + 1;
    if (j + 1 < n_tiles) fa_step<D, kWaves, QB, true>(st, j + 1, n_tiles, ring, c, sb, sa);
    c = c == 2 ? 0 : c + 1;
  }

  // ---- epilogue: O = O^T / l, transposed through LDS (the rings, free after
  //      the last step's barrier: no load is in flight then) into row-major
  //      bf16.  Lane holds query my_q(qb) and, for d block db and register r,
  //      d = 32*db + 8*(r/4) + 4*h + r%4.  Block rows 64*g .. 64*g+63 go to
  //      ring stage g.
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float l_run = st.l_part[qb] + other_half(st.l_part[qb]);
    const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
    const int brow = wave * St::kQ + qb * 32 + col;  // row within the workgroup's block
    uint8_t* os_ = ring + (brow >> 6) * kTileBytes;
    const int row = brow & 63;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = db * 32 + rq * 8 + h * 4;
        u32x2 w;
        w[0] = pack_bf16(st.acc_o[qb][db][rq * 4 + 0] * inv_l, st.acc_o[qb][db][rq * 4 + 1] * inv_l);
        w[1] = pack_bf16(st.acc_o[qb][db][rq * 4 + 2] * inv_l, st.acc_o[qb][db][rq * 4 + 3] * inv_l);
        *reinterpret_cast<u32x2*>(os_ + k_off<D>(row, d >> 3) + (d & 7) * 2) = w;
      }
    }
    const int q = st.my_q(qb);
    if (p.lse != nullptr && h == 0 && q < S) {
      p.lse[bh * S + q] = (st.m_run[qb] + __log2f(l_run)) * 0.69314718055994530942f;
    }
  }
  __syncthreads();
  uint16_t* Oh = p.o + head_off;
#pragma unroll
  for (int i = 0; i < BQ * kChunks / kThreads; ++i) {
    const int cc = tid + kThreads * i;
    const int row = cc / kChunks, ch = cc % kChunks;
    const uint8_t* os_ = ring + (row >> 6) * kTileBytes;
    const int q = q0 + row;
    if (q < S) {
      *reinterpret_cast<u32x4*>(Oh + static_cast<int64_t>(q) * D + ch * 8) =
          *reinterpret_cast<const u32x4*>(os_ + k_off<D>(row & 63, ch));
    }
  }
}

}  // namespace fa
}  // namespace asc

// Defines the attention kernels as PREFIX##d64 / PREFIX##d128 (head_dim 64 / 128),
// each taking one asc::fa::FaArgs by value, with the given linkage specifier.
#define ASC_FA_KERNEL(LINKAGE, NAME, D)                                                                            \
  LINKAGE __global__ void __launch_bounds__(asc::fa::FaConfig<D>::kWaves * 64, asc::fa::FaConfig<D>::kWgPerCu)    \
      NAME(asc::fa::FaArgs p) {                                                                                    \
    asc::fa::fa_fwd_body<D>(p);                                                                                    \
  }
#define ASC_FA_KERNELS(LINKAGE, PREFIX) \
  ASC_FA_KERNEL(LINKAGE, PREFIX##d64, 64)  \
  ASC_FA_KERNEL(LINKAGE, PREFIX##d128, 128)
