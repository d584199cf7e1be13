// Flash-attention forward, bf16 in/out, fp32 online-softmax statistics.
// The reference has no attention kernel; this is the build's asc2-style
// flash_attention_fwd_kernel (BASELINE config: batch 4, 32 heads, seq 4096,
// head_dim 128, scale 1/sqrt(128), causal and non-causal).
//
// Design (gfx950, wave64, MFMA 32x32x16 bf16):
//  - A wave owns 32 queries of one (batch, head); a workgroup has 4 waves
//    (128 queries; head_dim 64) or 8 waves (256 queries; head_dim 128).  Keys/values stream through LDS in tiles of 64,
//    double-buffered.
//  - Each wave computes S^T = K Q^T (keys x queries) instead of S = Q K^T:
//    in the MFMA result layout a lane then holds ONE query column and 16 keys
//    per 32x32 block, so the online-softmax max/sum of a query live in two
//    lanes (lane and lane^32) -- one cross-lane shuffle per statistic.
//  - O^T = V^T P^T: P^T is the B operand straight from the S^T registers (no
//    data movement; A and B agree on which key each operand slot holds), V^T is
//    read from the row-major V tile with ds_read_b64_tr_b16 (gfx950 LDS
//    transpose read).  Q^T stays in registers for the whole kernel.
//  - Online softmax in the exp2 domain: the max is taken on raw scores and
//    scale*log2(e) and the shift fold into one FMA before exp2; the reference
//    point only moves when a tile max exceeds it by more than 8 (exact
//    arithmetic either way, O and l are rescaled rarely); causal tiles above
//    the diagonal are skipped and the diagonal tile is masked; heavy (late)
//    query blocks are scheduled first.
// LDS tiles use XOR-swizzled 16-byte chunks so that both the MFMA operand
// reads and the transpose reads are free of bank conflicts.
#include <math.h>

#include "common.h"
#include "numeric.h"

namespace {

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

// Largest exponent (log2 domain) an unnormalised probability may reach before
// the running max is moved; bounds exp2 values by 2^8.
constexpr float kRescaleSlack = 8.0f;

// Per-wave state of the attention kernel (a wave owns 32 queries; a workgroup
// of kWaves waves owns 32*kWaves).
template <int D, int kWaves>
struct FaState {
  static constexpr int kChunks = D / 8;           // 16-byte chunks per row
  static constexpr int kTileBytes = BKV * D * 2;  // one K or V tile
  static constexpr int kKSteps = D / 16;          // MFMA k-steps over head_dim
  static constexpr int kDBlocks = D / 32;         // 32-wide d blocks of O^T
  static constexpr int kRowsPerLoad = 1024 / (D * 2);     // tile rows per 1 KiB wave load
  static constexpr int kLoadsPerWave = BKV / kRowsPerLoad / kWaves;  // per tile

  int lane, wave, col, h;
  int q0, S, my_q, wave_qmax, causal;
  float scale_log2;
  __amdgpu_buffer_rsrc_t rsrc_k, rsrc_v;
  int voff_k[4], voff_v;  // voff_k[i]: this wave's i-th K load (kLoadsPerWave <= 4)
  // Per-lane LDS read offsets, loop-invariant: the K swizzle of row kb*32+col
  // equals that of row col, and the V swizzle of row r0+j (r0 % 4 == 0) equals
  // that of row j, so every other term of a read address is an immediate.
  uint32_t kaddr[kKSteps];   // K row col, chunk 2*kk+h
  uint32_t vaddr[kDBlocks];  // V transpose read of d block db, rows 4h+j
  u32x4 qreg[kKSteps];
  f32x16 acc_o[kDBlocks];
  float m_run;   // reference point of the scaled scores (log2 domain), <= running max
  float l_part;  // this lane half's share of the running sum of exp2(s*scale_log2 - m_run)

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
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) {
      const int R = wave * kLoadsPerWave + i;
      // the row offset goes into the per-lane offset, not the SGPR offset: the
      // buffer range check (keys >= S read as zero) only covers the former
      const int roff = (k0 + kRowsPerLoad * R) * (D * 2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(kIsV ? rsrc_v : rsrc_k,
                                               (__attribute__((address_space(3))) void*)(dst + R * 1024), 16,
                                               (kIsV ? voff_v : voff_k[i]) + roff, 0, 0, 0);
    }
  }

  // causal: a wave whose queries all precede the tile skips it
  __device__ __forceinline__ bool active(int k0) const { return !(causal && k0 > wave_qmax); }

  // S^T = K Q^T for keys k0 .. k0+63 (two 32-key blocks).  Register r of block
  // kb then holds key k0 + 32*kb + 8*(r/4) + 4*h + r%4 for query my_q.
  // The kKSteps operand reads of a block go out together; each MFMA waits only
  // for its own.
  __device__ __forceinline__ void scores(const uint8_t* ks_, f32x16 (&s)[2]) const {
    const uint32_t base = lds_addr(ks_);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x16{};
      u32x4 a[kKSteps];
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) a[kk] = lds_read_b128(base + kaddr[kk], kb * 32 * (D * 2));
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        lds_wait(a[kk], kKSteps - 1 - kk);
        s[kb] = mfma_bf16(a[kk], qreg[kk], s[kb]);
      }
    }
  }

  // Keys >= S and (causal) keys after the query score -inf.
  __device__ __forceinline__ void mask(f32x16 (&s)[2], int k0) const {
    const bool need_mask = (k0 + BKV > S) || (causal && k0 + BKV - 1 > q0 + wave * 32);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + kb * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
          if (key >= S || (causal && key > my_q)) s[kb][r] = -INFINITY;
        }
      }
    }
  }

  // Tile max of the raw scores over both lane halves, times scale_log2
  // (sm_scale > 0, so the max of the scaled scores is the scaled max).
  __device__ __forceinline__ float tile_max(const f32x16 (&s)[2]) const {
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    return fmaxf(mt, other_half(mt)) * scale_log2;
  }

  // Lazy rescale: the reference point m_run only moves when the tile max
  // exceeds it by more than kRescaleSlack (log2 units), so exp2 values stay
  // below 2^kRescaleSlack and O / l are rescaled rarely.  The branch is
  // wave-uniform (any lane that needs it).
  __device__ __forceinline__ void rebase(float mt) {
    const bool upd = mt > m_run + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(upd) != 0) {
      const float alpha = upd ? __builtin_amdgcn_exp2f(m_run - mt) : 1.0f;
      if (upd) m_run = mt;
      l_part *= alpha;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) acc_o[db] *= alpha;
    }
  }

  // P^T operands: exp2(s * scale_log2 - m_run) rounded to bf16.  Block kb, step
  // u uses registers 8u..8u+7, i.e. keys 32kb + 16u + 4h + {0..3} and
  // 32kb + 16u + 8 + 4h + {0..3}.
  __device__ __forceinline__ void probs(const f32x16 (&s)[2], u32x4 (&pb)[2][2]) {
    const float neg_m = m_run == -INFINITY ? 0.f : -m_run;
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
    l_part += rs;
  }

  // V^T operands of d block db: for (kb, u) the rows kb*32 + u*16 + {0, 8}
  // of the tile, four MFMA A operands of two transpose reads each.
  __device__ __forceinline__ void vt_reads(uint32_t base, int db, u32x4 (&a)[4]) const {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const u32x2 lo = lds_read_tr16_b64(base + vaddr[db], (kb * 32 + u * 16) * (D * 2));
        const u32x2 hi = lds_read_tr16_b64(base + vaddr[db], (kb * 32 + u * 16 + 8) * (D * 2));
        a[kb * 2 + u] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
  }

  // O^T += V^T P^T; V^T comes from transpose reads of the row-major V tile.
  // The reads of d block db+1 are in flight while block db multiplies.
  __device__ __forceinline__ void pv(const uint8_t* vs_, const u32x4 (&pb)[2][2]) {
    const uint32_t base = lds_addr(vs_);
    u32x4 a[2][4];
    vt_reads(base, 0, a[0]);
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
      u32x4(&cur)[4] = a[db & 1];
      if (db + 1 < kDBlocks) {
        vt_reads(base, db + 1, a[(db + 1) & 1]);
        lds_wait(cur, 8);  // the newest 8 reads belong to block db+1
      } else {
        lds_wait(cur, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) acc_o[db] = mfma_bf16(cur[i], pb[i >> 1][i & 1], acc_o[db]);
    }
  }
};

// One pipeline step for key tile j.  On entry LDS holds K_{j+1} (k_next) and
// V_j (v_cur), and sc holds the masked scores of tile j with m_run already
// rebased for them.  The step streams V_{j+1} and K_{j+2} into the stages freed
// by the previous step, then overlaps the exp2 of tile j with the S^T MFMAs of
// tile j+1, and the P.V MFMAs of tile j with the max of tile j+1.  kGuard
// false (a clean step): tile j+1 exists, every wave is active for tiles j and
// j+1, and tile j+1 needs no mask -- the caller guarantees it.
template <int D, int kWaves, bool kGuard>
__device__ __forceinline__ void fa_step(FaState<D, kWaves>& st, int j, int n_tiles, uint8_t* k_load, uint8_t* v_load,
                                        const uint8_t* k_next, const uint8_t* v_cur, f32x16 (&sc)[2],
                                        f32x16 (&sn)[2]) {
  const int k1 = (j + 1) * BKV;
  const bool has_next = !kGuard || j + 1 < n_tiles;
  const bool act = !kGuard || st.active(j * BKV);
  const bool act_next = !kGuard || (has_next && st.active(k1));
  if (has_next) st.template load_tile<true>(v_load, k1);
  if (j + 2 < n_tiles) st.template load_tile<false>(k_load, k1 + BKV);
  u32x4 pb[2][2];
  if (act) st.probs(sc, pb);
  if (act_next) st.scores(k_next, sn);
  if (kGuard && act_next) st.mask(sn, k1);
  if (act) st.pv(v_cur, pb);
  const float mt = act_next ? st.tile_max(sn) : -INFINITY;
  // a wave waits for its own loads and LDS reads only, then the workgroup
  // meets (a plain s_barrier: __syncthreads' fence would drain more)
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  asm volatile("s_barrier" ::: "memory");
  if (act_next) st.rebase(mt);
}

// kWaves = 4: two workgroups per CU, the two waves of a SIMD come from different
// workgroups and drift apart.  kWaves = 8: one workgroup of 256 queries per CU,
// each K/V tile streamed once for twice the queries (half the DMA per query);
// the two waves of a SIMD belong to one workgroup and would run their exp2 and
// MFMA phases in lockstep, so waves 0-3 run at raised priority and their SIMD
// partners fill in behind them (non-causal +3.6% over kWaves = 4; causal with
// the grouped block order 1.5-2% faster than with 128-query blocks).
template <int D, int kWaves>
__global__ void __launch_bounds__(kWaves * 64, 8 / kWaves) fa_fwd_kernel(FaArgs p) {
  using St = FaState<D, kWaves>;
  constexpr int kTileBytes = St::kTileBytes;
  constexpr int kChunks = St::kChunks;
  constexpr int kKSteps = St::kKSteps;
  constexpr int kDBlocks = St::kDBlocks;
  constexpr int kThreads = kWaves * 64;
  constexpr int BQ = 32 * kWaves;  // queries per workgroup
  // K and V rings of two stages each, as distinct objects, so the compiler can
  // tell that loads into one stage do not alias reads of another.  K runs one
  // tile ahead of V.
  __shared__ __attribute__((aligned(16))) uint8_t kst0[kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t kst1[kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vst0[kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vst1[kTileBytes];

  St st;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  if (kWaves == 8 && (tid >> 6) < 4) __builtin_amdgcn_s_setprio(1);
  st.lane = lane;
  st.wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  st.col = lane & 31;  // query column within the wave's 32
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
  int qb;
  if (p.heads_total % 8 == 0) {
    const int64_t slot = bid >> 3;  // < heads_total / 8 * n_qblocks
    const int64_t per_group = static_cast<int64_t>(p.head_group) * p.n_qblocks;
    const int64_t grp = slot / per_group;
    const int64_t r = slot - grp * per_group;
    const int64_t g0 = grp * p.head_group;
    const int64_t heads_left = (p.heads_total >> 3) - g0;  // >= 1; the last group may be partial
    const int64_t gsz = heads_left < p.head_group ? heads_left : p.head_group;
    bh = (bid & 7) + 8 * (g0 + r % gsz);
    qb = static_cast<int>(r / gsz);
  } else {
    bh = bid % p.heads_total;
    qb = static_cast<int>(bid / p.heads_total);
  }
  if (p.causal) qb = p.n_qblocks - 1 - qb;
  const int q0 = qb * BQ;
  const int S = p.seq;
  const int64_t head_off = bh * static_cast<int64_t>(S) * D;
  const uint16_t* Qh = p.q + head_off;
  st.q0 = q0;
  st.S = S;
  st.causal = p.causal;
  st.scale_log2 = p.scale_log2;
  st.my_q = q0 + wave * 32 + col;
  st.wave_qmax = q0 + wave * 32 + 31;
  const int my_q = st.my_q;

  // Q^T operand: lane (query col, half h) holds Q[my_q][16*ks + 8h .. +8]
#pragma unroll
  for (int ks = 0; ks < kKSteps; ++ks) {
    if (my_q < S) {
      st.qreg[ks] = *reinterpret_cast<const u32x4*>(Qh + static_cast<int64_t>(my_q) * D + ks * 16 + h * 8);
    } else {
      st.qreg[ks] = u32x4{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int i = 0; i < kDBlocks; ++i) st.acc_o[i] = f32x16{};
  st.m_run = -INFINITY;
  st.l_part = 0.f;

  int kv_end = S;
  if (p.causal) kv_end = min(S, q0 + BQ);
  const int n_tiles = (kv_end + BKV - 1) / BKV;

  st.init_loads(p.k + head_off, p.v + head_off);
  st.template load_tile<false>(kst0, 0);
  st.template load_tile<true>(vst0, 0);
  if (n_tiles > 1) st.template load_tile<false>(kst1, BKV);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  asm volatile("s_barrier" ::: "memory");
  f32x16 sa[2], sb[2];
  st.scores(kst0, sa);  // tile 0 is active for every wave
  // step 0 refills kst0 with tile 2: every wave must be done reading tile 0
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  asm volatile("s_barrier" ::: "memory");
  st.mask(sa, 0);
  st.rebase(st.tile_max(sa));
  // Clean tiles need no mask and are active for every wave: all their keys are
  // < S and, for causal, precede the block's first query q0.  Step j is clean
  // when tile j+1 is; the clean steps run as pairs, the rest (at most four:
  // n_tiles - n_clean <= 2) guarded.  Tile j lives in stage j % 2 of each ring.
  const int n_clean = p.causal ? min(q0 / BKV, S / BKV) : S / BKV;
  int j = 0;
  for (; j + 2 < n_clean; j += 2) {
    fa_step<D, kWaves, false>(st, j, n_tiles, kst0, vst1, kst1, vst0, sa, sb);
    fa_step<D, kWaves, false>(st, j + 1, n_tiles, kst1, vst0, kst0, vst1, sb, sa);
  }
  for (; j < n_tiles; j += 2) {
    fa_step<D, kWaves, true>(st, j, n_tiles, kst0, vst1, kst1, vst0, sa, sb);
    if (j + 1 < n_tiles) fa_step<D, kWaves, true>(st, j + 1, n_tiles, kst1, vst0, kst0, vst1, sb, sa);
  }

  // ---- epilogue: O = O^T / l, transposed through LDS (the K ring, free after
  //      the last step's barrier) into row-major bf16.  Lane holds query my_q
  //      and, for d block db and register r, d = 32*db + 8*(r/4) + 4*h + r%4.
  //      Block rows 0..63 go to kst0, 64..127 to kst1, 128..191 to vst0,
  //      192..255 to vst1 (all four stages are free after the last barrier).
  const float l_run = st.l_part + other_half(st.l_part);
  const float m_run = st.m_run;
  const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
  {
    const int sg = wave >> 1;
    uint8_t* os_ = sg == 0 ? kst0 : sg == 1 ? kst1 : sg == 2 ? vst0 : vst1;
    const int row = (wave & 1) * 32 + col;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = db * 32 + rq * 8 + h * 4;
        u32x2 w;
        w[0] = pack_bf16(st.acc_o[db][rq * 4 + 0] * inv_l, st.acc_o[db][rq * 4 + 1] * inv_l);
        w[1] = pack_bf16(st.acc_o[db][rq * 4 + 2] * inv_l, st.acc_o[db][rq * 4 + 3] * inv_l);
        *reinterpret_cast<u32x2*>(os_ + k_off<D>(row, d >> 3) + (d & 7) * 2) = w;
      }
    }
  }
  if (p.lse != nullptr && h == 0 && my_q < S) {
    p.lse[bh * S + my_q] = (m_run + __log2f(l_run)) * 0.69314718055994530942f;
  }
  __syncthreads();
  uint16_t* Oh = p.o + head_off;
#pragma unroll
  for (int i = 0; i < BQ * kChunks / kThreads; ++i) {
    const int c = tid + kThreads * i;
    const int row = c / kChunks, ch = c % kChunks;
    const int sg = row >> 6;
    const uint8_t* os_ = sg == 0 ? kst0 : sg == 1 ? kst1 : sg == 2 ? vst0 : vst1;
    const int q = q0 + row;
    if (q < S) {
      *reinterpret_cast<u32x4*>(Oh + static_cast<int64_t>(q) * D + ch * 8) =
          *reinterpret_cast<const u32x4*>(os_ + k_off<D>(row & 63, ch));
    }
  }
}

template <int D, int kWaves>
int32_t launch(FaArgs p, hipStream_t stream) {
  constexpr int BQ = 32 * kWaves;
  p.n_qblocks = static_cast<int>((p.seq + BQ - 1) / BQ);
  p.head_group = 1;
  if (p.causal) {
    // workgroup slots of one XCD: its CUs x resident workgroups per CU
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) {
      return asc::set_error(static_cast<int32_t>(e), "asc_flash_attention_fwd_bf16: cannot read the CU count: %s",
                            hipGetErrorString(e));
    }
    // Twice the smallest group that fills them: at the bench shape (64 slots, 32
    // blocks per head) groups of 1, 2, 4, 8, 16 heads measured 582-621, 569-591,
    // 564-575, 572-578 and 581-586 us.
    const int64_t slots = static_cast<int64_t>(cus) / 8 * (8 / kWaves);
    const int64_t g = 2 * ((slots + p.n_qblocks - 1) / p.n_qblocks);
    const int64_t heads_xcd = p.heads_total / 8;
    p.head_group = static_cast<int>(g < 1 ? 1 : (g > heads_xcd && heads_xcd > 0 ? heads_xcd : g));
  }
  const int64_t blocks = p.heads_total * p.n_qblocks;
  // one workgroup per (head, query block): the grid's x dimension and its thread count
  // (blocks x kWaves x 64) must fit 32 bits
  ASC_REQUIRE(blocks <= (int64_t{1} << 31) - 1 && blocks * kWaves * 64 < (int64_t{1} << 32), ASC_ERR_UNSUPPORTED,
              "asc_flash_attention_fwd_bf16: %lld heads x %d query blocks exceed the launch grid limit",
              static_cast<long long>(p.heads_total), p.n_qblocks);
  hipLaunchKernelGGL((fa_fwd_kernel<D, kWaves>), dim3(static_cast<uint32_t>(blocks)), dim3(kWaves * 64), 0, stream,
                     p);
  return asc::check_launch("asc_flash_attention_fwd_bf16");
}

}  // namespace

extern "C" int32_t asc_flash_attention_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                                                int64_t batch, int64_t heads, int64_t seq_len, int32_t head_dim,
                                                float sm_scale, int32_t causal, asc_stream_t stream) {
  ASC_REQUIRE(batch >= 0 && heads >= 0 && seq_len >= 0, ASC_ERR_INVALID_ARG,
              "asc_flash_attention_fwd_bf16: negative shape");
  ASC_REQUIRE(head_dim == 64 || head_dim == 128, ASC_ERR_UNSUPPORTED,
              "asc_flash_attention_fwd_bf16: head_dim %d not supported (64, 128)", head_dim);
  // K/V of one head are addressed with 32-bit buffer offsets (one tile past the end included)
  ASC_REQUIRE((seq_len + BKV) * head_dim * 2 < (int64_t{1} << 31), ASC_ERR_UNSUPPORTED,
              "asc_flash_attention_fwd_bf16: seq_len %lld too large for head_dim %d",
              static_cast<long long>(seq_len), head_dim);
  ASC_REQUIRE(sm_scale > 0.f, ASC_ERR_INVALID_ARG, "asc_flash_attention_fwd_bf16: sm_scale must be positive");
  if (batch == 0 || heads == 0 || seq_len == 0) return ASC_OK;
  ASC_REQUIRE(q && k && v && o, ASC_ERR_INVALID_ARG, "asc_flash_attention_fwd_bf16: null buffer");
  ASC_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                reinterpret_cast<uintptr_t>(o)) & 15) == 0,
              ASC_ERR_ALIGNMENT, "asc_flash_attention_fwd_bf16: buffers must be 16-byte aligned");
  FaArgs p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.heads_total = batch * heads;
  p.seq = static_cast<int>(seq_len);
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  p.causal = causal ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (head_dim == 64) return launch<64, 4>(p, s);
  return launch<128, 8>(p, s);
}
