// Flash-attention forward, bf16 in/out, fp32 online-softmax statistics.
// The reference has no attention kernel; this is the build's asc2-style
// flash_attention_fwd_kernel (BASELINE config: batch 4, 32 heads, seq 4096,
// head_dim 128, scale 1/sqrt(128), causal and non-causal).
//
// Design (gfx950, wave64, MFMA 32x32x16 bf16):
//  - A workgroup owns 128 queries of one (batch, head): 4 waves x 32 queries.
//    Keys/values stream through LDS in tiles of 64, double-buffered.
//  - Each wave computes S^T = K Q^T (keys x queries) instead of S = Q K^T:
//    in the MFMA result layout a lane then holds ONE query column and 16 keys
//    per 32x32 block, so the online-softmax max/sum of a query live in two
//    lanes (lane and lane^32) -- one cross-lane shuffle per statistic.
//  - O^T = V^T P^T: P^T is the B operand straight from the S^T registers (no
//    data movement; A and B agree on which key each operand slot holds), V^T is
//    read from the row-major V tile with ds_read_b64_tr_b16 (gfx950 LDS
//    transpose read).  Q^T stays in registers for the whole kernel.
//  - Online softmax in the exp2 domain with scale*log2(e) folded into one
//    multiply; causal tiles above the diagonal are skipped and the diagonal
//    tile is masked; heavy (late) query blocks are scheduled first.
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
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int BQ = 32 * kWaves;  // queries per workgroup
constexpr int BKV = 64;          // keys per LDS tile

struct FaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t heads_total;  // batch * heads
  int seq;
  int n_qblocks;
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

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return static_cast<uint32_t>(asc::f32_to_bf16_rne(lo)) | (static_cast<uint32_t>(asc::f32_to_bf16_rne(hi)) << 16);
}

template <int D>
__global__ void __launch_bounds__(kThreads, 2) fa_fwd_kernel(FaArgs p) {
  constexpr int kChunks = D / 8;              // 16-byte chunks per row
  constexpr int kTileBytes = BKV * D * 2;     // one K or V tile
  constexpr int kKSteps = D / 16;             // MFMA k-steps over head_dim
  constexpr int kDBlocks = D / 32;            // 32-wide d blocks of O^T
  constexpr int kLoads = BKV * kChunks / kThreads;  // 16-byte loads per thread per tile
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 2 * kTileBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // query column within the wave's 32
  const int h = lane >> 5;    // lane half

  // heavy-first order for causal: all (batch, head) of the last query block first
  const int64_t bid = blockIdx.x;
  const int64_t bh = bid % p.heads_total;
  int qb = static_cast<int>(bid / p.heads_total);
  if (p.causal) qb = p.n_qblocks - 1 - qb;
  const int q0 = qb * BQ;
  const int S = p.seq;
  const int64_t head_off = bh * static_cast<int64_t>(S) * D;
  const uint16_t* Qh = p.q + head_off;
  const uint16_t* Kh = p.k + head_off;
  const uint16_t* Vh = p.v + head_off;

  const int my_q = q0 + wave * 32 + col;
  const int wave_qmax = q0 + wave * 32 + 31;

  // Q^T operand: lane (query col, half h) holds Q[my_q][16*ks + 8h .. +8]
  u32x4 qreg[kKSteps];
#pragma unroll
  for (int ks = 0; ks < kKSteps; ++ks) {
    if (my_q < S) {
      qreg[ks] = *reinterpret_cast<const u32x4*>(Qh + static_cast<int64_t>(my_q) * D + ks * 16 + h * 8);
    } else {
      qreg[ks] = u32x4{0, 0, 0, 0};
    }
  }

  int kv_end = S;
  if (p.causal) kv_end = min(S, q0 + BQ);
  const int n_tiles = (kv_end + BKV - 1) / BKV;

  u32x4 rk[kLoads], rv[kLoads];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int c = tid + kThreads * i;
      const int row = c / kChunks, ch = c % kChunks;
      const int key = k0 + row;
      if (key < S) {
        rk[i] = *reinterpret_cast<const u32x4*>(Kh + static_cast<int64_t>(key) * D + ch * 8);
        rv[i] = *reinterpret_cast<const u32x4*>(Vh + static_cast<int64_t>(key) * D + ch * 8);
      } else {
        rk[i] = u32x4{0, 0, 0, 0};
        rv[i] = u32x4{0, 0, 0, 0};
      }
    }
  };
  auto stash = [&](int stage) {
    uint8_t* ks_ = smem + stage * 2 * kTileBytes;
    uint8_t* vs_ = ks_ + kTileBytes;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int c = tid + kThreads * i;
      const int row = c / kChunks, ch = c % kChunks;
      *reinterpret_cast<u32x4*>(ks_ + k_off<D>(row, ch)) = rk[i];
      *reinterpret_cast<u32x4*>(vs_ + v_off<D>(row, ch * 8)) = rv[i];
    }
  };

  f32x16 acc_o[kDBlocks];
#pragma unroll
  for (int i = 0; i < kDBlocks; ++i) acc_o[i] = f32x16{};
  float m_run = -INFINITY;  // running max of scaled scores (log2 domain)
  float l_run = 0.f;        // running sum of exp2(s - m_run)

  fetch(0);
  stash(0);
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int stage = t & 1;
    const int k0 = t * BKV;
    if (t + 1 < n_tiles) fetch(k0 + BKV);
    const uint8_t* ks_ = smem + stage * 2 * kTileBytes;
    const uint8_t* vs_ = ks_ + kTileBytes;

    // causal: a wave whose queries all precede the tile skips it
    const bool active = !(p.causal && k0 > wave_qmax);
    if (active) {
      // ---- S^T = K Q^T for keys k0 .. k0+63 (two 32-key blocks)
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[kb] = f32x16{};
        const int row = kb * 32 + col;
#pragma unroll
        for (int kk = 0; kk < kKSteps; ++kk) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(ks_ + k_off<D>(row, kk * 2 + h));
          s[kb] = mfma_bf16(a, qreg[kk], s[kb]);
        }
      }
      // ---- scale, mask, tile max.  Register r of block kb holds key
      //      k0 + 32*kb + 8*(r/4) + 4*h + r%4 for query my_q.
      const bool need_mask = (k0 + BKV > S) || (p.causal && k0 + BKV - 1 > q0 + wave * 32);
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[kb][r] * p.scale_log2;
          if (need_mask) {
            const int key = k0 + kb * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
            if (key >= S || (p.causal && key > my_q)) x = -INFINITY;
          }
          s[kb][r] = x;
          mt = fmaxf(mt, x);
        }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float m_new = fmaxf(m_run, mt);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = __builtin_amdgcn_exp2f(s[kb][r] - m_use);
          s[kb][r] = e;
          rs += e;
        }
      }
      rs += __shfl_xor(rs, 32, 64);
      l_run = l_run * alpha + rs;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) acc_o[db] *= alpha;

      // ---- P^T operands: block kb, step u uses registers 8u..8u+7, i.e. keys
      //      32kb + 16u + 4h + {0..3} and 32kb + 16u + 8 + 4h + {0..3}.
      u32x4 pb[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          pb[kb][u][0] = pack_bf16(s[kb][8 * u + 0], s[kb][8 * u + 1]);
          pb[kb][u][1] = pack_bf16(s[kb][8 * u + 2], s[kb][8 * u + 3]);
          pb[kb][u][2] = pack_bf16(s[kb][8 * u + 4], s[kb][8 * u + 5]);
          pb[kb][u][3] = pack_bf16(s[kb][8 * u + 6], s[kb][8 * u + 7]);
        }

      // ---- O^T += V^T P^T.  ds_read_b64_tr_b16: in each 16-lane group, lane
      //      4j+q addresses row (rowstart + j), columns 4q..4q+3 of the group's
      //      16 columns; lane i of the group receives column i, rows rowstart..+3.
      const int g_lane = lane & 15;
      const int tr_row = g_lane >> 2;            // j
      const int tr_col = ((lane >> 4) & 1) * 16 + (g_lane & 3) * 4;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int r0 = kb * 32 + u * 16 + h * 4;
            const int cc = db * 32 + tr_col;
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(vs_ + v_off<D>(r0 + tr_row, cc)));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(vs_ + v_off<D>(r0 + 8 + tr_row, cc)));
            const u32x2 lo2 = __builtin_bit_cast(u32x2, lo);
            const u32x2 hi2 = __builtin_bit_cast(u32x2, hi);
            const u32x4 a = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
            acc_o[db] = mfma_bf16(a, pb[kb][u], acc_o[db]);
          }
        }
      }
    }
    if (t + 1 < n_tiles) stash(stage ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O = O^T / l, transposed through LDS into row-major bf16.
  //      Lane holds query my_q and, for d block db and register r,
  //      d = 32*db + 8*(r/4) + 4*h + r%4.
  const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
  uint8_t* os_ = smem;  // [BQ][D] bf16, row stride D*2, chunk swizzle like K
#pragma unroll
  for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d = db * 32 + rq * 8 + h * 4;
      u32x2 w;
      w[0] = pack_bf16(acc_o[db][rq * 4 + 0] * inv_l, acc_o[db][rq * 4 + 1] * inv_l);
      w[1] = pack_bf16(acc_o[db][rq * 4 + 2] * inv_l, acc_o[db][rq * 4 + 3] * inv_l);
      const int row = wave * 32 + col;
      *reinterpret_cast<u32x2*>(os_ + k_off<D>(row, d >> 3) + (d & 7) * 2) = w;
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
    const int q = q0 + row;
    if (q < S) {
      *reinterpret_cast<u32x4*>(Oh + static_cast<int64_t>(q) * D + ch * 8) =
          *reinterpret_cast<const u32x4*>(os_ + k_off<D>(row, ch));
    }
  }
}

template <int D>
int32_t launch(const FaArgs& p, hipStream_t stream) {
  const int64_t blocks = p.heads_total * p.n_qblocks;
  hipLaunchKernelGGL(fa_fwd_kernel<D>, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream, p);
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
  ASC_REQUIRE(seq_len < (1 << 30), ASC_ERR_UNSUPPORTED, "asc_flash_attention_fwd_bf16: seq_len too large");
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
  p.n_qblocks = static_cast<int>((seq_len + BQ - 1) / BQ);
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  p.causal = causal ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return head_dim == 128 ? launch<128>(p, s) : launch<64>(p, s);
}
