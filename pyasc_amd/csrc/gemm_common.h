// Pieces shared by the MFMA GEMM kernels (bf16/fp16 and int8) for gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asc {
namespace gemm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// LDS tiles are stored as rows of 8 chunks of 16 bytes (128 bytes per row, K
// contiguous).  The chunk index is XOR-swizzled with
//   g(row) = (row ^ (row >> 3)) & 7.
// A 128-bit LDS access is serviced 8 lanes (128 bytes) at a time, so each
// group of 8 lanes must touch 8 distinct chunk positions:
//  - MFMA operand reads: 8 consecutive rows, one chunk each -> row & 7 differs;
//  - transposed B writes: rows 8*nc + e for 8 values of nc -> (row >> 3) differs;
//  - A writes: one row, chunks 0..7.
// (Enumerated: conflict-free for all three; the previous ((row>>1)^(row>>3))
// form measured as many LDS bank-conflict cycles as active LDS cycles.)
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row ^ (row >> 3)) & 7); }

__device__ __forceinline__ uint32_t lds_offset(int row, int chunk) {
  return static_cast<uint32_t>(row * 128 + swz(row, chunk) * 16);
}

// Logical tile id for hardware block id `bid`.  Blocks are dispatched round-
// robin over the 8 XCDs (bid % 8); consecutive logical ids are made to live on
// one XCD so that neighbouring tiles share that XCD's L2.  Then a grouped
// (GROUP_M tile-rows) order keeps A and B panels hot while a group runs.
__device__ __forceinline__ void tile_coords(int bid, int nblocks, int tiles_m, int tiles_n, int group_m, int& tm,
                                            int& tn) {
  int logical = bid;
  if ((nblocks & 7) == 0) logical = (bid & 7) * (nblocks >> 3) + (bid >> 3);
  const int group_size = group_m * tiles_n;
  const int group = logical / group_size;
  const int first_m = group * group_m;
  const int gm = min(tiles_m - first_m, group_m);
  const int in_group = logical - group * group_size;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// 16-bit 8x8 transpose: in[r] holds 8 consecutive columns of row r; out[c]
// holds 8 consecutive rows of column c.  Each output dword takes the same
// half-word of two input rows (one v_perm_b32 each).
__device__ __forceinline__ void transpose8x8_b16(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int w = c >> 1;
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int j = 0; j < 4; ++j) out[c][j] = __builtin_amdgcn_perm(in[2 * j + 1][w], in[2 * j][w], sel);
  }
}

// 8-bit transpose of a 4x4 byte block: x[r] holds row r (bytes = columns);
// y[c] receives column c (bytes = rows).  Eight v_perm_b32: pair rows, then
// pair the pairs.
__device__ __forceinline__ void transpose4x4_b8(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3, uint32_t& y0,
                                                uint32_t& y1, uint32_t& y2, uint32_t& y3) {
  const uint32_t t01_lo = __builtin_amdgcn_perm(x1, x0, 0x05010400u);  // x0.b0 x1.b0 x0.b1 x1.b1
  const uint32_t t01_hi = __builtin_amdgcn_perm(x1, x0, 0x07030602u);  // x0.b2 x1.b2 x0.b3 x1.b3
  const uint32_t t23_lo = __builtin_amdgcn_perm(x3, x2, 0x05010400u);
  const uint32_t t23_hi = __builtin_amdgcn_perm(x3, x2, 0x07030602u);
  y0 = __builtin_amdgcn_perm(t23_lo, t01_lo, 0x05040100u);
  y1 = __builtin_amdgcn_perm(t23_lo, t01_lo, 0x07060302u);
  y2 = __builtin_amdgcn_perm(t23_hi, t01_hi, 0x05040100u);
  y3 = __builtin_amdgcn_perm(t23_hi, t01_hi, 0x07060302u);
}

// 8-bit 16x8 transpose: in[r] (r < 16) holds 8 consecutive columns of row r;
// out[c] (c < 8) receives the 16 rows of column c.
__device__ __forceinline__ void transpose16x8_b8(const u32x2 (&in)[16], u32x4 (&out)[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      uint32_t y0, y1, y2, y3;
      transpose4x4_b8(in[4 * q][w], in[4 * q + 1][w], in[4 * q + 2][w], in[4 * q + 3][w], y0, y1, y2, y3);
      out[4 * w + 0][q] = y0;
      out[4 * w + 1][q] = y1;
      out[4 * w + 2][q] = y2;
      out[4 * w + 3][q] = y3;
    }
  }
}

// ---- epilogue stores through quad transposes ------------------------------
// A 32x32 MFMA result block leaves lane l with column l%32 and, in registers
// 4g..4g+3, rows 8g + 4*(l/32) + 0..3.  Storing straight from that layout
// writes one element per lane per instruction.  Inside each quad of lanes
// (4q..4q+3, consecutive columns) the 4 registers of group g form a 4x4 block;
// transposing it (two lane exchanges, xor 2 then xor 1) leaves lane 4q+t with
// row 8g + 4*(l/32) + t, columns 4q..4q+3: one 8-byte (16-bit output) or
// 16-byte (32-bit output) store per lane and group, a quarter of the
// instructions.
__device__ __forceinline__ uint32_t quad_xor1(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ uint32_t quad_xor2(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x4E, 0xF, 0xF, true));
}

// 16-bit values: on entry d0 = (v0 | v1 << 16), d1 = (v2 | v3 << 16) with v_k the
// element of row k, column t (t = lane % 4); on exit the same packing holds the
// elements of row t, columns 0..3.
__device__ __forceinline__ void quad_transpose_b16(uint32_t& d0, uint32_t& d1, int t) {
  const bool hi2 = (t & 2) != 0;
  const uint32_t recv = quad_xor2(hi2 ? d0 : d1);
  if (hi2) {
    d0 = recv;  // rows 2,3 of column t-2
  } else {
    d1 = recv;  // rows 0,1 of column t+2
  }
  const bool odd = (t & 1) != 0;
  // even lanes send the high halves (the odd partner's row), odd lanes the low halves
  const uint32_t r = quad_xor1(odd ? __builtin_amdgcn_perm(d1, d0, 0x05040100u)
                                   : __builtin_amdgcn_perm(d1, d0, 0x07060302u));
  const uint32_t e0 = __builtin_amdgcn_perm(r, d0, 0x05040100u), e1 = __builtin_amdgcn_perm(r, d1, 0x07060100u);
  const uint32_t o0 = __builtin_amdgcn_perm(d0, r, 0x07060100u), o1 = __builtin_amdgcn_perm(d1, r, 0x07060302u);
  d0 = odd ? o0 : e0;
  d1 = odd ? o1 : e1;
}

// 32-bit values: v[k] = element (row k, column t) on entry, (row t, column k) on exit.
__device__ __forceinline__ void quad_transpose_b32(uint32_t (&v)[4], int t) {
  const bool hi2 = (t & 2) != 0;
  const uint32_t s0 = quad_xor2(hi2 ? v[0] : v[2]);
  const uint32_t s1 = quad_xor2(hi2 ? v[1] : v[3]);
  const uint32_t a0 = hi2 ? s0 : v[0], a1 = hi2 ? s1 : v[1], a2 = hi2 ? v[2] : s0, a3 = hi2 ? v[3] : s1;
  const bool odd = (t & 1) != 0;
  const uint32_t r0 = quad_xor1(odd ? a0 : a1);
  const uint32_t r1 = quad_xor1(odd ? a2 : a3);
  v[0] = odd ? r0 : a0;
  v[1] = odd ? a1 : r0;
  v[2] = odd ? r1 : a2;
  v[3] = odd ? a3 : r1;
}

// Stores a wave's 128 x (32 kJ) block of results (4 x kJ MFMA blocks, `acc`) at
// c + (m_base, n_base) (row stride ldc elements) through the quad transposes.
// conv(j, x) turns accumulator value x of block column j into the output bits
// (the low 16 bits for 16-bit outputs).  Blocks of one row band go out
// column-block after column-block, so each row's outputs leave in consecutive
// instructions.  The stores are plain (write-back): an instruction covers 32 or
// 64 bytes of each of its rows, and the L2 merges a line's pieces before writing
// it back.  Non-temporal stores sent the pieces to memory one by one: 1.42x the
// fp16 output in WRITE_SIZE for the int8 GEMM, against 1.006x now.  Every
// element must be in bounds.
template <int kOutBytes, int kJ, class AccT, class Conv>
__device__ __forceinline__ void store_wave_tile(const AccT (&acc)[4][kJ], Conv conv, void* c, int64_t ldc, int m_base,
                                                int n_base, int lane) {
  static_assert(kOutBytes == 2 || kOutBytes == 4, "16- or 32-bit outputs");
  const int t = lane & 3, q = (lane & 31) >> 2, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t row = m_base + i * 32 + g * 8 + h * 4 + t;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int64_t off = row * ldc + n_base + j * 32 + 4 * q;
        if constexpr (kOutBytes == 2) {
          uint32_t d0 = (conv(j, acc[i][j][4 * g + 0]) & 0xFFFFu) | (conv(j, acc[i][j][4 * g + 1]) << 16);
          uint32_t d1 = (conv(j, acc[i][j][4 * g + 2]) & 0xFFFFu) | (conv(j, acc[i][j][4 * g + 3]) << 16);
          quad_transpose_b16(d0, d1, t);
          *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(c) + off) = u32x2{d0, d1};
        } else {
          uint32_t v[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) v[k] = conv(j, acc[i][j][4 * g + k]);
          quad_transpose_b32(v, t);
          *reinterpret_cast<u32x4*>(static_cast<uint32_t*>(c) + off) = u32x4{v[0], v[1], v[2], v[3]};
        }
      }
    }
  }
}

}  // namespace gemm
}  // namespace asc
