// Pieces shared by the MFMA GEMM kernels (bf16/fp16 and int8) for gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asc {
namespace gemm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

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

}  // namespace gemm
}  // namespace asc
