// vadd device code: the element operations and the streaming bodies of asc2
// vadd_kernel (python/test/asc2/kernels/test_vadd.py:16-28).  Shared by the
// library (vadd.hip, launched through asc_vadd) and the standalone gfx950 code
// object (co/asc2_vadd.hip, loaded with hipModuleLoad by the asc2 launch path),
// so both launch paths run the same instructions.
//
// HBM-bound: 3 x 4 bytes per fp32 element.  Each thread moves 4 independent
// 16-byte vectors per operand (global_load_dwordx4) so a wave keeps 8 loads in
// flight; the physical grid is sized by the covered length, not by the
// Ascend-style logical grid, which only decides how far the writes reach.
#pragma once

#include "common.h"
#include "numeric.h"

namespace asc {
namespace vadd {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int kScalarMaxBlocks = 4096;

// 16-byte vector as a clang ext-vector so the nontemporal builtins accept it.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct AddF32 {
  using T = float;
  __device__ static float op(float a, float b) { return a + b; }
};
struct AddI32 {
  using T = int32_t;
  // two's-complement wraparound without signed-overflow UB
  __device__ static int32_t op(int32_t a, int32_t b) {
    return static_cast<int32_t>(static_cast<uint32_t>(a) + static_cast<uint32_t>(b));
  }
};
struct AddF16 {
  using T = uint16_t;
  // fp32 add then RNE to fp16 equals the correctly rounded fp16 add (24 >= 2*11+2 bits)
  __device__ static uint16_t op(uint16_t a, uint16_t b) {
    return asc::f32_to_f16_rne(asc::f16_to_f32(a) + asc::f16_to_f32(b));
  }
};
struct AddBF16 {
  using T = uint16_t;
  __device__ static uint16_t op(uint16_t a, uint16_t b) {
    return asc::f32_to_bf16_rne(asc::bf16_to_f32(a) + asc::bf16_to_f32(b));
  }
};

template <typename Op>
__device__ __forceinline__ u32x4 add_vec(u32x4 a, u32x4 b) {
  using T = typename Op::T;
  constexpr int kN = 16 / sizeof(T);
  T ea[kN], eb[kN], ec[kN];
  __builtin_memcpy(ea, &a, 16);
  __builtin_memcpy(eb, &b, 16);
#pragma unroll
  for (int i = 0; i < kN; ++i) ec[i] = Op::op(ea[i], eb[i]);
  u32x4 c;
  __builtin_memcpy(&c, ec, 16);
  return c;
}

// out[v] = x[v] + y[v] for 16-byte vectors v < n_vec; a workgroup of kThreads
// covers kThreads * kUnroll vectors.
template <typename Op>
__device__ __forceinline__ void vec_body(const u32x4* __restrict__ x, const u32x4* __restrict__ y,
                                         u32x4* __restrict__ out, int64_t n_vec) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
  u32x4 a[kUnroll], b[kUnroll];
  if (base + (kUnroll - 1) * kThreads < n_vec) {
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) a[j] = __builtin_nontemporal_load(x + base + j * kThreads);
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) b[j] = __builtin_nontemporal_load(y + base + j * kThreads);
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) __builtin_nontemporal_store(add_vec<Op>(a[j], b[j]), out + base + j * kThreads);
  } else {
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int64_t v = base + j * kThreads;
      if (v < n_vec) out[v] = add_vec<Op>(x[v], y[v]);
    }
  }
}

// Element-wise path for [begin, end): unaligned buffers and the sub-vector tail.
template <typename Op>
__device__ __forceinline__ void scalar_body(const typename Op::T* __restrict__ x, const typename Op::T* __restrict__ y,
                                            typename Op::T* __restrict__ out, int64_t begin, int64_t end) {
  for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < end;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    out[i] = Op::op(x[i], y[i]);
  }
}

// Element i = begin + global thread index, if below end: one element per thread,
// no grid-stride loop (the code object's form; it reads no grid size).
template <typename Op>
__device__ __forceinline__ void element_body(const typename Op::T* __restrict__ x, const typename Op::T* __restrict__ y,
                                             typename Op::T* __restrict__ out, int64_t begin, int64_t end) {
  const int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < end) out[i] = Op::op(x[i], y[i]);
}

// Workgroups of the vector kernel for n_vec vectors.
inline int64_t vec_blocks(int64_t n_vec) { return (n_vec + kThreads * kUnroll - 1) / (kThreads * kUnroll); }
// Workgroups of the element-wise kernel for n elements.
inline int64_t scalar_blocks(int64_t n) {
  const int64_t b = (n + kThreads - 1) / kThreads;
  return b < kScalarMaxBlocks ? b : kScalarMaxBlocks;
}

}  // namespace vadd
}  // namespace asc
