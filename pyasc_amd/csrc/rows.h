// Row access for the row kernels (softmax.hip, reduce.hip): a row of fp32
// values held in registers as float4 vectors.
#pragma once

#include "common.h"

namespace asc {
namespace rows {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct RowView {
  const float* x;
  float* out;
  int64_t rows;    // covered rows [0, rows)
  int64_t stride;  // elements between row starts
  int32_t len;     // columns processed per row
  bool vec_ok;     // rows start 16-byte aligned
};

// Vector q (elements 4q..4q+3) of a row, `pad` past `len`.
__device__ __forceinline__ float4 load_vec(const float* row, int q, int len, bool vec_ok, float pad) {
  const int e = q * 4;
  if (vec_ok && e + 3 < len) {
    // streamed once: non-temporal so the rows do not displace other cached data
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row + e));
    return make_float4(v.x, v.y, v.z, v.w);
  }
  float4 v;
  v.x = e + 0 < len ? row[e + 0] : pad;
  v.y = e + 1 < len ? row[e + 1] : pad;
  v.z = e + 2 < len ? row[e + 2] : pad;
  v.w = e + 3 < len ? row[e + 3] : pad;
  return v;
}

__device__ __forceinline__ void store_vec(float* row, int q, int len, bool vec_ok, float4 v) {
  const int e = q * 4;
  if (vec_ok && e + 3 < len) {
    __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4*>(row + e));
    return;
  }
  if (e + 0 < len) row[e + 0] = v.x;
  if (e + 1 < len) row[e + 1] = v.y;
  if (e + 2 < len) row[e + 2] = v.z;
  if (e + 3 < len) row[e + 3] = v.w;
}

// Vectors q0 + kStride*j (j < N) of a row, where q0 < kStride is the thread's
// index in its group.  The test that a vector lies inside the row for every
// thread of the group depends on kernel arguments only (uniform branch), so
// full vectors are plain 16-byte loads issued back to back; only a ragged
// tail takes the per-lane path.  (A per-lane choice between the two load
// forms would run both and serialise the loads on their shared registers.)
template <int N, int kStride>
__device__ __forceinline__ void load_row(float4 (&v)[N], const float* row, int q0, int len, bool vec_ok, float pad) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int q = q0 + kStride * j;
    if (vec_ok && kStride * (j + 1) * 4 <= len) {
      const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row) + q);
      v[j] = make_float4(t.x, t.y, t.z, t.w);
    } else {
      v[j] = load_vec(row, q, len, vec_ok, pad);
    }
  }
}

template <int N, int kStride>
__device__ __forceinline__ void store_row(const float4 (&v)[N], float* row, int q0, int len, bool vec_ok) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int q = q0 + kStride * j;
    if (vec_ok && kStride * (j + 1) * 4 <= len) {
      __builtin_nontemporal_store(f32x4{v[j].x, v[j].y, v[j].z, v[j].w}, reinterpret_cast<f32x4*>(row) + q);
    } else {
      store_vec(row, q, len, vec_ok, v[j]);
    }
  }
}

}  // namespace rows
}  // namespace asc
