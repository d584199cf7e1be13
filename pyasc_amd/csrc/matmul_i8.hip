// int8 GEMM with exact int32 accumulation and the per-output-channel fp16 dequant
// (python/test/generalization/adv/test_matmul_quant.py:23-51,94-106): the library's
// entry points and the launch plan the asc2 code-object path replays.  The device
// code is matmul_i8_kernels.h.
#include "matmul_i8_kernels.h"

namespace {

using asc::i8::BM;
using asc::i8::BN;
using asc::i8::I8Args;

ASC_I8_KERNELS(, gemm_i8_)

// One int8 GEMM launch: kernel index (fast / checked x int32 / fp16), arguments, grid.
struct I8Launch {
  int32_t kernel = 0;  // 2 * checked + dequant
  I8Args p{};
  int64_t blocks = 0;  // 0: nothing to launch
  int32_t threads = 0;
};

constexpr const char* kI8Kernels[4] = {"asc2_i8_fast_i32", "asc2_i8_fast_f16", "asc2_i8_checked_i32",
                                       "asc2_i8_checked_f16"};

int32_t make_launch(const int8_t* a, const int8_t* b, const float* scale, void* c, int64_t M, int64_t N, int64_t K,
                    int32_t trunc19, int mode, const char* who, I8Launch& L) {
  L = I8Launch{};
  ASC_REQUIRE(M >= 0 && N >= 0 && K >= 0, ASC_ERR_INVALID_ARG, "%s: negative shape", who);
  ASC_REQUIRE(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), ASC_ERR_UNSUPPORTED, "%s: shape too large", who);
  // |acc| <= K * 128 * 128 must fit int32
  ASC_REQUIRE(K <= (int64_t{1} << 17), ASC_ERR_UNSUPPORTED, "%s: K=%lld could overflow the int32 accumulator", who,
              (long long)K);
  if (M == 0 || N == 0) return ASC_OK;
  ASC_REQUIRE(a && b && c && (mode == 0 || scale), ASC_ERR_INVALID_ARG, "%s: null buffer", who);
  I8Args& p = L.p;
  p.a = a;
  p.b = b;
  p.scale = scale;
  p.c = c;
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.trunc19 = trunc19;
  p.tiles_m = static_cast<int>((M + BM - 1) / BM);
  p.tiles_n = static_cast<int>((N + BN - 1) / BN);
  // the direct-to-LDS path addresses each operand with 31-bit buffer offsets
  const bool offsets_fit = (BM * K + K) < (int64_t{1} << 31) && (K + 128) * N < (int64_t{1} << 31);
  // (the fast path's epilogue also stores 8 or 16 bytes per lane: C must be 16-byte aligned)
  const bool fast = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                      reinterpret_cast<uintptr_t>(c)) & 15) == 0 && offsets_fit &&
                    (M % BM) == 0 && (N % BN) == 0 && (K % 64) == 0 && K > 0;
  L.kernel = (fast ? 0 : 2) + mode;
  L.threads = fast ? asc::i8::kFastThreads : asc::i8::kThreads;
  L.blocks = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
  // one workgroup per output tile: the grid's thread count must fit 32 bits
  ASC_REQUIRE(L.blocks * L.threads < (int64_t{1} << 32), ASC_ERR_UNSUPPORTED, "%s: %lld output tiles exceed one launch",
              who, static_cast<long long>(L.blocks));
  return ASC_OK;
}

int32_t run(const int8_t* a, const int8_t* b, const float* scale, void* c, int64_t M, int64_t N, int64_t K,
            int32_t trunc19, int mode, asc_stream_t stream, const char* who) {
  I8Launch L;
  const int32_t rc = make_launch(a, b, scale, c, M, N, K, trunc19, mode, who, L);
  if (rc != ASC_OK || L.blocks == 0) return rc;
  decltype(&gemm_i8_fast_i32) const kernels[4] = {gemm_i8_fast_i32, gemm_i8_fast_f16, gemm_i8_checked_i32,
                                                  gemm_i8_checked_f16};
  hipLaunchKernelGGL(kernels[L.kernel], dim3(static_cast<uint32_t>(L.blocks)), dim3(L.threads), 0,
                     static_cast<hipStream_t>(stream), L.p);
  return asc::check_launch(who);
}

}  // namespace

extern "C" int32_t asc_matmul_i8_i32(const int8_t* a, const int8_t* b, int32_t* c, int64_t M, int64_t N, int64_t K,
                                     asc_stream_t stream) {
  return run(a, b, nullptr, c, M, N, K, 0, 0, stream, "asc_matmul_i8_i32");
}

extern "C" int32_t asc_matmul_i8_dequant_f16(const int8_t* a, const int8_t* b, const float* scale, void* c,
                                             int64_t M, int64_t N, int64_t K, int32_t trunc19, asc_stream_t stream) {
  return run(a, b, scale, c, M, N, K, trunc19, 1, stream, "asc_matmul_i8_dequant_f16");
}

extern "C" int32_t asc_matmul_i8_plan(const int8_t* a, const int8_t* b, const float* scale, void* c, int64_t M,
                                      int64_t N, int64_t K, int32_t dequant, int32_t trunc19,
                                      asc_launch_plan_t* plan) {
  ASC_REQUIRE(plan, ASC_ERR_INVALID_ARG, "asc_matmul_i8_plan: null plan");
  *plan = asc_launch_plan_t{};
  I8Launch L;
  const int32_t rc = make_launch(a, b, dequant ? scale : nullptr, c, M, N, K, dequant ? trunc19 : 0, dequant ? 1 : 0,
                                 dequant ? "asc_matmul_i8_dequant_f16" : "asc_matmul_i8_i32", L);
  if (rc != ASC_OK || L.blocks == 0) return rc;
  static_assert(sizeof(I8Args) <= sizeof(plan->args), "argument blob");
  __builtin_strncpy(plan->kernel, kI8Kernels[L.kernel], sizeof(plan->kernel) - 1);
  plan->grid = static_cast<uint32_t>(L.blocks);
  plan->block = static_cast<uint32_t>(L.threads);
  plan->args_size = sizeof(I8Args);
  __builtin_memcpy(plan->args, &L.p, sizeof(I8Args));
  return ASC_OK;
}
