// Dense matmul C = epilogue(A . B) for the asc2 cube path
// (python/asc/language/tile/binary_ops.py:180-221; kernels in
// python/test/asc2/kernels/test_matmul_{mnblock,tiled,fixpipe,l0c_to_l1}.py): the
// library's entry points and the launch plan the asc2 code-object path replays.
// The device code and the choice of kernels are described in matmul_kernels.h.
#include <stdlib.h>

#include <mutex>

#include "matmul_kernels.h"

// The intermediate of asc_matmul_chained_noalloc: one chained matmul's t (M * N
// 16-bit elements) at most, one copy per GPU, held until the process ends.  Host code
// uses the per-device address from hipGetSymbolAddress, never the array's name.
constexpr int64_t kChainedScratchBytes = int64_t{32} << 20;
static __device__ __align__(256) uint8_t scratch[kChainedScratchBytes];

namespace {

using asc::mm::BM;
using asc::mm::BN;
using asc::mm::Epilogue;
using asc::mm::GemmArgs;

ASC_MM_KERNELS(, mm_)

// Kernel index = 6 * output dtype (f32, f16, bf16) + kind, kind 0-5 in the order below.
constexpr int kKinds = 6;
constexpr const char* kKindNames[kKinds] = {"mfma_bf16_fast_", "mfma_bf16_checked_", "mfma_f16_fast_",
                                            "mfma_f16_checked_", "f32_mfma_", "f32_fma_"};
constexpr const char* kOutNames[3] = {"f32", "f16", "bf16"};
using KernelFn = void (*)(GemmArgs);
const KernelFn kKernels[3 * kKinds] = {
    mm_mfma_bf16_fast_f32,  mm_mfma_bf16_checked_f32,  mm_mfma_f16_fast_f32,  mm_mfma_f16_checked_f32,
    mm_f32_mfma_f32,        mm_f32_fma_f32,            mm_mfma_bf16_fast_f16, mm_mfma_bf16_checked_f16,
    mm_mfma_f16_fast_f16,   mm_mfma_f16_checked_f16,   mm_f32_mfma_f16,       mm_f32_fma_f16,
    mm_mfma_bf16_fast_bf16, mm_mfma_bf16_checked_bf16, mm_mfma_f16_fast_bf16, mm_mfma_f16_checked_bf16,
    mm_f32_mfma_bf16,       mm_f32_fma_bf16};

// One matmul launch: kernel index, arguments, grid.
struct MmLaunch {
  int kernel = 0;
  GemmArgs p{};
  int64_t blocks = 0;  // 0: nothing to launch
  int threads = 0;
};

int out_index(int32_t out_dtype) {
  return out_dtype == ASC_DT_FLOAT32 ? 0 : out_dtype == ASC_DT_FLOAT16 ? 1 : out_dtype == ASC_DT_BFLOAT16 ? 2 : -1;
}

int32_t make_launch(int32_t in_dtype, int32_t out_dtype, const void* a, const void* b, void* c, int64_t M, int64_t N,
                    int64_t K, int64_t lda, int64_t ldb, int64_t ldc, Epilogue epi, MmLaunch& L) {
  L = MmLaunch{};
  ASC_REQUIRE(M >= 0 && N >= 0 && K >= 0, ASC_ERR_INVALID_ARG, "asc_matmul: negative shape");
  ASC_REQUIRE(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), ASC_ERR_UNSUPPORTED, "asc_matmul: shape too large");
  ASC_REQUIRE(lda >= K && ldb >= N && ldc >= N, ASC_ERR_INVALID_ARG,
              "asc_matmul: leading dimensions (%lld, %lld, %lld) smaller than the rows", (long long)lda,
              (long long)ldb, (long long)ldc);
  if (M == 0 || N == 0) return ASC_OK;
  // with K == 0 no operand element is read (C receives the epilogue of 0)
  ASC_REQUIRE(c && (K == 0 || (a && b)), ASC_ERR_INVALID_ARG, "asc_matmul: null buffer");
  const int out = out_index(out_dtype);
  ASC_REQUIRE(in_dtype == ASC_DT_FLOAT32 || in_dtype == ASC_DT_FLOAT16 || in_dtype == ASC_DT_BFLOAT16,
              ASC_ERR_UNSUPPORTED, "asc_matmul: unsupported input dtype %d", in_dtype);
  ASC_REQUIRE(out >= 0, ASC_ERR_UNSUPPORTED, "asc_matmul: unsupported out dtype %d", out_dtype);
  GemmArgs& p = L.p;
  p.a = a;
  p.b = b;
  p.c = c;
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.lda = lda;
  p.ldb = ldb;
  p.ldc = ldc;
  p.epi = epi;
  p.tiles_m = static_cast<int>((M + BM - 1) / BM);
  p.tiles_n = static_cast<int>((N + BN - 1) / BN);
  int kind;
  if (in_dtype == ASC_DT_FLOAT32) {
    // one workgroup per 16x16 output block up to 2048 x 2048 outputs, per 64x64 tile above
    const int64_t blocks16 = ((M + 15) / 16) * ((N + 15) / 16);
    const bool small = blocks16 <= asc::mm::kF32MfmaMaxBlocks;
    kind = small ? 4 : 5;
    L.blocks = small ? blocks16 : ((M + 63) / 64) * ((N + 63) / 64);
    L.threads = 256;
  } else {
    const bool aligned = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0 &&
                         (lda % 8) == 0 && (ldb % 8) == 0;
    // the direct-to-LDS path addresses each operand with 31-bit buffer offsets
    const bool offsets_fit = (BM * lda + K) * 2 < (int64_t{1} << 31) && (K + 64) * ldb * 2 < (int64_t{1} << 31);
    // the fast path's epilogue stores 8 (16-bit C) or 16 (fp32 C) bytes per lane at 4-column steps
    const int64_t out_bytes = out_dtype == ASC_DT_FLOAT32 ? 4 : 2;
    const bool c_rows_aligned = (reinterpret_cast<uintptr_t>(c) & 15) == 0 && (ldc * out_bytes) % 16 == 0;
    // K == 0 takes the checked kernel: no k-tile runs and C receives cast(0).
    const bool fast = aligned && c_rows_aligned && offsets_fit && (M % BM) == 0 && (N % BN) == 0 &&
                      (K % 32) == 0 && K > 0;
    kind = (in_dtype == ASC_DT_BFLOAT16 ? 0 : 2) + (fast ? 0 : 1);
    L.blocks = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
    L.threads = fast ? asc::mm::kFastThreads : asc::mm::kThreads;
  }
  L.kernel = kKinds * out + kind;
  // one workgroup per output tile: the grid's thread count must fit 32 bits
  ASC_REQUIRE(L.blocks * L.threads < (int64_t{1} << 32), ASC_ERR_UNSUPPORTED,
              "asc_matmul: %lld output tiles exceed one launch", static_cast<long long>(L.blocks));
  return ASC_OK;
}

int32_t run(int32_t in_dtype, int32_t out_dtype, const void* a, const void* b, void* c, int64_t M, int64_t N,
            int64_t K, int64_t lda, int64_t ldb, int64_t ldc, Epilogue epi, asc_stream_t stream) {
  MmLaunch L;
  const int32_t rc = make_launch(in_dtype, out_dtype, a, b, c, M, N, K, lda, ldb, ldc, epi, L);
  if (rc != ASC_OK || L.blocks == 0) return rc;
  hipLaunchKernelGGL(kKernels[L.kernel], dim3(static_cast<uint32_t>(L.blocks)), dim3(L.threads), 0,
                     static_cast<hipStream_t>(stream), L.p);
  return asc::check_launch("asc_matmul");
}

// Shape and dtype checks of a chained matmul (no device call).
int32_t chained_check(int32_t in_dtype, int64_t M, int64_t N, int64_t K, const char* who) {
  ASC_REQUIRE(M >= 0 && N >= 0 && K >= 0, ASC_ERR_INVALID_ARG, "%s: negative shape", who);
  ASC_REQUIRE(in_dtype == ASC_DT_FLOAT16 || in_dtype == ASC_DT_BFLOAT16, ASC_ERR_UNSUPPORTED,
              "%s: input dtype %d is not float16 or bfloat16", who, in_dtype);
  ASC_REQUIRE(N == K, ASC_ERR_INVALID_ARG,
              "%s: the chained matmul multiplies (a @ b) by b again and needs N == K, got N=%lld, K=%lld", who,
              (long long)N, (long long)K);
  ASC_REQUIRE(M < (1 << 30) && N < (1 << 30), ASC_ERR_UNSUPPORTED, "%s: shape too large", who);
  return ASC_OK;
}

// t = cast(a . b) to in_dtype into `t` (t_bytes long), then c = cast(t . b) to out_dtype.
int32_t chained(int32_t in_dtype, int32_t out_dtype, const void* a, const void* b, void* c, int64_t M, int64_t N,
                int64_t K, void* t, int64_t t_bytes, asc_stream_t stream, const char* who) {
  const int32_t checked = chained_check(in_dtype, M, N, K, who);
  if (checked != ASC_OK) return checked;
  if (M == 0 || N == 0) return ASC_OK;
  const int64_t need = M * N * 2;
  ASC_REQUIRE(t_bytes >= need, ASC_ERR_INVALID_ARG, "%s: the intermediate needs %lld bytes, the workspace holds %lld",
              who, (long long)need, (long long)t_bytes);
  ASC_REQUIRE(t, ASC_ERR_INVALID_ARG, "%s: null workspace", who);
  const Epilogue none{nullptr, 0, 0.0f};
  const int32_t rc = run(in_dtype, in_dtype, a, b, t, M, N, K, K, N, N, none, stream);
  if (rc != ASC_OK) return rc;
  return run(in_dtype, out_dtype, t, b, c, M, N, N, N, N, N, none, stream);
}

// Device address of `scratch` on the current device, looked up on the first call on each
// device (with that device current) and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

int32_t scratch_address(void** out, const char* who) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  ASC_REQUIRE(err == hipSuccess, static_cast<int32_t>(err), "%s: hipGetDevice failed: %s", who,
              hipGetErrorString(err));
  ASC_REQUIRE(dev >= 0 && dev < kMaxDevices, ASC_ERR_UNSUPPORTED, "%s: device %d beyond the %d supported", who, dev,
              kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    ASC_REQUIRE(err == hipSuccess && p != nullptr, err == hipSuccess ? ASC_ERR_UNSUPPORTED : static_cast<int32_t>(err),
                "%s: hipGetSymbolAddress of the scratch buffer failed on device %d: %s", who, dev,
                hipGetErrorString(err));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return ASC_OK;
}

// Optional check of the rule that calls sharing one GPU's scratch buffer must not
// overlap (ASC_NOALLOC_CHECK=1 in the environment; a debugging aid, off by default).
// Each checked call records a per-device event on its stream after its two launches;
// a call on another stream while that event is still pending is refused with
// ASC_ERR_BUSY before anything is launched.  The event is created on the device's
// first checked call (the only allocation the check makes).  Streams under graph
// capture are not checked: their launches run at replay.
struct ScratchUse {
  hipStream_t stream = nullptr;
  hipEvent_t done = nullptr;
  bool recorded = false;
};
ScratchUse g_use[kMaxDevices];
std::mutex g_use_mu;

bool noalloc_check_enabled() {
  const char* v = getenv("ASC_NOALLOC_CHECK");
  return v != nullptr && v[0] != '\0' && !(v[0] == '0' && v[1] == '\0');
}

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

}  // namespace

extern "C" int32_t asc_matmul_chained_noalloc(int32_t in_dtype, int32_t out_dtype, const void* a, const void* b,
                                              void* c, int64_t M, int64_t N, int64_t K, asc_stream_t stream) {
  const char* who = "asc_matmul_chained_noalloc";
  const int32_t checked = chained_check(in_dtype, M, N, K, who);
  if (checked != ASC_OK) return checked;
  if (M == 0 || N == 0) return ASC_OK;
  ASC_REQUIRE(M * N * 2 <= kChainedScratchBytes, ASC_ERR_UNSUPPORTED,
              "%s: the intermediate of %lld x %lld needs %lld bytes, above the %lld-byte scratch buffer", who,
              (long long)M, (long long)N, (long long)(M * N * 2), (long long)kChainedScratchBytes);
  void* t = nullptr;
  const int32_t rc = scratch_address(&t, who);
  if (rc != ASC_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!noalloc_check_enabled() || capturing(s)) {
    return chained(in_dtype, out_dtype, a, b, c, M, N, K, t, kChainedScratchBytes, stream, who);
  }
  int dev = -1;
  ASC_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices, ASC_ERR_UNSUPPORTED,
              "%s: no current device", who);
  std::lock_guard<std::mutex> lock(g_use_mu);
  ScratchUse& use = g_use[dev];
  if (use.recorded && use.stream != s) {
    const hipError_t q = hipEventQuery(use.done);
    ASC_REQUIRE(q != hipErrorNotReady, ASC_ERR_BUSY,
                "%s: the previous call on this GPU (another stream) has not finished with the shared scratch "
                "buffer; order the streams (an event) or use one stream",
                who);
  }
  if (use.done == nullptr) {
    const hipError_t e = hipEventCreateWithFlags(&use.done, hipEventDisableTiming);
    ASC_REQUIRE(e == hipSuccess, static_cast<int32_t>(e), "%s: hipEventCreateWithFlags failed: %s", who,
                hipGetErrorString(e));
  }
  const int32_t run_rc = chained(in_dtype, out_dtype, a, b, c, M, N, K, t, kChainedScratchBytes, stream, who);
  if (run_rc != ASC_OK) return run_rc;
  const hipError_t e = hipEventRecord(use.done, s);
  ASC_REQUIRE(e == hipSuccess, static_cast<int32_t>(e), "%s: hipEventRecord failed: %s", who, hipGetErrorString(e));
  use.stream = s;
  use.recorded = true;
  return ASC_OK;
}

extern "C" int32_t asc_matmul_chained(int32_t in_dtype, int32_t out_dtype, const void* a, const void* b, void* c,
                                      int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                                      asc_stream_t stream) {
  return chained(in_dtype, out_dtype, a, b, c, M, N, K, workspace, workspace_bytes, stream, "asc_matmul_chained");
}

extern "C" int32_t asc_matmul(int32_t in_dtype, int32_t out_dtype, const void* a, const void* b, void* c, int64_t M,
                              int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int32_t relu,
                              asc_stream_t stream) {
  return run(in_dtype, out_dtype, a, b, c, M, N, K, lda, ldb, ldc, Epilogue{nullptr, relu ? 1 : 0, 0.0f}, stream);
}

extern "C" int32_t asc_matmul_bias_act(int32_t in_dtype, int32_t out_dtype, const void* a, const void* b, void* c,
                                       const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                       int64_t ldc, int32_t act, float alpha, asc_stream_t stream) {
  ASC_REQUIRE(act >= 0 && act <= 2, ASC_ERR_INVALID_ARG, "asc_matmul_bias_act: act must be 0, 1 or 2, got %d", act);
  return run(in_dtype, out_dtype, a, b, c, M, N, K, lda, ldb, ldc, Epilogue{bias, act, alpha}, stream);
}

extern "C" int32_t asc_matmul_plan(int32_t in_dtype, int32_t out_dtype, const void* a, const void* b, void* c,
                                   const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                   int64_t ldc, int32_t act, float alpha, asc_launch_plan_t* plan) {
  ASC_REQUIRE(plan, ASC_ERR_INVALID_ARG, "asc_matmul_plan: null plan");
  *plan = asc_launch_plan_t{};
  ASC_REQUIRE(act >= 0 && act <= 2, ASC_ERR_INVALID_ARG, "asc_matmul_plan: act must be 0, 1 or 2, got %d", act);
  MmLaunch L;
  const int32_t rc = make_launch(in_dtype, out_dtype, a, b, c, M, N, K, lda, ldb, ldc, Epilogue{bias, act, alpha}, L);
  if (rc != ASC_OK || L.blocks == 0) return rc;
  static_assert(sizeof(GemmArgs) <= sizeof(plan->args), "argument blob");
  __builtin_snprintf(plan->kernel, sizeof(plan->kernel), "asc2_mm_%s%s", kKindNames[L.kernel % kKinds],
                     kOutNames[L.kernel / kKinds]);
  plan->grid = static_cast<uint32_t>(L.blocks);
  plan->block = static_cast<uint32_t>(L.threads);
  plan->args_size = sizeof(GemmArgs);
  __builtin_memcpy(plan->args, &L.p, sizeof(GemmArgs));
  return ASC_OK;
}
