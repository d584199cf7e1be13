// Flash-attention forward for the build's asc2-style flash_attention_fwd_kernel
// (bf16 in/out, head_dim 64 or 128): the library's entry point and the launch plan
// the asc2 code-object path replays.  The device code is flash_attn_kernels.h.
#include "flash_attn_kernels.h"

namespace {

using asc::fa::BKV;
using asc::fa::FaArgs;
using asc::fa::FaConfig;

ASC_FA_KERNELS(, fa_fwd_)

// One attention launch: the kernel for the head_dim, its arguments and grid.
struct FaLaunch {
  int32_t head_dim = 0;
  FaArgs p{};
  int64_t blocks = 0;  // 0: nothing to launch
  int32_t threads = 0;
};

template <int D>
int32_t geometry(FaLaunch& L) {
  using Cfg = FaConfig<D>;
  FaArgs& p = L.p;
  constexpr int BQ = 32 * Cfg::QB * Cfg::kWaves;
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
    // Twice the smallest group that fills them.  At the bench shape (32 slots, 16
    // blocks per head) groups of 1, 2, 4 and 8 heads measured 561, 531, 533 and 536 us
    // in one run, and 2 against 4 in ten alternating rounds 530.3 against 520.2 us;
    // their reads past the L2 (FETCH_SIZE) were 1.00x, 1.37x, 1.46x and 2.15x Q + K + V (one
    // head's K and V, 2 MiB, stay in the 4 MB L2 while its blocks run; more heads at
    // once compete for it, fewer leave the heavy blocks of later heads to the end).
    const int64_t slots = static_cast<int64_t>(cus) / 8 * Cfg::kWgPerCu;
    const int64_t g = 2 * ((slots + p.n_qblocks - 1) / p.n_qblocks);
    const int64_t heads_xcd = p.heads_total / 8;
    p.head_group = static_cast<int>(g < 1 ? 1 : (g > heads_xcd && heads_xcd > 0 ? heads_xcd : g));
  }
  const int64_t blocks = p.heads_total * p.n_qblocks;
  // one workgroup per (head, query block): the grid's x dimension and its thread count
  // (blocks x kWaves x 64) must fit 32 bits
  ASC_REQUIRE(blocks <= (int64_t{1} << 31) - 1 && blocks * Cfg::kWaves * 64 < (int64_t{1} << 32), ASC_ERR_UNSUPPORTED,
              "asc_flash_attention_fwd_bf16: %lld heads x %d query blocks exceed the launch grid limit",
              static_cast<long long>(p.heads_total), p.n_qblocks);
  L.blocks = blocks;
  L.threads = Cfg::kWaves * 64;
  return ASC_OK;
}

int32_t make_launch(const void* q, const void* k, const void* v, void* o, float* lse, int64_t batch, int64_t heads,
                    int64_t seq_len, int32_t head_dim, float sm_scale, int32_t causal, FaLaunch& L) {
  L = FaLaunch{};
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
  FaArgs& p = L.p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.heads_total = batch * heads;
  p.seq = static_cast<int>(seq_len);
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  p.causal = causal ? 1 : 0;
  L.head_dim = head_dim;
  return head_dim == 64 ? geometry<64>(L) : geometry<128>(L);
}

}  // namespace

extern "C" int32_t asc_flash_attention_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                                                int64_t batch, int64_t heads, int64_t seq_len, int32_t head_dim,
                                                float sm_scale, int32_t causal, asc_stream_t stream) {
  FaLaunch L;
  const int32_t rc = make_launch(q, k, v, o, lse, batch, heads, seq_len, head_dim, sm_scale, causal, L);
  if (rc != ASC_OK || L.blocks == 0) return rc;
  hipLaunchKernelGGL(L.head_dim == 64 ? fa_fwd_d64 : fa_fwd_d128, dim3(static_cast<uint32_t>(L.blocks)),
                     dim3(L.threads), 0, static_cast<hipStream_t>(stream), L.p);
  return asc::check_launch("asc_flash_attention_fwd_bf16");
}

extern "C" int32_t asc_flash_attention_plan(const void* q, const void* k, const void* v, void* o, float* lse,
                                            int64_t batch, int64_t heads, int64_t seq_len, int32_t head_dim,
                                            float sm_scale, int32_t causal, asc_launch_plan_t* plan) {
  ASC_REQUIRE(plan, ASC_ERR_INVALID_ARG, "asc_flash_attention_plan: null plan");
  *plan = asc_launch_plan_t{};
  FaLaunch L;
  const int32_t rc = make_launch(q, k, v, o, lse, batch, heads, seq_len, head_dim, sm_scale, causal, L);
  if (rc != ASC_OK || L.blocks == 0) return rc;
  static_assert(sizeof(FaArgs) <= sizeof(plan->args), "argument blob");
  __builtin_strncpy(plan->kernel, L.head_dim == 64 ? "asc2_fa_fwd_d64" : "asc2_fa_fwd_d128", sizeof(plan->kernel) - 1);
  plan->grid = static_cast<uint32_t>(L.blocks);
  plan->block = static_cast<uint32_t>(L.threads);
  plan->args_size = sizeof(FaArgs);
  __builtin_memcpy(plan->args, &L.p, sizeof(FaArgs));
  return ASC_OK;
}
