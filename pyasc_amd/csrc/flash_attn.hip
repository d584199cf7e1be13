#include "common.h"
extern "C" int32_t asc_flash_attention_fwd_bf16(const void*, const void*, const void*, void*, float*, int64_t,
                                                int64_t, int64_t, int32_t, float, int32_t, asc_stream_t) {
  return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_flash_attention_fwd_bf16: not built yet");
}
