#include "common.h"
extern "C" int32_t asc_matmul(int32_t, int32_t, const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t,
                              int64_t, int64_t, int32_t, asc_stream_t) {
  return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_matmul: not built yet");
}
