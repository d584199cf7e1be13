#include "common.h"
extern "C" int32_t asc_matmul_i8_i32(const int8_t*, const int8_t*, int32_t*, int64_t, int64_t, int64_t,
                                     asc_stream_t) {
  return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_matmul_i8_i32: not built yet");
}
extern "C" int32_t asc_matmul_i8_dequant_f16(const int8_t*, const int8_t*, const float*, void*, int64_t, int64_t,
                                             int64_t, int32_t, asc_stream_t) {
  return asc::set_error(ASC_ERR_UNSUPPORTED, "asc_matmul_i8_dequant_f16: not built yet");
}
