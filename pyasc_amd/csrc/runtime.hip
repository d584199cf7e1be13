// Library-wide entry points: error reporting, version, device queries.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace asc {

int32_t set_error(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int32_t check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(static_cast<int32_t>(err), "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return ASC_OK;
}

}  // namespace asc

extern "C" {

const char* asc_last_error(void) { return g_last_error; }

const char* asc_version(void) { return "asc_hip 0.1.0 gfx950"; }

int32_t asc_device_info(int32_t device, int32_t* cu_count, int32_t* lds_bytes, int32_t* wave_size, char* arch) {
  hipDeviceProp_t prop;
  hipError_t err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) {
    return asc::set_error(static_cast<int32_t>(err), "asc_device_info: hipGetDeviceProperties(%d): %s", device,
                          hipGetErrorString(err));
  }
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (lds_bytes) *lds_bytes = static_cast<int32_t>(prop.sharedMemPerBlock);
  if (wave_size) *wave_size = prop.warpSize;
  if (arch) {
    strncpy(arch, prop.gcnArchName, 63);
    arch[63] = '\0';
  }
  return ASC_OK;
}

int32_t asc_stream_synchronize(asc_stream_t stream) {
  hipError_t err = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (err != hipSuccess) {
    return asc::set_error(static_cast<int32_t>(err), "asc_stream_synchronize: %s", hipGetErrorString(err));
  }
  return ASC_OK;
}

}  // extern "C"
