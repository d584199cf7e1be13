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

// ---- code objects (the counterpart of the reference's device-binary registration
// and KernelLaunchWrapper; see include/asc_hip.h)

int32_t asc_module_load(const char* path, void** module) {
  ASC_REQUIRE(path && module, ASC_ERR_INVALID_ARG, "asc_module_load: null argument");
  hipModule_t m = nullptr;
  const hipError_t err = hipModuleLoad(&m, path);
  if (err != hipSuccess) {
    return asc::set_error(static_cast<int32_t>(err), "asc_module_load: hipModuleLoad(%s): %s", path,
                          hipGetErrorString(err));
  }
  *module = m;
  return ASC_OK;
}

int32_t asc_module_unload(void* module) {
  ASC_REQUIRE(module, ASC_ERR_INVALID_ARG, "asc_module_unload: null module");
  const hipError_t err = hipModuleUnload(static_cast<hipModule_t>(module));
  if (err != hipSuccess) {
    return asc::set_error(static_cast<int32_t>(err), "asc_module_unload: %s", hipGetErrorString(err));
  }
  return ASC_OK;
}

int32_t asc_module_get_function(void* module, const char* name, void** function) {
  ASC_REQUIRE(module && name && function, ASC_ERR_INVALID_ARG, "asc_module_get_function: null argument");
  hipFunction_t f = nullptr;
  const hipError_t err = hipModuleGetFunction(&f, static_cast<hipModule_t>(module), name);
  if (err != hipSuccess) {
    return asc::set_error(static_cast<int32_t>(err), "asc_module_get_function(%s): %s", name,
                          hipGetErrorString(err));
  }
  *function = f;
  return ASC_OK;
}

int32_t asc_module_launch(void* function, uint32_t grid, uint32_t block, const void* args, uint64_t args_size,
                          asc_stream_t stream) {
  ASC_REQUIRE(function, ASC_ERR_INVALID_ARG, "asc_module_launch: null function");
  ASC_REQUIRE(grid > 0 && block > 0 && block <= 1024, ASC_ERR_INVALID_ARG,
              "asc_module_launch: grid %u / block %u out of range", grid, block);
  // one dispatch covers fewer than 2^32 threads
  ASC_REQUIRE(static_cast<uint64_t>(grid) * block < (uint64_t{1} << 32), ASC_ERR_UNSUPPORTED,
              "asc_module_launch: %u workgroups of %u threads exceed one launch", grid, block);
  ASC_REQUIRE(args_size == 0 || args, ASC_ERR_INVALID_ARG, "asc_module_launch: null argument blob");
  size_t size = static_cast<size_t>(args_size);
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(args), HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                    HIP_LAUNCH_PARAM_END};
  const hipError_t err = hipModuleLaunchKernel(static_cast<hipFunction_t>(function), grid, 1, 1, block, 1, 1, 0,
                                               static_cast<hipStream_t>(stream), nullptr, config);
  if (err != hipSuccess) {
    return asc::set_error(static_cast<int32_t>(err), "asc_module_launch: %s", hipGetErrorString(err));
  }
  return ASC_OK;
}

}  // extern "C"
