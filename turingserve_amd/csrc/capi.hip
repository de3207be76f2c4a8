// C ABI plumbing: version, thread-local error messages, device queries and the
// paged_attention dispatcher (decode rows, then prefill sequences), which mirrors
// ops/triton_ops.py:60-71.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace ts {

static thread_local char g_err[512] = "";

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(TS_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TS_OK;
}

// The device `stream` belongs to (the current device for the null stream): the one whose
// kernels the call launches, whatever device the calling thread has current.
int stream_device(void* stream, int* device) {
  hipError_t e = stream ? hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), device)
                        : hipGetDevice(device);
  if (e != hipSuccess)
    return set_error(TS_ERR_DEVICE, "cannot tell the stream's device: %s", hipGetErrorString(e));
  return TS_OK;
}

int device_cu_count(void* stream, int* out) {
  int dev = 0;
  const int st = stream_device(stream, &dev);
  return st != TS_OK ? st : ts_device_cu_count(dev, out);
}

}  // namespace ts

extern "C" const char* ts_version(void) { return "turingserve_hip 0.1.0 gfx950"; }

extern "C" const char* ts_last_error(void) { return ts::g_err; }

extern "C" int ts_device_cu_count(int device, int* cu_count) {
  ts::clear_error();
  TS_REQUIRE(cu_count != nullptr, TS_ERR_INVALID_ARG, "device_cu_count: null output");
  // One cached answer per device (a startup query, like utils/gpu.py:19-24 behind lru_cache).
  static int cache[ts::kMaxDevices] = {0};
  if (device >= 0 && device < ts::kMaxDevices && cache[device] > 0) {
    *cu_count = cache[device];
    return TS_OK;
  }
  int n = 0;
  hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess || n <= 0)
    return ts::set_error(TS_ERR_DEVICE, "device_cu_count: hipDeviceGetAttribute failed: %s",
                         hipGetErrorString(e));
  if (device >= 0 && device < ts::kMaxDevices) cache[device] = n;
  *cu_count = n;
  return TS_OK;
}
