// Library runtime: device init, thread-local error strings, device properties.
#include "tg_common.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <mutex>

static thread_local char g_err[1024] = "";

void tg_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int tg_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    tg_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return TG_ERR_HIP;
  }
  return TG_OK;
}

static std::mutex g_mu;
static int g_cus[64];

int tg_num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_cus[dev] == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
      g_cus[dev] = prop.multiProcessorCount;
    else
      g_cus[dev] = 256;
  }
  return g_cus[dev];
}

TG_EXPORT const char* tg_last_error(void) { return g_err; }

TG_EXPORT int tg_version(void) { return 10000; }  // 1.0.0

// Select the device and verify it is a gfx950 part.  The kernels in this
// library are compiled for gfx950 only.
TG_EXPORT int tg_init(int device) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    tg_set_error("tg_init: no HIP device visible (%s)", hipGetErrorString(e));
    return TG_ERR_HIP;
  }
  if (device < 0 || device >= n) {
    tg_set_error("tg_init: device %d out of range [0,%d)", device, n);
    return TG_ERR_INVALID;
  }
  e = hipSetDevice(device);
  if (e != hipSuccess) {
    tg_set_error("tg_init: hipSetDevice(%d): %s", device, hipGetErrorString(e));
    return TG_ERR_HIP;
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    tg_set_error("tg_init: hipGetDeviceProperties: %s", hipGetErrorString(e));
    return TG_ERR_HIP;
  }
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    tg_set_error("tg_init: device %d is %s; libtgbwd is built for gfx950 only", device,
                 prop.gcnArchName);
    return TG_ERR_UNSUPPORTED;
  }
  tg_num_cus();
  return TG_OK;
}

TG_EXPORT int tg_stream_sync(void* stream) {
  hipError_t e = hipStreamSynchronize(tg_stream(stream));
  if (e != hipSuccess) {
    tg_set_error("tg_stream_sync: %s", hipGetErrorString(e));
    return TG_ERR_HIP;
  }
  return TG_OK;
}
