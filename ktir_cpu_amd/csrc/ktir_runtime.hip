// Runtime half of the C ABI: device selection, the library stream, memory,
// events and error reporting.  The simulated HBM of the reference
// (memory.py:311-398) is a single device arena allocated through these calls by
// the host runtime; the reference's sparse dict of NumPy arrays becomes plain
// device memory.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include "ktir_common.h"

namespace ktir {

static thread_local char g_err[1024] = "";
static hipStream_t g_stream = nullptr;
static int* g_err_flag = nullptr;
static int g_device = -1;

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

hipStream_t stream() { return g_stream; }
int* device_error_flag() { return g_err_flag; }

}  // namespace ktir

using namespace ktir;

extern "C" const char* ktir_last_error(void) { return g_err; }

extern "C" int ktir_init(int device) {
  if (g_device == device && g_stream) return KTIR_OK;
  int n = 0;
  KTIR_HIP_CHECK(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return set_error(KTIR_E_ARG, "ktir_init: device %d of %d", device, n);
  KTIR_HIP_CHECK(hipSetDevice(device));
  KTIR_HIP_CHECK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  KTIR_HIP_CHECK(hipMalloc((void**)&g_err_flag, sizeof(int)));
  KTIR_HIP_CHECK(hipMemsetAsync(g_err_flag, 0, sizeof(int), g_stream));
  KTIR_HIP_CHECK(hipStreamSynchronize(g_stream));
  g_device = device;
  return rmw_scratch_setup(device);
}

extern "C" int ktir_shutdown(void) {
  if (!g_stream) return KTIR_OK;
  KTIR_HIP_CHECK(hipStreamSynchronize(g_stream));
  KTIR_HIP_CHECK(hipFree(g_err_flag));
  KTIR_HIP_CHECK(hipStreamDestroy(g_stream));
  g_err_flag = nullptr;
  g_stream = nullptr;
  g_device = -1;
  return KTIR_OK;
}

extern "C" int ktir_device_info(int* cu_count, int* clock_khz, int64_t* hbm_bytes, char* name, int name_len) {
  hipDeviceProp_t p;
  int dev = g_device < 0 ? 0 : g_device;
  KTIR_HIP_CHECK(hipGetDeviceProperties(&p, dev));
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (clock_khz) *clock_khz = p.clockRate;
  if (hbm_bytes) *hbm_bytes = (int64_t)p.totalGlobalMem;
  if (name && name_len > 0) {
    snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
  }
  return KTIR_OK;
}

extern "C" int ktir_malloc(uint64_t bytes, uint64_t* dptr) {
  void* p = nullptr;
  KTIR_HIP_CHECK(hipMalloc(&p, bytes ? bytes : 1));
  *dptr = (uint64_t)p;
  return KTIR_OK;
}

extern "C" int ktir_free(uint64_t dptr) {
  KTIR_HIP_CHECK(hipStreamSynchronize(g_stream));
  KTIR_HIP_CHECK(hipFree((void*)dptr));
  return KTIR_OK;
}

extern "C" int ktir_memcpy_h2d(uint64_t dst, const void* src, uint64_t bytes) {
  if (!bytes) return KTIR_OK;
  KTIR_HIP_CHECK(hipMemcpyAsync((void*)dst, src, bytes, hipMemcpyHostToDevice, g_stream));
  KTIR_HIP_CHECK(hipStreamSynchronize(g_stream));
  return KTIR_OK;
}

extern "C" int ktir_memcpy_d2h(void* dst, uint64_t src, uint64_t bytes) {
  if (!bytes) return KTIR_OK;
  KTIR_HIP_CHECK(hipMemcpyAsync(dst, (const void*)src, bytes, hipMemcpyDeviceToHost, g_stream));
  KTIR_HIP_CHECK(hipStreamSynchronize(g_stream));
  return KTIR_OK;
}

extern "C" int ktir_memcpy_d2d(uint64_t dst, uint64_t src, uint64_t bytes) {
  if (!bytes) return KTIR_OK;
  KTIR_HIP_CHECK(hipMemcpyAsync((void*)dst, (const void*)src, bytes, hipMemcpyDeviceToDevice, g_stream));
  return KTIR_OK;
}

extern "C" int ktir_memset(uint64_t dst, int value, uint64_t bytes) {
  if (!bytes) return KTIR_OK;
  KTIR_HIP_CHECK(hipMemsetAsync((void*)dst, value, bytes, g_stream));
  return KTIR_OK;
}

extern "C" int ktir_sync(void) {
  KTIR_HIP_CHECK(hipStreamSynchronize(g_stream));
  return KTIR_OK;
}

extern "C" int ktir_check_error_flag(void) {
  int h = 0;
  KTIR_HIP_CHECK(hipMemcpyAsync(&h, g_err_flag, sizeof(int), hipMemcpyDeviceToHost, g_stream));
  KTIR_HIP_CHECK(hipStreamSynchronize(g_stream));
  if (h) {
    KTIR_HIP_CHECK(hipMemsetAsync(g_err_flag, 0, sizeof(int), g_stream));
    KTIR_HIP_CHECK(hipStreamSynchronize(g_stream));
    return set_error(KTIR_E_INDEX, "indirect index is negative");
  }
  return KTIR_OK;
}

// Timing events: no system-scope fence when one is recorded, so recording
// it does not write back and invalidate the caches between the launches it
// separates (elapsed times only need the timestamps; ktir_sync or
// ktir_event_elapsed_ms waits for completion).
extern "C" int ktir_event_create(uint64_t* ev) {
  hipEvent_t e;
  KTIR_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
  *ev = (uint64_t)e;
  return KTIR_OK;
}

extern "C" int ktir_event_record(uint64_t ev) {
  KTIR_HIP_CHECK(hipEventRecord((hipEvent_t)ev, g_stream));
  return KTIR_OK;
}

extern "C" int ktir_event_elapsed_ms(uint64_t start, uint64_t stop, float* ms) {
  KTIR_HIP_CHECK(hipEventSynchronize((hipEvent_t)stop));
  KTIR_HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return KTIR_OK;
}

extern "C" int ktir_event_destroy(uint64_t ev) {
  KTIR_HIP_CHECK(hipEventDestroy((hipEvent_t)ev));
  return KTIR_OK;
}
