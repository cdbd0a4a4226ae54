// Error reporting, device properties and the memory / IPC helpers of the C ABI.
// These replace the ctypes calls into libcudart of runtime/audit.py:17-23 and :55-60,
// runtime/audit_kernel.py:146-158 and observe/cuda.py:12-58.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "ekv_common.hpp"

namespace ekv {

static thread_local char g_error[512] = "";

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_hip(hipError_t err, const char *what) {
  if (err == hipSuccess) return EKV_OK;
  return fail(EKV_ELAUNCH, "%s failed: %s (%d)", what, hipGetErrorString(err), (int)err);
}

int cu_count() {
  constexpr int kMaxDevices = 64;
  static int cached[kMaxDevices] = {0};
  static std::mutex lock;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return 256;
  std::lock_guard<std::mutex> guard(lock);
  if (cached[device] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[device] = n;
  }
  return cached[device];
}

}  // namespace ekv

using namespace ekv;

extern "C" {

const char *ekv_last_error(void) { return g_error; }

int ekv_abi_version(void) { return 1; }

int ekv_malloc(void **ptr, size_t bytes) {
  if (ptr == nullptr || bytes == 0) return fail(EKV_EINVAL, "ekv_malloc: null pointer or zero size");
  *ptr = nullptr;
  return check_hip(hipMalloc(ptr, bytes), "hipMalloc");
}

int ekv_free(void *ptr) { return check_hip(hipFree(ptr), "hipFree"); }

int ekv_memset(void *ptr, int value, size_t bytes) {
  if (ptr == nullptr) return fail(EKV_EINVAL, "ekv_memset: null pointer");
  return check_hip(hipMemset(ptr, value, bytes), "hipMemset");
}

int ekv_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return EKV_OK;
  if (dst == nullptr || src == nullptr) return fail(EKV_EINVAL, "ekv_memcpy_h2d: null pointer");
  return check_hip(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

int ekv_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return EKV_OK;
  if (dst == nullptr || src == nullptr) return fail(EKV_EINVAL, "ekv_memcpy_d2h: null pointer");
  return check_hip(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

int ekv_ipc_handle(const void *ptr, uint8_t handle[64]) {
  if (ptr == nullptr || handle == nullptr) return fail(EKV_EINVAL, "ekv_ipc_handle: null pointer");
  static_assert(sizeof(hipIpcMemHandle_t) == 64, "an IPC handle is 64 bytes");
  hipIpcMemHandle_t h;
  int rc = check_hip(hipIpcGetMemHandle(&h, const_cast<void *>(ptr)), "hipIpcGetMemHandle");
  if (rc != EKV_OK) return rc;
  memcpy(handle, &h, 64);
  return EKV_OK;
}

int ekv_ipc_open(const uint8_t handle[64], void **ptr) {
  if (ptr == nullptr || handle == nullptr) return fail(EKV_EINVAL, "ekv_ipc_open: null pointer");
  hipIpcMemHandle_t h;
  memcpy(&h, handle, 64);
  *ptr = nullptr;
  int rc = check_hip(hipIpcOpenMemHandle(ptr, h, hipIpcMemLazyEnablePeerAccess), "hipIpcOpenMemHandle");
  if (rc == EKV_OK && *ptr == nullptr) return fail(EKV_ELAUNCH, "hipIpcOpenMemHandle returned null");
  return rc;
}

int ekv_synchronize(void) { return check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

int ekv_device_count(int *count) {
  if (count == nullptr) return fail(EKV_EINVAL, "ekv_device_count: null pointer");
  return check_hip(hipGetDeviceCount(count), "hipGetDeviceCount");
}

}  // extern "C"
