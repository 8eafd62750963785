// Error reporting, version and device queries of libmingmoe.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "mm_common.h"

namespace mm {

static thread_local char g_last_error[1024] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MM_ERR_HIP, "HIP error in %s: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
  return MM_OK;
}

size_t dtype_size(int dtype) {
  switch (dtype) {
    case MM_BF16: case MM_FP16: return 2;
    case MM_FP32: case MM_INT32: return 4;
    case MM_INT8: return 1;
    case MM_INT64: return 8;
    default: return 0;
  }
}

int cu_count() {
  static std::mutex mu;
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

int allow_lds_ptr(const void* kernel, size_t bytes, const char* what) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> set;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = set[{kernel, dev}];
  if (bytes > have) {
    hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "HIP error setting LDS size of %s: %s", what, hipGetErrorString(e));
    have = bytes;
  }
  return MM_OK;
}

}  // namespace mm

extern "C" int mm_version(void) { return MM_ABI_VERSION; }

extern "C" size_t mm_last_error(char* buf, size_t len) {
  size_t n = strlen(mm::g_last_error);
  if (buf && len) {
    size_t c = n < len - 1 ? n : len - 1;
    memcpy(buf, mm::g_last_error, c);
    buf[c] = 0;
  }
  return n;
}
