// Error plumbing and device queries of the C ABI.
#include <cstring>
#include <mutex>

#include "zk_common.h"

namespace zk {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = 0; }

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return ZK_OK;
}

int device_cus() {
  static std::mutex mu;
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace zk

extern "C" {

const char* zk_last_error(void) { return zk::g_last_error; }

int zk_abi_version(void) { return 4; }

int zk_device_info(int device, char* arch, int arch_len, int* num_cus,
                   int* max_clock_khz, int64_t* hbm_bytes) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    zk::set_error("zk_device_info: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  if (arch && arch_len > 0) {
    strncpy(arch, prop.gcnArchName, arch_len - 1);
    arch[arch_len - 1] = 0;
  }
  if (num_cus) *num_cus = prop.multiProcessorCount;
  if (max_clock_khz) *max_clock_khz = prop.clockRate;
  if (hbm_bytes) *hbm_bytes = static_cast<int64_t>(prop.totalGlobalMem);
  return ZK_OK;
}

}  // extern "C"
