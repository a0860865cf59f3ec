// Status reporting and device queries shared by every entry point of libwptv.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "wptv_common.h"

namespace wptv {

namespace {
thread_local char last_error[512] = "";
constexpr int kMaxDevices = 64;
int cu_count[kMaxDevices] = {0};
int draw_cap[kMaxDevices] = {0};
std::mutex cu_mutex;
}  // namespace

int fail(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(last_error, sizeof(last_error), fmt, args);
  va_end(args);
  return status;
}

int launched(const char* kernel) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(WPTV_E_HIP, "%s: launch failed: %s", kernel, hipGetErrorString(err));
  return WPTV_OK;
}

int compute_units() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return 256;
  std::lock_guard<std::mutex> lock(cu_mutex);
  if (cu_count[device] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) n = 256;
    cu_count[device] = n;
  }
  return cu_count[device];
}

int draw_workgroups_cap() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return -1;
  std::lock_guard<std::mutex> lock(cu_mutex);
  if (draw_cap[device] == 0) {
    int cus = 0, threads = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        hipDeviceGetAttribute(&threads, hipDeviceAttributeMaxThreadsPerMultiProcessor, device) != hipSuccess ||
        cus <= 0 || threads < 256)
      return -1;
    draw_cap[device] = cus * (threads / 256);
  }
  return draw_cap[device];
}

}  // namespace wptv

extern "C" int wptv_abi_version(void) { return WPTV_ABI_VERSION; }

extern "C" const char* wptv_last_error(void) { return wptv::last_error; }
