// Library-wide C-ABI entry points: version, thread-local error string and
// the cached per-device properties the launchers size their grids with.
#include <mutex>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "mf_common.h"

namespace mf {

static thread_local std::string g_last_error;

void set_last_error(const std::string& msg) { g_last_error = msg; }

int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int device_info(DeviceInfo* out) {
  static std::mutex mu;
  static std::vector<DeviceInfo> cache;
  int dev = 0;
  MF_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= static_cast<int>(cache.size())) cache.resize(dev + 1);
  DeviceInfo& info = cache[dev];
  if (info.device < 0) {
    int cus = 0, lds = 0;
    MF_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    MF_HIP_CHECK(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    info.num_cus = cus;
    info.max_lds_per_block = lds;
    info.device = dev;
  }
  *out = info;
  return MF_OK;
}

int ensure_dynamic_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::set<std::pair<std::pair<const void*, int>, int>> done;  // ((kernel, device), bytes)
  int dev = 0;
  MF_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(std::make_pair(kernel, dev), bytes);
  if (done.count(key)) return MF_OK;
  MF_HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
  done.insert(key);
  return MF_OK;
}

}  // namespace mf

extern "C" int mf_abi_version(void) { return MF_ABI_VERSION; }

extern "C" const char* mf_last_error(void) { return mf::g_last_error.c_str(); }
