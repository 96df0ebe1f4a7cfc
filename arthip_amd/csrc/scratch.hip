// Device scratch of the no-allocation entry point (arthip_engine_run_device_noalloc).
//
// One file-scope array, which the code-object loader places on every GPU the
// library runs on and which stays there until the process ends. In host code
// the array's name is only a stand-in for the symbol: the address a kernel may
// use is the one hipGetSymbolAddress returns with the device current, resolved
// once per device and kept per device below.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <unordered_map>

#include "launch.h"

namespace arthip {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::unordered_map<int, void*> g_scratch_ptr;  // device -> address of its copy
}  // namespace

bool scratch_address(int device, void** ptr, std::string& error) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  const auto it = g_scratch_ptr.find(device);
  if (it != g_scratch_ptr.end()) {
    *ptr = it->second;
    return true;
  }
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) {
    error = std::string("hipGetSymbolAddress of the no-allocation scratch on device ") +
            std::to_string(device) + " failed: " + hipGetErrorString(e);
    return false;
  }
  g_scratch_ptr[device] = p;
  *ptr = p;
  return true;
}

}  // namespace arthip
