// Device scratch of the no-allocation entry point (arthip_engine_run_device_noalloc).
//
// One file-scope array, which the code-object loader places on every GPU the
// library runs on and which stays there until the process ends. In host code
// the array's name is only a stand-in for the symbol: the address a kernel may
// use is the one hipGetSymbolAddress returns with the device current, resolved
// once per device and kept per device below, next to the event that orders
// the calls of every engine handle that use that device's copy.
#include <hip/hip_runtime.h>

#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>

#include "launch.h"

namespace arthip {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

struct DeviceScratch {
  void* ptr = nullptr;         // this device's copy of `scratch`
  hipEvent_t done = nullptr;   // recorded at the end of every call that used it
  hipStream_t last = nullptr;  // stream of that call (null: none pending)
  std::mutex use;              // held from a call's first wait to its last record
};

std::mutex g_scratch_mu;
std::unordered_map<int, std::unique_ptr<DeviceScratch>> g_scratch;

DeviceScratch* find_device(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  const auto it = g_scratch.find(device);
  return it == g_scratch.end() ? nullptr : it->second.get();
}

}  // namespace

bool scratch_setup(int device, std::string& error) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch.count(device)) return true;
  auto d = std::make_unique<DeviceScratch>();
  hipError_t e = hipGetSymbolAddress(&d->ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || d->ptr == nullptr) {
    error = std::string("hipGetSymbolAddress of the no-allocation scratch on device ") +
            std::to_string(device) + " failed: " + hipGetErrorString(e);
    return false;
  }
  e = hipEventCreateWithFlags(&d->done, hipEventDisableTiming);
  if (e != hipSuccess) {
    error = std::string("hipEventCreate for the no-allocation scratch on device ") +
            std::to_string(device) + " failed: " + hipGetErrorString(e);
    return false;
  }
  g_scratch[device] = std::move(d);  // kept until the process ends, like the array
  return true;
}

ScratchUse::~ScratchUse() {
  if (locked_) static_cast<DeviceScratch*>(dev_)->use.unlock();
}

bool ScratchUse::Begin(int device, hipStream_t s, bool capturing, void** ptr,
                       std::string& error) {
  DeviceScratch* d = find_device(device);
  if (d == nullptr) {
    error = "the no-allocation scratch is not set up on device " + std::to_string(device) +
            " (its address or event could not be resolved when the engine started)";
    return false;
  }
  d->use.lock();
  dev_ = d;
  locked_ = true;
  stream_ = s;
  capturing_ = capturing;
  if (d->last != nullptr) {
    if (capturing) {
      // A captured call becomes graph nodes, which cannot wait on an event
      // recorded outside the capture: the last use must already be over.
      const hipError_t q = hipEventQuery(d->done);
      if (q == hipErrorNotReady) {
        error = "an earlier no-allocation call on this device is still executing; a call "
                "captured into a HIP graph cannot wait for it (synchronize before capturing)";
        return false;
      }
      if (q != hipSuccess) {
        error = std::string("hipEventQuery of the no-allocation scratch failed: ") +
                hipGetErrorString(q);
        return false;
      }
      d->last = nullptr;
    } else if (d->last != s) {
      const hipError_t w = hipStreamWaitEvent(s, d->done, 0);
      if (w != hipSuccess) {
        error = std::string("hipStreamWaitEvent on the last use of the no-allocation scratch "
                            "failed: ") +
                hipGetErrorString(w);
        return false;
      }
    }
  }
  *ptr = d->ptr;
  return true;
}

bool ScratchUse::End(std::string& error) {
  if (!locked_ || capturing_) return true;
  DeviceScratch* d = static_cast<DeviceScratch*>(dev_);
  // Recorded whether or not the call's launches all went out: what did go
  // out is on stream_, and the next user orders after it.
  const hipError_t r = hipEventRecord(d->done, stream_);
  if (r != hipSuccess) {
    error = std::string("hipEventRecord after a no-allocation call failed: ") +
            hipGetErrorString(r);
    d->last = nullptr;
    return false;
  }
  d->last = stream_;
  return true;
}

}  // namespace arthip
