// Static device workspace of the no-allocation entry point
// (dp_compute_device_noalloc): a file-scope device array, one copy per GPU,
// held until the process ends. Host code never uses the array's name as a
// device address: its per-device address comes from hipGetSymbolAddress,
// called once per device with that device current (at dp_create), and only
// that address is handed to the pipeline.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/dp_amd.h"
#include "kernels.h"

namespace dpamd {

namespace {
constexpr size_t kScratchBytes = DP_NOALLOC_SCRATCH_BYTES;  // 128 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};
// held by dp_compute_device_noalloc for a whole call: every handle on a
// device carves its buffers from the same scratch
std::mutex g_dev_mu[kMaxDevices];
}  // namespace

size_t noalloc_scratch_bytes() { return kScratchBytes; }

std::mutex& noalloc_device_mutex(int device) {
  if (device < 0 || device >= kMaxDevices)
    throw HipError{hipErrorInvalidDevice, "no-allocation scratch: device index out of range"};
  return g_dev_mu[device];
}

void* noalloc_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices)
    throw HipError{hipErrorInvalidDevice, "no-allocation scratch: device index out of range"};
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[device]) {
    void* p = nullptr;
    DPAMD_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_ptr[device] = p;
  }
  return g_ptr[device];
}

}  // namespace dpamd
