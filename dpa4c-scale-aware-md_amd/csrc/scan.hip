// Device-wide exclusive scans (hipCUB / rocPRIM) used for ghost, cell and
// reverse-list offsets.
#include <hipcub/hipcub.hpp>

#include "kernels.h"

namespace dpamd {

size_t scan_temp_bytes(int n) {
  size_t bytes = 0;
  DPAMD_HIP(hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, (const int*)nullptr, (int*)nullptr, n));
  return bytes;
}

void exclusive_scan_int(hipStream_t st, const int* in, int* out, int n, void* temp,
                        size_t temp_bytes) {
  if (n <= 0) return;
  DPAMD_HIP(hipcub::DeviceScan::ExclusiveSum(temp, temp_bytes, in, out, n, st));
}

}  // namespace dpamd
