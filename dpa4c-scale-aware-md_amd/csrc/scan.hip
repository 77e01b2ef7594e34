// Device-wide exclusive prefix sums of int arrays (ghost, cell, reverse-list
// and edge offsets), in two launches with no block ever waiting on another:
//   k_scan_parts: block b sums its tile of kScanTile elements into part[b];
//   k_scan_tiles: block b adds up part[0 .. b) itself (the block count is at
//     most a few thousand, so this costs a few loads per thread), then scans
//     its tile: the tile goes through LDS so that each thread owns kScanItems
//     consecutive elements, the thread totals are scanned within the wave
//     (shuffles) and across the block's waves (LDS), and each thread writes
//     its elements' exclusive sums.
// Integer addition is exact, so the result does not depend on any order.
// `in` and `out` must not overlap.
#include "kernels.h"

namespace dpamd {

namespace {

constexpr int kScanThreads = 256, kScanItems = 16, kScanTile = kScanThreads * kScanItems;
constexpr int kScanWaves = kScanThreads / kWave;
// tile in LDS with one pad int per 16 so that thread t's run of 16 starts in
// bank 17 t mod 64 (conflict-free reads of consecutive runs)
constexpr int kScanLds = kScanTile + kScanTile / 16;

__device__ __forceinline__ int lds_index(int e) { return e + (e >> 4); }

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// sum of v over the block (every thread gets it)
__device__ __forceinline__ int block_sum(int v, int* red) {
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  v = wave_sum(v);
  __syncthreads();  // red may still be read from a previous use
  if (lane == 0) red[w] = v;
  __syncthreads();
  int s = 0;
#pragma unroll
  for (int k = 0; k < kScanWaves; ++k) s += red[k];
  return s;
}

__global__ __launch_bounds__(kScanThreads) void k_scan_parts(const int* __restrict__ in, int n,
                                                             int* __restrict__ part) {
  __shared__ int red[kScanWaves];
  const long base = (long)blockIdx.x * kScanTile;
  int s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const long i = base + k * kScanThreads + threadIdx.x;
    if (i < n) s += in[i];
  }
  s = block_sum(s, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

__global__ __launch_bounds__(kScanThreads) void k_scan_tiles(const int* __restrict__ in, int n,
                                                             const int* __restrict__ part,
                                                             int* __restrict__ out) {
  __shared__ int tile[kScanLds];
  __shared__ int red[kScanWaves];
  __shared__ int wtot[kScanWaves];
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
  const long base = (long)blockIdx.x * kScanTile;
  // offset of this tile: the totals of the tiles before it
  int off = 0;
  for (int b = tid; b < (int)blockIdx.x; b += kScanThreads) off += part[b];
  off = block_sum(off, red);
  // coalesced load of the tile into LDS (zeros past n)
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int e = k * kScanThreads + tid;
    tile[lds_index(e)] = base + e < n ? in[base + e] : 0;
  }
  __syncthreads();
  // thread tid owns elements 16 tid .. 16 tid + 15
  int v[kScanItems], s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    v[k] = s;
    s += tile[lds_index(kScanItems * tid + k)];
  }
  // exclusive scan of the thread totals: within the wave, then over the waves
  int incl = s;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int u = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += u;
  }
  if (lane == kWave - 1) wtot[w] = incl;
  __syncthreads();
  int wbase = 0;
#pragma unroll
  for (int k = 0; k < kScanWaves; ++k) wbase += k < w ? wtot[k] : 0;
  const int tbase = off + wbase + incl - s;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) tile[lds_index(kScanItems * tid + k)] = tbase + v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int e = k * kScanThreads + tid;
    if (base + e < n) out[base + e] = tile[lds_index(e)];
  }
}

int scan_blocks(int n) { return (n + kScanTile - 1) / kScanTile; }

}  // namespace

size_t scan_temp_bytes(int n) { return sizeof(int) * (size_t)(scan_blocks(n) > 0 ? scan_blocks(n) : 1); }

void exclusive_scan_int(hipStream_t st, const int* in, int* out, int n, void* temp,
                        size_t temp_bytes) {
  if (n <= 0) return;
  const int nb = scan_blocks(n);
  if (temp_bytes < sizeof(int) * (size_t)nb)
    throw HipError{hipErrorInvalidValue, "exclusive_scan_int: temporary buffer too small"};
  int* part = static_cast<int*>(temp);
  if (nb > 1) {  // (a single tile has no earlier tiles to add up)
    hipLaunchKernelGGL(k_scan_parts, dim3(nb), dim3(kScanThreads), 0, st, in, n, part);
    DPAMD_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL(k_scan_tiles, dim3(nb), dim3(kScanThreads), 0, st, in, n, part, out);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace dpamd
