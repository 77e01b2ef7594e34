// Shared definitions of the gfx950 se_e2_a library: error plumbing, MFMA
// fragment types and wave-level helpers.
//
// MFMA fragment layouts on gfx950 (measured on MI355X, 64-lane wave,
// lane = 16*g + c with g = lane / 16, c = lane % 16):
//   v_mfma_f64_16x16x4f64  A[16x4]: lane holds A[c][g];  B[4x16]: lane holds B[g][c];
//                          D[16x16]: register r of lane holds D[g + 4r][c].
//   v_mfma_f32_16x16x4f32  A, B as above;  D: register r holds D[4g + r][c].
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

namespace dpamd {

typedef double d4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kMaxTypes = 8;

struct HipError {
  hipError_t code;
  std::string where;
};

#define DPAMD_HIP(expr)                                                            \
  do {                                                                             \
    hipError_t _e = (expr);                                                        \
    if (_e != hipSuccess) throw ::dpamd::HipError{_e, std::string(#expr) + " @ " + \
                                                         __FILE__ + ":" +          \
                                                         std::to_string(__LINE__)}; \
  } while (0)

#define DPAMD_LAUNCH_CHECK() DPAMD_HIP(hipGetLastError())

__device__ __forceinline__ d4 mfma_f64(double a, double b, d4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma_f32(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ d4 mfma(double a, double b, d4 c) { return mfma_f64(a, b, c); }
__device__ __forceinline__ f4 mfma(float a, float b, f4 c) { return mfma_f32(a, b, c); }

// Accumulator type and output-row mapping of the 16x16x4 MFMA per element type:
// register r of lane (g, c) holds D[row(g, r)][c].
template <class T>
struct Frag;
template <>
struct Frag<double> {
  using V = d4;
  static constexpr __host__ __device__ int row(int g, int r) { return g + 4 * r; }
};
template <>
struct Frag<float> {
  using V = f4;
  static constexpr __host__ __device__ int row(int g, int r) { return 4 * g + r; }
};

// Four consecutive elements read with 16-byte vector loads (one for float,
// two for double); the address must be 16-byte aligned.
template <class T>
struct alignas(16) Vec4 {
  T x, y, z, w;
};

// Make this wave's LDS writes visible to its own other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wait for every vector memory operation the wave has issued. Loads and
// stores share the vector memory counter, and with stores issued after a
// load the compiler's wait before the load's first use is vmcnt(0) or close to
// it (it does not treat stores as completing in order with loads), so that
// use also waits for the stores. A kernel that prefetches calls this where
// its loads have had their latency and no store has been issued since; the
// wait is visible to the compiler, and the later uses need none.
__device__ __forceinline__ void vmem_wait_all() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt(7), lgkmcnt(15): no wait
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ double shfl_xor_d(double v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

__device__ __forceinline__ float shfl_xor_d(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// v + shfl_xor(v, 16) and v + shfl_xor(v, 32) on the VALU, with no LDS round
// trip: v_permlane16_swap trades the odd 16-lane rows of its first operand
// with the even rows of its second, v_permlane32_swap the upper half of the
// first with the lower half of the second. With both operands = v, each lane
// then holds its own value and its xor partner's (in either order), and the
// sum equals v + shfl_xor(v, mask) exactly (addition commutes). Every lane of
// the wave must be active. The two results are copied to scalars before any
// bit cast: __builtin_bit_cast applied to an element of the returned vector
// has been compiled as a cast of element 0.
__device__ __forceinline__ unsigned lo32(double v) {
  return (unsigned)__builtin_bit_cast(unsigned long long, v);
}
__device__ __forceinline__ unsigned hi32(double v) {
  return (unsigned)(__builtin_bit_cast(unsigned long long, v) >> 32);
}
__device__ __forceinline__ double from32(unsigned hi, unsigned lo) {
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double add_xor16(double v) {
  const auto l = __builtin_amdgcn_permlane16_swap(lo32(v), lo32(v), true, false);
  const auto h = __builtin_amdgcn_permlane16_swap(hi32(v), hi32(v), true, false);
  const unsigned l0 = l[0], l1 = l[1], h0 = h[0], h1 = h[1];
  return from32(h0, l0) + from32(h1, l1);
}
__device__ __forceinline__ double add_xor32(double v) {
  const auto l = __builtin_amdgcn_permlane32_swap(lo32(v), lo32(v), true, false);
  const auto h = __builtin_amdgcn_permlane32_swap(hi32(v), hi32(v), true, false);
  const unsigned l0 = l[0], l1 = l[1], h0 = h[0], h1 = h[1];
  return from32(h0, l0) + from32(h1, l1);
}
__device__ __forceinline__ float add_xor16(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto s = __builtin_amdgcn_permlane16_swap(u, u, true, false);
  const unsigned a = s[0], b = s[1];
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float add_xor32(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto s = __builtin_amdgcn_permlane32_swap(u, u, true, false);
  const unsigned a = s[0], b = s[1];
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// The hardware deals a grid's workgroups to the XCDs round robin in linear-id
// order (x fastest), and each XCD has its own L2. xcd_swizzle() remaps the
// linear id so that consecutive logical blocks run on the same XCD: with x
// the column blocks of one row block, the blocks that read the same rows of
// A share one L2 instead of each XCD fetching them from HBM. A bijection on
// the grid for any block count.
constexpr int kXcds = 8;
__device__ __forceinline__ int3 xcd_swizzle() {
  const int nx = gridDim.x, ny = gridDim.y;
  const int nb = nx * ny * (int)gridDim.z;
  const int L = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
  const int q = nb / kXcds, r = nb % kXcds, x = L % kXcds;
  const int id = x * q + (x < r ? x : r) + L / kXcds;
  return int3{id % nx, (id / nx) % ny, id / (nx * ny)};
}

// Chunk walk of a persistent 1-D grid over `nchunks` equal chunks of work in
// a spatially ordered array: XCD x (the blocks b with b % 8 == x) takes the
// contiguous x-th eighth of the chunks and its blocks stride over it, so
// every neighbourhood is gathered through one XCD's L2 instead of all eight
// (a plain grid stride hands consecutive chunks to consecutive XCDs). Grids
// that are not a multiple of 8 blocks walk the plain stride.
struct ChunkWalk {
  int first, step, end;
};
__device__ __forceinline__ ChunkWalk xcd_chunks(int nchunks) {
  const int nb = gridDim.x, b = blockIdx.x;
  if (nb % kXcds != 0) return ChunkWalk{b, nb, nchunks};
  const int x = b % kXcds, q = nchunks / kXcds, r = nchunks % kXcds;
  const int beg = x * q + (x < r ? x : r);
  return ChunkWalk{beg + b / kXcds, nb / kXcds, beg + q + (x < r ? 1 : 0)};
}

// Status word bits raised by kernels and checked by the host after a step.
enum StatusBit : int {
  kStatusNeighbourOverflow = 1,  // > kMaxCand candidates within rcut of a centre
  kStatusReverseOverflow = 2,    // > kMaxRev edges pointing at one atom
  kStatusBadInput = 4,           // atom type or source index outside the model / graph
  kStatusSelOverflow = 8,        // more neighbours of one type than a strict sel holds
  kStatusFixedRange = 16,        // an edge gradient beyond the fixed-point accumulators' range
};

}  // namespace dpamd
