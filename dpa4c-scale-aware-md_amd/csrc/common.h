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

__device__ __forceinline__ double shfl_xor_d(double v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

__device__ __forceinline__ float shfl_xor_d(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// Status word bits raised by kernels and checked by the host after a step.
enum StatusBit : int {
  kStatusNeighbourOverflow = 1,  // > kMaxCand candidates within rcut of a centre
  kStatusReverseOverflow = 2,    // > kMaxRev edges pointing at one atom
  kStatusBadInput = 4,           // atom type or source index outside the model / graph
  kStatusSelOverflow = 8,        // more neighbours of one type than a strict sel holds
};

}  // namespace dpamd
