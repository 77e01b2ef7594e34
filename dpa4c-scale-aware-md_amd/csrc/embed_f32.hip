// Mixed-precision embedding kernels: the fp32 counterparts of the fp64
// forward and backward in embed.hip. The env row of each slot, its gradient
// and the edge gradient written for the force stage stay fp64; the nets, the
// T contraction and the u/v dot products are fp32 (reference precision rule
// for the mixed mode: fp32 embedding/fitting, fp64 env matrix, force and
// virial).
//
// The layer-2 and layer-3 products run on v_mfma_f32_16x16x32_bf16 at fp32
// accuracy: each fp32 operand is split exactly into three bf16 pieces and the
// six products that reach fp32 precision are accumulated in fp32 (mfma3). The
// weights are split once on the host (emb_shape.h), the activations and
// tangents in registers. On gfx950 the bf16 form does 8x the work of
// v_mfma_f32_16x16x4f32 in 0.65x its time.
//
// Work decomposition and tiles are those of the fp64 kernels. Unlike them,
// the forward saves no activations: the backward recomputes layers 2 and 3
// next to their tangents. On the bf16 matrix cores the products cost less
// than moving the 12 KB of fp32 activations per tile through HBM twice
// (measured on the 128,000-atom HEA: forward 2.50 -> 1.78 ms, backward
// 2.56 -> 3.18 ms, and the kernels after the forward no longer wait behind
// its write-back: step 9.75 -> 9.51 ms; saving layer 3 only was in between,
// 9.66 ms). What differs as well is the MFMA output layout: register r of lane
// (g, c) holds row 4g + r (fp64: g + 4r). Every layer therefore takes its
// k elements in the order that layout leaves the previous layer in
// registers: element e of 32-wide k chunk h of lane group g is feature
// 32h + 16(e/4) + 4g + e%4 (kf3 below with q = 8h + e), and the weights are
// packed in that order. Layer 1 (computed per lane) uses the same order when
// L1 is a multiple of 16, which keeps the layer-2 [x, x] residual in the
// lane's own registers.
//
// The forward's layer 3 is X2 W3 (register r of tile u: slot 4g + r, feature
// 16u + c); the backward recomputes it transposed, W3^T X2^T (feature 16u +
// 4g + r, slot c), with the six piece products in the forward's order
// (mfma3_t), so both kernels see the same activations bit for bit.
#include "bf16x3.h"
#include "env.h"
#include "fastmath.h"
#include "kernels.h"

namespace dpamd {

namespace {

// feature supplied by lane group g in k-step q of layer 3 (and of layer 2
// when L1 is a multiple of 16)
__device__ __forceinline__ int kf3(int q, int g) { return 16 * (q >> 2) + 4 * g + (q & 3); }

template <class S>
__device__ __forceinline__ int kf1(int q, int g) {
  if constexpr (S::X1_ALIGNED) return kf3(q, g);
  else return 4 * q + g;
}

// pre-split weights of (output tile, k chunk) block idx from LDS: three
// 16-byte reads, consecutive lanes on consecutive addresses
__device__ __forceinline__ Split3 wpieces(const float* region, int idx, int lane) {
  const bf8* w = reinterpret_cast<const bf8*>(region) + idx * 3 * 64 + lane;
  return Split3{w[0], w[64], w[128]};
}

// layer-3 input pieces of chunk h: element e is layer-2 result row
// 16(e/4) + 4g + e%4 of tile 2h + e/4 (x2[tile][row % 4] in the lane)
template <class S>
__device__ __forceinline__ Split3 x2_pieces(const float (&x2)[S::NT2][4], int h) {
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int t = 2 * h + (e >> 2);
    v[e] = t < S::NT2 ? x2[t][e & 3] : 0.0f;
  }
  return split3(v);
}

// Layer-3 output tiles per group (MFMA accumulators in flight). The forward
// is latency-bound on short neighbour sections (one or two tiles per item),
// so its registers go to occupancy: 128 VGPRs (4 waves per SIMD). The
// backward carries the recomputed primal next to the tangent and runs two
// waves per SIMD (up to 256 VGPRs; three waves spilled). An accumulation
// chain into one register issues back to back, so one or two tiles keep the
// matrix pipe fed.
constexpr int kU3F = 1;  // forward
constexpr int kU3B = 2;  // backward

template <class S>
constexpr int lds_params() {
  return (S::SIZE + 63) / 64 * 64;
}
template <class S>
constexpr int x2_ld() {
  return S::L2P + 4;
}
// LDS: padded net | env statistics of the pair (8 doubles = 16 floats) |
// per-wave scratch
template <class S>
constexpr int fwd_lds_floats(int waves) {
  return lds_params<S>() + 16 + waves * 16 * x2_ld<S>() + waves * 64;
}
// ... | per wave: dT and its folded copy (float) | the section-sum cells
// [16 slot lanes][12] (double, edge_out)
template <class S>
constexpr int bwd_lds_floats(int waves) {
  return lds_params<S>() + 16 + waves * 4 * (S::L3P + S::L2P) + waves * 2 * 16 * 12;
}

template <class S, int WAVES>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(4, 4))) void
k_embed_fwd32(EmbArgs a) {
  static_assert(S::L1 > 2, "layer-1 residual not supported");
  static_assert(S::K3P == S::L2P, "fp32 layout expected");
  extern __shared__ __align__(16) float lds32[];
  __shared__ int item_next;  // next item of the block (see the item loop)
  constexpr int PS = lds_params<S>();
  constexpr int X2LD = x2_ld<S>();
  float* P = lds32;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  double* EnvS = reinterpret_cast<double*>(lds32 + PS);  // PS is a multiple of 64
  float* X2s = lds32 + PS + 16 + w * 16 * X2LD;
  float* Rs = lds32 + PS + 16 + WAVES * 16 * X2LD + w * 64;

  const int p = find_pair(a);
  const int ti = p / a.ntypes, tj = p % a.ntypes;
  {
    const float* src = static_cast<const float*>(a.emb) + (long)p * a.stride;
    for (int q = threadIdx.x; q < S::SIZE; q += WAVES * 64) P[q] = src[q];
    if (threadIdx.x < 8) {
      const double v = a.envp[p * 8 + threadIdx.x];
      EnvS[threadIdx.x] = threadIdx.x < 4 ? v : 1.0 / v;  // avg[4], 1 / dstd[4]
    }
  }
  if (threadIdx.x == 0) item_next = 0;
  __syncthreads();
  const int nitems = a.type_off[ti + 1] - a.type_off[ti];
  // the block's WAVES * ipw items are handed out one at a time from an LDS
  // counter, so a wave whose items have few tiles takes more of them and the
  // block's waves finish together (the next block can start only when all
  // of this one's have)
  const int first_item = ((int)blockIdx.x - a.block_off[p]) * a.ipw * WAVES;
  for (;;) {
    int k = 0;
    if (lane == 0) k = atomicAdd(&item_next, 1);
    k = __builtin_amdgcn_readfirstlane(k);
    const int item = first_item + k;
    if (k >= a.ipw * WAVES || item >= nitems) break;
    const int i = a.items[a.type_off[ti] + item];
    const int nr = a.nreal[(long)i * a.ntypes + tj];
    const int* row = a.nlist + (long)i * a.nnei + a.sec[tj];
    // env statistics from LDS (staged once per block)
    const double* avg = EnvS;
    const double* sd = EnvS + 4;  // 1 / dstd
    const double xi = a.ext[3 * (long)i], yi = a.ext[3 * (long)i + 1], zi = a.ext[3 * (long)i + 2];

    float Tacc[S::NU3 * 4];
#pragma unroll
    for (int q = 0; q < S::NU3 * 4; ++q) Tacc[q] = 0.0f;
    // neighbour coordinates one tile ahead, their index two tiles ahead
    double nx0 = 0.0, nx1 = 0.0, nx2 = 0.0;
    if (c < nr) {
      const long j = row[c];
      nx0 = a.ext[3 * j];
      nx1 = a.ext[3 * j + 1];
      nx2 = a.ext[3 * j + 2];
    }
    int jn = 16 + c < nr ? row[16 + c] : 0;
    for (int tile = 0; tile < nr; tile += 16) {
      const int slot = tile + c;
      double Rn[4] = {0.0, 0.0, 0.0, 0.0};
      if (slot < nr) env_value(nx0 - xi, nx1 - yi, nx2 - zi, a.rcut_smth, a.rcut, a.inv_sw, avg, sd, Rn);
      if (slot + 16 < nr) {
        nx0 = a.ext[3 * (long)jn];
        nx1 = a.ext[3 * (long)jn + 1];
        nx2 = a.ext[3 * (long)jn + 2];
      }
      jn = slot + 32 < nr ? row[slot + 32] : 0;
      if (g == 0) {
#pragma unroll
        for (int m = 0; m < 4; ++m) Rs[c * 4 + m] = (float)Rn[m];
      }
      const float s = (float)Rn[0];

      // layer 1 -> B operand of layer 2: element e of k chunk h is feature
      // kf1(8h + e, g) of slot c
      float x1[8 * S::KC2];
#pragma unroll
      for (int q = 0; q < 8 * S::KC2; ++q) {
        const int f = kf1<S>(q, g);
        x1[q] = (f < S::L1) ? tanh_f32(s * P[S::OFF_W1 + f] + P[S::OFF_B1 + f]) : 0.0f;
      }
      // layer 2, transposed: register r of tile t is feature 16t + 4g + r
      f4 acc2[S::NT2];
      {
        Split3 xb[S::KC2];
#pragma unroll
        for (int h = 0; h < S::KC2; ++h) xb[h] = split3(x1 + 8 * h);
#pragma unroll
        for (int t = 0; t < S::NT2; ++t) {
          acc2[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int h = 0; h < S::KC2; ++h)
            acc2[t] = mfma3(wpieces(P + S::OFF_W2, t * S::KC2 + h, lane), xb[h], acc2[t]);
        }
      }
      float x2[S::NT2][4];
#pragma unroll
      for (int t = 0; t < S::NT2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int f = 16 * t + 4 * g + r;
          const float th = tanh_f32(acc2[t][r] + P[S::OFF_B2 + f]);
          float res = 0.0f;
          if constexpr (S::RES2 != 0) {
            if constexpr (S::X1_ALIGNED) {
              res = x1[(S::RES2 == 2 ? 4 * (t % (S::L1 / 16)) : 4 * t) + r];
            } else {
              const int f1 = (S::RES2 == 2) ? f % S::L1 : f;
              res = (f1 < S::L1) ? tanh_f32(s * P[S::OFF_W1 + f1] + P[S::OFF_B1 + f1]) : 0.0f;
            }
          }
          x2[t][r] = (f < S::L2) ? res + th : 0.0f;
        }
      }
      if constexpr (S::RES3 != 0) {
#pragma unroll
        for (int t = 0; t < S::NT2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) X2s[c * X2LD + 16 * t + 4 * g + r] = x2[t][r];
      }
      wave_lds_sync();
      // layer 3, non-transposed: register r of tile u is slot 4g + r, feature 16u + c
      Split3 xa[S::KC3];
#pragma unroll
      for (int h = 0; h < S::KC3; ++h) xa[h] = x2_pieces<S>(x2, h);
#pragma unroll
      for (int u0 = 0; u0 < S::NU3; u0 += kU3F) {
        __builtin_amdgcn_sched_barrier(0);
        f4 acc3[kU3F];
#pragma unroll
        for (int uu = 0; uu < kU3F; ++uu) acc3[uu] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int h = 0; h < S::KC3; ++h)
#pragma unroll
          for (int uu = 0; uu < kU3F; ++uu)
            if (u0 + uu < S::NU3)
              acc3[uu] = mfma3(xa[h], wpieces(P + S::OFF_W3, (u0 + uu) * S::KC3 + h, lane), acc3[uu]);
#pragma unroll
        for (int uu = 0; uu < kU3F; ++uu) {
          const int u = u0 + uu;
          if (u < S::NU3) {
            const int f = 16 * u + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int sl = 4 * g + r;
              const float th = tanh_f32(acc3[uu][r] + P[S::OFF_B3 + f]);
              float G = th;
              if constexpr (S::RES3 == 2) G += X2s[sl * X2LD + f % S::L2];
              if constexpr (S::RES3 == 1) G += X2s[sl * X2LD + f];
#pragma unroll
              for (int m = 0; m < 4; ++m) Tacc[u * 4 + m] += Rs[sl * 4 + m] * G;
            }
          }
        }
      }
      wave_lds_sync();
    }
#pragma unroll
    for (int q = 0; q < S::NU3 * 4; ++q) {
      float v = Tacc[q];
      v = add_xor32(add_xor16(v));
      Tacc[q] = v;
    }
    if (g == 0 && a.Tt) {
      // single neighbour type: this section is all of T
      const double npad = (double)(a.sel[tj] - nr);
      const double* tp = a.tpad + (long)p * 4 * S::L3;
      float* Tt = static_cast<float*>(a.Tt) + 4 * (long)(a.type_off[ti] + item);
#pragma unroll
      for (int u = 0; u < S::NU3; ++u) {
        const int f = 16 * u + c;
        if (f < S::L3) {
#pragma unroll
          for (int m = 0; m < 4; ++m)
            Tt[f * a.ldt + m] =
                (float)(((double)Tacc[u * 4 + m] + npad * tp[m * S::L3 + f]) * a.inv_nnei);
        }
      }
    } else if (g == 0) {
      float* out = static_cast<float*>(a.Tsec) + ((long)i * a.ntypes + tj) * 4 * S::L3;
#pragma unroll
      for (int u = 0; u < S::NU3; ++u) {
        const int f = 16 * u + c;
        if (f < S::L3) {
#pragma unroll
          for (int m = 0; m < 4; ++m) out[m * S::L3 + f] = Tacc[u * 4 + m];
        }
      }
    }
  }
  clear_fixed(a);
}

// AV: atom virials asked for (a.vacc non-null), see edge_out
template <class S, int WAVES, bool AV>
__global__ __launch_bounds__(WAVES * 64) void k_embed_bwd32(EmbArgs a) {
  static_assert(S::L1 > 2, "layer-1 residual not supported");
  static_assert(S::K3P == S::L2P, "fp32 layout expected");
  extern __shared__ __align__(16) float lds32[];
  __shared__ int item_next;  // next item of the block (see the item loop)
  constexpr int PS = lds_params<S>();
  float* P = lds32;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  double* EnvS = reinterpret_cast<double*>(lds32 + PS);  // PS is a multiple of 64
  float* dTs = lds32 + PS + 16 + w * 4 * (S::L3P + S::L2P);
  float* dTf = dTs + 4 * S::L3P;
  // 8-byte aligned: every region before it is a multiple of two floats
  double* own_w = reinterpret_cast<double*>(lds32 + PS + 16 + WAVES * 4 * (S::L3P + S::L2P)) + w * 16 * 12;

  const int p = find_pair(a);
  const int ti = p / a.ntypes, tj = p % a.ntypes;
  {
    const float* src = static_cast<const float*>(a.emb) + (long)p * a.stride;
    for (int q = threadIdx.x; q < S::SIZE; q += WAVES * 64) P[q] = src[q];
    if (threadIdx.x < 8) {
      const double v = a.envp[p * 8 + threadIdx.x];
      EnvS[threadIdx.x] = threadIdx.x < 4 ? v : 1.0 / v;  // avg[4], 1 / dstd[4]
    }
    for (int q = lane; q < 16 * 12; q += 64) own_w[q] = 0.0;
  }
  if (threadIdx.x == 0) item_next = 0;
  __syncthreads();
  const int nitems = a.type_off[ti + 1] - a.type_off[ti];
  // the block's WAVES * ipw items are handed out one at a time from an LDS
  // counter, so a wave whose items have few tiles takes more of them and the
  // block's waves finish together (the next block can start only when all
  // of this one's have)
  const int first_item = ((int)blockIdx.x - a.block_off[p]) * a.ipw * WAVES;
  for (;;) {
    int k = 0;
    if (lane == 0) k = atomicAdd(&item_next, 1);
    k = __builtin_amdgcn_readfirstlane(k);
    const int item = first_item + k;
    if (k >= a.ipw * WAVES || item >= nitems) break;
    const int i = a.items[a.type_off[ti] + item];
    const int nr = a.nreal[(long)i * a.ntypes + tj];
    const long ebase = (long)i * a.nnei + a.sec[tj];
    const int* row = a.nlist + ebase;
    // env statistics from LDS (staged once per block)
    const double* avg = EnvS;
    const double* sd = EnvS + 4;  // 1 / dstd
    const double xi = a.ext[3 * (long)i], yi = a.ext[3 * (long)i + 1], zi = a.ext[3 * (long)i + 2];
    {
      const float* dTi = static_cast<const float*>(a.dT) + (long)i * 4 * S::L3;
      for (int q = lane; q < 4 * S::L3P; q += 64) {
        const int m = q / S::L3P, f = q % S::L3P;
        dTs[q] = f < S::L3 ? dTi[m * S::L3 + f] : 0.0f;
      }
      for (int q = lane; q < 4 * S::L2P; q += 64) {
        const int m = q / S::L2P, f = q % S::L2P;
        float v = 0.0f;
        if (f < S::L2) {
          if constexpr (S::RES3 == 2) v = dTi[m * S::L3 + f] + dTi[m * S::L3 + f + S::L2];
          if constexpr (S::RES3 == 1) v = dTi[m * S::L3 + f];
        }
        dTf[q] = v;
      }
    }
    wave_lds_sync();

    // neighbour coordinates of tile k+1 fetched during tile k, the neighbour
    // index one tile earlier
    // (jx: the neighbour whose coordinates are in nx, for the slot's output)
    double nx0 = 0.0, nx1 = 0.0, nx2 = 0.0;
    int jn = 0, jx = 0;
    auto prefetch = [&](int tile) {
      if (tile + c < nr) {
        nx0 = a.ext[3 * (long)jn];
        nx1 = a.ext[3 * (long)jn + 1];
        nx2 = a.ext[3 * (long)jn + 2];
      }
      jx = jn;
      jn = tile + 16 + c < nr ? row[tile + 16 + c] : 0;
    };
    jn = c < nr ? row[c] : 0;
    if (nr > 0) prefetch(0);

    for (int tile = 0; tile < nr; tile += 16) {
      const int slot = tile + c;
      const bool valid = slot < nr;
      double d0 = 0.0, d1 = 0.0, d2 = 0.0;
      double Rn[4] = {0.0, 0.0, 0.0, 0.0};
      if (valid) {
        d0 = nx0 - xi;
        d1 = nx1 - yi;
        d2 = nx2 - zi;
        env_value(d0, d1, d2, a.rcut_smth, a.rcut, a.inv_sw, avg, sd, Rn);
      }
      const int jslot = jx;
      if (tile + 16 < nr) prefetch(tile + 16);
      const float s = (float)Rn[0];

      // layer 1 (recomputed) and its tangent
      float x1[8 * S::KC2], x1t[8 * S::KC2];
#pragma unroll
      for (int q = 0; q < 8 * S::KC2; ++q) {
        const int f = kf1<S>(q, g);
        if (f < S::L1) {
          const float wv = P[S::OFF_W1 + f];
          const float th = tanh_f32(s * wv + P[S::OFF_B1 + f]);
          x1[q] = th;
          x1t[q] = (1.0f - th * th) * wv;
        } else {
          x1[q] = 0.0f;
          x1t[q] = 0.0f;
        }
      }
      // layer 2 (transposed), the primal recomputed exactly as the forward
      // computed it, and its tangent
      f4 acc2[S::NT2], acc2t[S::NT2];
      {
        Split3 xb[S::KC2], xbt[S::KC2];
#pragma unroll
        for (int h = 0; h < S::KC2; ++h) {
          xb[h] = split3(x1 + 8 * h);
          xbt[h] = split3(x1t + 8 * h);
        }
#pragma unroll
        for (int t = 0; t < S::NT2; ++t) {
          acc2[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
          acc2t[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int h = 0; h < S::KC2; ++h) {
            const Split3 wp = wpieces(P + S::OFF_W2, t * S::KC2 + h, lane);
            acc2[t] = mfma3(wp, xb[h], acc2[t]);
            acc2t[t] = mfma3(wp, xbt[h], acc2t[t]);
          }
        }
      }
      float x2[S::NT2][4], x2t[S::NT2][4];
#pragma unroll
      for (int t = 0; t < S::NT2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int f = 16 * t + 4 * g + r;
          const float th = tanh_f32(acc2[t][r] + P[S::OFF_B2 + f]);
          float res = 0.0f, rest = 0.0f;
          if constexpr (S::RES2 != 0) {
            if constexpr (S::X1_ALIGNED) {
              const int q1 = (S::RES2 == 2 ? 4 * (t % (S::L1 / 16)) : 4 * t) + r;
              res = x1[q1];
              rest = x1t[q1];
            } else {
              const int f1 = (S::RES2 == 2) ? f % S::L1 : f;
              if (f1 < S::L1) {
                const float wv = P[S::OFF_W1 + f1];
                const float y = tanh_f32(s * wv + P[S::OFF_B1 + f1]);
                res = y;
                rest = (1.0f - y * y) * wv;
              }
            }
          }
          const bool live = f < S::L2;
          x2[t][r] = live ? res + th : 0.0f;
          x2t[t][r] = live ? rest + (1.0f - th * th) * acc2t[t][r] : 0.0f;
        }
      }
      // u = dT.G, v = dT.G': the layer-3 residual through the folded dT
      float up[4] = {0.0f, 0.0f, 0.0f, 0.0f}, vp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (S::RES3 != 0) {
#pragma unroll
        for (int t = 0; t < S::NT2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int f = 16 * t + 4 * g + r;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              const float wv = dTf[m * S::L2P + f];
              up[m] += wv * x2[t][r];
              vp[m] += wv * x2t[t][r];
            }
          }
      }
      // layer 3, transposed: register r of tile u is feature 16u + 4g + r.
      // The primal is recomputed with the forward's products in the forward's
      // order (mfma3_t: the transpose of the forward's X2 W3, bit for bit).
      Split3 xp[S::KC3], xt[S::KC3];
#pragma unroll
      for (int h = 0; h < S::KC3; ++h) {
        xp[h] = x2_pieces<S>(x2, h);
        xt[h] = x2_pieces<S>(x2t, h);
      }
#pragma unroll
      for (int u0 = 0; u0 < S::NU3; u0 += kU3B) {
        __builtin_amdgcn_sched_barrier(0);
        f4 acc3[kU3B], acc3t[kU3B];
#pragma unroll
        for (int uu = 0; uu < kU3B; ++uu) {
          acc3[uu] = f4{0.0f, 0.0f, 0.0f, 0.0f};
          acc3t[uu] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int h = 0; h < S::KC3; ++h)
#pragma unroll
          for (int uu = 0; uu < kU3B; ++uu)
            if (u0 + uu < S::NU3) {
              const Split3 wp = wpieces(P + S::OFF_W3, (u0 + uu) * S::KC3 + h, lane);
              acc3[uu] = mfma3_t(wp, xp[h], acc3[uu]);
              acc3t[uu] = mfma3(wp, xt[h], acc3t[uu]);
            }
#pragma unroll
        for (int uu = 0; uu < kU3B; ++uu) {
          const int u = u0 + uu;
          if (u < S::NU3) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int f = 16 * u + 4 * g + r;
              const float th = tanh_f32(acc3[uu][r] + P[S::OFF_B3 + f]);
              const float tt = (1.0f - th * th) * acc3t[uu][r];
#pragma unroll
              for (int m = 0; m < 4; ++m) {
                const float wv = dTs[m * S::L3P + f];
                up[m] += wv * th;
                vp[m] += wv * tt;
              }
            }
          }
        }
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        up[m] = add_xor32(add_xor16(up[m]));
        vp[m] = add_xor32(add_xor16(vp[m]));
      }
      // the slot's outputs: lane group 0 alone, or all four groups when atom
      // virials are asked for (edge_out shares the atomics out)
      if (valid && (AV || g == 0)) {
        double nd[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) nd[m] = (double)up[m] * a.inv_nnei;
        nd[0] += (Rn[0] * (double)vp[0] + Rn[1] * (double)vp[1] + Rn[2] * (double)vp[2] +
                  Rn[3] * (double)vp[3]) *
                 a.inv_nnei;
        // forces and virials as in the fp64 backward: the neighbour side in
        // fixed point onto slot jslot, the centre side into the lane's cells
        double gv[3];
        env_grad(d0, d1, d2, a.rcut_smth, a.rcut, a.inv_sw, sd, nd, gv);
        const double dv[3] = {d0, d1, d2};
        edge_out<AV>(a, ebase + slot, jslot, dv, gv, own_w + 12 * c, g);
      }
    }
    own_flush(a, i, tj, nr, ebase, own_w, lane);
  }
}

using ShapeWater32 = EmbShape<25, 50, 100, true>;
using ShapeMetal32 = EmbShape<32, 64, 128, true>;
// One block per CU holds the pre-split nets (about 61 KB) once: 16 waves
// (4 per SIMD) for the forward, 8 (2 per SIMD, its register budget) for the
// backward.
constexpr int kFwdWaves32 = 16;
constexpr int kBwdWaves32 = 8;

template <class S>
void fwd32_impl(hipStream_t st, const EmbArgs& a, int nblocks) {
  const size_t bytes = sizeof(float) * fwd_lds_floats<S>(kFwdWaves32);
  auto kern = k_embed_fwd32<S, kFwdWaves32>;
  DPAMD_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)bytes));
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(kFwdWaves32 * 64), bytes, st, a);
  DPAMD_LAUNCH_CHECK();
}

template <class S>
void bwd32_impl(hipStream_t st, const EmbArgs& a, int nblocks) {
  const size_t bytes = sizeof(float) * bwd_lds_floats<S>(kBwdWaves32);
  auto kern = a.vacc ? k_embed_bwd32<S, kBwdWaves32, true> : k_embed_bwd32<S, kBwdWaves32, false>;
  DPAMD_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)bytes));
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(kBwdWaves32 * 64), bytes, st, a);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace

int embed_waves_fwd32(const EmbLayout&) { return kFwdWaves32; }
int embed_waves_bwd32(const EmbLayout&) { return kBwdWaves32; }

void launch_embed_fwd32(hipStream_t st, const EmbLayout& e, const EmbArgs& a, int nblocks) {
  if (e.L1 == 25) fwd32_impl<ShapeWater32>(st, a, nblocks);
  else fwd32_impl<ShapeMetal32>(st, a, nblocks);
}

void launch_embed_bwd32(hipStream_t st, const EmbLayout& e, const EmbArgs& a, int nblocks) {
  if (e.L1 == 25) bwd32_impl<ShapeWater32>(st, a, nblocks);
  else bwd32_impl<ShapeMetal32>(st, a, nblocks);
}

}  // namespace dpamd
