// Fused environment matrix + embedding net + descriptor contraction on
// gfx950 FP64 MFMA (v_mfma_f64_16x16x4f64), and its backward.
//
// Work unit: one wave owns one (centre i, neighbour section tj) item and walks
// its real slots in tiles of 16; a workgroup holds the padded weights of one
// (ti, tj) net in LDS and serves WAVES items of that pair. G itself is never
// written to HBM: the forward kernel contracts each tile into T on the fly.
//
// Forward, per tile (lane = 16g + c, slot column c):
//   env row R (fp64) -> s = R[0]
//   layer 1 (elementwise) produced directly as the B operand of layer 2
//   layer 2 transposed, Y2^T = W2^T X1^T: its D registers (row g+4r) are the
//      natural-order B operand (k = feature 4q+g) of the next product
//   layer 3 non-transposed, Y3 = X2 W3 (A operand = layer-2 registers), so
//      each lane holds G[slot g+4r][feature 16u+c]; the [x,x] residual comes
//      from an LDS copy of X2
//   T[m][f] += sum_slots R[slot][m] G[slot][f] on VALU, lane-local, reduced
//      over the 4 lane groups once per item.
// The forward also saves tanh of layers 2 and 3 (per tile of 16 slots, in the
// backward's register order) so the backward does not recompute the primal.
// Backward, per tile: layer 1 recomputed (elementwise), then the forward-mode
//   tangent dG/ds through layers 2 and 3 (transposed MFMAs), then u = dT.G and
//   v = dT.G' as lane-partial dot products; the layer-3 residual enters
//   through a folded dT (dT[f'] + dT[f'+L2]) against X2 itself, so no residual
//   is materialised. dE/dR = u/nnei, dE/ds = R.v/nnei, and the edge gradient
//   g = sum_m dE/dR_m dR_m/dd is written per slot.
//
// Reference analogs: the tabulated radial + PairFiLM embedding analog
// include/dpa_chain/graph_compress.cuh:91-154, the per-row moment accumulation
// deepmd-op/overlays/op/pt/dpa4c/raw_kernel.cuh:71-120, the "reproduce the
// amplitude instead of storing it" recompute backward
// include/dpa_chain/graph_compress.cuh:9-10 and
// deepmd-op/overlays/op/pt/dpa4c/graph_compress_kernel.cuh:1458-1466.
#include "env.h"
#include "fastmath.h"
#include "kernels.h"

namespace dpamd {

// Layer-3 output tiles per group: MFMA accumulation chains in flight. Both
// kernels run two waves per SIMD (LDS holds one block of eight waves per CU);
// an accumulation chain into one register issues back to back, so fewer
// chains cost no matrix throughput and free registers. Two measure fastest
// in the forward: 12,288-atom water 0.634 ms against 0.672 with four (which
// then spilled); with the forward at 232 registers three and four chains fit
// without spilling (244-254), and still run 2-3 % slower on water, 0.3 % on
// Cu. The backward keeps one (two spill 20-30 registers).
constexpr int kU3 = 2;
constexpr int kU3B = 1;

// LDS: padded net | env statistics of the pair (8) | table of the tanh
// (kTanhTab32, padded to kTanhTab) | per-wave scratch
constexpr int kTanhTab = 648;
static_assert(kTanhTab >= kTanhTabN && kTanhTab % 8 == 0, "tanh table slot");
template <class S>
constexpr int fwd_lds_doubles(int waves) {
  return (S::SIZE + 31) / 32 * 32 + 8 + kTanhTab + waves * 16 * (S::L2P + 2) + waves * 64;
}

// tanh of n values (groups of four sharing a reciprocal, the tail padded
// with zeros, which evaluate to 0)
template <int N>
__device__ __forceinline__ void tanh_n(const double* z, double* y, const double* tab) {
#pragma unroll
  for (int q0 = 0; q0 < N; q0 += 4) {
    double zz[4], yy[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) zz[j] = q0 + j < N ? z[q0 + j] : 0.0;
    tanh_tab4(zz, yy, tab);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (q0 + j < N) y[q0 + j] = yy[j];
  }
}

// A last output tile with at most four real features (water's 50 and 100:
// 2 and 4 of 16) costs a tile's MFMAs and tanh for a few values; the kernels
// form it on the VALU instead: lane (g, c) sums its slot's k elements against
// the tail columns, the four lane groups are added, and lane group g keeps
// tail feature g.
template <int L>
constexpr bool vtail() {
  return L % 16 != 0 && L % 16 <= 4;
}
// element g of v[0 .. N) (0 past N)
template <int N>
__device__ __forceinline__ double pick(const double (&v)[N], int g) {
  double r = 0.0;
#pragma unroll
  for (int j = 0; j < N; ++j) r = g == j ? v[j] : r;
  return r;
}
// sum over the 16 slot lanes (c) of a lane group
__device__ __forceinline__ double add_c16(double v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// layer-1 stash [16 slots][K2P + 1] per wave, for a layer-2 [x, x] residual
// whose features do not fall in the lane that computed them (L1 % 16 != 0)
template <class S>
constexpr int x1_stash_doubles() {
  return (S::RES2 != 0 && !S::X1_ALIGNED) ? 16 * (S::K2P + 1) : 0;
}

// ... | per wave: section-sum cells [16 slot lanes][12] (edge_out) and the
// neighbour indices of the current and the next tile, int [2][16]
template <class S>
constexpr int bwd_lds_doubles(int waves) {
  return (S::SIZE + 31) / 32 * 32 + 8 + kTanhTab + waves * 4 * (S::L3P + S::L2P) +
         waves * x1_stash_doubles<S>() + waves * (16 * 12 + 16);
}

template <class S, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void k_embed_fwd(EmbArgs a) {
  static_assert(S::L1 > 2, "layer-1 residual not supported");
  extern __shared__ double lds[];
  __shared__ int item_next;  // next item of the block (see the item loop)
  constexpr int PS = (S::SIZE + 31) / 32 * 32;
  constexpr int X2LD = S::L2P + 2;
  double* P = lds;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  double* EnvS = lds + PS;
  double* Tab = lds + PS + 8;
  double* X2s = lds + PS + 8 + kTanhTab + w * 16 * X2LD;
  double* Rs = lds + PS + 8 + kTanhTab + WAVES * 16 * X2LD + w * 64;

  const int p = find_pair(a);
  const int ti = p / a.ntypes, tj = p % a.ntypes;
  {
    const double* src = static_cast<const double*>(a.emb) + (long)p * a.stride;
    for (int q = threadIdx.x; q < S::SIZE; q += WAVES * 64) P[q] = src[q];
    if (threadIdx.x < 8) {
      const double v = a.envp[p * 8 + threadIdx.x];
      EnvS[threadIdx.x] = threadIdx.x < 4 ? v : 1.0 / v;  // avg[4], 1 / dstd[4]
    }
    for (int q = threadIdx.x; q < kTanhTab; q += WAVES * 64)
      Tab[q] = q < kTanhTabN ? kTanhTab32[q] : 0.0;
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
    // env statistics from LDS: a global load inside the tile loop would be
    // ordered behind the activation traffic by the in-order vector memory
    // counter
    const double* avg = EnvS;
    const double* sd = EnvS + 4;  // 1 / dstd
    const double xi = a.ext[3 * (long)i], yi = a.ext[3 * (long)i + 1], zi = a.ext[3 * (long)i + 2];

    // layer-2 / layer-3 tails on the VALU (vtail); U3 MFMA tiles of layer 3
    constexpr bool T2V = vtail<S::L2>(), T3V = vtail<S::L3>();
    constexpr int NT2M = S::NT2 - (T2V ? 1 : 0), U3 = S::NU3 - (T3V ? 1 : 0);
    double Tacc[S::NU3 * 4];
#pragma unroll
    for (int q = 0; q < S::NU3 * 4; ++q) Tacc[q] = 0.0;
    if (a.Tt) {
      // single neighbour type (T stored whole at the end): the padded slots'
      // constant share npad * tpad starts in the accumulators of lane group 0
      // (the tail's in slot lane 0), which the end-of-item sums then carry,
      // so the stores of T need no load behind the tile's stores
      // (every lane loads, at a clamped feature, so that the loads issue
      // together and are waited for once)
      const double npad = (double)(a.sel[tj] - nr);
      const double* tp = a.tpad + (long)p * 4 * S::L3;
      double tv[S::NU3][4];
#pragma unroll
      for (int u = 0; u < S::NU3; ++u) {
        const int f = min(u < U3 ? 16 * u + c : 16 * U3 + g, S::L3 - 1);
#pragma unroll
        for (int m = 0; m < 4; ++m) tv[u][m] = tp[m * S::L3 + f];
      }
#pragma unroll
      for (int u = 0; u < U3; ++u) {
        const bool own = g == 0 && 16 * u + c < S::L3;
#pragma unroll
        for (int m = 0; m < 4; ++m) Tacc[u * 4 + m] = own ? npad * tv[u][m] : 0.0;
      }
      if constexpr (T3V) {
        const bool own = c == 0 && 16 * U3 + g < S::L3;
#pragma unroll
        for (int m = 0; m < 4; ++m) Tacc[4 * U3 + m] = own ? npad * tv[U3][m] : 0.0;
      }
    }
    constexpr int BLK = 16 * (S::L2P + S::L3P);
    double* act = static_cast<double*>(a.act) + ((long)i * a.tiles_per_atom + a.tile_off[tj]) * BLK;
    // the layer-3 tail's activation (slot c, feature 16 U3 + g), where the
    // backward reads tile U3's register 0
    double* act3t = act + 16 * S::L2P + 256 * U3 + 4 * c + g;

    // per-lane bases: layer 2 element (t, r) at act2[(4t + r) * 64], layer 3
    // element (u, r) of slot g + 4r at act3[256u + 16r]. The activations are
    // written with non-temporal stores: only the backward kernel reads them,
    // so they stay out of the caches the tiles' coordinate gathers use
    // (measured: 3 % off this kernel on Cu).
    double* act2 = act + c * 4 + g;
    double* act3 = act + 16 * S::L2P + (c >> 2) * 64 + g * 4 + (c & 3);
    // Neighbour coordinates of tile k+1 are fetched at the start of tile k,
    // from an index loaded one tile earlier, and waited for after tile k's
    // layer-2 products, before its first activation store (vmem_wait_all):
    // a wait at their use in tile k+1 would also wait for tile k's stores.
    // The index loads are unconditional, clamped into the section (sel >= 1),
    // so the index register is written by loads only (a conditional zero
    // would be a VALU write behind a pending load, which the compiler covers
    // with a wait on every outstanding memory operation).
    const int slast = a.sel[tj] - 1;
    double nx0 = 0.0, nx1 = 0.0, nx2 = 0.0;
    if (c < nr) {
      const long j = row[c];
      nx0 = a.ext[3 * j];
      nx1 = a.ext[3 * j + 1];
      nx2 = a.ext[3 * j + 2];
    }
    int jn = row[min(16 + c, slast)];
    vmem_wait_all();  // so that no use in the tile loop waits (see above)
    for (int tile = 0; tile < nr; tile += 16, act2 += BLK, act3 += BLK, act3t += BLK) {
      const int slot = tile + c;
      double Rn[4] = {0.0, 0.0, 0.0, 0.0};
      if (slot < nr) env_value(nx0 - xi, nx1 - yi, nx2 - zi, a.rcut_smth, a.rcut, a.inv_sw, avg, sd, Rn);
      if (slot + 16 < nr) {
        nx0 = a.ext[3 * (long)jn];
        nx1 = a.ext[3 * (long)jn + 1];
        nx2 = a.ext[3 * (long)jn + 2];
      }
      jn = row[min(slot + 32, slast)];
      if (g == 0) {
#pragma unroll
        for (int m = 0; m < 4; ++m) Rs[c * 4 + m] = Rn[m];
      }
      const double s = Rn[0];

      // layer 1 -> B operand of layer 2 (feature 4q+g of slot c), four at a
      // time (shared reciprocal); padded features have zero weights and bias
      double x1[S::NQ2];
      {
        double z[S::NQ2];
#pragma unroll
        for (int q = 0; q < S::NQ2; ++q) {
          const int f = 4 * q + g;
          z[q] = s * P[S::OFF_W1 + f] + P[S::OFF_B1 + f];
        }
        tanh_n<S::NQ2>(z, x1, Tab);
      }
      // a residual feature f % L1 lives in another lane group: stash layer 1
      // in this wave's X2 buffer (overwritten by X2 only after every read)
      constexpr int X1LD = S::K2P + 1;
      if constexpr (S::RES2 != 0 && !S::X1_ALIGNED) {
#pragma unroll
        for (int q = 0; q < S::NQ2; ++q) X2s[c * X1LD + 4 * q + g] = x1[q];
        wave_lds_sync();
      }
      // layer 2, transposed
      d4 acc2[S::NT2];
#pragma unroll
      for (int t = 0; t < S::NT2; ++t) acc2[t] = d4{0.0, 0.0, 0.0, 0.0};
      // (the epilogue's biases are read before the last k-step's products)
      double b2v[NT2M > 0 ? NT2M : 1][4];
#pragma unroll
      for (int q = 0; q < S::NQ2; ++q) {
        if (q + 1 == S::NQ2) {
#pragma unroll
          for (int t = 0; t < NT2M; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) b2v[t][r] = P[S::OFF_B2 + 16 * t + 4 * r + g];
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int t = 0; t < NT2M; ++t)
          acc2[t] = mfma_f64(P[S::OFF_W2 + (4 * q + g) * S::L2P + 16 * t + c], x1[q], acc2[t]);
      }
      double x2[S::NT2][4];
      if constexpr (T2V) {
        // tail features 16 NT2M + j: register 0 of tile NT2M (lane group g: j = g)
        constexpr int TL = S::L2 % 16;
        double pj[TL];
#pragma unroll
        for (int j = 0; j < TL; ++j) pj[j] = 0.0;
#pragma unroll
        for (int q = 0; q < S::NQ2; ++q) {
          const double* wr = P + S::OFF_W2 + (4 * q + g) * S::L2P + 16 * NT2M;
#pragma unroll
          for (int j = 0; j < TL; ++j) pj[j] = fma(x1[q], wr[j], pj[j]);
        }
#pragma unroll
        for (int j = 0; j < TL; ++j) pj[j] = add_xor32(add_xor16(pj[j]));
        const int f = 16 * NT2M + g;
        const double th = tanh_tab1(pick(pj, g) + P[S::OFF_B2 + f], Tab);
        // the next tile's coordinates and index have landed (see the loop
        // head); this tile's stores start here
        vmem_wait_all();
        __builtin_nontemporal_store(th, &act2[(4 * NT2M) * 64]);
        double res = 0.0;
        if constexpr (S::RES2 != 0) {
          if constexpr (S::X1_ALIGNED) {
            res = x1[(S::RES2 == 2 ? 4 * (NT2M % (S::L1 / 16)) : 4 * NT2M)];
          } else {
            const int f1 = (S::RES2 == 2) ? f % S::L1 : f;
            res = (f1 < S::L1) ? X2s[c * X1LD + f1] : 0.0;
          }
        }
        x2[NT2M][0] = (f < S::L2) ? res + th : 0.0;
        x2[NT2M][1] = x2[NT2M][2] = x2[NT2M][3] = 0.0;
      } else {
        vmem_wait_all();  // as above, before this tile's first store
      }
#pragma unroll
      for (int t = 0; t < NT2M; ++t) {
        double z2[4], th2v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) z2[r] = acc2[t][r] + b2v[t][r];
        tanh_tab4(z2, th2v, Tab);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int f = 16 * t + 4 * r + g;
          const double th = th2v[r];
          __builtin_nontemporal_store(th, &act2[(4 * t + r) * 64]);
          double res = 0.0;
          if constexpr (S::RES2 != 0) {
            if constexpr (S::X1_ALIGNED) {
              res = x1[(S::RES2 == 2 ? 4 * (t % (S::L1 / 16)) : 4 * t) + r];
            } else {
              const int f1 = (S::RES2 == 2) ? f % S::L1 : f;
              res = (f1 < S::L1) ? X2s[c * X1LD + f1] : 0.0;
            }
          }
          x2[t][r] = (f < S::L2) ? res + th : 0.0;
        }
      }
      if constexpr (S::RES3 != 0) {
#pragma unroll
        for (int t = 0; t < S::NT2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) X2s[c * X2LD + 16 * t + 4 * r + g] = x2[t][r];
      }
      wave_lds_sync();
      // layer 3, non-transposed, two output tiles at a time
#pragma unroll
      for (int u0 = 0; u0 < U3; u0 += kU3) {
        __builtin_amdgcn_sched_barrier(0);
        d4 acc3[kU3];
#pragma unroll
        for (int uu = 0; uu < kU3; ++uu) acc3[uu] = d4{0.0, 0.0, 0.0, 0.0};
        double wcur[kU3], wnxt[kU3];
        const double* W3 = P + S::OFF_W3 + g * S::L3P + 16 * u0 + c;
#pragma unroll
        for (int uu = 0; uu < kU3; ++uu) wcur[uu] = u0 + uu < U3 ? W3[16 * uu] : 0.0;
        double b3v[kU3], resv[kU3][4];
#pragma unroll
        for (int q = 0; q < S::NQ3; ++q) {
          if (q + 1 < S::NQ3) {
#pragma unroll
            for (int uu = 0; uu < kU3; ++uu)
              wnxt[uu] = u0 + uu < U3 ? W3[4 * (q + 1) * S::L3P + 16 * uu] : 0.0;
          } else {
            // the epilogue's bias and residual values, read during the last product
#pragma unroll
            for (int uu = 0; uu < kU3; ++uu) {
              const int f = 16 * (u0 + uu) + c;
              b3v[uu] = u0 + uu < U3 ? P[S::OFF_B3 + f] : 0.0;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int sl = g + 4 * r;
                resv[uu][r] = 0.0;
                if (u0 + uu < U3) {
                  if constexpr (S::RES3 == 2) resv[uu][r] = X2s[sl * X2LD + f % S::L2];
                  if constexpr (S::RES3 == 1) resv[uu][r] = X2s[sl * X2LD + f];
                }
              }
            }
          }
          const double av = x2[q / 4][q % 4];
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int uu = 0; uu < kU3; ++uu)
            if (u0 + uu < U3) acc3[uu] = mfma_f64(av, wcur[uu], acc3[uu]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int uu = 0; uu < kU3; ++uu) wcur[uu] = wnxt[uu];
        }
#pragma unroll
        for (int uu = 0; uu < kU3; ++uu) {
          const int u = u0 + uu;
          if (u < U3) {
            double z3[4], th3v[4];
            const double b3 = b3v[uu];
#pragma unroll
            for (int r = 0; r < 4; ++r) z3[r] = acc3[uu][r] + b3;
            tanh_tab4(z3, th3v, Tab);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int sl = g + 4 * r;
              const double th = th3v[r];
              // backward order: feature 16u + 4(c>>2) + (c&3) of slot sl
              __builtin_nontemporal_store(th, &act3[256 * u + 16 * r]);
              const double G = th + resv[uu][r];
#pragma unroll
              for (int m = 0; m < 4; ++m) Tacc[u * 4 + m] += Rs[sl * 4 + m] * G;
            }
          }
        }
      }
      if constexpr (T3V) {
        // tail features 16 U3 + j of this lane's slot c (lane group g: j = g);
        // T of the tail accumulates per slot lane (Tacc[4 U3 + m], summed over
        // the slot lanes at the end of the item)
        constexpr int TL = S::L3 % 16;
        double pj[TL];
#pragma unroll
        for (int j = 0; j < TL; ++j) pj[j] = 0.0;
#pragma unroll
        for (int t = 0; t < S::NT2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (16 * t + 4 * r >= 4 * S::NQ3) continue;  // past W3's rows (x2 is 0 there)
            const double* wr = P + S::OFF_W3 + (16 * t + 4 * r + g) * S::L3P + 16 * U3;
#pragma unroll
            for (int j = 0; j < TL; ++j) pj[j] = fma(x2[t][r], wr[j], pj[j]);
          }
#pragma unroll
        for (int j = 0; j < TL; ++j) pj[j] = add_xor32(add_xor16(pj[j]));
        const int f = 16 * U3 + g;
        const double th = tanh_tab1(pick(pj, g) + P[S::OFF_B3 + f], Tab);
        __builtin_nontemporal_store(th, act3t);
        double G = th;
        if constexpr (S::RES3 == 2) G += X2s[c * X2LD + f % S::L2];
        if constexpr (S::RES3 == 1) G += X2s[c * X2LD + f];
#pragma unroll
        for (int m = 0; m < 4; ++m) Tacc[4 * U3 + m] += Rn[m] * G;
      }
      wave_lds_sync();
    }
#pragma unroll
    for (int q = 0; q < U3 * 4; ++q) {
      double v = Tacc[q];
      v = add_xor32(add_xor16(v));
      Tacc[q] = v;
    }
    if constexpr (T3V) {
      // the tail's T: summed over the slot lanes, held by lane (g, 0) for
      // feature 16 U3 + g
#pragma unroll
      for (int m = 0; m < 4; ++m) Tacc[4 * U3 + m] = add_c16(Tacc[4 * U3 + m]);
      constexpr int TL = S::L3 % 16;
      if (c == 0 && g < TL) {
        const int f = 16 * U3 + g;
        if (a.Tt) {
          double* Tt = static_cast<double*>(a.Tt) + 4 * (long)(a.type_off[ti] + item);
#pragma unroll
          for (int m = 0; m < 4; ++m) Tt[f * a.ldt + m] = Tacc[4 * U3 + m] * a.inv_nnei;
        } else {
          double* out = static_cast<double*>(a.Tsec) + ((long)i * a.ntypes + tj) * 4 * S::L3;
#pragma unroll
          for (int m = 0; m < 4; ++m) out[m * S::L3 + f] = Tacc[4 * U3 + m];
        }
      }
    }
    if (g == 0 && a.Tt) {
      // single neighbour type: this section (padding share included) is all of T
      double* Tt = static_cast<double*>(a.Tt) + 4 * (long)(a.type_off[ti] + item);
#pragma unroll
      for (int u = 0; u < U3; ++u) {
        const int f = 16 * u + c;
        if (f < S::L3) {
#pragma unroll
          for (int m = 0; m < 4; ++m) Tt[f * a.ldt + m] = Tacc[u * 4 + m] * a.inv_nnei;
        }
      }
    } else if (g == 0) {
      double* out = static_cast<double*>(a.Tsec) + ((long)i * a.ntypes + tj) * 4 * S::L3;
#pragma unroll
      for (int u = 0; u < U3; ++u) {
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
__global__ __launch_bounds__(WAVES * 64) void k_embed_bwd(EmbArgs a) {
  static_assert(S::L1 > 2, "layer-1 residual not supported");
  extern __shared__ double lds[];
  __shared__ int item_next;  // next item of the block (see the item loop)
  constexpr int PS = (S::SIZE + 31) / 32 * 32;
  double* P = lds;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  double* EnvS = lds + PS;
  double* Tab = lds + PS + 8;
  double* dTs = lds + PS + 8 + kTanhTab + w * 4 * (S::L3P + S::L2P);
  double* dTf = dTs + 4 * S::L3P;
  // layer-1 stash (see x1_stash_doubles)
  double* X1s =
      lds + PS + 8 + kTanhTab + WAVES * 4 * (S::L3P + S::L2P) + w * x1_stash_doubles<S>();
  constexpr int X1LD = S::K2P + 1;
  double* own_w = lds + PS + 8 + kTanhTab + WAVES * 4 * (S::L3P + S::L2P) +
                  WAVES * x1_stash_doubles<S>() + w * (16 * 12 + 16);
  int* jbuf = reinterpret_cast<int*>(own_w + 16 * 12);

  const int p = find_pair(a);
  const int ti = p / a.ntypes, tj = p % a.ntypes;
  {
    const double* src = static_cast<const double*>(a.emb) + (long)p * a.stride;
    for (int q = threadIdx.x; q < S::SIZE; q += WAVES * 64) P[q] = src[q];
    if (threadIdx.x < 8) {
      const double v = a.envp[p * 8 + threadIdx.x];
      EnvS[threadIdx.x] = threadIdx.x < 4 ? v : 1.0 / v;  // avg[4], 1 / dstd[4]
    }
    for (int q = lane; q < 16 * 12; q += 64) own_w[q] = 0.0;
    for (int q = threadIdx.x; q < kTanhTab; q += WAVES * 64)
      Tab[q] = q < kTanhTabN ? kTanhTab32[q] : 0.0;
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
    // env statistics from LDS: a global load inside the tile loop would be
    // ordered behind the activation traffic by the in-order vector memory
    // counter
    const double* avg = EnvS;
    const double* sd = EnvS + 4;  // 1 / dstd
    const double xi = a.ext[3 * (long)i], yi = a.ext[3 * (long)i + 1], zi = a.ext[3 * (long)i + 2];
    constexpr int BLK = 16 * (S::L2P + S::L3P);
    const double* act = static_cast<double*>(a.act) + ((long)i * a.tiles_per_atom + a.tile_off[tj]) * BLK;

    {
      const double* dTi = static_cast<const double*>(a.dT) + (long)i * 4 * S::L3;
      for (int q = lane; q < 4 * S::L3P; q += 64) {
        const int m = q / S::L3P, f = q % S::L3P;
        dTs[q] = f < S::L3 ? dTi[m * S::L3 + f] : 0.0;
      }
      for (int q = lane; q < 4 * S::L2P; q += 64) {
        const int m = q / S::L2P, f = q % S::L2P;
        double v = 0.0;
        if (f < S::L2) {
          if constexpr (S::RES3 == 2) v = dTi[m * S::L3 + f] + dTi[m * S::L3 + f + S::L2];
          if constexpr (S::RES3 == 1) v = dTi[m * S::L3 + f];
        }
        dTf[q] = v;
      }
    }
    wave_lds_sync();

    const double* act2 = act + c * 4 + g;  // element (t, r) at act2[64 (4t + r)]
    const double* act3 = act2 + 16 * S::L2P;  // element (u, r) at act3[256u + 64r]
    // Neighbour coordinates of tile k+1 are fetched during tile k (their index
    // one tile earlier, so the memory counter never orders them behind other
    // loads). The saved activations of a tile are loaded at its start and
    // consumed after the layer-2 and layer-3 products: their latency is covered
    // by those products and by the other wave of the SIMD. Holding them a whole
    // tile ahead would need the registers of that second wave.
    // The neighbour index of each slot is parked in LDS (jbuf, by tile
    // parity) when its coordinates are fetched, for the slot's output.
    // (index loads unconditional and clamped into the section, as in the
    // forward; jbuf entries of padded slots are never read)
    const int slast = a.sel[tj] - 1;
    double nx0 = 0.0, nx1 = 0.0, nx2 = 0.0;
    int jn = row[min(c, slast)];
    if (c < nr) {
      nx0 = a.ext[3 * (long)jn];
      nx1 = a.ext[3 * (long)jn + 1];
      nx2 = a.ext[3 * (long)jn + 2];
    }
    if (g == 0) jbuf[c] = jn;
    jn = row[min(16 + c, slast)];
    // The coordinates and index loaded for the next tile are waited for
    // before the tile's own output atomics (vmem_wait_all), here for the
    // first tile: a wait at their use would also cover the atomics issued
    // after them.
    vmem_wait_all();

    for (int tile = 0; tile < nr; tile += 16, act2 += BLK, act3 += BLK) {
      const int par = (tile >> 4) & 1;
      const int slot = tile + c;
      const bool valid = slot < nr;
      // (registers whose features are all past L2 / L3 are neither loaded nor used)
      constexpr bool T2V = vtail<S::L2>(), T3V = vtail<S::L3>();
      constexpr int NT2M = S::NT2 - (T2V ? 1 : 0), U3 = S::NU3 - (T3V ? 1 : 0);
      double th2[S::NT2][4], th3[S::NU3][4];
#pragma unroll
      for (int t = 0; t < S::NT2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) th2[t][r] = 16 * t + 4 * r < S::L2 ? act2[(4 * t + r) * 64] : 0.0;
#pragma unroll
      for (int u = 0; u < S::NU3; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) th3[u][r] = 16 * u + 4 * r < S::L3 ? act3[256 * u + 64 * r] : 0.0;
      double d0 = 0.0, d1 = 0.0, d2 = 0.0;
      double Rn[4] = {0.0, 0.0, 0.0, 0.0};
      if (valid) {
        d0 = nx0 - xi;
        d1 = nx1 - yi;
        d2 = nx2 - zi;
        env_value(d0, d1, d2, a.rcut_smth, a.rcut, a.inv_sw, avg, sd, Rn);
      }
      if (slot + 16 < nr) {
        nx0 = a.ext[3 * (long)jn];
        nx1 = a.ext[3 * (long)jn + 1];
        nx2 = a.ext[3 * (long)jn + 2];
        if (g == 0) jbuf[16 * (par ^ 1) + c] = jn;
      }
      jn = row[min(slot + 32, slast)];
      const double s = Rn[0];

      // layer 1 (recomputed, elementwise) and its tangent; padded features
      // have zero weights and bias (tanh 0, tangent 0)
      double x1[S::NQ2], x1t[S::NQ2];
      {
        double z[S::NQ2];
#pragma unroll
        for (int q = 0; q < S::NQ2; ++q) {
          const int f = 4 * q + g;
          z[q] = s * P[S::OFF_W1 + f] + P[S::OFF_B1 + f];
        }
        tanh_n<S::NQ2>(z, x1, Tab);
#pragma unroll
        for (int q = 0; q < S::NQ2; ++q) x1t[q] = (1.0 - x1[q] * x1[q]) * P[S::OFF_W1 + 4 * q + g];
      }
      if constexpr (S::RES2 != 0 && !S::X1_ALIGNED) {
#pragma unroll
        for (int q = 0; q < S::NQ2; ++q) X1s[c * X1LD + 4 * q + g] = x1[q];
        wave_lds_sync();
      }
      // layer 2: tangent product only; tanh of the primal comes from the forward.
      // The weight fragments are read from LDS one k-step ahead of their
      // MFMAs, held there by scheduling fences (compiled freely, each pair of
      // MFMAs waited for its own reads).
      d4 acc2t[S::NT2];
#pragma unroll
      for (int t = 0; t < S::NT2; ++t) acc2t[t] = d4{0.0, 0.0, 0.0, 0.0};
      {
        double w2b[2][NT2M > 0 ? NT2M : 1];
        const double* W2 = P + S::OFF_W2 + g * S::L2P + c;
#pragma unroll
        for (int t = 0; t < NT2M; ++t) w2b[0][t] = W2[16 * t];
#pragma unroll
        for (int q = 0; q < S::NQ2; ++q) {
          if (q + 1 < S::NQ2) {
#pragma unroll
            for (int t = 0; t < NT2M; ++t) w2b[(q + 1) & 1][t] = W2[4 * (q + 1) * S::L2P + 16 * t];
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int t = 0; t < NT2M; ++t) acc2t[t] = mfma_f64(w2b[q & 1][t], x1t[q], acc2t[t]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if constexpr (T2V) {
        // tangent of the tail features 16 NT2M + j (lane group g: j = g, register 0)
        constexpr int TL = S::L2 % 16;
        double pj[TL];
#pragma unroll
        for (int j = 0; j < TL; ++j) pj[j] = 0.0;
#pragma unroll
        for (int q = 0; q < S::NQ2; ++q) {
          const double* wr = P + S::OFF_W2 + (4 * q + g) * S::L2P + 16 * NT2M;
#pragma unroll
          for (int j = 0; j < TL; ++j) pj[j] = fma(x1t[q], wr[j], pj[j]);
        }
#pragma unroll
        for (int j = 0; j < TL; ++j) pj[j] = add_xor32(add_xor16(pj[j]));
        acc2t[NT2M][0] = pick(pj, g);
      }
      double x2[S::NT2][4], x2t[S::NT2][4];
#pragma unroll
      for (int t = 0; t < S::NT2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int f = 16 * t + 4 * r + g;
          const double th = th2[t][r];
          double res = 0.0, rest = 0.0;
          if constexpr (S::RES2 != 0) {
            if constexpr (S::X1_ALIGNED) {
              const int q1 = (S::RES2 == 2 ? 4 * (t % (S::L1 / 16)) : 4 * t) + r;
              res = x1[q1];
              rest = x1t[q1];
            } else if (16 * t + 4 * r + 3 < S::L1) {
              // feature f < L1 in every lane group: the lane's own registers
              const int q1 = min(4 * t + r, S::NQ2 - 1);
              res = x1[q1];
              rest = x1t[q1];
            } else {
              const int f1 = (S::RES2 == 2) ? f % S::L1 : f;
              if (f1 < S::L1) {
                const double y = X1s[c * X1LD + f1];
                res = y;
                rest = (1.0 - y * y) * P[S::OFF_W1 + f1];
              }
            }
          }
          const bool live = f < S::L2;
          x2[t][r] = live ? res + th : 0.0;
          x2t[t][r] = live ? rest + (1.0 - th * th) * acc2t[t][r] : 0.0;
        }
      }
      // u = dT.G, v = dT.G': residual part through the folded dT against X2
      double up[4] = {0.0, 0.0, 0.0, 0.0}, vp[4] = {0.0, 0.0, 0.0, 0.0};
      if constexpr (S::RES3 != 0) {
#pragma unroll
        for (int t = 0; t < S::NT2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int f = 16 * t + 4 * r + g;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              const double wv = dTf[m * S::L2P + f];
              up[m] += wv * x2[t][r];
              vp[m] += wv * x2t[t][r];
            }
          }
      }
      // layer 3 tangent, transposed; tanh part of G from the forward.
      // The weight fragments stream one k-step ahead of their MFMAs across
      // the output tile groups too (the next group's first fragment is read
      // during this group's last product), held there by scheduling fences.
      const double* W3 = P + S::OFF_W3 + g * S::L3P + c;
      double w3b[2][kU3B];
#pragma unroll
      for (int uu = 0; uu < kU3B; ++uu) w3b[0][uu] = uu < U3 ? W3[16 * uu] : 0.0;
#pragma unroll
      for (int u0 = 0; u0 < U3; u0 += kU3B) {
        d4 acc3t[kU3B];
        double dtv[kU3B][4][4];
#pragma unroll
        for (int uu = 0; uu < kU3B; ++uu) acc3t[uu] = d4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int q = 0; q < S::NQ3; ++q) {
          const int st = (u0 / kU3B) * S::NQ3 + q;  // fragment step (compile time)
          if (q + 1 < S::NQ3) {
#pragma unroll
            for (int uu = 0; uu < kU3B; ++uu)
              w3b[(st + 1) & 1][uu] =
                  u0 + uu < U3 ? W3[4 * (q + 1) * S::L3P + 16 * (u0 + uu)] : 0.0;
          } else if (u0 + kU3B < U3) {
#pragma unroll
            for (int uu = 0; uu < kU3B; ++uu)
              w3b[(st + 1) & 1][uu] = u0 + kU3B + uu < U3 ? W3[16 * (u0 + kU3B + uu)] : 0.0;
          }
          if (q + 1 == S::NQ3) {
            // the group's dT values, read during its last product
#pragma unroll
            for (int uu = 0; uu < kU3B; ++uu)
#pragma unroll
              for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int m = 0; m < 4; ++m)
                  dtv[uu][r][m] = u0 + uu < U3 ? dTs[m * S::L3P + 16 * (u0 + uu) + 4 * r + g] : 0.0;
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int uu = 0; uu < kU3B; ++uu)
            if (u0 + uu < U3) acc3t[uu] = mfma_f64(w3b[st & 1][uu], x2t[q / 4][q % 4], acc3t[uu]);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int uu = 0; uu < kU3B; ++uu) {
          const int u = u0 + uu;
          if (u < U3) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (16 * u + 4 * r >= S::L3) continue;
              const double th = th3[u][r];
              const double tt = (1.0 - th * th) * acc3t[uu][r];
#pragma unroll
              for (int m = 0; m < 4; ++m) {
                const double wv = dtv[uu][r][m];
                up[m] += wv * th;
                vp[m] += wv * tt;
              }
            }
          }
        }
      }
      if constexpr (T3V) {
        // tangent of the tail features 16 U3 + j (lane group g: j = g, register 0)
        constexpr int TL = S::L3 % 16;
        double pj[TL];
#pragma unroll
        for (int j = 0; j < TL; ++j) pj[j] = 0.0;
#pragma unroll
        for (int t = 0; t < S::NT2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (16 * t + 4 * r >= 4 * S::NQ3) continue;  // past W3's rows (x2t is 0 there)
            const double* wr = P + S::OFF_W3 + (16 * t + 4 * r + g) * S::L3P + 16 * U3;
#pragma unroll
            for (int j = 0; j < TL; ++j) pj[j] = fma(x2t[t][r], wr[j], pj[j]);
          }
#pragma unroll
        for (int j = 0; j < TL; ++j) pj[j] = add_xor32(add_xor16(pj[j]));
        const int f = 16 * U3 + g;
        const double th = th3[U3][0];
        const double tt = (1.0 - th * th) * pick(pj, g);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const double wv = dTs[m * S::L3P + f];
          up[m] += wv * th;
          vp[m] += wv * tt;
        }
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        up[m] = add_xor32(add_xor16(up[m]));
        vp[m] = add_xor32(add_xor16(vp[m]));
      }
      // the slot's outputs: lane group 0 alone, or all four groups when atom
      // virials are asked for (edge_out shares the atomics out); the next
      // tile's coordinates and index have landed by now
      vmem_wait_all();
      if (valid && (AV || g == 0)) {
        double nd[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) nd[m] = up[m] * a.inv_nnei;
        nd[0] += (Rn[0] * vp[0] + Rn[1] * vp[1] + Rn[2] * vp[2] + Rn[3] * vp[3]) * a.inv_nnei;
        double gv[3];
        env_grad(d0, d1, d2, a.rcut_smth, a.rcut, a.inv_sw, sd, nd, gv);
        const double dv[3] = {d0, d1, d2};
        edge_out<AV>(a, ebase + slot, jbuf[16 * par + c], dv, gv, own_w + 12 * c, g);
      }
    }
    own_flush(a, i, tj, nr, ebase, own_w, lane);
  }
}

// T = (sum over sections of Tsec + padded-slot constant) / nnei, written in
// bucket order as a column-major array Tt [a][pos][4] (element (pos, a, m) at
// Tt[a * 4 nloc + 4 pos + m]): the first fitting GEMM forms D = T^T T[:, :16]
// from it one column a at a time with contiguous reads, and dE/dT reads it
// through L2. When requested, D = T^T T[:, :axis] [pos][L3*axis] as well. E is
// the element type (double, or float in mixed mode); the sums are formed in
// fp64 and rounded once. A block handles kDescAtoms consecutive positions so
// that every layout is written in contiguous runs.
constexpr int kDescAtoms = 8;

// Sum of the sections of items q and q + blockDim.x (item = atom k of the
// block and 4 consecutive elements e = 4g..4g+3 of its [4][L3] row) into the
// LDS copy. Every section value and padded-slot constant of both items is
// loaded before any is summed, so a thread has 4 NT vector loads in flight.
template <class E, int NT>
__device__ __forceinline__ void desc_sum(const DescArgs& a, double* Ts, int pos0, int na, int q) {
  const E* Tsec = static_cast<const E*>(a.Tsec);
  const int L3 = a.L3, per = 4 * L3, LR = L3 + 1, G = per / 4;
  constexpr int R = 2;
  Vec4<E> ts[R][NT];
  Vec4<double> tp[R][NT];
  int nrl[R][NT];
  int kk[R], e0[R];
  bool ok[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int qq = q + r * (int)blockDim.x;
    ok[r] = qq < na * G;
    kk[r] = ok[r] ? qq / G : 0;
    e0[r] = 4 * (qq - kk[r] * G);
    if (ok[r]) {
      const int i = a.items[pos0 + kk[r]];
      const int ti = a.ext_type[i];
#pragma unroll
      for (int tj = 0; tj < NT; ++tj) {
        const long sec = (long)i * NT + tj;
        ts[r][tj] = *reinterpret_cast<const Vec4<E>*>(Tsec + sec * per + e0[r]);
        tp[r][tj] = *reinterpret_cast<const Vec4<double>*>(a.tpad + (long)(ti * NT + tj) * per + e0[r]);
        nrl[r][tj] = a.nreal[sec];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (!ok[r]) continue;
    double v[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int tj = 0; tj < NT; ++tj) {
      const double np = (double)(a.sel[tj] - nrl[r][tj]);
      v[0] += (double)ts[r][tj].x + np * tp[r][tj].x;
      v[1] += (double)ts[r][tj].y + np * tp[r][tj].y;
      v[2] += (double)ts[r][tj].z + np * tp[r][tj].z;
      v[3] += (double)ts[r][tj].w + np * tp[r][tj].w;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int m = (e0[r] + c) / L3, col = e0[r] + c - m * L3;
      Ts[(kk[r] * 4 + m) * LR + col] = (double)(E)(v[c] * a.inv_nnei);
    }
  }
}

template <class E, int NT>
__global__ __launch_bounds__(256) void k_descriptor(DescArgs a) {
  // LDS copy [kDescAtoms][4][L3 + 1]: the padding keeps the column-major
  // pass (consecutive threads on consecutive (atom, m) rows) off one bank
  extern __shared__ double Ts[];
  const int L3 = a.L3, LR = L3 + 1;
  const int pos0 = blockIdx.x * kDescAtoms;
  const int na = min(kDescAtoms, a.nloc - pos0);
  if (a.from_tt) {
    // thread = (column, one of two atoms of a pass); L3 <= 128
    const int col = threadIdx.x & 127;
    for (int k = threadIdx.x >> 7; k < na; k += 2) {
      if (col >= L3) continue;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        Ts[(k * 4 + m) * LR + col] =
            (double)static_cast<const E*>(a.Tt)[((long)col * a.nloc + pos0 + k) * 4 + m];
    }
  } else {
    for (int q = threadIdx.x; q < na * L3; q += 2 * blockDim.x) desc_sum<E, NT>(a, Ts, pos0, na, q);
  }
  __syncthreads();
  if (!a.from_tt) {
    E* Tt = static_cast<E*>(a.Tt);
    for (int q = threadIdx.x; q < L3 * kDescAtoms * 4; q += blockDim.x) {
      const int km = q % (4 * kDescAtoms), c2 = q / (4 * kDescAtoms);  // km = 4k + m
      if ((km >> 2) < na) Tt[((long)c2 * a.nloc + pos0) * 4 + km] = (E)Ts[km * LR + c2];
    }
  }
  if (!a.D) return;
  const int nd = L3 * a.axis;
  for (int q = threadIdx.x; q < na * nd; q += blockDim.x) {
    const int k = q / nd, e = q % nd;
    const int ai = e / a.axis, bi = e % a.axis;
    const double* T = Ts + k * 4 * LR;
    static_cast<E*>(a.D)[(long)pos0 * nd + q] =
        (E)(T[ai] * T[bi] + T[LR + ai] * T[LR + bi] + T[2 * LR + ai] * T[2 * LR + bi] +
            T[3 * LR + ai] * T[3 * LR + bi]);
  }
}

// ---------------------------------------------------------------------------
using ShapeWater = EmbShape<25, 50, 100>;
using ShapeMetal = EmbShape<32, 64, 128>;
constexpr int kFwdWaves = 8;
constexpr int kBwdWaves = 8;

bool emb_supported(int L1, int L2, int L3) {
  return (L1 == 25 && L2 == 50 && L3 == 100) || (L1 == 32 && L2 == 64 && L3 == 128);
}

int embed_waves_fwd(const EmbLayout& e, bool f32) { return f32 ? embed_waves_fwd32(e) : kFwdWaves; }
int embed_waves_bwd(const EmbLayout& e, bool f32) { return f32 ? embed_waves_bwd32(e) : kBwdWaves; }

template <class S>
static void fwd_impl(hipStream_t st, const EmbArgs& a, int nblocks) {
  const size_t bytes = sizeof(double) * fwd_lds_doubles<S>(kFwdWaves);
  auto kern = k_embed_fwd<S, kFwdWaves>;
  DPAMD_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)bytes));
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(kFwdWaves * 64), bytes, st, a);
  DPAMD_LAUNCH_CHECK();
}

template <class S>
static void bwd_impl(hipStream_t st, const EmbArgs& a, int nblocks) {
  const size_t bytes = sizeof(double) * bwd_lds_doubles<S>(kBwdWaves);
  auto kern = a.vacc ? k_embed_bwd<S, kBwdWaves, true> : k_embed_bwd<S, kBwdWaves, false>;
  DPAMD_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)bytes));
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(kBwdWaves * 64), bytes, st, a);
  DPAMD_LAUNCH_CHECK();
}

void launch_embed_fwd(hipStream_t st, const EmbLayout& e, const EmbArgs& a, int nblocks,
                      bool f32) {
  if (nblocks <= 0) return;
  if (f32) launch_embed_fwd32(st, e, a, nblocks);
  else if (e.L1 == 25) fwd_impl<ShapeWater>(st, a, nblocks);
  else fwd_impl<ShapeMetal>(st, a, nblocks);
}

void launch_embed_bwd(hipStream_t st, const EmbLayout& e, const EmbArgs& a, int nblocks,
                      bool f32) {
  if (nblocks <= 0) return;
  if (f32) launch_embed_bwd32(st, e, a, nblocks);
  else if (e.L1 == 25) bwd_impl<ShapeWater>(st, a, nblocks);
  else bwd_impl<ShapeMetal>(st, a, nblocks);
}

template <int NT>
static void desc_dispatch(hipStream_t st, const DescArgs& a, bool f32, dim3 grid, size_t lds) {
  if constexpr (NT < kMaxTypes) {
    if (a.ntypes != NT) return desc_dispatch<NT + 1>(st, a, f32, grid, lds);
  }
  if (f32) hipLaunchKernelGGL((k_descriptor<float, NT>), grid, dim3(256), lds, st, a);
  else hipLaunchKernelGGL((k_descriptor<double, NT>), grid, dim3(256), lds, st, a);
}

void launch_descriptor(hipStream_t st, const DescArgs& a, bool f32) {
  if (a.nloc <= 0) return;
  if (a.L3 > 128) throw HipError{hipErrorInvalidValue, "descriptor kernel needs L3 <= 128"};
  const dim3 grid((a.nloc + kDescAtoms - 1) / kDescAtoms);
  const size_t lds = sizeof(double) * kDescAtoms * 4 * (a.L3 + 1);
  desc_dispatch<1>(st, a, f32, grid, lds);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace dpamd
