// Fitting net (D -> F0 -> F1 -> F2 -> 1, tanh, y = x + idt*tanh(xW+b) on
// square layers) forward + input gradient on gfx950 MFMA, per centre type
// over the atoms of that type (bucket order), and the descriptor backward
// dE/dD -> dE/dT. Element type T: double (FP64 MFMA) in fp64 mode, float
// (FP32 MFMA) in mixed mode; the per-atom energy is accumulated in fp64 in
// both.
//
// Each layer is one GEMM (rows = atoms) with its elementwise work fused into
// the epilogue: bias + tanh + residual in the forward, (dH_in + acc) * idt *
// (1 - t^2) in the backward. Reference semantics: h = act(xW+b) (+ residual),
// e = h.w_head + b_head + bias_atom_e[type]
// (deepmd-op/overlays/op/pt/graph_fitting.cu:1-25, :614-719); the reference's
// fused tile analog is deepmd-op/overlays/op/pt/tiled_fitting.cuh:4-60.

#include <algorithm>

#include "bf16x3.h"
#include "fastmath.h"
#include "kernels.h"

namespace dpamd {

template <class T>
struct GemmArgs {
  int M, N, K;
  const T* A;
  int lda;
  const T* B;
  int ldb;
  int epi;  // 0 plain store, 1 forward layer, 2 backward layer, 3 last layer + head
  const T* bias;
  const T* idt;
  T* C;
  int ldc;
  T* T_out;       // forward: tanh part
  const T* dHin;  // backward: incoming dH (row stride ld_dhin; 0 = broadcast)
  int ld_dhin;
  T* dH_out;      // backward: dH of this layer
  const T* Tk;    // backward: tanh part of this layer (ld = ldc)
  // A from T (AT kernels): element (row, a, m) of T at Tt[a * ldt + 4 row + m],
  // A[row][16a + b] = sum_m T[m][a] T[m][b]
  const T* Tt;
  long ldt;
  // split K: blockIdx.z takes chunks [z per, (z+1) per) of the K loop and
  // stores its partial product to ws + z M ldc (plain store); a separate
  // epilogue kernel sums the slices in order
  int split;
  T* ws;
  // fp32 only: B pre-split into bf16 fragments (pack_gemm_bf16 layout), which
  // selects the bf16 three-piece kernel k_gemm3; null for the fp32 / fp64 MFMA
  const void* Bf;
  // epi 3 (the last layer with the energy head fused): the head's weights Wo
  // [N] and the per-row partial energies epart[M][N / BN] (one per column
  // block, fp64), summed in column-block order by k_head_sum
  const T* Wo;
  double* epart;
};

// Block tile output: the split-K slice store, or the layer epilogue (plain,
// forward: bias + tanh + residual, backward: (dH_in + acc) idt (1 - t^2),
// last layer + head: see store_last).
// acc[n] register r of wave w holds C[row0 + 16w + Frag::row(g, r)][col0 + 16n + c];
// ro[r] is that row and ok[r] whether it exists (row < M).
// The global inputs of an epilogue are loaded two column tiles ahead of their
// use, so several loads are in flight at once without holding every tile's
// inputs in registers; each tile's work is kept in its own scheduling region
// (hoisting every tile's loads to the top raised the register count past
// four waves per SIMD). The per-element row check is compiled only for the
// last row block (FULL = false in gemm_store_rows).
template <class T, int NT>
using Acc = typename Frag<T>::V[NT];

// forward layer: C = x + idt t (or t without a timestep), T_out = t
template <class T, int NT>
__device__ __forceinline__ void store_forward(const GemmArgs<T>& a, const Acc<T, NT>& acc,
                                              const bool (&ok)[4], const long (&ro)[4], int col0,
                                              int c) {
  T res[NT][4];
  auto load = [&](int n) {
    if (a.idt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) res[n][r] = ok[r] ? a.A[ro[r] * a.lda + col0 + 16 * n + c] : T(0);
    }
  };
  load(0);
  if (NT > 1) load(1);
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    __builtin_amdgcn_sched_barrier(0);
    if (n + 2 < NT) load(n + 2);
    const int col = col0 + 16 * n + c;
    // the four tanh of this column at once (fp64: shared reciprocal; rows
    // past M hold zeros and are not stored)
    T z[4], th[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) z[r] = acc[n][r] + a.bias[col];
    tanh_act4(z, th);
    const T id = a.idt ? a.idt[col] : T(1);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (!ok[r]) continue;
      const long o = ro[r] * a.ldc + col;
      if (a.T_out) a.T_out[o] = th[r];
      a.C[o] = a.idt ? res[n][r] + id * th[r] : th[r];
    }
  }
}

// The last layer h = x + idt t (t = tanh(z)) with the energy head fused: h is
// consumed here and never stored. C receives the backward's seed
// dZ = Wo idt (1 - t^2) (the head's dE/dh is Wo), and each row's partial
// energy sum_col h Wo over this block's columns (fp64, summed over the 16
// column lanes of the row by a fixed xor tree) goes to epart. (The residual
// is read where it is used: a prefetched copy here kept twenty values live.)
template <class T, int NT>
__device__ __forceinline__ void store_last(const GemmArgs<T>& a, const Acc<T, NT>& acc,
                                           const bool (&ok)[4], const long (&ro)[4], int col0,
                                           int c) {
  double es[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    __builtin_amdgcn_sched_barrier(0);
    const int col = col0 + 16 * n + c;
    T z[4], th[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) z[r] = acc[n][r] + a.bias[col];
    tanh_act4(z, th);
    const T id = a.idt ? a.idt[col] : T(1), wo = a.Wo[col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (!ok[r]) continue;
      const T t = th[r];
      const T h = a.idt ? a.A[ro[r] * a.lda + col] + id * t : t;
      es[r] += (double)h * (double)wo;
      a.C[ro[r] * a.ldc + col] = wo * id * (T(1) - t * t);
    }
  }
  const int ncb = a.N / (16 * NT);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) es[r] += shfl_xor_d(es[r], off);
    if (c == 0 && ok[r]) a.epart[ro[r] * ncb + col0 / (16 * NT)] = es[r];
  }
}

// backward layer: dh = acc + dH_in, C = dh idt (1 - tk^2), dH_out = dh
template <class T, int NT>
__device__ __forceinline__ void store_backward(const GemmArgs<T>& a, const Acc<T, NT>& acc,
                                               const bool (&ok)[4], const long (&ro)[4],
                                               int col0, int c) {
  T tk[NT][4], dh[NT][4];
  auto load = [&](int n) {
#pragma unroll
    for (int r = 0; r < 4; ++r) tk[n][r] = ok[r] ? a.Tk[ro[r] * a.ldc + col0 + 16 * n + c] : T(0);
    if (a.dHin && a.ld_dhin > 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        dh[n][r] = ok[r] ? a.dHin[ro[r] * a.ld_dhin + col0 + 16 * n + c] : T(0);
    } else {
      const T d = a.dHin ? a.dHin[col0 + 16 * n + c] : T(0);
#pragma unroll
      for (int r = 0; r < 4; ++r) dh[n][r] = d;
    }
  };
  load(0);
  if (NT > 1) load(1);
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    __builtin_amdgcn_sched_barrier(0);
    if (n + 2 < NT) load(n + 2);
    const int col = col0 + 16 * n + c;
    const T id = a.idt ? a.idt[col] : T(1);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (!ok[r]) continue;
      const long o = ro[r] * a.ldc + col;
      const T d = acc[n][r] + dh[n][r];
      if (a.dH_out) a.dH_out[o] = d;
      a.C[o] = d * id * (T(1) - tk[n][r] * tk[n][r]);
    }
  }
}

template <class T, int NT, int EPI, bool FULL>
__device__ __forceinline__ void gemm_store_rows(const GemmArgs<T>& a, const Acc<T, NT>& acc,
                                                int row0, int col0, int zs, int w, int g, int c) {
  long ro[4];
  bool ok[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = row0 + 16 * w + Frag<T>::row(g, r);
    ok[r] = FULL || row < a.M;
    ro[r] = row;
  }
  if (a.split > 1 || EPI == 0) {
    T* out = a.split > 1 ? a.ws + (long)zs * a.M * a.ldc : a.C;
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (ok[r]) out[ro[r] * a.ldc + col0 + 16 * n + c] = acc[n][r];
    return;
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (EPI == 1) store_forward<T, NT>(a, acc, ok, ro, col0, c);
  if constexpr (EPI == 2) store_backward<T, NT>(a, acc, ok, ro, col0, c);
  if constexpr (EPI == 3) store_last<T, NT>(a, acc, ok, ro, col0, c);
}

template <class T, int NT, int EPI>
__device__ __forceinline__ void gemm_store(const GemmArgs<T>& a, const typename Frag<T>::V (&acc)[NT],
                                           int row0, int col0, int zs, int w, int g, int c) {
  if (row0 + 64 <= a.M) gemm_store_rows<T, NT, EPI, true>(a, acc, row0, col0, zs, w, g, c);
  else gemm_store_rows<T, NT, EPI, false>(a, acc, row0, col0, zs, w, g, c);
}

// C = epi(A[MxK] B[KxN]); B(k,n) = TRANSB ? B[n*ldb + k] : B[k*ldb + n].
// Block tile 64 x 16*NT: wave w owns rows 16w..16w+15 and all NT column tiles,
// so one A fragment feeds NT MFMAs. K advances 16 at a time through two LDS
// buffers: the next chunk is fetched into registers while the current one is
// multiplied, then stored into the other buffer (one barrier per chunk).
// AT: A is the descriptor D = T^T T[:, :16] of each row, formed while staging:
// K chunk a holds D[row][16a + b] = sum_m T[m][a] T[m][b]; thread (r, part)
// keeps T[m][4 part .. 4 part + 3] of row r in registers and fetches the 4
// values T[0..3][a] per chunk (contiguous in the column-major copy of T, so a
// wave reads 16 rows as one run) instead of 16 values of D.
template <class T, int NT, bool TRANSB, bool AT, int EPI>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs<T> a) {
  constexpr int BM = 64, BK = 16, BN = 16 * NT;
  constexpr int ALD = BK + 1, BLD = BN + 1;
  constexpr int NA = BM * BK / 256, NB = (BK * BN + 255) / 256;
  static_assert(!AT || NA == 4, "AT staging assumes 4 A elements per thread");
  __shared__ T As[2][BM * ALD];
  __shared__ T Bs[2][BK * BLD];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int3 bid = xcd_swizzle();
  const int row0 = bid.y * BM, col0 = bid.x * BN;
  // AT: this thread's row and column quarter, and T[m][4 part + j] of the row
  const int at_r = tid >> 2, at_part = tid & 3;
  const T* at_row = nullptr;  // T[.][0][row] of this thread's row
  T tb[4][4];
  if constexpr (AT) {
    if (row0 + at_r < a.M) at_row = a.Tt + 4 * (long)(row0 + at_r);
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        tb[m][j] = at_row ? at_row[(4 * at_part + j) * a.ldt + m] : T(0);
  }
  // element offsets of this thread's share of a K chunk, fixed over chunks
  int offA[NA], ldsA[NA], offB[NB], ldsB[NB];
#pragma unroll
  for (int u = 0; u < NA; ++u) {
    const int q = tid + 256 * u, r = q / BK, kk = q % BK, gr = row0 + r;
    offA[u] = gr < a.M ? gr * a.lda + kk : -1;
    ldsA[u] = r * ALD + kk;
  }
#pragma unroll
  for (int u = 0; u < NB; ++u) {
    const int q = tid + 256 * u;
    if (q < BK * BN) {
      if (!TRANSB) {
        const int kk = q / BN, n = q % BN;
        offB[u] = kk * a.ldb + col0 + n;
        ldsB[u] = kk * BLD + n;
      } else {
        const int n = q / BK, kk = q % BK;
        offB[u] = (col0 + n) * a.ldb + kk;
        ldsB[u] = kk * BLD + n;
      }
    } else {
      offB[u] = -1;
      ldsB[u] = 0;
    }
  }
  T ra[NA], rb[NB];
  auto fetch = [&](int k0) {
    const T* Bk = TRANSB ? a.B + k0 : a.B + (long)k0 * a.ldb;
    if constexpr (AT) {
      // ra[m] = T[m][a] of this thread's row, a = k0 / 16
#pragma unroll
      for (int m = 0; m < 4; ++m) ra[m] = at_row ? at_row[(k0 >> 4) * a.ldt + m] : T(0);
    } else {
      const T* Ak = a.A + k0;
#pragma unroll
      for (int u = 0; u < NA; ++u) ra[u] = offA[u] >= 0 ? Ak[offA[u]] : T(0);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) rb[u] = offB[u] >= 0 ? Bk[offB[u]] : T(0);
  };
  auto stash = [&](int buf) {
    if constexpr (AT) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        As[buf][at_r * ALD + 4 * at_part + j] =
            ra[0] * tb[0][j] + ra[1] * tb[1][j] + ra[2] * tb[2][j] + ra[3] * tb[3][j];
    } else {
#pragma unroll
      for (int u = 0; u < NA; ++u) As[buf][ldsA[u]] = ra[u];
    }
#pragma unroll
    for (int u = 0; u < NB; ++u)
      if (offB[u] >= 0) Bs[buf][ldsB[u]] = rb[u];
  };
  typename Frag<T>::V acc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n] = typename Frag<T>::V{0, 0, 0, 0};
  int kc0 = 0, nk = a.K / BK;
  if (a.split > 1) {
    const int per = (nk + a.split - 1) / a.split;
    kc0 = bid.z * per;
    nk = min(nk, kc0 + per);
  }
  // (a slice past the end of K keeps zeros: it is still stored, and summed)
  if (kc0 < nk) {
    fetch(kc0 * BK);
    stash(kc0 & 1);
  }
  __syncthreads();
  for (int kc = kc0; kc < nk; ++kc) {
    const int buf = kc & 1;
    if (kc + 1 < nk) fetch((kc + 1) * BK);
    const T* Ab = As[buf] + (16 * w + c) * ALD;
    const T* Bb = Bs[buf];
#pragma unroll
    for (int q = 0; q < BK / 4; ++q) {
      const T av = Ab[4 * q + g];
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[n] = mfma(av, Bb[(4 * q + g) * BLD + 16 * n + c], acc[n]);
    }
    if (kc + 1 < nk) stash(buf ^ 1);
    __syncthreads();
  }
  gemm_store<T, NT, EPI>(a, acc, row0, col0, bid.z, w, g, c);
}

// fp32 GEMM on the bf16 matrix cores at fp32 accuracy (mixed precision):
// C = epi(A[MxK] B[KxN]) with B pre-split on the host into fragments
// a.Bf [ceil(K/32)][N/16][3][64 lanes] (8 bf16 each: lane 16g + c of (chunk
// h, column tile n) holds the pieces of B(32h + 8g + e, 16n + c), e = 0..7,
// zero past K). Block tile 64 x 16 NT, wave w rows 16w..16w+15 as in k_gemm;
// K advances 32 at a time: the A chunk (fp32) and the block's B fragments
// (NT tiles) go through two LDS buffers, each wave splits its A fragment
// (row 16w + c, k 8g..8g+7) once per chunk and runs six bf16 MFMAs per column
// tile (mfma3). On gfx950 the fp32 16x16x4 MFMA is barely faster than the
// VALU; the bf16 form with the six-product split does about twice its work
// per unit time. AT: A is D = T^T T[:, :16] formed while staging; chunk kc
// holds D columns 32kc.. 32kc + 31 (a = 2kc, 2kc + 1), thread (row, part)
// stages columns 8 part .. 8 part + 7 and keeps T[m][8 (part % 2) + e].
template <int NT, bool AT, int EPI>
__global__ __launch_bounds__(256) void k_gemm3(GemmArgs<float> a) {
  constexpr int BM = 64, BK = 32, BN = 16 * NT, ALD = BK + 4;
  __shared__ __align__(16) float As[2][BM * ALD];
  __shared__ __align__(16) bf8 Bs[2][NT * 3 * 64];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int3 bid = xcd_swizzle();
  const int row0 = bid.y * BM, col0 = bid.x * BN;
  const int ntile = a.N / 16, tile0 = col0 / 16;
  const bf8* Bf = static_cast<const bf8*>(a.Bf);
  // staging share: row sr, k columns sk .. sk + 7 of the chunk
  const int sr = tid >> 2, part = tid & 3, sk = 8 * part;
  const int grow = row0 + sr;
  const float* arow = grow < a.M ? (AT ? a.Tt + 4 * (long)grow : a.A + (long)grow * a.lda) : nullptr;
  float tb[4][8];
  if constexpr (AT) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        tb[m][e] = arow ? arow[(8 * (part & 1) + e) * a.ldt + m] : 0.0f;
  }
  float ra[8];
  bf8 rb[(NT * 3 * 64 + 255) / 256];
  auto fetch = [&](int kc) {
    if constexpr (AT) {
      // ra[m] = T[m][a] of this row, a = 2 kc + part / 2
      const int ac = 2 * kc + (part >> 1);
#pragma unroll
      for (int m = 0; m < 4; ++m) ra[m] = arow ? arow[(long)ac * a.ldt + m] : 0.0f;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = 32 * kc + sk + e;
        ra[e] = (arow && k < a.K) ? arow[k] : 0.0f;
      }
    }
    const bf8* src = Bf + ((long)kc * ntile + tile0) * 192;
#pragma unroll
    for (int u = 0; u < (NT * 192 + 255) / 256; ++u) {
      const int q = tid + 256 * u;
      if (q < NT * 192) rb[u] = src[q];
    }
  };
  auto stash = [&](int buf) {
    float* dst = As[buf] + sr * ALD + sk;
    if constexpr (AT) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        dst[e] = ra[0] * tb[0][e] + ra[1] * tb[1][e] + ra[2] * tb[2][e] + ra[3] * tb[3][e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[e] = ra[e];
    }
#pragma unroll
    for (int u = 0; u < (NT * 192 + 255) / 256; ++u) {
      const int q = tid + 256 * u;
      if (q < NT * 192) Bs[buf][q] = rb[u];
    }
  };
  f4 acc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  int kc0 = 0, nk = (a.K + BK - 1) / BK;
  if (a.split > 1) {
    const int per = (nk + a.split - 1) / a.split;
    kc0 = bid.z * per;
    nk = min(nk, kc0 + per);
  }
  if (kc0 < nk) {
    fetch(kc0);
    stash(kc0 & 1);
  }
  __syncthreads();
  for (int kc = kc0; kc < nk; ++kc) {
    const int buf = kc & 1;
    if (kc + 1 < nk) fetch(kc + 1);
    const Split3 xa = split3(As[buf] + (16 * w + c) * ALD + 8 * g);
    // each column tile's B pieces are read from LDS one tile ahead of its
    // products (scheduling barriers keep the compiler from sinking the reads
    // to their use)
    auto bp = [&](int n) {
      const bf8* b = Bs[buf] + n * 192 + lane;
      return Split3{b[0], b[64], b[128]};
    };
    Split3 bc = bp(0);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      Split3 bn = bc;
      if (n + 1 < NT) bn = bp(n + 1);
      __builtin_amdgcn_sched_barrier(0);
      acc[n] = mfma3(xa, bc, acc[n]);
      __builtin_amdgcn_sched_barrier(0);
      bc = bn;
    }
    if (kc + 1 < nk) stash(buf ^ 1);
    __syncthreads();
  }
  gemm_store<float, NT, EPI>(a, acc, row0, col0, bid.z, w, g, c);
}

// Split-K forward epilogue of a layer without residual: C = tanh(sum over
// the split slices in order + bias), four consecutive columns per thread.
template <class T>
__global__ __launch_bounds__(256) void k_splitk_tanh(int M, int N, int split,
                                                    const T* __restrict__ ws,
                                                    const T* __restrict__ bias,
                                                    T* __restrict__ C) {
  const long q = (long)blockIdx.x * blockDim.x + threadIdx.x;  // 4-column group
  const int g4 = N / 4;
  if (q >= (long)M * g4) return;
  const long row = q / g4;
  const int col = 4 * (int)(q - row * g4);
  const long o = row * N + col;
  T z[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) z[j] = ws[o + j];
  for (int k = 1; k < split; ++k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) z[j] += ws[(long)k * M * N + o + j];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) z[j] += bias[col + j];
  T th[4];
  if constexpr (sizeof(T) == 8) {
    tanh_fast4(z, th);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) th[j] = tanh_act(z[j]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) C[o + j] = th[j];
}

// K slices for the first fitting layer: split only when the row blocks alone
// leave the device short of work (fewer than four blocks per compute unit),
// and keep at least 8 K chunks of 16 per slice (12,288-atom water: fitting
// 0.717 -> 0.694 ms against a two-block target; an eight-block target with
// 4-chunk slices was slower, 0.72 ms; the large types never split).
int fit_splits(int rows, int N, int K, int ncu) {
  const int cols = N % 128 == 0 ? N / 128 : N % 80 == 0 ? N / 80 : N % 64 == 0 ? N / 64 : N / 16;
  const long blocks = (long)cols * ((rows + 63) / 64);
  const int nk = K / 16;
  int split = 1;
  while (blocks * split < 4L * ncu && nk / (2 * split) >= 8) split *= 2;
  return split;
}

// Energy head, second half: e = sum of the row's column-block partials of
// h2.Wo (in column-block order) + bo + bias; the partials and the backward's
// seed come from the last layer's epilogue (gemm_store, epi 3).
__global__ __launch_bounds__(256) void k_head_sum(int rows, int ncb, const double* __restrict__ epart,
                                                  double bo, double bias, double* __restrict__ e) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  double acc = epart[(long)row * ncb];
  for (int k = 1; k < ncb; ++k) acc += epart[(long)row * ncb + k];
  e[row] = acc + bo + bias;
}

// dT[m][a] = sum_b dD[a][b] T[m][b] + (a < axis) sum_a' dD[a'][a] T[m][a'].
// One wave per atom, axis == 16, L3 <= 128, L3 % 4 == 0. dD is read as it
// lies, 4 rows per wave instruction: lane (g, c) = (lane / 16, lane % 16)
// holds v = dD[a0 + g][c].
//   First term: the lane's four products v T[m][c] are summed over the 16
//   lanes of its row by a transposing reduction (xor 8 and 4 exchange halves
//   of the lanes' value sets, xor 2 and 1 finish), which leaves lane c with
//   the sum for m = c / 4: five exchanges per row instead of sixteen.
//   Second term: lane c owns column b = c and accumulates v T[m][a] over its
//   rows; the four row groups are folded at the end (xor 16, 32).
// The first-term values of rows a < 16 meet their second term through LDS.
constexpr int kDtWaves = 4;
template <class T>
__global__ __launch_bounds__(kDtWaves * 64) void k_dT(int nb, int L3,
                                                     const int* __restrict__ items,
                                                     const T* __restrict__ Tt,
                                                     const T* __restrict__ dD,
                                                     T* __restrict__ dT) {
  constexpr int AX = 16;
  __shared__ T Ts[kDtWaves][4 * 128];
  __shared__ T F16[kDtWaves][4 * AX];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int pos0 = blockIdx.x * kDtWaves, pos = pos0 + w;
  // T of the block's positions from the column-major copy (element (pos, a,
  // m) at Tt[a * 4 nb + 4 pos + m]): column a of the kDtWaves consecutive
  // positions is one contiguous run of 4 kDtWaves values, read by as many
  // consecutive threads (a wave alone would use a quarter of each line)
  {
    constexpr int RUN = 4 * kDtWaves;
    const int k = threadIdx.x % RUN, pw = k >> 2, m = k & 3;
    if (pos0 + pw < nb) {
      const T* src = Tt + 4 * (long)pos0 + k;
      for (int a = threadIdx.x / RUN; a < L3; a += kDtWaves * 64 / RUN)
        Ts[pw][m * L3 + a] = src[(long)a * 4 * nb];
    }
  }
  __syncthreads();
  if (pos >= nb) return;
  const int i = items[pos];
  const T tb0 = Ts[w][c], tb1 = Ts[w][L3 + c], tb2 = Ts[w][2 * L3 + c], tb3 = Ts[w][3 * L3 + c];
  const bool hi8 = (c & 8) != 0, hi4 = (c & 4) != 0;
  const int mine = c >> 2;  // the m whose first-term sum this lane ends with
  const T* dDp = dD + (long)pos * L3 * AX;
  T* out = dT + (long)i * 4 * L3;
  T s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  for (int a0b = 0; a0b < L3; a0b += 32) {
    T vb[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) vb[u] = a0b + 4 * u < L3 ? dDp[(a0b + 4 * u) * AX + lane] : T(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int a0 = a0b + 4 * u;
      if (a0 >= L3) break;
      const int a = a0 + g;
      const T v = vb[u];
      s0 += v * Ts[w][a];
      s1 += v * Ts[w][L3 + a];
      s2 += v * Ts[w][2 * L3 + a];
      s3 += v * Ts[w][3 * L3 + a];
      const T p0 = v * tb0, p1 = v * tb1, p2 = v * tb2, p3 = v * tb3;
      // xor 8: keep the pair {m = 2 hi8, 2 hi8 + 1}, send the other
      const T k0 = hi8 ? p2 : p0, k1 = hi8 ? p3 : p1;
      const T q0 = k0 + shfl_xor_d(hi8 ? p0 : p2, 8);
      const T q1 = k1 + shfl_xor_d(hi8 ? p1 : p3, 8);
      // xor 4: keep m = 2 hi8 + hi4
      T r = (hi4 ? q1 : q0) + shfl_xor_d(hi4 ? q0 : q1, 4);
      r += shfl_xor_d(r, 2);
      r += shfl_xor_d(r, 1);
      // lane c (c % 4 == 0) of row group g holds dT1[mine][a]
      if ((c & 3) == 0) {
        if (a >= AX) out[mine * L3 + a] = r;
        else F16[w][mine * AX + a] = r;
      }
    }
  }
  s0 = add_xor32(add_xor16(s0));
  s1 = add_xor32(add_xor16(s1));
  s2 = add_xor32(add_xor16(s2));
  s3 = add_xor32(add_xor16(s3));
  wave_lds_sync();
  if (g == 0) {
    out[c] = F16[w][c] + s0;
    out[L3 + c] = F16[w][AX + c] + s1;
    out[2 * L3 + c] = F16[w][2 * AX + c] + s2;
    out[3 * L3 + c] = F16[w][3 * AX + c] + s3;
  }
}

// The same dT for any axis (a power of two <= 64; fitting shapes other than
// axis 16): one wave per atom, T of its position staged in the wave's LDS
// rows, lane l owning the columns a = l and l + 64. dD[pos] ([L3][axis]
// row-major) is read straight from memory: the first term walks a row
// (consecutive b), the second a column (stride axis) of the atom's block.
template <class T>
__global__ __launch_bounds__(kDtWaves * 64) void k_dT_any(int nb, int L3, int axis,
                                                         const int* __restrict__ items,
                                                         const T* __restrict__ Tt,
                                                         const T* __restrict__ dD,
                                                         T* __restrict__ dT) {
  __shared__ T Ts[kDtWaves][4 * 128];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pos = blockIdx.x * kDtWaves + w;
  if (pos >= nb) return;  // wave-uniform; no block barrier below
  for (int a = lane; a < L3; a += 64)
#pragma unroll
    for (int m = 0; m < 4; ++m) Ts[w][m * L3 + a] = Tt[(long)a * 4 * nb + 4L * pos + m];
  wave_lds_sync();
  const T* Dp = dD + (long)pos * L3 * axis;
  T* out = dT + (long)items[pos] * 4 * L3;
  for (int a = lane; a < L3; a += 64) {
    T acc[4] = {T(0), T(0), T(0), T(0)};
    for (int b = 0; b < axis; ++b) {
      const T d = Dp[(long)a * axis + b];
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m] += d * Ts[w][m * L3 + b];
    }
    if (a < axis)
      for (int a2 = 0; a2 < L3; ++a2) {
        const T d = Dp[(long)a2 * axis + a];
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[m] += d * Ts[w][m * L3 + a2];
      }
#pragma unroll
    for (int m = 0; m < 4; ++m) out[m * L3 + a] = acc[m];
  }
}

// Input gradient of the first fitting layer fused with the descriptor
// backward (fp64): for the rows (atoms of one type) of a block,
//   dD[a][b] = sum_k dZ0[k] W0[16a + b][k]         (FP64 MFMA, in registers)
//   dT[m][a] = sum_b dD[a][b] T[m][b] + (a < 16) sum_a' dD[a'][a] T[m][a']
// so dD is never stored. Wave w owns rows 16w .. 16w + 15 of the block and
// keeps their dZ0 rows in registers as MFMA B operands for the whole K = 4 NQ
// (60 k-steps for F0 = 240); the block walks the column groups a (16 columns
// b each) with W0^T[k][16a .. 16a + 15] staged in LDS (double-buffered, shared
// by all waves). Each MFMA tile is computed transposed, D'[b][row] =
// W0 dZ0^T, so register r of lane (g, c) holds dD[row c][a][b = g + 4r]:
//   first term  lane-local over r (T[row c][m][g + 4r] held in registers),
//               then over the four lane groups (xor 16, 32); lane (g, c)
//               keeps m = g and parks it in an LDS buffer of 16 columns,
//               flushed as 128-byte runs of dT[atom][m][a];
//   second term lane-local: acc2[r][m] += dD[row][a][b] T[row][m][a], with
//               T[row][m][a] of the block's rows staged in LDS per a.
// The column groups run 16 .. L3-1 and then 0 .. 15, so the last buffer holds
// the first term of a < 16 when the second term is complete; the two are
// added and written at the end. T is the column-major copy (element (pos, a,
// m) at Tt[a ldt + 4 pos + m]) with Tt pointing at the type's first row
// (bucket position pos0); dT is in atom order (items[pos0 + row] is the atom
// of a row); dD (inspection only) is written when non-null.
// Reference analog of the fused forward + gradient fitting entry:
// deepmd-op/overlays/op/pt/graph_fitting.cu:728-757.
#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

struct DdtArgs {
  int rows, K, L3;
  const double* dZ;   // [rows][K]
  const double* W0T;  // [K][16 L3]
  const double* Tt;
  long ldt;
  int pos0;
  const int* items;
  double* dT;  // [atoms][4][L3]
  double* dD;  // [rows][16 L3] or null
  // column-group split (blockIdx.y of nsplit; 1: no split): the split's
  // second-term partials go to ws[s][rows][4 m][16 b], the last split's
  // first terms of a < 16 to ws[nsplit][rows][4][16], and k_ddt_combine
  // assembles dT[.][m][b < 16] from them
  int nsplit;
  double* ws;
};

constexpr int kObRow = 66;  // row stride of k_dDdT's first-term buffer (64 + 2)

template <int WAVES, int NQ>
__global__ __launch_bounds__(WAVES * 64) void k_dDdT(DdtArgs p) {
  constexpr int BM = 16 * WAVES, K = 4 * NQ;
  extern __shared__ double lds[];
  double* Bs = lds;                   // [2][K][16]
  double* Ts = Bs + 2 * K * 16;       // [2][BM][4]
  // [WAVES][16 rows][4 m][16 columns], rows padded to kObRow doubles so that
  // the per-group writes (lane (g, c): row c, m = g) fall in distinct banks
  double* Ob = Ts + 2 * BM * 4;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int row0 = blockIdx.x * BM, wrow = row0 + 16 * w + c;  // this lane's row
  const bool rowok = wrow < p.rows;
  const int Dn = 16 * p.L3;
  double* Obw = Ob + w * 16 * kObRow;
  // this block's column groups: split s takes i in [i0, i1), the boundaries
  // 16-aligned within the a >= 16 groups (so every flush stays whole), the
  // last split also the 16 groups a < 16
  const int S = p.nsplit, s = blockIdx.y, R = p.L3 - 16;
  auto bound = [&](int k) { return k >= S ? p.L3 : 16 * ((2 * k * R + 16 * S) / (32 * S)); };
  const int i0 = bound(s), i1 = bound(s + 1);
  // dZ0 row of this lane as MFMA B operands: element k = 4q + g
  double Zb[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) Zb[q] = rowok ? p.dZ[(long)wrow * K + 4 * q + g] : 0.0;
  // T[row][m][b = g + 4r] of this lane's row (first term)
  const long tpos = 4L * wrow;
  // atom of this lane's row (rows of the wave are broadcast from lane c)
  const int my_atom = rowok ? p.items[p.pos0 + wrow] : 0;
  double Tc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m) Tc[r][m] = rowok ? p.Tt[(long)(g + 4 * r) * p.ldt + tpos + m] : 0.0;
  double acc2[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m) acc2[r][m] = 0.0;

  // Staging of column group a through the LDS DMA (global_load_lds, 16 bytes
  // per lane, lane L's granule at base + 16 L; no registers): W0^T rows k,
  // columns 16a .. 16a + 15 (granule q: k = q / 8, columns 2 (q % 8) + 0, 1),
  // and T column a of the block's rows (granule q: row q / 2, m 2 (q % 2) + 0,
  // 1; rows past the type's end read its last row and are not used).
  constexpr int NGB = K * 8, NGT = BM * 2;  // granules per group
  auto issue = [&](int buf, int a) {
    for (int i = w; 64 * i < NGB; i += WAVES) {
      const int q = 64 * i + lane;
      if (q < NGB)
        __builtin_amdgcn_global_load_lds(p.W0T + (long)(q >> 3) * Dn + 16 * a + 2 * (q & 7),
                                         LDS_PTR(Bs + buf * K * 16 + 128 * i), 16, 0, 0);
    }
    for (int i = w; 64 * i < NGT; i += WAVES) {
      const int q = 64 * i + lane;
      const int r = min(row0 + (q >> 1), p.rows - 1);
      __builtin_amdgcn_global_load_lds(p.Tt + (long)a * p.ldt + 4L * r + 2 * (q & 1),
                                       LDS_PTR(Ts + buf * BM * 4 + 128 * i), 16, 0, 0);
    }
  };
  auto col_of = [&](int i) { return i + 16 < p.L3 ? i + 16 : i + 16 - p.L3; };

  if (i0 < i1) issue(0, col_of(i0));
  for (int i = i0; i < i1; ++i) {
    const int a = col_of(i), buf = (i - i0) & 1;
    // group i has landed (each wave waits for its own transfers, then the
    // barrier), and no wave still reads the buffer group i + 1 goes to
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    if (i + 1 < i1) issue(buf ^ 1, col_of(i + 1));
    // D'[b][row] over K: register r of lane (g, c) = dD[row c][a][g + 4r]
    // two independent accumulation chains (the halves of K), operands read
    // from LDS two k-steps ahead
    const double* B = Bs + buf * K * 16 + g * 16 + c;
    constexpr int H = NQ / 2;
    static_assert(NQ % 2 == 0, "K halves");
    d4 acc0 = d4{0.0, 0.0, 0.0, 0.0}, acc1 = d4{0.0, 0.0, 0.0, 0.0};
    double b0[3], b1[3];
    b0[0] = B[0];
    b1[0] = B[64 * H];
    b0[1] = B[64];
    b1[1] = B[64 * (H + 1)];
#pragma unroll
    for (int q = 0; q < H; ++q) {
      if (q + 2 < H) {
        b0[(q + 2) % 3] = B[64 * (q + 2)];
        b1[(q + 2) % 3] = B[64 * (H + q + 2)];
      }
      acc0 = mfma_f64(b0[q % 3], Zb[q], acc0);
      acc1 = mfma_f64(b1[q % 3], Zb[H + q], acc1);
    }
    d4 acc;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = acc0[r] + acc1[r];
    // first term: sum over b = g + 4r (lane-local over r, then the groups)
    double s[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      double v = acc[0] * Tc[0][m];
      v = fma(acc[1], Tc[1][m], v);
      v = fma(acc[2], Tc[2][m], v);
      v = fma(acc[3], Tc[3][m], v);
      v = add_xor32(add_xor16(v));
      s[m] = v;
    }
    Obw[c * kObRow + g * 16 + (a & 15)] = g == 0 ? s[0] : g == 1 ? s[1] : g == 2 ? s[2] : s[3];
    // second term: T[row][m][a]
    const double* tr = Ts + buf * BM * 4 + (16 * w + c) * 4;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const double t = tr[m];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc2[r][m] = fma(acc[r], t, acc2[r][m]);
    }
    if (p.dD && rowok) {
#pragma unroll
      for (int r = 0; r < 4; ++r) p.dD[(long)wrow * Dn + 16 * a + g + 4 * r] = acc[r];
    }
    // a column group is complete: flush it (the group a < 16 stays for the end)
    if (a >= 16 && ((a & 15) == 15 || a == p.L3 - 1)) {
      wave_lds_sync();
      const int abase = a & ~15, na = a - abase + 1;
#pragma unroll
      for (int rl = 0; rl < 16; ++rl) {
        // pass rl: row rl of the wave, lane = (m, al)
        const int atom = __shfl(my_atom, rl, 64);
        const int m = lane >> 4, al = lane & 15;
        if (al < na && row0 + 16 * w + rl < p.rows)
          p.dT[((long)atom * 4 + m) * p.L3 + abase + al] = Obw[kObRow * rl + lane];
      }
      wave_lds_sync();
    }
  }
  // a < 16: first term from the buffer + second term
  wave_lds_sync();
  if (rowok && S == 1) {
    double* out = p.dT + (long)my_atom * 4 * p.L3;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int b = g + 4 * r;
        out[m * p.L3 + b] = Obw[c * kObRow + m * 16 + b] + acc2[r][m];
      }
  } else if (rowok) {
    double* part = p.ws + ((long)s * p.rows + wrow) * 64;
    double* first = p.ws + ((long)S * p.rows + wrow) * 64;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int b = g + 4 * r;
        part[m * 16 + b] = acc2[r][m];
        if (s == S - 1) first[m * 16 + b] = Obw[c * kObRow + m * 16 + b];
      }
  }
}

// dT[atom][m][b < 16] of a split k_dDdT: the last split's first term plus the
// splits' second-term partials, summed in split order. One thread per (row,
// m, b).
template <class T>
__global__ __launch_bounds__(256) void k_ddt_combine(int rows, int L3, int nsplit, int pos0,
                                                     const int* items, const double* ws, T* dT) {
  const long q = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= (long)rows * 64) return;
  const int row = (int)(q >> 6), e = (int)(q & 63), m = e >> 4, b = e & 15;
  double sum = ws[q];
  for (int k = 1; k < nsplit; ++k) sum += ws[(long)k * rows * 64 + q];
  dT[((long)items[pos0 + row] * 4 + m) * L3 + b] = (T)(ws[(long)nsplit * rows * 64 + q] + sum);
}

// Mixed-precision form of k_dDdT: the same decomposition with the products on
// the bf16 matrix cores at fp32 accuracy (three-piece split, mfma3), fp32
// T / dT and fp32 sums. Lane (g, c) keeps the pieces of its row's dZ0 (row c
// of the wave; elements 32h + 8g + e of k chunk h, zero past K) as B
// operands; the block walks the column groups a with group a's pre-split W0
// fragments (tile-major pack_gemm_bf16 of W0^T: [L3][NC][3][64 lanes] x 16
// bytes, lane 16g + c holding W0[16a + c][32h + 8g + e]) and T column a of
// its rows staged through the LDS DMA. Register r of lane (g, c) of the
// product D'[b][row] is dD[row c][a][b = 4g + r] (the bf16 MFMA's result
// layout); first and second terms, flushes and splits as in k_dDdT.
constexpr int kObRow3 = 65;  // row stride (floats) of the first-term buffer: 64 + 1
// Column groups whose staging is in flight ahead of the one being multiplied
// (LDS holds kDdt3Ahead + 1). Measured on HEA-128k: two or three ahead gained
// nothing over one (fitting 2.50-2.52 ms either way), reading each chunk's
// weight pieces one chunk ahead of its products did (2.61 -> 2.50 ms).
constexpr int kDdt3Ahead = 1;

struct DdtArgs3 {
  int rows, K, L3;
  const float* dZ;  // [rows][K]
  const bf8* W0f;   // tile-major fragments, NC * 192 per column group
  const float* Tt;
  long ldt;
  int pos0;
  const int* items;
  float* dT;  // [atoms][4][L3]
  float* dD;  // [rows][16 L3] or null
  int nsplit;
  double* ws;  // as k_dDdT's
};

template <int WAVES, int NC>
__global__ __launch_bounds__(WAVES * 64) void k_dDdT3(DdtArgs3 p) {
  constexpr int BM = 16 * WAVES, NGB = NC * 192;
  static_assert(BM % 64 == 0 && NC % 2 == 0, "block rows in whole granule passes; K halves");
  extern __shared__ __align__(16) float lds3[];
  constexpr int NBUF = kDdt3Ahead + 1;
  bf8* Ws = reinterpret_cast<bf8*>(lds3);       // [NBUF][NGB]
  float* Ts = lds3 + NBUF * NGB * 4;            // [NBUF][BM][4]
  float* Ob = Ts + NBUF * BM * 4;               // [WAVES][16 rows][kObRow3]
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int row0 = blockIdx.x * BM, wrow = row0 + 16 * w + c;
  const bool rowok = wrow < p.rows;
  const int Dn = 16 * p.L3;
  float* Obw = Ob + w * 16 * kObRow3;
  const int S = p.nsplit, s = blockIdx.y, R = p.L3 - 16;
  auto bound = [&](int k) { return k >= S ? p.L3 : 16 * ((2 * k * R + 16 * S) / (32 * S)); };
  const int i0 = bound(s), i1 = bound(s + 1);
  Split3 Zb[NC];
#pragma unroll
  for (int h = 0; h < NC; ++h) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = 32 * h + 8 * g + e;
      v[e] = (rowok && k < p.K) ? p.dZ[(long)wrow * p.K + k] : 0.0f;
    }
    Zb[h] = split3(v);
  }
  const long tpos = 4L * wrow;
  const int my_atom = rowok ? p.items[p.pos0 + wrow] : 0;
  // T[row c][m][b = 4g + r]
  float Tc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m) Tc[r][m] = rowok ? p.Tt[(long)(4 * g + r) * p.ldt + tpos + m] : 0.0f;
  float acc2[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m) acc2[r][m] = 0.0f;

  // group a through the LDS DMA (16 bytes per lane, lane L's granule at
  // base + 16 L): its NGB weight granules, contiguous in the tile-major pack,
  // and T column a of the block's rows (one granule per row; rows past the
  // type's end read its last row and are not used). Every wave issues the
  // same number of transfers per group, NOPS (the weights in whole passes of
  // 64 granules, T as one pass of 16 lanes for the wave's own rows), so that
  // a fixed vmcnt finds a group landed with later groups still in flight.
  static_assert(NGB % (64 * WAVES) == 0, "weight passes per wave");
  constexpr int NOPS = NGB / (64 * WAVES) + 1;
  auto issue = [&](int buf, int a) {
#pragma unroll
    for (int k = 0; k < NGB / (64 * WAVES); ++k) {
      const int i = w + WAVES * k, q = 64 * i + lane;
      __builtin_amdgcn_global_load_lds(p.W0f + (long)a * NGB + q, LDS_PTR(Ws + buf * NGB + 64 * i),
                                       16, 0, 0);
    }
    if (lane < 16) {
      const int r = min(row0 + 16 * w + lane, p.rows - 1);
      __builtin_amdgcn_global_load_lds(p.Tt + (long)a * p.ldt + 4L * r,
                                       LDS_PTR(Ts + buf * BM * 4 + 64 * w), 16, 0, 0);
    }
  };
  auto col_of = [&](int i) { return i + 16 < p.L3 ? i + 16 : i + 16 - p.L3; };

#pragma unroll
  for (int k = 0; k < kDdt3Ahead; ++k)
    if (i0 + k < i1) issue(k, col_of(i0 + k));
  for (int i = i0; i < i1; ++i) {
    const int a = col_of(i), buf = (i - i0) % NBUF;
    // group i has landed: each wave's transfers of the kDdt3Ahead - 1 groups
    // after it may still be in flight (waiting for everything when fewer were
    // issued, and at the output flushes, whose stores come later in the
    // in-order count, is merely conservative); then the barrier, after which
    // no wave still reads the buffer group i + kDdt3Ahead goes to
    if (i + kDdt3Ahead - 1 < i1)
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NOPS * (kDdt3Ahead - 1)) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    if (i + kDdt3Ahead < i1) issue((i - i0 + kDdt3Ahead) % NBUF, col_of(i + kDdt3Ahead));
    // D'[b][row] over K in two accumulation chains (the halves of the
    // chunks), each chunk's weight pieces read from LDS one chunk ahead
    const bf8* A = Ws + buf * NGB + lane;
    auto wp = [&](int h) { return Split3{A[192 * h], A[192 * h + 64], A[192 * h + 128]}; };
    f4 acc0 = f4{0.0f, 0.0f, 0.0f, 0.0f}, acc1 = f4{0.0f, 0.0f, 0.0f, 0.0f};
    Split3 w0 = wp(0), w1 = wp(NC / 2);
#pragma unroll
    for (int h = 0; h < NC / 2; ++h) {
      // (scheduling barriers keep the reads ahead of this chunk's products;
      // left alone the compiler sinks each read to its use)
      Split3 n0 = w0, n1 = w1;
      if (h + 1 < NC / 2) {
        n0 = wp(h + 1);
        n1 = wp(h + 1 + NC / 2);
      }
      __builtin_amdgcn_sched_barrier(0);
      acc0 = mfma3(w0, Zb[h], acc0);
      acc1 = mfma3(w1, Zb[h + NC / 2], acc1);
      __builtin_amdgcn_sched_barrier(0);
      w0 = n0;
      w1 = n1;
    }
    f4 acc;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = acc0[r] + acc1[r];
    // first term: sum over b = 4g + r (lane-local over r, then the groups)
    float sm[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      float v = acc[0] * Tc[0][m];
      v += acc[1] * Tc[1][m];
      v += acc[2] * Tc[2][m];
      v += acc[3] * Tc[3][m];
      sm[m] = add_xor32(add_xor16(v));
    }
    Obw[c * kObRow3 + g * 16 + (a & 15)] = g == 0 ? sm[0] : g == 1 ? sm[1] : g == 2 ? sm[2] : sm[3];
    // second term: T[row][m][a]
    const float* tr = Ts + buf * BM * 4 + (16 * w + c) * 4;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const float t = tr[m];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc2[r][m] += acc[r] * t;
    }
    if (p.dD && rowok) {
#pragma unroll
      for (int r = 0; r < 4; ++r) p.dD[(long)wrow * Dn + 16 * a + 4 * g + r] = acc[r];
    }
    if (a >= 16 && ((a & 15) == 15 || a == p.L3 - 1)) {
      wave_lds_sync();
      const int abase = a & ~15, na = a - abase + 1;
#pragma unroll
      for (int rl = 0; rl < 16; ++rl) {
        const int atom = __shfl(my_atom, rl, 64);
        const int m = lane >> 4, al = lane & 15;
        if (al < na && row0 + 16 * w + rl < p.rows)
          p.dT[((long)atom * 4 + m) * p.L3 + abase + al] = Obw[kObRow3 * rl + lane];
      }
      wave_lds_sync();
    }
  }
  wave_lds_sync();
  if (rowok && S == 1) {
    float* out = p.dT + (long)my_atom * 4 * p.L3;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int b = 4 * g + r;
        out[m * p.L3 + b] = Obw[c * kObRow3 + m * 16 + b] + acc2[r][m];
      }
  } else if (rowok) {
    double* part = p.ws + ((long)s * p.rows + wrow) * 64;
    double* first = p.ws + ((long)S * p.rows + wrow) * 64;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int b = 4 * g + r;
        part[m * 16 + b] = acc2[r][m];
        if (s == S - 1) first[m * 16 + b] = Obw[c * kObRow3 + m * 16 + b];
      }
  }
}

template <int WAVES>
static size_t ddt_lds_bytes(int K) {
  return sizeof(double) * (2 * K * 16 + 2 * 16 * WAVES * 4 + WAVES * 16 * kObRow);
}

// Launch with the epilogue as a template parameter, instantiated only for the
// epilogues each operand form is used with: the first layer (A from T) plain
// or forward, the other forward layers forward or last-layer-with-head, the
// transposed-B products plain or backward.
template <class T, int NT, bool TRANSB, bool AT, int EPI>
static void gemm_launch(hipStream_t st, const GemmArgs<T>& a, dim3 grid) {
  if constexpr (sizeof(T) == 4) {
    if (a.Bf) {  // B pre-split: the bf16 three-piece kernel (B's orientation is in the fragments)
      hipLaunchKernelGGL((k_gemm3<NT, AT, EPI>), grid, dim3(256), 0, st, a);
      DPAMD_LAUNCH_CHECK();
      return;
    }
  }
  hipLaunchKernelGGL((k_gemm<T, NT, TRANSB, AT, EPI>), grid, dim3(256), 0, st, a);
  DPAMD_LAUNCH_CHECK();
}

template <class T, int NT, bool TRANSB, bool AT = false>
static void gemm_nt(hipStream_t st, const GemmArgs<T>& a) {
  dim3 grid(a.N / (16 * NT), (a.M + 63) / 64, a.split > 1 ? a.split : 1);
  if constexpr (TRANSB) {
    if (a.epi == 0) return gemm_launch<T, NT, TRANSB, AT, 0>(st, a, grid);
    if (a.epi == 2) return gemm_launch<T, NT, TRANSB, AT, 2>(st, a, grid);
  } else if constexpr (AT) {
    if (a.epi == 1) return gemm_launch<T, NT, TRANSB, AT, 1>(st, a, grid);
  } else {
    if (a.epi == 1) return gemm_launch<T, NT, TRANSB, AT, 1>(st, a, grid);
    if (a.epi == 3) return gemm_launch<T, NT, TRANSB, AT, 3>(st, a, grid);
  }
  throw HipError{hipErrorInvalidValue, "fitting GEMM: epilogue not available for this operand form"};
}

// Column tile (in MFMA tiles of 16 columns) of a fitting GEMM: the widest of
// 8, 5, 4 or 1 that divides N; an fp64 GEMM over few rows takes 3 when it
// divides N, for 5/3 as many blocks (a type of 8,192 rows, N = 240: 384 ->
// 640 blocks of 64 rows; the layer is too short to fill the GPU otherwise).
constexpr int kFewRows = 16384;
template <class T>
static int col_tiles(int M, int N) {
  const int tiles = N / 16;
  if (sizeof(T) == 8 && M < kFewRows && tiles % 3 == 0 && tiles % 8 != 0) return 3;
  return tiles % 8 == 0 ? 8 : tiles % 5 == 0 ? 5 : tiles % 4 == 0 ? 4 : 1;
}
template <bool TRANSB, class T>
static void gemm(hipStream_t st, const GemmArgs<T>& a) {
  if (a.M <= 0) return;
  switch (col_tiles<T>(a.M, a.N)) {
    case 8: gemm_nt<T, 8, TRANSB>(st, a); break;
    case 5: gemm_nt<T, 5, TRANSB>(st, a); break;
    case 4: gemm_nt<T, 4, TRANSB>(st, a); break;
    case 3:
      if constexpr (sizeof(T) == 8) {
        gemm_nt<T, 3, TRANSB>(st, a);
        break;
      }
      [[fallthrough]];
    default: gemm_nt<T, 1, TRANSB>(st, a);
  }
}

// First layer with A formed from T: the column tile is the widest of 8, 5, 4
// or 1 MFMA tiles dividing N, as in gemm().
template <class T>
static void gemm_at(hipStream_t st, const GemmArgs<T>& a) {
  if (a.M <= 0) return;
  const int tiles = a.N / 16;
  if (tiles % 8 == 0) gemm_nt<T, 8, false, true>(st, a);
  else if (tiles % 5 == 0) gemm_nt<T, 5, false, true>(st, a);
  else if (tiles % 4 == 0) gemm_nt<T, 4, false, true>(st, a);
  else gemm_nt<T, 1, false, true>(st, a);
}

template <class T>
void launch_fitting(hipStream_t st, const FitNet<T>& net, int rows, const T* D, const T* Tt,
                    long ldt, int L3, const FitBufs<T>& b, T* dD, double* e_bucket,
                    const FitDdt* ddt) {
  using G = GemmArgs<T>;
  if (rows <= 0) return;
  const int Dn = net.L[0].in, F0 = net.L[0].out, F1 = net.L[1].out, F2 = net.L[2].out;
  // the GEMM kernels address A by 32-bit element offsets within a type
  if ((long)rows * std::max(Dn, F0) > 0x7fffffffL)
    throw HipError{hipErrorInvalidValue,
                   "fitting input of one atom type exceeds 2^31 elements (atoms x descriptor width)"};
  G g{};
  // forward
  g = G{};
  g.M = rows; g.N = F0; g.K = Dn; g.A = D; g.lda = Dn; g.B = net.L[0].W; g.ldb = F0;
  g.epi = 1; g.bias = net.L[0].b; g.idt = nullptr; g.C = b.H0; g.ldc = F0; g.Bf = net.L[0].Wf;
  if (b.split > 1) {
    g.split = b.split;
    g.ws = b.ws;
  }
  if (Tt) {
    if (Dn != 16 * L3)
      throw HipError{hipErrorInvalidValue, "descriptor formed from T needs axis 16"};
    g.Tt = Tt;
    g.ldt = ldt;
    gemm_at(st, g);
  } else {
    gemm<false>(st, g);
  }
  if (b.split > 1) {
    const long groups = (long)rows * (F0 / 4);
    hipLaunchKernelGGL(k_splitk_tanh<T>, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st,
                       rows, F0, b.split, b.ws, net.L[0].b, b.H0);
    DPAMD_LAUNCH_CHECK();
  }
  g = G{};
  g.M = rows; g.N = F1; g.K = F0; g.A = b.H0; g.lda = F0; g.B = net.L[1].W; g.ldb = F1;
  g.epi = 1; g.bias = net.L[1].b; g.idt = net.L[1].idt; g.C = b.H1; g.ldc = F1; g.T_out = b.T1;
  g.Bf = net.L[1].Wf;
  gemm<false>(st, g);
  // last layer with the energy head: dZ2 = Wo idt2 (1 - T2^2) and the
  // partial energies; h2 and T2 are not stored
  g = G{};
  g.M = rows; g.N = F2; g.K = F1; g.A = b.H1; g.lda = F1; g.B = net.L[2].W; g.ldb = F2;
  g.epi = 3; g.bias = net.L[2].b; g.idt = net.L[2].idt; g.C = b.dZa; g.ldc = F2;
  g.Bf = net.L[2].Wf; g.Wo = net.Wo; g.epart = b.epart;
  gemm<false>(st, g);
  const int ncb = F2 / (16 * col_tiles<T>(rows, F2));
  hipLaunchKernelGGL(k_head_sum, dim3((rows + 255) / 256), dim3(256), 0, st, rows, ncb, b.epart,
                     net.bo, net.bias, e_bucket);
  DPAMD_LAUNCH_CHECK();
  // backward: dH1 = [res2] Wo + dZ2 W2^T, dZ1 = dH1 idt1 (1 - T1^2)
  g = G{};
  g.M = rows; g.N = F1; g.K = F2; g.A = b.dZa; g.lda = F2; g.B = net.L[2].W; g.ldb = F2;
  g.epi = 2; g.idt = net.L[1].idt; g.C = b.dZb; g.ldc = F1;
  g.dHin = net.L[2].idt ? net.Wo : nullptr; g.ld_dhin = 0; g.dH_out = b.dH; g.Tk = b.T1;
  g.Bf = net.L[2].WfT;
  gemm<true>(st, g);
  // dH0 = [res1] dH1 + dZ1 W1^T, dZ0 = dH0 (1 - H0^2)
  g = G{};
  g.M = rows; g.N = F0; g.K = F1; g.A = b.dZb; g.lda = F1; g.B = net.L[1].W; g.ldb = F1;
  g.epi = 2; g.idt = nullptr; g.C = b.dZa; g.ldc = F0;
  g.dHin = net.L[1].idt ? b.dH : nullptr; g.ld_dhin = F1; g.dH_out = nullptr; g.Tk = b.H0;
  g.Bf = net.L[1].WfT;
  gemm<true>(st, g);
  // dD = dZ0 W0^T, or straight on to dE/dT
  if (ddt) {
    if constexpr (sizeof(T) == 8)
      launch_dDdT(st, rows, F0, L3, b.dZa, static_cast<const double*>(ddt->W0T), Tt, ldt, ddt->pos0,
                  ddt->items, static_cast<double*>(ddt->dT), static_cast<double*>(ddt->dD), ddt->ncu,
                  ddt->nsplit, ddt->ws);
    else
      launch_dDdT3(st, rows, F0, L3, b.dZa, ddt->W0T, Tt, ldt, ddt->pos0, ddt->items,
                   static_cast<float*>(ddt->dT), static_cast<float*>(ddt->dD), ddt->ncu, ddt->nsplit,
                   ddt->ws);
    return;
  }
  // fitting shapes the fused kernels do not cover (F0 != 240 or axis != 16):
  // the plain product dD = dZ0 W0^T, then launch_dT
  g = G{};
  g.M = rows; g.N = Dn; g.K = F0; g.A = b.dZa; g.lda = F0; g.B = net.L[0].W; g.ldb = F0;
  g.epi = 0; g.C = dD; g.ldc = Dn;
  gemm<true>(st, g);
}

bool ddt_supported(int K, int L3, int axis) { return K == 240 && axis == 16 && L3 >= 16 && L3 <= 128; }

// Block shape of the fused kernel for a type of `rows` rows: eight waves (128
// rows) when that gives every compute unit two blocks; four (64 rows) when
// it gives one; otherwise eight waves with the column groups split over
// blockIdx.y, enough ways to give every compute unit a block (at most one
// way per 16 groups a >= 16). Returns the split count; *waves the shape.
static int ddt_shape(int rows, int L3, int ncu, int* waves) {
  const int nb8 = (rows + 127) / 128;
  *waves = 8;
  if (nb8 >= 2 * ncu) return 1;
  if (nb8 >= ncu) {
    *waves = 4;
    return 1;
  }
  const int smax = std::max(1, (L3 - 16) / 16);
  return std::min(smax, (ncu + nb8 - 1) / nb8);
}

int ddt_splits(int rows, int L3, int ncu) {
  int waves = 0;
  return ddt_shape(rows, L3, ncu, &waves);
}

void launch_dDdT(hipStream_t st, int rows, int K, int L3, const double* dZ, const double* W0T,
                 const double* Tt, long ldt, int pos0, const int* items, double* dT, double* dD,
                 int ncu, int nsplit, double* ws) {
  if (rows <= 0) return;
  if (K != 240) throw HipError{hipErrorInvalidValue, "fused dE/dD kernel needs F0 = 240"};
  int waves = 0;
  const int S = ddt_shape(rows, L3, ncu, &waves);
  if (S != nsplit || (S > 1 && !ws))
    throw HipError{hipErrorInvalidValue, "fused dE/dD kernel: split workspace does not match"};
  DdtArgs p{rows, K, L3, dZ, W0T, Tt, ldt, pos0, items, dT, dD, S, ws};
  if (waves == 8) {
    const size_t bytes = ddt_lds_bytes<8>(K);
    DPAMD_HIP(hipFuncSetAttribute((const void*)k_dDdT<8, 60>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    hipLaunchKernelGGL((k_dDdT<8, 60>), dim3((rows + 127) / 128, S), dim3(512), bytes, st, p);
  } else {
    const size_t bytes = ddt_lds_bytes<4>(K);
    DPAMD_HIP(hipFuncSetAttribute((const void*)k_dDdT<4, 60>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    hipLaunchKernelGGL((k_dDdT<4, 60>), dim3((rows + 63) / 64, S), dim3(256), bytes, st, p);
  }
  DPAMD_LAUNCH_CHECK();
  if (S > 1) {
    const long n = (long)rows * 64;
    hipLaunchKernelGGL(k_ddt_combine<double>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       rows, L3, S, pos0, items, ws, dT);
    DPAMD_LAUNCH_CHECK();
  }
}

template <int WAVES>
static size_t ddt3_lds_bytes(int NC) {
  constexpr int NBUF = kDdt3Ahead + 1;
  return (size_t)NBUF * NC * 192 * 16 +
         sizeof(float) * (NBUF * 16 * WAVES * 4 + WAVES * 16 * kObRow3);
}

void launch_dDdT3(hipStream_t st, int rows, int K, int L3, const float* dZ, const void* W0f,
                  const float* Tt, long ldt, int pos0, const int* items, float* dT, float* dD,
                  int ncu, int nsplit, double* ws) {
  if (rows <= 0) return;
  if (K != 240) throw HipError{hipErrorInvalidValue, "fused dE/dD kernel needs F0 = 240"};
  constexpr int NC = 8;  // 32-wide k chunks of K = 240 (zero-padded to 256)
  int waves = 0;
  const int S = ddt_shape(rows, L3, ncu, &waves);
  if (S != nsplit || (S > 1 && !ws))
    throw HipError{hipErrorInvalidValue, "fused dE/dD kernel: split workspace does not match"};
  DdtArgs3 p{rows, K, L3, dZ, static_cast<const bf8*>(W0f), Tt, ldt, pos0, items, dT, dD, S, ws};
  if (waves == 8) {
    const size_t bytes = ddt3_lds_bytes<8>(NC);
    DPAMD_HIP(hipFuncSetAttribute((const void*)k_dDdT3<8, NC>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    hipLaunchKernelGGL((k_dDdT3<8, NC>), dim3((rows + 127) / 128, S), dim3(512), bytes, st, p);
  } else {
    const size_t bytes = ddt3_lds_bytes<4>(NC);
    DPAMD_HIP(hipFuncSetAttribute((const void*)k_dDdT3<4, NC>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    hipLaunchKernelGGL((k_dDdT3<4, NC>), dim3((rows + 63) / 64, S), dim3(256), bytes, st, p);
  }
  DPAMD_LAUNCH_CHECK();
  if (S > 1) {
    const long n = (long)rows * 64;
    hipLaunchKernelGGL(k_ddt_combine<float>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, rows,
                       L3, S, pos0, items, ws, dT);
    DPAMD_LAUNCH_CHECK();
  }
}

template <class T>
void launch_dT(hipStream_t st, int nloc, int L3, int axis, const int* items, const T* Tt,
               const T* dD, T* dT) {
  if (nloc <= 0) return;
  if (L3 > 128 || axis < 1 || axis > 64 || axis > L3)
    throw HipError{hipErrorInvalidValue, "dE/dT kernel needs L3 <= 128 and axis <= min(64, L3)"};
  const dim3 grid((nloc + kDtWaves - 1) / kDtWaves), block(kDtWaves * 64);
  if (axis == 16 && L3 % 4 == 0)
    hipLaunchKernelGGL(k_dT<T>, grid, block, 0, st, nloc, L3, items, Tt, dD, dT);
  else
    hipLaunchKernelGGL(k_dT_any<T>, grid, block, 0, st, nloc, L3, axis, items, Tt, dD, dT);
  DPAMD_LAUNCH_CHECK();
}

template void launch_fitting<double>(hipStream_t, const FitNet<double>&, int, const double*,
                                     const double*, long, int, const FitBufs<double>&, double*,
                                     double*, const FitDdt*);
template void launch_fitting<float>(hipStream_t, const FitNet<float>&, int, const float*,
                                    const float*, long, int, const FitBufs<float>&, float*,
                                    double*, const FitDdt*);
template void launch_dT<double>(hipStream_t, int, int, int, const int*, const double*,
                                const double*, double*);
template void launch_dT<float>(hipStream_t, int, int, int, const int*, const float*, const float*,
                               float*);

}  // namespace dpamd
