// Fitting net (D -> F0 -> F1 -> F2 -> 1, tanh, y = x + idt*tanh(xW+b) on
// square layers) forward + input gradient on gfx950 FP64 MFMA, per centre
// type over the atoms of that type (bucket order), and the descriptor
// backward dE/dD -> dE/dT.
//
// Each layer is one GEMM (rows = atoms) with its elementwise work fused into
// the epilogue: bias + tanh + residual in the forward, (dH_in + acc) * idt *
// (1 - t^2) in the backward. Reference semantics: h = act(xW+b) (+ residual),
// e = h.w_head + b_head + bias_atom_e[type]
// (deepmd-op/overlays/op/pt/graph_fitting.cu:1-25, :614-719); the reference's
// fused tile analog is deepmd-op/overlays/op/pt/tiled_fitting.cuh:4-60.
#include "fastmath.h"
#include "kernels.h"

namespace dpamd {

struct GemmArgs {
  int M, N, K;
  const double* A;
  int lda;
  const double* B;
  int ldb;
  int epi;  // 0 plain store, 1 forward layer, 2 backward layer
  const double* bias;
  const double* idt;
  double* C;
  int ldc;
  double* T_out;       // forward: tanh part
  const double* dHin;  // backward: incoming dH (row stride ld_dhin; 0 = broadcast)
  int ld_dhin;
  double* dH_out;      // backward: dH of this layer
  const double* Tk;    // backward: tanh part of this layer (ld = ldc)
};

// C = epi(A[MxK] B[KxN]); B(k,n) = TRANSB ? B[n*ldb + k] : B[k*ldb + n].
// 64 x BN block tile, K staged through LDS 16 at a time; wave w owns rows
// 16w..16w+15 and all BN columns (BN/16 MFMA tiles sharing one A fragment).
template <int BN, bool TRANSB>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
  constexpr int BM = 64, BK = 16, NT = BN / 16;
  __shared__ double As[BM][BK + 1];
  __shared__ double Bs[BK][BN + 1];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
  d4 acc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n] = d4{0.0, 0.0, 0.0, 0.0};
  for (int k0 = 0; k0 < a.K; k0 += BK) {
    for (int q = tid; q < BM * BK; q += 256) {
      const int r = q / BK, kk = q % BK, gr = row0 + r;
      As[r][kk] = gr < a.M ? a.A[(long)gr * a.lda + k0 + kk] : 0.0;
    }
    for (int q = tid; q < BK * BN; q += 256) {
      if (!TRANSB) {
        const int kk = q / BN, n = q % BN;
        Bs[kk][n] = a.B[(long)(k0 + kk) * a.ldb + col0 + n];
      } else {
        const int n = q / BK, kk = q % BK;
        Bs[kk][n] = a.B[(long)(col0 + n) * a.ldb + k0 + kk];
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < BK / 4; ++q) {
      const double av = As[16 * w + c][4 * q + g];
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[n] = mfma_f64(av, Bs[4 * q + g][16 * n + c], acc[n]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int col = col0 + 16 * n + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 16 * w + g + 4 * r;
      if (row >= a.M) continue;
      const long o = (long)row * a.ldc + col;
      const double v = acc[n][r];
      if (a.epi == 0) {
        a.C[o] = v;
      } else if (a.epi == 1) {
        const double t = tanh_fast(v + a.bias[col]);
        if (a.T_out) a.T_out[o] = t;
        a.C[o] = a.idt ? a.A[(long)row * a.lda + col] + a.idt[col] * t : t;
      } else {
        const double dh = v + (a.dHin ? a.dHin[(long)row * a.ld_dhin + col] : 0.0);
        if (a.dH_out) a.dH_out[o] = dh;
        const double tk = a.Tk[o];
        a.C[o] = dh * (a.idt ? a.idt[col] : 1.0) * (1.0 - tk * tk);
      }
    }
  }
}

// Energy head and the seed of the backward: e = h2.Wo + bo + bias,
// dZ2 = Wo * idt2 * (1 - t2^2). One wave per atom row.
__global__ __launch_bounds__(256) void k_head(int rows, int F2, const double* __restrict__ H2,
                                              const double* __restrict__ T2,
                                              const double* __restrict__ Wo,
                                              const double* __restrict__ idt2, double bo,
                                              double bias, double* __restrict__ e,
                                              double* __restrict__ dZ2) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  double acc = 0.0;
  for (int f = lane; f < F2; f += 64) {
    const long o = (long)row * F2 + f;
    acc += H2[o] * Wo[f];
    const double t = T2[o];
    dZ2[o] = Wo[f] * (idt2 ? idt2[f] : 1.0) * (1.0 - t * t);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += shfl_xor_d(acc, off);
  if (lane == 0) e[row] = acc + bo + bias;
}

// dT[m][a] = sum_b dD[a][b] T[m][b] + (a < axis) sum_a' dD[a'][a] T[m][a'].
__global__ __launch_bounds__(256) void k_dT(int L3, int axis, const int* __restrict__ items,
                                            const double* __restrict__ T,
                                            const double* __restrict__ dD,
                                            double* __restrict__ dT) {
  extern __shared__ double sm[];
  const int pos = blockIdx.x, i = items[pos];
  double* Ts = sm;
  double* dDs = sm + 4 * L3;
  const int nd = L3 * axis;
  for (int q = threadIdx.x; q < 4 * L3; q += blockDim.x) Ts[q] = T[(long)i * 4 * L3 + q];
  for (int q = threadIdx.x; q < nd; q += blockDim.x) dDs[q] = dD[(long)pos * nd + q];
  __syncthreads();
  for (int q = threadIdx.x; q < 4 * L3; q += blockDim.x) {
    const int m = q / L3, ai = q % L3;
    const double* Tm = Ts + m * L3;
    double v = 0.0;
    for (int b = 0; b < axis; ++b) v += dDs[ai * axis + b] * Tm[b];
    if (ai < axis)
      for (int a2 = 0; a2 < L3; ++a2) v += dDs[a2 * axis + ai] * Tm[a2];
    dT[(long)i * 4 * L3 + q] = v;
  }
}

template <int BN, bool TRANSB>
static void gemm_bn(hipStream_t st, const GemmArgs& a) {
  dim3 grid(a.N / BN, (a.M + 63) / 64);
  hipLaunchKernelGGL((k_gemm<BN, TRANSB>), grid, dim3(256), 0, st, a);
  DPAMD_LAUNCH_CHECK();
}

template <bool TRANSB>
static void gemm(hipStream_t st, const GemmArgs& a) {
  if (a.M <= 0) return;
  if (a.N % 80 == 0) gemm_bn<80, TRANSB>(st, a);
  else if (a.N % 64 == 0) gemm_bn<64, TRANSB>(st, a);
  else gemm_bn<16, TRANSB>(st, a);
}

void launch_fitting(hipStream_t st, const FitNet& net, int rows, const double* D,
                    const FitBufs& b, double* dD, double* e_bucket) {
  if (rows <= 0) return;
  const int Dn = net.L[0].in, F0 = net.L[0].out, F1 = net.L[1].out, F2 = net.L[2].out;
  GemmArgs g{};
  // forward
  g = GemmArgs{};
  g.M = rows; g.N = F0; g.K = Dn; g.A = D; g.lda = Dn; g.B = net.L[0].W; g.ldb = F0;
  g.epi = 1; g.bias = net.L[0].b; g.idt = nullptr; g.C = b.H0; g.ldc = F0;
  gemm<false>(st, g);
  g = GemmArgs{};
  g.M = rows; g.N = F1; g.K = F0; g.A = b.H0; g.lda = F0; g.B = net.L[1].W; g.ldb = F1;
  g.epi = 1; g.bias = net.L[1].b; g.idt = net.L[1].idt; g.C = b.H1; g.ldc = F1; g.T_out = b.T1;
  gemm<false>(st, g);
  g = GemmArgs{};
  g.M = rows; g.N = F2; g.K = F1; g.A = b.H1; g.lda = F1; g.B = net.L[2].W; g.ldb = F2;
  g.epi = 1; g.bias = net.L[2].b; g.idt = net.L[2].idt; g.C = b.H2; g.ldc = F2; g.T_out = b.T2;
  gemm<false>(st, g);
  hipLaunchKernelGGL(k_head, dim3((rows + 3) / 4), dim3(256), 0, st, rows, F2, b.H2, b.T2, net.Wo,
                     net.L[2].idt, net.bo, net.bias, e_bucket, b.dZa);
  DPAMD_LAUNCH_CHECK();
  // backward: dH1 = [res2] Wo + dZ2 W2^T, dZ1 = dH1 idt1 (1 - T1^2)
  g = GemmArgs{};
  g.M = rows; g.N = F1; g.K = F2; g.A = b.dZa; g.lda = F2; g.B = net.L[2].W; g.ldb = F2;
  g.epi = 2; g.idt = net.L[1].idt; g.C = b.dZb; g.ldc = F1;
  g.dHin = net.L[2].idt ? net.Wo : nullptr; g.ld_dhin = 0; g.dH_out = b.dH; g.Tk = b.T1;
  gemm<true>(st, g);
  // dH0 = [res1] dH1 + dZ1 W1^T, dZ0 = dH0 (1 - H0^2)
  g = GemmArgs{};
  g.M = rows; g.N = F0; g.K = F1; g.A = b.dZb; g.lda = F1; g.B = net.L[1].W; g.ldb = F1;
  g.epi = 2; g.idt = nullptr; g.C = b.dZa; g.ldc = F0;
  g.dHin = net.L[1].idt ? b.dH : nullptr; g.ld_dhin = F1; g.dH_out = nullptr; g.Tk = b.H0;
  gemm<true>(st, g);
  // dD = dZ0 W0^T
  g = GemmArgs{};
  g.M = rows; g.N = Dn; g.K = F0; g.A = b.dZa; g.lda = F0; g.B = net.L[0].W; g.ldb = F0;
  g.epi = 0; g.C = dD; g.ldc = Dn;
  gemm<true>(st, g);
}

void launch_dT(hipStream_t st, int nloc, int L3, int axis, const int* items, const double* T,
               const double* dD, double* dT) {
  if (nloc <= 0) return;
  const size_t bytes = sizeof(double) * (4 * L3 + L3 * axis);
  hipLaunchKernelGGL(k_dT, dim3(nloc), dim3(256), bytes, st, L3, axis, items, T, dD, dT);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace dpamd
