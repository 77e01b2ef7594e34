// DPA4C-Nano energy / force evaluation on gfx950: the compressed degree-wise
// descriptor of dpa4c-runtime/include/dpa_chain/graph_compress.cuh and
// deepmd-op/overlays/op/pt/dpa4c/graph_compress_kernel.cuh (profile: 8 scalar
// channels, degrees <= 2, no spin, no radial modes), its one-hidden-layer
// fitting net (deepmd-op/overlays/op/pt/graph_fitting.cu:333-341) and the
// analytic backward to per-edge gradients dE/dd, d = x_src - x_dst.
//
// Three passes, all fp32 arithmetic with fp64 energies (the reference's
// precision split):
//   k_c4_moments    G lanes per destination node stride over its edges; each
//                   lane evaluates the whole edge (geometry, C3 envelope,
//                   quintic radial table, PairFiLM, degree-1/2 harmonics) and
//                   accumulates the 40 moments and 2 envelope masses in
//                   registers, reduced over the group by a butterfly. One
//                   lane per edge means no geometry is recomputed per channel.
//   k_c4_node       one thread per node: normalisation, alignment and probe
//                   projections, the 70 invariants, standardisation, the
//                   fitting net forward and its input gradient (weights read
//                   as wave-uniform scalar loads), then the readout VJP down
//                   to cotangents of the 42 raw sums.
//   k_c4_edge_grad  G lanes per node recompute each edge and contract it with
//                   the node's cotangents into dE/dd.
//   k_c4_edge_force on the standalone path (complete list folded onto
//                   owners) both directions of every edge at once, straight
//                   into forces and virials.
// Forces otherwise come from the shared gather (force.hip) on the LAMMPS
// path, or from k_c4_graph_force over the caller's two CSR views on the
// canonical graph path (deepmd-op/overlays/op/pt/edge_force_virial.cu:67-180 form:
// force[n] = sum(dst=n) g - sum(src=n) g, atom_virial[src] -= g (x) d).
#include <algorithm>

#include "fastmath.h"
#include "kernels.h"

namespace dpamd {
namespace {

constexpr int kBlock = 256;
constexpr int kEdgeBlock = 512;  // persistent edge passes: 32 nodes per block sweep
constexpr int kG = 16;           // lanes per node in the edge passes
constexpr int kLdsTableMax = 64 * 1024;
constexpr float kSq2 = 1.41421356237309505f;
constexpr float kSq3 = 1.73205080756887729f;
constexpr float kInvSq2 = 0.70710678118654752f;
constexpr float kInvSq5 = 0.44721359549995794f;
constexpr float kInvSq6 = 0.40824829046386302f;
constexpr float kKappa222 = -0.58554004376911988f;  // graph_compress.cuh:38

// Offsets in a node's 44-float moment / cotangent record.
constexpr int kS = 0, kV = 8, kT = 20, kMs = 40, kMa = 41;

struct Geo {
  float u[3];
  float ir, r, env;
  float x;  // position inside the table interval
  int idx;
};

__device__ __forceinline__ void geometry(const C4Params& p, const float d[3], Geo& g) {
  const float sq = fmaf(d[2], d[2], fmaf(d[1], d[1], fmaf(d[0], d[0], p.eps2)));
  g.ir = rsqrtf(sq);
  g.r = sq * g.ir;
#pragma unroll
  for (int k = 0; k < 3; ++k) g.u[k] = d[k] * g.ir;
  const float uu = fminf(fmaxf((p.rcut - g.r) * p.inv_rcut, 0.f), 1.f);
  const float x = 1.f - uu;
  const float ser = fmaf(x, fmaf(x, fmaf(x, fmaf(x, 35.f, 20.f), 10.f), 4.f), 1.f);
  const float uu2 = uu * uu;
  g.env = uu2 * uu2 * ser;
  // canonical table lookup (graph_compress.cuh:98-108); clamped at both ends
  // so that any input, NaN included, stays inside the table
  int idx = (int)(g.r * p.inv_stride);
  idx = min(max(idx, 0), p.n_int - 1);
  g.idx = idx;
  g.x = g.r - (float)idx * p.stride;
}

// d env / dr (graph_compress.cuh:229-241)
__device__ __forceinline__ float env_deriv(const C4Params& p, float r) {
  if (r <= 0.f || r >= p.rcut) return 0.f;
  const float x = r * p.inv_rcut, u = 1.f - x;
  const float ser = fmaf(x, fmaf(x, fmaf(x, fmaf(x, 35.f, 20.f), 10.f), 4.f), 1.f);
  const float dser = fmaf(x, fmaf(x, fmaf(x, 140.f, 60.f), 20.f), 4.f);
  const float u2 = u * u;
  return (-4.f * u2 * u * ser + u2 * u2 * dser) * p.inv_rcut;
}

__device__ __forceinline__ void harm2(const float u[3], float y[5]) {
  y[0] = kSq3 * u[0] * u[1];
  y[1] = kSq3 * u[1] * u[2];
  y[2] = 0.5f * (3.f * u[2] * u[2] - 1.f);
  y[3] = kSq3 * u[0] * u[2];
  y[4] = 0.5f * kSq3 * (u[0] * u[0] - u[1] * u[1]);
}

// radial_c(x) for the 8 channels from the interval's [6][8] coefficients
// Rows of `stride` float4 (12 in global memory; 13 in LDS, where a 12-float4
// stride puts every row on one of only 4 bank groups and the lanes' random
// rows collide, while 13 is coprime to the 16 float4 bank slots).
__device__ __forceinline__ void radial(const f4* tab, int stride, const Geo& g, float rad[8],
                                       float* drad) {
  const f4* row = tab + g.idx * stride;
  f4 c[12];
#pragma unroll
  for (int q = 0; q < 12; ++q) c[q] = row[q];
  const float x = g.x;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const float c0 = c[0 + h][l], c1 = c[2 + h][l], c2 = c[4 + h][l], c3 = c[6 + h][l],
                  c4 = c[8 + h][l], c5 = c[10 + h][l];
      rad[4 * h + l] = fmaf(fmaf(fmaf(fmaf(fmaf(c5, x, c4), x, c3), x, c2), x, c1), x, c0);
      if (drad)
        drad[4 * h + l] =
            fmaf(fmaf(fmaf(fmaf(5.f * c5, x, 4.f * c4), x, 3.f * c3), x, 2.f * c2), x, c1);
    }
}

__device__ __forceinline__ void film_of(const f4* flm, int pair, float a[8], float b[8]) {
  const f4* fr = flm + pair * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f4 v = fr[q];
    a[2 * q] = v[0];
    b[2 * q] = v[1];
    a[2 * q + 1] = v[2];
    b[2 * q + 1] = v[3];
  }
}

// The radial table and the PairFiLM rows every edge reads: staged once per
// block into LDS when they fit (each lane reads a random 192-byte table row,
// which from L2 would cost more than the edge's arithmetic), else read from
// global memory.
constexpr int kLdsRow = 13;  // float4 per table row in LDS

template <bool Lds>
__device__ __forceinline__ int table_stride() {
  return Lds ? kLdsRow : 12;
}

template <bool Lds>
__device__ __forceinline__ void stage_tables(const C4Params& p, const f4*& tab, const f4*& flm) {
  if constexpr (Lds) {
    extern __shared__ f4 c4_lds[];
    const int n1 = p.n_int * 12, n2 = p.nt * p.nt * 4;
    const f4* gt = reinterpret_cast<const f4*>(p.table);
    const f4* gf = reinterpret_cast<const f4*>(p.film);
    for (int q = threadIdx.x; q < n1; q += blockDim.x) c4_lds[(q / 12) * kLdsRow + q % 12] = gt[q];
    const int t1 = p.n_int * kLdsRow;
    for (int q = threadIdx.x; q < n2; q += blockDim.x) c4_lds[t1 + q] = gf[q];
    __syncthreads();
    tab = c4_lds;
    flm = c4_lds + t1;
  } else {
    tab = reinterpret_cast<const f4*>(p.table);
    flm = reinterpret_cast<const f4*>(p.film);
  }
}

// ---- edge sources ---------------------------------------------------------
// Sel-sorted list: the node's edges are the first nreal[t] slots of each
// type section, k-th edge overall -> (section, slot) by the running counts.
struct NlSrc {
  C4Nlist a;
  struct Node {
    double x[3];
    int cnt[kMaxTypes];
    int n;
    long row;
  };
  __device__ int node_type(int i) const { return a.ext_type[i]; }
  __device__ void open(const C4Params& p, int i, Node& nd) const {
    nd.row = (long)i * a.nnei;
    nd.n = 0;
#pragma unroll
    for (int t = 0; t < kMaxTypes; ++t) {
      nd.cnt[t] = t < p.nt ? a.nreal[(long)i * p.nt + t] : 0;
      nd.n += nd.cnt[t];
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) nd.x[k] = a.ext[3 * (long)i + k];
  }
  // returns false for an edge this pass must skip
  __device__ bool edge(const C4Params& p, const Node& nd, int k, float d[3], int& tj,
                       long& out) const {
    int j;
    return edge(p, nd, k, d, tj, out, j);
  }
  __device__ bool edge(const C4Params&, const Node& nd, int k, float d[3], int& tj, long& out,
                       int& j) const {
    int kk = k, base = 0;
    bool found = false;
#pragma unroll
    for (int t = 0; t < kMaxTypes; ++t) {
      if (!found) {
        if (kk < nd.cnt[t]) {
          found = true;
          base = a.sec[t];
        } else {
          kk -= nd.cnt[t];
        }
      }
    }
    out = nd.row + base + kk;
    j = a.nlist[out];
    tj = a.ext_type[j];
#pragma unroll
    for (int c = 0; c < 3; ++c) d[c] = (float)(a.ext[3 * (long)j + c] - nd.x[c]);
    return true;
  }
};

// Canonical graph: destination CSR of fp32 edge vectors.
struct GraphSrc {
  C4Graph a;
  struct Node {
    long beg;
    int n;
  };
  __device__ int node_type(int i) const { return (int)a.atype[i]; }
  __device__ void open(const C4Params&, int i, Node& nd) const {
    nd.beg = a.row_ptr[i];
    const long end = a.row_ptr[i + 1];
    // a row outside the edge storage is an input error: no edges
    if (nd.beg < 0 || end < nd.beg || end > a.storage || end - nd.beg > (1L << 20)) {
      atomicOr(a.status, kStatusBadInput);
      nd.n = 0;
      return;
    }
    nd.n = (int)(end - nd.beg);
  }
  __device__ bool edge(const C4Params& p, const Node& nd, int k, float d[3], int& tj,
                       long& out) const {
    out = nd.beg + k;
    if (out < 0 || out >= a.storage) {
      atomicOr(a.status, kStatusBadInput);
      out = -1;
      return false;
    }
    const long j = (long)a.source[out];
    if (j >= a.nall) {
      atomicOr(a.status, kStatusBadInput);
      return false;
    }
    tj = (int)a.atype[j];
#pragma unroll
    for (int c = 0; c < 3; ++c) d[c] = a.edge_vec[3 * out + c];
    return true;
  }
};

// ---- pass 1: moments --------------------------------------------------------
// Persistent blocks (grid of a few blocks per CU, the tables staged once):
// the nodes go in chunks of gpb (one node per group of kG lanes), walked
// XCD by XCD (xcd_chunks) so that neighbouring nodes share one L2.
template <class Src, bool Lds>
__global__ __launch_bounds__(kEdgeBlock) void k_c4_moments(C4Params p, Src src, int nnodes,
                                                          float* __restrict__ mom, int* status) {
  const f4 *tab, *flm;
  stage_tables<Lds>(p, tab, flm);
  const int lane = threadIdx.x & (kG - 1);
  constexpr int gpb = kEdgeBlock / kG;
  const ChunkWalk cw = xcd_chunks((nnodes + gpb - 1) / gpb);
  for (int ch = cw.first; ch < cw.end; ch += cw.step) {
  const int base = ch * gpb;
  const int node = base + (int)threadIdx.x / kG;
  float S[8], V[3][4], T[5][4], ms = 0.f, ma = 0.f;
#pragma unroll
  for (int c = 0; c < 8; ++c) S[c] = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int k = 0; k < 3; ++k) V[k][c] = 0.f;
#pragma unroll
    for (int m = 0; m < 5; ++m) T[m][c] = 0.f;
  }
  const int ti = node < nnodes ? src.node_type(node) : -1;
  if (ti >= 0 && ti < p.nt) {
    typename Src::Node nd;
    src.open(p, node, nd);
    for (int k = lane; k < nd.n; k += kG) {
      float d[3];
      int tj;
      long slot;
      if (!src.edge(p, nd, k, d, tj, slot)) continue;
      if (tj < 0 || tj >= p.nt) {
        atomicOr(status, kStatusBadInput);
        continue;
      }
      Geo g;
      geometry(p, d, g);
      float rad[8], fa[8], fb[8], y[5];
      radial(tab, table_stride<Lds>(), g, rad, nullptr);
      film_of(flm, ti * p.nt + tj, fa, fb);
      harm2(g.u, y);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float amp = fmaf(fa[c], rad[c], fb[c]) * g.env;
        S[c] += amp;
        if (c < 4) {
          const float ang = amp * g.env;
#pragma unroll
          for (int q = 0; q < 3; ++q) V[q][c] = fmaf(ang, g.u[q], V[q][c]);
#pragma unroll
          for (int m = 0; m < 5; ++m) T[m][c] = fmaf(ang, y[m], T[m][c]);
        }
      }
      const float e2 = g.env * g.env;
      ms += e2;
      ma = fmaf(e2, e2, ma);
    }
  } else if (node < nnodes && ti >= p.nt) {
    if (lane == 0) atomicOr(status, kStatusBadInput);
  }
  // butterfly over the group: every lane ends with the node's totals
#pragma unroll
  for (int off = 1; off < kG; off <<= 1) {
#pragma unroll
    for (int c = 0; c < 8; ++c) S[c] += __shfl_xor(S[c], off, kWave);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int k = 0; k < 3; ++k) V[k][c] += __shfl_xor(V[k][c], off, kWave);
#pragma unroll
      for (int m = 0; m < 5; ++m) T[m][c] += __shfl_xor(T[m][c], off, kWave);
    }
    ms += __shfl_xor(ms, off, kWave);
    ma += __shfl_xor(ma, off, kWave);
  }
  if (node < nnodes && lane == 0) {
    f4* o = reinterpret_cast<f4*>(mom + (long)node * kC4Mom);
    o[0] = f4{S[0], S[1], S[2], S[3]};
    o[1] = f4{S[4], S[5], S[6], S[7]};
#pragma unroll
    for (int k = 0; k < 3; ++k) o[2 + k] = f4{V[k][0], V[k][1], V[k][2], V[k][3]};
#pragma unroll
    for (int m = 0; m < 5; ++m) o[5 + m] = f4{T[m][0], T[m][1], T[m][2], T[m][3]};
    o[10] = f4{ms, ma, 0.f, 0.f};
  }
  }
}

// ---- pass 2: readout, fitting, readout VJP (one thread per node) ---------
// packed degree-two components -> symmetric traceless 3x3 (graph_compress.cuh:520-530)
__device__ __forceinline__ void stf(const float q[5], float M[3][3]) {
  M[0][0] = -q[2] * kInvSq6 + q[4] * kInvSq2;
  M[1][1] = -q[2] * kInvSq6 - q[4] * kInvSq2;
  M[2][2] = 2.f * q[2] * kInvSq6;
  M[0][1] = M[1][0] = q[0] * kInvSq2;
  M[1][2] = M[2][1] = q[1] * kInvSq2;
  M[0][2] = M[2][0] = q[3] * kInvSq2;
}

// adjoint of stf: 3x3 cotangent -> packed cotangent (graph_compress.cuh:547-554)
__device__ __forceinline__ void stf_adjoint(const float G[3][3], float q[5]) {
  q[0] += (G[0][1] + G[1][0]) * kInvSq2;
  q[1] += (G[1][2] + G[2][1]) * kInvSq2;
  q[2] += (-G[0][0] - G[1][1] + 2.f * G[2][2]) * kInvSq6;
  q[3] += (G[0][2] + G[2][0]) * kInvSq2;
  q[4] += (G[0][0] - G[1][1]) * kInvSq2;
}

__device__ __forceinline__ void mat3(const float A[3][3], const float B[3][3], float C[3][3]) {
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) C[i][j] = A[i][0] * B[0][j] + A[i][1] * B[1][j] + A[i][2] * B[2][j];
}

__device__ __forceinline__ void matvec(const float A[3][3], const float v[3], float o[3]) {
#pragma unroll
  for (int i = 0; i < 3; ++i) o[i] = A[i][0] * v[0] + A[i][1] * v[1] + A[i][2] * v[2];
}

// Normalised moments and the aligned / probe projections of one node.
struct Readout {
  float ns, na;
  float av[3][4], at[5][4], pv[3][4], pt[5][2];
  float Sm[2][3][3];  // STF of the two degree-two probes
};

__device__ __forceinline__ void project(const C4Params& p, const float m[kC4Mom], Readout& R) {
  R.ns = rsqrtf(m[kMs] + p.floor);
  R.na = rsqrtf(m[kMa] + p.floor);
  const float* Ma = p.ro;
  const float* Mt = p.ro + 16;
  const float* Pv = p.ro + 32;
  const float* Pt = p.ro + 48;
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) s = fmaf(m[kV + 4 * k + i] * R.na, Ma[4 * i + j], s);
      R.av[k][j] = s;
    }
#pragma unroll
  for (int q = 0; q < 5; ++q)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) s = fmaf(m[kT + 4 * q + i] * R.na, Mt[4 * i + j], s);
      R.at[q][j] = s;
    }
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) s = fmaf(R.av[k][i], Pv[4 * i + j], s);
      R.pv[k][j] = s;
    }
#pragma unroll
  for (int q = 0; q < 5; ++q)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) s = fmaf(R.at[q][i], Pt[2 * i + j], s);
      R.pt[q][j] = s;
    }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float q5[5] = {R.pt[0][k], R.pt[1][k], R.pt[2][k], R.pt[3][k], R.pt[4][k]};
    stf(q5, R.Sm[k]);
  }
}

__device__ __forceinline__ void load_mom(const float* src, float m[kC4Mom]) {
  const f4* s = reinterpret_cast<const f4*>(src);
#pragma unroll
  for (int q = 0; q < 11; ++q) {
    const f4 v = s[q];
    m[4 * q] = v[0];
    m[4 * q + 1] = v[1];
    m[4 * q + 2] = v[2];
    m[4 * q + 3] = v[3];
  }
}

__device__ __forceinline__ float act_val(int act, float z, float& dact) {
  if (act == 0) {
    const float t = tanh_f32(z);
    dact = fmaf(-t, t, 1.f);
    return t;
  }
  // silu z sigma(z), sigma = 1 / (1 + 2^(-z log2 e))
  const float sg = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.44269504088896341f * z));
  dact = sg * fmaf(z, 1.f - sg, 1.f);
  return z * sg;
}

template <class IT>
__global__ __launch_bounds__(kBlock) void k_c4_node(C4Params p, int nnodes,
                                                   const IT* __restrict__ type,
                                                   const float* __restrict__ mom,
                                                   double* __restrict__ energy,
                                                   float* __restrict__ cot) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i >= nnodes) return;
  const int ti = (int)type[i];
  f4* co = reinterpret_cast<f4*>(cot + (long)i * kC4Mom);
  if (ti < 0 || ti >= p.nt) {
    energy[i] = 0.0;
#pragma unroll
    for (int q = 0; q < 11; ++q) co[q] = f4{0.f, 0.f, 0.f, 0.f};
    return;
  }
  float D[kC4Out];
  {
    float m[kC4Mom];
    load_mom(mom + (long)i * kC4Mom, m);
    Readout R;
    project(p, m, R);
    int o = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) D[o++] = m[kS + c] * R.ns;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = r; c < 4; ++c)
        D[o++] = (R.av[0][r] * R.av[0][c] + R.av[1][r] * R.av[1][c] + R.av[2][r] * R.av[2][c]) *
                 (r == c ? 1.f : kSq2);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = r; c < 4; ++c) {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 5; ++q) s = fmaf(R.at[q][r], R.at[q][c], s);
        D[o++] = s * (r == c ? 1.f : kSq2);
      }
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int s = f; s < 4; ++s)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const float vs[3] = {R.pv[0][s], R.pv[1][s], R.pv[2][s]};
          float w[3];
          matvec(R.Sm[k], vs, w);
          const float val = R.pv[0][f] * w[0] + R.pv[1][f] * w[1] + R.pv[2][f] * w[2];
          D[o++] = -kInvSq5 * val * (f == s ? 1.f : kSq2);
        }
    {
      float P00[3][3], P01[3][3];
      mat3(R.Sm[0], R.Sm[0], P00);
      mat3(R.Sm[0], R.Sm[1], P01);
      float t000 = 0.f, t001 = 0.f, t011 = 0.f, t111 = 0.f;
      float P11[3][3];
      mat3(R.Sm[1], R.Sm[1], P11);
#pragma unroll
      for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 3; ++b) {
          t000 = fmaf(P00[a][b], R.Sm[0][a][b], t000);
          t001 = fmaf(P00[a][b], R.Sm[1][a][b], t001);
          t011 = fmaf(P01[a][b], R.Sm[1][a][b], t011);
          t111 = fmaf(P11[a][b], R.Sm[1][a][b], t111);
        }
      D[o++] = kKappa222 * t000;
      D[o++] = kKappa222 * kSq3 * t001;
      D[o++] = kKappa222 * kSq3 * t011;
      D[o++] = kKappa222 * t111;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float vv[3] = {R.pv[0][v], R.pv[1][v], R.pv[2][v]};
        float w[3];
        matvec(R.Sm[k], vv, w);
        D[o++] = w[0] * w[0] + w[1] * w[1] + w[2] * w[2];
      }
    D[o++] = sqrtf(m[kMs] + p.floor);
    D[o++] = sqrtf(m[kMa] + p.floor);
#pragma unroll
    for (int c = 0; c < 8; ++c) D[o++] = p.temb[ti * 8 + c];
#pragma unroll
    for (int q = 0; q < kC4Out; ++q) D[q] = (D[q] - p.mean[q]) * p.istd[q];
  }
  // fitting: e = sum_h wh[h] act(D . W0[:, h] + b0[h]) (+ D[h] on a square
  // residual layer) + bh + bias[type]; dD accumulated in the same pass
  float dD[kC4Out];
#pragma unroll
  for (int q = 0; q < kC4Out; ++q) dD[q] = 0.f;
  const bool res = (p.resnet & 1) && p.H == kC4Out;
  float e = 0.f;
  for (int h = 0; h < p.H; ++h) {
    const float* w = p.w0t + (long)h * kC4W0Ld;
    float z = p.b0[h];
#pragma unroll
    for (int q = 0; q < kC4Out; ++q) z = fmaf(D[q], w[q], z);
    float da;
    const float a = act_val(p.act, z, da);
    const float wh = p.wh[h];
    e = fmaf(wh, a, e);
    const float dz = wh * da;
#pragma unroll
    for (int q = 0; q < kC4Out; ++q) dD[q] = fmaf(dz, w[q], dD[q]);
  }
  if (res) {
    for (int h = 0; h < kC4Out; ++h) e = fmaf(p.wh[h], D[h], e);
#pragma unroll
    for (int q = 0; q < kC4Out; ++q) dD[q] += p.wh[q];
  }
  energy[i] = (double)(e + p.bh) + p.bias[ti];
  // ---- readout VJP: dD (standardised) -> cotangents of the raw sums ----
#pragma unroll
  for (int q = 0; q < kC4Out; ++q) dD[q] *= p.istd[q];
  float m[kC4Mom];
  load_mom(mom + (long)i * kC4Mom, m);
  Readout R;
  project(p, m, R);
  float gav[3][4], gat[5][4], gpv[3][4], gpt[5][2], gS[2][3][3];
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) gav[k][j] = gpv[k][j] = 0.f;
#pragma unroll
  for (int q = 0; q < 5; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) gat[q][j] = 0.f;
    gpt[q][0] = gpt[q][1] = 0.f;
  }
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) gS[k][a][b] = 0.f;
  int o = 8;
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = r; c < 4; ++c) {
      const float w = dD[o++] * (r == c ? 1.f : kSq2);
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        gav[k][r] = fmaf(w, R.av[k][c], gav[k][r]);
        gav[k][c] = fmaf(w, R.av[k][r], gav[k][c]);
      }
    }
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = r; c < 4; ++c) {
      const float w = dD[o++] * (r == c ? 1.f : kSq2);
#pragma unroll
      for (int q = 0; q < 5; ++q) {
        gat[q][r] = fmaf(w, R.at[q][c], gat[q][r]);
        gat[q][c] = fmaf(w, R.at[q][r], gat[q][c]);
      }
    }
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int s = f; s < 4; ++s)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const float coef = -kInvSq5 * dD[o++] * (f == s ? 1.f : kSq2);
        const float vf[3] = {R.pv[0][f], R.pv[1][f], R.pv[2][f]};
        const float vs[3] = {R.pv[0][s], R.pv[1][s], R.pv[2][s]};
        float Sr[3], Sl[3];
        matvec(R.Sm[k], vs, Sr);
        matvec(R.Sm[k], vf, Sl);
#pragma unroll
        for (int a = 0; a < 3; ++a) {
          gpv[a][f] = fmaf(coef, Sr[a], gpv[a][f]);
          gpv[a][s] = fmaf(coef, Sl[a], gpv[a][s]);
#pragma unroll
          for (int b = 0; b < 3; ++b) gS[k][a][b] = fmaf(coef * vf[a], vs[b], gS[k][a][b]);
        }
      }
  {
    // tr(ABC) over the entries (000), (001), (011), (111): d/dA = (BC)^T = C B
    // for symmetric factors, and likewise for B and C
    const float c0 = kKappa222 * dD[o++];
    const float c1 = kKappa222 * kSq3 * dD[o++];
    const float c2 = kKappa222 * kSq3 * dD[o++];
    const float c3 = kKappa222 * dD[o++];
    float P00[3][3], P01[3][3], P10[3][3], P11[3][3];
    mat3(R.Sm[0], R.Sm[0], P00);
    mat3(R.Sm[0], R.Sm[1], P01);
    mat3(R.Sm[1], R.Sm[0], P10);
    mat3(R.Sm[1], R.Sm[1], P11);
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        // (000): 3 S0^2 ; (001) A=B=S0, C=S1: dA = S1 S0, dB = S0 S1, dC = S0 S0
        // (011) A=S0, B=C=S1: dA = S1 S1, dB = S1 S0, dC = S0 S1 ; (111): 3 S1^2
        gS[0][a][b] += 3.f * c0 * P00[a][b] + c1 * (P10[a][b] + P01[a][b]) + c2 * P11[a][b];
        gS[1][a][b] += c1 * P00[a][b] + c2 * (P10[a][b] + P01[a][b]) + 3.f * c3 * P11[a][b];
      }
  }
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float vv[3] = {R.pv[0][v], R.pv[1][v], R.pv[2][v]};
      float w[3], gw[3], sg[3];
      matvec(R.Sm[k], vv, w);
      const float g2 = 2.f * dD[o++];
#pragma unroll
      for (int a = 0; a < 3; ++a) gw[a] = g2 * w[a];
      matvec(R.Sm[k], gw, sg);
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        gpv[a][v] += sg[a];
#pragma unroll
        for (int b = 0; b < 3; ++b) gS[k][a][b] = fmaf(gw[a], vv[b], gS[k][a][b]);
      }
    }
  const float gdiv0 = dD[o++], gdiv1 = dD[o++];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    float q5[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
    stf_adjoint(gS[k], q5);
#pragma unroll
    for (int q = 0; q < 5; ++q) gpt[q][k] += q5[q];
  }
  const float* Ma = p.ro;
  const float* Mt = p.ro + 16;
  const float* Pv = p.ro + 32;
  const float* Pt = p.ro + 48;
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
      float s = gav[k][i2];
#pragma unroll
      for (int j = 0; j < 4; ++j) s = fmaf(gpv[k][j], Pv[4 * i2 + j], s);
      gav[k][i2] = s;
    }
#pragma unroll
  for (int q = 0; q < 5; ++q)
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2)
      gat[q][i2] = fmaf(gpt[q][0], Pt[2 * i2], fmaf(gpt[q][1], Pt[2 * i2 + 1], gat[q][i2]));
  float c[kC4Mom];
  float g_ns = 0.f, g_na = 0.f;
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
    c[kS + cc] = dD[cc] * R.ns;
    g_ns = fmaf(dD[cc], m[kS + cc], g_ns);
  }
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) s = fmaf(gav[k][j], Ma[4 * i2 + j], s);
      c[kV + 4 * k + i2] = s * R.na;
      g_na = fmaf(s, m[kV + 4 * k + i2], g_na);
    }
#pragma unroll
  for (int q = 0; q < 5; ++q)
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) s = fmaf(gat[q][j], Mt[4 * i2 + j], s);
      c[kT + 4 * q + i2] = s * R.na;
      g_na = fmaf(s, m[kT + 4 * q + i2], g_na);
    }
  // ns = (ms + floor)^-1/2 and divisor sqrt(ms + floor): d/dms = -ns^3/2, ns/2
  c[kMs] = 0.5f * R.ns * (gdiv0 - g_ns * R.ns * R.ns);
  c[kMa] = 0.5f * R.na * (gdiv1 - g_na * R.na * R.na);
  c[42] = c[43] = 0.f;
#pragma unroll
  for (int q = 0; q < 11; ++q) co[q] = f4{c[4 * q], c[4 * q + 1], c[4 * q + 2], c[4 * q + 3]};
}

// ---- pass 3: edge gradients -------------------------------------------------
// dE/dd of one edge seen from a centre with cotangents c: PairFiLM (fa, fb)
// of (centre type, neighbour type), direction u from the centre, y = Y2(u),
// the radial values / slopes and d env / dr of the edge's length. Every
// operation is an explicit fmaf or product and contraction is off, so two
// inlined copies produce the same bits for the same inputs: the reverse
// direction of an edge evaluated by its other end then equals the forward
// evaluation exactly (negating u commutes with every operation below), which
// keeps sum F = 0 to fp64 rounding on the fused standalone path.
__device__ __forceinline__ void contract(const float c[kC4Mom], const float fa[8],
                                         const float fb[8], const Geo& g, const float u[3],
                                         const float y[5], const float rad[8],
                                         const float drad[8], float denv_dr, float out[3]) {
#pragma clang fp contract(off)
  const float env = g.env;
  float denv = 0.f, dr = 0.f, du[3] = {0.f, 0.f, 0.f}, hy[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
    const float film = fmaf(fa[cc], rad[cc], fb[cc]);
    const float amp = film * env;
    float damp = c[kS + cc];
    if (cc < 4) {
      const float ang = amp * env;
      float q = 0.f;
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        q = fmaf(c[kV + 4 * a + cc], u[a], q);
        du[a] = fmaf(ang, c[kV + 4 * a + cc], du[a]);
      }
#pragma unroll
      for (int m = 0; m < 5; ++m) {
        q = fmaf(c[kT + 4 * m + cc], y[m], q);
        hy[m] = fmaf(ang, c[kT + 4 * m + cc], hy[m]);
      }
      damp = fmaf(env, q, damp);
      denv = fmaf(amp, q, denv);
    }
    denv = fmaf(damp, film, denv);
    dr = fmaf((damp * env) * fa[cc], drad[cc], dr);
  }
  denv = fmaf(2.f * env, c[kMs], denv);
  denv = fmaf(((4.f * env) * env) * env, c[kMa], denv);
  dr = fmaf(denv, denv_dr, dr);
  // harmonics: dY/du (graph_compress.cuh:702-713)
  du[0] = fmaf(kSq3, fmaf(hy[4], u[0], fmaf(hy[3], u[2], hy[0] * u[1])), du[0]);
  du[1] = fmaf(kSq3, fmaf(-hy[4], u[1], fmaf(hy[1], u[2], hy[0] * u[0])), du[1]);
  du[2] = fmaf(3.f * hy[2], u[2], fmaf(kSq3, fmaf(hy[3], u[0], hy[1] * u[1]), du[2]));
  const float dot = fmaf(u[2], du[2], fmaf(u[1], du[1], u[0] * du[0]));
  // u = d / r with r = sqrt(|d|^2 + eps^2): du/dd = (I - u u^T) / r, dr/dd = u
#pragma unroll
  for (int a = 0; a < 3; ++a) out[a] = fmaf(fmaf(-u[a], dot, du[a]), g.ir, dr * u[a]);
}

template <class Src, bool Lds>
__global__ __launch_bounds__(kEdgeBlock) void k_c4_edge_grad(C4Params p, Src src, int nnodes,
                                                            const float* __restrict__ cot,
                                                            double* __restrict__ eg) {
  const f4 *tab, *flm;
  stage_tables<Lds>(p, tab, flm);
  const int lane = threadIdx.x & (kG - 1);
  constexpr int gpb = kEdgeBlock / kG;
  const ChunkWalk cw = xcd_chunks((nnodes + gpb - 1) / gpb);
  for (int ch = cw.first; ch < cw.end; ch += cw.step) {
  const int base = ch * gpb;
  const int node = base + (int)threadIdx.x / kG;
  if (node >= nnodes) continue;
  const int ti = src.node_type(node);
  const bool valid = ti >= 0 && ti < p.nt;
  typename Src::Node nd;
  src.open(p, node, nd);
  if (nd.n == 0) continue;
  float c[kC4Mom];
  load_mom(cot + (long)node * kC4Mom, c);
  for (int k = lane; k < nd.n; k += kG) {
    float d[3];
    int tj = -1;
    long slot = -1;
    // edges the forward skipped (bad type or source) get a zero gradient
    const bool ok = src.edge(p, nd, k, d, tj, slot);
    if (!ok || !valid || tj < 0 || tj >= p.nt) {
      if (slot >= 0)
#pragma unroll
        for (int a = 0; a < 3; ++a) eg[3 * slot + a] = 0.0;
      continue;
    }
    Geo g;
    geometry(p, d, g);
    float rad[8], drad[8], fa[8], fb[8], y[5];
    radial(tab, table_stride<Lds>(), g, rad, drad);
    film_of(flm, ti * p.nt + tj, fa, fb);
    harm2(g.u, y);
    float gr[3];
    contract(c, fa, fb, g, g.u, y, rad, drad, env_deriv(p, g.r), gr);
#pragma unroll
    for (int a = 0; a < 3; ++a) eg[3 * slot + a] = (double)gr[a];
  }
  }
}

// Both directions of every edge in one pass, for a complete (never
// truncated) list folded onto owners: the edge t -> j (owner i) has the
// reverse i -> image of t with vector -d, whose gradient is i's cotangents
// contracted with the same geometry (the degree-two harmonics are even in u,
// the radial and envelope terms depend on r only) under the swapped pair
// (tj, ti). So, per centre t and with no reverse list, atomics or scatter:
//   force[t]       = sum_e g(t->j) - g(i->t)
//   atom_virial[t] = -sum over edges into t of g (x) d_in = sum_e g(i->t) (x) d
//   cpart[t]       = (sum_e g(t->j), -sum_e g(t->j) (x) d), the centre-side
//                    force and frame-virial partials the reduction sums.
// Sums run in a fixed order (lane stride, then a butterfly): deterministic.
// Twelve waves per block (three per SIMD, 168 registers): the centre's
// cotangents sit in LDS (read by every edge of its lane group, not held in
// registers), and the atom virial is accumulated only when asked for (AV).
constexpr int kForceBlock = 768;
template <bool Lds, bool AV>
__global__ __launch_bounds__(kForceBlock) void k_c4_edge_force(
    C4Params p, NlSrc src, int nnodes, const int* __restrict__ mapping,
    const float* __restrict__ cot, double* __restrict__ force, double* __restrict__ atom_virial,
    double* __restrict__ cpart) {
  __shared__ f4 cown[kForceBlock / kG][kC4Mom / 4];
  const f4 *tab, *flm;
  stage_tables<Lds>(p, tab, flm);
  const int lane = threadIdx.x & (kG - 1), grp = (int)threadIdx.x / kG;
  constexpr int gpb = kForceBlock / kG;
  const ChunkWalk cw = xcd_chunks((nnodes + gpb - 1) / gpb);
  for (int ch = cw.first; ch < cw.end; ch += cw.step) {
  const int base = ch * gpb;
  const int node = base + grp;
  double f[3] = {0.0, 0.0, 0.0}, fo[3] = {0.0, 0.0, 0.0};
  double vo[9] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  double av[9] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  const int ti = node < nnodes ? src.node_type(node) : -1;
  // the group's cotangents into LDS (the group's lanes are one wave's; its
  // reads of the previous node's are all done)
  if (node < nnodes && lane < kC4Mom / 4)
    cown[grp][lane] = reinterpret_cast<const f4*>(cot + (long)node * kC4Mom)[lane];
  wave_lds_sync();
  if (ti >= 0 && ti < p.nt) {
    NlSrc::Node nd;
    src.open(p, node, nd);
    const float* c = reinterpret_cast<const float*>(cown[grp]);
    for (int k = lane; k < nd.n; k += kG) {
      // read the cotangents from LDS on every edge (keeps them out of the
      // registers: the compiler may not hoist the reads past this)
      asm volatile("" ::: "memory");
      float d[3];
      int tj, j;
      long slot;
      src.edge(p, nd, k, d, tj, slot, j);
      const int i = mapping[j];
      Geo g;
      geometry(p, d, g);
      float rad[8], drad[8], fa[8], fb[8], y[5];
      radial(tab, table_stride<Lds>(), g, rad, drad);
      harm2(g.u, y);
      const float de = env_deriv(p, g.r);
      float gf[3], gb[3];
      film_of(flm, ti * p.nt + tj, fa, fb);
      contract(c, fa, fb, g, g.u, y, rad, drad, de, gf);
      {
        float cn[kC4Mom];
        load_mom(cot + (long)i * kC4Mom, cn);
        film_of(flm, tj * p.nt + ti, fa, fb);
        const float um[3] = {-g.u[0], -g.u[1], -g.u[2]};
        contract(cn, fa, fb, g, um, y, rad, drad, de, gb);
      }
      double dd[3];
#pragma unroll
      for (int a = 0; a < 3; ++a) dd[a] = src.a.ext[3 * (long)j + a] - nd.x[a];
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        fo[a] += (double)gf[a];
        f[a] += (double)gf[a] - (double)gb[a];
#pragma unroll
        for (int b = 0; b < 3; ++b) {
          vo[3 * a + b] = fma(-(double)gf[a], dd[b], vo[3 * a + b]);
          if constexpr (AV) av[3 * a + b] = fma((double)gb[a], dd[b], av[3 * a + b]);
        }
      }
    }
  }
#pragma unroll
  for (int off = 1; off < kG; off <<= 1) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      f[a] += __shfl_xor(f[a], off, kWave);
      fo[a] += __shfl_xor(fo[a], off, kWave);
    }
#pragma unroll
    for (int a = 0; a < 9; ++a) {
      vo[a] += __shfl_xor(vo[a], off, kWave);
      if constexpr (AV) av[a] += __shfl_xor(av[a], off, kWave);
    }
  }
  if (node < nnodes && lane == 0) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      force[3 * (long)node + a] = f[a];
      cpart[12 * (long)node + a] = fo[a];
    }
#pragma unroll
    for (int a = 0; a < 9; ++a) cpart[12 * (long)node + 3 + a] = vo[a];
    if constexpr (AV)
#pragma unroll
      for (int a = 0; a < 9; ++a) atom_virial[9 * (long)node + a] = av[a];
  }
  }
}

// ---- canonical graph force / virial -------------------------------------
__global__ __launch_bounds__(kBlock) void k_c4_graph_force(
    int nall, const long* __restrict__ drow, const long* __restrict__ srow,
    const unsigned* __restrict__ sorder, const float* __restrict__ edge_vec,
    const double* __restrict__ eg, long storage, double* __restrict__ force,
    double* __restrict__ atom_virial, int* status) {
  const int lane = threadIdx.x & (kG - 1);
  const int node = (int)(((long)blockIdx.x * kBlock + threadIdx.x) / kG);
  double f[3] = {0.0, 0.0, 0.0}, v[9] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  if (node < nall) {
    for (long e = drow[node] + lane; e < drow[node + 1]; e += kG) {
      if (e < 0 || e >= storage) {
        atomicOr(status, kStatusBadInput);
        break;
      }
#pragma unroll
      for (int a = 0; a < 3; ++a) f[a] += eg[3 * e + a];
    }
    for (long q = srow[node] + lane; q < srow[node + 1]; q += kG) {
      if (q < 0 || q >= storage) {
        atomicOr(status, kStatusBadInput);
        break;
      }
      const long e = (long)sorder[q];
      if (e >= storage) {
        atomicOr(status, kStatusBadInput);
        continue;
      }
      const double g[3] = {eg[3 * e], eg[3 * e + 1], eg[3 * e + 2]};
      const double d[3] = {edge_vec[3 * e], edge_vec[3 * e + 1], edge_vec[3 * e + 2]};
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        f[a] -= g[a];
#pragma unroll
        for (int b = 0; b < 3; ++b) v[3 * a + b] = fma(-g[a], d[b], v[3 * a + b]);
      }
    }
  }
#pragma unroll
  for (int off = 1; off < kG; off <<= 1) {
#pragma unroll
    for (int a = 0; a < 3; ++a) f[a] += __shfl_xor(f[a], off, kWave);
#pragma unroll
    for (int a = 0; a < 9; ++a) v[a] += __shfl_xor(v[a], off, kWave);
  }
  if (node >= nall || lane != 0) return;
#pragma unroll
  for (int a = 0; a < 3; ++a) force[3 * (long)node + a] = f[a];
  if (atom_virial)
#pragma unroll
    for (int a = 0; a < 9; ++a) atom_virial[9 * (long)node + a] = v[a];
}

// Gradients of the edge slots past the local destination rows (ghost rows
// and reserved storage) are zero: the model has no edges there.
__global__ void k_c4_zero_tail(const long* __restrict__ drow, int nloc, long storage,
                               double* __restrict__ eg) {
  const long beg = drow[nloc] > 0 ? drow[nloc] : 0;
  for (long q = beg * 3 + (long)blockIdx.x * blockDim.x + threadIdx.x; q < storage * 3;
       q += (long)gridDim.x * blockDim.x)
    eg[q] = 0.0;
}

inline dim3 group_grid(long n) { return dim3((unsigned)((n * kG + kBlock - 1) / kBlock)); }

// LDS bytes of the staged tables (0: they do not fit and stay in global memory)
size_t table_lds_bytes(const C4Params& p) {
  const size_t b = ((size_t)p.n_int * kLdsRow + (size_t)p.nt * p.nt * 4) * sizeof(f4);
  return b <= (size_t)kLdsTableMax ? b : 0;
}

// persistent grid: `per_cu` blocks per compute unit, fewer if the nodes run out
dim3 edge_grid(const C4Params& p, long n, int per_cu) {
  const long need = (n + kEdgeBlock / kG - 1) / (kEdgeBlock / kG);
  return dim3((unsigned)std::max<long>(1, std::min<long>(need, (long)p.ncu * per_cu)));
}

template <class Src>
void moments_launch(hipStream_t st, const C4Params& p, const Src& src, int n, float* mom,
                    int* status) {
  if (n <= 0) return;
  const size_t lds = table_lds_bytes(p);
  if (lds)
    hipLaunchKernelGGL((k_c4_moments<Src, true>), edge_grid(p, n, 2), dim3(kEdgeBlock), lds, st,
                       p, src, n, mom, status);
  else
    hipLaunchKernelGGL((k_c4_moments<Src, false>), edge_grid(p, n, 2), dim3(kEdgeBlock), 0, st,
                       p, src, n, mom, status);
  DPAMD_LAUNCH_CHECK();
}

template <class Src>
void edge_grad_launch(hipStream_t st, const C4Params& p, const Src& src, int n, const float* cot,
                      double* eg) {
  if (n <= 0) return;
  const size_t lds = table_lds_bytes(p);
  if (lds)
    hipLaunchKernelGGL((k_c4_edge_grad<Src, true>), edge_grid(p, n, 1), dim3(kEdgeBlock), lds, st,
                       p, src, n, cot, eg);
  else
    hipLaunchKernelGGL((k_c4_edge_grad<Src, false>), edge_grid(p, n, 1), dim3(kEdgeBlock), 0, st,
                       p, src, n, cot, eg);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace

void launch_c4_moments(hipStream_t st, const C4Params& p, const C4Nlist& s, int n, float* mom,
                       int* status) {
  moments_launch(st, p, NlSrc{s}, n, mom, status);
}

void launch_c4_moments(hipStream_t st, const C4Params& p, const C4Graph& s, int n, float* mom,
                       int* status) {
  moments_launch(st, p, GraphSrc{s}, n, mom, status);
}

void launch_c4_node(hipStream_t st, const C4Params& p, int n, const int* type, const float* mom,
                    double* energy, float* cot) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_c4_node<int>, dim3((n + kBlock - 1) / kBlock), dim3(kBlock), 0, st, p, n,
                     type, mom, energy, cot);
  DPAMD_LAUNCH_CHECK();
}

void launch_c4_node(hipStream_t st, const C4Params& p, int n, const long* type, const float* mom,
                    double* energy, float* cot) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_c4_node<long>, dim3((n + kBlock - 1) / kBlock), dim3(kBlock), 0, st, p, n,
                     type, mom, energy, cot);
  DPAMD_LAUNCH_CHECK();
}

void launch_c4_edge_grad(hipStream_t st, const C4Params& p, const C4Nlist& s, int n,
                         const float* cot, double* eg) {
  edge_grad_launch(st, p, NlSrc{s}, n, cot, eg);
}

void launch_c4_edge_grad(hipStream_t st, const C4Params& p, const C4Graph& s, int n,
                         const float* cot, double* eg) {
  edge_grad_launch(st, p, GraphSrc{s}, n, cot, eg);
}

void launch_c4_edge_force(hipStream_t st, const C4Params& p, const C4Nlist& s, int n,
                          const int* mapping, const float* cot, double* force,
                          double* atom_virial, double* cpart) {
  if (n <= 0) return;
  const size_t lds = table_lds_bytes(p);
  constexpr int gpb = kForceBlock / kG;
  const dim3 grid((unsigned)std::max<long>(1, std::min<long>((n + gpb - 1) / gpb, (long)p.ncu)));
  auto go = [&](auto kern, size_t bytes) {
    hipLaunchKernelGGL(kern, grid, dim3(kForceBlock), bytes, st, p, NlSrc{s}, n, mapping, cot,
                       force, atom_virial, cpart);
  };
  if (lds)
    atom_virial ? go(k_c4_edge_force<true, true>, lds) : go(k_c4_edge_force<true, false>, lds);
  else
    atom_virial ? go(k_c4_edge_force<false, true>, 0) : go(k_c4_edge_force<false, false>, 0);
  DPAMD_LAUNCH_CHECK();
}

void launch_c4_zero_tail(hipStream_t st, const long* drow, int nloc, long storage, double* eg) {
  if (storage <= 0) return;
  hipLaunchKernelGGL(k_c4_zero_tail, dim3(256), dim3(256), 0, st, drow, nloc, storage, eg);
  DPAMD_LAUNCH_CHECK();
}

void launch_c4_graph_force(hipStream_t st, int nall, const long* drow, const long* srow,
                           const unsigned* sorder, const float* edge_vec, const double* eg,
                           long storage, double* force, double* atom_virial, int* status) {
  if (nall <= 0) return;
  hipLaunchKernelGGL(k_c4_graph_force, group_grid(nall), dim3(kBlock), 0, st, nall, drow, srow,
                     sorder, edge_vec, eg, storage, force, atom_virial, status);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace dpamd
