// ProdForce / ProdVirial as a gather over the transposed neighbour list, plus
// the deterministic energy / virial reduction.
//
// Every edge e = (centre i, slot) with neighbour j contributes +g_e to the
// centre and -g_e to the target atom t = mapping[j] (standalone: ghost images
// folded onto owners) or t = j (LAMMPS path: ghost slots kept for reverse
// communication). One wave per atom t sums both sides: its own row of edges
// (t < nloc, coalesced) and the edges pointing at it, found through a reverse
// list built by count / scan / fill. The incoming edges are ranked by edge id
// in LDS first, so the sum order is fixed and the result bit-reproducible,
// with no floating-point atomics. Atom virial -g (x) (x_j - x_i) is charged to
// the target, as in deepmd-op/overlays/op/pt/edge_force_virial.cu:1-14,
// :138-146 (dual-CSR gather, one warp per node there, one 64-lane wave here);
// the frame virial is summed per centre from its own row. The frame sums
// follow the fixed two-stage fp64 reduction of edge_force_virial.cu:187-256.
#include "fixed.h"
#include "kernels.h"

namespace dpamd {

// se_e2_a: the embedding backward leaves each centre's own-row sums per
// neighbour section in cpsec [nloc][nsec][12] (fp64) and adds every edge's
// target side to fixed-point sums facc / vacc. One thread per target atom:
// force = own sums (sections in order) - incoming sum; atom virial = the
// incoming sum (charged to the neighbour). Centres of a negative type
// (absent, "virtual" atoms) have no sections. The same pass forms the first
// stage of the energy / virial reduction: block b sums the bucket energies
// e_bucket[p] and the centres' frame virials (the own sums' last nine) of
// its 256 indices into partials[b][10], which k_reduce_ev2 adds in block
// order.
__global__ __launch_bounds__(256) void k_finalize_ev(int ntarget, int nloc, int nbucket, int nsec,
                                                     const int* __restrict__ type,
                                                     const double* __restrict__ cpsec,
                                                     const unsigned long long* __restrict__ facc,
                                                     const unsigned long long* __restrict__ vacc,
                                                     const double* __restrict__ e_bucket,
                                                     double* __restrict__ force,
                                                     double* __restrict__ atom_virial,
                                                     double* __restrict__ partials) {
  __shared__ double sm[10][4];
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  double own[12];
#pragma unroll
  for (int q = 0; q < 12; ++q) own[q] = 0.0;
  if (t < nloc) {
    const int ns = type[t] >= 0 ? nsec : 0;
    for (int sec = 0; sec < ns; ++sec) {
      const double* cp = cpsec + ((long)t * nsec + sec) * 12;
#pragma unroll
      for (int q = 0; q < 12; ++q) own[q] += cp[q];
    }
  }
  if (t < ntarget) {
#pragma unroll
    for (int c = 0; c < 3; ++c) force[3L * t + c] = own[c] - from_fixed(facc[3L * t + c]);
    if (atom_virial) {
#pragma unroll
      for (int q = 0; q < 9; ++q) atom_virial[9L * t + q] = from_fixed(vacc[9L * t + q]);
    }
  }
  double part[10];
  part[0] = t < nbucket ? e_bucket[t] : 0.0;
#pragma unroll
  for (int q = 0; q < 9; ++q) part[1 + q] = own[3 + q];
  // ten block sums; each wave's partial in its own LDS row
#pragma unroll
  for (int q = 0; q < 10; ++q) {
    double v = part[q];
    v += __shfl_xor(v, 32, 64);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 1, 64);
    if ((threadIdx.x & 63) == 0) sm[q][threadIdx.x >> 6] = v;
  }
  __syncthreads();
  if (threadIdx.x < 10) {
    const double* r = sm[threadIdx.x];
    partials[(long)blockIdx.x * 10 + threadIdx.x] = (r[0] + r[1]) + (r[2] + r[3]);
  }
}

// Sums of extended atoms j in [j0, n) added onto their owners mapping[j] in
// dst (which may be src itself when every owner is below j0).
__global__ __launch_bounds__(256) void k_fold_fixed(int j0, int cap, const int* __restrict__ d_count,
                                                    const int* __restrict__ mapping,
                                                    const unsigned long long* src_f,
                                                    const unsigned long long* src_v,
                                                    unsigned long long* dst_f,
                                                    unsigned long long* dst_v) {
  const int n = d_count ? *d_count : cap;
  const int j = j0 + blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const long t = mapping[j];
#pragma unroll
  for (int c = 0; c < 3; ++c) atomicAdd(dst_f + 3 * t + c, src_f[3L * j + c]);
  if (src_v) {
#pragma unroll
    for (int q = 0; q < 9; ++q) atomicAdd(dst_v + 9 * t + q, src_v[9L * j + q]);
  }
}

__global__ __launch_bounds__(256) void k_zero_u64(long cap, const int* __restrict__ d_count,
                                                  int per, unsigned long long* __restrict__ p) {
  const long n = (d_count ? (long)*d_count : cap) * per;
  for (long q = (long)blockIdx.x * blockDim.x + threadIdx.x; q < n; q += (long)gridDim.x * blockDim.x)
    p[q] = 0ull;
}

void launch_fold_fixed(hipStream_t st, int j0, int cap, const int* d_count, const int* mapping,
                       const unsigned long long* src_f, const unsigned long long* src_v,
                       unsigned long long* dst_f, unsigned long long* dst_v) {
  if (cap <= j0 || !mapping) return;
  hipLaunchKernelGGL(k_fold_fixed, dim3((cap - j0 + 255) / 256), dim3(256), 0, st, j0, cap, d_count,
                     mapping, src_f, src_v, dst_f, dst_v);
  DPAMD_LAUNCH_CHECK();
}

void launch_zero_u64(hipStream_t st, long cap, const int* d_count, int per, unsigned long long* p) {
  if (cap <= 0) return;
  const long blocks = std::min<long>((cap * per + 255) / 256, 2048);
  hipLaunchKernelGGL(k_zero_u64, dim3((unsigned)blocks), dim3(256), 0, st, cap, d_count, per, p);
  DPAMD_LAUNCH_CHECK();
}

// The count keeps each edge's rank among the edges into its target (the value
// its increment returned), so the fill is a plain scatter; that order is
// arbitrary and the gather ranks the ids again.
__global__ void k_rev_count(long nedge, const int* __restrict__ nlist,
                            const int* __restrict__ mapping, int* __restrict__ count,
                            int* __restrict__ rank) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nedge) return;
  const int j = nlist[e];
  if (j < 0) return;
  rank[e] = atomicAdd(&count[mapping ? mapping[j] : j], 1);
}

__global__ void k_rev_fill(long nedge, const int* __restrict__ nlist,
                           const int* __restrict__ mapping, const int* __restrict__ off,
                           const int* __restrict__ rank, int* __restrict__ rev) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nedge) return;
  const int j = nlist[e];
  if (j < 0) return;
  const int t = mapping ? mapping[j] : j;
  rev[off[t] + rank[e]] = (int)e;
}

constexpr int kGatherWaves = 4;

// Sort this wave's incoming edge ids (s_in[0..n)) into s_out by rank: one
// pass over the list ranks all K ids a lane holds (q = lane + 64k). Edge ids
// are distinct.
template <int K>
__device__ __forceinline__ void rank_edges(int n, const int* s_in, int* s_out) {
  const int lane = threadIdx.x & 63;
  int ek[K], rank[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int q = lane + 64 * k;
    ek[k] = q < n ? s_in[q] : 0x7fffffff;
    rank[k] = 0;
  }
  for (int p = 0; p < n; ++p) {
    const int o = s_in[p];
#pragma unroll
    for (int k = 0; k < K; ++k) rank[k] += o < ek[k] ? 1 : 0;
  }
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (lane + 64 * k < n) s_out[rank[k]] = ek[k];
}

// force[t] = sum over t's own row of g (t < nloc) - sum over edges into t of g;
// atom_virial[t] = -sum over edges into t of g (x) d; cpart[t] (t < nloc) =
// the row's force and frame-virial sums (3 + 9).
__global__ __launch_bounds__(kGatherWaves * 64) void k_force_gather(
    int ntarget, int nloc, int nnei, const int* __restrict__ rev_off,
    const int* __restrict__ rev, const int* __restrict__ nlist, const double* __restrict__ ext,
    const double* __restrict__ edge_grad, double* __restrict__ cpart,
    double* __restrict__ force, double* __restrict__ atom_virial, int* __restrict__ status) {
  __shared__ int s_in[kGatherWaves][kMaxRev];
  __shared__ int s_sorted[kGatherWaves][kMaxRev];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * kGatherWaves + w;
  if (t >= ntarget) return;
  const int beg = rev_off[t];
  int n = rev_off[t + 1] - beg;
  if (n > kMaxRev) {
    if (lane == 0) atomicOr(status, kStatusReverseOverflow);
    n = kMaxRev;
  }
  for (int q = lane; q < n; q += 64) s_in[w][q] = rev[beg + q];
  // own row (centre side) while the reverse ids land in LDS
  double fo[3] = {0.0, 0.0, 0.0};
  double vo[9] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  if (t < nloc) {
    const double xi = ext[3 * (long)t], yi = ext[3 * (long)t + 1], zi = ext[3 * (long)t + 2];
    for (int sl = lane; sl < nnei; sl += 64) {
      const long e = (long)t * nnei + sl;
      const long j = nlist[e];
      if (j < 0) continue;
      const double g[3] = {edge_grad[3 * e], edge_grad[3 * e + 1], edge_grad[3 * e + 2]};
      const double d[3] = {ext[3 * j] - xi, ext[3 * j + 1] - yi, ext[3 * j + 2] - zi};
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        fo[a] += g[a];
#pragma unroll
        for (int b = 0; b < 3; ++b) vo[3 * a + b] -= g[a] * d[b];
      }
    }
  }
  wave_lds_sync();
  switch ((n + 63) / 64) {
    case 0: break;
    case 1: rank_edges<1>(n, s_in[w], s_sorted[w]); break;
    case 2: rank_edges<2>(n, s_in[w], s_sorted[w]); break;
    case 3: rank_edges<3>(n, s_in[w], s_sorted[w]); break;
    case 4: rank_edges<4>(n, s_in[w], s_sorted[w]); break;
    default: rank_edges<kMaxRev / 64>(n, s_in[w], s_sorted[w]); break;
  }
  wave_lds_sync();
  double f[3] = {0.0, 0.0, 0.0};
  double v[9] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  for (int q = lane; q < n; q += 64) {
    const long e = s_sorted[w][q];
    const double g0 = edge_grad[3 * e], g1 = edge_grad[3 * e + 1], g2 = edge_grad[3 * e + 2];
    f[0] -= g0;
    f[1] -= g1;
    f[2] -= g2;
    if (atom_virial) {
      const long i = e / nnei;
      const long j = nlist[e];
      const double d[3] = {ext[3 * j] - ext[3 * i], ext[3 * j + 1] - ext[3 * i + 1],
                           ext[3 * j + 2] - ext[3 * i + 2]};
      const double g[3] = {g0, g1, g2};
#pragma unroll
      for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 3; ++b) v[3 * a + b] -= g[a] * d[b];
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      f[q] += shfl_xor_d(f[q], off);
      fo[q] += shfl_xor_d(fo[q], off);
    }
    if (atom_virial) {
#pragma unroll
      for (int q = 0; q < 9; ++q) v[q] += shfl_xor_d(v[q], off);
    }
    if (t < nloc) {
#pragma unroll
      for (int q = 0; q < 9; ++q) vo[q] += shfl_xor_d(vo[q], off);
    }
  }
  if (lane == 0) {
    if (t < nloc) {
      double* cp = cpart + (long)t * 12;
      for (int q = 0; q < 3; ++q) cp[q] = fo[q];
      for (int q = 0; q < 9; ++q) cp[3 + q] = vo[q];
    }
    force[3 * (long)t] = f[0] + fo[0];
    force[3 * (long)t + 1] = f[1] + fo[1];
    force[3 * (long)t + 2] = f[2] + fo[2];
    if (atom_virial)
      for (int q = 0; q < 9; ++q) atom_virial[9 * (long)t + q] = v[q];
  }
}

constexpr int kRedBlocks = 256;

// Stage 1: block b sums energies of bucket positions and centre virials of
// centres b, b + 256, ...; stage 2 (one block) adds the 256 partials in order.
__global__ __launch_bounds__(256) void k_reduce_ev1(int nbucket, int nloc,
                                                    const double* __restrict__ e_bucket,
                                                    const double* __restrict__ cpart,
                                                    double* __restrict__ partials) {
  __shared__ double sm[10][256];
  double acc[10];
#pragma unroll
  for (int q = 0; q < 10; ++q) acc[q] = 0.0;
  const long stride = (long)kRedBlocks * 256;
  for (long p = (long)blockIdx.x * 256 + threadIdx.x; p < nbucket; p += stride) acc[0] += e_bucket[p];
  for (long s = (long)blockIdx.x * 256 + threadIdx.x; s < nloc; s += stride)
    for (int q = 0; q < 9; ++q) acc[1 + q] += cpart[s * 12 + 3 + q];
  for (int q = 0; q < 10; ++q) sm[q][threadIdx.x] = acc[q];
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if ((int)threadIdx.x < h)
      for (int q = 0; q < 10; ++q) sm[q][threadIdx.x] += sm[q][threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x < 10) partials[blockIdx.x * 10 + threadIdx.x] = sm[threadIdx.x][0];
}

// (nparts partials: thread k adds partials k, k + 256, ... in order first)
__global__ __launch_bounds__(256) void k_reduce_ev2(int nparts, const double* __restrict__ partials,
                                                    double* __restrict__ out10,
                                                    double* __restrict__ energy,
                                                    double* __restrict__ virial) {
  __shared__ double sm[10][256];
  for (int q = 0; q < 10; ++q) {
    double v = 0.0;
    for (int k = threadIdx.x; k < nparts; k += 256) v += partials[(long)k * 10 + q];
    sm[q][threadIdx.x] = v;
  }
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if ((int)threadIdx.x < h)
      for (int q = 0; q < 10; ++q) sm[q][threadIdx.x] += sm[q][threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x < 10) {
    const double v = sm[threadIdx.x][0];
    out10[threadIdx.x] = v;
    if (threadIdx.x == 0 && energy) *energy = v;
    if (threadIdx.x > 0 && virial) virial[threadIdx.x - 1] = v;
  }
}

__global__ void k_scatter_energy(int n, const int* __restrict__ items,
                                 const double* __restrict__ e_bucket,
                                 double* __restrict__ atom_energy) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p < n) atom_energy[items[p]] = e_bucket[p];
}

void launch_rev_count(hipStream_t st, long nedge, int, const int* nlist, const int* mapping,
                      int* count, int* rank) {
  if (nedge <= 0) return;
  hipLaunchKernelGGL(k_rev_count, dim3((unsigned)((nedge + 255) / 256)), dim3(256), 0, st, nedge,
                     nlist, mapping, count, rank);
  DPAMD_LAUNCH_CHECK();
}

void launch_rev_fill(hipStream_t st, long nedge, int, const int* nlist, const int* mapping,
                     const int* off, const int* rank, int* rev) {
  if (nedge <= 0) return;
  hipLaunchKernelGGL(k_rev_fill, dim3((unsigned)((nedge + 255) / 256)), dim3(256), 0, st, nedge,
                     nlist, mapping, off, rank, rev);
  DPAMD_LAUNCH_CHECK();
}

void launch_force_gather(hipStream_t st, int ntarget, int nloc, int nnei, const int* rev_off,
                         const int* rev, const int* nlist, const double* ext,
                         const double* edge_grad, double* cpart, double* force,
                         double* atom_virial, int* status) {
  if (ntarget <= 0) return;
  hipLaunchKernelGGL(k_force_gather, dim3((ntarget + kGatherWaves - 1) / kGatherWaves),
                     dim3(kGatherWaves * 64), 0, st, ntarget, nloc, nnei, rev_off, rev, nlist,
                     ext, edge_grad, cpart, force, atom_virial, status);
  DPAMD_LAUNCH_CHECK();
}

void launch_reduce_ev(hipStream_t st, int nbucket, int nloc, const double* e_bucket,
                      const double* cpart, double* partials, double* out10, double* energy,
                      double* virial) {
  hipLaunchKernelGGL(k_reduce_ev1, dim3(kRedBlocks), dim3(256), 0, st, nbucket, nloc, e_bucket,
                     cpart, partials);
  DPAMD_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_reduce_ev2, dim3(1), dim3(256), 0, st, kRedBlocks, partials, out10, energy,
                     virial);
  DPAMD_LAUNCH_CHECK();
}

int finalize_ev_blocks(int ntarget, int nloc, int nbucket) {
  return (std::max(std::max(ntarget, nloc), std::max(nbucket, 1)) + 255) / 256;
}

void launch_finalize_ev(hipStream_t st, int ntarget, int nloc, int nbucket, int nsec,
                        const int* type, const double* cpsec, const unsigned long long* facc,
                        const unsigned long long* vacc, const double* e_bucket, double* force,
                        double* atom_virial, double* partials, double* out10, double* energy,
                        double* virial) {
  const int nparts = finalize_ev_blocks(ntarget, nloc, nbucket);
  hipLaunchKernelGGL(k_finalize_ev, dim3(nparts), dim3(256), 0, st, ntarget, nloc, nbucket, nsec,
                     type, cpsec, facc, vacc, e_bucket, force, atom_virial, partials);
  DPAMD_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_reduce_ev2, dim3(1), dim3(256), 0, st, nparts, partials, out10, energy,
                     virial);
  DPAMD_LAUNCH_CHECK();
}

void launch_scatter_energy(hipStream_t st, int n, const int* items, const double* e_bucket,
                           double* atom_energy) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_scatter_energy, dim3((n + 255) / 256), dim3(256), 0, st, n, items, e_bucket,
                     atom_energy);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace dpamd
