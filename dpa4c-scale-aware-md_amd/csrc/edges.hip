// Edge-list front end: the caller's device edge graph (the contract of
// DeepPot::compute_edges_gpu, deepmd-op/overlays/api_cc/src/DeepPotPTExpt.cc:
// 2402-2470: edge_index [2][nedge], row 0 the neighbour / source node, row 1
// the centre / destination, edge_vec [nedge][3] = r_neighbour - r_centre) is
// turned into the extended-atom arrays the neighbour-list and model stages
// read. Every centre sits at the origin and edge e's neighbour at its bond
// vector (extended atom nloc + e, owner = its source node), so each distance
// the kernels form is the caller's vector exactly, no coordinates are needed,
// and the force gather folds each edge onto its source through the mapping.
#include "kernels.h"

namespace dpamd {
namespace {

// an edge is kept iff both its nodes lie in the graph (the same test in both
// kernels: a rank exists exactly for the kept edges)
__device__ __forceinline__ bool edge_ok(int s, int d, int nloc, int nnode) {
  return s >= 0 && s < nnode && d >= 0 && d < nloc;
}

template <class T>
__global__ void k_edges_ext(int nloc, int nedge, int nnode, const int* __restrict__ ei,
                            const T* __restrict__ vec, const int* __restrict__ atype,
                            double* __restrict__ ext, int* __restrict__ ext_type,
                            int* __restrict__ mapping, int* __restrict__ count,
                            int* __restrict__ rank, int* __restrict__ status) {
  const long q = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (q < nloc) {
    ext[3 * q] = ext[3 * q + 1] = ext[3 * q + 2] = 0.0;
    ext_type[q] = atype[q];
    mapping[q] = (int)q;
  }
  if (q >= nedge) return;
  const int s = ei[q], d = ei[nedge + q];
  const bool ok = edge_ok(s, d, nloc, nnode);
  const long x = nloc + q;
#pragma unroll
  for (int k = 0; k < 3; ++k) ext[3 * x + k] = (double)vec[3 * q + k];
  // an edge outside the graph has no type: the list never keeps it
  ext_type[x] = ok ? atype[s] : -1;
  mapping[x] = ok ? s : 0;
  if (ok) {
    rank[q] = atomicAdd(&count[d], 1);
  } else {
    atomicOr(status, kStatusBadInput);
  }
}

__global__ void k_edges_fill(int nloc, int nedge, int nnode, const int* __restrict__ ei,
                             const int* __restrict__ off, const int* __restrict__ rank,
                             long* __restrict__ cand_off, int* __restrict__ cand) {
  const long q = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (q <= nloc) cand_off[q] = off[q];
  if (q >= nedge) return;
  const int d = ei[nedge + q];
  if (!edge_ok(ei[q], d, nloc, nnode)) return;
  cand[off[d] + rank[q]] = nloc + (int)q;
}

}  // namespace

template <class T>
void launch_edges_ext(hipStream_t st, int nloc, int nedge, int nnode, const int* ei, const T* vec,
                      const int* atype, double* ext, int* ext_type, int* mapping, int* count,
                      int* rank, int* status) {
  const long n = std::max<long>(nloc, nedge);
  if (n <= 0) return;
  hipLaunchKernelGGL(k_edges_ext<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, nloc,
                     nedge, nnode, ei, vec, atype, ext, ext_type, mapping, count, rank, status);
  DPAMD_LAUNCH_CHECK();
}
template void launch_edges_ext<double>(hipStream_t, int, int, int, const int*, const double*,
                                       const int*, double*, int*, int*, int*, int*, int*);
template void launch_edges_ext<float>(hipStream_t, int, int, int, const int*, const float*,
                                      const int*, double*, int*, int*, int*, int*, int*);

void launch_edges_fill(hipStream_t st, int nloc, int nedge, int nnode, const int* ei,
                       const int* off, const int* rank, long* cand_off, int* cand) {
  const long n = std::max<long>(nloc + 1, nedge);
  hipLaunchKernelGGL(k_edges_fill, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, nloc,
                     nedge, nnode, ei, off, rank, cand_off, cand);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace dpamd
