// Neighbour stage on gfx950: periodic ghost images, cell binning over the
// extended atoms, and the per-type sel-sorted neighbour list.
//
// This file is compiled with -ffp-contract=off: every squared distance is the
// plain IEEE sequence dx = xj - xi, r2 = dx*dx + dy*dy + dz*dz, and ghost
// coordinates are x + na*a + nb*b + nc*c evaluated left to right, so the list
// (which depends on exact comparisons of r2 at the sel truncation) is
// bit-identical to the CPU oracle's.
//
// Reference analogs: the warp-per-centre binned build
// lammps/overlays/src/KOKKOS/npair_kokkos.cpp:281-356 (here a 64-lane wave per
// centre with ballot compaction), the ballot/prefix compaction of
// lammps-deepmd-plugin/src/compact_canonical_graph_kokkos.h:447-491 and
// :643-745, and the exact-cut predicate include/dpa_chain/exact_cut.cuh:10-20.
// The sel formatting itself (upstream format_nlist) is absent from the
// reference: candidates with r2 <= rcut^2 are ranked by (type, r2, j) and the
// first sel[t] of type t fill section t, the rest -1.
#include "kernels.h"

#include <type_traits>

namespace dpamd {

__device__ __forceinline__ void to_frac(const BoxParams& bp, double x0, double x1, double x2,
                                        double* s) {
  s[2] = x2 / bp.h[8];
  s[1] = (x1 - s[2] * bp.h[7]) / bp.h[4];
  s[0] = (x0 - s[1] * bp.h[3] - s[2] * bp.h[6]) / bp.h[0];
}

// (also clears clear[0 .. nclear) for the next kernels, and sets *nall = nloc
// when given: no launches of their own)
__global__ void k_wrap(int nloc, const double* __restrict__ coord, const int* __restrict__ atype,
                       BoxParams bp, double* __restrict__ ext, int* __restrict__ ext_type,
                       int* __restrict__ mapping, double* __restrict__ sfrac, int nclear,
                       int* __restrict__ clear, int* __restrict__ nall) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < nclear) clear[k] = 0;
  if (nall && k == 0) *nall = nloc;
  if (k >= nloc) return;
  const double x0 = coord[3 * k], x1 = coord[3 * k + 1], x2 = coord[3 * k + 2];
  double w0 = x0, w1 = x1, w2 = x2;
  if (bp.periodic) {
    double s[3];
    to_frac(bp, x0, x1, x2, s);
    const double n0 = floor(s[0]), n1 = floor(s[1]), n2 = floor(s[2]);
    w0 = x0 - n0 * bp.h[0] - n1 * bp.h[3] - n2 * bp.h[6];
    w1 = x1 - n1 * bp.h[4] - n2 * bp.h[7];
    w2 = x2 - n2 * bp.h[8];
    double sw[3];
    to_frac(bp, w0, w1, w2, sw);
    sfrac[3 * k] = sw[0];
    sfrac[3 * k + 1] = sw[1];
    sfrac[3 * k + 2] = sw[2];
  }
  ext[3 * k] = w0;
  ext[3 * k + 1] = w1;
  ext[3 * k + 2] = w2;
  ext_type[k] = atype[k];
  mapping[k] = k;
}

__device__ __forceinline__ void decode_shift(const BoxParams& bp, int s, int* n) {
  const int wa = 2 * bp.nrep[0] + 1, wb = 2 * bp.nrep[1] + 1;
  const int q0 = (bp.nrep[2] * wb + bp.nrep[1]) * wa + bp.nrep[0];
  const int q = s < q0 ? s : s + 1;
  n[0] = q % wa - bp.nrep[0];
  n[1] = (q / wa) % wb - bp.nrep[1];
  n[2] = q / (wa * wb) - bp.nrep[2];
}

// The shift after n in decode_shift's order (an odometer over the image
// vectors that skips the zero vector): a block walking consecutive shifts
// decodes only its first.
__device__ __forceinline__ void next_shift(const BoxParams& bp, int* n) {
  for (int rep = 0; rep < 2; ++rep) {
    if (++n[0] > bp.nrep[0]) {
      n[0] = -bp.nrep[0];
      if (++n[1] > bp.nrep[1]) {
        n[1] = -bp.nrep[1];
        ++n[2];
      }
    }
    if (n[0] != 0 || n[1] != 0 || n[2] != 0) return;
  }
}

// Whether image s of atom k lies in the extended region.
__device__ __forceinline__ bool ghost_in(const BoxParams& bp, const double* __restrict__ sfrac,
                                         int k, const int (&n)[3]) {
  const double f0 = sfrac[3 * k] + (double)n[0];
  const double f1 = sfrac[3 * k + 1] + (double)n[1];
  const double f2 = sfrac[3 * k + 2] + (double)n[2];
  return f0 >= -bp.rcf[0] && f0 < bp.hi[0] && f1 >= -bp.rcf[1] && f1 < bp.hi[1] &&
         f2 >= -bp.rcf[2] && f2 < bp.hi[2];
}

// Ghost images in (shift, atom) order. Block (b, y) owns images s = y * spb ..
// y * spb + spb - 1 of the tile of atoms [256 b, 256 b + 256): k_ghost_count
// writes, per shift, how many of them land in the extended region
// (count[s * ntiles + b]); an exclusive scan of those counts gives every
// (shift, tile) its first ghost slot, and k_ghost_place re-tests the images
// and writes them there in atom order (wave ballots, then the earlier waves'
// totals through LDS, double-buffered by shift parity so one barrier per
// shift suffices). The order is that of one flag per (shift, atom) scanned in
// shift-major order, with nshift * nloc / 256 counts instead of nshift * nloc
// flags. spb (shifts per block) keeps the grid near a few thousand blocks:
// one shift per block for small systems, several for large ones.
constexpr int kGhostTile = 256;
__global__ __launch_bounds__(kGhostTile) void k_ghost_count(int nloc, int spb, BoxParams bp,
                                                           const double* __restrict__ sfrac,
                                                           int* __restrict__ count) {
  __shared__ int wc[2][kGhostTile / kWave];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = blockIdx.x * kGhostTile + threadIdx.x;
  const int s0 = blockIdx.y * spb, s1 = min(bp.nshift, s0 + spb);
  int n[3];
  decode_shift(bp, s0, n);
  for (int s = s0; s < s1; ++s, next_shift(bp, n)) {
    const bool in = k < nloc && ghost_in(bp, sfrac, k, n);
    const int c = __popcll(__ballot(in));  // (every lane votes: outside the lane-0 branch)
    if (lane == 0) wc[s & 1][w] = c;
    __syncthreads();  // (the other buffer was last read before the previous barrier)
    if (threadIdx.x == 0) {
      int t = 0;
#pragma unroll
      for (int q = 0; q < kGhostTile / kWave; ++q) t += wc[s & 1][q];
      count[(long)s * gridDim.x + blockIdx.x] = t;
    }
  }
}

__global__ __launch_bounds__(kGhostTile) void k_ghost_place(int nloc, int spb, BoxParams bp,
                                                           const double* __restrict__ sfrac,
                                                           const int* __restrict__ count,
                                                           const int* __restrict__ first,
                                                           double* __restrict__ ext,
                                                           int* __restrict__ ext_type,
                                                           int* __restrict__ mapping,
                                                           int* __restrict__ nall) {
  __shared__ int wc[2][kGhostTile / kWave];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = blockIdx.x * kGhostTile + threadIdx.x;
  const int s0 = blockIdx.y * spb, s1 = min(bp.nshift, s0 + spb);
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    const long last = (long)bp.nshift * gridDim.x - 1;  // the last (shift, tile)
    *nall = nloc + first[last] + count[last];
  }
  double x0 = 0.0, x1 = 0.0, x2 = 0.0;
  int tk = 0;
  if (k < nloc) {
    x0 = ext[3 * k];
    x1 = ext[3 * k + 1];
    x2 = ext[3 * k + 2];
    tk = ext_type[k];
  }
  int n[3];
  decode_shift(bp, s0, n);
  for (int s = s0; s < s1; ++s, next_shift(bp, n)) {
    const bool in = k < nloc && ghost_in(bp, sfrac, k, n);
    const unsigned long long m = __ballot(in);
    if (lane == 0) wc[s & 1][w] = __popcll(m);
    __syncthreads();
    if (in) {
      int before = (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
      for (int q = 0; q < w; ++q) before += wc[s & 1][q];
      const int o = nloc + first[(long)s * gridDim.x + blockIdx.x] + before;
      const double na = (double)n[0], nb = (double)n[1], nc = (double)n[2];
      ext[3 * o] = x0 + na * bp.h[0] + nb * bp.h[3] + nc * bp.h[6];
      ext[3 * o + 1] = x1 + nb * bp.h[4] + nc * bp.h[7];
      ext[3 * o + 2] = x2 + nc * bp.h[8];
      ext_type[o] = tk;
      mapping[o] = k;
    }
  }
}

__device__ __forceinline__ int cell_of_point(const BoxParams& bp, double x0, double x1, double x2) {
  double s[3];
  to_frac(bp, x0 - bp.origin[0], x1 - bp.origin[1], x2 - bp.origin[2], s);
  int c[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    int v = (int)floor((s[d] - bp.cell_lo[d]) / bp.cw[d]);
    v = v < 0 ? 0 : (v >= bp.ncell[d] ? bp.ncell[d] - 1 : v);
    c[d] = v;
  }
  return (c[2] * bp.ncell[1] + c[1]) * bp.ncell[0] + c[0];
}

// The atom count is cap, or *d_count when given (ghost count known on the
// device only; the grid then covers the capacity cap).
// Each atom's rank among the atoms of its cell comes from the count increment,
// so the scatter needs no second round of atomics (the order within a cell is
// arbitrary; the neighbour list sorts its candidates, or k_cell_order orders
// them). The lanes of a wave that fall in one cell (consecutive atoms often
// do) share one atomic: the first such lane adds the group's size, and each
// lane's rank is the returned count plus its place in the group.
__global__ void k_cell_assign(int cap, const int* __restrict__ d_count, BoxParams bp,
                              const double* __restrict__ ext, int* __restrict__ cell_of,
                              int* __restrict__ cell_rank, int* __restrict__ cell_count) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= (d_count ? *d_count : cap)) return;
  const int c = cell_of_point(bp, ext[3 * n], ext[3 * n + 1], ext[3 * n + 2]);
  cell_of[n] = c;
  unsigned long long left = __ballot(true);
  while (left) {  // wave-uniform: one round per distinct cell among the active lanes
    const int lead = __ffsll((long long)left) - 1;
    const int cl = __builtin_amdgcn_readlane(c, lead);
    const unsigned long long m = __ballot(c == cl) & left;
    int base = 0;
    if (threadIdx.x % kWave == lead) base = atomicAdd(&cell_count[cl], __popcll(m));
    base = __builtin_amdgcn_readlane(base, lead);
    if (c == cl)
      cell_rank[n] = base + (int)__builtin_amdgcn_mbcnt_hi(
                                (unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
    left &= ~m;
  }
}

__global__ void k_cell_scatter(int cap, const int* __restrict__ d_count,
                               const int* __restrict__ cell_of, const int* __restrict__ cell_rank,
                               const int* __restrict__ cell_start,
                               const double* __restrict__ ext, const int* __restrict__ ext_type,
                               CellAtom* __restrict__ sorted) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= (d_count ? *d_count : cap)) return;
  const int c = cell_of[n];
  const int p = cell_start[c] + cell_rank[n];
  CellAtom a;
  a.x = ext[3 * n];
  a.y = ext[3 * n + 1];
  a.z = ext[3 * n + 2];
  a.idx = n;
  a.type = ext_type[n];
  sorted[p] = a;
}

// Atoms of a cell in ascending index order (the scatter's order comes from
// atomic ranks): one wave per cell holds the cell's records in registers (K
// per lane), ranks them by index against the indices read back from the
// lanes (no memory access in the rank loop) and writes them back, so candidate
// order -- and with it an unsorted neighbour list -- is reproducible. Cells of
// more than kCellSortMax atoms keep the scatter's order (every access stays in
// bounds).
constexpr int kCellSortK = 8;
constexpr int kCellSortMax = 64 * kCellSortK;
template <int K>
__device__ __forceinline__ void cell_order_k(int beg, int cnt, CellAtom* __restrict__ sorted) {
  const int lane = threadIdx.x & 63;
  CellAtom a[K];
  int rank[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    rank[k] = 0;
    a[k].idx = 0x7fffffff;
    if (lane + 64 * k < cnt) a[k] = sorted[beg + lane + 64 * k];
  }
#pragma unroll
  for (int k2 = 0; k2 < K; ++k2) {
    const int m_end = min(cnt - 64 * k2, 64);  // wave-uniform
    for (int m = 0; m < m_end; ++m) {
      const int om = __builtin_amdgcn_readlane(a[k2].idx, m);
#pragma unroll
      for (int k = 0; k < K; ++k) rank[k] += om < a[k].idx ? 1 : 0;
    }
  }
  // every load above has been consumed (the ranks need all of them) before
  // the stores below
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (lane + 64 * k < cnt) sorted[beg + rank[k]] = a[k];
}

__global__ __launch_bounds__(256) void k_cell_order(int ncell, const int* __restrict__ cell_start,
                                                   CellAtom* __restrict__ sorted) {
  const int c = (int)(((long)blockIdx.x * 256 + threadIdx.x) >> 6);
  if (c >= ncell) return;
  const int beg = cell_start[c], cnt = cell_start[c + 1] - beg;
  if (cnt <= 1 || cnt > kCellSortMax) return;
  if (cnt <= 64) cell_order_k<1>(beg, cnt, sorted);
  else if (cnt <= 128) cell_order_k<2>(beg, cnt, sorted);
  else cell_order_k<kCellSortK>(beg, cnt, sorted);
}

// ---------------------------------------------------------------------------
// sel formatting shared by the cell and the CSR front ends. One wave per
// centre; candidates within rcut are compacted into LDS, ranked by
// (type, r2, j) and placed in their type section.
constexpr int kNlWaves = 4;

// Sort key: (type, r2) packed into one unsigned 64-bit integer whose order is
// the lexicographic order of the pair: r2 is positive, so its IEEE bits are
// monotone; offset by bits(2^-64) they fit in 59 bits for r2 < 256 (rcut < 16
// is enforced at model load) and the type goes above them. Ties (equal type
// and r2) are broken by the neighbour index j, as in the oracle.
struct NlKey {
  unsigned long long key;
  int j;
  int t;
};

struct NlLds {
  NlKey k[kNlWaves][kMaxCand];
  int claim[kNlWaves][kMaxCand];  // rank -> candidate, to detect equal keys
};

__device__ __forceinline__ unsigned long long nl_pack(int t, double r2) {
  const unsigned long long lo = 0x3BF0000000000000ull;  // bits of 2^-64
  unsigned long long b = (unsigned long long)__double_as_longlong(r2);
  b = b > lo ? b - lo : 0ull;
  return ((unsigned long long)t << 59) | b;
}

__device__ __forceinline__ void nl_push(bool keep, double r2, int j, int t, int& n, NlKey* s) {
  const unsigned long long m = __ballot(keep);
  const int lane = threadIdx.x & 63;
  const int before = __popcll(m & ((1ull << lane) - 1ull));
  if (keep) {
    const int q = n + before;
    if (q < kMaxCand) {
      NlKey e;
      e.key = nl_pack(t, r2);
      e.j = j;
      e.t = t;
      s[q] = e;
    }
  }
  n += __popcll(m);
}

// nl_push with the wave's keep mask given (the ballot of keep, formed by the
// caller from single compares)
__device__ __forceinline__ void nl_push_mask(unsigned long long m, bool keep, double r2, int j,
                                             int t, int& n, NlKey* s) {
  if (keep) {
    const int q = n + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32),
                                                     __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
    if (q < kMaxCand) {
      NlKey e;
      e.key = nl_pack(t, r2);
      e.j = j;
      e.t = t;
      s[q] = e;
    }
  }
  n += __popcll(m);
}

// Rank = #{keys below} + #{equal keys with a smaller index}. The first pass
// counts keys below only; equal keys are rare (exact r^2 ties), so each
// candidate then claims the LDS slot of its rank, and only if two candidates
// of the wave claimed the same slot does a second pass add the index
// tie-break.
template <int K>
__device__ __forceinline__ void nl_rank_place(const NlParams& np, int n, const NlKey* s,
                                              int* claim, const int* first,
                                              int* __restrict__ row) {
  const int lane = threadIdx.x & 63;
  unsigned long long ek[K];
  int ej[K], rank[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int q = lane + kWave * k;
    ek[k] = ~0ull;
    ej[k] = 0x7fffffff;
    rank[k] = 0;
    if (q < n) {
      ek[k] = s[q].key;
      ej[k] = s[q].j;
    }
  }
  for (int p = 0; p < n; ++p) {
    const unsigned long long ok = s[p].key;
#pragma unroll
    for (int k = 0; k < K; ++k) rank[k] += ok < ek[k] ? 1 : 0;
  }
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (lane + kWave * k < n) claim[rank[k]] = lane + kWave * k;
  wave_lds_sync();
  bool clash = false;
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (lane + kWave * k < n && claim[rank[k]] != lane + kWave * k) clash = true;
  if (__ballot(clash)) {
    for (int p = 0; p < n; ++p) {
      const unsigned long long ok = s[p].key;
      const int oj = s[p].j;
#pragma unroll
      for (int k = 0; k < K; ++k) rank[k] += (ok == ek[k] && oj < ej[k]) ? 1 : 0;
    }
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int q = lane + kWave * k;
    if (q < n) {
      const int t = s[q].t;
      const int r = rank[k] - first[t];
      if (r < np.sel[t]) row[np.sec[t] + r] = ej[k];
    }
  }
}

__device__ void nl_place(const NlParams& np, int i, int n, const NlKey* s, int* claim,
                         int* __restrict__ nlist, int* __restrict__ nreal,
                         int* __restrict__ status) {
  const int lane = threadIdx.x & 63;
  if (n > kMaxCand) {
    if (lane == 0) atomicOr(status, kStatusNeighbourOverflow);
    n = kMaxCand;
  }
  wave_lds_sync();
  int* row = nlist + (long)i * np.nnei;
  int cnt[kMaxTypes];
#pragma unroll
  for (int t = 0; t < kMaxTypes; ++t) cnt[t] = 0;
  for (int base = 0; base < n; base += kWave) {
    const int q = base + lane;
    const int tq = q < n ? s[q].t : -1;
#pragma unroll
    for (int t = 0; t < kMaxTypes; ++t) {
      if (t >= np.ntypes) break;  // wave-uniform: the arrays stay in registers
      cnt[t] += __popcll(__ballot(tq == t));
    }
  }
  int first[kMaxTypes];  // candidates of lower types
  int acc = 0;
#pragma unroll
  for (int t = 0; t < kMaxTypes; ++t) {
    first[t] = acc;
    acc += cnt[t];
  }
  if (np.unsorted) {
    // candidate order (reproducible with cell-ordered atoms), each type's
    // candidates compacted into its section
    int put[kMaxTypes];
#pragma unroll
    for (int t = 0; t < kMaxTypes; ++t) put[t] = 0;
    for (int base = 0; base < n; base += kWave) {
      const int q = base + lane;
      const int tq = q < n ? s[q].t : -1;
      const int jq = q < n ? s[q].j : -1;
#pragma unroll
      for (int t = 0; t < kMaxTypes; ++t) {
        if (t >= np.ntypes) break;
        const unsigned long long m = __ballot(tq == t);
        const int pos = put[t] + __popcll(m & ((1ull << lane) - 1ull));
        if (tq == t && pos < np.sel[t]) row[np.sec[t] + pos] = jq;
        put[t] += __popcll(m);
      }
    }
  } else {
  // rank of each candidate in (key, j) order: one pass over the list ranks
  // every candidate this lane holds (q = lane + 64k, k < K)
  switch ((n + kWave - 1) / kWave) {
    case 0: break;
    case 1: nl_rank_place<1>(np, n, s, claim, first, row); break;
    case 2: nl_rank_place<2>(np, n, s, claim, first, row); break;
    case 3: nl_rank_place<3>(np, n, s, claim, first, row); break;
    case 4: nl_rank_place<4>(np, n, s, claim, first, row); break;
    default: nl_rank_place<kMaxCand / kWave>(np, n, s, claim, first, row); break;
  }
  }
  for (int t = 0; t < np.ntypes; ++t) {
    if (np.sel_strict && cnt[t] > np.sel[t] && lane == 0) atomicOr(status, kStatusSelOverflow);
    const int kept = cnt[t] < np.sel[t] ? cnt[t] : np.sel[t];
    for (int sl = np.sec[t] + kept + lane; sl < np.sec[t + 1]; sl += kWave) row[sl] = -1;
    if (lane == 0) nreal[(long)i * np.ntypes + t] = kept;
  }
}

__device__ __forceinline__ void nl_empty_row(const NlParams& np, int i, int* __restrict__ nlist,
                                             int* __restrict__ nreal) {
  const int lane = threadIdx.x & 63;
  for (int s = lane; s < np.nnei; s += kWave) nlist[(long)i * np.nnei + s] = -1;
  if (lane < np.ntypes) nreal[(long)i * np.ntypes + lane] = 0;
}

// The stencil runs of centre cell ci: lane k < 9 gets run k's first sorted
// index (rbeg) and length (rcnt), and every lane the inclusive prefix of the
// lengths over lanes 0..lane (incl).
__device__ __forceinline__ void stencil_runs(const BoxParams& bp, int ci, int lane,
                                             const int* __restrict__ cell_start, int& rbeg,
                                             int& rcnt, int& incl) {
  const int c0 = ci % bp.ncell[0], c1 = (ci / bp.ncell[0]) % bp.ncell[1];
  const int c2 = ci / (bp.ncell[0] * bp.ncell[1]);
  rbeg = 0;
  rcnt = 0;
  if (lane < 9) {
    const int y = c1 + lane % 3 - 1, z = c2 + lane / 3 - 1;
    if (y >= 0 && y < bp.ncell[1] && z >= 0 && z < bp.ncell[2]) {
      const int x0 = c0 > 0 ? c0 - 1 : 0, x1 = c0 + 1 < bp.ncell[0] ? c0 + 1 : bp.ncell[0] - 1;
      const int rowc = (z * bp.ncell[1] + y) * bp.ncell[0];
      rbeg = cell_start[rowc + x0];
      rcnt = cell_start[rowc + x1 + 1] - rbeg;
    }
  }
  incl = rcnt;
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) {
    const int v = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += v;
  }
}

// Where candidate q of the concatenated runs lies in the cell-sorted array.
// The runs' offsets live in a register table (lane k: run k; lanes 9, 10: the
// end, as sentinels) read with a wave-uniform lane index, and a wave-uniform
// cursor follows the run that holds each batch's first candidate: a lane
// then needs one compare and select for the next boundary, and a batch that
// reaches past a second boundary (a run shorter than the batch, or an empty
// run) takes the general path over the later boundaries. Batches must be
// visited in increasing order.
struct RunCursor {
  int roffv, rdelv;  // lane k < 9: run k starts at roffv; candidate q is sorted[q + rdelv]
  int k, dcur, onext, dnext;
  __device__ __forceinline__ RunCursor(int lane, int incl, int rcnt, int rbeg, int total) {
    roffv = lane < 9 ? incl - rcnt : total;
    rdelv = rbeg - roffv;
    k = 0;
    dcur = __builtin_amdgcn_readlane(rdelv, 0);
    onext = __builtin_amdgcn_readlane(roffv, 1);
    dnext = __builtin_amdgcn_readlane(rdelv, 1);
  }
  // sorted index of candidate qc of the batch starting at b (qc < total)
  __device__ __forceinline__ int locate(int b, int qc) {
    while (onext <= b) {  // wave-uniform; empty runs are passed over here
      ++k;
      dcur = dnext;
      onext = __builtin_amdgcn_readlane(roffv, k + 1);
      dnext = __builtin_amdgcn_readlane(rdelv, k + 1);
    }
    int at = qc + dcur + (qc >= onext ? dnext - dcur : 0);
    if (__builtin_amdgcn_readlane(roffv, k + 2) < b + kWave) {
      asm volatile("");  // rare: kept as a branch, not evaluated for every batch
      for (int kk = k + 2; kk < 9; ++kk) {
        const int o = __builtin_amdgcn_readlane(roffv, kk);
        if (o >= b + kWave) break;
        if (qc >= o) at = qc + __builtin_amdgcn_readlane(rdelv, kk);
      }
    }
    return at;
  }
};

// Record `at` of the cell-sorted array: by a 32-bit byte offset from the
// array's (wave-uniform) base, one address instruction per lane, unless the
// array's capacity reaches 2^32 bytes (Wide).
template <bool Wide>
__device__ __forceinline__ CellAtom load_cand(const CellAtom* __restrict__ sorted, int at) {
  if constexpr (Wide) return sorted[at];
  return *reinterpret_cast<const CellAtom*>(reinterpret_cast<const char*>(sorted) +
                                            (unsigned)at * (unsigned)sizeof(CellAtom));
}

// The 27-cell stencil as 9 contiguous runs of the cell-sorted atoms (cells
// x-1..x+1 of one (y, z) row are adjacent in cell order). Lanes 0..8 read the
// run bounds at once (stencil_runs); candidate q of the concatenated runs is
// then found through RunCursor, so the candidates of a wave-wide batch are
// loaded independently (four rounds of 64 in flight) instead of cell after
// cell. The keep test is a set of single compares whose lane masks are ANDed
// on the scalar unit (a ballot of a combined boolean costs two instructions
// to rebuild the mask). Candidate order does not matter: the rank pass orders
// by (type, r^2, j).
template <bool Wide>
__global__ __launch_bounds__(kNlWaves * 64) void k_nlist_cells(
    int nloc, BoxParams bp, NlParams np, const double* __restrict__ ext,
    const int* __restrict__ ext_type, const int* __restrict__ cell_of,
    const int* __restrict__ cell_start, const CellAtom* __restrict__ sorted,
    int* __restrict__ nlist, int* __restrict__ nreal, int* __restrict__ status) {
  __shared__ NlLds lds;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = blockIdx.x * kNlWaves + w;
  if (i >= nloc) return;
  const int ti = ext_type[i];
  if (ti < 0 || ti >= np.ntypes) {
    nl_empty_row(np, i, nlist, nreal);
    return;
  }
  const double xi = ext[3 * i], yi = ext[3 * i + 1], zi = ext[3 * i + 2];
  int rbeg, rcnt, incl;
  stencil_runs(bp, cell_of[i], lane, cell_start, rbeg, rcnt, incl);
  const int total = __builtin_amdgcn_readlane(incl, 8);
  RunCursor rc(lane, incl, rcnt, rbeg, total);
  const unsigned nt = (unsigned)np.ntypes;
  int n = 0;
  for (int base = 0; base < total; base += 4 * kWave) {
    CellAtom ca[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int b = base + kWave * u;
      if (b < total) {  // wave-uniform
        const int qc = min(b + lane, total - 1);
        ca[u] = load_cand<Wide>(sorted, rc.locate(b, qc));
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int b = base + kWave * u;
      if (b >= total) break;  // wave-uniform
      const int j = ca[u].idx, t = ca[u].type;
      const double dx = ca[u].x - xi;
      const double dy = ca[u].y - yi;
      const double dz = ca[u].z - zi;
      const double r2 = dx * dx + dy * dy + dz * dz;
      // (bitwise, and ballots of single compares: each compare stays a lane
      // mask, combined on the scalar unit)
      const bool keep = (b + lane < total) & (j != i) & ((unsigned)t < nt) & (r2 <= np.rc2);
      const unsigned long long m = __ballot(b + lane < total) & __ballot(j != i) &
                                   __ballot((unsigned)t < nt) & __ballot(r2 <= np.rc2);
      nl_push_mask(m, keep, r2, j, t, n, lds.k[w]);
    }
  }
  nl_place(np, i, n, lds.k[w], lds.claim[w], nlist, nreal, status);
}

// Candidate-order list (NlParams::unsorted) over the same 9 runs. A kept
// candidate goes straight to its type section at its type's running count (one
// ballot and one masked prefix count per type and batch of 64), written into
// the wave's row in LDS (nnei ints per wave: no candidate array, so the LDS
// does not limit residency) and copied out whole at the end; no global store
// is issued inside the scan, so no candidate load waits behind one (the vector
// memory counter is in order). Candidates are found through RunCursor;
// lanes past the last candidate load the last one again and are not kept. Output, status bits and section order are those of k_nlist_cells
// with unsorted set: candidates in concatenation order, at most sel[t] per
// type, the rest -1. NT is the model's type count (np.ntypes).
template <int NT, bool Wide>
__global__ __launch_bounds__(kNlWaves * 64) void k_nlist_cells_seq(
    int nloc, BoxParams bp, NlParams np, const double* __restrict__ ext,
    const int* __restrict__ ext_type, const int* __restrict__ cell_of,
    const int* __restrict__ cell_start, const CellAtom* __restrict__ sorted,
    int* __restrict__ nlist, int* __restrict__ nreal, int* __restrict__ status) {
  extern __shared__ int nl_rows[];  // [kNlWaves][nnei]
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = blockIdx.x * kNlWaves + w;
  if (i >= nloc) return;
  const int ti = ext_type[i];
  if (ti < 0 || ti >= NT) {
    nl_empty_row(np, i, nlist, nreal);
    return;
  }
  const int nnei = np.nnei;
  int* lrow = nl_rows + w * nnei;
  for (int s = lane; s < nnei; s += kWave) lrow[s] = -1;
  const double xi = ext[3 * i], yi = ext[3 * i + 1], zi = ext[3 * i + 2];
  int rbeg, rcnt, incl;
  stencil_runs(bp, cell_of[i], lane, cell_start, rbeg, rcnt, incl);
  const int total = __builtin_amdgcn_readlane(incl, 8);
  RunCursor rc(lane, incl, rcnt, rbeg, total);
  int put[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) put[t] = 0;
  for (int base = 0; base < total; base += 2 * kWave) {
    CellAtom ca[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = base + kWave * u;
      if (b < total) {  // wave-uniform
        const int qc = min(b + lane, total - 1);
        ca[u] = load_cand<Wide>(sorted, rc.locate(b, qc));
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = base + kWave * u;
      if (b >= total) break;  // wave-uniform
      const int j = ca[u].idx, t = ca[u].type;
      const double dx = ca[u].x - xi;
      const double dy = ca[u].y - yi;
      const double dz = ca[u].z - zi;
      const double r2 = dx * dx + dy * dy + dz * dz;
      // (bitwise, and ballots of single compares: each compare stays a lane
      // mask, combined on the scalar unit)
      const bool keep = (b + lane < total) & (j != i) & (r2 <= np.rc2);
      const unsigned long long km =
          __ballot(b + lane < total) & __ballot(j != i) & __ballot(r2 <= np.rc2);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        const bool mine = keep & (t == tt);
        const unsigned long long m = __ballot(t == tt) & km;
        const unsigned pos = __builtin_amdgcn_mbcnt_hi(
            (unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u)) + (unsigned)put[tt];
        if (mine & (pos < (unsigned)np.sel[tt])) lrow[np.sec[tt] + pos] = j;
        put[tt] += __popcll(m);
      }
    }
  }
  wave_lds_sync();
  int* row = nlist + (long)i * nnei;
  for (int s = lane; s < nnei; s += kWave) row[s] = lrow[s];
  int n = 0;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    n += put[t];
    if (np.sel_strict && put[t] > np.sel[t] && lane == 0) atomicOr(status, kStatusSelOverflow);
    if (lane == 0) nreal[(long)i * NT + t] = put[t] < np.sel[t] ? put[t] : np.sel[t];
  }
  // the LDS form holds at most kMaxCand kept candidates; the same bound is
  // reported here so both forms fail alike
  if (n > kMaxCand && lane == 0) atomicOr(status, kStatusNeighbourOverflow);
}

// LAMMPS front end: candidates come from the caller's full list (CSR by centre).
__global__ __launch_bounds__(kNlWaves * 64) void k_nlist_csr(
    int nloc, NlParams np, const double* __restrict__ ext, const int* __restrict__ ext_type,
    const long* __restrict__ cand_off, const int* __restrict__ cand, int* __restrict__ nlist,
    int* __restrict__ nreal, int* __restrict__ status) {
  __shared__ NlLds lds;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = blockIdx.x * kNlWaves + w;
  if (i >= nloc) return;
  const int ti = ext_type[i];
  if (ti < 0 || ti >= np.ntypes) {
    nl_empty_row(np, i, nlist, nreal);
    return;
  }
  const double xi = ext[3 * i], yi = ext[3 * i + 1], zi = ext[3 * i + 2];
  const long beg = cand_off[i], end = cand_off[i + 1];
  int n = 0;
  for (long base = beg; base < end; base += kWave) {
    const long p = base + lane;
    bool keep = false;
    double r2 = 0.0;
    int j = -1, t = -1;
    if (p < end) {
      j = cand[p];
      t = ext_type[j];
      const double dx = ext[3 * (long)j] - xi;
      const double dy = ext[3 * (long)j + 1] - yi;
      const double dz = ext[3 * (long)j + 2] - zi;
      r2 = dx * dx + dy * dy + dz * dz;
      keep = (j != i) && t >= 0 && t < np.ntypes && r2 <= np.rc2;
    }
    nl_push(keep, r2, j, t, n, lds.k[w]);
  }
  nl_place(np, i, n, lds.k[w], lds.claim[w], nlist, nreal, status);
}

// ---------------------------------------------------------------------------
// Host launchers
void launch_wrap(hipStream_t st, int nloc, const double* coord, const int* atype,
                 const BoxParams& bp, double* ext, int* ext_type, int* mapping, double* sfrac,
                 int nclear, int* clear, int* nall) {
  const int n = std::max(std::max(nloc, nclear), nall ? 1 : 0);
  if (n <= 0) return;
  hipLaunchKernelGGL(k_wrap, dim3((n + 255) / 256), dim3(256), 0, st, nloc, coord, atype, bp, ext,
                     ext_type, mapping, sfrac, nclear, clear, nall);
  DPAMD_LAUNCH_CHECK();
}

int ghost_tiles(int nloc) { return (nloc + kGhostTile - 1) / kGhostTile; }

// shifts per block, and the grid: (tiles, shift groups)
static dim3 ghost_grid(int nloc, const BoxParams& bp, int* spb) {
  const long tiles = ghost_tiles(nloc), pairs = tiles * bp.nshift;
  *spb = (int)std::max(1L, (pairs + 4095) / 4096);
  const int groups = (bp.nshift + *spb - 1) / *spb;
  if (groups > 65535) throw HipError{hipErrorInvalidValue, "too many periodic images"};
  return dim3((unsigned)tiles, (unsigned)groups);
}

void launch_ghost_count(hipStream_t st, int nloc, const BoxParams& bp, const double* sfrac,
                        int* count) {
  if (nloc <= 0 || bp.nshift <= 0) return;
  int spb = 1;
  const dim3 grid = ghost_grid(nloc, bp, &spb);
  hipLaunchKernelGGL(k_ghost_count, grid, dim3(kGhostTile), 0, st, nloc, spb, bp, sfrac, count);
  DPAMD_LAUNCH_CHECK();
}

void launch_ghost_place(hipStream_t st, int nloc, const BoxParams& bp, const double* sfrac,
                        const int* count, const int* first, double* ext, int* ext_type,
                        int* mapping, int* nall) {
  if (nloc <= 0 || bp.nshift <= 0) return;
  int spb = 1;
  const dim3 grid = ghost_grid(nloc, bp, &spb);
  hipLaunchKernelGGL(k_ghost_place, grid, dim3(kGhostTile), 0, st, nloc, spb, bp, sfrac, count,
                     first, ext, ext_type, mapping, nall);
  DPAMD_LAUNCH_CHECK();
}

void launch_cell_assign(hipStream_t st, int cap, const int* d_count, const BoxParams& bp,
                        const double* ext, int* cell_of, int* cell_rank, int* cell_count) {
  if (cap <= 0) return;
  hipLaunchKernelGGL(k_cell_assign, dim3((cap + 255) / 256), dim3(256), 0, st, cap, d_count, bp,
                     ext, cell_of, cell_rank, cell_count);
  DPAMD_LAUNCH_CHECK();
}

void launch_cell_scatter(hipStream_t st, int cap, const int* d_count, const int* cell_of,
                         const int* cell_rank, const int* cell_start, const double* ext,
                         const int* ext_type, CellAtom* sorted) {
  if (cap <= 0) return;
  hipLaunchKernelGGL(k_cell_scatter, dim3((cap + 255) / 256), dim3(256), 0, st, cap, d_count,
                     cell_of, cell_rank, cell_start, ext, ext_type, sorted);
  DPAMD_LAUNCH_CHECK();
}

void launch_cell_order(hipStream_t st, int ncell, const int* cell_start, CellAtom* sorted) {
  if (ncell <= 0) return;
  hipLaunchKernelGGL(k_cell_order, dim3((unsigned)(((long)ncell * 64 + 255) / 256)), dim3(256), 0,
                     st, ncell, cell_start, sorted);
  DPAMD_LAUNCH_CHECK();
}

__global__ void k_fill_int(long n, int v, int* __restrict__ p) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

void launch_fill_int(hipStream_t st, long n, int v, int* p) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_fill_int, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, n, v, p);
  DPAMD_LAUNCH_CHECK();
}

void launch_nlist_cells(hipStream_t st, int nloc, const BoxParams& bp, const NlParams& np,
                        const double* ext, const int* ext_type, const int* cell_of,
                        const int* cell_start, const CellAtom* sorted, long sorted_cap,
                        int* nlist, int* nreal, int* status) {
  if (nloc <= 0) return;
  const dim3 grid((nloc + kNlWaves - 1) / kNlWaves), block(kNlWaves * 64);
  const bool wide = sorted_cap * (long)sizeof(CellAtom) >= (1L << 32);
  const size_t lds = np.unsorted ? kNlWaves * np.nnei * sizeof(int) : 0;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, block, lds, st, nloc, bp, np, ext, ext_type, cell_of,
                       cell_start, sorted, nlist, nreal, status);
  };
  auto seq = [&](auto wide_tag) {
    constexpr bool W = decltype(wide_tag)::value;
    switch (np.ntypes) {
      case 1: go(k_nlist_cells_seq<1, W>); break;
      case 2: go(k_nlist_cells_seq<2, W>); break;
      case 3: go(k_nlist_cells_seq<3, W>); break;
      case 4: go(k_nlist_cells_seq<4, W>); break;
      case 5: go(k_nlist_cells_seq<5, W>); break;
      case 6: go(k_nlist_cells_seq<6, W>); break;
      case 7: go(k_nlist_cells_seq<7, W>); break;
      default: go(k_nlist_cells_seq<kMaxTypes, W>); break;
    }
  };
  if (np.unsorted) {
    if (wide) seq(std::true_type{});
    else seq(std::false_type{});
  } else {
    if (wide) go(k_nlist_cells<true>);
    else go(k_nlist_cells<false>);
  }
  DPAMD_LAUNCH_CHECK();
}

void launch_nlist_csr(hipStream_t st, int nloc, const NlParams& np, const double* ext,
                      const int* ext_type, const long* cand_off, const int* cand, int* nlist,
                      int* nreal, int* status) {
  if (nloc <= 0) return;
  hipLaunchKernelGGL(k_nlist_csr, dim3((nloc + kNlWaves - 1) / kNlWaves), dim3(kNlWaves * 64), 0,
                     st, nloc, np, ext, ext_type, cand_off, cand, nlist, nreal, status);
  DPAMD_LAUNCH_CHECK();
}

}  // namespace dpamd
