/*
 * dp_amd.h — C ABI of the MI355X-native DeePMD evaluator (libdpamd.so): se_e2_a
 * models and the DPA4C compressed descriptor (Nano profile).
 *
 * This is the drop-in boundary for the per-step energy / force / virial call
 * that `pair_style deepmd` makes through the DeePMD C++ model API. Every entry
 * point takes plain pointers and sizes; no torch or C++ types cross it.
 * Return value: 0 on success, a negative DP_ERR_* code on failure, with the
 * message available from dp_last_error(). The C++ façade in
 * include/deepmd_amd/DeepPot.h turns failures into deepmd::deepmd_exception,
 * as the reference does (deepmd-op/overlays/api_cc/src/DeepPotPTExpt.cc:295-309,
 * caught by lammps-deepmd-plugin/src/pair_deepmd.cpp:372-374).
 *
 * Conventions (lammps-deepmd-plugin/src/pair_deepmd.cpp:293-307, :603-621):
 *   coord  [natoms][3] Angstrom, row-major;  atype [natoms] model type index,
 *          negative = virtual atom (no energy, no force, not a neighbour);
 *   box    [9] row-major h = [xx,0,0, xy,yy,0, xz,yz,zz] (lower-triangular,
 *          LAMMPS shape), or NULL for an open (non-periodic) system;
 *   energy [1] eV;  force [natoms][3] eV/A;  virial [9] eV, row-major
 *          W[3c+d] = -sum_edges g_c (x_j - x_i)_d;
 *   atom_energy [natoms];  atom_virial [natoms][9], charged to the neighbour
 *          (source) atom as in deepmd-op/overlays/op/pt/edge_force_virial.cu:1-14.
 * Any optional output pointer may be NULL.
 *
 * Threading: one handle per host thread; calls on one handle are serialised
 * by the caller (the reference keeps thread_local caches per model,
 * DeepPotPTExpt.cc:138).
 */
#ifndef DP_AMD_H
#define DP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DP_MAX_TYPES 8

enum {
  DP_OK = 0,
  DP_ERR_ARG = -1,      /* bad argument (null pointer, bad size, bad box) */
  DP_ERR_MODEL = -2,    /* model file missing, malformed or unsupported */
  DP_ERR_HIP = -3,      /* HIP runtime failure (allocation, launch, copy) */
  DP_ERR_CAPACITY = -4, /* a neighbour count exceeded a fixed kernel capacity */
  DP_ERR_NO_GPU = -5    /* no usable gfx950 device */
};

/* DP_PREC_MODEL: the precision the model file was written for (se_e2_a files
 * carry it in their header; DPA4C models are mixed by definition). */
enum { DP_PREC_FP64 = 0, DP_PREC_MIXED = 1, DP_PREC_MODEL = -1 };

/* Model families: se_e2_a (DPAMDSEA files) and the DPA4C compressed
 * degree-wise descriptor in its Nano profile (DPAMDC4N files). */
enum { DP_MODEL_SE_E2_A = 0, DP_MODEL_DPA4C = 1 };

typedef struct dp_model dp_model;

typedef struct {
  int ntypes;
  int nnei;
  int sel[DP_MAX_TYPES];
  double rcut;
  double rcut_smth;
  int emb[3];
  int axis;
  int fit[3];
  int dim_fparam;   /* always 0 for se_e2_a energy models here */
  int dim_aparam;   /* always 0 */
  int precision;    /* DP_PREC_* in use (DP_PREC_MIXED for DPA4C: fp32 nets) */
  char type_map[DP_MAX_TYPES][16];
  int model_kind;   /* DP_MODEL_*; for DPA4C emb = {C0, C1, C2} channel widths,
                       fit[0] = hidden width, axis = rcut_smth = 0 */
} dp_model_info;

/* Stage buffers of the last evaluation that dp_debug_copy can read back. */
enum {
  DP_STAGE_NLIST = 0,      /* int32 [nloc][nnei] (extended-atom indices, -1 pad) */
  DP_STAGE_EXT_COORD = 1,  /* f64 [nall][3] extended coordinates */
  DP_STAGE_MAPPING = 2,    /* int32 [nall] owner of each extended atom */
  DP_STAGE_DESCRPT = 3,    /* f64 [nloc][M1*axis] descriptor D (fp32 values in mixed mode) */
  DP_STAGE_ATOM_ENERGY = 4,/* f64 [nloc] */
  DP_STAGE_EDGE_GRAD = 5,  /* f64 [nloc][nnei][3] dE/d(x_j - x_i) */
  DP_STAGE_DEDD = 6,       /* f64 [nloc][M1*axis] dE/dD (fp32 values in mixed mode) */
  DP_STAGE_EXT_TYPE = 7,   /* int32 [nall] */
  DP_STAGE_C4_MOMENTS = 8, /* DPA4C: f32 [nloc][44] raw sums: scalar [8], vector [3][4],
                              tensor [5][4], sum env^2, sum env^4, 2 pad */
  DP_STAGE_C4_COTANGENTS = 9 /* DPA4C: f32 [nloc][44] dE/d(raw sums), same layout */
};

/*
 * Load a model and bind it to device `gpu_rank`.
 * Replaces deepmd::DeepPot::init(model, gpu_rank, file_content)
 * (deepmd-op/overlays/api_cc/include/DeepPot.h:475-477; called at
 * lammps-deepmd-plugin/src/pair_deepmd.cpp:668). If `file_content` is non-NULL
 * the model is read from those `content_len` bytes instead of `path`.
 * `precision` DP_PREC_MODEL takes the precision recorded in the model file
 * (upstream, the evaluation precision is a property of the trained model);
 * DP_PREC_FP64 evaluates everything in fp64; DP_PREC_MIXED
 * evaluates the embedding nets, the descriptor and the fitting net in fp32
 * (FP32 MFMA) and the env matrix, edge gradients, forces, virials and energy
 * sums in fp64 -- the reference's mixed-precision rule (fp32
 * embedding/fitting, fp64 env matrix, force and virial accumulation), checked
 * against its acceptance limits (data/numeric-tolerances.json:3-9).
 */
int dp_create(const char* path, int gpu_rank, const void* file_content, size_t content_len,
              int precision, dp_model** out);

/* Release the handle and every device buffer it owns. */
void dp_destroy(dp_model* model);

/*
 * Model metadata: cutoff(), numb_types(), dim_fparam(), dim_aparam(),
 * get_type_map() of the reference model API
 * (deepmd-op/overlays/api_cc/include/DeepPotPTExpt.h:103-154; used at
 * lammps-deepmd-plugin/src/pair_deepmd.cpp:672-677, :1000).
 */
int dp_get_info(const dp_model* model, dp_model_info* info);

/* Message of the last failure on this handle ("" if none). */
const char* dp_last_error(const dp_model* model);

/*
 * Standalone evaluation from coordinates and box: ghost images, neighbour
 * list and evaluation are built on the GPU; ghost forces / virials are folded
 * onto their owners. Replaces DeepPot::compute(ener, force, virial,
 * [atom_energy, atom_virial,] coord, atype, box)
 * (deepmd-op/overlays/api_cc/include/DeepPot.h:503-522, :605-628;
 * backend path DeepPotPTExpt.cc:1643-1957). Host pointers.
 */
int dp_compute(dp_model* model, int natoms, const double* coord, const int* atype,
               const double* box, double* energy, double* force, double* virial,
               double* atom_energy, double* atom_virial);

/*
 * LAMMPS neighbour-list evaluation. coord/atype cover nall = nloc + nghost
 * atoms; the neighbour list (inum, ilist, numneigh, firstneigh) is LAMMPS'
 * full list with skin, indices into the nall atoms (masked with `neigh_mask`,
 * pass 0x1FFFFFFF for LAMMPS' NEIGHMASK, or 0 for no mask). force and
 * atom_virial cover all nall atoms; ghost contributions stay in ghost slots for
 * LAMMPS' reverse communication. `ago == 0` means the list was rebuilt and is
 * re-uploaded; otherwise the cached list is reused and only re-filtered.
 * Replaces DeepPot::compute(ener, force, virial, [atom_energy, atom_virial,]
 * coord, atype, box, nghost, lmp_list, ago)
 * (deepmd-op/overlays/api_cc/include/DeepPot.h:551-576, :661-690; called at
 * lammps-deepmd-plugin/src/pair_deepmd.cpp:370-371, :381-383). Host pointers.
 */
int dp_compute_nlist(dp_model* model, int nall, int nghost, const double* coord,
                     const int* atype, const double* box, int inum, const int* ilist,
                     const int* numneigh, const int* const* firstneigh, int neigh_mask, int ago,
                     double* energy, double* force, double* virial, double* atom_energy,
                     double* atom_virial);

/*
 * Device-resident standalone evaluation: every array pointer is device memory
 * on the handle's GPU except `box` (host, 9 doubles); work is ordered on
 * `stream` (a hipStream_t, NULL = default stream) and the call returns after
 * the outputs are complete on that stream. `ago == 0` refreshes the per-type
 * bucketing of atype (read back once); otherwise the previous one is reused.
 * Device analog of DeepPot::compute_canonical_graph_gpu / compute_edges_gpu
 * (deepmd-op/overlays/api_cc/include/DeepPot.h:395-445), which also write in
 * place into caller-owned device buffers (DeepPotPTExpt.cc:2843-2847).
 */
int dp_compute_device(dp_model* model, int natoms, const double* d_coord, const int* d_atype,
                      const double* box, int ago, double* d_energy, double* d_force,
                      double* d_virial, double* d_atom_energy, double* d_atom_virial,
                      void* stream);

/*
 * Asynchronous form of dp_compute_device for an MD loop that keeps its data on
 * the GPU: the evaluation is enqueued on `stream` and the call returns without
 * waiting for it, so consecutive steps (and the caller's own kernels between
 * them) queue back to back with no host round trip. With ago != 0 and the
 * same natoms as the previous call nothing is read back, and nothing is
 * allocated once the buffers have grown to the system's size; ago == 0 reads
 * the types back once, as dp_compute_device does. The outputs are complete
 * when `stream` reaches the point of the call. A capacity error raised by the
 * kernels (more than 512 neighbours within rcut of one atom, more than 1024
 * edges pointing at one atom) is returned by the first later call of this
 * function that sees it, or by dp_sync; the outputs of that evaluation and of
 * those queued after it are then invalid. Any other entry point first waits
 * for the queued evaluations (and returns such an error). Analog of the
 * reference's GPU-resident step, which hands the model outputs to the MD
 * engine's stream through events with no host synchronisation
 * (deepmd-op/overlays/api_cc/include/DeepPot.h:14-18,
 * deepmd-op/overlays/api_cc/src/DeepPotPTExpt.cc:194-222, used at
 * deepmd-op/overlays/lmp/pair_deepmd_kokkos.cpp:555-606).
 */
int dp_compute_device_async(dp_model* model, int natoms, const double* d_coord,
                            const int* d_atype, const double* box, int ago, double* d_energy,
                            double* d_force, double* d_virial, double* d_atom_energy,
                            double* d_atom_virial, void* stream);

/*
 * dp_compute_device (with ago == 0) that allocates nothing: every work
 * buffer of the evaluation is carved from a static scratch array of
 * DP_NOALLOC_SCRATCH_BYTES (128 MiB) that the library holds on each GPU it
 * runs on until the process ends, and no hipMalloc, hipFree or allocating
 * library routine is called (no vendor GEMM either: the plain GEMMs run as
 * this library's own kernels, and the per-type chains on `stream` alone).
 * The caller passes inputs and outputs; the handle's own buffers are left as
 * they were. A system whose work buffers exceed the scratch is rejected
 * with DP_ERR_CAPACITY (the outputs are then unspecified; the handle keeps
 * working). Every handle on one GPU shares that GPU's scratch: the library
 * serialises the calls of several host threads on one GPU (a per-device
 * lock held for the whole call), but work the caller queues on other streams
 * that reads or writes the scratch's contents is not ordered against it.
 * The call is synchronous: it reads the atom types back to the host and
 * returns when the outputs are complete, so it cannot be recorded into a
 * HIP graph; on a stream that is being captured it returns DP_ERR_ARG
 * without touching the stream. No counterpart in the reference: for
 * callers that cannot allocate device memory (serving loops and harnesses
 * that forbid hipMalloc).
 */
#define DP_NOALLOC_SCRATCH_BYTES (128u << 20)
int dp_compute_device_noalloc(dp_model* model, int natoms, const double* d_coord,
                              const int* d_atype, const double* box, double* d_energy,
                              double* d_force, double* d_virial, double* d_atom_energy,
                              double* d_atom_virial, void* stream);

/* With the environment variable DPAMD_GRAPH=1 set when the handle is
 * created, dp_compute_device_async replays the evaluation as a HIP graph: the
 * first call with a given key (natoms, every pointer, the box, the stream)
 * runs eagerly and sizes the buffers, the second captures the evaluation on a
 * stream of the handle's own, and later calls with the same key replay it
 * (a new key captures again; a failed capture turns graphs off for the
 * handle). Stage timing (dp_stage_times) runs eagerly. As the reference's
 * DPA_MODEL_GRAPH replay (deepmd-op/overlays/api_cc/src/DeepPotPTExpt.cc:
 * 122-191), keyed on pointers and sizes. dp_graph_stats reports the captures
 * and replays so far and returns 1 while graphs are in use, 0 otherwise. */
int dp_graph_stats(const dp_model* model, long* captures, long* replays);

/* Waits for every evaluation queued by dp_compute_device_async; returns
 * DP_ERR_CAPACITY (and clears the flag) if any of them overflowed, DP_OK
 * otherwise. Stage times then refer to the last of them. No counterpart in the
 * reference, whose errors surface at the next synchronous call. */
int dp_sync(dp_model* model);

/*
 * DPA4C evaluation of a compact canonical graph, all pointers device memory:
 * d_atype [nall_nodes] int64 model types; edges sorted by destination, with
 * d_destination_row_ptr [nall_nodes + 1] their CSR over destination nodes,
 * d_source [edge_storage] the source node of each edge and d_edge_vec
 * [edge_storage][3] fp32 x_source - x_destination; d_source_row_ptr /
 * d_source_order the CSR of the same edges by source (positions into the edge
 * arrays). Only local destinations (< nloc) carry model edges; slots past them
 * are reserved. Writes d_atom_energy [nloc], d_force [nall_nodes][3] =
 * sum(dst=n) g - sum(src=n) g and d_atom_virial [nall_nodes][9] = -sum(src=n)
 * g (x) d with g = dE/dd, ghost contributions left in ghost slots; work is
 * ordered on `stream` and complete when the call returns. Replaces
 * DeepPot::compute_canonical_graph_gpu (deepmd-op/overlays/api_cc/include/
 * DeepPot.h:430-442, DeepPotPTExpt.cc:2747-2908, same argument meanings and
 * the same dimension checks); forces follow
 * deepmd-op/overlays/op/pt/edge_force_virial.cu:1-14. DP_ERR_MODEL for an
 * se_e2_a model, DP_ERR_ARG for a type or source outside the model / graph.
 */
int dp_compute_canonical_graph_device(dp_model* model, double* d_atom_energy, double* d_force,
                                      double* d_atom_virial, const int64_t* d_atype,
                                      const uint32_t* d_source, const float* d_edge_vec,
                                      const int64_t* d_destination_row_ptr,
                                      const int64_t* d_source_row_ptr,
                                      const uint32_t* d_source_order, int nloc, int nall_nodes,
                                      int64_t edge_storage, void* stream);

/*
 * Device-resident evaluation of a caller-built edge graph, all arrays device
 * memory, work ordered on `stream` and complete on return. Replaces
 * DeepPot::compute_edges_gpu (deepmd-op/overlays/api_cc/include/DeepPot.h:
 * 395-429; backend DeepPotPTExpt.cc:2402-2740; called by the Kokkos pair,
 * lmp/pair_deepmd_kokkos.cpp:586-597), with its argument meanings:
 * d_edge_index int32 [2][nedge], row 0 the neighbour (source) node and row 1
 * the centre (destination, < nloc); d_edge_vec [nedge][3] = r_neighbour -
 * r_centre (fp64, or fp32 in the _f32 form); d_atype int32 [nall_nodes]
 * model types; nall_nodes = nloc folds every edge onto local source nodes
 * (single domain), nall_nodes > nloc keeps ghost nodes whose forces the
 * caller's reverse communication folds. Edges beyond rcut (a skin) are
 * filtered; d_coord is accepted for the signature and not read (the edge
 * vectors carry the geometry). Outputs: d_atom_energy [nloc], d_force
 * [nall_nodes][3], d_atom_virial [nall_nodes][9] (charged to the source
 * node). Works for both model families; an edge naming a node outside the
 * graph gives DP_ERR_ARG. For se_e2_a the local types are read back each call
 * (nloc ints) to group centres by type.
 */
int dp_compute_edges_device(dp_model* model, double* d_atom_energy, double* d_force,
                            double* d_atom_virial, const double* d_coord, const int* d_atype,
                            const int* d_edge_index, const double* d_edge_vec, int nloc,
                            int nedge, int nall_nodes, void* stream);
int dp_compute_edges_device_f32(dp_model* model, double* d_atom_energy, double* d_force,
                                double* d_atom_virial, const double* d_coord, const int* d_atype,
                                const int* d_edge_index, const float* d_edge_vec, int nloc,
                                int nedge, int nall_nodes, void* stream);

/* Copy a stage buffer of the last evaluation (DP_STAGE_*) to host memory.
 * Returns the buffer's size in bytes (copies min(size, capacity) bytes);
 * negative on error. No counterpart in the reference: parity tests use it to
 * compare each pipeline stage with the CPU oracle (the reference's own
 * analogue is its DPA_DUMP_FRAME hook, graph_compress.cu:1354-1378). */
long dp_debug_copy(dp_model* model, int stage, void* dst, size_t capacity);

/* keep != 0: the evaluations that follow also store their per-slot edge
 * gradients, so dp_debug_copy can return DP_STAGE_EDGE_GRAD (the se_e2_a
 * force stage otherwise scatters them into the forces without writing them);
 * keep == 0 (the default) switches that off again. No counterpart in the
 * reference: a parity-test hook, like dp_debug_copy. */
int dp_debug_keep(dp_model* model, int keep);

/* se_e2_a in fp64 forms dE/dT from the fitting's input gradient with a fused
 * kernel (dE/dD never stored) when every atom type has at least `rows` atoms
 * (default 12288; 0: always), and otherwise as the plain product
 * dE/dD = dZ0 W0^T followed by a separate dE/dT pass, which is faster for
 * few atoms per type. Both forms give the same results to rounding. No
 * counterpart in the reference: a parity-test hook, so that both forms are
 * checked at the sizes the oracle evaluates. */
int dp_debug_fused_rows(dp_model* model, int rows);

/* Per-stage GPU time in milliseconds (hipEvent pairs) of the last synchronous
 * evaluation, or the mean over the evaluations queued by
 * dp_compute_device_async up to the last dp_sync, filled into times[0..n-1] in
 * pipeline order; returns the number of stages and writes their names into
 * names (NUL separated) when non-NULL. `enable` switches the timers on or off
 * for the evaluations that follow. The reference's analogue is its DPA_KTIME
 * stage timer (graph_compress.cu:1394-1427). */
int dp_stage_times(dp_model* model, int enable, double* times, int n, char* names, size_t names_len);

/* Peak device bytes allocated by this handle so far (memory high-water mark). */
size_t dp_device_bytes(const dp_model* model);

#ifdef __cplusplus
}
#endif

#endif /* DP_AMD_H */
