// Host representation of an se_e2_a model file (layout documented in the
// package's model.py) and the device-side packing the kernels read.
#pragma once

#include <string>
#include <vector>

#include "kernels.h"

namespace dpamd {

struct ModelHost {
  int ntypes = 0, nnei = 0;
  int sel[kMaxTypes] = {0};
  int sec[kMaxTypes + 1] = {0};
  double rcut = 0, rcut_smth = 0;
  int emb[3] = {0, 0, 0};
  int axis = 0;
  int fit[3] = {0, 0, 0};
  int precision = 0;  // the file's DP_PREC_FP64 / DP_PREC_MIXED
  std::vector<std::string> type_map;
  std::vector<double> davg, dstd;  // [nt][nt][4]
  std::vector<double> emb_params;  // [nt*nt][emb_block]
  std::vector<double> fit_params;  // [nt][fit_block]
  std::vector<double> bias;        // [nt]
  long emb_block = 0, fit_block = 0;
};

// Parse and validate; returns "" on success or a message.
std::string parse_model(const unsigned char* buf, size_t len, ModelHost& m);

// Padded embedding nets [npair][layout.stride], env stats [npair][8],
// padded-slot constants tpad[npair][4][L3] = Rpad[m] * G(s_pad)[f].
void pack_embedding(const ModelHost& m, const EmbLayout& e, std::vector<double>& emb,
                    std::vector<double>& envp, std::vector<double>& tpad);

// fp32 layout only: fills the W2 / W3 regions of the fp32-rounded packed nets
// (pack_embedding's output converted to float) with the weights rounded to
// fp32 and split exactly into three bf16 pieces, in the lane order the
// mixed-precision kernels read (emb_shape.h).
void pack_embedding_bf16(const ModelHost& m, const EmbLayout& e, std::vector<float>& emb32);

// Appends the fragments of the fp32 GEMM operand B [K][N] (B(k, n) = W[k][n],
// or W[n][k] when `trans`; W row-major [rows][cols] fp64, rounded to fp32 and
// split exactly into three bf16 pieces) in the layout the bf16 GEMM reads:
// [ceil(K/32)][N/16][3][64 lanes][8], lane 16g + c of (chunk h, tile n)
// holding B(32h + 8g + e, 16n + c), e = 0..7, zero past K. N % 16 == 0.
// tile_major: [N/16][ceil(K/32)][3][64][8] instead (all chunks of a column
// tile contiguous, the order the fused input-gradient kernel stages them).
void pack_gemm_bf16(const double* W, int rows, int cols, bool trans, std::vector<uint16_t>& out,
                    bool tile_major = false);

// Offsets (in doubles) of each fitting layer inside a type's block.
struct FitOffsets {
  long W[3], b[3], idt[3], Wo, bo;
};
FitOffsets fit_offsets(const ModelHost& m);

// Host representation of a DPA4C-Nano model file (layout documented in the
// package's dpa4c.py). Parsing also fills the neighbour-list fields of a
// ModelHost (ntypes, sel / sec / nnei, rcut, type_map) so the standalone
// pipeline builds the edge list the same way for both model kinds.
struct C4Host {
  double eps = 0, floor = 0, stride = 0;
  int n_int = 0, H = 0, act = 0, resnet = 0;
  std::vector<float> table, film, ro, temb, mean, istd, w0t, b0, wh;
  float bh = 0.f;
  std::vector<double> bias;
};
std::string parse_c4_model(const unsigned char* buf, size_t len, ModelHost& m, C4Host& c);

}  // namespace dpamd
