// Padded layout of one embedding net (s -> L1 -> L2 -> L3) as the MFMA
// kernels read it from LDS. Shared by the host packer and the kernels so the
// two cannot drift.
//
//   w1[K2P] b1[K2P] | W2[K2P][W2LD] b2[L2P] | W3[K3P][W3LD] b3[L3P]
//
// K2P = 4*ceil(L1/4) (k-steps of layer 2), L2P = 16*ceil(L2/16) (16-row
// output tiles of layer 2), K3P = 4*ceil(L2/4), L3P = 16*ceil(L3/16). Row
// strides W2LD / W3LD are L2P / L3P.
// Padding entries are zero, so padded features evaluate to tanh(0) = 0.
//
// fp32 layout (F32, mixed precision; element type float). Layers 2 and 3 run
// on v_mfma_f32_16x16x32_bf16 with every fp32 operand split exactly into
// three bf16 pieces (hi + mid + lo), so their weights are stored pre-split as
// the operands the 64 lanes read, 16 bytes per lane:
//
//   w1[K2P] b1[K2P] | W2B[NT2][KC2][3][64 lanes][8] b2[L2P] |
//   W3B[NU3][KC3][3][64 lanes][8] b3[L3P]                      (8 = bf16 x 8)
//
// Lane 16g + c of (output tile t, 32-wide k chunk h, piece p) holds piece p of
// W[k][16t + c] for k = kperm(h, g, e), e = 0..7: the order in which the
// activations sit in the lane's registers (layer-2 input: the layer-1 features
// the lane computes; layer-3 input: layer 2's MFMA result rows
// 16(e/4) + 4g + e%4 of tiles 2h and 2h + 1). One W3B serves both the
// forward (B operand) and the backward tangent (A operand): each lane holds
// row / column c of its tile and k slice g in both roles. K3P = L2P here.
#pragma once

namespace dpamd {

// k index of element e (0..7) of lane group g in 32-wide k chunk h of the
// bf16 operands: layer-3 input (layer-2 result rows), and layer-2 input when
// L1 is a multiple of 16; otherwise layer 1 is computed as features 4q + g.
inline constexpr int bf16_kperm(int h, int g, int e, bool row_order) {
  return row_order ? 32 * h + 16 * (e >> 2) + 4 * g + (e & 3) : 32 * h + 4 * e + g;
}

struct EmbLayout {
  int L1, L2, L3;
  int NQ2, K2P, NT2, L2P, NQ3, K3P, NU3, L3P, W2LD, W3LD;
  int KC2, KC3;  // 32-wide k chunks of layers 2 and 3 (fp32 layout)
  bool f32;
  int off_w1, off_b1, off_w2, off_b2, off_w3, off_b3, size, stride;
};

inline EmbLayout make_emb_layout(int L1, int L2, int L3, bool f32 = false) {
  EmbLayout e;
  e.L1 = L1;
  e.L2 = L2;
  e.L3 = L3;
  e.NQ2 = (L1 + 3) / 4;
  e.K2P = 4 * e.NQ2;
  e.NT2 = (L2 + 15) / 16;
  e.L2P = 16 * e.NT2;
  e.NQ3 = (L2 + 3) / 4;
  e.K3P = f32 ? 16 * ((L2 + 15) / 16) : 4 * e.NQ3;
  e.NU3 = (L3 + 15) / 16;
  e.L3P = 16 * e.NU3;
  e.W2LD = e.L2P;
  e.W3LD = e.L3P;
  e.KC2 = (e.K2P + 31) / 32;
  e.KC3 = (e.L2P + 31) / 32;
  e.f32 = f32;
  e.off_w1 = 0;
  e.off_b1 = e.K2P;
  e.off_w2 = 2 * e.K2P;
  e.off_b2 = e.off_w2 + (f32 ? e.NT2 * e.KC2 * 3 * 256 : e.K2P * e.W2LD);
  e.off_w3 = e.off_b2 + e.L2P;
  e.off_b3 = e.off_w3 + (f32 ? e.NU3 * e.KC3 * 3 * 256 : e.K3P * e.W3LD);
  e.size = e.off_b3 + e.L3P;
  e.stride = (e.size + 31) / 32 * 32;
  return e;
}

template <int L1_, int L2_, int L3_, bool F32 = false>
struct EmbShape {
  static constexpr int L1 = L1_, L2 = L2_, L3 = L3_;
  static constexpr int NQ2 = (L1 + 3) / 4;
  static constexpr int K2P = 4 * NQ2;
  static constexpr int NT2 = (L2 + 15) / 16;
  static constexpr int L2P = 16 * NT2;
  static constexpr int NQ3 = (L2 + 3) / 4;
  static constexpr int K3P = F32 ? L2P : 4 * NQ3;
  static constexpr int NU3 = (L3 + 15) / 16;
  static constexpr int L3P = 16 * NU3;
  static constexpr int W2LD = L2P;
  static constexpr int W3LD = L3P;
  static constexpr int KC2 = (K2P + 31) / 32;
  static constexpr int KC3 = (L2P + 31) / 32;
  static constexpr int OFF_W1 = 0;
  static constexpr int OFF_B1 = K2P;
  static constexpr int OFF_W2 = 2 * K2P;
  static constexpr int OFF_B2 = OFF_W2 + (F32 ? NT2 * KC2 * 3 * 256 : K2P * W2LD);
  static constexpr int OFF_W3 = OFF_B2 + L2P;
  static constexpr int OFF_B3 = OFF_W3 + (F32 ? NU3 * KC3 * 3 * 256 : K3P * W3LD);
  static constexpr int SIZE = OFF_B3 + L3P;
  // residual kinds: 0 none, 1 identity, 2 concat [x, x]
  static constexpr int RES2 = (L2 == L1) ? 1 : (L2 == 2 * L1 ? 2 : 0);
  static constexpr int RES3 = (L3 == L2) ? 1 : (L3 == 2 * L2 ? 2 : 0);
  static constexpr bool X1_ALIGNED = (L1 % 16) == 0;  // layer-2 residual is register-local
};

}  // namespace dpamd
