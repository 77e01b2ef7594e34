// Padded layout of one embedding net (s -> L1 -> L2 -> L3) as the MFMA
// kernels read it from LDS. Shared by the host packer and the kernels so the
// two cannot drift.
//
//   w1[K2P] b1[K2P] | W2[K2P][W2LD] b2[L2P] | W3[K3P][W3LD] b3[L3P]
//
// K2P = 4*ceil(L1/4) (k-steps of layer 2), L2P = 16*ceil(L2/16) (16-row
// output tiles of layer 2), K3P = 4*ceil(L2/4), L3P = 16*ceil(L3/16). Row
// strides W2LD / W3LD are L2P / L3P, plus 4 floats in the fp32 layout: there
// the four lane groups of an MFMA B-operand read take rows 4 apart, which
// with a stride that is a multiple of the 64 LDS banks all land on the same
// 16 banks; +4 floats moves each group onto its own 16.
// Padding entries are zero, so padded features evaluate to tanh(0) = 0.
// The fp32 kernels (F32) take the k-steps of layer 3 in the order the fp32
// MFMA leaves layer 2 in registers (features 16t + 4g + r), which reaches
// past K3P when L2 is not a multiple of 16, so their W3 has L2P rows
// (K3P = L2P); the element type of the packed array is then float.
#pragma once

namespace dpamd {

struct EmbLayout {
  int L1, L2, L3;
  int NQ2, K2P, NT2, L2P, NQ3, K3P, NU3, L3P, W2LD, W3LD;
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
  e.W2LD = e.L2P + (f32 ? 4 : 0);
  e.W3LD = e.L3P + (f32 ? 4 : 0);
  e.off_w1 = 0;
  e.off_b1 = e.K2P;
  e.off_w2 = 2 * e.K2P;
  e.off_b2 = e.off_w2 + e.K2P * e.W2LD;
  e.off_w3 = e.off_b2 + e.L2P;
  e.off_b3 = e.off_w3 + e.K3P * e.W3LD;
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
  static constexpr int W2LD = L2P + (F32 ? 4 : 0);
  static constexpr int W3LD = L3P + (F32 ? 4 : 0);
  static constexpr int OFF_W1 = 0;
  static constexpr int OFF_B1 = K2P;
  static constexpr int OFF_W2 = 2 * K2P;
  static constexpr int OFF_B2 = OFF_W2 + K2P * W2LD;
  static constexpr int OFF_W3 = OFF_B2 + L2P;
  static constexpr int OFF_B3 = OFF_W3 + K3P * W3LD;
  static constexpr int SIZE = OFF_B3 + L3P;
  // residual kinds: 0 none, 1 identity, 2 concat [x, x]
  static constexpr int RES2 = (L2 == L1) ? 1 : (L2 == 2 * L1 ? 2 : 0);
  static constexpr int RES3 = (L3 == L2) ? 1 : (L3 == 2 * L2 ? 2 : 0);
  static constexpr bool X1_ALIGNED = (L1 % 16) == 0;  // layer-2 residual is register-local
};

}  // namespace dpamd
