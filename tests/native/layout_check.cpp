// The padded-net layout used by the host packer (make_emb_layout) must equal
// the compile-time layout the kernels index with (EmbShape), for both the
// fp64 and the fp32 (mixed-precision) kernels and every supported width set.
// Also checks the fp32 property the kernels rely on: W3 has L2P rows, so every
// layer-3 k-step feature 16(q/4) + 4g + q%4 (q < 4 NT2) is a valid row.
#include <cstdio>

#include "../../dpa4c-scale-aware-md_amd/csrc/emb_shape.h"

template <class S>
static int check(bool f32) {
  const dpamd::EmbLayout e = dpamd::make_emb_layout(S::L1, S::L2, S::L3, f32);
  int bad = 0;
  auto eq = [&](const char* name, int a, int b) {
    if (a != b) {
      std::printf("%d-%d-%d f32=%d: %s host %d kernel %d\n", S::L1, S::L2, S::L3, (int)f32, name, a, b);
      ++bad;
    }
  };
  eq("NQ2", e.NQ2, S::NQ2);
  eq("K2P", e.K2P, S::K2P);
  eq("NT2", e.NT2, S::NT2);
  eq("L2P", e.L2P, S::L2P);
  eq("NQ3", e.NQ3, S::NQ3);
  eq("K3P", e.K3P, S::K3P);
  eq("NU3", e.NU3, S::NU3);
  eq("L3P", e.L3P, S::L3P);
  eq("off_w1", e.off_w1, S::OFF_W1);
  eq("off_b1", e.off_b1, S::OFF_B1);
  eq("off_w2", e.off_w2, S::OFF_W2);
  eq("off_b2", e.off_b2, S::OFF_B2);
  eq("off_w3", e.off_w3, S::OFF_W3);
  eq("off_b3", e.off_b3, S::OFF_B3);
  eq("size", e.size, S::SIZE);
  if (e.stride < e.size || e.stride % 32 != 0) {
    std::printf("bad stride %d\n", e.stride);
    ++bad;
  }
  if (f32) {
    for (int q = 0; q < 4 * S::NT2; ++q)
      for (int g = 0; g < 4; ++g) {
        const int f = 16 * (q >> 2) + 4 * g + (q & 3);
        if (f >= S::K3P) {
          std::printf("fp32 layer-3 row %d beyond K3P %d\n", f, S::K3P);
          ++bad;
        }
      }
    eq("KC2", e.KC2, S::KC2);
    eq("KC3", e.KC3, S::KC3);
    // the bf16 weight regions are read 16 bytes per lane
    if (e.off_w2 % 4 || e.off_w3 % 4) {
      std::printf("bf16 regions not 16-byte aligned: %d %d\n", e.off_w2, e.off_w3);
      ++bad;
    }
    // each k chunk's (g, e) -> k map is a bijection onto its 32 k values, and
    // the layer-3 one is the order of layer 2's result rows (tile 2h + e/4,
    // row 4g + e%4), which the kernels split as the A / B operand
    for (int row_order = 0; row_order < 2; ++row_order)
      for (int h = 0; h < 2; ++h) {
        int seen[32] = {0};
        for (int g = 0; g < 4; ++g)
          for (int ee = 0; ee < 8; ++ee) {
            const int k = dpamd::bf16_kperm(h, g, ee, row_order != 0);
            if (k < 32 * h || k >= 32 * h + 32) {
              std::printf("kperm(%d,%d,%d) = %d outside its chunk\n", h, g, ee, k);
              ++bad;
            } else {
              ++seen[k - 32 * h];
            }
            if (row_order && k != 16 * (2 * h + (ee >> 2)) + 4 * g + (ee & 3)) {
              std::printf("layer-3 kperm(%d,%d,%d) = %d not a layer-2 row\n", h, g, ee, k);
              ++bad;
            }
          }
        for (int k = 0; k < 32; ++k)
          if (seen[k] != 1) {
            std::printf("kperm chunk %d covers k %d %d times\n", h, k, seen[k]);
            ++bad;
          }
      }
  }
  return bad;
}

int main() {
  int bad = 0;
  bad += check<dpamd::EmbShape<25, 50, 100>>(false);
  bad += check<dpamd::EmbShape<32, 64, 128>>(false);
  bad += check<dpamd::EmbShape<25, 50, 100, true>>(true);
  bad += check<dpamd::EmbShape<32, 64, 128, true>>(true);
  std::printf(bad ? "layout mismatch\n" : "layouts agree\n");
  return bad ? 1 : 0;
}
