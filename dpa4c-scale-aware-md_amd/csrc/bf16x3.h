// fp32 products on gfx950's bf16 matrix cores at fp32 accuracy: each fp32
// operand is split exactly into three bf16 pieces and the six cross products
// that reach fp32 precision are accumulated in fp32. Shared by the
// mixed-precision embedding and fitting kernels.
#pragma once

#include "common.h"

namespace dpamd {

// bf16 operands of v_mfma_f32_16x16x32_bf16: lane 16g + c holds A[c][8g + e]
// and B[8g + e][c], e = 0..7; D register r holds D[4g + r][c], as in the fp32
// 16x16x4 form (checked on MI355X).
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4 mfma_bf16(bf8 a, bf8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// An fp32 operand as three bf16 pieces, x = h + m + l exactly: h = bf16(x)
// leaves a remainder of at most 16 significant bits, m = bf16 of that one of
// at most 8, which l holds exactly (round to nearest even throughout).
struct Split3 {
  bf8 h, m, l;
};

__device__ __forceinline__ Split3 split3(const float* v) {
  Split3 s;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = (__bf16)v[e];
    const float r1 = v[e] - (float)h;
    const __bf16 m = (__bf16)r1;
    s.h[e] = h;
    s.m[e] = m;
    s.l[e] = (__bf16)(r1 - (float)m);
  }
  return s;
}

// (a_h + a_m + a_l)(b_h + b_m + b_l) to fp32 accuracy: the six products down
// to 2^-18 of the leading one (the three dropped are below 2^-26), smallest
// first. Six bf16 MFMAs of K 32 take about half the time of the eight fp32
// 16x16x4 MFMAs they replace (measured on MI355X: 9.4 vs 14.4 ns each).
__device__ __forceinline__ f4 mfma3(const Split3& a, const Split3& b, f4 c) {
  c = mfma_bf16(a.m, b.m, c);
  c = mfma_bf16(a.l, b.h, c);
  c = mfma_bf16(a.h, b.l, c);
  c = mfma_bf16(a.m, b.h, c);
  c = mfma_bf16(a.h, b.m, c);
  return mfma_bf16(a.h, b.h, c);
}

// The transposed product of mfma3(b, a): the same six piece products
// accumulated in the same order, so D = mfma3_t(a, b, .) is the transpose of
// mfma3(b, a, .) term for term (each bf16 x bf16 product is exact in fp32).
__device__ __forceinline__ f4 mfma3_t(const Split3& a, const Split3& b, f4 c) {
  c = mfma_bf16(a.m, b.m, c);
  c = mfma_bf16(a.h, b.l, c);
  c = mfma_bf16(a.l, b.h, c);
  c = mfma_bf16(a.h, b.m, c);
  c = mfma_bf16(a.m, b.h, c);
  return mfma_bf16(a.h, b.h, c);
}

}  // namespace dpamd
