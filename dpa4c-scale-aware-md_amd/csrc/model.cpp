// Model file parsing, validation and packing into the kernels' layouts.
// The metadata read here mirrors what the reference's model API reads from a
// model (rcut, type_map/ntypes, sel; deepmd-op/overlays/api_cc/src/DeepPotPTExpt.cc:368-478).
#include "model.h"

#include <cmath>
#include <cstring>

namespace dpamd {

namespace {

struct Reader {
  const unsigned char* p;
  size_t n, off = 0;
  bool ok = true;
  template <class T>
  T get() {
    T v{};
    if (off + sizeof(T) > n) {
      ok = false;
      return v;
    }
    std::memcpy(&v, p + off, sizeof(T));
    off += sizeof(T);
    return v;
  }
  void floats(std::vector<float>& out, size_t count) {
    out.resize(count);
    if (off + count * 4 > n) {
      ok = false;
      return;
    }
    std::memcpy(out.data(), p + off, count * 4);
    off += count * 4;
  }
  void doubles(std::vector<double>& out, size_t count) {
    out.resize(count);
    if (off + count * 8 > n) {
      ok = false;
      return;
    }
    std::memcpy(out.data(), p + off, count * 8);
    off += count * 8;
  }
};

}  // namespace

std::string parse_model(const unsigned char* buf, size_t len, ModelHost& m) {
  if (len < 8 || std::memcmp(buf, "DPAMDSEA", 8) != 0) return "not a DPAMDSEA se_e2_a model file";
  Reader r{buf, len, 8};
  const uint32_t ver = r.get<uint32_t>();
  if (ver != 1) return "unsupported model file version " + std::to_string(ver);
  const uint32_t nt = r.get<uint32_t>();
  if (nt < 1 || nt > (uint32_t)kMaxTypes) return "ntypes must be in [1, 8]";
  m.ntypes = (int)nt;
  m.nnei = 0;
  for (int t = 0; t < m.ntypes; ++t) {
    m.sel[t] = (int)r.get<uint32_t>();
    m.sec[t] = m.nnei;
    m.nnei += m.sel[t];
  }
  m.sec[m.ntypes] = m.nnei;
  m.rcut = r.get<double>();
  m.rcut_smth = r.get<double>();
  for (int k = 0; k < 3; ++k) m.emb[k] = (int)r.get<uint32_t>();
  m.axis = (int)r.get<uint32_t>();
  for (int k = 0; k < 3; ++k) m.fit[k] = (int)r.get<uint32_t>();
  // precision the model was written for: 0 fp64 (also every file written
  // while this word was reserved), 1 mixed
  const uint32_t prec = r.get<uint32_t>();
  if (prec > 1) return "model precision field must be 0 (fp64) or 1 (mixed)";
  m.precision = (int)prec;
  m.type_map.clear();
  for (int t = 0; t < m.ntypes; ++t) {
    char name[17] = {0};
    for (int q = 0; q < 16; ++q) name[q] = (char)r.get<uint8_t>();
    m.type_map.emplace_back(name);
  }
  if (!r.ok) return "model file truncated in header";
  if (!(m.rcut > 0) || !(m.rcut_smth >= 0) || !(m.rcut_smth < m.rcut))
    return "need 0 <= rcut_smth < rcut";
  if (!(m.rcut < 16.0)) return "rcut must be below 16 A";
  for (int t = 0; t < m.ntypes; ++t)
    if (m.sel[t] <= 0) return "sel entries must be positive";
  const int L1 = m.emb[0], L2 = m.emb[1], L3 = m.emb[2];
  if (!emb_supported(L1, L2, L3))
    return "embedding widths " + std::to_string(L1) + "-" + std::to_string(L2) + "-" +
           std::to_string(L3) + " not compiled (supported: 25-50-100, 32-64-128)";
  if (m.axis < 1 || m.axis > L3 || m.axis > 64 || (m.axis & (m.axis - 1)) != 0)
    return "axis must be a power of two <= min(64, L3)";
  const int Dn = L3 * m.axis;
  for (int k = 0; k < 3; ++k)
    if (m.fit[k] <= 0 || m.fit[k] % 16 != 0) return "fitting widths must be multiples of 16";
  if (Dn % 16 != 0) return "descriptor width L3*axis must be a multiple of 16";
  if (m.fit[0] == Dn) return "a residual first fitting layer is not supported";
  m.emb_block = (long)L1 + L1 + (long)L1 * L2 + L2 + (long)L2 * L3 + L3;
  const int ins[3] = {Dn, m.fit[0], m.fit[1]};
  m.fit_block = 0;
  for (int k = 0; k < 3; ++k)
    m.fit_block += (long)ins[k] * m.fit[k] + m.fit[k] + (m.fit[k] == ins[k] ? m.fit[k] : 0);
  m.fit_block += m.fit[2] + 1;
  const size_t nt2 = (size_t)m.ntypes * m.ntypes;
  r.doubles(m.davg, nt2 * 4);
  r.doubles(m.dstd, nt2 * 4);
  r.doubles(m.emb_params, nt2 * m.emb_block);
  r.doubles(m.fit_params, (size_t)m.ntypes * m.fit_block);
  r.doubles(m.bias, (size_t)m.ntypes);
  if (!r.ok) return "model file truncated in parameters";
  if (r.off != len) return "trailing bytes after model parameters";
  for (double s : m.dstd)
    if (!(s != 0.0)) return "dstd entries must be non-zero";
  return "";
}

FitOffsets fit_offsets(const ModelHost& m) {
  FitOffsets o{};
  const int ins[3] = {m.emb[2] * m.axis, m.fit[0], m.fit[1]};
  long p = 0;
  for (int k = 0; k < 3; ++k) {
    o.W[k] = p;
    p += (long)ins[k] * m.fit[k];
    o.b[k] = p;
    p += m.fit[k];
    if (m.fit[k] == ins[k]) {
      o.idt[k] = p;
      p += m.fit[k];
    } else {
      o.idt[k] = -1;
    }
  }
  o.Wo = p;
  o.bo = p + m.fit[2];
  return o;
}

namespace {

// Host fp64 evaluation of one embedding net at s (padded-slot constant).
void embed_host(const ModelHost& m, const double* P, double s, std::vector<double>& out) {
  const int L1 = m.emb[0], L2 = m.emb[1], L3 = m.emb[2];
  const double* W1 = P;
  const double* b1 = W1 + L1;
  const double* W2 = b1 + L1;
  const double* b2 = W2 + (long)L1 * L2;
  const double* W3 = b2 + L2;
  const double* b3 = W3 + (long)L2 * L3;
  auto layer = [](const std::vector<double>& x, const double* W, const double* b, int out_n) {
    const int in = (int)x.size();
    std::vector<double> y(out_n);
    for (int f = 0; f < out_n; ++f) {
      double z = 0.0;
      for (int k = 0; k < in; ++k) z += x[k] * W[(long)k * out_n + f];
      const double t = std::tanh(z + b[f]);
      double res = 0.0;
      if (out_n == in) res = x[f];
      else if (out_n == 2 * in) res = x[f % in];
      y[f] = res + t;
    }
    return y;
  };
  std::vector<double> x{s};
  x = layer(x, W1, b1, L1);
  x = layer(x, W2, b2, L2);
  out = layer(x, W3, b3, L3);
}

}  // namespace

void pack_embedding(const ModelHost& m, const EmbLayout& e, std::vector<double>& emb,
                    std::vector<double>& envp, std::vector<double>& tpad) {
  const int nt = m.ntypes, np = nt * nt;
  const int L1 = m.emb[0], L2 = m.emb[1], L3 = m.emb[2];
  emb.assign((size_t)np * e.stride, 0.0);
  envp.assign((size_t)np * 8, 0.0);
  tpad.assign((size_t)np * 4 * L3, 0.0);
  for (int p = 0; p < np; ++p) {
    const double* P = m.emb_params.data() + (size_t)p * m.emb_block;
    const double* W1 = P;
    const double* b1 = W1 + L1;
    const double* W2 = b1 + L1;
    const double* b2 = W2 + (long)L1 * L2;
    const double* W3 = b2 + L2;
    const double* b3 = W3 + (long)L2 * L3;
    double* Q = emb.data() + (size_t)p * e.stride;
    for (int f = 0; f < L1; ++f) {
      Q[e.off_w1 + f] = W1[f];
      Q[e.off_b1 + f] = b1[f];
    }
    if (!e.f32) {  // the fp32 layout's W2 / W3 are bf16 pieces (pack_embedding_bf16)
      for (int k = 0; k < L1; ++k)
        for (int n = 0; n < L2; ++n) Q[e.off_w2 + k * e.W2LD + n] = W2[(long)k * L2 + n];
      for (int k = 0; k < L2; ++k)
        for (int n = 0; n < L3; ++n) Q[e.off_w3 + k * e.W3LD + n] = W3[(long)k * L3 + n];
    }
    for (int n = 0; n < L2; ++n) Q[e.off_b2 + n] = b2[n];
    for (int n = 0; n < L3; ++n) Q[e.off_b3 + n] = b3[n];
    for (int q = 0; q < 4; ++q) {
      envp[(size_t)p * 8 + q] = m.davg[(size_t)p * 4 + q];
      envp[(size_t)p * 8 + 4 + q] = m.dstd[(size_t)p * 4 + q];
    }
    double Rpad[4];
    for (int q = 0; q < 4; ++q) Rpad[q] = (0.0 - m.davg[(size_t)p * 4 + q]) / m.dstd[(size_t)p * 4 + q];
    std::vector<double> G;
    embed_host(m, P, Rpad[0], G);
    for (int q = 0; q < 4; ++q)
      for (int f = 0; f < L3; ++f) tpad[((size_t)p * 4 + q) * L3 + f] = Rpad[q] * G[f];
  }
}

namespace {
uint16_t bf16_rne(float x) {  // round to nearest even (finite x)
  uint32_t u;
  std::memcpy(&u, &x, 4);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
float bf16_value(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}
// w = hi + mid + lo exactly (each rounding leaves at most 16, then 8 bits)
void split3(float w, uint16_t out[3]) {
  out[0] = bf16_rne(w);
  const float r1 = w - bf16_value(out[0]);
  out[1] = bf16_rne(r1);
  const float r2 = r1 - bf16_value(out[1]);
  out[2] = bf16_rne(r2);
}
// one net's pre-split weights W [K][N] (row-major, fp64) into a bf16 region
// [tiles][chunks][3][64][8] with the given k order; entries past K or N are 0
void pack_pieces(const double* W, int K, int N, int tiles, int chunks, bool row_order,
                 uint16_t* dst) {
  for (int t = 0; t < tiles; ++t)
    for (int h = 0; h < chunks; ++h)
      for (int lane = 0; lane < 64; ++lane) {
        const int g = lane >> 4, c = lane & 15, n = 16 * t + c;
        for (int e = 0; e < 8; ++e) {
          const int k = bf16_kperm(h, g, e, row_order);
          const float w = (k < K && n < N) ? (float)W[(long)k * N + n] : 0.0f;
          uint16_t pc[3];
          split3(w, pc);
          for (int q = 0; q < 3; ++q)
            dst[((((long)t * chunks + h) * 3 + q) * 64 + lane) * 8 + e] = pc[q];
        }
      }
}
}  // namespace

void pack_gemm_bf16(const double* W, int rows, int cols, bool trans, std::vector<uint16_t>& out,
                    bool tile_major) {
  const int K = trans ? cols : rows, N = trans ? rows : cols;
  const int chunks = (K + 31) / 32, tiles = N / 16;
  const size_t base = out.size();
  out.resize(base + (size_t)chunks * tiles * 3 * 64 * 8, 0);
  uint16_t* dst = out.data() + base;
  for (int h = 0; h < chunks; ++h)
    for (int t = 0; t < tiles; ++t)
      for (int lane = 0; lane < 64; ++lane) {
        const int g = lane >> 4, c = lane & 15, n = 16 * t + c;
        for (int e = 0; e < 8; ++e) {
          const int k = 32 * h + 8 * g + e;
          const double v = k < K ? (trans ? W[(long)n * cols + k] : W[(long)k * cols + n]) : 0.0;
          uint16_t pc[3];
          split3((float)v, pc);
          for (int q = 0; q < 3; ++q)
            dst[(((tile_major ? (size_t)t * chunks + h : (size_t)h * tiles + t) * 3 + q) * 64 +
                 lane) * 8 + e] = pc[q];
        }
      }
}

void pack_embedding_bf16(const ModelHost& m, const EmbLayout& e, std::vector<float>& emb32) {
  const int np = m.ntypes * m.ntypes;
  const int L1 = m.emb[0], L2 = m.emb[1], L3 = m.emb[2];
  for (int p = 0; p < np; ++p) {
    const double* P = m.emb_params.data() + (size_t)p * m.emb_block;
    const double* W2 = P + 2 * L1;
    const double* W3 = W2 + (long)L1 * L2 + L2;
    float* Q = emb32.data() + (size_t)p * e.stride;
    pack_pieces(W2, L1, L2, e.NT2, e.KC2, L1 % 16 == 0,
                reinterpret_cast<uint16_t*>(Q + e.off_w2));
    pack_pieces(W3, L2, L3, e.NU3, e.KC3, true, reinterpret_cast<uint16_t*>(Q + e.off_w3));
  }
}

std::string parse_c4_model(const unsigned char* buf, size_t len, ModelHost& m, C4Host& c) {
  if (len < 8 || std::memcmp(buf, "DPAMDC4N", 8) != 0) return "not a DPAMDC4N DPA4C model file";
  Reader r{buf, len, 8};
  const uint32_t ver = r.get<uint32_t>();
  if (ver != 1) return "unsupported model file version " + std::to_string(ver);
  const uint32_t nt = r.get<uint32_t>();
  if (nt < 1 || nt > (uint32_t)kMaxTypes) return "ntypes must be in [1, 8]";
  m = ModelHost{};
  m.ntypes = (int)nt;
  for (int t = 0; t < m.ntypes; ++t) {
    m.sel[t] = (int)r.get<uint32_t>();
    m.sec[t] = m.nnei;
    m.nnei += m.sel[t];
  }
  m.sec[m.ntypes] = m.nnei;
  m.rcut = r.get<double>();
  c.eps = r.get<double>();
  c.floor = r.get<double>();
  c.stride = r.get<double>();
  c.n_int = (int)r.get<uint32_t>();
  const uint32_t channels = r.get<uint32_t>(), lmax = r.get<uint32_t>();
  const uint32_t nl = r.get<uint32_t>();
  if (!r.ok) return "model file truncated in header";
  if (channels != 8 || lmax != 2)
    return "only the DPA4C Nano profile (8 channels, lmax 2) is compiled";
  if (nl != 1) return "only a fitting net with one hidden layer (DPA4C Nano) is compiled";
  c.H = (int)r.get<uint32_t>();
  c.act = (int)r.get<uint32_t>();
  c.resnet = (int)r.get<uint32_t>();
  m.type_map.clear();
  for (int t = 0; t < m.ntypes; ++t) {
    char name[17] = {0};
    for (int q = 0; q < 16; ++q) name[q] = (char)r.get<uint8_t>();
    m.type_map.emplace_back(name);
  }
  if (!r.ok) return "model file truncated in header";
  if (!(m.rcut > 0) || !(m.rcut < 16.0)) return "rcut must be in (0, 16) A";
  if (!(c.eps >= 0) || !(c.floor >= 0) || !(c.stride > 0)) return "need eps, floor >= 0, stride > 0";
  if (c.n_int < 1 || c.n_int > (1 << 20)) return "bad table interval count";
  if ((c.n_int - 1) * c.stride < m.rcut - 1e-9) return "radial table does not cover rcut";
  if (c.H < 1 || c.H > 1024) return "hidden width must be in [1, 1024]";
  if (c.act != 0 && c.act != 1) return "activation must be 0 (tanh) or 1 (silu)";
  for (int t = 0; t < m.ntypes; ++t)
    if (m.sel[t] <= 0) return "sel entries must be positive";
  if (m.nnei > 4096) return "sum(sel) must be at most 4096";
  const int ntt = m.ntypes * m.ntypes;
  r.floats(c.table, (size_t)c.n_int * 48);
  r.floats(c.film, (size_t)ntt * 16);
  r.floats(c.ro, 16 + 16 + 16 + 8);
  r.floats(c.temb, (size_t)m.ntypes * 8);
  r.floats(c.mean, kC4Out);
  r.floats(c.istd, kC4Out);
  std::vector<float> w0;
  r.floats(w0, (size_t)kC4Out * c.H);
  r.floats(c.b0, (size_t)c.H);
  r.floats(c.wh, (size_t)c.H);
  std::vector<float> bh;
  r.floats(bh, 1);
  r.doubles(c.bias, (size_t)m.ntypes);
  if (!r.ok) return "model file truncated in parameters";
  if (r.off != len) return "trailing bytes in model file";
  c.bh = bh[0];
  // first layer transposed: row h holds W0[:, h], padded to kC4W0Ld
  c.w0t.assign((size_t)c.H * kC4W0Ld, 0.f);
  for (int q = 0; q < kC4Out; ++q)
    for (int h = 0; h < c.H; ++h) c.w0t[(size_t)h * kC4W0Ld + q] = w0[(size_t)q * c.H + h];
  return "";
}

}  // namespace dpamd
