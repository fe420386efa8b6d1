// Parity test of the C++ operator shim (inferd_amd/csrc/qwen35_ops.h) against the CPU oracle (oracle/liboracle.so),
// written like the reference's seeded inline kernel tests (engine/tools/gemm_dbg.mm:14-55, qa8_dbg.mm:14-66): build a
// layer from a fixed seed, run the operator, compare with the host reference, print one line per case.
//
//   qwen35_ops_test             every GPU case; exit 0 when all pass
//   qwen35_ops_test --bad-bits  gemm() on a 16-bit QLinear: must print its error and exit(1) (no GPU needed)
//   qwen35_ops_test --ckpt DIR  the device loaders (ckpt_dev.h) on a checkpoint written by tests/test_shim.py:
//                               uploads bit-identical to the host loader, and gemm() on the loaded layer
//   qwen35_ops_test --moe-c4 T  encode_moe on T64 expert stacks at BASELINE config 4's geometry (H 2048, 512 experts,
//                               top-10, I 512, a shared expert) for T tokens
//
// Tolerances are BASELINE's: max |err| <= 1e-2 RMS(ref) after the output's own bf16 rounding; routing indices
// bit-exact.
#include <cmath>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "ckpt_dev.h"
#include "qwen35_ops.h"

extern "C" {
void orc_pack_w4(const uint8_t* codes, uint32_t* wq, int N, int K);
void orc_pack_w8(const uint8_t* codes, uint32_t* wq, int N, int K);
void orc_moe_decode(const uint16_t* xn, int T, int H, int I, int k, const int* idx, const float* wt, const float* sg,
                    const uint32_t* gu_wq, const uint16_t* gu_s, const uint16_t* gu_b, const uint32_t* dn_wq,
                    const uint16_t* dn_s, const uint16_t* dn_b, const uint32_t* sh_gu_wq, const uint16_t* sh_gu_s,
                    const uint16_t* sh_gu_b, const uint32_t* sh_dn_wq, const uint16_t* sh_dn_s, const uint16_t* sh_dn_b,
                    uint16_t* out, int assign);
void orc_moe_decode_b(const uint16_t* xn, int T, int H, int I, int k, const int* idx, const float* wt, const float* sg,
                      const uint32_t* gu_wq, const uint16_t* gu_s, const uint16_t* gu_b, const uint32_t* dn_wq,
                      const uint16_t* dn_s, const uint16_t* dn_b, const uint32_t* sh_gu_wq, const uint16_t* sh_gu_s,
                      const uint16_t* sh_gu_b, const uint32_t* sh_dn_wq, const uint16_t* sh_dn_s,
                      const uint16_t* sh_dn_b, int sh_bits, uint16_t* out, int assign);
void orc_qmv_b(const uint16_t* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
               int bits, uint32_t xr, float* Y, int M, int nthreads);
void orc_qmm_b(const uint16_t* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
               int bits, uint32_t xr, float* Y, int M, int nthreads);
void orc_flip(uint32_t* wq, int64_t n32, uint32_t mask);
void orc_qmv(const uint16_t* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
             uint32_t xr, float* Y, int M, int nthreads);
void orc_qmm(const uint16_t* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
             uint32_t xr, float* Y, int M, int nthreads);
void orc_store(const float* Y, void* C, int ldc, int M, int N, int mode);
void orc_a8_quant(const uint16_t* A, int lda, int M, int K, int per_token, int8_t* U, float* XS);
void orc_wxa8(const int8_t* U, const float* XS, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
              int bits, uint32_t xr, float* Y, int M, int nthreads);
void orc_silu_mul(const uint16_t* gu, uint16_t* h, int I, int rows);
void orc_rmsnorm(const uint16_t* x, int in_stride, const uint16_t* w, uint16_t* out, int out_stride, int rows, int D,
                 float eps);
void orc_moe_route(const void* logits, int logits_bf16, int T, int E, int k, int stride, int norm, int shared_gate,
                   int* idx, float* wt, float* sg);
void orc_moe_experts(const uint16_t* xn, int T, int H, int I, int E, int k, const int* idx, const float* wt,
                     const float* sg, const uint32_t* gu_wq, const uint16_t* gu_s, const uint16_t* gu_b,
                     const uint32_t* dn_wq, const uint16_t* dn_s, const uint16_t* dn_b, const uint32_t* sh_gu_wq,
                     const uint16_t* sh_gu_s, const uint16_t* sh_gu_b, const uint32_t* sh_dn_wq,
                     const uint16_t* sh_dn_s, const uint16_t* sh_dn_b, int shared_qmv, uint16_t* out, int assign,
                     int nthreads);
void orc_moe_combine(uint16_t* x, const uint16_t* yd, const float* wt, const uint16_t* ys, const float* sg,
                     const int* inv, int T, int H, int k, int assign);
void orc_moe_dispatch(const int* idx, int R, int E, int* offsets, int* perm, int* inv);
void orc_moe_gather_w4a8(const int8_t* U, const float* XS, const int* perm, int div, const int* offsets,
                         const uint32_t* wq, const uint16_t* s, const uint16_t* b, int E, int N, int K, float* Y,
                         int nthreads);
}

using namespace inferd;

namespace {

int failures = 0;

// The figures of the last bf16_err call, printed by report(): raw = max |got - ref| / RMS(ref) with nothing
// subtracted; ulp1 = the share of elements exactly one bf16 step from a bf16 reference (-1 for an fp32 reference).
double g_raw = 0, g_ulp1 = -1, g_ulp2 = -1, g_far = -1, g_rel_rms = 0;

// err: the figure the bar applies to (net); raw and the one-step share are those of the last bf16_err call
void report(bool pass, const std::string& what, double err) {
  printf("%s %-60s net %.3e raw %.3e", pass ? "ok  " : "FAIL", what.c_str(), err, g_raw);
  if (g_ulp1 >= 0) printf(" ulp1 %.4f ulp2 %.5f far %.1e rel_rms %.1e", g_ulp1, g_ulp2, g_far, g_rel_rms);
  printf("\n");
  fflush(stdout);
  g_raw = 0, g_ulp1 = -1, g_ulp2 = -1, g_far = -1, g_rel_rms = 0;
  if (!pass) failures++;
}

float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <class T>
BufRef upload(const std::vector<T>& v) {
  void* p = nullptr;
  hip_ok(hipMalloc(&p, std::max<size_t>(v.size() * sizeof(T), 256)), "upload");
  hip_ok(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "upload");
  return BufRef(p);
}
template <class T>
std::vector<T> download(const BufRef& r, size_t n) {
  std::vector<T> v(n);
  hip_ok(hipDeviceSynchronize(), "download");
  hip_ok(hipMemcpy(v.data(), r.ptr<void>(), n * sizeof(T), hipMemcpyDeviceToHost), "download");
  return v;
}

// bf16 values -> integers in value order (adjacent bf16 values differ by 1)
int ord16(uint16_t h) { return (h & 0x8000) ? -(int)(h & 0x7FFF) : (int)(h & 0x7FFF); }

// BASELINE's max |err| / RMS(ref) on a bf16 output. Against an fp32 reference: less half a bf16 step of ref (a
// correctly rounded output is within half a step of the value it rounds). Against a bf16 reference: over the
// elements more than one bf16 step away, with no slack; the shares one, two and more steps away go to g_ulp1,
// g_ulp2 and g_far, RMS(got - ref) / RMS(ref) to g_rel_rms (the figures a chain of bf16 stages compared end to end
// is held to, since no per-element bar holds there).
double bf16_err(const std::vector<uint16_t>& got, const std::vector<float>& ref, bool ref_is_bf16) {
  double ss = 0, worst = 0, raw = 0, se = 0;
  size_t one = 0, two = 0, far = 0;
  for (float r : ref) ss += (double)r * r;
  const double rms = std::sqrt(ss / std::max<size_t>(ref.size(), 1));
  for (size_t i = 0; i < ref.size(); i++) {
    const double r = ref[i];
    const double d = std::fabs(bf2f(got[i]) - r);
    raw = std::max(raw, d);
    se += d * d;
    if (ref_is_bf16) {
      const int steps = std::abs(ord16(got[i]) - ord16(f2bf(ref[i])));
      if (steps == 1) one++;
      if (steps == 2) two++;
      if (steps > 2) far++;
      if (steps > 1) worst = std::max(worst, d);
    } else {
      const double ulp = r == 0 ? 0 : std::ldexp(1.0, std::ilogb(r) - 7);
      worst = std::max(worst, d - 0.5 * ulp);
    }
  }
  const double div = rms > 0 ? rms : 1;
  g_raw = raw / div;
  g_ulp1 = ref_is_bf16 ? (double)one / std::max<size_t>(ref.size(), 1) : -1;
  g_ulp2 = ref_is_bf16 ? (double)two / std::max<size_t>(ref.size(), 1) : -1;
  g_far = ref_is_bf16 ? (double)far / std::max<size_t>(ref.size(), 1) : -1;
  g_rel_rms = std::sqrt(se / std::max<size_t>(ref.size(), 1)) / div;
  return worst / div;
}

struct HostLinear {
  int N, K;
  std::vector<uint32_t> wq;
  std::vector<uint16_t> s, b;
};

HostLinear make_linear(int N, int K, std::mt19937& rng) {
  HostLinear h{N, K, {}, {}, {}};
  std::vector<uint8_t> codes((size_t)N * K);
  std::uniform_int_distribution<int> q(0, 15);
  for (auto& c : codes) c = (uint8_t)q(rng);
  h.wq.resize((size_t)N * K / 8);
  orc_pack_w4(codes.data(), h.wq.data(), N, K);
  std::uniform_real_distribution<float> su(0.005f, 0.02f);
  h.s.resize((size_t)N * K / 64);
  h.b.resize(h.s.size());
  for (size_t i = 0; i < h.s.size(); i++) {
    h.s[i] = f2bf(su(rng));
    h.b[i] = f2bf(-8.f * bf2f(h.s[i]));
  }
  return h;
}

// As make_linear, with the codes taken from random 32-bit words (every nibble uniform on 0..15): for the large stacks
HostLinear make_linear_words(int N, int K, std::mt19937& rng) {
  HostLinear h{N, K, std::vector<uint32_t>((size_t)N * K / 8), {}, {}};
  for (auto& w : h.wq) w = (uint32_t)rng();
  std::uniform_real_distribution<float> su(0.005f, 0.02f);
  h.s.resize((size_t)N * K / 64);
  h.b.resize(h.s.size());
  for (size_t i = 0; i < h.s.size(); i++) {
    h.s[i] = f2bf(su(rng));
    h.b[i] = f2bf(-8.f * bf2f(h.s[i]));
  }
  return h;
}

QLinear device_linear(const HostLinear& h) {
  QLinear W;
  W.wq = upload(h.wq);
  W.s = upload(h.s);
  W.b = upload(h.b);
  W.N = h.N;
  W.K = h.K;
  return W;
}

std::vector<uint16_t> activations(int M, int K, std::mt19937& rng) {
  std::normal_distribution<float> nd(0.f, 1.f);
  std::vector<uint16_t> a((size_t)M * K);
  for (auto& v : a) v = f2bf(nd(rng));
  return a;
}

// fp32 y of the reference's W4A8 / W8A8 route: per-group int8 activations (a8_quant) times the (unflipped) codes
// form: the activation quantizer (0: a8_quant, the W4A8 route's; 2: qa8_quant, the QA8 route's)
std::vector<float> ref_wxa8(const std::vector<uint16_t>& A, int M, int K, const uint32_t* wq, const uint16_t* s,
                            const uint16_t* b, int N, int bits, int form = 0) {
  std::vector<int8_t> U((size_t)M * K);
  std::vector<float> XS((size_t)M * (K / 64) * 2), y((size_t)M * N);
  orc_a8_quant(A.data(), K, M, K, form, U.data(), XS.data());
  orc_wxa8(U.data(), XS.data(), wq, s, b, N, K, bits, 0, y.data(), M, 0);
  return y;
}

// fp32 y (before the store) of the GEMM semantics the routed kernel implements
std::vector<float> ref_gemm(const std::vector<uint16_t>& A, const HostLinear& h, int M, bool qmv_semantics) {
  std::vector<float> y((size_t)M * h.N);
  (qmv_semantics ? orc_qmv : orc_qmm)(A.data(), h.K, h.wq.data(), h.s.data(), h.b.data(), h.N, h.K, 0, y.data(), M,
                                      0);
  return y;
}

void test_gemm(Qwen35& m, Enc& e, std::mt19937& rng) {
  const int N = 384, K = 1024;
  const HostLinear h = make_linear(N, K, rng);
  QLinear W = device_linear(h);
  // MLX layout: decode GEMV semantics up to 32 rows, the prefill GEMM's (bf16-rounded dequant) above
  for (int M : {1, 8, 32, 33, 128, 200}) {
    const auto A = activations(M, K, rng);
    BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * N));
    m.gemm(e, dA, W, dC, M, 0);
    const double err = bf16_err(download<uint16_t>(dC, (size_t)M * N), ref_gemm(A, h, M, M <= 32), false);
    report(err <= 1e-2, "gemm MLX layout M=" + std::to_string(M) + " mode 0", err);
    (void)hipFree(dA.buf), (void)hipFree(dC.buf);
  }
  // modes 1 (residual add) and 2 (fp32)
  {
    const int M = 8;
    const auto A = activations(M, K, rng);
    const auto C0 = activations(M, N, rng);
    BufRef dA = upload(A), dC = upload(C0), dF = upload(std::vector<float>((size_t)M * N));
    m.gemm(e, dA, W, dC, M, 1);
    m.gemm(e, dA, W, dF, M, 2);
    const auto y = ref_gemm(A, h, M, true);
    std::vector<float> yr((size_t)M * N);
    for (size_t i = 0; i < yr.size(); i++) yr[i] = y[i] + bf2f(C0[i]);  // mode 1 rounds y + C once
    const double e1 = bf16_err(download<uint16_t>(dC, (size_t)M * N), yr, false);
    report(e1 <= 1e-2, "gemm mode 1 (C += y)", e1);
    const auto f = download<float>(dF, (size_t)M * N);
    double ss = 0, worst = 0;
    for (size_t i = 0; i < y.size(); i++) ss += (double)y[i] * y[i], worst = std::max(worst, (double)std::fabs(f[i] - y[i]));
    const double e2 = worst / std::sqrt(ss / y.size());
    report(e2 <= 1e-3, "gemm mode 2 (fp32)", e2);
    (void)hipFree(dA.buf), (void)hipFree(dC.buf), (void)hipFree(dF.buf);
  }
  // flipped in place: the decode GEMV up to qmv_max rows, the W4A8 route (int8 activations) from there to w4a8_max
  {
    HostLinear hf = h;
    orc_flip(hf.wq.data(), (int64_t)hf.wq.size(), 0x88888888u);
    QLinear Wf = device_linear(hf);
    Wf.flipped = true;
    for (int M : {2, 5, 40}) {
      const auto A = activations(M, K, rng);
      BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * N));
      m.gemm(e, dA, Wf, dC, M, 0);
      const bool a8 = m.w4a8_route(Wf, M);
      const auto y = a8 ? ref_wxa8(A, M, K, h.wq.data(), h.s.data(), h.b.data(), N, 4) : ref_gemm(A, h, M, true);
      const double err = bf16_err(download<uint16_t>(dC, (size_t)M * N), y, false);
      report(err <= 1e-2 && a8 == (M > 2), std::string("gemm flipped weights M=") + std::to_string(M) +
                                               (a8 ? " (W4A8 route)" : ""), err);
      (void)hipFree(dA.buf), (void)hipFree(dC.buf);
    }
    // the fused producers: rmsnorm_for / silu_mul_for write the next GEMM's int8 rows (a8_ready), bit-identical to
    // the plain producer followed by the GEMM's own quantizer (FUSE_A8 = 0)
    const int M = 40, I = K / 2;
    std::uniform_real_distribution<float> pw(0.5f, 2.f);
    std::vector<uint16_t> nw((size_t)K);
    for (auto& v : nw) v = f2bf(pw(rng));
    const auto x = activations(M, K, rng), gu = activations(M, 2 * I, rng);
    HostLinear hd = make_linear(N, I, rng), hdf = hd;
    orc_flip(hdf.wq.data(), (int64_t)hdf.wq.size(), 0x88888888u);
    QLinear Wd = device_linear(hdf);
    Wd.flipped = true;
    BufRef dx = upload(x), dw = upload(nw), dxn = upload(std::vector<uint16_t>((size_t)M * K));
    BufRef dgu = upload(gu), dact = upload(std::vector<uint16_t>((size_t)M * I));
    std::vector<uint16_t> outs[2][2];
    for (int fuse : {3, 0}) {
      m.fuse_a8 = fuse;
      BufRef c1 = upload(std::vector<uint16_t>((size_t)M * N)), c2 = upload(std::vector<uint16_t>((size_t)M * N));
      m.rmsnorm_for(e, dx, dw, dxn, M, K, Wf);
      const bool r1 = m.a8_ready;
      m.gemm(e, dxn, Wf, c1, M, 0);
      m.silu_mul_for(e, dgu, dact, I, M, Wd);
      const bool r2 = m.a8_ready;
      m.gemm(e, dact, Wd, c2, M, 0);
      report(r1 == (fuse >= 3) && r2 == (fuse >= 1) && !m.a8_ready,
             "fused producers set a8_ready (FUSE_A8=" + std::to_string(fuse) + ")", 0);
      outs[fuse ? 0 : 1][0] = download<uint16_t>(c1, (size_t)M * N);
      outs[fuse ? 0 : 1][1] = download<uint16_t>(c2, (size_t)M * N);
      (void)hipFree(c1.buf), (void)hipFree(c2.buf);
    }
    m.fuse_a8 = 3;
    report(outs[0][0] == outs[1][0], "rmsnorm_for -> gemm (int8 rows fused) == rmsnorm -> gemm, bit for bit", 0);
    report(outs[0][1] == outs[1][1], "silu_mul_for -> gemm (int8 rows fused) == silu_mul -> gemm, bit for bit", 0);
    std::vector<uint16_t> xr((size_t)M * K), hr((size_t)M * I);
    orc_rmsnorm(x.data(), K, nw.data(), xr.data(), K, M, K, m.cfg.eps);
    orc_silu_mul(gu.data(), hr.data(), I, M);
    double e1 = bf16_err(outs[0][0], ref_wxa8(xr, M, K, h.wq.data(), h.s.data(), h.b.data(), N, 4), false);
    report(e1 <= 1e-2, "rmsnorm_for -> gemm (W4A8) vs the oracle", e1);
    e1 = bf16_err(outs[0][1], ref_wxa8(hr, M, I, hd.wq.data(), hd.s.data(), hd.b.data(), N, 4), false);
    report(e1 <= 1e-2, "silu_mul_for -> gemm (W4A8) vs the oracle", e1);
    // the same flipped layers with their T64 copies (the unflipped codes, as the loader packs them): the W4A8 route
    // then runs on T64 (the decode GEMV up to 16 rows, the affine K-split kernel above) with the same per-group
    // int8 activations, for plain and fused producers
    void* tf = nullptr;
    void* td = nullptr;
    hip_ok(hipMalloc(&tf, ifd_t64_bytes(N, K, 1)), "t64");
    hip_ok(hipMalloc(&td, ifd_t64_bytes(N, I, 1)), "t64");
    ok(ifd_pack_t64(Wf.wq.ptr<uint32_t>(), Wf.s.ptr<uint16_t>(), Wf.b.ptr<uint16_t>(), N, K, 0, 0x88888888u, 1, tf,
                    e.stream),
       "pack_t64");
    ok(ifd_pack_t64(Wd.wq.ptr<uint32_t>(), Wd.s.ptr<uint16_t>(), Wd.b.ptr<uint16_t>(), N, I, 0, 0x88888888u, 1, td,
                    e.stream),
       "pack_t64");
    Wf.t64 = BufRef(tf), Wd.t64 = BufRef(td);
    for (int Mt : {3, 16, 17, 40, 100, 200}) {
      const auto A = activations(Mt, K, rng);
      BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)Mt * N));
      m.gemm(e, dA, Wf, dC, Mt, 0);
      const double err =
          bf16_err(download<uint16_t>(dC, (size_t)Mt * N), ref_wxa8(A, Mt, K, h.wq.data(), h.s.data(), h.b.data(), N, 4),
                   false);
      report(err <= 1e-2 && m.w4a8_route(Wf, Mt), "gemm flipped weights, T64 copy, M=" + std::to_string(Mt) +
                                                      " (W4A8 route on T64)", err);
      (void)hipFree(dA.buf), (void)hipFree(dC.buf);
    }
    {
      BufRef c1 = upload(std::vector<uint16_t>((size_t)M * N)), c2 = upload(std::vector<uint16_t>((size_t)M * N));
      m.rmsnorm_for(e, dx, dw, dxn, M, K, Wf);
      m.gemm(e, dxn, Wf, c1, M, 0);
      m.silu_mul_for(e, dgu, dact, I, M, Wd);
      m.gemm(e, dact, Wd, c2, M, 0);
      double e3 = bf16_err(download<uint16_t>(c1, (size_t)M * N),
                           ref_wxa8(xr, M, K, h.wq.data(), h.s.data(), h.b.data(), N, 4), false);
      report(e3 <= 1e-2, "rmsnorm_for -> gemm (W4A8 on T64) vs the oracle", e3);
      e3 = bf16_err(download<uint16_t>(c2, (size_t)M * N),
                    ref_wxa8(hr, M, I, hd.wq.data(), hd.s.data(), hd.b.data(), N, 4), false);
      report(e3 <= 1e-2, "silu_mul_for -> gemm (W4A8 on T64) vs the oracle", e3);
      (void)hipFree(c1.buf), (void)hipFree(c2.buf);
    }
    for (void* p : {dx.buf, dw.buf, dxn.buf, dgu.buf, dact.buf, Wd.wq.buf, Wd.s.buf, Wd.b.buf, Wf.wq.buf, Wf.s.buf,
                    Wf.b.buf, tf, td})
      (void)hipFree(p);
  }
  // T64 copy: decode GEMV semantics up to 64 rows, prefill semantics above
  {
    void* t = nullptr;
    hip_ok(hipMalloc(&t, ifd_t64_bytes(N, K, 1)), "t64");
    ok(ifd_pack_t64(W.wq.ptr<uint32_t>(), W.s.ptr<uint16_t>(), W.b.ptr<uint16_t>(), N, K, 0, 0, 1, t, e.stream),
       "pack_t64");
    QLinear Wt = W;
    Wt.t64 = BufRef(t);
    for (int M : {1, 16, 17, 64, 65, 128, 300}) {
      const auto A = activations(M, K, rng);
      BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * N));
      m.gemm(e, dA, Wt, dC, M, 0);
      const double err = bf16_err(download<uint16_t>(dC, (size_t)M * N), ref_gemm(A, h, M, M <= 64), false);
      report(err <= 1e-2, "gemm T64 M=" + std::to_string(M), err);
      (void)hipFree(dA.buf), (void)hipFree(dC.buf);
    }
    // K-slice [256, 768) of the T64 copy and of the MLX layout
    for (bool use_t64 : {true, false}) {
      const int M = 8, k0 = 256, kn = 512;
      QLinear Ws = kslice_of(use_t64 ? Wt : W, k0, kn);
      const auto A = activations(M, kn, rng);
      HostLinear hs{N, kn, std::vector<uint32_t>((size_t)N * kn / 8), std::vector<uint16_t>((size_t)N * kn / 64),
                    std::vector<uint16_t>((size_t)N * kn / 64)};
      for (int n = 0; n < N; n++) {
        memcpy(&hs.wq[(size_t)n * kn / 8], &h.wq[(size_t)n * K / 8 + k0 / 8], kn / 2);
        memcpy(&hs.s[(size_t)n * kn / 64], &h.s[(size_t)n * K / 64 + k0 / 64], kn / 32);
        memcpy(&hs.b[(size_t)n * kn / 64], &h.b[(size_t)n * K / 64 + k0 / 64], kn / 32);
      }
      BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * N));
      m.gemm(e, dA, Ws, dC, M, 0);
      const double err = bf16_err(download<uint16_t>(dC, (size_t)M * N), ref_gemm(A, hs, M, true), false);
      report(err <= 1e-2, std::string("gemm kslice_of ") + (use_t64 ? "(T64)" : "(MLX layout)"), err);
      (void)hipFree(dA.buf), (void)hipFree(dC.buf);
    }
    (void)hipFree(t);
  }
  // rows_of: output rows [128, 256)
  {
    const int M = 4, lo = 128, n = 128;
    QLinear Wr = rows_of(W, lo, n);
    const auto A = activations(M, K, rng);
    BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * n));
    m.gemm(e, dA, Wr, dC, M, 0);
    const auto y = ref_gemm(A, h, M, true);
    std::vector<float> yr((size_t)M * n);
    for (int r = 0; r < M; r++)
      for (int c = 0; c < n; c++) yr[(size_t)r * n + c] = y[(size_t)r * N + lo + c];
    const double err = bf16_err(download<uint16_t>(dC, (size_t)M * n), yr, false);
    report(err <= 1e-2, "gemm rows_of [128, 256)", err);
    (void)hipFree(dA.buf), (void)hipFree(dC.buf);
  }
  (void)hipFree(W.wq.buf), (void)hipFree(W.s.buf), (void)hipFree(W.b.buf);
  // 8-bit weights (qmv8 arithmetic up to 32 rows, MLX 8-bit qmm above), flipped storage and a rows_of view
  {
    std::vector<uint8_t> codes((size_t)N * K);
    std::uniform_int_distribution<int> q(0, 255);
    for (auto& c : codes) c = (uint8_t)q(rng);
    std::vector<uint32_t> wq8((size_t)N * K / 4);
    orc_pack_w8(codes.data(), wq8.data(), N, K);
    std::uniform_real_distribution<float> su(0.0003f, 0.0012f), bu(-0.1f, 0.1f);
    std::vector<uint16_t> s8((size_t)N * K / 64), b8(s8.size());
    for (size_t i = 0; i < s8.size(); i++) s8[i] = f2bf(su(rng)), b8[i] = f2bf(bu(rng));
    std::vector<uint32_t> wq8f = wq8;
    for (auto& w : wq8f) w ^= 0x80808080u;
    for (bool flipped : {false, true}) {
      QLinear W8;
      W8.wq = upload(flipped ? wq8f : wq8), W8.s = upload(s8), W8.b = upload(b8);
      W8.N = N, W8.K = K, W8.bits = 8, W8.flipped = flipped;
      for (int M : {1, 33, 200}) {
        const auto A = activations(M, K, rng);
        std::vector<float> y((size_t)M * N);
        const bool a8 = m.w4a8_route(W8, M);  // flipped 8-bit weights below w4a8_max rows: W8A8
        if (a8) y = ref_wxa8(A, M, K, wq8.data(), s8.data(), b8.data(), N, 8);
        else (M <= 32 ? orc_qmv_b : orc_qmm_b)(A.data(), K, wq8.data(), s8.data(), b8.data(), N, K, 8, 0, y.data(), M, 0);
        BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * N));
        m.gemm(e, dA, W8, dC, M, 0);
        const double err = bf16_err(download<uint16_t>(dC, (size_t)M * N), y, false);
        report(err <= 1e-2 && a8 == (flipped && M > 2),
               std::string("gemm 8-bit") + (flipped ? " flipped" : "") + " M=" + std::to_string(M) +
                   (a8 ? " (W8A8 route)" : ""),
               err);
        if (M == 1) {  // rows_of [128, 256) of the same layer
          QLinear Wr = rows_of(W8, 128, 128);
          BufRef dR = upload(std::vector<uint16_t>(128));
          m.gemm(e, dA, Wr, dR, 1, 0);
          std::vector<float> yr(y.begin() + 128, y.begin() + 256);
          const double er = bf16_err(download<uint16_t>(dR, 128), yr, false);
          report(er <= 1e-2, "gemm 8-bit rows_of [128, 256)", er);
          (void)hipFree(dR.buf);
        }
        (void)hipFree(dA.buf), (void)hipFree(dC.buf);
      }
      (void)hipFree(W8.wq.buf), (void)hipFree(W8.s.buf), (void)hipFree(W8.b.buf);
    }
    // a T64x8 copy: every 8-bit route runs on it, qmv8 arithmetic up to 16 rows and qmm rounding above, whole and
    // as a K-slice
    QLinear W8;
    W8.wq = upload(wq8), W8.s = upload(s8), W8.b = upload(b8);
    W8.N = N, W8.K = K, W8.bits = 8;
    void* t = nullptr;
    hip_ok(hipMalloc(&t, ifd_t64x8_bytes(N, K)), "t64x8");
    ok(ifd_pack_t64x8(W8.wq.ptr<uint32_t>(), W8.s.ptr<uint16_t>(), W8.b.ptr<uint16_t>(), N, K, 0, 0, t, e.stream),
       "pack_t64x8");
    W8.t64 = BufRef(t);
    for (int M : {1, 16, 24, 33, 200}) {
      const auto A = activations(M, K, rng);
      std::vector<float> y((size_t)M * N);
      (M <= 16 ? orc_qmv_b : orc_qmm_b)(A.data(), K, wq8.data(), s8.data(), b8.data(), N, K, 8, 0, y.data(), M, 0);
      BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * N));
      m.gemm(e, dA, W8, dC, M, 0);
      const double err = bf16_err(download<uint16_t>(dC, (size_t)M * N), y, false);
      report(err <= 1e-2, "gemm 8-bit T64x8 M=" + std::to_string(M), err);
      (void)hipFree(dA.buf), (void)hipFree(dC.buf);
    }
    {
      const int M = 40, k0 = 192, kn = 320;
      QLinear Ws = kslice_of(W8, k0, kn);
      const auto A = activations(M, kn, rng);
      std::vector<uint32_t> ws((size_t)N * kn / 4);
      std::vector<uint16_t> ss((size_t)N * kn / 64), bs(ss.size());
      for (int n = 0; n < N; n++) {
        memcpy(&ws[(size_t)n * kn / 4], &wq8[(size_t)n * K / 4 + k0 / 4], kn);
        memcpy(&ss[(size_t)n * kn / 64], &s8[(size_t)n * K / 64 + k0 / 64], kn / 32);
        memcpy(&bs[(size_t)n * kn / 64], &b8[(size_t)n * K / 64 + k0 / 64], kn / 32);
      }
      std::vector<float> y((size_t)M * N);
      orc_qmm_b(A.data(), kn, ws.data(), ss.data(), bs.data(), N, kn, 8, 0, y.data(), M, 0);
      BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * N));
      m.gemm(e, dA, Ws, dC, M, 0);
      const double err = bf16_err(download<uint16_t>(dC, (size_t)M * N), y, false);
      report(err <= 1e-2 && (bool)Ws.t64, "gemm 8-bit kslice_of (T64x8)", err);
      (void)hipFree(dA.buf), (void)hipFree(dC.buf);
    }
    // the same 8-bit layer with and without its T64x8 copy: both routes keep the qmv8 arithmetic up to 16 rows (the
    // MLX layout up to 32), so at M = 3 and 16 they differ by fp32 summation order at most; at M = 24 the T64x8 route
    // has the qmm rounding (every weight rounded to bf16(s q + b)) and the MLX route still the qmv8 arithmetic.
    // Differences in bf16 steps of the larger of the two values. Budget: M <= 16, no element more than one step
    // apart; M = 24, RMS(difference) <= 5e-3 RMS and max |difference| <= 2e-2 RMS (two roundings of the same sum,
    // each within BASELINE's 1e-2 of it).
    {
      QLinear Wm = W8;
      Wm.t64 = BufRef();
      for (int M : {3, 16, 24}) {
        const auto A = activations(M, K, rng);
        BufRef dA = upload(A), c1 = upload(std::vector<uint16_t>((size_t)M * N)),
               c2 = upload(std::vector<uint16_t>((size_t)M * N));
        m.gemm(e, dA, W8, c1, M, 0);
        m.gemm(e, dA, Wm, c2, M, 0);
        const auto o1 = download<uint16_t>(c1, (size_t)M * N), o2 = download<uint16_t>(c2, (size_t)M * N);
        double ss = 0, sd = 0, worst = 0, maxst = 0;
        for (size_t i = 0; i < o1.size(); i++) {
          const double a = bf2f(o1[i]), bb = bf2f(o2[i]), d = std::fabs(a - bb), big = std::max(std::fabs(a), std::fabs(bb));
          ss += bb * bb, sd += d * d;
          worst = std::max(worst, d);
          if (d > 0) maxst = std::max(maxst, d / std::ldexp(1.0, std::ilogb(big) - 7));
        }
        const double rms = std::sqrt(ss / o1.size()), rd = std::sqrt(sd / o1.size()) / rms;
        const bool pass = M <= 16 ? maxst <= 1.0 : rd <= 5e-3 && worst <= 2e-2 * rms;
        printf("     8-bit T64x8 vs MLX layout M=%d: max steps %.1f, RMS(diff)/RMS %.2e, max|diff|/RMS %.2e\n", M,
               maxst, rd, worst / rms);
        report(pass, "gemm 8-bit, T64x8 copy vs MLX layout M=" + std::to_string(M), worst / rms);
        (void)hipFree(dA.buf), (void)hipFree(c1.buf), (void)hipFree(c2.buf);
      }
    }
    (void)hipFree(t), (void)hipFree(W8.wq.buf), (void)hipFree(W8.s.buf), (void)hipFree(W8.b.buf);
  }
}

void test_encode_moe(std::mt19937& rng) {
  Config c;
  c.hidden = 512, c.experts = 32, c.topk = 4, c.moe_inter = 128, c.eps = 1e-6f;
  const int H = c.hidden, E = c.experts, k = c.topk, I = c.moe_inter, Is = 128;
  // layer: stacked experts [E, 2I, H] and [E, H, I], shared expert, bf16 router with the shared gate row
  const HostLinear egu = make_linear(E * 2 * I, H, rng), edn = make_linear(E * H, I, rng);
  const HostLinear sgu = make_linear(2 * Is, H, rng), sdn = make_linear(H, Is, rng);
  std::normal_distribution<float> nr(0.f, 0.02f);
  std::vector<uint16_t> router((size_t)(E + 1) * H), post((size_t)H);
  for (auto& v : router) v = f2bf(nr(rng));
  std::uniform_real_distribution<float> pw(0.5f, 2.f);
  for (auto& v : post) v = f2bf(pw(rng));
  Layer ly;
  ly.post_norm = upload(post);
  ly.gate_up = device_linear(sgu);
  ly.down = device_linear(sdn);
  ly.router.wq = upload(router);
  ly.router.E = 1, ly.router.N = E + 1, ly.router.K = H, ly.router.bits = 16;
  const QLinear g = device_linear(egu), d = device_linear(edn);
  ly.egu.wq = g.wq, ly.egu.s = g.s, ly.egu.b = g.b, ly.egu.E = E, ly.egu.N = 2 * I, ly.egu.K = H, ly.egu.bits = 4;
  ly.edown.wq = d.wq, ly.edown.s = d.s, ly.edown.b = d.b, ly.edown.E = E, ly.edown.N = H, ly.edown.K = I,
  ly.edown.bits = 4;
  // the shared expert's gate/up also as a T64 copy: encode_moe then takes the fused gate/up + SwiGLU call
  void* sgu_t64 = nullptr;
  hip_ok(hipMalloc(&sgu_t64, ifd_t64_bytes(2 * Is, H, 1)), "t64");
  ok(ifd_pack_t64(ly.gate_up.wq.ptr<uint32_t>(), ly.gate_up.s.ptr<uint16_t>(), ly.gate_up.b.ptr<uint16_t>(), 2 * Is, H,
                  0, 0, 1, sgu_t64, nullptr),
     "pack_t64");
  const QLinear sgu_mlx = ly.gate_up;
  // T64 copies of the routed stacks and of the shared down: the decode route then streams them (up to 8 tokens) when
  // the shared expert has both copies
  void* et64[3] = {};
  {
    const int NN[3] = {2 * I, H, H}, KK[3] = {H, I, Is}, EE[3] = {E, E, 1};
    const BufRef wq[3] = {ly.egu.wq, ly.edown.wq, ly.down.wq}, sc[3] = {ly.egu.s, ly.edown.s, ly.down.s},
                 bi[3] = {ly.egu.b, ly.edown.b, ly.down.b};
    for (int i = 0; i < 3; i++) {
      hip_ok(hipMalloc(&et64[i], ifd_t64_bytes(NN[i], KK[i], EE[i])), "t64");
      ok(ifd_pack_t64(wq[i].ptr<uint32_t>(), sc[i].ptr<uint16_t>(), bi[i].ptr<uint16_t>(), NN[i], KK[i], 0, 0u, EE[i],
                      et64[i], nullptr),
         "pack_t64");
    }
    hip_ok(hipDeviceSynchronize(), "pack_t64");
  }
  // an 8-bit router [E + 1, H] (the shared gate last), w = s q + b with b = -128 s
  std::vector<uint32_t> r8wq((size_t)(E + 1) * H / 4);
  std::vector<uint16_t> r8s((size_t)(E + 1) * H / 64), r8b(r8s.size());
  {
    std::vector<uint8_t> codes((size_t)(E + 1) * H);
    std::uniform_int_distribution<int> q(0, 255);
    for (auto& v : codes) v = (uint8_t)q(rng);
    orc_pack_w8(codes.data(), r8wq.data(), E + 1, H);
    std::uniform_real_distribution<float> su(0.0001f, 0.0003f);
    for (size_t i = 0; i < r8s.size(); i++) r8s[i] = f2bf(su(rng)), r8b[i] = f2bf(-128.f * bf2f(r8s[i]));
  }
  // an 8-bit shared expert (the reference's moe_gu2_4_8 / moe_dn2_4_8), taken on the decode route
  auto make_linear8 = [&](int N, int K) {
    HostLinear h{N, K, std::vector<uint32_t>((size_t)N * K / 4), std::vector<uint16_t>((size_t)N * K / 64), {}};
    std::vector<uint8_t> codes((size_t)N * K);
    std::uniform_int_distribution<int> q(0, 255);
    for (auto& v : codes) v = (uint8_t)q(rng);
    orc_pack_w8(codes.data(), h.wq.data(), N, K);
    std::uniform_real_distribution<float> su(0.0003f, 0.0012f), bu(-0.1f, 0.1f);
    h.b.resize(h.s.size());
    for (size_t i = 0; i < h.s.size(); i++) h.s[i] = f2bf(su(rng)), h.b[i] = f2bf(bu(rng));
    return h;
  };
  const HostLinear sgu8 = make_linear8(2 * Is, H), sdn8 = make_linear8(H, Is);
  QLinear sgu8_d = device_linear(sgu8), sdn8_d = device_linear(sdn8);
  sgu8_d.bits = 8, sdn8_d.bits = 8;
  const QLinear sdn_mlx = ly.down;
  const MoeW router16 = ly.router;
  MoeW router8;
  router8.wq = upload(r8wq), router8.s = upload(r8s), router8.b = upload(r8b);
  router8.E = 1, router8.N = E + 1, router8.K = H, router8.bits = 8;
  struct Case {
    int T, max_rows;
    bool t64, r8, s8 = false, et64 = false;
  };
  // the decode route (up to qmv_max tokens; up to 8 with the 8-bit router), the per-row route below 128 routed rows
  // (T <= 31 at top-4, 16 tokens per launch group), the sorted route beyond; the fused T64 shared gate/up; state
  // allocated for more rows than the call (its scratch covers every row count); the 8-bit router on all three; the
  // decode route on the routed experts' T64 copies (et64), streamed when the shared expert has both T64 copies
  // (4-bit) and on the MLX layout otherwise; the per-row route on those copies (8-token launch groups)
  for (const Case cs : {Case{1, 1, false, false}, Case{24, 24, false, false}, Case{31, 40, false, true},
                        Case{3, 3, false, false}, Case{8, 8, false, false}, Case{16, 16, false, false},
                        Case{100, 100, false, false}, Case{16, 16, true, false}, Case{100, 100, true, false},
                        Case{100, 256, true, false}, Case{3, 3, false, true}, Case{12, 12, false, true},
                        Case{40, 40, false, true}, Case{3, 3, false, false, true}, Case{8, 8, false, true, true},
                        Case{1, 1, true, false, false, true}, Case{2, 4, true, false, false, true},
                        Case{8, 8, true, true, false, true}, Case{5, 5, false, true, false, true},
                        Case{8, 8, false, true, true, true}, Case{5, 5, true, false, false, true},
                        Case{20, 24, true, false, false, true}}) {
    const int T = cs.T;
    ly.gate_up = cs.s8 ? sgu8_d : sgu_mlx;
    ly.down = cs.s8 ? sdn8_d : sdn_mlx;
    if (cs.t64) ly.gate_up.t64 = BufRef(sgu_t64);
    ly.egu.t64 = cs.et64 ? BufRef(et64[0]) : BufRef(), ly.edown.t64 = cs.et64 ? BufRef(et64[1]) : BufRef();
    if (cs.et64 && !cs.s8) ly.down.t64 = BufRef(et64[2]);
    ly.router = cs.r8 ? router8 : router16;
    Qwen35 m(c, cs.max_rows, Is, 0);
    Enc e;
    const auto x0 = activations(T, H, rng);
    hip_ok(hipMemcpy(m.x.ptr<void>(), x0.data(), x0.size() * 2, hipMemcpyHostToDevice), "x");
    m.encode_moe(e, ly, T);
    const auto x1 = download<uint16_t>(m.x, (size_t)T * H);
    const auto xn = download<uint16_t>(m.xn, (size_t)T * H);
    const auto logits = download<float>(m.rlog, (size_t)T * (E + 1));
    const auto idx = download<int>(m.ridx, (size_t)T * k);
    const auto wt = download<float>(m.rw, (size_t)T * k);
    const auto sg = download<float>(m.rsg, (size_t)T);
    const bool dec = m.moe_decode_route(ly, T), rows = m.moe_rows_route(ly, T);
    const std::string tag = " T=" + std::to_string(T) + (cs.max_rows > T ? " of " + std::to_string(cs.max_rows) : "") +
                            (ly.gate_up.t64 ? " (T64 shared gate/up)" : "") + (cs.r8 ? " (8-bit router)" : "") +
                            (cs.s8 ? " (8-bit shared expert)" : "") +
                            (dec    ? (m.moe_decode_t64(ly, T) ? " [decode, T64]" : " [decode]")
                             : rows ? (ly.egu.t64 ? " [per-row, T64]" : " [per-row]")
                                    : " [sorted]");
    // the reference's routes: moe2 up to 8 tokens with an 8-bit router (and here up to qmv_max tokens with any),
    // the per-row products below 128 routed rows, the sorted path from there
    report(dec == (T <= m.qmv_max || (T <= 8 && cs.r8)) && rows == (!dec && T * k < 128) &&
               m.moe_decode_t64(ly, T) == (dec && cs.et64 && cs.t64 && !cs.s8),
           "encode_moe route" + tag, 0);
    if (cs.r8) {  // the logits against the oracle's qmv8 on the GPU's normalised rows
      std::vector<float> yl((size_t)T * (E + 1));
      orc_qmv_b(xn.data(), H, r8wq.data(), r8s.data(), r8b.data(), E + 1, H, 8, 0, yl.data(), T, 0);
      double ss = 0, w = 0;
      for (size_t i = 0; i < yl.size(); i++) ss += (double)yl[i] * yl[i], w = std::max(w, (double)std::fabs(yl[i] - logits[i]));
      const double el = w / std::sqrt(ss / yl.size());
      report(el <= 1e-5, "encode_moe 8-bit router logits (fp32)" + tag, el);
    }
    // rmsnorm: within one bf16 step of the oracle
    std::vector<uint16_t> xr((size_t)T * H);
    orc_rmsnorm(x0.data(), H, post.data(), xr.data(), H, T, H, c.eps);
    std::vector<float> xrf(xr.size());
    for (size_t i = 0; i < xr.size(); i++) xrf[i] = bf2f(xr[i]);
    const double en = bf16_err(xn, xrf, true);
    report(en == 0.0, "encode_moe rmsnorm" + tag, en);
    // routing on the GPU's own logits: bit-exact indices
    std::vector<int> ri((size_t)T * k);
    std::vector<float> rwt((size_t)T * k), rsg((size_t)T);
    orc_moe_route(logits.data(), 0, T, E, k, E + 1, 1, 1, ri.data(), rwt.data(), rsg.data());
    double ew = 0;
    for (size_t i = 0; i < rwt.size(); i++) ew = std::max(ew, (double)std::fabs(rwt[i] - wt[i]));
    for (int t = 0; t < T; t++) ew = std::max(ew, (double)std::fabs(rsg[t] - sg[t]));
    report(ri == idx && ew <= 1e-5, "encode_moe routing (indices bit-exact)" + tag, ew);
    // the block's output added into x, from the GPU's normalised rows and routing
    std::vector<uint16_t> want = x0;
    // the per-row route's shared expert goes through gemm(): the decode GEMV arithmetic at these rows (up to 32 on
    // the MLX layout, 16 on T64), as on the decode route
    if (cs.s8) {  // the decode or the per-row route
      report(dec || rows, "encode_moe takes the decode or per-row route with an 8-bit shared expert" + tag, 0);
      orc_moe_decode_b(xn.data(), T, H, I, k, ri.data(), rwt.data(), rsg.data(), egu.wq.data(), egu.s.data(),
                       egu.b.data(), edn.wq.data(), edn.s.data(), edn.b.data(), sgu8.wq.data(), sgu8.s.data(),
                       sgu8.b.data(), sdn8.wq.data(), sdn8.s.data(), sdn8.b.data(), 8, want.data(), 0);
    } else if (dec || rows)  // the decode GEMV arithmetic for every expert product
      orc_moe_decode(xn.data(), T, H, I, k, ri.data(), rwt.data(), rsg.data(), egu.wq.data(), egu.s.data(),
                     egu.b.data(), edn.wq.data(), edn.s.data(), edn.b.data(), sgu.wq.data(), sgu.s.data(),
                     sgu.b.data(), sdn.wq.data(), sdn.s.data(), sdn.b.data(), want.data(), 0);
    else
      orc_moe_experts(xn.data(), T, H, I, E, k, ri.data(), rwt.data(), rsg.data(), egu.wq.data(), egu.s.data(),
                      egu.b.data(), edn.wq.data(), edn.s.data(), edn.b.data(), sgu.wq.data(), sgu.s.data(),
                      sgu.b.data(), sdn.wq.data(), sdn.s.data(), sdn.b.data(), T <= 32 ? 1 : 0, want.data(), 0, 0);
    std::vector<float> wf(want.size());
    for (size_t i = 0; i < want.size(); i++) wf[i] = bf2f(want[i]);
    // a chain of bf16 stages on both sides, compared end to end: RMS error, raw and the one-step share are bounded
    // (the stages themselves are checked one by one at the bar in tests/test_gpu_moe.py)
    (void)bf16_err(x1, wf, true);
    report(g_rel_rms <= 1e-2 && g_raw <= 5e-2 && g_ulp1 <= 0.05,
           "encode_moe x += moe(xn) (end to end)" + tag, g_raw);
  }
  (void)hipFree(sgu_t64);
  for (void* q : et64) (void)hipFree(q);
  (void)hipFree(router8.wq.buf), (void)hipFree(router8.s.buf), (void)hipFree(router8.b.buf);
  for (void* q : {sgu8_d.wq.buf, sgu8_d.s.buf, sgu8_d.b.buf, sdn8_d.wq.buf, sdn8_d.s.buf, sdn8_d.b.buf})
    (void)hipFree(q);
}

// A MoE layer at one geometry, with both the MLX-layout stacks and their T64 copies on the device.
struct MoeGeo {
  int H, E, k, I;
};
struct MoeLayer {
  MoeGeo g;
  HostLinear egu, edn, sgu, sdn;
  std::vector<uint16_t> router, post;
  Layer ly;                      // MLX buffers + T64 stacks; the shared expert with its T64 copies
  void* t64[4] = {};             // egu, edn, sgu, sdn T64 copies
  MoeLayer(const MoeGeo& geo, std::mt19937& rng) : g(geo) {
    const int H = g.H, E = g.E, I = g.I;
    egu = make_linear_words(E * 2 * I, H, rng), edn = make_linear_words(E * H, I, rng);
    sgu = make_linear_words(2 * I, H, rng), sdn = make_linear_words(H, I, rng);
    std::normal_distribution<float> nr(0.f, 0.02f);
    router.resize((size_t)(E + 1) * H), post.resize(H);
    for (auto& v : router) v = f2bf(nr(rng));
    std::uniform_real_distribution<float> pw(0.5f, 2.f);
    for (auto& v : post) v = f2bf(pw(rng));
    ly.post_norm = upload(post);
    ly.router.wq = upload(router);
    ly.router.E = 1, ly.router.N = E + 1, ly.router.K = H, ly.router.bits = 16;
    const QLinear gq = device_linear(egu), dq = device_linear(edn);
    ly.egu.wq = gq.wq, ly.egu.s = gq.s, ly.egu.b = gq.b, ly.egu.E = E, ly.egu.N = 2 * I, ly.egu.K = H, ly.egu.bits = 4;
    ly.edown.wq = dq.wq, ly.edown.s = dq.s, ly.edown.b = dq.b, ly.edown.E = E, ly.edown.N = H, ly.edown.K = I,
    ly.edown.bits = 4;
    ly.gate_up = device_linear(sgu), ly.down = device_linear(sdn);
    const QLinear* src[4] = {&gq, &dq, &ly.gate_up, &ly.down};
    const int NN[4] = {2 * I, H, 2 * I, H}, KK[4] = {H, I, H, I}, EE[4] = {E, E, 1, 1};
    for (int i = 0; i < 4; i++) {
      hip_ok(hipMalloc(&t64[i], ifd_t64_bytes(NN[i], KK[i], EE[i])), "t64");
      ok(ifd_pack_t64(src[i]->wq.ptr<uint32_t>(), src[i]->s.ptr<uint16_t>(), src[i]->b.ptr<uint16_t>(), NN[i], KK[i], 0,
                      0u, EE[i], t64[i], nullptr),
         "pack_t64");
    }
    ly.egu.t64 = BufRef(t64[0]), ly.edown.t64 = BufRef(t64[1]);
    ly.gate_up.t64 = BufRef(t64[2]), ly.down.t64 = BufRef(t64[3]);
    hip_ok(hipDeviceSynchronize(), "pack_t64");
  }
  ~MoeLayer() {
    for (void* p : {ly.post_norm.buf, ly.router.wq.buf, ly.egu.wq.buf, ly.egu.s.buf, ly.egu.b.buf, ly.edown.wq.buf,
                    ly.edown.s.buf, ly.edown.b.buf, ly.gate_up.wq.buf, ly.gate_up.s.buf, ly.gate_up.b.buf,
                    ly.down.wq.buf, ly.down.s.buf, ly.down.b.buf, t64[0], t64[1], t64[2], t64[3]})
      if (p) (void)hipFree(p);
  }
};

// encode_moe on the sorted route over T64 expert stacks. shared: 0 no shared expert; 1 the shared expert with T64
// copies (expert E of the gathered launches); 2 the shared expert without T64 copies (gemm() on the MLX layout, then
// the T64 launches for the routed experts). Checks: rmsnorm within one bf16 step; routing indices bit-exact
// on the GPU's own logits; x += MoE(xn) against the oracle's composition on the GPU's normalised rows and routing, for
// `check` tokens spread over the batch (every token when check >= T; each token's output depends on its own row only).
void run_moe_t64(MoeLayer& L, int T, int max_rows, int shared, int check, int nthreads, std::mt19937& rng) {
  const MoeGeo g = L.g;
  const int H = g.H, E = g.E, k = g.k, I = g.I;
  Config c;
  c.hidden = H, c.experts = E, c.topk = k, c.moe_inter = I, c.eps = 1e-6f;
  Layer ly = L.ly;
  if (shared == 0) ly.gate_up = QLinear(), ly.down = QLinear(), ly.router.N = E;
  if (shared == 2) ly.gate_up.t64 = BufRef(), ly.down.t64 = BufRef();
  Qwen35 m(c, max_rows, shared ? I : 0, 0);
  Enc e;
  const auto x0 = activations(T, H, rng);
  hip_ok(hipMemcpy(m.x.ptr<void>(), x0.data(), x0.size() * 2, hipMemcpyHostToDevice), "x");
  m.encode_moe(e, ly, T);
  const auto x1 = download<uint16_t>(m.x, (size_t)T * H);
  const auto xn = download<uint16_t>(m.xn, (size_t)T * H);
  const int E1 = shared ? E + 1 : E;
  const auto logits = download<float>(m.rlog, (size_t)T * E1);
  const auto idx = download<int>(m.ridx, (size_t)T * k);
  const auto wt = download<float>(m.rw, (size_t)T * k);
  const auto sg = download<float>(m.rsg, (size_t)T);
  const bool dec = m.moe_decode_route(ly, T), t64 = m.moe_t64_route(ly), fold = m.shared_as_expert(ly, T);
  const bool dt64 = m.moe_decode_t64(ly, T);
  const std::string tag = " T=" + std::to_string(T) + " H=" + std::to_string(H) + " E=" + std::to_string(E) +
                          " k=" + std::to_string(k) + " I=" + std::to_string(I) +
                          (shared == 0 ? " (no shared expert)"
                           : dec       ? (shared == 1 ? " (shared on T64)" : " (shared on the MLX layout)")
                           : fold      ? " (shared = expert E)"
                                       : " (shared via gemm)") +
                          (dec ? (dt64 ? " [decode, T64]" : " [decode]") : t64 ? " [sorted, T64]" : " [sorted, MLX]");
  // up to qmv_max tokens the decode route, on the T64 copies when the shared expert (if any) has them too
  if (T <= m.qmv_max) report(dec && dt64 == (shared != 2), "encode_moe takes the decode route" + tag, 0);
  else report(!dec && t64 && fold == (shared == 1), "encode_moe takes the T64 sorted route" + tag, 0);
  // rmsnorm: within one bf16 step of the oracle (the sum of squares runs in another order)
  std::vector<uint16_t> xr((size_t)T * H);
  orc_rmsnorm(x0.data(), H, L.post.data(), xr.data(), H, T, H, c.eps);
  std::vector<float> xrf(xr.size());
  for (size_t i = 0; i < xr.size(); i++) xrf[i] = bf2f(xr[i]);
  const double en = bf16_err(xn, xrf, true);
  report(en == 0.0, "encode_moe rmsnorm" + tag, en);
  std::vector<int> ri((size_t)T * k);
  std::vector<float> rwt((size_t)T * k), rsg((size_t)T);
  orc_moe_route(logits.data(), 0, T, E, k, E1, 1, shared ? 1 : 0, ri.data(), rwt.data(), rsg.data());
  double ew = 0;
  for (size_t i = 0; i < rwt.size(); i++) ew = std::max(ew, (double)std::fabs(rwt[i] - wt[i]));
  for (int t = 0; t < T && shared; t++) ew = std::max(ew, (double)std::fabs(rsg[t] - sg[t]));
  report(ri == idx && ew <= 1e-5, "encode_moe routing (indices bit-exact)" + tag, ew);
  // the checked tokens: all, or `check` spread evenly
  std::vector<int> tok;
  for (int i = 0; i < std::min(T, check); i++) tok.push_back(check >= T ? i : (int)((long)i * T / check));
  const int C = (int)tok.size();
  std::vector<uint16_t> xs((size_t)C * H), want((size_t)C * H), got((size_t)C * H);
  std::vector<int> si((size_t)C * k);
  std::vector<float> sw((size_t)C * k), ss((size_t)C);
  for (int i = 0; i < C; i++) {
    const int t = tok[i];
    memcpy(&xs[(size_t)i * H], &xn[(size_t)t * H], H * 2);
    memcpy(&want[(size_t)i * H], &x0[(size_t)t * H], H * 2);
    memcpy(&got[(size_t)i * H], &x1[(size_t)t * H], H * 2);
    for (int j = 0; j < k; j++) si[(size_t)i * k + j] = idx[(size_t)t * k + j], sw[(size_t)i * k + j] = wt[(size_t)t * k + j];
    ss[i] = sg[t];
  }
  // the shared expert as expert E gets the gathered GEMM's qmm rounding; through gemm() on the MLX layout, the decode
  // GEMV arithmetic up to 32 rows (ifd_gemm_w4) and qmm's above
  const int shared_qmv = shared == 2 && T <= 32 ? 1 : 0;
  if (dec)  // the decode GEMV arithmetic for every expert product
    orc_moe_decode(xs.data(), C, H, I, k, si.data(), sw.data(), ss.data(), L.egu.wq.data(), L.egu.s.data(),
                   L.egu.b.data(), L.edn.wq.data(), L.edn.s.data(), L.edn.b.data(), shared ? L.sgu.wq.data() : nullptr,
                   L.sgu.s.data(), L.sgu.b.data(), L.sdn.wq.data(), L.sdn.s.data(), L.sdn.b.data(), want.data(), 0);
  else
    orc_moe_experts(xs.data(), C, H, I, E, k, si.data(), sw.data(), ss.data(), L.egu.wq.data(), L.egu.s.data(),
                    L.egu.b.data(), L.edn.wq.data(), L.edn.s.data(), L.edn.b.data(),
                    shared ? L.sgu.wq.data() : nullptr, L.sgu.s.data(), L.sgu.b.data(), L.sdn.wq.data(),
                    L.sdn.s.data(), L.sdn.b.data(), shared_qmv, want.data(), 0, nthreads);
  std::vector<float> wf(want.size());
  for (size_t i = 0; i < want.size(); i++) wf[i] = bf2f(want[i]);
  // a chain of bf16 stages on both sides, compared end to end (the stages are checked one by one at the bar in
  // tests/test_gpu_moe.py)
  (void)bf16_err(got, wf, true);
  report(g_rel_rms <= 1e-2 && g_raw <= 5e-2 && g_ulp1 <= 0.05,
         "encode_moe x += moe(xn) on " + std::to_string(C) + " tokens (end to end)" + tag, g_raw);
}

void test_encode_moe_t64(std::mt19937& rng) {
  MoeLayer L(MoeGeo{512, 32, 4, 256}, rng);
  // 32-row tiles (R < 24 E) and 64-row tiles (T = 300: R = 1200), the shared expert folded in, through gemm(), or
  // absent; state allocated for more rows than the call
  run_moe_t64(L, 40, 40, 1, 1 << 30, 0, rng);
  run_moe_t64(L, 40, 100, 2, 1 << 30, 0, rng);
  run_moe_t64(L, 300, 300, 1, 1 << 30, 0, rng);
  run_moe_t64(L, 300, 300, 2, 1 << 30, 0, rng);
  run_moe_t64(L, 64, 64, 0, 1 << 30, 0, rng);
  // the decode route on the same stacks: the shared expert on its T64 copies, on the MLX layout, or absent
  run_moe_t64(L, 1, 1, 1, 1 << 30, 0, rng);
  run_moe_t64(L, 2, 8, 2, 1 << 30, 0, rng);
  run_moe_t64(L, 2, 2, 0, 1 << 30, 0, rng);
}

// The QA8 routes (QA8=1): gemm() of at least qa8_min rows on the qa8 int8 rows (MLX layout, unflipped and flipped, and
// the T64 copy; modes 0-2), one row fewer on the plain route; and encode_moe's sorted path on the gathered int8
// GEMMs, against the oracle's composition of the qa8 quantizer, the per-group integer products, SwiGLU and the
// combine (the shared expert through gemm_swiglu / gemm(): qmm below qa8_min rows, QA8 from there, where the T64
// copy's fused SwiGLU call gives way to gemm() + silu_mul).
void test_qa8(std::mt19937& rng) {
  setenv("QA8", "1", 1);
  {
    Config c;
    Qwen35 m(c, 300, 0, 64 << 20, 1024);
    Enc e;
    const int N = 384, K = 1024;
    const HostLinear h = make_linear(N, K, rng);
    HostLinear hf = h;
    orc_flip(hf.wq.data(), (int64_t)hf.wq.size(), 0x88888888u);
    QLinear W = device_linear(h), Wf = device_linear(hf), Wt = W;
    Wf.flipped = true;
    void* t = nullptr;
    hip_ok(hipMalloc(&t, ifd_t64_bytes(N, K, 1)), "t64");
    ok(ifd_pack_t64(W.wq.ptr<uint32_t>(), W.s.ptr<uint16_t>(), W.b.ptr<uint16_t>(), N, K, 0, 0, 1, t, e.stream),
       "pack_t64");
    Wt.t64 = BufRef(t);
    struct Case {
      const QLinear* W;
      const char* name;
      int M, mode;
    };
    for (const Case cs : {Case{&W, "MLX layout", 255, 0}, Case{&W, "MLX layout", 256, 0}, Case{&W, "MLX layout", 300, 0},
                          Case{&Wf, "MLX layout, flipped", 300, 0}, Case{&Wt, "T64", 255, 0}, Case{&Wt, "T64", 300, 0},
                          Case{&Wt, "T64", 300, 1}, Case{&Wt, "T64", 300, 2}}) {
      const int M = cs.M;
      const auto A = activations(M, K, rng);
      const auto C0 = activations(M, N, rng);
      const bool q8 = m.qa8_route(*cs.W, M);
      BufRef dA = upload(A), dC = cs.mode == 2 ? upload(std::vector<float>((size_t)M * N)) : upload(C0);
      m.gemm(e, dA, *cs.W, dC, M, cs.mode);
      // the plain route at 255 rows: qmm on the MLX layout; T64's stream-K or prefill tiles (qmm) at these shapes
      auto y = q8 ? ref_wxa8(A, M, K, h.wq.data(), h.s.data(), h.b.data(), N, 4, 2) : ref_gemm(A, h, M, false);
      const std::string tag = std::string("gemm ") + cs.name + " M=" + std::to_string(M) + " mode " +
                              std::to_string(cs.mode) + (q8 ? " (QA8 route)" : " (plain route)");
      if (cs.mode == 2) {
        const auto f = download<float>(dC, (size_t)M * N);
        double ss = 0, w = 0;
        for (size_t i = 0; i < y.size(); i++) ss += (double)y[i] * y[i], w = std::max(w, (double)std::fabs(f[i] - y[i]));
        const double err = w / std::sqrt(ss / y.size());
        report(err <= 1e-4 && q8 == (M >= 256), tag, err);
      } else {
        if (cs.mode == 1)
          for (size_t i = 0; i < y.size(); i++) y[i] += bf2f(C0[i]);
        const double err = bf16_err(download<uint16_t>(dC, (size_t)M * N), y, false);
        report(err <= 1e-2 && q8 == (M >= 256), tag, err);
      }
      (void)hipFree(dA.buf), (void)hipFree(dC.buf);
    }
    for (void* p : {W.wq.buf, W.s.buf, W.b.buf, Wf.wq.buf, Wf.s.buf, Wf.b.buf, t}) (void)hipFree(p);
  }
  // encode_moe: T = 40 with the shared expert on the MLX layout (qmm); T = 300 with its T64 copies (QA8 from 256
  // rows); T = 64 without one. The routed experts take the int8 gathered GEMMs whatever copies the stacks have.
  MoeLayer L(MoeGeo{512, 32, 4, 256}, rng);
  const int H = 512, E = 32, k = 4, I = 256;
  for (const int cs : {0, 1, 2}) {
    const int T = cs == 0 ? 40 : cs == 1 ? 300 : 64, R = T * k;
    const bool has_shared = cs != 2;
    Config c;
    c.hidden = H, c.experts = E, c.topk = k, c.moe_inter = I, c.eps = 1e-6f;
    Layer ly = L.ly;
    if (!has_shared) ly.gate_up = QLinear(), ly.down = QLinear(), ly.router.N = E;
    if (cs == 0) ly.gate_up.t64 = BufRef(), ly.down.t64 = BufRef();
    Qwen35 m(c, T, has_shared ? I : 0, 0);
    Enc e;
    const auto x0 = activations(T, H, rng);
    hip_ok(hipMemcpy(m.x.ptr<void>(), x0.data(), x0.size() * 2, hipMemcpyHostToDevice), "x");
    m.encode_moe(e, ly, T);
    const auto x1 = download<uint16_t>(m.x, (size_t)T * H);
    const auto xn = download<uint16_t>(m.xn, (size_t)T * H);
    const auto idx = download<int>(m.ridx, (size_t)T * k);
    const auto wt = download<float>(m.rw, (size_t)T * k);
    const auto sg = download<float>(m.rsg, (size_t)T);
    const std::string tag = " T=" + std::to_string(T) +
                            (has_shared ? (ly.gate_up.t64 ? " (shared expert, T64 copies)" : " (shared expert, MLX)")
                                        : " (no shared expert)");
    report(m.qa8g_route(ly, T) && !m.moe_decode_route(ly, T), "encode_moe takes the QA8 sorted route" + tag, 0);
    // shared expert: gemm() on xn, silu_mul, gemm() (QA8 from qa8_min rows, else qmm)
    std::vector<uint16_t> ys;
    if (has_shared) {
      const bool q8 = T >= m.qa8_min;
      auto dense = [&](const std::vector<uint16_t>& a, const HostLinear& w, int N, int K) {
        std::vector<float> y((size_t)T * N);
        if (q8) y = ref_wxa8(a, T, K, w.wq.data(), w.s.data(), w.b.data(), N, 4, 2);
        else orc_qmm(a.data(), K, w.wq.data(), w.s.data(), w.b.data(), N, K, 0, y.data(), T, 0);
        std::vector<uint16_t> o(y.size());
        for (size_t i = 0; i < y.size(); i++) o[i] = f2bf(y[i]);
        return o;
      };
      const auto gu = dense(xn, L.sgu, 2 * I, H);
      std::vector<uint16_t> act((size_t)T * I);
      orc_silu_mul(gu.data(), act.data(), I, T);
      ys = dense(act, L.sdn, H, I);
    }
    // routed experts: the token rows' qa8 form through perm; SwiGLU of the bf16 product; its rows' qa8 form
    std::vector<int> off(E + 1), perm(R), inv(R);
    orc_moe_dispatch(idx.data(), R, E, off.data(), perm.data(), inv.data());
    std::vector<int8_t> U((size_t)R * std::max(H, I));
    std::vector<float> XS((size_t)R * (std::max(H, I) / 64) * 2), y1((size_t)R * 2 * I), y2((size_t)R * H);
    orc_a8_quant(xn.data(), H, T, H, 2, U.data(), XS.data());
    orc_moe_gather_w4a8(U.data(), XS.data(), perm.data(), k, off.data(), L.egu.wq.data(), L.egu.s.data(),
                        L.egu.b.data(), E, 2 * I, H, y1.data(), 0);
    std::vector<uint16_t> egu(y1.size()), eact((size_t)R * I), edn(y2.size());
    for (size_t i = 0; i < y1.size(); i++) egu[i] = f2bf(y1[i]);
    orc_silu_mul(egu.data(), eact.data(), I, R);
    orc_a8_quant(eact.data(), I, R, I, 2, U.data(), XS.data());
    orc_moe_gather_w4a8(U.data(), XS.data(), nullptr, 1, off.data(), L.edn.wq.data(), L.edn.s.data(), L.edn.b.data(),
                        E, H, I, y2.data(), 0);
    for (size_t i = 0; i < y2.size(); i++) edn[i] = f2bf(y2[i]);
    std::vector<uint16_t> want = x0;
    orc_moe_combine(want.data(), edn.data(), wt.data(), has_shared ? ys.data() : nullptr, sg.data(), inv.data(), T, H,
                    k, 0);
    std::vector<float> wf(want.size());
    for (size_t i = 0; i < want.size(); i++) wf[i] = bf2f(want[i]);
    (void)bf16_err(x1, wf, true);
    report(g_rel_rms <= 1e-2 && g_raw <= 5e-2 && g_ulp1 <= 0.05, "encode_moe x += moe(xn) (QA8, end to end)" + tag,
           g_raw);
  }
  unsetenv("QA8");
}

// encode_moe with 8-bit routed experts on the sorted route (MLX-layout stacks, the reference's mlx_gqmm_b8 through
// gqmm at W.bits, qwen35.h:1835): x += MoE(xn) against the composition of the oracle's 8-bit qmm per routed row
// (gathered GEMM = each row's own expert product), SwiGLU, the shared expert's 4-bit qmm and the weighted combine.
void test_encode_moe_8bit_sorted(std::mt19937& rng) {
  const int H = 512, E = 16, k = 4, I = 128, T = 40, R = T * k;
  Config c;
  c.hidden = H, c.experts = E, c.topk = k, c.moe_inter = I, c.eps = 1e-6f;
  auto make8 = [&](int N, int K) {
    HostLinear h{N, K, std::vector<uint32_t>((size_t)N * K / 4), std::vector<uint16_t>((size_t)N * K / 64), {}};
    for (auto& w : h.wq) w = (uint32_t)rng();
    std::uniform_real_distribution<float> su(0.0003f, 0.0012f);
    h.b.resize(h.s.size());
    for (size_t i = 0; i < h.s.size(); i++) h.s[i] = f2bf(su(rng)), h.b[i] = f2bf(-128.f * bf2f(h.s[i]));
    return h;
  };
  const HostLinear egu = make8(E * 2 * I, H), edn = make8(E * H, I);
  const HostLinear sgu = make_linear(2 * I, H, rng), sdn = make_linear(H, I, rng);
  std::normal_distribution<float> nr(0.f, 0.02f);
  std::vector<uint16_t> router((size_t)(E + 1) * H), post((size_t)H);
  for (auto& v : router) v = f2bf(nr(rng));
  for (auto& v : post) v = f2bf(1.f);
  Layer ly;
  ly.post_norm = upload(post);
  ly.router.wq = upload(router);
  ly.router.E = 1, ly.router.N = E + 1, ly.router.K = H, ly.router.bits = 16;
  const QLinear gq = device_linear(egu), dq = device_linear(edn);
  ly.egu.wq = gq.wq, ly.egu.s = gq.s, ly.egu.b = gq.b, ly.egu.E = E, ly.egu.N = 2 * I, ly.egu.K = H, ly.egu.bits = 8;
  ly.edown.wq = dq.wq, ly.edown.s = dq.s, ly.edown.b = dq.b, ly.edown.E = E, ly.edown.N = H, ly.edown.K = I,
  ly.edown.bits = 8;
  ly.gate_up = device_linear(sgu), ly.down = device_linear(sdn);
  Qwen35 m(c, T, I, 0);
  Enc e;
  const auto x0 = activations(T, H, rng);
  hip_ok(hipMemcpy(m.x.ptr<void>(), x0.data(), x0.size() * 2, hipMemcpyHostToDevice), "x");
  m.encode_moe(e, ly, T);
  const auto x1 = download<uint16_t>(m.x, (size_t)T * H);
  const auto xn = download<uint16_t>(m.xn, (size_t)T * H);
  const auto idx = download<int>(m.ridx, (size_t)R);
  const auto wt = download<float>(m.rw, (size_t)R);
  const auto sg = download<float>(m.rsg, (size_t)T);
  const std::string tag = " T=40 E=16 k=4 (8-bit routed experts)";
  report(!m.moe_decode_route(ly, T) && !m.moe_t64_route(ly), "encode_moe takes the MLX sorted route" + tag, 0);
  // routed rows r = t k + j in row order: yd[r] = bf16(qmm8(act_r, down_e)), act_r = silu_mul(bf16(qmm8(xn_t, gu_e)))
  std::vector<uint16_t> yd((size_t)R * H), gu(2 * I), act(I);
  std::vector<float> y1(2 * I), y2(H);
  for (int r = 0; r < R; r++) {
    const int ex = idx[r], t = r / k;
    orc_qmm_b(&xn[(size_t)t * H], H, &egu.wq[(size_t)ex * 2 * I * H / 4], &egu.s[(size_t)ex * 2 * I * H / 64],
              &egu.b[(size_t)ex * 2 * I * H / 64], 2 * I, H, 8, 0, y1.data(), 1, 0);
    for (int i = 0; i < 2 * I; i++) gu[i] = f2bf(y1[i]);
    orc_silu_mul(gu.data(), act.data(), I, 1);
    orc_qmm_b(act.data(), I, &edn.wq[(size_t)ex * H * I / 4], &edn.s[(size_t)ex * H * I / 64],
              &edn.b[(size_t)ex * H * I / 64], H, I, 8, 0, y2.data(), 1, 0);
    for (int h = 0; h < H; h++) yd[(size_t)r * H + h] = f2bf(y2[h]);
  }
  // the shared expert through gemm() on the MLX layout: the decode GEMV arithmetic up to 32 rows, qmm's above
  std::vector<float> ys1((size_t)T * 2 * I), ys2((size_t)T * H);
  std::vector<uint16_t> sgu_o((size_t)T * 2 * I), sact((size_t)T * I), ys((size_t)T * H);
  (T <= 32 ? orc_qmv : orc_qmm)(xn.data(), H, sgu.wq.data(), sgu.s.data(), sgu.b.data(), 2 * I, H, 0, ys1.data(), T, 0);
  for (size_t i = 0; i < ys1.size(); i++) sgu_o[i] = f2bf(ys1[i]);
  orc_silu_mul(sgu_o.data(), sact.data(), I, T);
  (T <= 32 ? orc_qmv : orc_qmm)(sact.data(), I, sdn.wq.data(), sdn.s.data(), sdn.b.data(), H, I, 0, ys2.data(), T, 0);
  for (size_t i = 0; i < ys2.size(); i++) ys[i] = f2bf(ys2[i]);
  std::vector<int> inv(R);
  for (int r = 0; r < R; r++) inv[r] = r;
  std::vector<uint16_t> want = x0;
  orc_moe_combine(want.data(), yd.data(), wt.data(), ys.data(), sg.data(), inv.data(), T, H, k, 0);
  std::vector<float> wf(want.size());
  for (size_t i = 0; i < want.size(); i++) wf[i] = bf2f(want[i]);
  (void)bf16_err(x1, wf, true);
  report(g_rel_rms <= 1e-2 && g_raw <= 5e-2 && g_ulp1 <= 0.05, "encode_moe x += moe(xn) (end to end)" + tag, g_raw);
  for (void* p : {ly.post_norm.buf, ly.router.wq.buf, gq.wq.buf, gq.s.buf, gq.b.buf, dq.wq.buf, dq.s.buf, dq.b.buf,
                  ly.gate_up.wq.buf, ly.gate_up.s.buf, ly.gate_up.b.buf, ly.down.wq.buf, ly.down.s.buf, ly.down.b.buf})
    (void)hipFree(p);
}

template <class T>
bool same_as_device(const std::vector<T>& host, const BufRef& d) {
  return host.empty() || download<T>(d, host.size()) == host;
}

// The device loaders against the host loader (bit-exact uploads) and gemm() on what they loaded. The checkpoint holds
// mlp.gate_proj / mlp.up_proj (4-bit, fused N = 2 x 256, K = 1024, group 128 from config.json), a bf16 x.weight
// [128, 512] and a switch_mlp gate stack [4, 64, 256].
void test_load(const std::string& dir, std::mt19937& rng) {
  Checkpoint ck(dir);
  Gpu g;
  const std::vector<std::string> gu = {"mlp.gate_proj", "mlp.up_proj"};
  const HostQLinear hq = load_qlinear(ck, gu);
  const QLinear W = load_qlinear(g, ck, gu);
  report(W.N == hq.N && W.K == hq.K && W.bits == 4 && same_as_device(hq.wq, W.wq) && same_as_device(hq.s, W.s) &&
             same_as_device(hq.b, W.b) && (bool)W.t64,
         "load_qlinear upload (fused, group 128 expanded, T64 packed)", 0);
  const HostLinear h{hq.N, hq.K, hq.wq, hq.s, hq.b};
  Config c;
  Qwen35 m(c, 0, 0, 64 << 20);
  Enc e{g.stream};
  for (int M : {1, 128}) {
    const auto A = activations(M, h.K, rng);
    BufRef dA = upload(A), dC = upload(std::vector<uint16_t>((size_t)M * h.N));
    m.gemm(e, dA, W, dC, M, 0);
    const double err = bf16_err(download<uint16_t>(dC, (size_t)M * h.N), ref_gemm(A, h, M, M <= 64), false);
    report(err <= 1e-2, "gemm on the loaded layer M=" + std::to_string(M), err);
    (void)hipFree(dA.buf), (void)hipFree(dC.buf);
  }
  const HostQLinear h8 = load_qlinear_bf16(ck, {"x.weight"}, 8);
  const QLinear W8 = load_qlinear_bf16_q8(g, ck, {"x.weight"}, 8);
  report(W8.bits == 8 && (bool)W8.t64 && same_as_device(h8.wq, W8.wq) && same_as_device(h8.s, W8.s) &&
             same_as_device(h8.b, W8.b),
         "load_qlinear_bf16_q8 upload (8-bit, T64x8 packed)", 0);
  const HostQLinear h16 = load_qlinear(ck, {"x"});
  const QLinear W16 = load_qlinear(g, ck, {"x"});
  report(W16.bits == 16 && same_as_device(h16.w16, W16.wq), "load_qlinear bf16 passthrough upload", 0);
  const HostMoeW hm = load_moe(ck, {"mlp.switch_mlp.gate_proj"});
  const MoeW mw = load_moe(g, ck, {"mlp.switch_mlp.gate_proj"});
  report(mw.E == hm.E && mw.N == hm.N && mw.K == hm.K && same_as_device(hm.wq, mw.wq) && same_as_device(hm.s, mw.s) &&
             same_as_device(hm.b, mw.b),
         "load_moe upload", 0);
  g.release();
}

}  // namespace

int main(int argc, char** argv) {
  if (argc > 1 && std::string(argv[1]) == "--bad-bits") {
    Config c;
    Qwen35 m(c, 0, 0, 0);  // no state, no GPU call
    Enc e;
    QLinear W;
    W.bits = 16, W.N = 64, W.K = 64;
    m.gemm(e, BufRef(), W, BufRef(), 1, 0);
    printf("gemm returned for a 16-bit linear\n");
    return 0;
  }
  std::mt19937 rng(20251201);
  if (argc > 2 && std::string(argv[1]) == "--moe-c4") {
    // H 2048, 512 experts, top-10, I 512, the shared expert; the oracle on up to 96 tokens spread
    // over the batch, on 16 threads
    const int T = atoi(argv[2]);
    MoeLayer L(MoeGeo{2048, 512, 10, 512}, rng);
    run_moe_t64(L, T, T, 1, 96, 16, rng);
    printf(failures ? "%d FAILED\n" : "ALL OK\n", failures);
    return failures ? 1 : 0;
  }
  if (argc > 2 && std::string(argv[1]) == "--ckpt") {
    test_load(argv[2], rng);
    printf(failures ? "%d FAILED\n" : "ALL OK\n", failures);
    return failures ? 1 : 0;
  }
  {
    Config c;
    Qwen35 m(c, 256, 0, 64 << 20, 1024);  // int8 staging for the W4A8 route: up to 256 rows of K <= 1024
    Enc e;
    test_gemm(m, e, rng);
  }
  test_encode_moe(rng);
  test_encode_moe_t64(rng);
  test_encode_moe_8bit_sorted(rng);
  test_qa8(rng);
  printf(failures ? "%d FAILED\n" : "ALL OK\n", failures);
  return failures ? 1 : 0;
}
