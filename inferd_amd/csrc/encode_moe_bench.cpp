// encode_moe_bench — times the drop-in operator Qwen35::encode_moe (qwen35_ops.h; reference engine/src/qwen35.h:1869)
// at BASELINE config 4's geometry: hidden 2048, 512 experts, top-10 softmax routing renormalised over the picks, one
// always-on shared expert (no gate row: its weight is 1), SwiGLU experts of width 512, 4-bit group-64 affine weights
// (q ~ U{0..15}, s ~ U(0.005, 0.02) rounded to bf16, b = -8 s), a bf16 N(0, 0.02) router. The layer is held the way
// the device loader leaves it: the MLX-layout stacks plus their T64 copies (ckpt_dev.h upload_moe / upload_qlinear),
// so the sorted route runs the T64 gathered GEMMs with the shared expert as expert E (below 128 routed rows, T <= 12,
// the per-row route on the same copies); `--mlx` drops the copies and times the MLX-layout routes instead. Two weight copies alternate (1.85 GB, over 3x the 256 MB Infinity Cache).
//
//   encode_moe_bench [--mlx] [--graph] T...    one JSON line: {"T16": {"us": ..., "tok_s": ...}, ...}
//
// --graph: each weight copy's encode_moe call is captured once in a HIP graph and the timed calls replay it (the
// operator issues no allocation, memset or synchronisation, so the call is capturable): the GPU time of the
// operator without the host's per-launch cost.
//
// Timing: HIP events on the operator's stream around each of `iters` calls, after warm calls that keep the GPU loaded
// for 30 ms (its clock settles in that time). Every call starts from the same hidden state: encode_moe adds its
// output into x, and a drifting x would concentrate the routing on a few experts; the device-to-device copy that
// restores x sits between the event pairs, outside the timed intervals.
#include <chrono>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "qwen35_ops.h"

using namespace inferd;

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint64_t next64() {  // splitmix64
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
float uni() { return (float)((next64() >> 40) * (1.0 / 16777216.0)); }
float gauss() {  // sum of four uniforms, variance-normalised: enough for timing inputs
  return (uni() + uni() + uni() + uni() - 2.f) * 1.7320508f;
}
uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void* dalloc(size_t bytes) {
  void* p = nullptr;
  hip_ok(hipMalloc(&p, bytes), "bench alloc");
  return p;
}

// one [wq | s | b] buffer of `rows` rows of K inputs (4-bit), filled with the config's distribution
struct Affine {
  BufRef wq, s, b;
};
Affine make_affine(size_t rows, int K) {
  const size_t nw = rows * K / 8, ng = rows * K / 64;
  char* buf = (char*)dalloc(nw * 4 + 2 * ng * 2);
  std::vector<uint32_t> w(nw);
  for (auto& v : w) v = (uint32_t)next64();
  std::vector<uint16_t> s(ng), b(ng);
  for (size_t i = 0; i < ng; i++) s[i] = f2bf(0.005f + 0.015f * uni()), b[i] = f2bf(-8.f * bf2f(s[i]));
  hip_ok(hipMemcpy(buf, w.data(), nw * 4, hipMemcpyHostToDevice), "bench upload");
  hip_ok(hipMemcpy(buf + nw * 4, s.data(), ng * 2, hipMemcpyHostToDevice), "bench upload");
  hip_ok(hipMemcpy(buf + nw * 4 + ng * 2, b.data(), ng * 2, hipMemcpyHostToDevice), "bench upload");
  return Affine{BufRef(buf, 0), BufRef(buf, nw * 4), BufRef(buf, nw * 4 + ng * 2)};
}
BufRef pack(const Affine& a, int N, int K, int E) {
  void* t = dalloc(ifd_t64_bytes(N, K, E));
  ok(ifd_pack_t64(a.wq.ptr<uint32_t>(), a.s.ptr<uint16_t>(), a.b.ptr<uint16_t>(), N, K, 0, 0u, E, t, nullptr),
     "pack_t64");
  return BufRef(t);
}

}  // namespace

int main(int argc, char** argv) {
  bool mlx = false, graph = false;
  std::vector<int> Ts;
  for (int i = 1; i < argc; i++) {
    if (std::string(argv[i]) == "--mlx") mlx = true;
    else if (std::string(argv[i]) == "--graph") graph = true;
    else Ts.push_back(atoi(argv[i]));
  }
  if (Ts.empty()) Ts = {16, 128, 2048};
  const int H = 2048, E = 512, k = 10, I = 512, ncp = 2;
  int Tmax = 0;
  for (int T : Ts) Tmax = std::max(Tmax, T);
  Config c;
  c.hidden = H, c.experts = E, c.topk = k, c.moe_inter = I, c.eps = 1e-6f;
  c.router_gemm_min = 64;  // bf16 router logits from 64 rows (qwen35.h:1919-1929)

  std::vector<Layer> layers(ncp);
  std::vector<uint16_t> router((size_t)E * H), post(H);
  for (auto& v : router) v = f2bf(0.02f * gauss());
  for (auto& v : post) v = f2bf(1.f);
  BufRef drouter(dalloc(router.size() * 2)), dpost(dalloc(post.size() * 2));
  hip_ok(hipMemcpy(drouter.buf, router.data(), router.size() * 2, hipMemcpyHostToDevice), "bench upload");
  hip_ok(hipMemcpy(dpost.buf, post.data(), post.size() * 2, hipMemcpyHostToDevice), "bench upload");
  for (auto& ly : layers) {
    ly.post_norm = dpost;
    ly.router.wq = drouter;
    ly.router.E = 1, ly.router.N = E, ly.router.K = H, ly.router.bits = 16;
    const Affine gu = make_affine((size_t)E * 2 * I, H), dn = make_affine((size_t)E * H, I);
    ly.egu.wq = gu.wq, ly.egu.s = gu.s, ly.egu.b = gu.b, ly.egu.E = E, ly.egu.N = 2 * I, ly.egu.K = H, ly.egu.bits = 4;
    ly.edown.wq = dn.wq, ly.edown.s = dn.s, ly.edown.b = dn.b, ly.edown.E = E, ly.edown.N = H, ly.edown.K = I,
    ly.edown.bits = 4;
    const Affine sgu = make_affine(2 * I, H), sdn = make_affine(H, I);
    ly.gate_up.wq = sgu.wq, ly.gate_up.s = sgu.s, ly.gate_up.b = sgu.b, ly.gate_up.N = 2 * I, ly.gate_up.K = H;
    ly.down.wq = sdn.wq, ly.down.s = sdn.s, ly.down.b = sdn.b, ly.down.N = H, ly.down.K = I;
    if (!mlx) {
      ly.egu.t64 = pack(gu, 2 * I, H, E), ly.edown.t64 = pack(dn, H, I, E);
      ly.gate_up.t64 = pack(sgu, 2 * I, H, 1), ly.down.t64 = pack(sdn, H, I, 1);
    }
  }
  hip_ok(hipDeviceSynchronize(), "bench setup");

  Qwen35 m(c, Tmax, I, 0);
  hipStream_t st;
  hip_ok(hipStreamCreate(&st), "bench stream");
  Enc e{st};
  std::vector<uint16_t> x0((size_t)Tmax * H);
  for (auto& v : x0) v = f2bf(gauss());
  constexpr int iters = 20;
  std::vector<hipEvent_t> ev(2 * iters);
  for (auto& v : ev) hip_ok(hipEventCreate(&v), "event");
  void* xsave = dalloc((size_t)Tmax * H * 2);
  hip_ok(hipMemcpy(xsave, x0.data(), x0.size() * 2, hipMemcpyHostToDevice), "bench x");
  std::string out = "{";
  for (size_t ti = 0; ti < Ts.size(); ti++) {
    const int T = Ts[ti];
    const size_t xb = (size_t)T * H * 2;
    std::function<void(int)> moe_fn;
    auto call = [&](int i) {
      hip_ok(hipMemcpyAsync(m.x.ptr<void>(), xsave, xb, hipMemcpyDeviceToDevice, st), "bench x");
      moe_fn(i);
    };
    // with --graph: one captured encode_moe per weight copy, replayed by moe_fn
    std::vector<hipGraphExec_t> gx;
    if (graph) {
      for (int c = 0; c < ncp; c++) {
        m.encode_moe(e, layers[c], T);  // first calls outside capture (one-time kernel attributes)
        hip_ok(hipStreamSynchronize(st), "bench warm");
        hipGraph_t g;
        hip_ok(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal), "capture");
        m.encode_moe(e, layers[c], T);
        hip_ok(hipStreamEndCapture(st, &g), "capture");
        hipGraphExec_t x;
        hip_ok(hipGraphInstantiate(&x, g, nullptr, nullptr, 0), "instantiate");
        gx.push_back(x);
      }
    }
    moe_fn = [&](int i) {
      if (graph) hip_ok(hipGraphLaunch(gx[i % ncp], st), "replay");
      else m.encode_moe(e, layers[i % ncp], T);
    };
    int i = 0;
    for (; i < 3; i++) call(i);
    hip_ok(hipStreamSynchronize(st), "bench warm");
    const auto t0 = std::chrono::steady_clock::now();
    while (std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() < 30.0) {
      for (int r = 0; r < 4; r++, i++) call(i);
      hip_ok(hipStreamSynchronize(st), "bench warm");
    }
    for (int r = 0; r < iters; r++, i++) {
      hip_ok(hipMemcpyAsync(m.x.ptr<void>(), xsave, xb, hipMemcpyDeviceToDevice, st), "bench x");
      hip_ok(hipEventRecord(ev[2 * r], st), "event");
      moe_fn(i);
      hip_ok(hipEventRecord(ev[2 * r + 1], st), "event");
    }
    hip_ok(hipStreamSynchronize(st), "event");
    double ms = 0;
    for (int r = 0; r < iters; r++) {
      float t = 0;
      hip_ok(hipEventElapsedTime(&t, ev[2 * r], ev[2 * r + 1]), "event");
      ms += t;
    }
    const double us = ms * 1e3 / iters;
    for (auto x : gx) hip_ok(hipGraphExecDestroy(x), "graph");
    // the route the operator took at this T, and whether it ran on the T64 copies
    const Layer& l0 = layers[0];
    const bool dec = m.moe_decode_route(l0, T), rows = m.moe_rows_route(l0, T);
    const bool on_t64 = dec ? m.moe_decode_t64(l0, T) : rows ? (bool)l0.egu.t64 : m.moe_t64_route(l0);
    char buf[160];
    snprintf(buf, sizeof buf, "%s\"T%d\": {\"us\": %.2f, \"tok_s\": %.1f, \"route\": \"%s\", \"t64\": %s}",
             ti ? ", " : "", T, us, T / (us * 1e-6), dec ? "decode" : rows ? "per-row" : "sorted",
             on_t64 ? "true" : "false");
    out += buf;
  }
  out += "}";
  printf("%s\n", out.c_str());
  return 0;
}
