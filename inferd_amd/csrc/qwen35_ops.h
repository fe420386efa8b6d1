// qwen35_ops.h — inferd's engine-facing operators of the quantized-matmul path, over the C ABI (inferd_qmm.h).
//
// Keeps the reference's C++ shapes so that engine code calling them needs no change:
//   void Qwen35::gemm(Enc& e, const BufRef& A, const QLinear& W, const BufRef& C, int M, int mode, bool defer)
//        (reference engine/src/qwen35.h:1465-1558)
//   void Qwen35::encode_moe(Enc& e, const Layer& ly, int T)                 (reference engine/src/qwen35.h:1869-1980)
// with BufRef (gpu.h:113-120), QLinear (weights.h:226-236), rows_of / kslice_of (weights.h:239-268), MoeW (moe.h:8-11)
// and the Layer members encode_moe reads (qwen35.h:311-316).
//
// What differs, by design:
//  - Enc is a HIP stream: work is enqueued in call order and nothing synchronises, as the reference encodes into one
//    serial compute encoder (gpu.h:122-163).
//  - QLinear may carry `t64`, the MI355X weight layout made once at load by ifd_pack_t64 (the role of the
//    reference's lane4 copy `lp` / `lsb`). When present (and K % 256 == 0) gemm() runs on it.
//  - The split-K reduce is never deferred: `defer` is accepted and has no effect.
// Errors keep the reference's behaviour: a message on stderr and exit(1) (qwen35.h:1469, 1477), here for every
// status the C ABI returns.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "inferd_qmm.h"

namespace inferd {

[[noreturn]] inline void die(const char* op, const char* msg) {
  fprintf(stderr, "%s: %s\n", op, msg);
  exit(1);
}
inline void ok(int status, const char* op) {
  if (status != IFD_OK) {
    fprintf(stderr, "%s: %s (%s)\n", op, ifd_status_str(status), ifd_last_error());
    exit(1);
  }
}
inline void hip_ok(hipError_t e, const char* op) {
  if (e != hipSuccess) {
    fprintf(stderr, "%s: %s\n", op, hipGetErrorString(e));
    exit(1);
  }
}

// A device buffer plus a byte offset: the unit every kernel argument is bound as.
struct BufRef {
  void* buf = nullptr;
  size_t off = 0;
  BufRef() = default;
  BufRef(void* b, size_t o = 0) : buf(b), off(o) {}
  BufRef at(size_t bytes) const { return BufRef(buf, off + bytes); }
  template <class T>
  T* ptr() const {
    return buf ? (T*)((char*)buf + off) : nullptr;
  }
  explicit operator bool() const { return buf != nullptr; }
};

// The ordered command stream operators encode into.
struct Enc {
  hipStream_t stream = nullptr;
};

// An MLX affine group-64 linear [N, K], 4 or 8 bits: wq uint32 [N][K bits/32], s/b bf16 [N][K/64] (rows ldk long in a
// K-slice).
struct QLinear {
  BufRef wq, s, b;
  BufRef t64;            // optional T64 copy (ifd_pack_t64), read by gemm() when present
  int ldk = 0;           // a K-slice view: the full matrix's row length; 0 = K
  bool flipped = false;  // codes stored q ^ 8 (4 bits) or q ^ 0x80 (8 bits) (ifd_flip_w4); readers flip back
  int N = 0, K = 0, bits = 4;
};

// Output rows [lo, lo + n) of a linear, sharing its buffers. A T64 copy interleaves the bands of every group, so a
// row view does not keep it (as the reference drops its lane4 copy off tile boundaries).
inline QLinear rows_of(const QLinear& q, int lo, int n) {
  QLinear r = q;
  r.t64 = BufRef();
  r.N = n;
  const size_t ld = q.ldk ? q.ldk : q.K;
  r.wq = q.wq.at((size_t)lo * ld * q.bits / 8);
  r.s = q.s.at((size_t)lo * (ld / 64) * 2);
  r.b = q.b.at((size_t)lo * (ld / 64) * 2);
  return r;
}

// Input columns [k0, k0 + kn) (multiples of 64). The T64 copy is group-major, so a K-slice of it is the tiles from
// group k0 / 64 on: kept when k0 and kn are multiples of 256 (whole T64 GEMM chunks).
inline QLinear kslice_of(const QLinear& q, int k0, int kn) {
  QLinear r = q;
  r.ldk = q.ldk ? q.ldk : q.K;
  r.K = kn;
  r.wq = q.wq.at((size_t)k0 * q.bits / 8);
  r.s = q.s.at((size_t)k0 / 64 * 2);
  r.b = q.b.at((size_t)k0 / 64 * 2);
  if (q.t64 && k0 % 256 == 0 && kn % 256 == 0)
    r.t64 = q.t64.at((size_t)(k0 / 64) * ((q.N + 31) / 32) * 1152);
  else
    r.t64 = BufRef();
  return r;
}

// A stacked affine matrix [E, N, K] (bits 4), or a bf16 matrix (bits 16: wq holds [E * N][K] bf16).
struct MoeW {
  BufRef wq, s, b;
  int E = 0, N = 0, K = 0, bits = 0;
};

// The members of a decoder layer the MoE block reads.
struct Layer {
  BufRef post_norm;          // rmsnorm weight bf16 [hidden]
  QLinear gate_up, down;     // shared expert: [2 Is, H] and [H, Is]
  MoeW router, egu, edown;   // router bf16 [E (+1 shared gate row), H]; experts [E, 2I, H] and [E, H, I]
};

struct Config {
  int hidden = 0, experts = 0, topk = 0, moe_inter = 0;
  float eps = 1e-6f;
  int router_gemm_min = 0;   // T at or above which router logits are rounded to bf16 (0 = never)
};

// The model-owned state the two operators use: hidden state x [T][H] (encode_moe adds the block's output into it),
// its normalised copy xn, routing outputs and every scratch buffer, allocated once for up to max_rows tokens
// (the reference allocates them with the model, qwen35.h:394-407, 520-600).
struct Qwen35 {
  Config cfg;
  int max_rows = 0;
  BufRef x, xn;               // bf16 [max_rows][H]
  BufRef rlog;                // router logits fp32 [max_rows][E + 1] (bf16 when rounded)
  BufRef ridx, rw, rsg;       // int [T][k], float [T][k], float [T]
  BufRef proj, act, sh_out;   // shared expert: bf16 [T][2 Is], [T][Is], [T][H]
  BufRef moffs, mperm, minv, mtiles, mntiles;  // dispatch
  BufRef eact, edown_out;     // routed experts: bf16 [R][I], [R][H]
  BufRef splitk;              // gemm()'s split-K partials and the dispatch workspace
  size_t splitk_bytes = 0;

  // shared_inter: the shared expert's intermediate size (0: none). gemm_scratch: bytes for gemm() calls made outside
  // encode_moe (the largest ifd_gemm_w4_workspace / ifd_gemm_t64_workspace of the model's shapes).
  Qwen35(const Config& c, int max_rows_, int shared_inter, size_t gemm_scratch) : cfg(c), max_rows(max_rows_) {
    const int H = c.hidden, E = c.experts, k = c.topk, I = c.moe_inter, R = max_rows * k;
    size_t need = gemm_scratch;
    if (max_rows > 0 && E > 0) {
      need = std::max(need, ifd_moe_dispatch_workspace(R, E));
      need = std::max(need, ifd_moe_decode_workspace(std::min(max_rows, 8), H, I, E, k));
      if (shared_inter > 0) {
        need = std::max(need, ifd_gemm_w4_workspace(max_rows, 2 * shared_inter, H));
        need = std::max(need, ifd_gemm_w4_workspace(max_rows, H, shared_inter));
        need = std::max(need, ifd_gemm_t64_workspace(max_rows, 2 * shared_inter, H));
        need = std::max(need, ifd_gemm_t64_swiglu_workspace(max_rows, 2 * shared_inter, H));
        need = std::max(need, ifd_gemm_t64_workspace(max_rows, H, shared_inter));
      }
      x = alloc((size_t)max_rows * H * 2);
      xn = alloc((size_t)max_rows * H * 2);
      rlog = alloc((size_t)max_rows * (E + 1) * 4);
      ridx = alloc((size_t)R * 4);
      rw = alloc((size_t)R * 4);
      rsg = alloc((size_t)max_rows * 4);
      if (shared_inter > 0) {
        proj = alloc((size_t)max_rows * 2 * shared_inter * 2);
        act = alloc((size_t)max_rows * shared_inter * 2);
        sh_out = alloc((size_t)max_rows * H * 2);
      }
      moffs = alloc((size_t)(E + 1) * 4);
      mperm = alloc((size_t)R * 4);
      minv = alloc((size_t)R * 4);
      mtiles = alloc((size_t)ifd_moe_tiles_max(R, E) * 2 * 4);
      mntiles = alloc(4);
      eact = alloc((size_t)R * I * 2);
      edown_out = alloc((size_t)R * H * 2);
    }
    if (need) {
      splitk = alloc(need);
      hip_ok(hipMemset(splitk.buf, 0, need), "Qwen35");  // the workspace's leading counters start at zero
    }
    splitk_bytes = need;
  }
  ~Qwen35() {
    for (void* p : {x.buf, xn.buf, rlog.buf, ridx.buf, rw.buf, rsg.buf, proj.buf, act.buf, sh_out.buf, moffs.buf,
                    mperm.buf, minv.buf, mtiles.buf, mntiles.buf, eact.buf, edown_out.buf, splitk.buf})
      if (p) (void)hipFree(p);
  }
  Qwen35(const Qwen35&) = delete;
  Qwen35& operator=(const Qwen35&) = delete;

  // H [M][N/2] = SwiGLU of A . W^T for a [gate | up] linear: one fused call on T64 weights, else the reference's
  // gemm into proj + silu_mul (qwen35.h:1910-1912).
  void gemm_swiglu(Enc& e, const BufRef& A, const QLinear& W, const BufRef& H, int M) {
    if (W.bits == 4 && W.t64 && W.K % 256 == 0 && W.N % 16 == 0) {
      const size_t need = ifd_gemm_t64_swiglu_workspace(M, W.N, W.K);
      if (need > splitk_bytes) die("gemm_swiglu", "split-K scratch smaller than this shape needs");
      ok(ifd_gemm_t64_swiglu(A.ptr<void>(), W.K, W.t64.ptr<void>(), W.N, W.K, H.ptr<void>(), W.N / 2, M,
                             splitk.ptr<void>(), splitk_bytes, e.stream),
         "gemm_swiglu");
      return;
    }
    gemm(e, A, W, proj, M, 0);
    ok(ifd_silu_mul(proj.ptr<void>(), H.ptr<void>(), W.N / 2, M, e.stream), "gemm_swiglu");
  }

  // C (mode) = A . W^T for M rows: mode 0 writes bf16, 1 adds into bf16 C, 2 writes fp32. A is [M][K] (row stride
  // K), C [M][N] (row stride N).
  void gemm(Enc& e, const BufRef& A, const QLinear& W, const BufRef& C, int M, int mode, bool defer = false) {
    (void)defer;
    if (W.bits == 8) {  // the reference's qmv8 / 8-bit qmm routes (qwen35.h:1520-1558)
      const size_t need = ifd_gemm_w8_workspace(M, W.N, W.K);
      if (need > splitk_bytes) die("gemm", "split-K scratch smaller than this shape needs");
      ok(ifd_gemm_w8(A.ptr<void>(), W.K, W.wq.ptr<uint32_t>(), W.s.ptr<uint16_t>(), W.b.ptr<uint16_t>(), W.N, W.K,
                     W.ldk, W.flipped ? 0x80808080u : 0u, C.ptr<void>(), W.N, M, mode, splitk.ptr<void>(),
                     splitk_bytes, e.stream),
         "gemm");
      return;
    }
    if (W.bits != 4) {
      fprintf(stderr, "gemm: %d-bit weights are outside this path (4- and 8-bit affine only)\n", W.bits);
      exit(1);
    }
    if (W.t64 && W.K % 256 == 0) {
      const size_t need = ifd_gemm_t64_workspace(M, W.N, W.K);
      if (need > splitk_bytes) die("gemm", "split-K scratch smaller than this shape needs");
      ok(ifd_gemm_t64(A.ptr<void>(), W.K, W.t64.ptr<void>(), W.N, W.K, C.ptr<void>(), W.N, M, mode, splitk.ptr<void>(),
                      splitk_bytes, e.stream),
         "gemm");
      return;
    }
    const size_t need = ifd_gemm_w4_workspace(M, W.N, W.K);
    if (need > splitk_bytes) die("gemm", "split-K scratch smaller than this shape needs");
    ok(ifd_gemm_w4(A.ptr<void>(), W.K, W.wq.ptr<uint32_t>(), W.s.ptr<uint16_t>(), W.b.ptr<uint16_t>(), W.N, W.K,
                   W.ldk, W.flipped ? 0x88888888u : 0u, C.ptr<void>(), W.N, M, mode, splitk.ptr<void>(), splitk_bytes,
                   e.stream),
       "gemm");
  }

  // The MoE block on the hidden state x [T][H]: xn = rmsnorm(x, post_norm); shared expert; router; top-k softmax
  // routing; dispatch by expert; gathered gate/up with SwiGLU; gathered down; x = bf16(x + bf16(weighted sum +
  // sg * shared)) (reference sorted path, qwen35.h:1909-1980).
  void encode_moe(Enc& e, const Layer& ly, int T) {
    const int H = cfg.hidden, E = cfg.experts, k = cfg.topk, I = cfg.moe_inter, R = T * k;
    if (T > max_rows) die("encode_moe", "more rows than the state was allocated for");
    if (ly.router.bits != 16) die("encode_moe", "the router must be bf16 (bits 16)");
    if (ly.egu.bits != 4 || ly.edown.bits != 4) die("encode_moe", "routed experts must be 4-bit affine");
    if (ly.router.K != H || ly.router.E * ly.router.N < E || ly.egu.E != E || ly.egu.N != 2 * I || ly.egu.K != H ||
        ly.edown.E != E || ly.edown.N != H || ly.edown.K != I)
      die("encode_moe", "layer shapes do not match the config");
    if (T == 0) return;
    const int E1 = ly.router.E * ly.router.N;  // E, or E + 1 with the shared expert's gate row
    ok(ifd_rmsnorm(x.ptr<void>(), H, ly.post_norm.ptr<void>(), xn.ptr<void>(), H, T, H, cfg.eps, e.stream),
       "encode_moe");
    // up to 8 tokens: the decode MoE (the reference's moe2 route, qwen35.h:1823-1829, 1876-1908), each distinct expert
    // read once; it needs the shared expert (if any) unflipped 4-bit with the routed experts' intermediate size
    const bool has_shared = ly.gate_up.N > 0;
    const bool shared_fits = !has_shared || (ly.gate_up.bits == 4 && ly.down.bits == 4 && ly.gate_up.N == 2 * I &&
                                             ly.gate_up.K == H && ly.down.N == H && ly.down.K == I &&
                                             !ly.gate_up.flipped && !ly.down.flipped && !ly.gate_up.ldk &&
                                             !ly.down.ldk);
    if (T <= 8 && k <= 16 && E <= 512 && H % 512 == 0 && I % 64 == 0 && E1 <= E + 1 && shared_fits) {
      const size_t need = ifd_moe_decode_workspace(T, H, I, E, k);
      if (need > splitk_bytes) die("encode_moe", "scratch smaller than the decode MoE needs");
      ok(ifd_moe_decode(xn.ptr<void>(), T, H, ly.router.wq.ptr<void>(), E, k, 1, E1 > E ? 1 : 0,
                        ly.egu.wq.ptr<uint32_t>(), ly.egu.s.ptr<uint16_t>(), ly.egu.b.ptr<uint16_t>(),
                        ly.edown.wq.ptr<uint32_t>(), ly.edown.s.ptr<uint16_t>(), ly.edown.b.ptr<uint16_t>(), I,
                        has_shared ? ly.gate_up.wq.ptr<uint32_t>() : nullptr,
                        has_shared ? ly.gate_up.s.ptr<uint16_t>() : nullptr,
                        has_shared ? ly.gate_up.b.ptr<uint16_t>() : nullptr,
                        has_shared ? ly.down.wq.ptr<uint32_t>() : nullptr,
                        has_shared ? ly.down.s.ptr<uint16_t>() : nullptr,
                        has_shared ? ly.down.b.ptr<uint16_t>() : nullptr, x.ptr<void>(), 0, ridx.ptr<int>(),
                        rw.ptr<float>(), rsg.ptr<float>(), rlog.ptr<float>(), splitk.ptr<void>(), splitk_bytes,
                        e.stream),
         "encode_moe");
      return;
    }
    // shared expert -> sh_out
    const bool shared = ly.gate_up.N > 0;
    if (shared) {
      gemm_swiglu(e, xn, ly.gate_up, act, T);
      gemm(e, act, ly.down, sh_out, T, 0);
    }
    // router
    const int lbf = cfg.router_gemm_min > 0 && T >= cfg.router_gemm_min;
    ok(ifd_moe_router_logits(xn.ptr<void>(), ly.router.wq.ptr<void>(), T, H, E1, lbf, rlog.ptr<void>(), e.stream),
       "encode_moe");
    ok(ifd_moe_route(rlog.ptr<void>(), lbf, T, E, k, E1, 1, E1 > E ? 1 : 0, ridx.ptr<int>(), rw.ptr<float>(),
                     rsg.ptr<float>(), e.stream),
       "encode_moe");
    // routed experts, rows sorted by expert
    ok(ifd_moe_dispatch(ridx.ptr<int>(), R, E, moffs.ptr<int>(), mperm.ptr<int>(), minv.ptr<int>(), mtiles.ptr<int>(),
                        mntiles.ptr<int>(), splitk.ptr<void>(), splitk_bytes, e.stream),
       "encode_moe");
    const int mt = ifd_moe_tiles_max(R, E);
    ok(ifd_moe_gather_qmm(xn.ptr<void>(), mperm.ptr<int>(), k, moffs.ptr<int>(), mtiles.ptr<int>(), mntiles.ptr<int>(),
                          mt, ly.egu.wq.ptr<uint32_t>(), ly.egu.s.ptr<uint16_t>(), ly.egu.b.ptr<uint16_t>(), E, 2 * I,
                          H, 1, eact.ptr<void>(), R, e.stream),
       "encode_moe");
    ok(ifd_moe_gather_qmm(eact.ptr<void>(), nullptr, 1, moffs.ptr<int>(), mtiles.ptr<int>(), mntiles.ptr<int>(), mt,
                          ly.edown.wq.ptr<uint32_t>(), ly.edown.s.ptr<uint16_t>(), ly.edown.b.ptr<uint16_t>(), E, H, I,
                          0, edown_out.ptr<void>(), R, e.stream),
       "encode_moe");
    ok(ifd_moe_combine(x.ptr<void>(), edown_out.ptr<void>(), rw.ptr<float>(), shared ? sh_out.ptr<void>() : nullptr,
                       rsg.ptr<float>(), minv.ptr<int>(), T, H, k, 0, e.stream),
       "encode_moe");
  }

 private:
  static BufRef alloc(size_t bytes) {
    void* p = nullptr;
    hip_ok(hipMalloc(&p, std::max<size_t>(bytes, 256)), "Qwen35 state");
    return BufRef(p);
  }
};

}  // namespace inferd
