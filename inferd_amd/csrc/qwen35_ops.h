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
//  - bf16 weights (bits 16) are outside this path: gemm() reports it and exits, as for any route it lacks.
// The W4A8 route and its fused producers follow the reference: flipped 4- and 8-bit weights for qmv_max < M <
// w4a8_max take the int8 GEMM (w4a8_route, qwen35.h:1576; w4a8, :1323-1365), and rmsnorm_for / silu_mul_for write the next
// GEMM's int8 rows when it takes that route (a8_ready, :1560-1561, 1982-2001, 2874-2876). encode_moe routes an 8-bit
// router as the reference does (moe_router8 for the decode launches, the per-row qmv8 logits otherwise,
// :1878-1882, 1930-1941).
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
  BufRef t64;            // optional T64 copy (ifd_pack_t64; 8 bits: T64x8, ifd_pack_t64x8), read by gemm() when present
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
// group k0 / 64 on: kept when k0 and kn are multiples of 256 (whole T64 GEMM chunks; any 64-group for T64x8).
inline QLinear kslice_of(const QLinear& q, int k0, int kn) {
  QLinear r = q;
  r.ldk = q.ldk ? q.ldk : q.K;
  r.K = kn;
  r.wq = q.wq.at((size_t)k0 * q.bits / 8);
  r.s = q.s.at((size_t)k0 / 64 * 2);
  r.b = q.b.at((size_t)k0 / 64 * 2);
  const int kq = q.bits == 8 ? 64 : 256, tile = q.bits == 8 ? 2176 : 1152;
  if (q.t64 && k0 % kq == 0 && kn % kq == 0)
    r.t64 = q.t64.at((size_t)(k0 / 64) * ((q.N + 31) / 32) * tile);
  else
    r.t64 = BufRef();
  return r;
}

// A stacked affine matrix [E, N, K] (bits 4 or 8), or a bf16 matrix (bits 16: wq holds [E * N][K] bf16). A 4-bit stack
// may carry `t64`, its E experts packed by ifd_pack_t64 (the MI355X layout, made once at load); encode_moe's sorted
// route reads it when both expert stacks have one.
struct MoeW {
  BufRef wq, s, b;
  BufRef t64;
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

inline int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

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
  BufRef moffs, mperm, minv, mtiles, mntiles;  // dispatch (room for the shared expert as expert E: E + 2 offsets,
                                               // R + T rows)
  BufRef eact, edown_out;     // routed experts (and the shared expert's rows after them): bf16 [R + T][I], [R + T][H]
  BufRef splitk;              // gemm()'s split-K partials and the dispatch workspace
  size_t splitk_bytes = 0;
  BufRef a8u, a8x;            // int8 rows [max_rows][a8_k] and their (sx, sx sum xq) per 64-group, fp32
  int a8_k = 0;

  // Routing thresholds of the reference (qwen35.h:1049, 1055, 1575; the same environment variables): up to
  // qmv_max rows the decode GEMV, W4A8 for flipped 4-bit weights below w4a8_max rows; fuse_a8 0 off, 1 silu_mul_a8,
  // 3 also rmsnorm_a8; moe_sort_min: routed rows from which the MoE sorts by expert (fewer: per-row expert
  // products, qwen35.h:1830).
  int qmv_max = env_int("QMV_MAX", 2), w4a8_max = env_int("W4A8_MAX", 256);
  bool use_w4a8 = env_int("W4A8", 1) != 0;
  int fuse_a8 = env_int("FUSE_A8", 3), moe_sort_min = env_int("MOE_SORT_MIN", 128);
  // The next GEMM's int8 activations are already in a8u / a8x (written by rmsnorm_for or silu_mul_for).
  bool a8_ready = false;
  // flipped 4-bit (W4A8) or 8-bit (W8A8: the same kernel with 8-bit codes, qwen35.h:1352) weights
  bool w4a8_route(const QLinear& W, int M) const {
    return use_w4a8 && (W.bits == 4 || W.bits == 8) && W.flipped && !W.ldk && M > qmv_max && M < w4a8_max &&
           W.K % 64 == 0;
  }
  // QA8 (qwen35.h:1164-1206, 1847-1868): steps of at least qa8_min rows run on per-(row, 64-group) int8 activations
  // from the qa8 quantizer (xq = clamp(rint(x 127 / amax), -127, 127), ifd_a8_quant form 2) times the 4-bit codes:
  // the dense GEMMs, and (moe_qa8, from moe_qa8_min tokens) the sorted MoE's gathered expert GEMMs. The reference
  // turns it on by itself only on GPUs with neural accelerators (qa8_auto, :1084-1092) and leaves it off on the
  // others, as this build does unless QA8=1 (the same variables as the reference): then the results take the
  // arithmetic of such a run. The MoE's int8 rows need staging the constructor allocates only when QA8 is on.
  int qa8_on = env_int("QA8", 0), qa8_min = env_int("QA8_MIN", 256);
  int moe_qa8 = env_int("MOE_QA8", 1), moe_qa8_min = env_int("MOE_QA8_MIN", 9);
  BufRef q8u, q8x;  // the MoE's int8 rows [max_rows k][max(H, I)] and their (sx, sx sum xq) per 64-group
  bool qa8_route(const QLinear& W, int M) const {
    return qa8_on > 0 && W.bits == 4 && !W.ldk && W.K % 256 == 0 && W.N % 32 == 0 && M >= qa8_min && M <= max_rows &&
           !a8_ready && W.K <= a8_k;
  }
  bool qa8g_route(const Layer& ly, int T) const {
    return moe_qa8 && qa8_on > 0 && T >= moe_qa8_min && ly.egu.bits == 4 && ly.edown.bits == 4 &&
           cfg.hidden % 256 == 0 && cfg.moe_inter % 256 == 0 && cfg.experts <= 1024;
  }

  // shared_inter: the shared expert's intermediate size (0: none). gemm_scratch: bytes for gemm() calls made outside
  // encode_moe (the largest workspace query of the model's shapes over every row count). a8_k: the longest K of a
  // W4A8 GEMM (0: the hidden size or shared_inter, whichever is larger).
  Qwen35(const Config& c, int max_rows_, int shared_inter, size_t gemm_scratch, int a8_k_ = 0)
      : cfg(c), max_rows(max_rows_) {
    const int H = c.hidden, E = c.experts, k = c.topk, I = c.moe_inter, R = max_rows * k;
    a8_k = a8_k_ > 0 ? a8_k_ : std::max(H, shared_inter);
    size_t need = gemm_scratch;
    if (max_rows > 0 && E > 0) {
      need = std::max(need, ifd_moe_dispatch_workspace(R, E));
      need = std::max(need, ifd_moe_decode_workspace(std::min(max_rows, 16), H, I, E, k));
      need = std::max(need, ifd_moe_gather_qmm_t64_workspace(64));  // the balanced schedule's pieces (either height)
      // a workspace size is not monotone in the row count (each route sizes its own), so take every T a call may
      // pass: 1 .. max_rows
      for (int T = 1; T <= max_rows; T++) {
        need = std::max(need, ifd_moe_dispatch_workspace(T * k, E));
        if (T <= 16) need = std::max(need, ifd_moe_decode_workspace(T, H, I, E, k));
        if (T <= 16) need = std::max(need, ifd_moe_decode_t64_workspace(T, H, I, E, k));
        need = std::max(need, ifd_moe_rows_t64_workspace(T, H, I, E, k));
        need = std::max(need, ifd_gemm_w8_workspace(T, E + 1, H));  // an 8-bit router's logits
        if (shared_inter > 0) {
          need = std::max(need, ifd_gemm_w4_workspace(T, 2 * shared_inter, H));
          need = std::max(need, ifd_gemm_w4_workspace(T, H, shared_inter));
          need = std::max(need, ifd_gemm_t64_workspace(T, 2 * shared_inter, H));
          need = std::max(need, ifd_gemm_t64_swiglu_workspace(T, 2 * shared_inter, H));
          need = std::max(need, ifd_gemm_t64_workspace(T, H, shared_inter));
          need = std::max(need, ifd_qmm_w4a8_workspace(T, 2 * shared_inter, H));
          need = std::max(need, ifd_qmm_w4a8_workspace(T, H, shared_inter));
          need = std::max(need, ifd_gemm_t64_w4a8_workspace(T, 2 * shared_inter, H));
          need = std::max(need, ifd_gemm_t64_w4a8_workspace(T, H, shared_inter));
          need = std::max(need, ifd_gemm_t64x8_workspace(T, 2 * shared_inter, H));  // an 8-bit shared expert
          need = std::max(need, ifd_gemm_t64x8_workspace(T, H, shared_inter));
        }
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
      const int Rt = R + max_rows;  // the T64 route appends the shared expert's rows as expert E
      moffs = alloc((size_t)(E + 2) * 4);
      mperm = alloc((size_t)Rt * 4);
      minv = alloc((size_t)R * 4);
      mtiles = alloc((size_t)std::max(ifd_moe_tiles_max(R, E), ifd_moe_tiles_max(Rt, E + 1)) * 2 * 4);
      mntiles = alloc(4);
      eact = alloc((size_t)Rt * I * 2);
      edown_out = alloc((size_t)Rt * H * 2);
    }
    if (max_rows > 0 && a8_k > 0) {
      a8u = alloc((size_t)max_rows * a8_k);
      a8x = alloc((size_t)max_rows * (a8_k / 64) * 2 * 4);
    }
    if (qa8_on > 0 && max_rows > 0 && E > 0) {
      const size_t rows = (size_t)max_rows * k, w = std::max(H, I);
      q8u = alloc(rows * w);
      q8x = alloc(rows * (w / 64) * 2 * 4);
    }
    if (need) {
      splitk = alloc(need);
      hip_ok(hipMemset(splitk.buf, 0, need), "Qwen35");  // the workspace's leading counters start at zero
    }
    splitk_bytes = need;
  }
  ~Qwen35() {
    for (void* p : {x.buf, xn.buf, rlog.buf, ridx.buf, rw.buf, rsg.buf, proj.buf, act.buf, sh_out.buf, moffs.buf,
                    mperm.buf, minv.buf, mtiles.buf, mntiles.buf, eact.buf, edown_out.buf, splitk.buf, a8u.buf,
                    a8x.buf, q8u.buf, q8x.buf})
      if (p) (void)hipFree(p);
  }
  Qwen35(const Qwen35&) = delete;
  Qwen35& operator=(const Qwen35&) = delete;

  // H [M][N/2] = SwiGLU of A . W^T for a [gate | up] linear: one fused call on T64 weights, else the reference's
  // gemm into proj + silu_mul (qwen35.h:1910-1912).
  void gemm_swiglu(Enc& e, const BufRef& A, const QLinear& W, const BufRef& H, int M) {
    if (W.bits == 4 && W.t64 && W.K % 256 == 0 && W.N % 16 == 0 && !w4a8_route(W, M) && !qa8_route(W, M) &&
        !a8_ready) {
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
    if (W.ldk && a8_ready) die("gemm", "K-slice view off the qmm path");  // qwen35.h:1469
    if (qa8_route(W, M)) {  // qwen35.h:1472
      qa8(e, A, W, C, M, mode);
      return;
    }
    if (w4a8_route(W, M)) {
      w4a8(e, A, W, C, M, mode);
      return;
    }
    if (a8_ready) die("gemm", "a8_ready with a non-W4A8 GEMM");  // qwen35.h:1477
    if (W.bits == 8) {  // the reference's qmv8 / 8-bit qmm routes (qwen35.h:1520-1558)
      // On the T64x8 copy: the qmv8 arithmetic up to 16 rows, the 8-bit qmm rounding above, which is the
      // reference's route past qmv_max (= 2 by default, qwen35.h:1049, 1525-1558).
      if (W.t64) {
        const size_t need = ifd_gemm_t64x8_workspace(M, W.N, W.K);
        if (need > splitk_bytes) die("gemm", "split-K scratch smaller than this shape needs");
        ok(ifd_gemm_t64x8(A.ptr<void>(), W.K, W.t64.ptr<void>(), W.N, W.K, C.ptr<void>(), W.N, M, mode,
                          splitk.ptr<void>(), splitk_bytes, e.stream),
           "gemm");
        return;
      }
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

  // The reference's W4A8 GEMM (qwen35.h:1323-1365): per-group int8 activations (a8_quant, unless a fused producer
  // wrote them) times the flipped 4- or 8-bit codes on the integer path. A 4-bit layer's T64 copy (always the
  // unflipped codes) runs it on the T64 kernels with the same per-group scales.
  void w4a8(Enc& e, const BufRef& A, const QLinear& W, const BufRef& C, int M, int mode) {
    if (M > max_rows || W.K > a8_k) die("gemm", "W4A8 rows past the int8 staging buffers (max_rows, a8_k)");
    if (!a8_ready)
      ok(ifd_a8_quant(A.ptr<void>(), W.K, M, W.K, 0, a8u.ptr<int8_t>(), a8x.ptr<float>(), e.stream), "gemm");
    a8_ready = false;
    if (W.bits == 4 && W.t64 && W.K % 256 == 0) {
      const size_t need = ifd_gemm_t64_w4a8_workspace(M, W.N, W.K);
      if (need > splitk_bytes) die("gemm", "split-K scratch smaller than this shape needs");
      ok(ifd_gemm_t64_w4a8(a8u.ptr<int8_t>(), a8x.ptr<float>(), 0, W.t64.ptr<void>(), W.N, W.K, C.ptr<void>(), W.N, M,
                           mode, splitk.ptr<void>(), splitk_bytes, e.stream),
         "gemm");
      return;
    }
    const bool w8 = W.bits == 8;
    const size_t need = w8 ? ifd_qmm_w8a8_workspace(M, W.N, W.K) : ifd_qmm_w4a8_workspace(M, W.N, W.K);
    if (need > splitk_bytes) die("gemm", "split-K scratch smaller than this shape needs");
    ok((w8 ? ifd_qmm_w8a8 : ifd_qmm_w4a8)(a8u.ptr<int8_t>(), a8x.ptr<float>(), 0, W.wq.ptr<uint32_t>(),
                                          W.s.ptr<uint16_t>(), W.b.ptr<uint16_t>(), W.N, W.K, 0,
                                          w8 ? 0x80808080u : 0x88888888u, C.ptr<void>(), W.N, M, mode,
                                          splitk.ptr<void>(), splitk_bytes, e.stream),
       "gemm");
  }

  // The reference's QA8 GEMM (qwen35.h:1187-1206): the rows' qa8 int8 form, then per group y += s sx P + b (sx sum xq)
  // on the 4-bit codes (unflipped: a flipped layer's MLX codes are read through xr; its T64 copy holds them
  // unflipped), on the T64 kernels when the layer has its copy.
  void qa8(Enc& e, const BufRef& A, const QLinear& W, const BufRef& C, int M, int mode) {
    ok(ifd_a8_quant(A.ptr<void>(), W.K, M, W.K, 2, a8u.ptr<int8_t>(), a8x.ptr<float>(), e.stream), "gemm");
    if (W.t64) {
      const size_t need = ifd_gemm_t64_w4a8_workspace(M, W.N, W.K);
      if (need > splitk_bytes) die("gemm", "split-K scratch smaller than this shape needs");
      ok(ifd_gemm_t64_w4a8(a8u.ptr<int8_t>(), a8x.ptr<float>(), 0, W.t64.ptr<void>(), W.N, W.K, C.ptr<void>(), W.N, M,
                           mode, splitk.ptr<void>(), splitk_bytes, e.stream),
         "gemm");
      return;
    }
    const size_t need = ifd_qmm_w4a8_workspace(M, W.N, W.K);
    if (need > splitk_bytes) die("gemm", "split-K scratch smaller than this shape needs");
    ok(ifd_qmm_w4a8(a8u.ptr<int8_t>(), a8x.ptr<float>(), 0, W.wq.ptr<uint32_t>(), W.s.ptr<uint16_t>(),
                    W.b.ptr<uint16_t>(), W.N, W.K, 0, W.flipped ? 0x88888888u : 0u, C.ptr<void>(), W.N, M, mode,
                    splitk.ptr<void>(), splitk_bytes, e.stream),
       "gemm");
  }

  // rmsnorm of rows [rows][D] into out, fused with the W4A8 activation quantization when `next` (the GEMM that reads
  // out) takes that route (reference rmsnorm_for, qwen35.h:1982-2001).
  void rmsnorm_for(Enc& e, const BufRef& in, const BufRef& w, const BufRef& out, int rows, int D, const QLinear& next) {
    if (fuse_a8 < 3 || !w4a8_route(next, rows) || D % 64 || D > a8_k || rows > max_rows) {
      ok(ifd_rmsnorm(in.ptr<void>(), D, w.ptr<void>(), out.ptr<void>(), D, rows, D, cfg.eps, e.stream), "rmsnorm_for");
      return;
    }
    ok(ifd_rmsnorm_a8(in.ptr<void>(), D, w.ptr<void>(), out.ptr<void>(), D, rows, D, cfg.eps, 0, a8u.ptr<int8_t>(),
                      a8x.ptr<float>(), e.stream),
       "rmsnorm_for");
    a8_ready = true;
  }

  // h = silu_mul(gu) for the MLP's down projection `down` (gu [rows][2 I] -> act [rows][I]); when down takes the
  // W4A8 route, its int8 rows instead (act is not written; reference qwen35.h:2868-2878).
  void silu_mul_for(Enc& e, const BufRef& gu, const BufRef& act, int I, int rows, const QLinear& down) {
    if (fuse_a8 && w4a8_route(down, rows) && I % 64 == 0 && I <= a8_k && rows <= max_rows) {
      ok(ifd_silu_mul_a8(gu.ptr<void>(), I, rows, 0, a8u.ptr<int8_t>(), a8x.ptr<float>(), e.stream), "silu_mul_for");
      a8_ready = true;
      return;
    }
    ok(ifd_silu_mul(gu.ptr<void>(), act.ptr<void>(), I, rows, e.stream), "silu_mul_for");
  }

  // The MoE routes encode_moe takes for T tokens (qwen35.h:1876, 1947, 1956): the four decode launches (the
  // reference's moe2, :1823-1829: up to min(MOE_V2, 8) tokens with an 8-bit router; here also up to qmv_max tokens
  // with any router, where the per-row route computes the same values: its shared expert goes through gemm()'s
  // decode GEMV at those rows); below moe_sort_min routed rows otherwise the per-row expert products
  // (moe_rows_route); else rows sorted by expert.
  int moe_v2 = env_int("MOE_V2", 8);
  bool moe_decode_route(const Layer& ly, int T) const {
    const int H = cfg.hidden, E = cfg.experts, k = cfg.topk, I = cfg.moe_inter;
    const int E1 = ly.router.E * ly.router.N;
    const bool has_shared = ly.gate_up.N > 0;
    // a 4- or 8-bit shared expert (moe_gu2_4_4 / moe_gu2_4_8, moe.metal:465-487)
    const bool shared_fits = !has_shared || ((ly.gate_up.bits == 4 || ly.gate_up.bits == 8) &&
                                             ly.down.bits == ly.gate_up.bits && ly.gate_up.N == 2 * I &&
                                             ly.gate_up.K == H && ly.down.N == H && ly.down.K == I &&
                                             !ly.gate_up.flipped && !ly.down.flipped && !ly.gate_up.ldk &&
                                             !ly.down.ldk);
    // 4-bit routed experts (moe_gu2 / moe_dn2 are built for EB = 4 only, moe.metal:465-548)
    return (T <= qmv_max || (T <= std::min(moe_v2, 8) && ly.router.bits == 8)) && k <= 16 && E <= 512 &&
           H % 512 == 0 && I % 64 == 0 && E1 <= E + 1 && shared_fits && ly.egu.bits == 4 && ly.edown.bits == 4;
  }
  // The reference's per-row expert products (moe_qmv4 + moe_silu_mul + moe_combine, qwen35.h:1947-1955) on
  // ifd_moe_rows, with the shared expert through gemm() (:1909-1914): any T below moe_sort_min routed rows that the
  // decode launches do not take, 4-bit routed experts of the decode kernels' shapes (ifd_moe_rows_t64 on the routed
  // experts' T64 copies when they exist).
  bool moe_rows_route(const Layer& ly, int T) const {
    const int H = cfg.hidden, E = cfg.experts, k = cfg.topk, I = cfg.moe_inter;
    return !moe_decode_route(ly, T) && T * k < moe_sort_min && k <= 16 && E <= 512 && H % 512 == 0 && I % 64 == 0 &&
           ly.egu.bits == 4 && ly.edown.bits == 4;
  }

  // On the decode route, the T64 copies of the routed experts (and of a 4-bit shared expert, if any) are streamed
  // in place of the MLX-layout stacks: the same per-row qmv4 arithmetic
  bool moe_decode_t64(const Layer& ly, int T) const {
    const bool has_shared = ly.gate_up.N > 0;
    return moe_decode_route(ly, T) && T <= 16 && ly.egu.t64 && ly.edown.t64 &&
           (!has_shared || (ly.gate_up.bits == 4 && ly.gate_up.t64 && ly.down.t64));
  }
  // The sorted route on the experts' T64 stacks (ifd_moe_gather_qmm_t64: the same bf16(s q + b) dequant and fp32 sums
  // as the MLX-layout gathered GEMM): both stacks 4-bit with T64 copies, H and I multiples of 256.
  bool moe_t64_route(const Layer& ly) const {
    return ly.egu.t64 && ly.edown.t64 && ly.egu.bits == 4 && ly.edown.bits == 4 && cfg.hidden % 256 == 0 &&
           cfg.moe_inter % 256 == 0;
  }
  // On that route the shared expert runs as expert E of the same two launches when it is a 4-bit linear pair of the
  // routed experts' width with T64 copies that gemm() would also run in bf16 (not the W4A8 route): its rows get the
  // qmm rounding gemm() gives them past qmv_max rows (qwen35.h:1525-1558, 1909-1914).
  // On the per-row route over the routed experts' T64 copies, the shared expert runs as one more slot of those
  // launches (the decode GEMV's qmv4 arithmetic, which gemm() on its T64 copies also computes up to 16 rows) when it
  // is a 4-bit linear pair of the routed experts' width with T64 copies that gemm() would run in bf16.
  bool shared_in_rows_t64(const Layer& ly, int T) const {
    const int H = cfg.hidden, I = cfg.moe_inter;
    const QLinear &gu = ly.gate_up, &dn = ly.down;
    return moe_rows_route(ly, T) && ly.egu.t64 && ly.edown.t64 && T <= 16 && gu.N > 0 && gu.bits == 4 &&
           dn.bits == 4 && gu.t64 && dn.t64 && gu.N == 2 * I && gu.K == H && dn.N == H && dn.K == I && !gu.ldk &&
           !dn.ldk && !gu.flipped && !dn.flipped && !w4a8_route(gu, T) && !w4a8_route(dn, T) && !qa8_route(gu, T) &&
           !qa8_route(dn, T);
  }
  bool shared_as_expert(const Layer& ly, int T) const {
    const int H = cfg.hidden, I = cfg.moe_inter;
    const QLinear &gu = ly.gate_up, &dn = ly.down;
    return moe_t64_route(ly) && gu.N > 0 && gu.bits == 4 && dn.bits == 4 && gu.t64 && dn.t64 && gu.N == 2 * I &&
           gu.K == H && dn.N == H && dn.K == I && !gu.ldk && !dn.ldk && T > qmv_max && !w4a8_route(gu, T) &&
           !w4a8_route(dn, T) && !qa8_route(gu, T) && !qa8_route(dn, T);
  }

  // The MoE block on the hidden state x [T][H]: xn = rmsnorm(x, post_norm); shared expert; router; top-k softmax
  // routing; dispatch by expert; gathered gate/up with SwiGLU; gathered down; x = bf16(x + bf16(weighted sum +
  // sg * shared)) (reference sorted path, qwen35.h:1909-1980).
  void encode_moe(Enc& e, const Layer& ly, int T) {
    const int H = cfg.hidden, E = cfg.experts, k = cfg.topk, I = cfg.moe_inter, R = T * k;
    if (T > max_rows) die("encode_moe", "more rows than the state was allocated for");
    if (ly.router.bits != 16 && !(ly.router.bits == 8 && ly.router.E == 1))
      die("encode_moe", "the router must be bf16 (bits 16) or one 8-bit matrix (bits 8)");
    if ((ly.egu.bits != 4 && ly.egu.bits != 8) || (ly.edown.bits != 4 && ly.edown.bits != 8))
      die("encode_moe", "routed experts must be 4- or 8-bit affine");
    if (ly.router.K != H || ly.router.E * ly.router.N < E || ly.egu.E != E || ly.egu.N != 2 * I || ly.egu.K != H ||
        ly.edown.E != E || ly.edown.N != H || ly.edown.K != I)
      die("encode_moe", "layer shapes do not match the config");
    if (T == 0) return;
    const int E1 = ly.router.E * ly.router.N;  // E, or E + 1 with the shared expert's gate row
    const bool has_shared = ly.gate_up.N > 0;
    if (has_shared) rmsnorm_for(e, x, ly.post_norm, xn, T, H, ly.gate_up);
    else ok(ifd_rmsnorm(x.ptr<void>(), H, ly.post_norm.ptr<void>(), xn.ptr<void>(), H, T, H, cfg.eps, e.stream), "encode_moe");
    // An 8-bit router's logits (fp32, per group s sum q x + b sum x: the reference's moe_router8 / moe_qmv8f; bf16
    // from router_gemm_min rows, as its quantized GEMM rounds them) come from the 8-bit GEMM.
    const bool r8 = ly.router.bits == 8;
    const int lbf = cfg.router_gemm_min > 0 && T >= cfg.router_gemm_min;
    // fp32 logits keep the per-row qmv8 arithmetic for every T: the 8-bit GEMM computes it up to 32 rows, so the
    // rows go 32 at a time (each row's logits are the same whatever the chunk)
    auto router8_logits = [&](int bf16_out) {
      const int step = bf16_out ? T : 32;
      for (int r0 = 0; r0 < T; r0 += step) {
        const int rows = std::min(step, T - r0);
        const size_t need = ifd_gemm_w8_workspace(rows, E1, H);
        if (need > splitk_bytes) die("encode_moe", "scratch smaller than the 8-bit router needs");
        ok(ifd_gemm_w8(xn.at((size_t)r0 * H * 2).ptr<void>(), H, ly.router.wq.ptr<uint32_t>(),
                       ly.router.s.ptr<uint16_t>(), ly.router.b.ptr<uint16_t>(), E1, H, 0, 0u,
                       rlog.at((size_t)r0 * E1 * (bf16_out ? 2 : 4)).ptr<void>(), E1, rows, bf16_out ? 0 : 2,
                       splitk.ptr<void>(), splitk_bytes, e.stream),
           "encode_moe");
      }
    };
    // the decode MoE (the reference's moe2 route), each distinct expert read once; it needs the shared expert (if
    // any) unflipped, 4- or 8-bit, with the routed experts' intermediate size. The per-row route over the routed
    // experts' T64 copies, with the shared expert (if any) as one more slot, is the same computation (every routed
    // and shared product in the qmv4 arithmetic), so up to 8 tokens it takes the same launches, router included
    // (from 9 tokens the router kernel's last block routes two tokens per wave, and the separate routing is faster).
    const bool rows_dec = moe_rows_route(ly, T) && T <= 8 && ly.egu.t64 && ly.edown.t64 &&
                          (!has_shared || shared_in_rows_t64(ly, T));
    if (moe_decode_route(ly, T) || rows_dec) {
      a8_ready = false;  // the norm's int8 rows (if it made them) are not the next GEMM's input (qwen35.h:1906)
      const size_t need = ifd_moe_decode_workspace(T, H, I, E, k);
      if (need > splitk_bytes) die("encode_moe", "scratch smaller than the decode MoE needs");
      const int sbits = has_shared ? ly.gate_up.bits : 4;
      if (moe_decode_t64(ly, T) || rows_dec) {
        if (ifd_moe_decode_t64_workspace(T, H, I, E, k) > splitk_bytes)
          die("encode_moe", "scratch smaller than the decode MoE needs");
        if (r8) router8_logits(0);
        ok(ifd_moe_decode_t64(xn.ptr<void>(), T, H, r8 ? nullptr : ly.router.wq.ptr<void>(),
                              r8 ? rlog.ptr<float>() : nullptr, E, k, 1, E1 > E ? 1 : 0, ly.egu.t64.ptr<void>(),
                              ly.edown.t64.ptr<void>(), I, has_shared ? ly.gate_up.t64.ptr<void>() : nullptr,
                              has_shared ? ly.down.t64.ptr<void>() : nullptr, x.ptr<void>(), 0, ridx.ptr<int>(),
                              rw.ptr<float>(), rsg.ptr<float>(), r8 ? nullptr : rlog.ptr<float>(), splitk.ptr<void>(),
                              splitk_bytes, e.stream),
           "encode_moe");
        return;
      }
      if (r8) {
        router8_logits(0);
        ok(ifd_moe_decode_logits_ex(rlog.ptr<float>(), xn.ptr<void>(), T, H, E, k, 1, E1 > E ? 1 : 0,
                                 ly.egu.wq.ptr<uint32_t>(), ly.egu.s.ptr<uint16_t>(), ly.egu.b.ptr<uint16_t>(),
                                 ly.edown.wq.ptr<uint32_t>(), ly.edown.s.ptr<uint16_t>(), ly.edown.b.ptr<uint16_t>(), I,
                                 has_shared ? ly.gate_up.wq.ptr<uint32_t>() : nullptr,
                                 has_shared ? ly.gate_up.s.ptr<uint16_t>() : nullptr,
                                 has_shared ? ly.gate_up.b.ptr<uint16_t>() : nullptr,
                                 has_shared ? ly.down.wq.ptr<uint32_t>() : nullptr,
                                 has_shared ? ly.down.s.ptr<uint16_t>() : nullptr,
                                 has_shared ? ly.down.b.ptr<uint16_t>() : nullptr, sbits, x.ptr<void>(), 0,
                                 ridx.ptr<int>(), rw.ptr<float>(), rsg.ptr<float>(), splitk.ptr<void>(), splitk_bytes,
                                 e.stream),
           "encode_moe");
        return;
      }
      ok(ifd_moe_decode_ex(xn.ptr<void>(), T, H, ly.router.wq.ptr<void>(), E, k, 1, E1 > E ? 1 : 0,
                        ly.egu.wq.ptr<uint32_t>(), ly.egu.s.ptr<uint16_t>(), ly.egu.b.ptr<uint16_t>(),
                        ly.edown.wq.ptr<uint32_t>(), ly.edown.s.ptr<uint16_t>(), ly.edown.b.ptr<uint16_t>(), I,
                        has_shared ? ly.gate_up.wq.ptr<uint32_t>() : nullptr,
                        has_shared ? ly.gate_up.s.ptr<uint16_t>() : nullptr,
                        has_shared ? ly.gate_up.b.ptr<uint16_t>() : nullptr,
                        has_shared ? ly.down.wq.ptr<uint32_t>() : nullptr,
                        has_shared ? ly.down.s.ptr<uint16_t>() : nullptr,
                        has_shared ? ly.down.b.ptr<uint16_t>() : nullptr, sbits, x.ptr<void>(), 0, ridx.ptr<int>(),
                        rw.ptr<float>(), rsg.ptr<float>(), rlog.ptr<float>(), splitk.ptr<void>(), splitk_bytes,
                        e.stream),
         "encode_moe");
      return;
    }
    // shared expert -> sh_out (its gate/up may read the norm's int8 rows; the SwiGLU feeds the down GEMM in bf16,
    // qwen35.h:1910-1914), unless it runs as expert E of the T64 launches
    const bool rows = moe_rows_route(ly, T), q8 = !rows && qa8g_route(ly, T);
    if (q8 && !q8u.buf) die("encode_moe", "the MoE's QA8 route needs its int8 staging: construct with QA8=1");
    const bool t64 = !rows && !q8 && moe_t64_route(ly), fold = t64 && shared_as_expert(ly, T);
    // on the per-row route over T64 copies the shared expert can run as one more slot of the same launches
    const bool srow = shared_in_rows_t64(ly, T);
    const bool shared = has_shared && !fold && !srow;
    if (shared) {
      gemm_swiglu(e, xn, ly.gate_up, act, T);
      a8_ready = false;
      gemm(e, act, ly.down, sh_out, T, 0);
    }
    a8_ready = false;
    // router
    if (r8) router8_logits(lbf);
    else
      ok(ifd_moe_router_logits(xn.ptr<void>(), ly.router.wq.ptr<void>(), T, H, E1, lbf, rlog.ptr<void>(), e.stream),
         "encode_moe");
    ok(ifd_moe_route(rlog.ptr<void>(), lbf, T, E, k, E1, 1, E1 > E ? 1 : 0, ridx.ptr<int>(), rw.ptr<float>(),
                     rsg.ptr<float>(), e.stream),
       "encode_moe");
    if (rows && ly.egu.t64 && ly.edown.t64) {  // the same on the routed experts' T64 copies
      if (ifd_moe_rows_t64_workspace(T, H, I, E, k) > splitk_bytes)
        die("encode_moe", "scratch smaller than the per-row MoE needs");
      ok(ifd_moe_rows_t64(xn.ptr<void>(), T, H, E, k, ridx.ptr<int>(), rw.ptr<float>(), rsg.ptr<float>(),
                          ly.egu.t64.ptr<void>(), ly.edown.t64.ptr<void>(), I,
                          srow ? ly.gate_up.t64.ptr<void>() : nullptr, srow ? ly.down.t64.ptr<void>() : nullptr,
                          shared ? sh_out.ptr<void>() : nullptr, x.ptr<void>(), 0, splitk.ptr<void>(), splitk_bytes,
                          e.stream),
         "encode_moe");
      return;
    }
    if (rows) {  // a few routed rows: one decode-GEMV product per (token, expert) row, the shared rows in the combine
      const size_t need = ifd_moe_rows_workspace(T, H, I, E, k);
      if (need > splitk_bytes) die("encode_moe", "scratch smaller than the per-row MoE needs");
      ok(ifd_moe_rows(xn.ptr<void>(), T, H, E, k, ridx.ptr<int>(), rw.ptr<float>(), rsg.ptr<float>(),
                      ly.egu.wq.ptr<uint32_t>(), ly.egu.s.ptr<uint16_t>(), ly.egu.b.ptr<uint16_t>(),
                      ly.edown.wq.ptr<uint32_t>(), ly.edown.s.ptr<uint16_t>(), ly.edown.b.ptr<uint16_t>(), I,
                      shared ? sh_out.ptr<void>() : nullptr, x.ptr<void>(), 0, splitk.ptr<void>(), splitk_bytes,
                      e.stream),
         "encode_moe");
      return;
    }
    if (t64) {
      // routed experts on their T64 stacks, rows sorted by expert in tiles of tr rows; with `fold`, tokens 0..T-1
      // follow as expert E's segment (the shared expert) and its output rows R..R+T-1 are the combine's ys
      const int tr = ifd_moe_t64_tile_rows(R, E), Rt = R + (fold ? T : 0);
      ok(ifd_moe_dispatch_ex(ridx.ptr<int>(), R, E, k, tr, fold ? T : 0, moffs.ptr<int>(), mperm.ptr<int>(),
                             minv.ptr<int>(), mtiles.ptr<int>(), mntiles.ptr<int>(), splitk.ptr<void>(), splitk_bytes,
                             e.stream),
         "encode_moe");
      // both products on the balanced schedule, their pieces in the scratch (its counter header kept zero)
      ok(ifd_moe_gather_qmm_t64(xn.ptr<void>(), H, mperm.ptr<int>(), k, moffs.ptr<int>(), mtiles.ptr<int>(),
                                mntiles.ptr<int>(), tr, ly.egu.t64.ptr<void>(),
                                fold ? ly.gate_up.t64.ptr<void>() : nullptr, E, 2 * I, H, 1, eact.ptr<void>(), I, Rt,
                                splitk.ptr<void>(), splitk_bytes, e.stream),
         "encode_moe");
      ok(ifd_moe_gather_qmm_t64(eact.ptr<void>(), I, nullptr, 1, moffs.ptr<int>(), mtiles.ptr<int>(),
                                mntiles.ptr<int>(), tr, ly.edown.t64.ptr<void>(),
                                fold ? ly.down.t64.ptr<void>() : nullptr, E, H, I, 0, edown_out.ptr<void>(), H, Rt,
                                splitk.ptr<void>(), splitk_bytes, e.stream),
         "encode_moe");
      const void* ys = fold ? edown_out.at((size_t)R * H * 2).ptr<void>() : shared ? sh_out.ptr<void>() : nullptr;
      ok(ifd_moe_combine(x.ptr<void>(), edown_out.ptr<void>(), rw.ptr<float>(), ys, rsg.ptr<float>(), minv.ptr<int>(),
                         T, H, k, 0, e.stream),
         "encode_moe");
      return;
    }
    // routed experts, rows sorted by expert
    ok(ifd_moe_dispatch(ridx.ptr<int>(), R, E, moffs.ptr<int>(), mperm.ptr<int>(), minv.ptr<int>(), mtiles.ptr<int>(),
                        mntiles.ptr<int>(), splitk.ptr<void>(), splitk_bytes, e.stream),
       "encode_moe");
    const int mt = ifd_moe_tiles_max(R, E);
    if (q8) {
      // QA8's gathered GEMMs (qa8g, qwen35.h:1960-1966): the token rows' int8 form read through perm for gate/up
      // (SwiGLU fused: silu_mul of the bf16 product, as moe_silu_mul), then the sorted SwiGLU rows' int8 form for down
      ok(ifd_a8_quant(xn.ptr<void>(), H, T, H, 2, q8u.ptr<int8_t>(), q8x.ptr<float>(), e.stream), "encode_moe");
      ok(ifd_moe_gather_qmm_a8(q8u.ptr<int8_t>(), q8x.ptr<float>(), mperm.ptr<int>(), k, moffs.ptr<int>(),
                               mtiles.ptr<int>(), mntiles.ptr<int>(), mt, ly.egu.wq.ptr<uint32_t>(),
                               ly.egu.s.ptr<uint16_t>(), ly.egu.b.ptr<uint16_t>(), E, 2 * I, H, 1, eact.ptr<void>(), R,
                               e.stream),
         "encode_moe");
      ok(ifd_a8_quant(eact.ptr<void>(), I, R, I, 2, q8u.ptr<int8_t>(), q8x.ptr<float>(), e.stream), "encode_moe");
      ok(ifd_moe_gather_qmm_a8(q8u.ptr<int8_t>(), q8x.ptr<float>(), nullptr, 1, moffs.ptr<int>(), mtiles.ptr<int>(),
                               mntiles.ptr<int>(), mt, ly.edown.wq.ptr<uint32_t>(), ly.edown.s.ptr<uint16_t>(),
                               ly.edown.b.ptr<uint16_t>(), E, H, I, 0, edown_out.ptr<void>(), R, e.stream),
         "encode_moe");
      ok(ifd_moe_combine(x.ptr<void>(), edown_out.ptr<void>(), rw.ptr<float>(), shared ? sh_out.ptr<void>() : nullptr,
                         rsg.ptr<float>(), minv.ptr<int>(), T, H, k, 0, e.stream),
         "encode_moe");
      return;
    }
    // 4- or 8-bit stacks (the reference's gqmm at W.bits, qwen35.h:1835)
    ok(ifd_moe_gather_qmm_ex(xn.ptr<void>(), mperm.ptr<int>(), k, moffs.ptr<int>(), mtiles.ptr<int>(),
                             mntiles.ptr<int>(), mt, ly.egu.wq.ptr<uint32_t>(), ly.egu.s.ptr<uint16_t>(),
                             ly.egu.b.ptr<uint16_t>(), E, 2 * I, H, ly.egu.bits, 1, eact.ptr<void>(), R, e.stream),
       "encode_moe");
    ok(ifd_moe_gather_qmm_ex(eact.ptr<void>(), nullptr, 1, moffs.ptr<int>(), mtiles.ptr<int>(), mntiles.ptr<int>(), mt,
                             ly.edown.wq.ptr<uint32_t>(), ly.edown.s.ptr<uint16_t>(), ly.edown.b.ptr<uint16_t>(), E, H,
                             I, ly.edown.bits, 0, edown_out.ptr<void>(), R, e.stream),
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
