// The C ABI (include/inferd_qmm.h): argument checks, routing, workspace layout, and the one-shot MoE FFN.
#include <algorithm>

#include "host.h"
#include "kernels.h"
#include "t64.h"

using namespace ifd;

namespace {

inline hipStream_t S(void* st) { return (hipStream_t)st; }

int fill_gemm(W4Gemm& g, const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N,
              int K, int ldk, uint32_t xr, void* C, int ldc, int M, int mode, int bits = 4) {
  IFD_TRY(check_w4_args(A, lda, wq, s, b, N, K, ldk, xr, C, ldc, M, mode, 2, bits));
  g.bits = bits;
  g.A = A;
  g.lda = lda;
  g.wq = wq;
  g.s = s;
  g.b = b;
  g.N = N;
  g.K = K;
  g.ldk = ldk ? ldk : K;
  g.xr = xr;
  g.C = C;
  g.ldc = ldc;
  g.M = M;
  g.mode = mode;
  return IFD_OK;
}

// The decode path serves up to this many rows (one to four 32-row MFMA tiles); above it the prefill GEMM.
constexpr int kQmvMaxRows = 128;

}  // namespace

extern "C" {

int ifd_version(void) { return 1; }

const char* ifd_status_str(int status) {
  switch (status) {
    case IFD_OK: return "ok";
    case IFD_ERR_ARG: return "invalid argument";
    case IFD_ERR_WORKSPACE: return "workspace too small";
    case IFD_ERR_LAUNCH: return "kernel launch failed";
    case IFD_ERR_UNSUPPORTED: return "unsupported";
    default: return "unknown status";
  }
}

const char* ifd_last_error(void) { return last_error_buf(); }

namespace {
// A public workspace: [kWsHeader bytes of counters, kept zero][kernel scratch]. Sizes reported to callers include
// the header whenever any scratch is needed.
size_t with_header(size_t body) { return body ? body + kWsHeader : 0; }
struct WsView {
  unsigned* cnt = nullptr;
  void* body = nullptr;
  size_t bytes = 0;
};
WsView ws_view(void* w, size_t bytes) {
  WsView v;
  if (w && bytes >= kWsHeader) v.cnt = (unsigned*)w, v.body = (char*)w + kWsHeader, v.bytes = bytes - kWsHeader;
  return v;
}
}  // namespace

size_t ifd_gemm_w4_workspace(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  return with_header(M <= kQmvMaxRows ? qmv_workspace(M, N, K) : qmm_workspace(M, N, K));
}

int ifd_qmv_w4(const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk,
               uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes, void* stream) {
  W4Gemm g;
  IFD_TRY(fill_gemm(g, A, lda, wq, s, b, N, K, ldk, xr, C, ldc, M, mode));
  IFD_CHECK(M <= kQmvMaxRows, "ifd_qmv_w4 takes M <= %d (M=%d)", kQmvMaxRows, M);
  const WsView w = ws_view(workspace, ws_bytes);
  return launch_qmv(g, w.body, w.bytes, S(stream));
}

int ifd_qmm_w4(const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk,
               uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes, void* stream) {
  W4Gemm g;
  IFD_TRY(fill_gemm(g, A, lda, wq, s, b, N, K, ldk, xr, C, ldc, M, mode));
  const WsView w = ws_view(workspace, ws_bytes);
  return launch_qmm(g, w.body, w.bytes, S(stream));
}

int ifd_gemm_w4(const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk,
                uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes, void* stream) {
  W4Gemm g;
  IFD_TRY(fill_gemm(g, A, lda, wq, s, b, N, K, ldk, xr, C, ldc, M, mode));
  const WsView w = ws_view(workspace, ws_bytes);
  if (M <= kQmvMaxRows) return launch_qmv(g, w.body, w.bytes, S(stream));
  return launch_qmm(g, w.body, w.bytes, S(stream));
}

int ifd_flip_w4(uint32_t* wq, size_t n32, uint32_t mask, void* stream) {
  IFD_CHECK(n32 == 0 || wq, "null pointer");
  return launch_flip(wq, n32, mask, S(stream));
}

int ifd_silu_mul(const void* gu, void* h, int I, int rows, void* stream) {
  IFD_CHECK(I > 0 && I % 8 == 0 && rows >= 0, "bad shape I=%d rows=%d (I must be a multiple of 8)", I, rows);
  IFD_CHECK(rows == 0 || (gu && h && aligned(gu, 16) && aligned(h, 16)), "gu and h must be 16-byte aligned");
  return launch_silu_mul((const uint16_t*)gu, 2 * I, (uint16_t*)h, I, I, rows, S(stream));
}

int ifd_rmsnorm(const void* x, int in_stride, const void* w, void* out, int out_stride, int rows, int D, float eps,
                void* stream) {
  IFD_CHECK(rows >= 0 && D > 0 && in_stride >= D && out_stride >= D, "bad shape rows=%d D=%d strides %d/%d", rows, D,
            in_stride, out_stride);
  IFD_CHECK(rows == 0 || (x && w && out), "null pointer");
  IFD_CHECK(eps >= 0.f, "eps must be >= 0");
  return launch_rmsnorm((const uint16_t*)x, in_stride, (const uint16_t*)w, (uint16_t*)out, out_stride, rows, D, eps,
                        S(stream));
}

int ifd_rmsnorm_a8(const void* x, int in_stride, const void* w, void* out, int out_stride, int rows, int D, float eps,
                   int per_token, int8_t* U, float* XS, void* stream) {
  IFD_CHECK(rows >= 0 && D > 0 && D % 64 == 0 && in_stride >= D && out_stride >= D,
            "bad shape rows=%d D=%d strides %d/%d (D multiple of 64)", rows, D, in_stride, out_stride);
  IFD_CHECK(rows == 0 || (x && w && out && U && XS), "null pointer");
  IFD_CHECK(eps >= 0.f, "eps must be >= 0");
  return launch_rmsnorm_a8((const uint16_t*)x, in_stride, (const uint16_t*)w, (uint16_t*)out, out_stride, rows, D, eps,
                           per_token ? 1 : 0, U, XS, S(stream));
}

int ifd_silu_mul_a8(const void* gu, int I, int rows, int per_token, int8_t* U, float* XS, void* stream) {
  IFD_CHECK(I > 0 && I % 64 == 0 && rows >= 0, "bad shape I=%d rows=%d (I multiple of 64)", I, rows);
  IFD_CHECK(rows == 0 || (gu && U && XS), "null pointer");
  return launch_silu_mul_a8((const uint16_t*)gu, 2 * I, I, rows, per_token ? 1 : 0, U, XS, S(stream));
}

int ifd_splitk_res_norm(const float* part, int S_, void* x, int ldx, const void* w, void* out, int out_stride, int rows,
                        int D, float eps, int per_token, int8_t* U, float* XS, void* stream) {
  IFD_CHECK(rows >= 0 && D > 0 && S_ >= 1 && ldx >= D && out_stride >= D, "bad shape rows=%d D=%d S=%d strides %d/%d",
            rows, D, S_, ldx, out_stride);
  IFD_CHECK(rows == 0 || (part && x && w && out), "null pointer");
  IFD_CHECK(!U || (XS && D % 64 == 0), "quantized output needs XS and D %% 64 == 0 (D=%d)", D);
  IFD_CHECK(eps >= 0.f, "eps must be >= 0");
  return launch_splitk_res_norm(part, S_, (uint16_t*)x, ldx, (const uint16_t*)w, (uint16_t*)out, out_stride, rows, D,
                                eps, U ? (per_token ? 2 : 1) : 0, U, XS, S(stream));
}

int ifd_a8_quant(const void* A, int lda, int M, int K, int per_token, int8_t* U, float* XS, void* stream) {
  IFD_CHECK(M >= 0 && K > 0 && K % 64 == 0 && lda >= K && lda % 8 == 0, "bad shape M=%d K=%d lda=%d", M, K, lda);
  IFD_CHECK(M == 0 || (A && U && XS), "null pointer");
  IFD_CHECK(M == 0 || (aligned(A, 16) && aligned(U, 8)), "A must be 16-byte and U 8-byte aligned");
  IFD_CHECK(per_token >= 0 && per_token <= 2, "per_token=%d must be 0 (per group), 1 (per token) or 2 (qa8 form)",
            per_token);
  return launch_a8_quant((const uint16_t*)A, lda, M, K, per_token, U, XS, S(stream));
}

size_t ifd_qmm_w4a8_workspace(int M, int N, int K) { return with_header(w4a8_workspace(M, N, K)); }

int ifd_qmm_w4a8(const int8_t* U, const float* XS, int per_token, const uint32_t* wq, const uint16_t* s,
                 const uint16_t* b, int N, int K, int ldk, uint32_t xr, void* C, int ldc, int M, int mode,
                 void* workspace, size_t ws_bytes, void* stream) {
  W4Gemm g;
  IFD_TRY(fill_gemm(g, U, K, wq, s, b, N, K, ldk, xr, C, ldc, M, mode));
  IFD_CHECK(M == 0 || XS, "null XS");
  g.XS = XS;
  const WsView w = ws_view(workspace, ws_bytes);
  return launch_w4a8(g, per_token ? 1 : 0, w.body, w.bytes, S(stream));
}

// ---- 8-bit weights -----------------------------------------------------------------------------------------------
size_t ifd_gemm_w8_workspace(int M, int N, int K) { return ifd_gemm_w4_workspace(M, N, K); }

int ifd_gemm_w8(const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk,
                uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes, void* stream) {
  W4Gemm g;
  IFD_TRY(fill_gemm(g, A, lda, wq, s, b, N, K, ldk, xr, C, ldc, M, mode, 8));
  const WsView w = ws_view(workspace, ws_bytes);
  if (M <= kQmvMaxRows) return launch_qmv(g, w.body, w.bytes, S(stream));
  return launch_qmm(g, w.body, w.bytes, S(stream));
}

size_t ifd_qmm_w8a8_workspace(int M, int N, int K) { return with_header(w4a8_workspace(M, N, K)); }

int ifd_qmm_w8a8(const int8_t* U, const float* XS, int per_token, const uint32_t* wq, const uint16_t* s,
                 const uint16_t* b, int N, int K, int ldk, uint32_t xr, void* C, int ldc, int M, int mode,
                 void* workspace, size_t ws_bytes, void* stream) {
  W4Gemm g;
  IFD_TRY(fill_gemm(g, U, K, wq, s, b, N, K, ldk, xr, C, ldc, M, mode, 8));
  IFD_CHECK(M == 0 || XS, "null XS");
  g.XS = XS;
  const WsView w = ws_view(workspace, ws_bytes);
  return launch_w4a8(g, per_token ? 1 : 0, w.body, w.bytes, S(stream));
}

// ---- T64 layout ------------------------------------------------------------------------------------------------
size_t ifd_t64_bytes(int N, int K, int E) {
  if (N <= 0 || K <= 0 || K % 64 || E <= 0) return 0;
  return (size_t)E * t64_bytes(N, K);
}

int ifd_pack_t64(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr, int E,
                 void* out, void* stream) {
  IFD_CHECK(N > 0 && K > 0 && K % 64 == 0 && E > 0, "bad shape N=%d K=%d E=%d", N, K, E);
  IFD_CHECK(ldk == 0 || (ldk >= K && ldk % 64 == 0), "ldk=%d must be 0 or a multiple of 64 >= K", ldk);
  IFD_CHECK(xr == 0u || xr == 0x88888888u, "xr=0x%x must be 0 or 0x88888888", xr);
  IFD_CHECK(wq && s && b && out && aligned(out, 16), "null or misaligned pointer");
  return launch_pack_t64(wq, s, b, N, K, ldk ? ldk : K, xr, E, out, S(stream));
}

size_t ifd_gemm_t64_workspace(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  return with_header(M <= 16 ? qmv_t_workspace(M, N, K, 0) : gemm_t_workspace(M, N, K, 0));
}

size_t ifd_gemm_t64_swiglu_workspace(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  return with_header(M <= 16 ? qmv_t_workspace(M, N, K, kModeSwiglu) : gemm_t_workspace(M, N, K, kModeSwiglu));
}

int ifd_gemm_t64_swiglu(const void* A, int lda, const void* wt, int N, int K, void* H, int ldh, int M,
                        void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(M >= 0 && N > 0 && K > 0 && K % 256 == 0 && N % 16 == 0,
            "bad shape M=%d N=%d K=%d (K multiple of 256, N = 2 I with I a multiple of 8)", M, N, K);
  IFD_CHECK(lda >= K && lda % 8 == 0 && ldh >= N / 2 && ldh % 8 == 0, "bad strides lda=%d ldh=%d", lda, ldh);
  if (M == 0) return IFD_OK;
  IFD_CHECK(A && wt && H && aligned(A, 16) && aligned(wt, 16) && aligned(H, 16), "null or misaligned pointer");
  IFD_CHECK(!workspace || aligned(workspace, 16), "workspace must be 16-byte aligned");
  const WsView w = ws_view(workspace, ws_bytes);
  if (M <= 16)
    return launch_qmv_t((const uint16_t*)A, lda, wt, N, K, H, ldh, M, kModeSwiglu, w.cnt, w.body, w.bytes, S(stream));
  return launch_gemm_t((const uint16_t*)A, lda, wt, N, K, H, ldh, M, kModeSwiglu, w.body, w.bytes, S(stream));
}

size_t ifd_gemm_t64_multi_workspace(int M, int n, const int* Ns, int K) {
  if (M <= 0 || M > 16 || n < 1 || n > 8 || !Ns || K <= 0 || K % 256) return 0;
  for (int l = 0; l < n; l++)
    if (Ns[l] <= 0) return 0;
  return with_header(qmv_t_multi_workspace(M, n, Ns, K));
}

int ifd_gemm_t64_multi(const void* A, int lda, int n, const void* const* wts, const int* Ns, int K, void* const* Cs,
                       const int* ldcs, int M, int mode, void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(n >= 1 && n <= 8 && wts && Ns && Cs && ldcs, "n=%d linears (1 to 8) with their arrays", n);
  IFD_CHECK(M >= 0 && M <= 16 && K > 0 && K % 256 == 0, "bad shape M=%d K=%d (M <= 16, K multiple of 256)", M, K);
  IFD_CHECK(mode >= 0 && mode <= 2, "mode=%d must be 0, 1 or 2", mode);
  IFD_CHECK(lda >= K && lda % 8 == 0, "bad stride lda=%d", lda);
  for (int l = 0; l < n; l++) {
    IFD_CHECK(Ns[l] > 0 && ldcs[l] >= Ns[l], "linear %d: N=%d ldc=%d", l, Ns[l], ldcs[l]);
    IFD_CHECK(wts[l] && Cs[l] && aligned(wts[l], 16), "linear %d: null or misaligned pointer", l);
  }
  if (M == 0) return IFD_OK;
  IFD_CHECK(A && aligned(A, 16), "null or misaligned pointer");
  IFD_CHECK(!workspace || aligned(workspace, 16), "workspace must be 16-byte aligned");
  const WsView w = ws_view(workspace, ws_bytes);
  return launch_qmv_t_multi((const uint16_t*)A, lda, n, wts, Ns, K, Cs, ldcs, M, mode, w.cnt, w.body, w.bytes,
                            S(stream));
}

int ifd_gemm_t64(const void* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                 void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(M >= 0 && N > 0 && K > 0 && K % 256 == 0, "bad shape M=%d N=%d K=%d (K multiple of 256)", M, N, K);
  IFD_CHECK(mode >= 0 && mode <= 2, "mode=%d must be 0, 1 or 2", mode);
  IFD_CHECK(lda >= K && lda % 8 == 0 && ldc >= N, "bad strides lda=%d ldc=%d", lda, ldc);
  if (M == 0) return IFD_OK;
  IFD_CHECK(A && wt && C && aligned(A, 16) && aligned(wt, 16), "null or misaligned pointer");
  IFD_CHECK(!workspace || aligned(workspace, 16), "workspace must be 16-byte aligned");
  const WsView w = ws_view(workspace, ws_bytes);
  if (M <= 16)
    return launch_qmv_t((const uint16_t*)A, lda, wt, N, K, C, ldc, M, mode, w.cnt, w.body, w.bytes, S(stream));
  return launch_gemm_t((const uint16_t*)A, lda, wt, N, K, C, ldc, M, mode, w.body, w.bytes, S(stream));
}

// Per-group activations: [Ab = bf16(U) | sxT | the GEMM's own workspace] in the body.
namespace {
struct W4a8gLayout {
  size_t ab, sxt, gemm, total;
  int Mp;
};
W4a8gLayout w4a8g_layout(int M, int N, int K, int mode) {
  W4a8gLayout L{};
  L.Mp = w4a8g_mp(M);
  L.ab = 0;
  L.sxt = align_up((size_t)M * K * 2, 256);
  L.gemm = L.sxt + align_up((size_t)(K / 64) * L.Mp * 4, 256);
  L.total = L.gemm + (M <= 16 ? qmv_t_workspace(M, N, K, mode) : gemm_t_a8_workspace(M, N, K, mode));
  return L;
}
}  // namespace

size_t ifd_gemm_t64_w4a8_workspace(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128) return 0;
  // either form of the activations: per token, or per group (modes 0 and 1 size alike, mode 2 no larger)
  return with_header(std::max(w4a8_t_workspace(M, N, K), w4a8g_layout(M, N, K, 0).total));
}

int ifd_gemm_t64_w4a8(const int8_t* U, const float* XS, int per_token, const void* wt, int N, int K, void* C, int ldc,
                      int M, int mode, void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(M >= 0 && N > 0 && K > 0 && K % 256 == 0, "bad shape M=%d N=%d K=%d (K multiple of 256)", M, N, K);
  IFD_CHECK(mode >= 0 && mode <= 2, "mode=%d must be 0, 1 or 2", mode);
  IFD_CHECK(ldc >= N, "bad stride ldc=%d", ldc);
  IFD_CHECK(per_token == 0 || per_token == 1, "per_token=%d must be 0 (per 64-group) or 1 (per row)", per_token);
  if (M == 0) return IFD_OK;
  IFD_CHECK(U && XS && wt && C && aligned(U, 16) && aligned(wt, 16), "null or misaligned pointer");
  IFD_CHECK(!workspace || aligned(workspace, 16), "workspace must be 16-byte aligned");
  const WsView w = ws_view(workspace, ws_bytes);
  if (per_token) return launch_w4a8_t(U, XS, wt, N, K, C, ldc, M, mode, w.body, w.bytes, S(stream));
  // per (row, 64-group) scales: xq as bf16 integers through the affine T64 kernels
  const W4a8gLayout L = w4a8g_layout(M, N, K, mode);
  if (!w.body || w.bytes < L.total)
    return fail(IFD_ERR_WORKSPACE, "gemm_t64_w4a8 needs %zu bytes of workspace, got %zu", with_header(L.total),
                ws_bytes);
  char* b = (char*)w.body;
  uint16_t* Ab = (uint16_t*)(b + L.ab);
  float* sxT = (float*)(b + L.sxt);
  hipStream_t st = S(stream);
  IFD_TRY(launch_w4a8g_prep(U, XS, M, K, Ab, sxT, L.Mp, st));
  if (M <= 16)
    return launch_qmv_t_a8(Ab, XS, wt, N, K, C, ldc, M, mode, w.cnt, b + L.gemm, w.bytes - L.gemm, st);
  return launch_gemm_t_a8(Ab, sxT, L.Mp, wt, N, K, C, ldc, M, mode, b + L.gemm, w.bytes - L.gemm, st);
}

// ---- T64x8 layout (8-bit weights) --------------------------------------------------------------------------------
size_t ifd_t64x8_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % 64) return 0;
  return t64x8_bytes(N, K);
}

int ifd_pack_t64x8(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr,
                   void* out, void* stream) {
  IFD_CHECK(N > 0 && K > 0 && K % 64 == 0, "bad shape N=%d K=%d", N, K);
  IFD_CHECK(ldk == 0 || (ldk >= K && ldk % 64 == 0), "ldk=%d must be 0 or a multiple of 64 >= K", ldk);
  IFD_CHECK(xr == 0u || xr == 0x80808080u, "xr=0x%x must be 0 or 0x80808080", xr);
  IFD_CHECK(wq && s && b && out && aligned(out, 16), "null or misaligned pointer");
  return launch_pack_t64x8(wq, s, b, N, K, ldk ? ldk : K, xr, out, S(stream));
}

// the T64x8 decode GEMV serves M <= 16 when K % 128 == 0, the stream-K GEMM the rest
static bool t64x8_qmv(int M, int K) { return M <= 16 && K % 128 == 0; }

size_t ifd_gemm_t64x8_workspace(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  return with_header(t64x8_qmv(M, K) ? qmv_t_workspace(M, N, K, 0, 8) : gemm_sk8_workspace(M, N, K));
}

int ifd_gemm_t64x8(const void* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                   void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(M >= 0 && N > 0 && K > 0 && K % 64 == 0, "bad shape M=%d N=%d K=%d (K multiple of 64)", M, N, K);
  IFD_CHECK(mode >= 0 && mode <= 2, "mode=%d must be 0, 1 or 2", mode);
  IFD_CHECK(lda >= K && lda % 8 == 0 && ldc >= N, "bad strides lda=%d ldc=%d", lda, ldc);
  if (M == 0) return IFD_OK;
  IFD_CHECK(A && wt && C && aligned(A, 16) && aligned(wt, 16), "null or misaligned pointer");
  IFD_CHECK(!workspace || aligned(workspace, 16), "workspace must be 16-byte aligned");
  const WsView w = ws_view(workspace, ws_bytes);
  if (t64x8_qmv(M, K))
    return launch_qmv_t8((const uint16_t*)A, lda, wt, N, K, C, ldc, M, mode, w.cnt, w.body, w.bytes, S(stream));
  return launch_gemm_sk8((const uint16_t*)A, lda, wt, N, K, C, ldc, M, mode, w.body, w.bytes, S(stream));
}

size_t ifd_gemm_t64x8_w8a8_workspace(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  return with_header(w8a8_t_workspace(M, N, K));
}

int ifd_gemm_t64x8_w8a8(const int8_t* U, const float* XS, int per_token, const void* wt, int N, int K, void* C,
                        int ldc, int M, int mode, void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(M >= 0 && N > 0 && K > 0 && K % 64 == 0, "bad shape M=%d N=%d K=%d (K multiple of 64)", M, N, K);
  IFD_CHECK(mode >= 0 && mode <= 2, "mode=%d must be 0, 1 or 2", mode);
  IFD_CHECK(ldc >= N, "bad stride ldc=%d", ldc);
  if (!per_token) return fail(IFD_ERR_UNSUPPORTED, "T64x8 W8A8 takes per-token activations (per_token = 1)");
  if (M == 0) return IFD_OK;
  IFD_CHECK(U && XS && wt && C && aligned(U, 16) && aligned(wt, 16), "null or misaligned pointer");
  IFD_CHECK(!workspace || aligned(workspace, 16), "workspace must be 16-byte aligned");
  const WsView w = ws_view(workspace, ws_bytes);
  return launch_w8a8_t(U, XS, wt, N, K, C, ldc, M, mode, w.body, w.bytes, S(stream));
}

int ifd_moe_router_logits(const void* x, const void* w, int T, int H, int E1, int out_bf16, void* logits,
                          void* stream) {
  IFD_CHECK(T >= 0 && H > 0 && H % 64 == 0 && E1 > 0, "bad shape T=%d H=%d E1=%d (H multiple of 64)", T, H, E1);
  IFD_CHECK(T == 0 || (x && w && logits && aligned(x, 16) && aligned(w, 16)), "x and w must be 16-byte aligned");
  return launch_router_logits((const uint16_t*)x, (const uint16_t*)w, T, H, E1, out_bf16, logits, S(stream));
}

int ifd_moe_route(const void* logits, int logits_bf16, int T, int E, int k, int stride, int norm, int shared_gate,
                  int* idx, float* wt, float* sg, void* stream) {
  IFD_CHECK(E > 0 && E <= 512 && k > 0 && k <= 16 && k <= E && T >= 0, "bad routing shape E=%d k=%d", E, k);
  IFD_CHECK(stride >= E + (shared_gate ? 1 : 0), "stride=%d too small for E=%d (+ shared gate)", stride, E);
  IFD_CHECK(T == 0 || (logits && idx && wt && sg), "null pointer");
  return launch_moe_route(logits, logits_bf16, T, E, k, stride, norm, shared_gate, idx, wt, sg, S(stream));
}

int ifd_moe_tiles_max(int R, int E) { return moe_tiles_max(R, E); }
size_t ifd_moe_dispatch_workspace(int R, int E) { return with_header(moe_dispatch_workspace(R, E)); }

int ifd_moe_dispatch(const int* idx, int R, int E, int* offsets, int* perm, int* inv, int* tiles, int* ntiles,
                     void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(R >= 0 && E > 0 && E <= 1024, "bad dispatch shape R=%d E=%d (E <= 1024)", R, E);
  IFD_CHECK(offsets && tiles && ntiles && (R == 0 || (idx && perm && inv)), "null pointer");
  const WsView w = ws_view(workspace, ws_bytes);
  return launch_moe_dispatch(idx, R, E, offsets, perm, inv, tiles, ntiles, w.body, w.bytes, S(stream));
}

int ifd_moe_gather(const void* x, const int* perm, int div, int R, int H, void* xs, void* stream) {
  IFD_CHECK(R >= 0 && H > 0 && H % 8 == 0 && div > 0, "bad shape R=%d H=%d div=%d", R, H, div);
  IFD_CHECK(R == 0 || (x && perm && xs && aligned(x, 16) && aligned(xs, 16)), "x, xs must be 16-byte aligned");
  return launch_moe_gather((const uint16_t*)x, perm, div, R, H, (uint16_t*)xs, S(stream));
}

int ifd_moe_gather_qmm_ex(const void* A, const int* perm, int div, const int* offsets, const int* tiles,
                          const int* ntiles, int max_tiles, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                          int E, int N, int K, int bits, int silu, void* C, int R, void* stream) {
  IFD_CHECK(bits == 4 || bits == 8, "bits=%d must be 4 or 8", bits);
  IFD_CHECK(R >= 0 && E > 0 && N > 0 && K > 0 && K % 64 == 0 && div > 0, "bad shape E=%d N=%d K=%d", E, N, K);
  IFD_CHECK(!silu || N % 2 == 0, "silu needs an even N (gate | up)");
  IFD_CHECK(max_tiles >= 0, "bad max_tiles");
  IFD_CHECK(R == 0 || (A && offsets && tiles && ntiles && wq && s && b && C), "null pointer");
  IFD_CHECK(R == 0 || (aligned(A, 16) && aligned(wq, 16)), "A and wq must be 16-byte aligned");
  return launch_moe_gather_qmm((const uint16_t*)A, perm, div, tiles, ntiles, offsets, max_tiles, wq, s, b, N, K,
                               silu ? 1 : 0, (uint16_t*)C, R, S(stream), bits);
}

int ifd_moe_gather_qmm(const void* A, const int* perm, int div, const int* offsets, const int* tiles,
                       const int* ntiles, int max_tiles, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int E,
                       int N, int K, int silu, void* C, int R, void* stream) {
  return ifd_moe_gather_qmm_ex(A, perm, div, offsets, tiles, ntiles, max_tiles, wq, s, b, E, N, K, 4, silu, C, R,
                               stream);
}

int ifd_moe_gather_qmm_a8(const int8_t* U, const float* XS, const int* perm, int div, const int* offsets,
                          const int* tiles, const int* ntiles, int max_tiles, const uint32_t* wq, const uint16_t* s,
                          const uint16_t* b, int E, int N, int K, int silu, void* C, int R, void* stream) {
  IFD_CHECK(R >= 0 && E > 0 && N > 0 && K > 0 && K % 64 == 0 && div > 0, "bad shape E=%d N=%d K=%d", E, N, K);
  IFD_CHECK(!silu || N % 2 == 0, "silu needs an even N (gate | up)");
  IFD_CHECK(max_tiles >= 0, "bad max_tiles");
  IFD_CHECK(R == 0 || (U && XS && offsets && tiles && ntiles && wq && s && b && C), "null pointer");
  IFD_CHECK(R == 0 || (aligned(U, 16) && aligned(XS, 8) && aligned(wq, 16)), "U and wq must be 16-byte aligned");
  return launch_moe_gather_qmm_a8(U, XS, perm, div, tiles, ntiles, offsets, max_tiles, wq, s, b, N, K, silu ? 1 : 0,
                                  (uint16_t*)C, R, S(stream));
}

int ifd_moe_combine(void* out, const void* yd, const float* wt, const void* ys, const float* sg, const int* inv, int T,
                    int H, int k, int assign, void* stream) {
  IFD_CHECK(T >= 0 && H > 0 && H % 8 == 0 && k > 0, "bad shape T=%d H=%d k=%d", T, H, k);
  IFD_CHECK(T == 0 || (out && yd && wt && inv && (!ys || sg)), "null pointer");
  IFD_CHECK(T == 0 || (aligned(out, 16) && aligned(yd, 16) && (!ys || aligned(ys, 16))), "bf16 rows must be aligned");
  return launch_moe_combine((uint16_t*)out, (const uint16_t*)yd, wt, (const uint16_t*)ys, sg, inv, T, H, k, assign,
                            S(stream));
}

// ---- one-shot MoE FFN ------------------------------------------------------------------------------------------
namespace {
struct MoeLayout {
  size_t logits, idx, wt, sg, offsets, perm, inv, tiles, ntiles, disp, sh_gu, sh_act, sh_ws, ys, eact, edn, total;
};
MoeLayout moe_layout(int T, int H, int I, int E, int k, int Is) {
  MoeLayout L{};
  const int R = T * k, E1 = E + 1;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align_up(std::max<size_t>(bytes, 1), 256);
    return at;
  };
  L.logits = take((size_t)T * E1 * 4);
  L.idx = take((size_t)R * 4);
  L.wt = take((size_t)R * 4);
  L.sg = take((size_t)T * 4);
  L.offsets = take((size_t)(E + 1) * 4);
  L.perm = take((size_t)R * 4);
  L.inv = take((size_t)R * 4);
  L.tiles = take((size_t)moe_tiles_max(R, E) * 2 * 4);
  L.ntiles = take(4);
  L.disp = take(moe_dispatch_workspace(R, E));
  L.sh_gu = take(Is ? (size_t)T * 2 * Is * 2 : 0);
  L.sh_act = take(Is ? (size_t)T * Is * 2 : 0);
  L.sh_ws = take(Is ? std::max(ifd_gemm_w4_workspace(T, 2 * Is, H), ifd_gemm_w4_workspace(T, H, Is)) : 0);
  L.ys = take(Is ? (size_t)T * H * 2 : 0);
  L.eact = take((size_t)R * I * 2);
  L.edn = take((size_t)R * H * 2);
  L.total = o;
  return L;
}
}  // namespace

size_t ifd_moe_ffn_workspace(int T, int H, int I, int E, int k, int Is) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  return with_header(moe_layout(T, H, I, E, k, Is).total);
}

int ifd_moe_ffn(const void* xn, int T, int H, const void* router, int E, int k, int norm, int shared_gate,
                int logits_bf16, const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b,
                const uint32_t* edn_wq, const uint16_t* edn_s, const uint16_t* edn_b, int I, const uint32_t* sgu_wq,
                const uint16_t* sgu_s, const uint16_t* sgu_b, const uint32_t* sdn_wq, const uint16_t* sdn_s,
                const uint16_t* sdn_b, int Is, void* out, int assign, int* idx, float* wt, float* sg,
                void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(T >= 0 && H > 0 && H % 64 == 0 && I > 0 && I % 64 == 0 && E > 0 && E <= 512 && k > 0 && k <= 16,
            "bad MoE shape T=%d H=%d I=%d E=%d k=%d", T, H, I, E, k);
  const bool shared = sgu_wq != nullptr;
  IFD_CHECK(!shared || (Is > 0 && Is % 64 == 0 && sgu_s && sgu_b && sdn_wq && sdn_s && sdn_b), "bad shared expert");
  IFD_CHECK(!shared_gate || shared, "a shared gate needs a shared expert");
  if (T == 0) return IFD_OK;
  IFD_CHECK(xn && router && egu_wq && egu_s && egu_b && edn_wq && edn_s && edn_b && out, "null pointer");
  const MoeLayout L = moe_layout(T, H, I, E, k, shared ? Is : 0);
  const WsView wv = ws_view(workspace, ws_bytes);
  if (!wv.body || wv.bytes < L.total)
    return fail(IFD_ERR_WORKSPACE, "moe_ffn needs %zu bytes of workspace, got %zu", with_header(L.total), ws_bytes);
  // the layout is carved from the scratch after the header; the shared expert's GEMMs get a sub-area sized by their
  // own public query, whose leading counter bytes are not kept zero: only counter-free GEMM paths may run there
  char* w = (char*)wv.body;
  hipStream_t st = S(stream);
  const int R = T * k, E1 = E + (shared_gate ? 1 : 0);
  int* ridx = idx ? idx : (int*)(w + L.idx);
  float* rwt = wt ? wt : (float*)(w + L.wt);
  float* rsg = sg ? sg : (float*)(w + L.sg);
  // router -> routing (row E of the router, when present, is the shared expert's gate)
  IFD_TRY(launch_router_logits((const uint16_t*)xn, (const uint16_t*)router, T, H, E1, logits_bf16, w + L.logits, st));
  IFD_TRY(launch_moe_route(w + L.logits, logits_bf16, T, E, k, E1, norm, shared_gate, ridx, rwt, rsg, st));
  // shared expert: gate_up -> SwiGLU -> down into ys
  const uint16_t* ys = nullptr;
  if (shared) {
    IFD_TRY(ifd_gemm_w4(xn, H, sgu_wq, sgu_s, sgu_b, 2 * Is, H, 0, 0, w + L.sh_gu, 2 * Is, T, 0, w + L.sh_ws,
                        ifd_gemm_w4_workspace(T, 2 * Is, H), stream));
    IFD_TRY(launch_silu_mul((const uint16_t*)(w + L.sh_gu), 2 * Is, (uint16_t*)(w + L.sh_act), Is, Is, T, st));
    IFD_TRY(ifd_gemm_w4(w + L.sh_act, Is, sdn_wq, sdn_s, sdn_b, H, Is, 0, 0, w + L.ys, H, T, 0, w + L.sh_ws,
                        ifd_gemm_w4_workspace(T, H, Is), stream));
    ys = (const uint16_t*)(w + L.ys);
  }
  // dispatch -> gathered gate/up with fused SwiGLU -> gathered down -> combine
  int* offsets = (int*)(w + L.offsets);
  int* perm = (int*)(w + L.perm);
  int* inv = (int*)(w + L.inv);
  int* tiles = (int*)(w + L.tiles);
  int* ntiles = (int*)(w + L.ntiles);
  IFD_TRY(launch_moe_dispatch(ridx, R, E, offsets, perm, inv, tiles, ntiles, w + L.disp, moe_dispatch_workspace(R, E),
                              st));
  const int mt = moe_tiles_max(R, E);
  IFD_TRY(launch_moe_gather_qmm((const uint16_t*)xn, perm, k, tiles, ntiles, offsets, mt, egu_wq, egu_s, egu_b, 2 * I,
                                H, 1, (uint16_t*)(w + L.eact), R, st));
  IFD_TRY(launch_moe_gather_qmm((const uint16_t*)(w + L.eact), nullptr, 1, tiles, ntiles, offsets, mt, edn_wq, edn_s,
                                edn_b, H, I, 0, (uint16_t*)(w + L.edn), R, st));
  return launch_moe_combine((uint16_t*)out, (const uint16_t*)(w + L.edn), rwt, ys, rsg, inv, T, H, k, assign, st);
}

// ---- the MoE FFN on T64 expert stacks ------------------------------------------------------------------------------
int ifd_moe_dispatch_ex(const int* idx, int R, int E, int k, int tile_rows, int shared_rows, int* offsets, int* perm,
                        int* inv, int* tiles, int* ntiles, void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(R >= 0 && E > 0 && E <= 1023 && k > 0 && shared_rows >= 0, "bad dispatch shape R=%d E=%d k=%d", R, E, k);
  IFD_CHECK(tile_rows == 32 || tile_rows == 64, "tile_rows=%d must be 32 or 64", tile_rows);
  IFD_CHECK(offsets && tiles && ntiles && (R + shared_rows == 0 || perm) && (R == 0 || (idx && inv)), "null pointer");
  const WsView w = ws_view(workspace, ws_bytes);
  return launch_moe_dispatch(idx, R, E, offsets, perm, inv, tiles, ntiles, w.body, w.bytes, S(stream), tile_rows,
                             shared_rows, k);
}

size_t ifd_moe_gather_qmm_t64_workspace(int tile_rows) {
  if (tile_rows != 32 && tile_rows != 64) return 0;
  return with_header(moe_gather_t64_part_bytes(tile_rows));
}

int ifd_moe_gather_qmm_t64(const void* A, int lda, const int* perm, int div, const int* offsets, const int* tiles,
                           const int* ntiles, int tile_rows, const void* wt, const void* wt_shared, int E, int N, int K,
                           int silu, void* C, int ldc, int rows, void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(rows >= 0 && E > 0 && N > 0 && K > 0 && div > 0, "bad shape E=%d N=%d K=%d rows=%d", E, N, K, rows);
  IFD_CHECK(lda >= K && lda % 8 == 0 && ldc >= (silu ? N / 2 : N) && ldc % 8 == 0, "bad strides lda=%d ldc=%d", lda,
            ldc);
  IFD_CHECK(rows == 0 || (A && offsets && tiles && ntiles && wt && C), "null pointer");
  IFD_CHECK(rows == 0 || (aligned(A, 16) && aligned(wt, 16) && aligned(C, 16) && (!wt_shared || aligned(wt_shared, 16))),
            "A, C and the stacks must be 16-byte aligned");
  float* part = nullptr;
  size_t part_bytes = 0;
  unsigned* cnt = nullptr;
  if (workspace) {  // the balanced schedule
    const WsView w = ws_view(workspace, ws_bytes);
    if (ws_bytes < ifd_moe_gather_qmm_t64_workspace(tile_rows) || !aligned(workspace, 16))
      return fail(IFD_ERR_WORKSPACE, "moe_gather_qmm_t64 needs %zu bytes of 16-byte aligned workspace, got %zu",
                  ifd_moe_gather_qmm_t64_workspace(tile_rows), ws_bytes);
    part = (float*)w.body, part_bytes = w.bytes, cnt = w.cnt;
  }
  return launch_moe_gather_qmm_t64((const uint16_t*)A, lda, perm, div, tiles, ntiles, offsets, tile_rows, wt,
                                   wt_shared, E, N, K, silu ? 1 : 0, (uint16_t*)C, ldc, rows, part, part_bytes, cnt,
                                   S(stream));
}

namespace {
// rows per tile of the T64 gathered GEMM: 64-row tiles once an expert holds about 24 routed rows on average
int moe_t64_tile_rows(int R, int E) { return R >= 24 * E ? 64 : 32; }
}  // namespace

int ifd_moe_t64_tile_rows(int R, int E) { return moe_t64_tile_rows(std::max(R, 0), std::max(E, 1)); }

namespace {
struct MoeT64Layout {
  size_t logits, idx, wt, sg, offsets, perm, inv, tiles, ntiles, disp, eact, ydn, part, total;
};
MoeT64Layout moe_t64_layout(int T, int H, int I, int E, int k, int shared) {
  MoeT64Layout L{};
  const int R = T * k, Rt = R + (shared ? T : 0);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align_up(std::max<size_t>(bytes, 1), 256);
    return at;
  };
  L.logits = take((size_t)T * (E + 1) * 4);
  L.idx = take((size_t)R * 4);
  L.wt = take((size_t)R * 4);
  L.sg = take((size_t)T * 4);
  L.offsets = take((size_t)(E + 2) * 4);
  L.perm = take((size_t)Rt * 4);
  L.inv = take((size_t)R * 4);
  L.tiles = take((size_t)moe_tiles_max(Rt, E + 1) * 2 * 4);
  L.ntiles = take(4);
  L.disp = take(moe_dispatch_workspace(R, E));
  L.eact = take((size_t)Rt * I * 2);
  L.ydn = take((size_t)Rt * H * 2);
  L.part = take(moe_gather_t64_part_bytes(moe_t64_tile_rows(R, E)));
  L.total = o;
  return L;
}
}  // namespace

size_t ifd_moe_ffn_t64_workspace(int T, int H, int I, int E, int k, int shared) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  return with_header(moe_t64_layout(T, H, I, E, k, shared ? 1 : 0).total);
}

int ifd_moe_ffn_t64(const void* xn, int T, int H, const void* router, int E, int k, int norm, int shared_gate,
                    int logits_bf16, const void* egu_t64, const void* edn_t64, int I, const void* sgu_t64,
                    const void* sdn_t64, void* out, int assign, int* idx, float* wt, float* sg, void* workspace,
                    size_t ws_bytes, void* stream) {
  IFD_CHECK(T >= 0 && H > 0 && H % 256 == 0 && I > 0 && I % 256 == 0 && E > 0 && E <= 512 && k > 0 && k <= 16 &&
                k <= E,
            "bad MoE shape T=%d H=%d I=%d E=%d k=%d (H and I multiples of 256)", T, H, I, E, k);
  const bool shared = sgu_t64 != nullptr;
  IFD_CHECK(!shared || sdn_t64, "the shared expert needs both stacks");
  IFD_CHECK(!shared_gate || shared, "a shared gate needs a shared expert");
  if (T == 0) return IFD_OK;
  IFD_CHECK(xn && router && egu_t64 && edn_t64 && out, "null pointer");
  IFD_CHECK(aligned(xn, 16) && aligned(router, 16) && aligned(egu_t64, 16) && aligned(edn_t64, 16) &&
                aligned(out, 16) && (!shared || (aligned(sgu_t64, 16) && aligned(sdn_t64, 16))),
            "tokens, router, stacks and out must be 16-byte aligned");
  const MoeT64Layout L = moe_t64_layout(T, H, I, E, k, shared ? 1 : 0);
  const WsView wv = ws_view(workspace, ws_bytes);
  if (!wv.body || wv.bytes < L.total)
    return fail(IFD_ERR_WORKSPACE, "moe_ffn_t64 needs %zu bytes of workspace, got %zu", with_header(L.total),
                ws_bytes);
  char* w = (char*)wv.body;
  hipStream_t st = S(stream);
  const int R = T * k, Rt = R + (shared ? T : 0), E1 = E + (shared_gate ? 1 : 0);
  int* ridx = idx ? idx : (int*)(w + L.idx);
  float* rwt = wt ? wt : (float*)(w + L.wt);
  float* rsg = sg ? sg : (float*)(w + L.sg);
  int* offsets = (int*)(w + L.offsets);
  int* perm = (int*)(w + L.perm);
  int* inv = (int*)(w + L.inv);
  int* tiles = (int*)(w + L.tiles);
  int* ntiles = (int*)(w + L.ntiles);
  uint16_t* eact = (uint16_t*)(w + L.eact);
  uint16_t* ydn = (uint16_t*)(w + L.ydn);
  const int tr = moe_t64_tile_rows(R, E);
  IFD_TRY(launch_router_logits((const uint16_t*)xn, (const uint16_t*)router, T, H, E1, logits_bf16, w + L.logits, st));
  IFD_TRY(launch_moe_route(w + L.logits, logits_bf16, T, E, k, E1, norm, shared_gate, ridx, rwt, rsg, st));
  IFD_TRY(launch_moe_dispatch(ridx, R, E, offsets, perm, inv, tiles, ntiles, w + L.disp, moe_dispatch_workspace(R, E),
                              st, tr, shared ? T : 0, k));
  // the balanced schedule: the pieces in the workspace, the counters in its header
  float* part = (float*)(w + L.part);
  const size_t pb = moe_gather_t64_part_bytes(tr);
  IFD_TRY(launch_moe_gather_qmm_t64((const uint16_t*)xn, H, perm, k, tiles, ntiles, offsets, tr, egu_t64, sgu_t64, E,
                                    2 * I, H, 1, eact, I, Rt, part, pb, wv.cnt, st));
  IFD_TRY(launch_moe_gather_qmm_t64(eact, I, nullptr, 1, tiles, ntiles, offsets, tr, edn_t64, sdn_t64, E, H, I, 0,
                                    ydn, H, Rt, part, pb, wv.cnt, st));
  // the shared expert's rows follow the routed ones in token order
  return launch_moe_combine((uint16_t*)out, ydn, rwt, shared ? ydn + (size_t)R * H : nullptr, rsg, inv, T, H, k,
                            assign, st);
}

// ---- the dense decode MLP block -----------------------------------------------------------------------------------
namespace {
size_t mlp_gemm_scratch(int M, int H, int I) {
  const size_t gu = M <= 16 ? qmv_t_workspace(M, 2 * I, H, kModeSwiglu) : gemm_t_workspace(M, 2 * I, H, kModeSwiglu);
  const size_t dn = M <= 16 ? qmv_t_workspace(M, H, I, 1) : gemm_t_workspace(M, H, I, 1);
  return align_up(std::max(gu, dn), 256);
}
}  // namespace

size_t ifd_mlp_decode_workspace(int M, int H, int I) {
  if (M <= 0 || H <= 0 || I <= 0) return 0;
  return with_header(mlp_gemm_scratch(M, H, I) + align_up((size_t)M * H * 2, 256) + (size_t)M * I * 2);
}

int ifd_mlp_decode(void* x, int ldx, const void* norm_w, float eps, const void* gu_t64, const void* dn_t64, int M,
                   int H, int I, void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(M >= 0 && H > 0 && H % 256 == 0 && I > 0 && I % 256 == 0, "bad shape M=%d H=%d I=%d (H, I multiples of 256)",
            M, H, I);
  IFD_CHECK(ldx >= H && ldx % 8 == 0, "bad stride ldx=%d", ldx);
  IFD_CHECK(eps >= 0.f, "eps must be >= 0");
  if (M == 0) return IFD_OK;
  IFD_CHECK(x && norm_w && gu_t64 && dn_t64 && aligned(x, 16) && aligned(gu_t64, 16) && aligned(dn_t64, 16),
            "null or misaligned pointer");
  const size_t need = ifd_mlp_decode_workspace(M, H, I);
  const WsView w = ws_view(workspace, ws_bytes);
  if (!workspace || ws_bytes < need || !aligned(workspace, 16))
    return fail(IFD_ERR_WORKSPACE, "mlp_decode needs %zu bytes of 16-byte aligned workspace, got %zu", need, ws_bytes);
  hipStream_t st = S(stream);
  const size_t G = mlp_gemm_scratch(M, H, I);
  uint16_t* xn = (uint16_t*)((char*)w.body + G);
  uint16_t* act = (uint16_t*)((char*)w.body + G + align_up((size_t)M * H * 2, 256));
  IFD_TRY(launch_rmsnorm((const uint16_t*)x, ldx, (const uint16_t*)norm_w, xn, H, M, H, eps, st));
  if (M <= 16) {
    IFD_TRY(launch_qmv_t(xn, H, gu_t64, 2 * I, H, act, I, M, kModeSwiglu, w.cnt, w.body, G, st));
    return launch_qmv_t(act, I, dn_t64, H, I, x, ldx, M, 1, w.cnt, w.body, G, st);
  }
  IFD_TRY(launch_gemm_t(xn, H, gu_t64, 2 * I, H, act, I, M, kModeSwiglu, w.body, G, st));
  return launch_gemm_t(act, I, dn_t64, H, I, x, ldx, M, 1, w.body, G, st);
}

// ---- measurement probes ------------------------------------------------------------------------------------------
int ifd_probe_stream_read(const void* src, size_t bytes, void* sink, int blocks, void* stream) {
  IFD_CHECK(src && sink && aligned(src, 16) && aligned(sink, 16) && bytes % 16 == 0 && blocks > 0,
            "probe_stream_read: 16-byte aligned src and sink, bytes %% 16 == 0, blocks > 0");
  return launch_probe_read(src, bytes, sink, blocks, S(stream));
}

int ifd_probe_mfma(int int8, int iters, int blocks, float* out, void* stream) {
  IFD_CHECK(out && iters > 0 && blocks > 0 && (int8 == 0 || int8 == 1), "probe_mfma: bad arguments");
  return launch_probe_mfma(int8, iters, blocks, out, S(stream));
}

// ---- decode MoE (T <= 16) ---------------------------------------------------------------------------------------
size_t ifd_moe_decode_workspace(int T, int H, int I, int E, int k) {
  if (T <= 0 || T > 16 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  return with_header(mdec_layout(T, H, I, E, k).total);
}

int ifd_moe_decode_ex(const void* xn, int T, int H, const void* router, int E, int k, int norm, int shared_gate,
                      const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b, const uint32_t* edn_wq,
                      const uint16_t* edn_s, const uint16_t* edn_b, int I, const uint32_t* sgu_wq,
                      const uint16_t* sgu_s, const uint16_t* sgu_b, const uint32_t* sdn_wq, const uint16_t* sdn_s,
                      const uint16_t* sdn_b, int shared_bits, void* out, int assign, int* idx, float* wt, float* sg,
                      float* logits, void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(shared_bits == 4 || shared_bits == 8, "shared_bits=%d must be 4 or 8", shared_bits);
  IFD_CHECK(T >= 0 && T <= 16, "the decode MoE takes T <= 16 tokens (T=%d): larger batches use ifd_moe_ffn", T);
  IFD_CHECK(H > 0 && H % 512 == 0 && H / 128 < kWsCounters && I > 0 && I % 64 == 0 && E > 0 && E <= 512 && k > 0 &&
                k <= 16 && k <= E,
            "bad decode MoE shape H=%d I=%d E=%d k=%d (H multiple of 512, I of 64, E <= 512, k <= 16)", H, I, E, k);
  const bool shared = sgu_wq != nullptr;
  IFD_CHECK(!shared || (sgu_s && sgu_b && sdn_wq && sdn_s && sdn_b), "bad shared expert");
  IFD_CHECK(!shared_gate || shared, "a shared gate needs a shared expert");
  if (T == 0) return IFD_OK;
  IFD_CHECK(xn && router && egu_wq && egu_s && egu_b && edn_wq && edn_s && edn_b && out, "null pointer");
  IFD_CHECK(aligned(xn, 16) && aligned(router, 16) && aligned(egu_wq, 16) && aligned(edn_wq, 16) &&
                (!shared || (aligned(sgu_wq, 16) && aligned(sdn_wq, 16))),
            "tokens, router and weights must be 16-byte aligned");
  const WsView wv = ws_view(workspace, ws_bytes);
  MdecCall c{xn, router, T, H, E, k, I, norm ? 1 : 0, shared_gate ? 1 : 0, assign ? 1 : 0, egu_wq, egu_s, egu_b,
             edn_wq, edn_s, edn_b, sgu_wq, sgu_s, sgu_b, sdn_wq, sdn_s, sdn_b, out, idx, wt, sg, logits, nullptr,
             shared_bits};
  return launch_moe_decode(c, wv.cnt, wv.body, wv.bytes, S(stream));
}

size_t ifd_moe_decode_t64_workspace(int T, int H, int I, int E, int k) {
  if (T <= 0 || T > 16 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  return with_header(mdec_layout(T, H, I, E, k, true).total);
}

int ifd_moe_decode_t64(const void* xn, int T, int H, const void* router, const float* logits_in, int E, int k,
                       int norm, int shared_gate, const void* egu_t64, const void* edn_t64, int I, const void* sgu_t64,
                       const void* sdn_t64, void* out, int assign, int* idx, float* wt, float* sg, float* logits,
                       void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(T >= 0 && T <= 16, "the decode MoE on T64 stacks takes T <= 16 tokens (T=%d)", T);
  IFD_CHECK(H > 0 && H % 512 == 0 && H / 128 < kWsCounters && I > 0 && I % 64 == 0 && E > 0 && E <= 512 && k > 0 &&
                k <= 16 && k <= E,
            "bad decode MoE shape H=%d I=%d E=%d k=%d (H multiple of 512, I of 64, E <= 512, k <= 16)", H, I, E, k);
  const bool shared = sgu_t64 != nullptr;
  IFD_CHECK(shared == (sdn_t64 != nullptr), "the shared expert needs both stacks");
  IFD_CHECK(!shared_gate || shared, "a shared gate needs a shared expert");
  IFD_CHECK((router == nullptr) != (logits_in == nullptr), "exactly one of router and logits_in");
  if (T == 0) return IFD_OK;
  IFD_CHECK(xn && egu_t64 && edn_t64 && out, "null pointer");
  IFD_CHECK(aligned(xn, 16) && (!router || aligned(router, 16)) && (!logits_in || aligned(logits_in, 4)) &&
                aligned(egu_t64, 16) && aligned(edn_t64, 16) && (!shared || (aligned(sgu_t64, 16) && aligned(sdn_t64, 16))),
            "tokens, router and stacks must be 16-byte aligned");
  const WsView wv = ws_view(workspace, ws_bytes);
  MdecCall c{xn, router, T, H, E, k, I, norm ? 1 : 0, shared_gate ? 1 : 0, assign ? 1 : 0, nullptr, nullptr, nullptr,
             nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, out, idx, wt, sg, logits,
             logits_in, 4};
  c.egu_t64 = egu_t64, c.edn_t64 = edn_t64, c.sgu_t64 = sgu_t64, c.sdn_t64 = sdn_t64;
  return launch_moe_decode(c, wv.cnt, wv.body, wv.bytes, S(stream));
}

int ifd_moe_decode(const void* xn, int T, int H, const void* router, int E, int k, int norm, int shared_gate,
                   const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b, const uint32_t* edn_wq,
                   const uint16_t* edn_s, const uint16_t* edn_b, int I, const uint32_t* sgu_wq, const uint16_t* sgu_s,
                   const uint16_t* sgu_b, const uint32_t* sdn_wq, const uint16_t* sdn_s, const uint16_t* sdn_b,
                   void* out, int assign, int* idx, float* wt, float* sg, float* logits, void* workspace,
                   size_t ws_bytes, void* stream) {
  return ifd_moe_decode_ex(xn, T, H, router, E, k, norm, shared_gate, egu_wq, egu_s, egu_b, edn_wq, edn_s, edn_b, I,
                           sgu_wq, sgu_s, sgu_b, sdn_wq, sdn_s, sdn_b, 4, out, assign, idx, wt, sg, logits, workspace,
                           ws_bytes, stream);
}

int ifd_moe_decode_logits_ex(const float* logits_in, const void* xn, int T, int H, int E, int k, int norm,
                             int shared_gate, const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b,
                             const uint32_t* edn_wq, const uint16_t* edn_s, const uint16_t* edn_b, int I,
                             const uint32_t* sgu_wq, const uint16_t* sgu_s, const uint16_t* sgu_b,
                             const uint32_t* sdn_wq, const uint16_t* sdn_s, const uint16_t* sdn_b, int shared_bits,
                             void* out, int assign, int* idx, float* wt, float* sg, void* workspace, size_t ws_bytes,
                             void* stream) {
  IFD_CHECK(shared_bits == 4 || shared_bits == 8, "shared_bits=%d must be 4 or 8", shared_bits);
  IFD_CHECK(T >= 0 && T <= 16, "the decode MoE takes T <= 16 tokens (T=%d): larger batches use ifd_moe_ffn", T);
  IFD_CHECK(H > 0 && H % 512 == 0 && H / 128 < kWsCounters && I > 0 && I % 64 == 0 && E > 0 && E <= 512 && k > 0 &&
                k <= 16 && k <= E,
            "bad decode MoE shape H=%d I=%d E=%d k=%d (H multiple of 512, I of 64, E <= 512, k <= 16)", H, I, E, k);
  const bool shared = sgu_wq != nullptr;
  IFD_CHECK(!shared || (sgu_s && sgu_b && sdn_wq && sdn_s && sdn_b), "bad shared expert");
  IFD_CHECK(!shared_gate || shared, "a shared gate needs a shared expert");
  if (T == 0) return IFD_OK;
  IFD_CHECK(logits_in && xn && egu_wq && egu_s && egu_b && edn_wq && edn_s && edn_b && out, "null pointer");
  IFD_CHECK(aligned(xn, 16) && aligned(logits_in, 4) && aligned(egu_wq, 16) && aligned(edn_wq, 16) &&
                (!shared || (aligned(sgu_wq, 16) && aligned(sdn_wq, 16))),
            "tokens and weights must be 16-byte aligned");
  const WsView wv = ws_view(workspace, ws_bytes);
  MdecCall c{xn, nullptr, T, H, E, k, I, norm ? 1 : 0, shared_gate ? 1 : 0, assign ? 1 : 0, egu_wq, egu_s, egu_b,
             edn_wq, edn_s, edn_b, sgu_wq, sgu_s, sgu_b, sdn_wq, sdn_s, sdn_b, out, idx, wt, sg, nullptr, logits_in,
             shared_bits};
  return launch_moe_decode(c, wv.cnt, wv.body, wv.bytes, S(stream));
}

size_t ifd_moe_rows_workspace(int T, int H, int I, int E, int k) {
  return ifd_moe_decode_workspace(std::min(T, 16), H, I, E, k);
}

int ifd_moe_rows(const void* xn, int T, int H, int E, int k, const int* idx, const float* wt, const float* sg,
                 const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b, const uint32_t* edn_wq,
                 const uint16_t* edn_s, const uint16_t* edn_b, int I, const void* ys, void* out, int assign,
                 void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(T >= 0, "T=%d", T);
  IFD_CHECK(H > 0 && H % 512 == 0 && H / 128 < kWsCounters && I > 0 && I % 64 == 0 && E > 0 && E <= 512 && k > 0 &&
                k <= 16 && k <= E,
            "bad MoE row shape H=%d I=%d E=%d k=%d (H multiple of 512, I of 64, E <= 512, k <= 16)", H, I, E, k);
  if (T == 0) return IFD_OK;
  IFD_CHECK(xn && idx && wt && egu_wq && egu_s && egu_b && edn_wq && edn_s && edn_b && out, "null pointer");
  IFD_CHECK(!ys || sg, "the shared expert's rows need their gate weights sg");
  IFD_CHECK(aligned(xn, 16) && aligned(egu_wq, 16) && aligned(edn_wq, 16) && aligned(idx, 4) && aligned(wt, 4) &&
                (!ys || aligned(ys, 2)),
            "tokens and weights must be 16-byte aligned");
  const WsView wv = ws_view(workspace, ws_bytes);
  MdecCall c{xn, nullptr, T, H, E, k, I, 1, 0, assign ? 1 : 0, egu_wq, egu_s, egu_b, edn_wq, edn_s, edn_b, nullptr,
             nullptr, nullptr, nullptr, nullptr, nullptr, out, const_cast<int*>(idx), const_cast<float*>(wt),
             const_cast<float*>(sg), nullptr, nullptr, 4};
  c.routed = 1, c.ys = ys;
  return launch_moe_decode(c, wv.cnt, wv.body, wv.bytes, S(stream));
}

size_t ifd_moe_rows_t64_workspace(int T, int H, int I, int E, int k) {
  if (T <= 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  size_t need = 0;  // the launch groups hold up to 16 tokens, the last one fewer
  for (int t = 1; t <= std::min(T, 16); t++) need = std::max(need, mdec_layout(t, H, I, E, k, true).total);
  return with_header(need);
}

int ifd_moe_rows_t64(const void* xn, int T, int H, int E, int k, const int* idx, const float* wt, const float* sg,
                     const void* egu_t64, const void* edn_t64, int I, const void* sgu_t64, const void* sdn_t64,
                     const void* ys, void* out, int assign, void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(T >= 0, "T=%d", T);
  IFD_CHECK(H > 0 && H % 512 == 0 && H / 128 < kWsCounters && I > 0 && I % 64 == 0 && E > 0 && E <= 512 && k > 0 &&
                k <= 16 && k <= E,
            "bad MoE row shape H=%d I=%d E=%d k=%d (H multiple of 512, I of 64, E <= 512, k <= 16)", H, I, E, k);
  if (T == 0) return IFD_OK;
  IFD_CHECK(xn && idx && wt && egu_t64 && edn_t64 && out, "null pointer");
  const bool shared = sgu_t64 != nullptr;
  IFD_CHECK(shared == (sdn_t64 != nullptr), "the shared expert needs both stacks");
  IFD_CHECK(!(shared && ys), "the shared expert as weights or as rows, not both");
  IFD_CHECK(!(ys || shared) || sg, "the shared expert needs its gate weights sg");
  IFD_CHECK(aligned(xn, 16) && aligned(egu_t64, 16) && aligned(edn_t64, 16) && aligned(idx, 4) && aligned(wt, 4) &&
                (!ys || aligned(ys, 2)) && (!shared || (aligned(sgu_t64, 16) && aligned(sdn_t64, 16))),
            "tokens and stacks must be 16-byte aligned");
  const WsView wv = ws_view(workspace, ws_bytes);
  MdecCall c{xn, nullptr, T, H, E, k, I, 1, 0, assign ? 1 : 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
             nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, out, const_cast<int*>(idx), const_cast<float*>(wt),
             const_cast<float*>(sg), nullptr, nullptr, 4};
  c.routed = 1, c.ys = ys;
  c.egu_t64 = egu_t64, c.edn_t64 = edn_t64, c.sgu_t64 = sgu_t64, c.sdn_t64 = sdn_t64;
  return launch_moe_decode(c, wv.cnt, wv.body, wv.bytes, S(stream));
}

int ifd_moe_decode_logits(const float* logits_in, const void* xn, int T, int H, int E, int k, int norm,
                          int shared_gate, const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b,
                          const uint32_t* edn_wq, const uint16_t* edn_s, const uint16_t* edn_b, int I,
                          const uint32_t* sgu_wq, const uint16_t* sgu_s, const uint16_t* sgu_b,
                          const uint32_t* sdn_wq, const uint16_t* sdn_s, const uint16_t* sdn_b, void* out, int assign,
                          int* idx, float* wt, float* sg, void* workspace, size_t ws_bytes, void* stream) {
  return ifd_moe_decode_logits_ex(logits_in, xn, T, H, E, k, norm, shared_gate, egu_wq, egu_s, egu_b, edn_wq, edn_s,
                                  edn_b, I, sgu_wq, sgu_s, sgu_b, sdn_wq, sdn_s, sdn_b, 4, out, assign, idx, wt, sg,
                                  workspace, ws_bytes, stream);
}

}  // extern "C"
