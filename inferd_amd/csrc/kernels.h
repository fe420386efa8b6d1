// Internal launcher interface between the C ABI (capi.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ifd {

// One dense 4- or 8-bit GEMM request: C (mode) = A . W^T. A is bf16 [M][lda] (or int8 [M][K] + XS for W4A8 / W8A8).
struct W4Gemm {
  const void* A = nullptr;
  int lda = 0;
  const float* XS = nullptr;  // W4A8 only: (sx, sx * sum xq) per row and group
  const uint32_t* wq = nullptr;
  const uint16_t* s = nullptr;
  const uint16_t* b = nullptr;
  int N = 0, K = 0, ldk = 0;  // ldk: weight row length in values (K-slice views), never 0 here
  uint32_t xr = 0;
  void* C = nullptr;
  int ldc = 0, M = 0, mode = 0;
  int bits = 4;  // 4 or 8 (MLX affine, group 64)
};

// Decode GEMV path (M <= 128).
size_t qmv_workspace(int M, int N, int K);
int launch_qmv(const W4Gemm& g, void* ws, size_t ws_bytes, hipStream_t st);
// Prefill GEMM path (any M).
size_t qmm_workspace(int M, int N, int K);
int launch_qmm(const W4Gemm& g, void* ws, size_t ws_bytes, hipStream_t st);
// W4A8.
int launch_a8_quant(const uint16_t* A, int lda, int M, int K, int per_token, int8_t* U, float* XS, hipStream_t st);
size_t w4a8_workspace(int M, int N, int K);
int launch_w4a8(const W4Gemm& g, int per_token, void* ws, size_t ws_bytes, hipStream_t st);
int launch_flip(uint32_t* wq, size_t n32, uint32_t mask, hipStream_t st);
int launch_silu_mul(const uint16_t* gu, int ldgu, uint16_t* h, int ldh, int I, int rows, hipStream_t st);
int launch_rmsnorm(const uint16_t* x, int in_stride, const uint16_t* w, uint16_t* out, int out_stride, int rows,
                   int D, float eps, hipStream_t st);
// Fused producers (fused.hip).
int launch_rmsnorm_a8(const uint16_t* x, int in_stride, const uint16_t* w, uint16_t* out, int out_stride, int rows,
                      int D, float eps, int per_token, int8_t* U, float* XS, hipStream_t st);
int launch_silu_mul_a8(const uint16_t* gu, int ldgu, int I, int rows, int per_token, int8_t* U, float* XS,
                       hipStream_t st);
int launch_splitk_res_norm(const float* part, int S, uint16_t* x, int ldx, const uint16_t* w, uint16_t* out,
                           int out_stride, int rows, int D, float eps, int a8, int8_t* U, float* XS, hipStream_t st);
// Every public workspace starts with kWsHeader bytes of completion counters (uint32), which the library keeps at zero
// between calls: the caller zeroes them once when the workspace is allocated. Kernel scratch follows the header.
constexpr size_t kWsHeader = 4096;
constexpr int kWsCounters = (int)(kWsHeader / sizeof(unsigned));
// Zeroes the kWsHeader-byte counter header at ws with a fill kernel on st (workspace.hip).
int launch_zero_header(void* ws, hipStream_t st);
// Measurement probes (probe.hip): a coalesced stream read of `bytes` and an MFMA-only loop.
int launch_probe_read(const void* src, size_t bytes, void* sink, int blocks, hipStream_t st);
int launch_probe_mfma(int int8, int iters, int blocks, float* out, hipStream_t st);

// Library-internal store mode past the public 0 (bf16), 1 (bf16 residual add) and 2 (fp32): the GEMM's N columns are
// [gate (N/2) | up (N/2)] and C receives the SwiGLU h [M][N/2] (ldc = its row stride), bit-identical to a mode-0 GEMM
// followed by silu_mul.
constexpr int kModeSwiglu = 3;
// Split-K reduction: C (mode) = sum over S partials [S][M][N] fp32, in split order.
int launch_splitk_reduce(const float* part, int S, int M, int N, void* C, int ldc, int mode, hipStream_t st);
// Workspace of a GEMM epilogue with S K-splits: the fp32 partials, or for the SwiGLU mode without a split the bf16
// product [M][N] that silu_mul then reads.
size_t epilogue_ws_bytes(int S, int M, int N, int mode);
// After a GEMM kernel that wrote partials (S > 1) or, in the SwiGLU mode, the bf16 product into ws: the reduction or
// silu_mul into C. Nothing to do otherwise.
int launch_epilogue(const void* ws, int S, int M, int N, void* C, int ldc, int mode, hipStream_t st);

// T64 layout (t64.h).
int launch_pack_t64(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr,
                    int E, void* out, hipStream_t st);
size_t qmv_t_workspace(int M, int N, int K, int mode, int bits = 4);
size_t gemm_t_workspace(int M, int N, int K, int mode);
// 256-row-tile prefill GEMM on T64 weights (modes 0-2); gemm_t routes prefill shapes to it.
size_t gemm_t8_workspace(int M, int N, int K);
int launch_gemm_t8(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                   void* ws, size_t ws_bytes, hipStream_t st);
int launch_gemm_t(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                  void* ws, size_t ws_bytes, hipStream_t st);
// Stream-K GEMM for decode batches (gemm_sk.hip): every CU streams an equal share of the weights; the cut tiles are
// summed by a fixup kernel.
bool gemm_sk_applies(int M, int N, int K, int mode);
size_t gemm_sk_workspace(int M, int N, int K, int mode);
int launch_gemm_sk(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                   void* ws, size_t ws_bytes, hipStream_t st);
// The fixup of a 128-row-tile stream-K split (gemm_sk.hip): sums the pieces of the cut tiles among the stream-K
// tiles tile0 .. tile0 + ntiles - 1, scales row m by rs[m rs_stride] (rs null: no scale) and stores them.
int launch_sk_fixup_rows(const float* part, int tiles_m, int tiles_n, int tile0, int ntiles, int G, int nblk, void* C,
                         int ldc, int M, int N, int mode, const float* rs, int rs_stride, hipStream_t st);
// W4A8 on T64 weights, per-token int8 activations (U [M][K], XS [M][G][2] from a8_quant).
size_t w4a8_t_workspace(int M, int N, int K);
int launch_w4a8_t(const int8_t* U, const float* XS, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                  void* ws, size_t ws_bytes, hipStream_t st);
// The decode GEMV on T64x8 weights (M <= 16, K % 128 == 0; the qmv8 arithmetic s sum q x + b sum x); its workspace
// is qmv_t_workspace(M, N, K, mode, 8).
int launch_qmv_t8(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                  unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st);
// The same stream-K GEMM on T64x8 weights (8-bit codes, dequantized to bf16(s q + b)); any M >= 1.
size_t gemm_sk8_workspace(int M, int N, int K);
int launch_gemm_sk8(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                    void* ws, size_t ws_bytes, hipStream_t st);
// T64x8 (t64.h): the repack of an MLX 8-bit linear, and W8A8 on it with per-token int8 activations.
int launch_pack_t64x8(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr,
                      void* out, hipStream_t st);
size_t w8a8_t_workspace(int M, int N, int K);
int launch_w8a8_t(const int8_t* U, const float* XS, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                  void* ws, size_t ws_bytes, hipStream_t st);
// cnt: kWsCounters zeroed counters (the workspace header) for the in-kernel split-K fixup; null -> a reduction kernel
int launch_qmv_t(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                 unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st);
// n linears sharing A and K in one decode-GEMV launch (ifd_gemm_t64_multi)
size_t qmv_t_multi_workspace(int M, int n, const int* Ns, int K);
int launch_qmv_t_multi(const uint16_t* A, int lda, int n, const void* const* wts, const int* Ns, int K,
                       void* const* Cs, const int* ldcs, int M, int mode, unsigned* cnt, void* ws, size_t ws_bytes,
                       hipStream_t st);
// W4A8 with per-(row, 64-group) int8 activations on T64 weights, in the affine bf16-MFMA form (xq as exact bf16
// integers): the prep writes Ab = bf16(U) [M][K] and sxT = sx transposed [G][Mp] (zero past M); M <= 16 runs the
// decode GEMV (qmv_t_workspace(M, N, K, mode)), more rows the affine k_gemm_t (gemm_t_a8_workspace).
int w4a8g_mp(int M);
int launch_w4a8g_prep(const int8_t* U, const float* XS, int M, int K, uint16_t* Ab, float* sxT, int Mp, hipStream_t st);
int launch_qmv_t_a8(const uint16_t* Ab, const float* XS, const void* wt, int N, int K, void* C, int ldc, int M,
                    int mode, unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st);
size_t gemm_t_a8_workspace(int M, int N, int K, int mode);
int launch_gemm_t_a8(const uint16_t* Ab, const float* sxT, int Mp, const void* wt, int N, int K, void* C, int ldc,
                     int M, int mode, void* ws, size_t ws_bytes, hipStream_t st);

// MoE.
int launch_router_logits(const uint16_t* x, const uint16_t* w, int T, int H, int E1, int out_bf16, void* logits,
                         hipStream_t st);
int launch_moe_route(const void* logits, int logits_bf16, int T, int E, int k, int stride, int norm, int shared_gate,
                     int* idx, float* wt, float* sg, hipStream_t st);
int moe_tiles_max(int R, int E);
size_t moe_dispatch_workspace(int R, int E);
int launch_moe_dispatch(const int* idx, int R, int E, int* offsets, int* perm, int* inv, int* tiles, int* ntiles,
                        void* ws, size_t ws_bytes, hipStream_t st);
// The same with tile_rows-row tiles and, when shared_rows > 0, a segment for the shared expert as expert E: sorted
// rows [R, R + shared_rows) are tokens 0, 1, ... (perm = t * kdiv), tiles after the routed ones, offsets[E + 1] =
// R + shared_rows. offsets holds E + 2 entries then, perm R + shared_rows, tiles moe_tiles_max(R + shared_rows, E + 1).
int launch_moe_dispatch(const int* idx, int R, int E, int* offsets, int* perm, int* inv, int* tiles, int* ntiles,
                        void* ws, size_t ws_bytes, hipStream_t st, int tile_rows, int shared_rows, int kdiv);
int launch_moe_gather(const uint16_t* x, const int* perm, int div, int R, int H, uint16_t* xs, hipStream_t st);
int launch_moe_gather_qmm(const uint16_t* A, const int* perm, int div, const int* tiles, const int* ntiles,
                          const int* offsets, int max_tiles, const uint32_t* wq, const uint16_t* s,
                          const uint16_t* b, int N, int K, int silu, uint16_t* C, int R, hipStream_t st,
                          int bits = 4);
int launch_moe_gather_qmm_a8(const int8_t* U, const float* XS, const int* perm, int div, const int* tiles,
                             const int* ntiles, const int* offsets, int max_tiles, const uint32_t* wq,
                             const uint16_t* s, const uint16_t* b, int N, int K, int silu, uint16_t* C, int R,
                             hipStream_t st);
int launch_moe_combine(uint16_t* out, const uint16_t* yd, const float* wt, const uint16_t* ys, const float* sg,
                       const int* inv, int T, int H, int k, int assign, hipStream_t st);
// The gathered expert GEMM on T64 expert stacks (moe_t64.hip): the dispatch's tiles of tile_rows (32 or 64) rows,
// the shared expert (wsh) as expert E, rows = sorted rows of C (ldc its row stride). part (at least
// moe_gather_t64_part_bytes(tile_rows) bytes) and cnt (the workspace's zeroed counter header): the balanced schedule,
// whose cut items sum their K ranges' pieces in K order; part null: whole items per block (the same bits as
// launch_moe_gather_qmm).
size_t moe_gather_t64_part_bytes(int tile_rows);
int launch_moe_gather_qmm_t64(const uint16_t* A, int lda, const int* perm, int div, const int* tiles,
                              const int* ntiles, const int* offsets, int tile_rows, const void* wt, const void* wsh,
                              int E, int N, int K, int silu, uint16_t* C, int ldc, int rows, float* part,
                              size_t part_bytes, unsigned* cnt, hipStream_t st);

// Decode MoE for T <= 16 tokens (moe_dec.hip): router, routing + distinct-expert plan, gate/up + SwiGLU, down +
// combine; the combine's counters are H / 128 uint32 of the workspace header.
struct MdecCall {
  const void* xn;
  const void* router;
  int T, H, E, k, I, norm, shared_gate, assign;
  const uint32_t* egu_wq;
  const uint16_t* egu_s;
  const uint16_t* egu_b;
  const uint32_t* edn_wq;
  const uint16_t* edn_s;
  const uint16_t* edn_b;
  const uint32_t* sgu_wq;
  const uint16_t* sgu_s;
  const uint16_t* sgu_b;
  const uint32_t* sdn_wq;
  const uint16_t* sdn_s;
  const uint16_t* sdn_b;
  void* out;
  int* idx;
  float* wt;
  float* sg;
  float* logits;
  const float* logits_in;  // non-null: routing starts from these fp32 logits [T][E1] (router unused)
  int sh_bits = 4;         // the shared expert's width, 4 or 8
  int routed = 0;          // idx / wt / sg hold the caller's routing (router and logits unused); any T
  const void* ys = nullptr;  // with routed: the shared expert's output rows [T][H] (bf16) for the combine, or null
  // the T64 path (T <= 8, not routed): the stacks packed by ifd_pack_t64 (egu [E][2I][H], edn [E][H][I]) and the
  // shared expert's T64 copies (4-bit) or null; the MLX-layout pointers are then unused
  const void* egu_t64 = nullptr;
  const void* edn_t64 = nullptr;
  const void* sgu_t64 = nullptr;
  const void* sdn_t64 = nullptr;
};
struct MdecLayout {
  size_t part, plan, act, d, idx, wt, sg, gpart, total;
  int gS, gps;  // the T64 path's gate/up K split
};
MdecLayout mdec_layout(int T, int H, int I, int E, int k, bool t64 = false);
int launch_moe_decode(const MdecCall& c, unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st);

}  // namespace ifd
