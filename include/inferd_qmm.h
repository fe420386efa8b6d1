/* inferd_qmm.h — C ABI of the MI355X (gfx950) W4 quantized-matmul hot path.
 *
 * Drop-in for the kernels under inferd's engine-facing operators
 *   void Qwen35::gemm(Enc&, const BufRef& A, const QLinear& W, const BufRef& C, int M, int mode, bool defer)
 *        (reference engine/src/qwen35.h:1465)
 *   void Qwen35::encode_moe(Enc&, const Layer&, int T)            (reference engine/src/qwen35.h:1869)
 * The C++ shim that keeps those signatures is inferd_amd/csrc/qwen35_ops.h.
 *
 * Conventions (all entry points):
 *  - Pointers are caller-owned DEVICE pointers; nothing is allocated, freed or synchronised inside. Work is enqueued
 *    on `stream` (a hipStream_t; NULL = the default stream) in call order, as the reference encodes into the
 *    caller's serial compute encoder (engine/src/gpu.h:122-163).
 *  - bf16 tensors are 16-bit bit patterns (uint16_t storage), row-major.
 *  - Weights: MLX affine 4-bit, group 64 (reference engine/src/weights.h:226-236): wq uint32 [N][ldk/8] with element
 *    j of a little-endian word at bits 4j; s, b bf16 [N][ldk/64]; w[n][k] = s[n][k/64] * q[n][k] + b[n][k/64].
 *    ldk = 0 means ldk = K; ldk > K is a K-slice view (reference kslice_of, weights.h:259-268).
 *    xr = 0x88888888 when the nibbles were flipped in place by ifd_flip_w4 (reference QLinear::flipped), else 0.
 *  - GEMM store modes (reference engine/kernels/core.metal:14-15): 0 C = bf16(y); 1 C = bf16(y + C) (residual);
 *    2 C = y as fp32.
 *  - Every entry point returns IFD_OK or an error code and never exits the process (the reference prints and calls
 *    exit(1), qwen35.h:1469, 1477); ifd_last_error() returns a message for the calling thread.
 *  - Workspaces (the *_workspace() queries give the bytes, 0 = none needed; pass at least that many): the first 4096
 *    bytes of a workspace are completion counters that the library keeps at zero between calls. ZERO THEM ONCE when
 *    the workspace is allocated (hipMemset, or allocate zeroed); the rest is scratch, any content. One workspace may
 *    serve every entry point, but calls that share a workspace must not run concurrently.
 */
#ifndef INFERD_QMM_H
#define INFERD_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  IFD_OK = 0,
  IFD_ERR_ARG = 1,         /* bad shape, stride, null or misaligned pointer */
  IFD_ERR_WORKSPACE = 2,   /* workspace missing or smaller than the *_workspace() query */
  IFD_ERR_LAUNCH = 3,      /* HIP reported an error launching a kernel */
  IFD_ERR_UNSUPPORTED = 4  /* valid request outside what this build implements */
};

int ifd_version(void);
const char* ifd_status_str(int status);
const char* ifd_last_error(void);

/* ---- workspace counter header (no counterpart in the reference, whose split-K scratch holds no counters) -------
 * ifd_workspace_check synchronises `stream`, reads the first 4096 bytes of the workspace and returns IFD_OK when
 * every counter is zero, IFD_ERR_WORKSPACE (with the first non-zero counter in ifd_last_error()) otherwise. A call
 * that failed after a partial launch, or a kernel that did not finish, can leave counters non-zero, and later
 * split-K results on that workspace would be wrong. ifd_workspace_reset zeroes the header on `stream` with a fill
 * kernel (no memset node: it may be captured into a HIP graph). ws_bytes >= 4096. */
int ifd_workspace_check(const void* workspace, size_t ws_bytes, void* stream);
int ifd_workspace_reset(void* workspace, size_t ws_bytes, void* stream);

/* ---- dense linears (reference Qwen35::gemm and its sub-paths, engine/src/qwen35.h:1465-1558) ---------------- */

/* Bytes of workspace ifd_gemm_w4 / ifd_qmv_w4 / ifd_qmm_w4 need for this shape (split-K partials). */
size_t ifd_gemm_w4_workspace(int M, int N, int K);

/* Decode GEMV path, M <= 128 (replaces qmv4 / qmm_splitk + splitk_reduce, core.metal:85-171,
 * qmm_splitk.metal:14-107; host qwen35.h:1520-1556). A bf16 [M][lda]. */
int ifd_qmv_w4(const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
               int ldk, uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes,
               void* stream);

/* Prefill GEMM path, any M (replaces MLX affine_qmm_t_nax, quantized_nax.h:1206-1267; host mlx_qmm,
 * qwen35.h:1427-1462). */
int ifd_qmm_w4(const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
               int ldk, uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes,
               void* stream);

/* Routed GEMM: picks the GEMV path for M <= 128 and the prefill path above (reference Qwen35::gemm,
 * qwen35.h:1465). */
int ifd_gemm_w4(const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
                int ldk, uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes,
                void* stream);

/* In-place flip, wq[i] ^= mask for i < n32 (reference w_flip, w4a8.metal:19-22; flip, qwen35.h:1306-1322): mask
 * 0x88888888 for 4-bit weights, 0x80808080 for 8-bit. */
int ifd_flip_w4(uint32_t* wq, size_t n32, uint32_t mask, void* stream);

/* SwiGLU h[r][i] = bf16(float(bf16(g * sigmoid(g))) * u) over rows gu = [gate (I) | up (I)]
 * (reference silu_mul, core.metal:777-787; moe_silu_mul, moe.metal:103-111). */
int ifd_silu_mul(const void* gu, void* h, int I, int rows, void* stream);

/* RMS norm over rows of D bf16 values: out[r][i] = bf16(float(x[r][i]) * rsqrt(sum_i x^2 / D + eps) * float(w[i])),
 * fp32 sum of squares (reference rmsnorm, core.metal:486-500; host Qwen35::rmsnorm, qwen35.h:2004-2012; the
 * normalisation encode_moe applies first, rmsnorm_for, qwen35.h:1982-2002). Rows are in_stride / out_stride
 * values apart. */
int ifd_rmsnorm(const void* x, int in_stride, const void* w, void* out, int out_stride, int rows, int D, float eps,
                void* stream);

/* ---- fused producers of the decode step (bit-identical to their unfused sequences) -------------------------------
 * rmsnorm fused with the W4A8 activation quantization of the next GEMM: out as ifd_rmsnorm, and U int8 [rows][D] /
 * XS float [rows][D/64][2] as ifd_a8_quant of out (per_token as there). Replaces the reference's rmsnorm_a8
 * (engine/kernels/core.metal:502-537, per group there), issued by rmsnorm_for (engine/src/qwen35.h:1982-2000).
 * D % 64 == 0. */
int ifd_rmsnorm_a8(const void* x, int in_stride, const void* w, void* out, int out_stride, int rows, int D, float eps,
                   int per_token, int8_t* U, float* XS, void* stream);
/* silu_mul fused with the W4A8 activation quantization of the down projection: U [rows][I] / XS [rows][I/64][2] of
 * h = silu_mul(gu) (h is not written), as ifd_silu_mul then ifd_a8_quant. Replaces silu_mul_a8
 * (core.metal:789-814; issued at qwen35.h:2874). I % 64 == 0. */
int ifd_silu_mul_a8(const void* gu, int I, int rows, int per_token, int8_t* U, float* XS, void* stream);
/* A deferred split-K residual reduce fused into the next rmsnorm: x[r] = bf16(sum_z part[z][r] + x[r]) in split
 * order (as the split-K reduction with mode 1), then out = rmsnorm(x) and, when U is not null, U / XS as
 * ifd_a8_quant of out. part fp32 [S][rows][D]. Replaces splitk_res_norm / splitk_res_norm_a8 (core.metal:539-595),
 * issued by rmsnorm_for (qwen35.h:1982-1998). With U, D % 64 == 0. */
int ifd_splitk_res_norm(const float* part, int S, void* x, int ldx, const void* w, void* out, int out_stride, int rows,
                        int D, float eps, int per_token, int8_t* U, float* XS, void* stream);

/* ---- 8-bit weights (reference qmv8, core.metal:175-248; w4a8_gemm with BITS = 8, w4a8.metal:43-98, 104-109; the
 * 8-bit routes of Qwen35::gemm, qwen35.h:1520-1558) --------------------------------------------------------------
 * MLX affine 8-bit, group 64: wq uint32 [N][ldk/4] with element j of a little-endian word in byte j; s, b as for
 * 4 bits; w = s q + b, q in 0..255. xr = 0x80808080 when the bytes were flipped in place (ifd_flip_w4 with that
 * mask: q ^ 0x80), else 0. Same arguments, workspace and store modes as the 4-bit entry points. */
size_t ifd_gemm_w8_workspace(int M, int N, int K);
/* Routed GEMM: the qmv8 arithmetic (s sum q x + b sum x per group, fp32) for M <= 32, bf16(s q + b) dequant with
 * fp32 accumulation (MLX's 8-bit qmm) above. */
int ifd_gemm_w8(const void* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
                int ldk, uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes,
                void* stream);
/* W8A8: C (mode) = sum_g [ s sx P + (b + 128 s) (sx sum xq) ], P = sum (q - 128) xq over the group (exact int32);
 * U, XS from ifd_a8_quant with the same per_token. */
int ifd_qmm_w8a8(const int8_t* U, const float* XS, int per_token, const uint32_t* wq, const uint16_t* s,
                 const uint16_t* b, int N, int K, int ldk, uint32_t xr, void* C, int ldc, int M, int mode,
                 void* workspace, size_t ws_bytes, void* stream);
size_t ifd_qmm_w8a8_workspace(int M, int N, int K);

/* ---- T64: the MI355X weight layout (no counterpart in the reference; its role is that of the reference's
 * load-time weight transforms, flip and the lane4/qmst copies, qwen35.h:1209-1322) -------------------------------
 * A one-time repack of the MLX layout into 1152-byte tiles (per 64-group and 32-column band: the codes in MFMA
 * fragment order + the (s, b) pairs), group-major, so that decode streams HBM in 1 KB contiguous wave loads.
 * Same size as the source (0.5625 B per weight); E stacked experts are packed expert by expert. */
size_t ifd_t64_bytes(int N, int K, int E);
int ifd_pack_t64(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr, int E,
                 void* out, void* stream);
size_t ifd_gemm_t64_workspace(int M, int N, int K);
/* C (mode) = A . W^T with W in T64 layout (K % 256 == 0). */
int ifd_gemm_t64(const void* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                 void* workspace, size_t ws_bytes, void* stream);
/* ifd_gemm_t64 without a caller workspace. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * workspace is a static device array of IFD_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; requests
 * whose ifd_gemm_t64_workspace exceeds it return IFD_ERR_WORKSPACE. Each call clears the array's counter header with
 * a fill kernel and allocates nothing. Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race. Same results, bit for bit, as ifd_gemm_t64. */
#define IFD_NOALLOC_SCRATCH_BYTES ((size_t)68 << 20)
int ifd_gemm_t64_noalloc(const void* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                         void* stream);
/* Gate/up projection with its SwiGLU: W (T64) holds [gate (N/2) | up (N/2)] rows and H [M][N/2] (row stride ldh)
 * receives silu_mul of the bf16 product: bit-identical to ifd_gemm_t64 (mode 0) followed by ifd_silu_mul for
 * M <= 16 and on the prefill tiles; on the stream-K rows between, the fused tiles cut K at other places than the
 * plain GEMM's, so a gate or up sum may differ from it by one bf16 step before the SwiGLU. Replaces
 * the reference's gemm + silu_mul pair (qwen35.h:1910-1912, shared expert; qwen35.h:2868-2878, dense MLP) with one
 * call that never stores the [M][N] product when K is split (the SwiGLU runs in the split-K reduction).
 * N % 16 == 0, ldh % 8 == 0, A, H and the workspace 16-byte aligned. */
size_t ifd_gemm_t64_swiglu_workspace(int M, int N, int K);
int ifd_gemm_t64_swiglu(const void* A, int lda, const void* wt, int N, int K, void* H, int ldh, int M,
                        void* workspace, size_t ws_bytes, void* stream);
/* Several T64 linears that share one input, in one launch: C_l (mode 0-2) = A . W_l^T for l < n (1 <= n <= 8),
 * W_l [Ns[l]][K] packed by ifd_pack_t64, C_l with leading dimension ldcs[l]; M <= 16 (the decode GEMV), K % 256 == 0.
 * No counterpart in the reference, which issues one gemm() per linear (e.g. in_proj then iproj on the same xn,
 * engine/src/qwen35.h:2577-2581): this is that set as one launch, the decode GEMV over the linears' concatenated
 * bands with one K split for all of them. It amortises the per-launch cost (about 2.5 us back to back) that bounds a
 * small decode linear (5120 x 5120 at M = 1). Same qmv arithmetic as ifd_gemm_t64 at these rows; the K split (and so
 * the fp32 summation order) is planned for the concatenated width. The workspace's counter header is required when
 * the launch splits K. */
size_t ifd_gemm_t64_multi_workspace(int M, int n, const int* Ns, int K);
int ifd_gemm_t64_multi(const void* A, int lda, int n, const void* const* wts, const int* Ns, int K, void* const* Cs,
                       const int* ldcs, int M, int mode, void* workspace, size_t ws_bytes, void* stream);

/* ---- W4A8 (reference a8_quant + w4a8_gemm, w4a8.metal:24-98; host w4a8, qwen35.h:1323-1366) ------------------ */

/* Activation quantizer: U int8 [M][K], XS float [M][K/64][2] = (sx, sx * sum xq) per row and group.
 * per_token = 0: one scale per row and 64-group (the reference's a8_quant, w4a8.metal:24-41); 1: one scale per row
 * (amax over K), repeated in every group's XS entry. sx = amax / 127 (1 if amax == 0), xq = rint(x / sx).
 * per_token = 2: the int8 prefill's quantizer (reference qa8_quant, qa8.metal:30-49): per 64-group,
 * xq = clamp(rint(x * (127 / amax)), -127, 127) (0 if amax == 0), sx = amax / 127; U in natural K order. With
 * ifd_qmm_w4a8 (per_token = 0) it gives the reference's qa8 path (qa8_gemm, qa8.metal:52-210: the same per-group
 * identity on unflipped codes). K % 64 == 0; A 16-byte aligned with lda % 8 == 0, U 8-byte aligned. */
int ifd_a8_quant(const void* A, int lda, int M, int K, int per_token, int8_t* U, float* XS, void* stream);

/* C (mode) = sum_g [ s sx P + b (sx sum xq) ], P = sum q xq over the group (exact int32); U, XS from
 * ifd_a8_quant with the same per_token. */
int ifd_qmm_w4a8(const int8_t* U, const float* XS, int per_token, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N,
                 int K, int ldk, uint32_t xr, void* C, int ldc, int M, int mode, void* workspace, size_t ws_bytes,
                 void* stream);
size_t ifd_qmm_w4a8_workspace(int M, int N, int K);

/* W4A8 on T64 weights (per-token activations from ifd_a8_quant with per_token = 1; W packed by ifd_pack_t64):
 * C (mode) = sx[m] * sum_g (S P_g + B X_g) on int8 MFMA, the w4a8_gemm identity (w4a8.metal:8, 78-87) with unflipped
 * codes. K % 256 == 0. per_token = 0 returns IFD_ERR_UNSUPPORTED. */
size_t ifd_gemm_t64_w4a8_workspace(int M, int N, int K);
int ifd_gemm_t64_w4a8(const int8_t* U, const float* XS, int per_token, const void* wt, int N, int K, void* C, int ldc,
                      int M, int mode, void* workspace, size_t ws_bytes, void* stream);

/* ---- T64x8: the T64 arrangement for 8-bit weights (no counterpart in the reference, as T64) ---------------------
 * 2176-byte tiles per 64-group and 32-column band: the codes as int8 q - 128 in v_mfma_i32_32x32x32_i8 B-fragment
 * order + the (s, b) pairs; group-major. Same size as the MLX 8-bit source (1.0625 B per weight). xr: the source's
 * flip mask (0, or 0x80808080 for a flipped 8-bit layer). */
size_t ifd_t64x8_bytes(int N, int K);
int ifd_pack_t64x8(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr,
                   void* out, void* stream);
/* C (mode) = A . W^T with W in T64x8 layout (K % 64 == 0). M <= 16 with K % 128 == 0: the reference's qmv8
 * arithmetic (core.metal:175-248: per group s * sum q x + b * sum x in fp32) on the T64 decode GEMV; otherwise every
 * weight dequantized to bf16(s q + b) with fp32 accumulation, MLX's 8-bit qmm (quantized.h:528-535, the reference's
 * affine_qmm_t at BITS = 8), on the stream-K bf16 MFMA kernel. */
size_t ifd_gemm_t64x8_workspace(int M, int N, int K);
int ifd_gemm_t64x8(const void* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                   void* workspace, size_t ws_bytes, void* stream);
/* W8A8 on T64x8 weights (per-token activations from ifd_a8_quant with per_token = 1): replaces ifd_qmm_w8a8 for
 * packed weights, the same sum C (mode) = sx[m] * sum_g [ s P_g + (b + 128 s) X_g ], P_g = sum (q - 128) xq (exact
 * int32), as w4a8_gemm with BITS = 8 (w4a8.metal:43-98, :57). K % 64 == 0. per_token = 0 returns
 * IFD_ERR_UNSUPPORTED. */
size_t ifd_gemm_t64x8_w8a8_workspace(int M, int N, int K);
int ifd_gemm_t64x8_w8a8(const int8_t* U, const float* XS, int per_token, const void* wt, int N, int K, void* C,
                        int ldc, int M, int mode, void* workspace, size_t ws_bytes, void* stream);

/* ---- MoE (reference encode_moe sorted path, qwen35.h:1869-1980; kernels moe.metal:60-187) -------------------- */

/* Router logits [T][E1] = x [T][H] . W [E1][H]^T, bf16 operands, fp32 accumulation; out_bf16 = 1 rounds to bf16
 * (reference: bf16 GEMM logits for >= 64 rows, qwen35.h:1919-1929), 0 writes fp32 (moe_qmv16f, moe.metal:198-213). */
int ifd_moe_router_logits(const void* x, const void* w, int T, int H, int E1, int out_bf16, void* logits,
                          void* stream);

/* Softmax top-k (reference moe_route / moe_route_bf, moe.metal:60-101, qwen4.metal:1462-1503): idx int [T][k],
 * wt float [T][k] (renormalised over the picks when norm != 0), sg float [T] = sigmoid(logit[E]) when
 * shared_gate == 1, 1.0 when 0 (always-on shared expert). Ties go to the lowest expert index. E <= 512, k <= 16. */
int ifd_moe_route(const void* logits, int logits_bf16, int T, int E, int k, int stride, int norm, int shared_gate,
                  int* idx, float* wt, float* sg, void* stream);

/* Stable counting sort of routed rows r = t*k + j by expert (reference moe_sort, moe.metal:130-161, whose order
 * inside a segment is atomic-order; this one keeps row order): offsets int [E+1], perm int [R] (sorted position ->
 * r), inv int [R] (r -> sorted position). tiles int [ifd_moe_tiles_max(R, E)][2] = (expert, first sorted row) of
 * every 32-row tile of every expert segment and ntiles int [1]: the schedule of ifd_moe_gather_qmm
 * (reference schedule_row_tile, third_party/mlx/.../steel/utils.h:502-542). Workspace: ifd_moe_dispatch_workspace. */
int ifd_moe_tiles_max(int R, int E);
size_t ifd_moe_dispatch_workspace(int R, int E);
int ifd_moe_dispatch(const int* idx, int R, int E, int* offsets, int* perm, int* inv, int* tiles, int* ntiles,
                     void* workspace, size_t ws_bytes, void* stream);

/* xs[q][:] = x[perm[q] / div][:] (reference moe_gather, moe.metal:163-170). */
int ifd_moe_gather(const void* x, const int* perm, int div, int R, int H, void* xs, void* stream);

/* Gathered expert GEMM over expert-sorted rows (reference affine_gather_qmm_rhs, quantized_nax.h:1467-1681):
 * C[q][n] = bf16( sum_k A_row(q)[k] * w_e[n][k] ), e = expert of sorted row q, A_row(q) = A[perm[q] / div] when
 * perm != NULL else A[q]; offsets/tiles/ntiles from ifd_moe_dispatch, max_tiles = ifd_moe_tiles_max(R, E).
 * Stacks wq [E][N][K/8], s/b [E][N][K/64] (reference MoeW, moe.h:8-11). silu != 0 (N even): the stack holds [gate (N/2) | up (N/2)] rows per expert and C receives
 * SwiGLU(gate, up) [R][N/2] directly. */
int ifd_moe_gather_qmm(const void* A, const int* perm, int div, const int* offsets, const int* tiles,
                       const int* ntiles, int max_tiles, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int E,
                       int N, int K, int silu, void* C, int R, void* stream);
/* The same for 4- or 8-bit expert stacks (bits; 8: wq uint32 [E][N][K/4]), the reference's gqmm at W.bits = 8
 * (mlx_gqmm_b8, qwen35.h:1835; MLX gather_qmm, quantized_nax.h:1467-1681): bf16(s q + b) dequant, fp32 sums. */
int ifd_moe_gather_qmm_ex(const void* A, const int* perm, int div, const int* offsets, const int* tiles,
                          const int* ntiles, int max_tiles, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                          int E, int N, int K, int bits, int silu, void* C, int R, void* stream);

/* The gathered expert GEMM on int8 activations (reference qa8g_gemm, qa8.metal:212-397; host qa8g,
 * qwen35.h:1847-1868): U int8 [rows][K] and XS [rows][K/64][2] from ifd_a8_quant with per-group scales (per_token 0
 * or 2), sorted row q reads row perm[q] / div (perm NULL: row q); per group y += s sx P + b (sx sum xq),
 * P = sum q xq exact. Same schedule, weights, silu and output as ifd_moe_gather_qmm; K / 64 * 256 bytes <= 64 KB. */
int ifd_moe_gather_qmm_a8(const int8_t* U, const float* XS, const int* perm, int div, const int* offsets,
                          const int* tiles, const int* ntiles, int max_tiles, const uint32_t* wq, const uint16_t* s,
                          const uint16_t* b, int E, int N, int K, int silu, void* C, int R, void* stream);

/* out[t][h] = bf16(acc) (assign) or bf16(out + bf16(acc)), acc = sum_j wt[t][j] yd[inv[t*k+j]][h] + sg[t] ys[t][h]
 * (ys may be NULL) (reference moe_combine_sorted, moe.metal:172-187). */
int ifd_moe_combine(void* out, const void* yd, const float* wt, const void* ys, const float* sg, const int* inv,
                    int T, int H, int k, int assign, void* stream);

/* One-shot MoE FFN on normalised tokens xn [T][H] (reference encode_moe after rmsnorm_for, qwen35.h:1909-1980):
 * router (bf16 [E + (shared_gate ? 1 : 0)][H]) -> route -> dispatch -> gathered gate/up + SwiGLU -> gathered down
 * -> combine with the shared expert (dense 4-bit gate_up [2 Is][H], down [H][Is]; sh_* may be NULL for none).
 * logits_bf16 selects the router's output rounding. Routing outputs are written to the caller's idx/wt/sg if
 * non-NULL. Workspace: ifd_moe_ffn_workspace. */
size_t ifd_moe_ffn_workspace(int T, int H, int I, int E, int k, int Is);
int ifd_moe_ffn(const void* xn, int T, int H, const void* router, int E, int k, int norm, int shared_gate,
                int logits_bf16, const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b,
                const uint32_t* edn_wq, const uint16_t* edn_s, const uint16_t* edn_b, int I,
                const uint32_t* sgu_wq, const uint16_t* sgu_s, const uint16_t* sgu_b, const uint32_t* sdn_wq,
                const uint16_t* sdn_s, const uint16_t* sdn_b, int Is, void* out, int assign, int* idx, float* wt,
                float* sg, void* workspace, size_t ws_bytes, void* stream);

/* ---- the MoE FFN on T64 expert stacks (ifd_pack_t64 with E experts) ------------------------------------------
 * ifd_moe_dispatch with a tile height (32 or 64 rows) and an optional segment for the shared expert as expert index
 * E: shared_rows > 0 appends sorted rows [R, R + shared_rows) = tokens 0, 1, ... (perm = t * k), their tiles after
 * the routed ones, and offsets[E + 1] = R + shared_rows. Sizes: offsets E + 2 entries, perm R + shared_rows, tiles
 * ifd_moe_tiles_max(R + shared_rows, E + 1) pairs; workspace ifd_moe_dispatch_workspace(R, E). */
int ifd_moe_dispatch_ex(const int* idx, int R, int E, int k, int tile_rows, int shared_rows, int* offsets, int* perm,
                        int* inv, int* tiles, int* ntiles, void* workspace, size_t ws_bytes, void* stream);
/* The tile height ifd_moe_ffn_t64 dispatches R routed rows over E experts with (64 once an expert holds about 24 rows
 * on average, else 32): the schedule a caller composing ifd_moe_dispatch_ex and ifd_moe_gather_qmm_t64 itself uses
 * to get the one-shot call's tiles. */
int ifd_moe_t64_tile_rows(int R, int E);
/* The gathered expert GEMM of ifd_moe_gather_qmm on T64 stacks (bf16(s q + b) dequant, fp32 sums): wt = E experts
 * [E][N][K] packed by ifd_pack_t64, wt_shared (may be NULL) the shared expert [N][K] taking the dispatch's expert-E
 * segment; tiles / ntiles / offsets / tile_rows from ifd_moe_dispatch_ex; rows = the sorted rows of C (ldc its row
 * stride). silu: the stack holds [gate (N/2) | up (N/2)] and C receives the SwiGLU [rows][N/2]. Output columns in
 * whole 256-column tiles (N % 256 == 0, with silu N / 2 % 256 == 0), K % 128 == 0.
 * workspace NULL: each GPU block takes whole (row tile, 256-column tile) items, and the sums are those of
 * ifd_moe_gather_qmm bit for bit. With a workspace (ifd_moe_gather_qmm_t64_workspace(tile_rows) bytes, counter header
 * zeroed once): the balanced schedule, every block an equal share of the items' 64-group pairs, which takes no
 * longer whatever the item count; an item split between blocks sums the fp32 sums of its K ranges in K order
 * (deterministic, within fp32 rounding of the unsplit sum). No counterpart in the reference, whose gather_qmm has no
 * work split of its own. */
size_t ifd_moe_gather_qmm_t64_workspace(int tile_rows);
int ifd_moe_gather_qmm_t64(const void* A, int lda, const int* perm, int div, const int* offsets, const int* tiles,
                           const int* ntiles, int tile_rows, const void* wt, const void* wt_shared, int E, int N, int K,
                           int silu, void* C, int ldc, int rows, void* workspace, size_t ws_bytes, void* stream);
/* One-shot MoE FFN on T64 stacks (reference encode_moe after rmsnorm_for, qwen35.h:1909-1980): router -> route ->
 * dispatch with the shared expert (sgu_t64 [2 I][H], sdn_t64 [H][I], the routed experts' I, or NULL) as expert E ->
 * gathered gate/up + SwiGLU -> gathered down (both on the balanced schedule of ifd_moe_gather_qmm_t64) -> combine;
 * the arithmetic of ifd_moe_ffn. H and I multiples of 256. Workspace: ifd_moe_ffn_t64_workspace (shared: 1 with a
 * shared expert). */
size_t ifd_moe_ffn_t64_workspace(int T, int H, int I, int E, int k, int shared);
int ifd_moe_ffn_t64(const void* xn, int T, int H, const void* router, int E, int k, int norm, int shared_gate,
                    int logits_bf16, const void* egu_t64, const void* edn_t64, int I, const void* sgu_t64,
                    const void* sdn_t64, void* out, int assign, int* idx, float* wt, float* sg, void* workspace,
                    size_t ws_bytes, void* stream);

/* The dense decode MLP block on T64 weights (reference encode_layer's MLP, qwen35.h:2867-2892):
 * x += down(SwiGLU(gate_up(rmsnorm(x, norm_w, eps)))) for M rows of x [M][ldx] (bf16, updated in place), through
 * the same kernels as ifd_rmsnorm -> ifd_gemm_t64_swiglu -> ifd_gemm_t64 (mode 1) and bit-identical to that
 * sequence; the normalised rows and the SwiGLU output stay in the workspace. gu_t64: [2 I][H] (gate rows, then up
 * rows), dn_t64: [H][I], packed by ifd_pack_t64. H and I multiples of 256. Workspace: ifd_mlp_decode_workspace. */
size_t ifd_mlp_decode_workspace(int M, int H, int I);
int ifd_mlp_decode(void* x, int ldx, const void* norm_w, float eps, const void* gu_t64, const void* dn_t64, int M,
                   int H, int I, void* workspace, size_t ws_bytes, void* stream);

/* Decode MoE for T <= 16 tokens (reference moe_plan / moe_gu2 / moe_dn2 and their router, moe.metal:267-551; host
 * qwen35.h:1876-1908; beyond 8 tokens, while T k < 128, the reference's per-row expert GEMVs moe_qmv4 +
 * moe_silu_mul + moe_combine, moe.metal:6-58, 103-187, host qwen35.h:1801-1807, 1947-1955, which compute the same
 * per-row arithmetic): router logits (fp32) -> routing -> the distinct experts of the step -> gate/up + SwiGLU ->
 * down + combine, three launches, each distinct expert's weights read once for all tokens that picked it. Every
 * expert product uses the decode GEMV arithmetic (qmv4), and a token's result does not depend on the others. The shared expert (sgu [2I][H], sdn [H][I], 4-bit, or NULL)
 * shares the routed experts' I. out = bf16(acc) (assign) or bf16(out + bf16(acc)), acc = sum_j wt[t][j] d_j +
 * sg[t] d_shared. idx / wt / sg / logits ([T][E + shared_gate] fp32, the values routed on) are written if non-NULL.
 * H % 512 == 0, I % 64 == 0, E <= 512, k <= 16. Workspace: ifd_moe_decode_workspace (its header counters zeroed
 * once, as for every workspace). */
size_t ifd_moe_decode_workspace(int T, int H, int I, int E, int k);
int ifd_moe_decode(const void* xn, int T, int H, const void* router, int E, int k, int norm, int shared_gate,
                   const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b, const uint32_t* edn_wq,
                   const uint16_t* edn_s, const uint16_t* edn_b, int I, const uint32_t* sgu_wq, const uint16_t* sgu_s,
                   const uint16_t* sgu_b, const uint32_t* sdn_wq, const uint16_t* sdn_s, const uint16_t* sdn_b,
                   void* out, int assign, int* idx, float* wt, float* sg, float* logits, void* workspace,
                   size_t ws_bytes, void* stream);
/* The decode MoE of ifd_moe_decode on T64 stacks (the layout ifd_pack_t64 writes, the device loader's default copy):
 * egu_t64 = E experts [E][2I][H], edn_t64 = [E][H][I], the shared expert's T64 copies sgu_t64 [2I][H] / sdn_t64
 * [H][I] (4-bit) or NULL. Up to 16 tokens, as ifd_moe_decode. The router is either `router` (bf16 [E1][H],
 * as ifd_moe_decode) or the caller's fp32 logits `logits_in` [T][E1] (as ifd_moe_decode_logits_ex): exactly one is
 * non-NULL. The same per-row qmv4 arithmetic (fp32 sums in another order); each wave streams one 32-column band's
 * 1152-byte tiles, and gate/up splits K over blocks. Workspace: ifd_moe_decode_t64_workspace. */
size_t ifd_moe_decode_t64_workspace(int T, int H, int I, int E, int k);
int ifd_moe_decode_t64(const void* xn, int T, int H, const void* router, const float* logits_in, int E, int k,
                       int norm, int shared_gate, const void* egu_t64, const void* edn_t64, int I, const void* sgu_t64,
                       const void* sdn_t64, void* out, int assign, int* idx, float* wt, float* sg, float* logits,
                       void* workspace, size_t ws_bytes, void* stream);
/* The same from router logits the caller computed: logits_in fp32 [T][E + shared_gate] (the shared expert's gate
 * logit last). For routers the decode kernel does not read, such as the reference's 8-bit router (moe_router8,
 * moe.metal:553-600, routed at qwen35.h:1878-1882): ifd_gemm_w8 in mode 2 computes those logits with its qmv8
 * arithmetic, per group s sum q x + b sum x. Same workspace as ifd_moe_decode. */
int ifd_moe_decode_logits(const float* logits_in, const void* xn, int T, int H, int E, int k, int norm,
                          int shared_gate, const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b,
                          const uint32_t* edn_wq, const uint16_t* edn_s, const uint16_t* edn_b, int I,
                          const uint32_t* sgu_wq, const uint16_t* sgu_s, const uint16_t* sgu_b,
                          const uint32_t* sdn_wq, const uint16_t* sdn_s, const uint16_t* sdn_b, void* out, int assign,
                          int* idx, float* wt, float* sg, void* workspace, size_t ws_bytes, void* stream);
/* ifd_moe_decode and ifd_moe_decode_logits with the shared expert's width: shared_bits 4, or 8 for an MLX 8-bit
 * shared expert (wq uint32 [2I][H/4] and [H][I/4]), which runs the qmv8 arithmetic (per group s sum q x + b sum x)
 * beside the 4-bit routed experts: the reference's moe_gu2_4_8 / moe_dn2_4_8 (moe.metal:465-476, 544-547). */
int ifd_moe_decode_ex(const void* xn, int T, int H, const void* router, int E, int k, int norm, int shared_gate,
                      const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b, const uint32_t* edn_wq,
                      const uint16_t* edn_s, const uint16_t* edn_b, int I, const uint32_t* sgu_wq,
                      const uint16_t* sgu_s, const uint16_t* sgu_b, const uint32_t* sdn_wq, const uint16_t* sdn_s,
                      const uint16_t* sdn_b, int shared_bits, void* out, int assign, int* idx, float* wt, float* sg,
                      float* logits, void* workspace, size_t ws_bytes, void* stream);
int ifd_moe_decode_logits_ex(const float* logits_in, const void* xn, int T, int H, int E, int k, int norm,
                             int shared_gate, const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b,
                             const uint32_t* edn_wq, const uint16_t* edn_s, const uint16_t* edn_b, int I,
                             const uint32_t* sgu_wq, const uint16_t* sgu_s, const uint16_t* sgu_b,
                             const uint32_t* sdn_wq, const uint16_t* sdn_s, const uint16_t* sdn_b, int shared_bits,
                             void* out, int assign, int* idx, float* wt, float* sg, void* workspace, size_t ws_bytes,
                             void* stream);

/* The reference's per-row expert products below moe_sort_min routed rows when the four-launch route does not apply
 * (moe_qmv4 on the gate/up and down stacks, moe_silu_mul, moe_combine: moe.metal:6-58, 103-111, 115-128; host
 * qwen35.h:1947-1955), on the caller's routing: idx / wt [T][k] and sg [T] from ifd_moe_route, and the shared expert's
 * output rows ys [T][H] (bf16; NULL: none) that the caller computed as the reference does, through gemm()
 * (qwen35.h:1909-1914). The decode MoE's kernels with the router and routing left out: each distinct expert's weights
 * read once per 16 tokens, the decode GEMV arithmetic (qmv4) for every routed product, SwiGLU of the bf16 gate and up,
 * then out = bf16(acc) (assign) or bf16(out + bf16(acc)), acc = sum_j wt[t][j] d_j + sg[t] ys[t] in fp32 (pick
 * order, shared last). Any T: 16 tokens per launch group, each token's result depends on its own row only. A row of
 * idx holds k distinct experts in [0, E), as ifd_moe_route writes it. Shapes as ifd_moe_decode. Workspace:
 * ifd_moe_rows_workspace. */
size_t ifd_moe_rows_workspace(int T, int H, int I, int E, int k);
int ifd_moe_rows(const void* xn, int T, int H, int E, int k, const int* idx, const float* wt, const float* sg,
                 const uint32_t* egu_wq, const uint16_t* egu_s, const uint16_t* egu_b, const uint32_t* edn_wq,
                 const uint16_t* edn_s, const uint16_t* edn_b, int I, const void* ys, void* out, int assign,
                 void* workspace, size_t ws_bytes, void* stream);
/* ifd_moe_rows on the routed experts' T64 stacks (ifd_pack_t64 with E; as ifd_moe_decode_t64): the same routing,
 * arithmetic and combine, 16 tokens per launch group. The shared expert (weight sg[t]) comes either as its output rows
 * ys, as in ifd_moe_rows, or as its 4-bit T64 copies sgu_t64 [2I][H] / sdn_t64 [H][I], which the same launches run
 * as one more slot in the qmv4 arithmetic (the arithmetic of the T64 gemm() up to 16 rows, sums in another order);
 * or neither. Workspace: ifd_moe_rows_t64_workspace. */
size_t ifd_moe_rows_t64_workspace(int T, int H, int I, int E, int k);
int ifd_moe_rows_t64(const void* xn, int T, int H, int E, int k, const int* idx, const float* wt, const float* sg,
                     const void* egu_t64, const void* edn_t64, int I, const void* sgu_t64, const void* sdn_t64,
                     const void* ys, void* out, int assign, void* workspace, size_t ws_bytes, void* stream);

/* ---- measurement probes (outside the operator path) ----------------------------------------------------------
 * The HBM and MFMA ceilings a benchmark reports beside the datasheet peaks, in the role of the reference's
 * micro-benchmarks (bw_read, micro/kernels.metal:8-16; fma_rate, micro/fma_rate.mm).
 * ifd_probe_stream_read reads `bytes` of src once (coalesced 1 KB wave loads, `blocks` blocks of 256 threads); sink
 * (4096 bytes) is written only in a case that cannot occur. ifd_probe_mfma runs `blocks` blocks of 4 waves, each wave
 * 8 independent chains of `iters` MFMAs on register operands: int8 = 0 v_mfma_f32_32x32x16_bf16 (32768 FLOP each),
 * 1 v_mfma_i32_32x32x32_i8 (65536 OP each); out float [blocks * 256]. */
int ifd_probe_stream_read(const void* src, size_t bytes, void* sink, int blocks, void* stream);
int ifd_probe_mfma(int int8, int iters, int blocks, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* INFERD_QMM_H */
