// T64-layout kernels: the repack from the reference layout and the decode GEMV on T64 weights.
//
// The decode kernel computes what the reference's qmv4 computes (engine/kernels/core.metal:85-171): per 64-group
// s * sum q x + b * sum x in fp32, here with the products on bf16 MFMA (codes enter as exact bf16 (128 + q)) and the
// group epilogue s * P + (b - 128 s) * X in fp32.
#include "common.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"

namespace ifd {

// ---- repack ------------------------------------------------------------------------------------------------------
// One thread per (expert, group, band, lane): 16 bytes of codes (unflipped, T64 nibble order) and, for h == 0, the
// row's (s, b) dword.
__global__ __launch_bounds__(256) void k_pack_t64(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ s,
                                                  const uint16_t* __restrict__ b, int N, int K, int ldk, uint32_t xr,
                                                  int E, uint8_t* __restrict__ out) {
  const int G = K / kGroup, nb = t64_bands(N), ldw = ldk / 8, ldg = ldk / kGroup;
  const size_t total = (size_t)E * G * nb * 64;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i % 64), band = (int)(i / 64 % nb), g = (int)(i / 64 / nb % G), e = (int)(i / 64 / nb / G);
  const int j = lane & 31, h = lane >> 5, n = band * 32 + j;
  uint8_t* tile = out + (size_t)e * t64_bytes(N, K) + ((size_t)g * nb + band) * kT64Tile;
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  uint32_t sb = 0;
  if (n < N) {
    const size_t row = (size_t)e * N + n;
    const uint32_t* src = wq + row * ldw + (size_t)g * 8 + 4 * h;
#pragma unroll
    for (int t = 0; t < 4; t++) v[t] = t64_word(src[t] ^ xr);
    sb = (uint32_t)s[row * ldg + g] | ((uint32_t)b[row * ldg + g] << 16);
  }
  *(u32x4*)(tile + 16 * lane) = v;
  if (h == 0) *(uint32_t*)(tile + kT64Codes + 4 * j) = sb;
}

int launch_pack_t64(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr,
                    int E, void* out, hipStream_t st) {
  const size_t total = (size_t)E * (K / kGroup) * t64_bands(N) * 64;
  if (total == 0) return IFD_OK;
  hipLaunchKernelGGL(k_pack_t64, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, wq, s, b, N, K, ldk, xr, E,
                     (uint8_t*)out);
  return check_launch("pack_t64");
}

// ---- decode GEMV, M <= 16 --------------------------------------------------------------------------------------
// Block: 256 threads = 4 waves = 4 bands (128 output columns) x one K split. The activation rows of the split are
// staged once in LDS (natural order) with their 64-group sums; then each wave streams its band's tiles in
// ping-pong blocks of kTB groups (one 16-byte code load + one (s, b) dword per lane per group) and reads
// activations from LDS. Prefetch loads are unconditional (the last block is re-read past the end) so every path
// leaves the same number of loads outstanding and the waits stay one block behind.
struct QmvTArgs {
  const uint16_t* A;
  int lda;
  const uint8_t* wt;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;
  int gps;
};

constexpr int kTB = 4;  // groups per pipeline block

__device__ __forceinline__ u32x4 t64_bf16_off128(uint32_t w) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; i++) r[i] = ((w >> (4 * i)) & 0x000F000Fu) | 0x43004300u;  // (q_2i, q_2i+1) + 128
  return r;
}

template <int RACT>
__global__ __launch_bounds__(256, 2) void k_qmv_t(QmvTArgs p) {
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int G = p.K / kGroup, nb = t64_bands(p.N);
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps), Gz = g1 - g0;
  const int Kz = Gz * kGroup, ldA = Kz + 8, M = p.M;
  uint16_t* As = lds;
  float* Xs = (float*)((char*)lds + ((size_t)M * ldA * 2 + 15) / 16 * 16);  // [Gz][16]

  // ---- stage A[0:M][g0*64 : g1*64] and the 64-group sums
  const int cpr = Kz / 8, total = M * cpr;
  for (int c0 = 0; c0 < total; c0 += 256) {
    const int c = c0 + tid;
    const bool ok = c < total;
    const int m = ok ? c / cpr : 0, kc = ok ? c % cpr : 0;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (ok) v = *(const u32x4*)(p.A + (size_t)m * p.lda + (size_t)g0 * kGroup + 8 * kc);
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) sum += bf2f((uint16_t)(v[e] & 0xFFFFu)) + bf2f((uint16_t)(v[e] >> 16));
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    if (ok) {
      *(u32x4*)(As + (size_t)m * ldA + 8 * kc) = v;
      if ((kc & 7) == 0) Xs[(kc >> 3) * 16 + m] = sum;
    }
  }
  for (int i = tid; i < Gz * 16; i += 256)
    if ((i & 15) >= M) Xs[i] = 0.f;
  __syncthreads();

  const int band = blockIdx.x * 4 + wave;
  if (band >= nb) return;  // no barrier follows
  const bool aok = j < M;
  const uint16_t* arow = As + (size_t)(aok ? j : 0) * ldA + 32 * h;
  const uint8_t* tcol = p.wt + (size_t)band * kT64Tile;  // + g * nb * kT64Tile
  const size_t gstride = (size_t)nb * kT64Tile;

  f32x16 acc = zero16();
  struct Blk {
    u32x4 w[kTB];
    uint32_t sb[kTB];
  };
  auto load_blk = [&](Blk& B, int g) {
#pragma unroll
    for (int i = 0; i < kTB; i++) {
      const uint8_t* t = tcol + (size_t)(g + i) * gstride;
      B.w[i] = *(const u32x4*)(t + 16 * lane);
      B.sb[i] = *(const uint32_t*)(t + kT64Codes + 4 * j);
    }
  };
  auto compute_blk = [&](const Blk& B, int g) {
#pragma unroll
    for (int i = 0; i < kTB; i++) {
      const int gl = g + i - g0;
      u32x4 af[4];
      const uint16_t* ag = arow + (size_t)gl * 64;
#pragma unroll
      for (int t = 0; t < 4; t++) af[t] = aok ? *(const u32x4*)(ag + 8 * t) : u32x4{0u, 0u, 0u, 0u};
      const float4 x0 = *(const float4*)(Xs + gl * 16 + 4 * h);
      float4 x1 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (RACT > 4) x1 = *(const float4*)(Xs + gl * 16 + 8 + 4 * h);
      f32x16 P = zero16();
#pragma unroll
      for (int t = 0; t < 4; t++) P = mfma_bf16(af[t], t64_bf16_off128(B.w[i][t]), P);
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      const float sc = bf2f((uint16_t)(B.sb[i] & 0xFFFFu)), bi = bf2f((uint16_t)(B.sb[i] >> 16));
      const float bp = __builtin_fmaf(-128.f, sc, bi);
#pragma unroll
      for (int r = 0; r < RACT; r++) acc[r] = __builtin_fmaf(sc, P[r], __builtin_fmaf(bp, xs[r], acc[r]));
    }
  };
  const int glast = g1 - kTB;
  Blk b0, b1;
  load_blk(b0, g0);
  for (int g = g0;; g += 2 * kTB) {
    load_blk(b1, min(g + kTB, glast));
    compute_blk(b0, g);
    if (g + kTB >= g1) break;
    load_blk(b0, min(g + 2 * kTB, glast));
    compute_blk(b1, g + kTB);
    if (g + 2 * kTB >= g1) break;
  }
  const int col = band * 32 + j;
  if (col >= p.N) return;
  const bool split = gridDim.y > 1;
#pragma unroll
  for (int r = 0; r < RACT; r++) {
    const int row = 8 * (r / 4) + 4 * h + (r % 4);
    if (row >= M) continue;
    if (split) p.part[((size_t)blockIdx.y * M + row) * p.N + col] = acc[r];
    else store_mode(p.C, (size_t)row * p.ldc + col, acc[r], p.mode);
  }
}

// Split plan: ~2 blocks per CU, whole kTB-group blocks per split, <= ~40 KB of staged activations per block.
struct TPlan {
  int S, gps;
};
static TPlan qmv_t_plan(int M, int N, int K) {
  const int G = K / kGroup, bx = (t64_bands(N) + 3) / 4;
  long S = (512 + bx - 1) / bx;
  S = std::max<long>(S, ((long)M * K * 2 + 40959) / 40960);
  S = std::min<long>(S, std::max(1, G / (2 * kTB)));
  S = std::min<long>(S, std::max(1, 1024 / std::max(M, 1)));
  int gps = (int)((G + S - 1) / S);
  gps = (gps + kTB - 1) / kTB * kTB;
  return TPlan{(G + gps - 1) / gps, gps};
}

size_t qmv_t_workspace(int M, int N, int K, int mode) {
  if (M > 16) return 0;
  return epilogue_ws_bytes(qmv_t_plan(M, N, K).S, M, N, mode);
}

int launch_qmv_t(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode, void* ws,
                 size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (M > 16) return fail(IFD_ERR_UNSUPPORTED, "T64 decode kernel takes M <= 16");
  if (K % (kGroup * kTB)) return fail(IFD_ERR_ARG, "T64 decode needs K %% %d == 0 (K=%d)", kGroup * kTB, K);
  const TPlan pl = qmv_t_plan(M, N, K);
  const size_t need = epilogue_ws_bytes(pl.S, M, N, mode);
  if (need > ws_bytes || (need && !ws))
    return fail(IFD_ERR_WORKSPACE, "qmv_t64 needs %zu bytes of workspace, got %zu", need, ws_bytes);
  // the SwiGLU mode without a split stores the bf16 product into the workspace for silu_mul
  const bool via_ws = mode == kModeSwiglu && pl.S == 1;
  QmvTArgs p{A, lda, (const uint8_t*)wt, N, K, via_ws ? ws : C, via_ws ? N : ldc, M, via_ws ? 0 : mode, (float*)ws,
             pl.gps};
  const int Kz = pl.gps * kGroup;
  const size_t lds = ((size_t)M * (Kz + 8) * 2 + 15) / 16 * 16 + (size_t)pl.gps * 16 * sizeof(float);
  if (lds > 64 * 1024) return fail(IFD_ERR_UNSUPPORTED, "qmv_t64: %zu bytes of LDS needed", lds);
  dim3 grid((t64_bands(N) + 3) / 4, pl.S), block(256);
  if (M <= 8) hipLaunchKernelGGL(k_qmv_t<4>, grid, block, lds, st, p);
  else hipLaunchKernelGGL(k_qmv_t<8>, grid, block, lds, st, p);
  IFD_TRY(check_launch("qmv_t64"));
  return launch_epilogue(ws, pl.S, M, N, C, ldc, mode, st);
}

}  // namespace ifd
