// Prefill GEMM on T64 weights, 256-row tiles: C (mode) = A . W^T with every weight dequantized to bf16(s q + b) (MLX
// qmm rounding, quantized.h:528-535) and fp32 accumulation (reference affine_qmm_t_nax,
// third_party/mlx/.../quantized_nax.h:938-1076, 1206-1267).
//
// Block: 8 waves (two per SIMD), tile 256 rows x 8 bands (256 columns); wave w owns band w over all 8 M tiles of 32
// rows (128 fp32 accumulators per lane). Each dequantized B fragment feeds 8 MFMAs: half the dequant VALU per MFMA of
// a 128-row tile; every wave reads the whole activation slab from LDS.
// K advances one 64-group per step through two LDS rings filled by direct global -> LDS DMA: kT8NS activation slabs
// [256][64 bf16] (16-byte columns XOR-swizzled by row pair: conflict-free fragment reads) and kT8NW weight stages
// (8 code halves, 8 (s, b) rows), one step further ahead. Per step wave w DMAs 4 KB of activations and its code tile;
// wave 0 the (s, b). Every DMA is issued by a whole wave under wave-uniform control flow (the LDS base goes to M0).
#include <algorithm>

#include "common.h"
#include "dma.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"
#include "t64_dev.h"

namespace ifd {

constexpr int kT8NS = 3;   // activation slabs in the LDS ring
constexpr int kT8NW = 4;   // weight stages in the LDS ring (one step further ahead)
constexpr int kT8Band = 4;  // M tiles per band of the tile order

struct GemmT8Args {
  const uint16_t* A;
  int lda;
  const uint8_t* wt;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;  // K-split partials, compact [S][ntail][256][256] (tail launch only)
  int gps, tiles_m, tiles_n;
  int tile0, ntail;
};

__host__ __device__ inline void t8_tile(int L, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int per_band = kT8Band * tiles_n;
  const int bandi = L / per_band, within = L % per_band;
  const int bm = tiles_m - bandi * kT8Band < kT8Band ? tiles_m - bandi * kT8Band : kT8Band;
  tm = bandi * kT8Band + within % bm;
  tn = within / bm;
}

__global__ __launch_bounds__(512, 1) void k_gemm_t8(GemmT8Args p) {
  constexpr int MT = 8, BM = 256, NBB = 8;
  constexpr int A_BYTES = BM * 128;                     // activation slab [256][64 bf16]
  constexpr int W_BYTES = NBB * kT64Codes + NBB * 128;  // code halves [8][1024] + (s, b) rows [8][128]
  constexpr int VPC = 4 + 1;                            // DMA instructions per wave per step (wave 0: one more)
  extern __shared__ __align__(16) uint8_t lds[];
  uint8_t* const aring = lds;                    // kT8NS slabs
  uint8_t* const wring = lds + kT8NS * A_BYTES;  // kT8NW weight stages
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, h = lane >> 5;

  const int Lrel = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  t8_tile(p.tile0 + Lrel, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int nbands = t64_bands(p.N);
  const int G = p.K / kGroup;
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps), Gz = g1 - g0;

  // activation DMA i (0..3) of this wave covers rows 8 (4 wave + i) .. + 7: lane -> row 8 (4 wave + i) + lane / 8,
  // physical 16-byte column lane % 8 holding logical column (lane % 8) ^ ((row / 2) % 8). Rows past M re-read row
  // M - 1 (their outputs are not stored).
  const uint16_t* asrc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 8 * (4 * wave + i) + lane / 8;
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    asrc[i] = p.A + (size_t)min(m0 + r, p.M - 1) * p.lda + 8 * c;
  }
  const size_t gstride = (size_t)nbands * kT64Tile;
  const uint8_t* tb = p.wt + (size_t)min(tn * NBB + wave, nbands - 1) * kT64Tile + 16 * lane;
  const uint8_t* sbsrc = p.wt + (size_t)min(tn * NBB + lane / 8, nbands - 1) * kT64Tile + kT64Codes + 16 * (lane & 7);

  // groups past the split re-read its last group into a stage nobody reads again: every step issues the same DMAs
  auto issue_w = [&](int step) {
    const size_t g = (size_t)min(g0 + step, g1 - 1);
    uint8_t* st = wring + (step % kT8NW) * W_BYTES;
    dma16(tb + g * gstride, st + wave * kT64Codes);
    if (wave == 0) dma16(sbsrc + g * gstride, st + NBB * kT64Codes);
  };
  auto issue_a = [&](int step) {
    const size_t g = (size_t)min(g0 + step, g1 - 1);
    uint8_t* st = aring + (step % kT8NS) * A_BYTES;
#pragma unroll
    for (int i = 0; i < 4; i++) dma16(asrc[i] + g * kGroup, st + (4 * wave + i) * 1024);
  };

  f32x16 acc[MT];
#pragma unroll
  for (int a = 0; a < MT; a++) acc[a] = zero16();

  // activation fragments of M tile a: MFMA step t takes k = 32 h + 8 t .. + 7 (logical column 4 h + t)
  auto load_a = [&](const uint8_t* st, int a, u32x4 (&af)[4]) {
    const int r = a * 32 + j;
#pragma unroll
    for (int t = 0; t < 4; t++) af[t] = *(const u32x4*)(st + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
  };

  // the wave's band of group `step`, dequantized from its weight stage (one fragment set feeds the 8 M tiles)
  auto dequant = [&](int step, u32x4 (&bf)[4]) {
    const uint8_t* wst = wring + (step % kT8NW) * W_BYTES;
    const u32x4 codes = *(const u32x4*)(wst + wave * kT64Codes + 16 * lane);
    const uint32_t sb = *(const uint32_t*)(wst + NBB * kT64Codes + wave * 128 + 4 * j);
    const float sc = bf2f((uint16_t)(sb & 0xFFFFu)), bi = bf2f((uint16_t)(sb >> 16)), sa = t64_sa(sc), sbs = t64_sb(sc);
#pragma unroll
    for (int t = 0; t < 4; t++) bf[t] = t64_dequant(codes[t], sa, sbs, bi);
  };

  // Pipeline: the weights of group s + 1 and the activations of group s are in LDS at step s. Per wave and step the
  // DMAs are [activations of s + 2, weights of s + 3]: waiting for all but the last step's DMAs leaves exactly those
  // in flight. The weight stage overwritten at step s (kT8NW = 4) held group s - 1, read at step s - 1; the slab
  // overwritten (kT8NS = 3) held group s - 1 too. Step s: the wave dequantizes its band of group s, then runs the
  // 32 MFMAs with activation fragments read one M tile ahead.
  issue_w(0);
  issue_a(0);
  issue_w(1);
  issue_a(1);
  issue_w(2);
  for (int s = 0; s < Gz; s++) {
    if (wave == 0) wait_vm_barrier<VPC + 1>();
    else wait_vm_barrier<VPC>();
    issue_a(s + 2);
    issue_w(s + 3);
    u32x4 bf[4];
    dequant(s, bf);
    const uint8_t* ast = aring + (s % kT8NS) * A_BYTES;
    u32x4 af[2][4];
    load_a(ast, 0, af[0]);
#pragma unroll
    for (int a = 0; a < MT; a++) {
      if (a + 1 < MT) load_a(ast, a + 1, af[(a + 1) & 1]);
#pragma unroll
      for (int t = 0; t < 4; t++) acc[a] = mfma_bf16(af[a & 1][t], bf[t], acc[a]);
    }
  }
  wait_vm_barrier<0>();

  const bool split = gridDim.y > 1;
  const int col = (tn * NBB + wave) * 32 + j;
  if (col >= p.N) return;
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m0 + a * 32 + 8 * (r / 4) + 4 * h + (r % 4);
      if (row >= p.M) continue;
      if (split)
        p.part[(((size_t)blockIdx.y * p.ntail + Lrel) * BM + (row - m0)) * 256 + (col - tn * 256)] = acc[a][r];
      else
        store_mode(p.C, (size_t)row * p.ldc + col, acc[a][r], p.mode);
    }
}

// C (mode) = the split sum of the compact tail partials, 4 columns per thread, in split order.
__global__ __launch_bounds__(256) void k_t8_tail_reduce(const float* __restrict__ part, int St, int ntail, int tile0,
                                                         int tiles_m, int tiles_n, int M, int N, void* C, int ldc,
                                                         int mode) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, per_tile = (size_t)256 * 64;
  if (i >= (size_t)ntail * per_tile) return;
  const int t = (int)(i / per_tile), e = (int)(i % per_tile), r = e / 64, c = (e % 64) * 4;
  int tm, tn;
  t8_tile(tile0 + t, tiles_m, tiles_n, tm, tn);
  const int row = tm * 256 + r, col = tn * 256 + c;
  if (row >= M || col >= N) return;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int z = 0; z < St; z++) {
    const float4 q = *(const float4*)(part + (((size_t)z * ntail + t) * 256 + r) * 256 + c);
    v.x += q.x, v.y += q.y, v.z += q.z, v.w += q.w;
  }
  const float vv[4] = {v.x, v.y, v.z, v.w};
  for (int k = 0; k < 4 && col + k < N; k++) store_mode(C, (size_t)row * ldc + col + k, vv[k], mode);
}

// Plan: whole rounds of 256 tiles run with all of K; a tail of at most half a round runs K-split St ways in a
// second launch (compact partials + their reduction), so the last round is not mostly idle.
struct T8Plan {
  int tiles, full, St, gpt;
};
static T8Plan gemm_t8_plan(int M, int N, int K) {
  T8Plan pl{};
  const int G = K / kGroup;
  pl.tiles = ((M + 255) / 256) * ((t64_bands(N) + 7) / 8);
  pl.full = pl.tiles;
  const int tail = pl.tiles % 256;
  if (pl.tiles >= 256 && tail > 0 && tail <= 128) {
    const int St = std::min(std::min(256 / tail, 8), G / 4);
    if (St >= 2) {
      pl.gpt = (G + St - 1) / St;
      pl.St = (G + pl.gpt - 1) / pl.gpt;
      pl.full = pl.tiles - tail;
    }
  }
  return pl;
}

size_t gemm_t8_workspace(int M, int N, int K) {
  const T8Plan pl = gemm_t8_plan(M, N, K);
  return pl.St ? (size_t)pl.St * (pl.tiles - pl.full) * 256 * 256 * sizeof(float) : 0;
}

int launch_gemm_t8(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                   void* ws, size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  const T8Plan pl = gemm_t8_plan(M, N, K);
  const size_t need = gemm_t8_workspace(M, N, K);
  if (need > ws_bytes || (need && !ws))
    return fail(IFD_ERR_WORKSPACE, "gemm_t8 needs %zu bytes of workspace, got %zu", need, ws_bytes);
  constexpr size_t lds = (size_t)kT8NS * 256 * 128 + (size_t)kT8NW * (8 * kT64Codes + 8 * 128);
  static bool attr = false;
  if (!attr) {
    hipFuncSetAttribute((const void*)k_gemm_t8, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr = true;
  }
  const int tiles_m = (M + 255) / 256, tiles_n = (t64_bands(N) + 7) / 8;
  const int G = K / kGroup;
  GemmT8Args p{A, lda, (const uint8_t*)wt, N, K, C, ldc, M, mode, (float*)ws, G, tiles_m, tiles_n, 0, 0};
  hipLaunchKernelGGL(k_gemm_t8, dim3(pl.full, 1), dim3(512), lds, st, p);
  IFD_TRY(check_launch("gemm_t8"));
  if (!pl.St) return IFD_OK;
  const int ntail = pl.tiles - pl.full;
  GemmT8Args q{A, lda, (const uint8_t*)wt, N, K, C, ldc, M, mode, (float*)ws, pl.gpt, tiles_m, tiles_n, pl.full,
               ntail};
  hipLaunchKernelGGL(k_gemm_t8, dim3(ntail, pl.St), dim3(512), lds, st, q);
  IFD_TRY(check_launch("gemm_t8 tail"));
  const size_t n = (size_t)ntail * 256 * 64;
  hipLaunchKernelGGL(k_t8_tail_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const float*)ws, pl.St,
                     ntail, pl.full, tiles_m, tiles_n, M, N, C, ldc, mode);
  return check_launch("gemm_t8 tail reduce");
}

}  // namespace ifd
