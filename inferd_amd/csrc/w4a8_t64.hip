// W4A8 GEMM on T64 weights with per-token int8 activations, on int8 MFMA.
//
// Replaces the reference's w4a8_gemm (engine/kernels/w4a8.metal:43-98) and its identity (:8, epilogue :78-87):
//   y[m][n] = sx[m] * sum_g ( s_g[n] * P_g[m][n] + b_g[n] * X_g[m] ),  P_g = sum_{k in g} q xq,  X_g = sum_{k in g} xq
// with q the unflipped 4-bit code (T64 stores codes unflipped), xq the int8 activation and sx the row's scale.
//
// Block and pipeline as k_gemm_t (gemm_t64.hip): 8 waves in two K-quads (quad kq takes group kq of every two-group
// chunk; wave wq of a quad the bands wq NB .. + NB - 1 over all BM = 32 MT rows), a kWaNS-stage LDS ring filled by
// direct global -> LDS DMA, one barrier per chunk. A stage holds the int8 activation slab [BM][128] (16-byte columns
// XOR-swizzled by row pair: conflict-free fragment reads), the code halves of the chunk's 2 NBB tiles and their
// (s, b) dwords.
// Per group and (M tile, band): two v_mfma_i32_32x32x32_i8 give P exactly (the codes unpack to bytes with two masks
// and two byte permutes per word), and acc += s * float(P): two VALU per accumulator per group, the floor of any
// per-group-scaled integer product. The bias part sum_g b_g X_g[m] is a GEMM over the groups (K = G): it runs once
// per tile after the K loop, as bf16 MFMAs into the same accumulators, with X = 256 hi + lo split into two exact
// bf16 integer planes (prepared by k_w4a8_xprep) and b collected in LDS during the loop (exact products, fp32 sums).
#include <algorithm>

#include "common.h"
#include "dma.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"

namespace ifd {

constexpr int kWaNS = 3;        // LDS pipeline stages
constexpr int kWaMaxGz = 96;    // groups per K split at most (the per-tile bias matrix lives in LDS)
constexpr int kWaThreads = 512;
constexpr int kWaBand = 4;      // M tiles per band of the tile order

// X_g = sum xq of each (row, group), recovered exactly from XS = (sx, sx * sum xq) (|sum| <= 8128), split as
// 256 hi + lo and stored as two bf16 planes [2][M][Gx] (both parts exact in bf16); groups past G are zero.
__global__ __launch_bounds__(256) void k_w4a8_xprep(const float* __restrict__ XS, int M, int G, int Gx,
                                                    uint16_t* __restrict__ Xhl) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * Gx) return;
  const int m = (int)(i / Gx), g = (int)(i % Gx);
  float hi = 0.f, lo = 0.f;
  if (g < G) {
    const float x = rintf(XS[((size_t)m * G + g) * 2 + 1] / XS[((size_t)m * G + g) * 2]);
    hi = floorf(x * (1.f / 256.f));
    lo = x - 256.f * hi;
    hi *= 256.f;
  }
  Xhl[i] = f2bf(hi);
  Xhl[(size_t)M * Gx + i] = f2bf(lo);
}

// The per-group W4A8 form's operands: Ab = U as exact bf16 integers [M][K] (8 per thread) and sxT[g][m] = sx of
// (row m, group g) = XS[m][g][0], zero for m in [M, Mp).
__global__ __launch_bounds__(256) void k_w4a8g_prep(const int8_t* __restrict__ U, const float* __restrict__ XS, int M,
                                                    int K, uint16_t* __restrict__ Ab, float* __restrict__ sxT,
                                                    int Mp) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, n8 = (size_t)M * K / 8;
  if (i < n8) {
    const u32x2 q = *(const u32x2*)(U + 8 * i);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t w = q[e / 2] >> (16 * (e % 2));
      const float lo = (float)(int8_t)(w & 0xFFu), hi = (float)(int8_t)((w >> 8) & 0xFFu);
      o[e] = (uint32_t)f2bf(lo) | (uint32_t)f2bf(hi) << 16;  // integers |x| <= 128: exact in bf16
    }
    *(u32x4*)(Ab + 8 * i) = u32x4{o[0], o[1], o[2], o[3]};
  }
  const int G = K / kGroup;
  if (i < (size_t)G * Mp) {
    const int g = (int)(i / Mp), m = (int)(i % Mp);
    sxT[i] = m < M ? XS[((size_t)m * G + g) * 2] : 0.f;
  }
}

int w4a8g_mp(int M) { return (M + 127) / 128 * 128 + 256; }

int launch_w4a8g_prep(const int8_t* U, const float* XS, int M, int K, uint16_t* Ab, float* sxT, int Mp,
                      hipStream_t st) {
  const size_t n = std::max((size_t)M * K / 8, (size_t)(K / kGroup) * Mp);
  if (n == 0) return IFD_OK;
  hipLaunchKernelGGL(k_w4a8g_prep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, U, XS, M, K, Ab, sxT, Mp);
  return check_launch("w4a8g prep");
}

struct W4A8TArgs {
  const int8_t* U;    // [M][K] int8, row stride K
  const float* XS;    // [M][G][2]: sx = XS[m][0][0] (per token)
  const uint16_t* Xhl;  // [2][M][Gx] bf16
  int Gx;
  const uint8_t* wt;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;       // K-split partials: [S][M][N] (ntail == 0) or compact [S][ntail][BM][BN] (tail tiles)
  int gps, tiles_m, tiles_n;
  int tile0, ntail;  // this launch covers tiles tile0 .. tile0 + gridDim.x - 1 of the tile order
};

// Tile order: bands of kWaBand M tiles walked M-fastest (neighbouring blocks share weight tiles in L2).
__host__ __device__ inline void wa_tile(int L, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int per_band = kWaBand * tiles_n;
  const int bandi = L / per_band, within = L % per_band;
  const int bm = tiles_m - bandi * kWaBand < kWaBand ? tiles_m - bandi * kWaBand : kWaBand;
  tm = bandi * kWaBand + within % bm;
  tn = within / bm;
}

// eight codes of one T64 word -> eight unsigned bytes in k order (code e in nibble (0,4,1,5,2,6,3,7)[e]): the low
// nibbles of the bytes hold codes 0, 4, 1, 5 and the high nibbles 2, 6, 3, 7
__device__ __forceinline__ void t64_bytes(uint32_t w, uint32_t& d0, uint32_t& d1) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  d0 = __builtin_amdgcn_perm(hi, lo, 0x06040200u);  // codes 0 1 2 3
  d1 = __builtin_amdgcn_perm(hi, lo, 0x07050301u);  // codes 4 5 6 7
}

template <int MT, int NB>
__global__ __launch_bounds__(kWaThreads, 1) void k_w4a8_t(W4A8TArgs p) {
  static_assert(MT == 2 || MT == 4, "activation DMAs: MT / 2 per wave");
  static_assert(NB >= 1 && NB <= 2, "one (s, b) DMA covers a group's NBB <= 8 tiles");
  constexpr int BM = 32 * MT, NBB = 4 * NB;
  constexpr int A_BYTES = BM * 128;             // [BM][128 int8]
  constexpr int C_BYTES = 2 * NBB * kT64Codes;  // [2 groups][NBB bands][1024]
  constexpr int ST = A_BYTES + C_BYTES + 2 * 1024;
  constexpr int VPC = MT / 2 + NB;              // DMA instructions per wave per chunk (waves 0, 1: one more)
  constexpr int NE = MT * NB * 16;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = wave >> 2, wq = wave & 3;
  const int j = lane & 31, h = lane >> 5;

  const int Lrel = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  wa_tile(p.tile0 + Lrel, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int nbands = t64_bands(p.N);
  const int G = p.K / kGroup;
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps), Gz = g1 - g0;
  const int Gzp = (Gz + 15) / 16 * 16;
  const int nch = Gz / 2, lastg = g0 + 2 * (nch - 1);
  // b of the tile's columns and this split's groups: [NBB * 32 columns][Gzp] bf16, after the pipeline stages
  uint16_t* bb = (uint16_t*)(lds + kWaNS * ST);

  // activation DMA: instruction i of this wave covers rows 8 (wave MT / 2 + i) .. + 7; lane -> LDS slot lane of that
  // 1 KB: row r = 8 (wave MT / 2 + i) + lane / 8, physical 16-byte column lane % 8 holding logical column
  // (lane % 8) ^ ((r / 2) % 8). Rows past M re-read row M - 1 (their outputs are not stored).
  const int8_t* asrc[MT / 2];
#pragma unroll
  for (int i = 0; i < MT / 2; i++) {
    const int r = 8 * (wave * (MT / 2) + i) + lane / 8;
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    asrc[i] = p.U + (size_t)min(m0 + r, p.M - 1) * p.K + 16 * c;
  }
  const size_t gstride = (size_t)nbands * kT64Tile;
  const uint8_t* tb[NB];
#pragma unroll
  for (int b = 0; b < NB; b++)
    tb[b] = p.wt + (size_t)min(tn * NBB + wq * NB + b, nbands - 1) * kT64Tile + (size_t)kq * gstride + 16 * lane;
  const uint8_t* sbsrc = p.wt +
                         (size_t)min(tn * NBB + (lane % (8 * NBB)) / 8, nbands - 1) * kT64Tile + kT64Codes +
                         16 * (lane & 7) + (size_t)(wave & 1) * gstride;

  auto issue = [&](int chunk, int stage) {
    const size_t g = (size_t)min(g0 + 2 * chunk, lastg);
    uint8_t* st = lds + stage * ST;
#pragma unroll
    for (int i = 0; i < MT / 2; i++) dma16(asrc[i] + g * kGroup, st + (wave * (MT / 2) + i) * 1024);
#pragma unroll
    for (int b = 0; b < NB; b++)
      dma16(tb[b] + g * gstride, st + A_BYTES + (kq * NBB + wq * NB + b) * kT64Codes);
    if (wave < 2) dma16(sbsrc + g * gstride, st + A_BYTES + C_BYTES + wave * 1024);
  };

  // zero b for the padding groups [Gz, Gzp) (ordered before the loop's writes by its first barrier)
  for (int i = tid; i < NBB * 32 * (Gzp - Gz); i += kWaThreads)
    bb[(i / (Gzp - Gz)) * Gzp + Gz + i % (Gzp - Gz)] = 0;

  f32x16 acc[MT][NB];
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[a][b] = zero16();

  // One group per quad and chunk, as MT x NB steps (a, b), a-major. Software-pipelined: the two MFMAs of step t are
  // issued before the epilogue of step t - 1 (P double-buffered), so the matrix unit works under the cvt/fma VALU;
  // the activation fragments of M tile a + 1 are read while tile a computes.
  auto compute = [&](int c, int stage) {
    const uint8_t* st = lds + stage * ST;
    const int gl = 2 * c + kq;  // this quad's group, relative to g0
    u32x4 bf[NB][2];
    float sc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const int band = wq * NB + b;
      const u32x4 codes = *(const u32x4*)(st + A_BYTES + (kq * NBB + band) * kT64Codes + 16 * lane);
      const uint32_t sb = *(const uint32_t*)(st + A_BYTES + C_BYTES + kq * 1024 + band * 128 + 4 * j);
      sc[b] = bf2f((uint16_t)(sb & 0xFFFFu));
      if (h == 0) bb[(band * 32 + j) * Gzp + gl] = (uint16_t)(sb >> 16);
      // B fragments: step s takes words 2s, 2s + 1 (k = 32 h + 16 s + 0..15)
#pragma unroll
      for (int s = 0; s < 2; s++) {
        uint32_t d[4];
        t64_bytes(codes[2 * s], d[0], d[1]);
        t64_bytes(codes[2 * s + 1], d[2], d[3]);
        bf[b][s] = u32x4{d[0], d[1], d[2], d[3]};
      }
    }
    auto afrag = [&](int a, int s) {
      const int r = a * 32 + j;
      return *(const u32x4*)(st + r * 128 + 16 * ((4 * kq + 2 * h + s) ^ ((r >> 1) & 7)));
    };
    u32x4 af[2][2];  // M tiles a and a + 1 (tile a + 1 read when step (a, 0) issues, from a = 1 on)
    af[0][0] = afrag(0, 0);
    af[0][1] = afrag(0, 1);
    af[1][0] = afrag(1, 0);
    af[1][1] = afrag(1, 1);
    i32x16 P[2];
    P[0] = mfma_i8(af[0][0], bf[0][0], izero16());
    P[0] = mfma_i8(af[0][1], bf[0][1], P[0]);
#pragma unroll
    for (int t = 1; t <= MT * NB; t++) {
      if (t < MT * NB) {
        const int a = t / NB, b = t % NB;
        if (b == 0 && a >= 1 && a + 1 < MT) {
          af[(a + 1) & 1][0] = afrag(a + 1, 0);
          af[(a + 1) & 1][1] = afrag(a + 1, 1);
        }
        P[t & 1] = mfma_i8(af[a & 1][0], bf[b][0], izero16());
        P[t & 1] = mfma_i8(af[a & 1][1], bf[b][1], P[t & 1]);
      }
      const int ap = (t - 1) / NB, bp = (t - 1) % NB;
#pragma unroll
      for (int r2 = 0; r2 < 16; r2++)
        acc[ap][bp][r2] = __builtin_fmaf(sc[bp], (float)P[(t - 1) & 1][r2], acc[ap][bp][r2]);
    }
  };

#pragma unroll
  for (int s = 0; s < kWaNS - 1; s++) issue(s, s);
  for (int c = 0; c < nch; c++) {
    if (wave < 2) wait_vm_barrier<(VPC + 1) * (kWaNS - 2)>();
    else wait_vm_barrier<VPC * (kWaNS - 2)>();
    issue(c + kWaNS - 1, (c + kWaNS - 1) % kWaNS);
    compute(c, c % kWaNS);
  }
  // every DMA landed, every fragment read and b write done
  wait_vm_barrier<0>();

  // bias part over this split's groups: quad kq takes M tiles [kq MT / 2, (kq + 1) MT / 2) of every band
  const size_t plane = (size_t)p.M * p.Gx;
#pragma unroll
  for (int a = 0; a < MT; a++) {
    if (a / (MT / 2) != kq) continue;  // wave-uniform; acc stays statically indexed (registers, not scratch)
    const uint16_t* xr = p.Xhl + (size_t)min(m0 + a * 32 + j, p.M - 1) * p.Gx + g0 + 8 * h;
    auto ld8 = [](const uint16_t* q) {  // 8 bf16 from an 8-byte aligned address (g0 is a multiple of 4 groups)
      const u32x2 x0 = *(const u32x2*)q, x1 = *(const u32x2*)(q + 4);
      return u32x4{x0[0], x0[1], x1[0], x1[1]};
    };
    for (int kk = 0; kk < Gzp / 16; kk++) {
      const u32x4 xhi = ld8(xr + 16 * kk), xlo = ld8(xr + plane + 16 * kk);
#pragma unroll
      for (int b = 0; b < NB; b++) {
        const u32x4 bv = *(const u32x4*)(bb + ((wq * NB + b) * 32 + j) * Gzp + 16 * kk + 8 * h);
        acc[a][b] = mfma_bf16(xhi, bv, acc[a][b]);
        acc[a][b] = mfma_bf16(xlo, bv, acc[a][b]);
      }
    }
  }
  __syncthreads();  // bb and the stages are free: LDS is reused for the quad reduction

  // quad 1 hands its sums to quad 0
  float* red = (float*)lds + (size_t)wq * NE * 64 + lane;
  if (kq == 1) {
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) red[((a * NB + b) * 16 + r) * 64] = acc[a][b][r];
  }
  __syncthreads();
  if (kq == 1) return;

  const bool split = gridDim.y > 1;
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m0 + a * 32 + 8 * (r / 4) + 4 * h + (r % 4);
      if (row >= p.M) continue;
      const float sx = p.XS[(size_t)row * G * 2];
#pragma unroll
      for (int b = 0; b < NB; b++) {
        const int col = (tn * NBB + wq * NB + b) * 32 + j;
        if (col >= p.N) continue;
        const float v = sx * (acc[a][b][r] + red[((a * NB + b) * 16 + r) * 64]);
        if (!split)
          store_mode(p.C, (size_t)row * p.ldc + col, v, p.mode);
        else if (p.ntail)
          p.part[(((size_t)blockIdx.y * p.ntail + Lrel) * BM + (row - m0)) * (NBB * 32) + (col - tn * NBB * 32)] = v;
        else
          p.part[((size_t)blockIdx.y * p.M + row) * p.N + col] = v;
      }
    }
}

// Tile/split plan: MT by M, NB = 2 (128 x 256 or 64 x 256 tiles). K is split only when a split would exceed
// kWaMaxGz groups (the per-tile bias matrix lives in LDS); splits are whole multiples of 4 groups. When whole rounds
// of 256 tiles leave a tail of at most half a round, the tail tiles run in a second launch with K split St ways
// (St tail blocks per CU instead of one long block), their fp32 partials in a compact [St][tail][BM][BN] buffer.
struct WaPlan {
  int MT, S, gps;       // main launch
  int tiles, full;      // tiles in all; tiles of the main launch (the rest is the tail)
  int St, gpt;          // tail split and its groups per split (St == 0: no tail launch)
};
static int round4(int g) { return (g + 3) / 4 * 4; }
static WaPlan w4a8_t_plan(int M, int N, int K) {
  WaPlan pl{};
  pl.MT = M <= 64 ? 2 : 4;
  const int G = K / kGroup;
  pl.tiles = ((M + 32 * pl.MT - 1) / (32 * pl.MT)) * ((t64_bands(N) + 7) / 8);
  pl.S = (G + kWaMaxGz - 1) / kWaMaxGz;
  pl.gps = round4((G + pl.S - 1) / pl.S);
  pl.S = (G + pl.gps - 1) / pl.gps;
  pl.full = pl.tiles;
  const int tail = pl.tiles % 256;
  if (pl.S == 1 && pl.tiles >= 256 && tail > 0 && tail <= 128) {
    int St = std::min(std::min(256 / tail, 8), G / 8);
    if (St >= 2) {
      pl.gpt = round4((G + St - 1) / St);
      pl.St = (G + pl.gpt - 1) / pl.gpt;
      pl.full = pl.tiles - tail;
    }
  }
  return pl;
}

static size_t xprep_bytes(int M, int K) {
  const int Gx = (K / kGroup + 15) / 16 * 16 + 16;
  return align_up((size_t)2 * M * Gx * sizeof(uint16_t), 256);
}

static size_t wa_part_bytes(const WaPlan& pl, int M, int N) {
  if (pl.S > 1) return (size_t)pl.S * M * N * sizeof(float);
  if (pl.St) return (size_t)pl.St * (pl.tiles - pl.full) * (32 * pl.MT) * 256 * sizeof(float);
  return 0;
}

// C (mode) = the split sum of the compact tail partials, 4 columns per thread, in split order.
__global__ __launch_bounds__(256) void k_wa_tail_reduce(const float* __restrict__ part, int St, int ntail, int tile0,
                                                         int tiles_m, int tiles_n, int BM, int M, int N, void* C,
                                                         int ldc, int mode) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, per_tile = (size_t)BM * 64;
  if (i >= (size_t)ntail * per_tile) return;
  const int t = (int)(i / per_tile), e = (int)(i % per_tile), r = e / 64, c = (e % 64) * 4;
  int tm, tn;
  wa_tile(tile0 + t, tiles_m, tiles_n, tm, tn);
  const int row = tm * BM + r, col = tn * 256 + c;
  if (row >= M || col >= N) return;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int z = 0; z < St; z++) {
    const float4 q = *(const float4*)(part + (((size_t)z * ntail + t) * BM + r) * 256 + c);
    v.x += q.x, v.y += q.y, v.z += q.z, v.w += q.w;
  }
  const float vv[4] = {v.x, v.y, v.z, v.w};
  for (int k = 0; k < 4 && col + k < N; k++) store_mode(C, (size_t)row * ldc + col + k, vv[k], mode);
}

// ---- W4A8 stream-K for M > 64: 128-row tiles, every CU an equal share of the (tile, group pair) units -----------
//
// Work is the set of units (tile, pair of 64-groups), tile = 128 rows x 8 bands (256 columns). With T tiles over
// nblk blocks (one per CU), the first q nblk = (T / nblk) nblk tiles are whole-tile work: block b takes tiles
// b q .. b q + q - 1. The other nsk = T % nblk tiles are split stream-K: block b takes their units
// [b U / nblk, (b + 1) U / nblk), U = nsk G2, first. A run is that share (at most two segments, each a piece of its
// tile unless it covers the whole tile) followed by the block's whole tiles, streamed as one sequence of steps.
// Pieces go to the block's two partial slots (unscaled fp32 sums in MFMA fragment order); k_sk_fixup sums each cut
// tile's pieces in unit order, applies the row scale sx and stores the tile.
//
// Block: 8 waves, two per SIMD; wave w owns band w over the 4 M tiles. A step is one group pair; per M tile a: for
// each group, two v_mfma_i32_32x32x32_i8 give its exact P and acc += s float(P) (two VALU per accumulator, the floor
// of a per-group-scaled integer product); the bias terms b X_g of both groups enter acc through one bf16 MFMA whose
// only non-zero k entries are X_g = hi + lo (two exact bf16 parts) of the two groups against their (b, b). So a
// pair's whole contribution is added at its step and a segment can end at any pair.
// One LDS ring of kWsR stages filled by direct global -> LDS DMA; a stage holds a pair's int8 activation slab
// [128][2 x 64] (16-byte columns XOR-swizzled by row pair), the 8 bands' code halves and (s, b) rows of both groups
// and the 128 rows' X pairs of both groups in 16-byte slots (from k_w4a8_xprep_t). Every wave issues its 16 slab rows
// and its band's two code halves; waves 0 and 1 also the (s, b) rows of one group each, waves 2 and 3 the X pairs of
// 64 rows each. They are buffer loads with a scalar pair offset; each role's code is compiled on its own, so every
// wait is a constant. The stream keeps issuing past the run's last unit (re-reading it) so that the count holds to
// the last step. One barrier per pair of groups.
constexpr int kWsR = 4;
constexpr int kWsA = 128 * 128;
constexpr int kWsC = 2 * 8 * kT64Codes;
constexpr int kWsSB = 2 * 1024;
constexpr int kWsX = 2048;
constexpr int kWsStage = kWsA + kWsC + kWsSB + kWsX;
constexpr int kWsRow = 256 + 4;  // staged tile row stride (floats)
constexpr size_t kWsLds = (size_t)kWsR * kWsStage > (size_t)128 * kWsRow * 4 ? (size_t)kWsR * kWsStage
                                                                               : (size_t)128 * kWsRow * 4;
static_assert(kWsLds <= 160 * 1024, "LDS plan");

struct W4A8SkArgs {
  const int8_t* U;     // [M][K]
  const float* XS;     // [M][G][2]
  const u32x4* Xt;     // [G / 2][Mx]: (X pair of group 2 p, X pair of group 2 p + 1, 0, 0), rows past M zero
  int Mx;
  const uint8_t* wt;
  uint32_t w_bytes, u_bytes, x_bytes;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;
  uint32_t part_bytes;
  int tiles_m, tiles_n, G2, nblk;  // G2: group pairs per tile (the units)
  int q, tile0, nsk;               // whole tiles per block; the stream-K tiles tile0 .. tile0 + nsk - 1
};

// X_g of (row, group) as an exact bf16 pair (bf16 hi | bf16 lo << 16): hi = 256 floor(X / 256), lo = X - hi.
// Xt[p][m] = (pair of group 2 p, pair of group 2 p + 1, 0, 0), zero for m >= M: a 16-byte slot that the kernel reads
// as a whole MFMA operand.
__global__ __launch_bounds__(256) void k_w4a8_xprep_t(const float* __restrict__ XS, int M, int G, int Mx,
                                                      u32x4* __restrict__ Xt) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)(G / 2) * Mx) return;
  const int pr = (int)(i / Mx), m = (int)(i % Mx);
  uint32_t v[2] = {0u, 0u};
  if (m < M) {
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int g = 2 * pr + e;
      const float x = rintf(XS[((size_t)m * G + g) * 2 + 1] / XS[((size_t)m * G + g) * 2]);
      const float hi = floorf(x * (1.f / 256.f)) * 256.f;
      v[e] = (uint32_t)f2bf(hi) | (uint32_t)f2bf(x - hi) << 16;
    }
  }
  Xt[i] = u32x4{v[0], v[1], 0u, 0u};
}

__device__ __forceinline__ void ws_dma(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, (int)voff, (int)soff, 0, 0);
}

// ROLE 0: waves 0-3 (also the (s, b) rows of group 2 p + wave for waves 0, 1; the X pairs of rows 64 (wave - 2) ..
// + 63 for waves 2, 3), ROLE 1: waves 4-7.
template <int ROLE>
__device__ __forceinline__ void ws_body(const W4A8SkArgs& p, uint8_t* lds, const int wave, const int b) {
  constexpr int R = kWsR, D = ROLE == 0 ? 5 : 4;
  static_assert(R >= 4 && (R - 2) * D <= 63, "ring depth, vmcnt range");
  float* const stg = (float*)lds;  // staged tile [128][kWsRow], after the K loop
  const int tid = threadIdx.x, lane = tid & 63;
  const int j = lane & 31, h = lane >> 5;
  const int G2 = p.G2, G = 2 * G2;
  const long Usk = (long)p.nsk * G2;
  const int ur0 = (int)((long)b * Usk / p.nblk), ur1 = (int)((long)(b + 1) * Usk / p.nblk);
  const int nr = ur1 - ur0, n = nr + p.q * G2;
  const int nbands = t64_bands(p.N);
  const uint32_t gstride = (uint32_t)nbands * kT64Tile;

  // unit i of the run -> (tile, pair)
  auto unit = [&](int i, int& tile, int& g) __attribute__((always_inline)) {
    if (i < nr) {
      tile = p.tile0 + (ur0 + i) / G2, g = (ur0 + i) % G2;
    } else {
      tile = b * p.q + (i - nr) / G2, g = (i - nr) % G2;
    }
  };

  const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc((void*)p.U, 0, (int)p.u_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)p.wt, 0, (int)p.w_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)p.Xt, 0, (int)p.x_bytes, 0x00020000);

  // ---- the DMA stream: per-lane offsets of the current tile, the pair in a scalar
  uint32_t va[2], vw, v3 = 0;
  auto set_tile = [&](int tile) __attribute__((always_inline)) {
    const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
#pragma unroll
    for (int d = 0; d < 2; d++) {
      const int r = 16 * wave + 8 * d + lane / 8;  // slab row of this lane's 16 bytes
      va[d] = (uint32_t)min(tm * 128 + r, p.M - 1) * (uint32_t)p.K + 16u * ((lane & 7) ^ ((r >> 1) & 7));
    }
    vw = (uint32_t)min(8 * tn + wave, nbands - 1) * kT64Tile + 16u * lane;
    if constexpr (ROLE == 0) {
      if (wave < 2) v3 = (uint32_t)min(8 * tn + lane / 8, nbands - 1) * kT64Tile + kT64Codes + 16u * (lane & 7);
      else v3 = (uint32_t)(tm * 128 + 64 * (wave - 2) + lane) * 16u;
    }
  };
  int s_i = 0, s_tile, s_g;
  unit(0, s_tile, s_g);
  set_tile(s_tile);
  auto issue = [&](int slot) __attribute__((always_inline)) {
    uint8_t* st = lds + slot * kWsStage;
#pragma unroll
    for (int d = 0; d < 2; d++) ws_dma(ru, st + (2 * wave + d) * 1024, va[d], (uint32_t)s_g * 128u);
#pragma unroll
    for (int g = 0; g < 2; g++)
      ws_dma(rw, st + kWsA + (8 * g + wave) * kT64Codes, vw, (uint32_t)(2 * s_g + g) * gstride);
    if constexpr (ROLE == 0) {
      if (wave < 2) ws_dma(rw, st + kWsA + kWsC + wave * 1024, v3, (uint32_t)(2 * s_g + wave) * gstride);
      else ws_dma(rx, st + kWsA + kWsC + kWsSB + (wave - 2) * 1024, v3, (uint32_t)s_g * (uint32_t)p.Mx * 16u);
    }
  };
  auto advance = [&]() __attribute__((always_inline)) {
    if (s_i >= n - 1) return;  // past the run's last unit the stream re-reads it
    s_i++;
    if (++s_g == G2 || s_i == nr) {
      unit(s_i, s_tile, s_g);
      set_tile(s_tile);
    }
  };

  f32x16 acc[4];
#pragma unroll
  for (int a = 0; a < 4; a++) acc[a] = zero16();

  // activation fragments of tile a, group g, MFMA step s2 (k = 32 h + 16 s2 + 0..15 of the group) and the X slot
  auto read_a = [&](const uint8_t* st, int a, u32x4 (&af)[2][2], u32x4& xv) __attribute__((always_inline)) {
    const int r = a * 32 + j;
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
      for (int s2 = 0; s2 < 2; s2++) af[g][s2] = *(const u32x4*)(st + r * 128 + 16 * ((4 * g + 2 * h + s2) ^ ((r >> 1) & 7)));
    xv = *(const u32x4*)(st + kWsA + kWsC + kWsSB + 16 * r);
  };
  struct Codes {
    u32x4 w[2];
    uint32_t sb[2];
  };
  auto read_codes = [&](const uint8_t* st, Codes& cd) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < 2; g++) {
      cd.w[g] = *(const u32x4*)(st + kWsA + (8 * g + wave) * kT64Codes + 16 * lane);
      cd.sb[g] = *(const uint32_t*)(st + kWsA + kWsC + g * 1024 + wave * 128 + 4 * j);
    }
  };

  // Step i: on entry A[0] / X[0] hold tile 0's operands of step i and cd its codes. Waits for stage i + 1 (R - 3
  // younger stages in flight), issues stage i + R - 1 into the stage read at step i - 1, then per M tile a: the four
  // i8 MFMAs of the pair's P, the bias MFMA, tile a + 1's operands (for a = 3: tile 0 of step i + 1) and the epilogue
  // of tile a - 1 (P double-buffered); last, step i + 1's codes.
  u32x4 A[2][2][2], X[2];
  Codes cd;
  auto step = [&](int i) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((R - 3) * D) : "memory");
    const int slot = i % R;
    issue(slot == 0 ? R - 1 : slot - 1);
    advance();
    const uint8_t* st = lds + slot * kWsStage;
    const uint8_t* stn = lds + (slot + 1 == R ? 0 : slot + 1) * kWsStage;
    u32x4 bq[2][2];
    float sc[2];
    uint32_t bb[2];
#pragma unroll
    for (int g = 0; g < 2; g++) {
#pragma unroll
      for (int s2 = 0; s2 < 2; s2++) {
        uint32_t d[4];
        t64_bytes(cd.w[g][2 * s2], d[0], d[1]);
        t64_bytes(cd.w[g][2 * s2 + 1], d[2], d[3]);
        bq[g][s2] = u32x4{d[0], d[1], d[2], d[3]};
      }
      sc[g] = bf2f((uint16_t)(cd.sb[g] & 0xFFFFu));
      bb[g] = h ? 0u : ((cd.sb[g] >> 16) | (cd.sb[g] & 0xFFFF0000u));
    }
    const u32x4 xb = {bb[0], bb[1], 0u, 0u};
    i32x16 P[2][2];
#pragma unroll
    for (int a = 0; a < 4; a++) {
      const int c = a & 1;
#pragma unroll
      for (int g = 0; g < 2; g++) {
        P[c][g] = mfma_i8(A[c][g][0], bq[g][0], izero16());
        P[c][g] = mfma_i8(A[c][g][1], bq[g][1], P[c][g]);
      }
      acc[a] = mfma_bf16(X[c], xb, acc[a]);
      read_a(a < 3 ? st : stn, (a + 1) & 3, A[c ^ 1], X[c ^ 1]);
      if (a > 0) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
          acc[a - 1][e] = __builtin_fmaf(sc[0], (float)P[c ^ 1][0][e], acc[a - 1][e]);
          acc[a - 1][e] = __builtin_fmaf(sc[1], (float)P[c ^ 1][1][e], acc[a - 1][e]);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 16; e++) {
      acc[3][e] = __builtin_fmaf(sc[0], (float)P[1][0][e], acc[3][e]);
      acc[3][e] = __builtin_fmaf(sc[1], (float)P[1][1][e], acc[3][e]);
    }
    read_codes(stn, cd);
  };

  // prologue: stages 0 .. R - 2 issued, stage 0's first operands read
#pragma unroll
  for (int k = 0; k < R - 1; k++) {
    issue(k);
    advance();
  }
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((R - 2) * D) : "memory");
  read_a(lds, 0, A[0], X[0]);
  read_codes(lds, cd);

  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.part, 0, (int)p.part_bytes, 0x00020000);
  auto write_slot = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
      for (int qq = 0; qq < 4; qq++) {
        const u32x4 x = {__float_as_uint(acc[a][4 * qq]), __float_as_uint(acc[a][4 * qq + 1]),
                         __float_as_uint(acc[a][4 * qq + 2]), __float_as_uint(acc[a][4 * qq + 3])};
        const int off = (((slot * 8 + wave) * 16 + a * 4 + qq) * 64 + lane) * 16;
        __builtin_amdgcn_raw_buffer_store_b128(x, rs, off, 0, 0);
      }
  };
  // a whole tile in the middle of the run: its rows scaled and stored from the fragments
  auto store_direct = [&](int tile) __attribute__((always_inline)) {
    const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
    const int col = (8 * tn + wave) * 32 + j;
    if (col >= p.N) return;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int row = tm * 128 + a * 32 + 8 * (e / 4) + 4 * h + (e % 4);
        if (row < p.M) store_mode(p.C, (size_t)row * p.ldc + col, p.XS[(size_t)row * G * 2] * acc[a][e], p.mode);
      }
  };

  // segments: the stream-K share (pieces, unless a segment covers its whole tile), then the whole tiles
  int i = 0, piece = 0, tile = 0;
  bool whole = false;
  for (;;) {
    int g;
    unit(i, tile, g);
    const int len = i < nr ? min(G2 - g, nr - i) : G2;
    for (int k = i; k < i + len; k++) step(k);
    i += len;
    whole = len == G2;
    if (i >= n) break;
    if (whole) {
      store_direct(tile);
    } else {
      write_slot(2 * b + piece);
      piece++;
    }
#pragma unroll
    for (int a = 0; a < 4; a++) acc[a] = zero16();
  }
  // every DMA (the stream ran on past the end) and piece store has landed; LDS is free once all waves are here
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (!whole) {
    write_slot(2 * b + piece);
    return;
  }
  // the last whole tile, staged through LDS and stored as rows
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int e = 0; e < 16; e++) stg[(a * 32 + 8 * (e / 4) + 4 * h + (e % 4)) * kWsRow + 32 * wave + j] = acc[a][e];
  __syncthreads();
  const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
  for (int e = tid; e < 128 * 64; e += 512) {
    const int row = e >> 6, c4 = (e & 63) * 4, grow = tm * 128 + row, gcol = tn * 256 + c4;
    if (grow >= p.M || gcol >= p.N) continue;
    const float sx = p.XS[(size_t)grow * G * 2];
    const float4 v4 = *(const float4*)(stg + row * kWsRow + c4);
    const float sv[4] = {sx * v4.x, sx * v4.y, sx * v4.z, sx * v4.w};
    const size_t o = (size_t)grow * p.ldc + gcol;
    if (gcol + 4 <= p.N && (o & 3) == 0 && p.mode != 1) {
      if (p.mode == 2) *(float4*)((float*)p.C + o) = make_float4(sv[0], sv[1], sv[2], sv[3]);
      else *(u32x2*)((uint16_t*)p.C + o) = u32x2{pack_bf2(sv[0], sv[1]), pack_bf2(sv[2], sv[3])};
    } else {
      for (int k = 0; k < 4 && gcol + k < p.N; k++) store_mode(p.C, o + k, sv[k], p.mode);
    }
  }
}

__global__ __launch_bounds__(512, 1) void k_w4a8_sk(W4A8SkArgs p) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = xcd_remap(blockIdx.x, p.nblk);
  if (wave < 4) ws_body<0>(p, lds, wave, b);
  else ws_body<1>(p, lds, wave, b);
}

// Stream-K plan: q whole tiles per block, the last T % nblk tiles split over the blocks (units: group pairs)
struct WsPlan {
  int tiles_m, tiles_n, G2, nblk, q, tile0, nsk, Mx;
};
static WsPlan w4a8_sk_plan(int M, int N, int K) {
  WsPlan pl{};
  pl.tiles_m = (M + 127) / 128;
  pl.tiles_n = (t64_bands(N) + 7) / 8;
  pl.G2 = K / (2 * kGroup);
  pl.Mx = pl.tiles_m * 128;
  const int tiles = pl.tiles_m * pl.tiles_n, cus = cu_count();
  pl.q = tiles / cus;
  pl.nsk = tiles - pl.q * cus;
  pl.tile0 = pl.q * cus;
  // with no whole tiles, never more blocks than units
  pl.nblk = pl.q ? cus : std::min(cus, pl.nsk * pl.G2);
  return pl;
}
static bool w4a8_sk_applies(int M) { return M > 64; }
static size_t ws_xt_bytes(const WsPlan& pl) { return align_up((size_t)pl.G2 * pl.Mx * 16, 256); }
static size_t ws_part_bytes(const WsPlan& pl) { return pl.nsk ? (size_t)2 * pl.nblk * 8 * 16 * 64 * 16 : 0; }

static int launch_w4a8_sk(const int8_t* U, const float* XS, const void* wt, int N, int K, void* C, int ldc, int M,
                          int mode, void* ws, hipStream_t st) {
  const WsPlan pl = w4a8_sk_plan(M, N, K);
  if (t64_bytes(N, K) >= ((size_t)1 << 31) || (size_t)M * K >= ((size_t)1 << 31) ||
      ws_xt_bytes(pl) >= ((size_t)1 << 31) || ws_part_bytes(pl) >= ((size_t)1 << 31) ||
      ((uint64_t)pl.nsk * pl.G2 + 1) * (pl.nblk + 1) >= ((uint64_t)1 << 32))
    return fail(IFD_ERR_UNSUPPORTED, "w4a8_t64: operands past 2 GiB");
  u32x4* Xt = (u32x4*)ws;
  float* part = (float*)((char*)ws + ws_xt_bytes(pl));
  const size_t nx = (size_t)pl.G2 * pl.Mx;
  hipLaunchKernelGGL(k_w4a8_xprep_t, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, st, XS, M, 2 * pl.G2, pl.Mx,
                     Xt);
  IFD_TRY(check_launch("w4a8_xprep_t"));
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)k_w4a8_sk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kWsLds);
    attr = true;
  }
  W4A8SkArgs a{U, XS, Xt, pl.Mx, (const uint8_t*)wt, (uint32_t)t64_bytes(N, K), (uint32_t)((size_t)M * K),
               (uint32_t)(nx * 16), N, K, C, ldc, M, mode, part, (uint32_t)ws_part_bytes(pl), pl.tiles_m, pl.tiles_n,
               pl.G2, pl.nblk, pl.q, pl.tile0, pl.nsk};
  hipLaunchKernelGGL(k_w4a8_sk, dim3(pl.nblk), dim3(512), kWsLds, st, a);
  IFD_TRY(check_launch("w4a8_sk"));
  if (!pl.nsk) return IFD_OK;
  // the fixup runs when some stream-K tile is cut between blocks
  const long U2 = (long)pl.nsk * pl.G2;
  bool cut = false;
  for (long t = 0; t < pl.nsk && !cut; t++)
    cut = (t * pl.G2 * pl.nblk + pl.nblk - 1) / U2 != ((t * pl.G2 + pl.G2 - 1) * pl.nblk + pl.nblk - 1) / U2;
  if (!cut) return IFD_OK;
  return launch_sk_fixup_rows(part, pl.tiles_m, pl.tiles_n, pl.tile0, pl.nsk, pl.G2, pl.nblk, C, ldc, M, N, mode, XS,
                              4 * pl.G2, st);
}

template <int MT>
static int launch_w4a8_t_cfg(const W4A8TArgs& p, int blocks, int S, hipStream_t st) {
  constexpr int NB = 2;
  const size_t pipe = (size_t)kWaNS * (32 * MT * 128 + 2 * 4 * NB * kT64Codes + 2 * 1024);
  const size_t bbb = (size_t)4 * NB * 32 * ((p.gps + 15) / 16 * 16) * sizeof(uint16_t);
  const size_t red = (size_t)4 * MT * NB * 16 * 64 * sizeof(float);
  const size_t lds = std::max(pipe + bbb, red);
  if (lds > 160 * 1024) return fail(IFD_ERR_UNSUPPORTED, "w4a8_t64: %zu bytes of LDS needed", lds);
  static bool attr = false;
  if (!attr) {
    hipFuncSetAttribute((const void*)k_w4a8_t<MT, NB>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    attr = true;
  }
  hipLaunchKernelGGL((k_w4a8_t<MT, NB>), dim3(blocks, S), dim3(kWaThreads), lds, st, p);
  return check_launch("w4a8_t64");
}

size_t w4a8_t_workspace(int M, int N, int K) {
  if (w4a8_sk_applies(M)) {
    const WsPlan pl = w4a8_sk_plan(M, N, K);
    return ws_xt_bytes(pl) + ws_part_bytes(pl);
  }
  const WaPlan pl = w4a8_t_plan(M, N, K);
  return xprep_bytes(M, K) + wa_part_bytes(pl, M, N);
}

int launch_w4a8_t(const int8_t* U, const float* XS, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                  void* ws, size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (K % 128) return fail(IFD_ERR_ARG, "T64 W4A8 needs K %% 128 == 0 (K=%d)", K);
  const size_t need = w4a8_t_workspace(M, N, K);
  if (need > ws_bytes || !ws)
    return fail(IFD_ERR_WORKSPACE, "w4a8_t64 needs %zu bytes of workspace, got %zu", need, ws_bytes);
  if (w4a8_sk_applies(M)) return launch_w4a8_sk(U, XS, wt, N, K, C, ldc, M, mode, ws, st);
  const WaPlan pl = w4a8_t_plan(M, N, K);
  const int G = K / kGroup, Gx = (G + 15) / 16 * 16 + 16;
  uint16_t* Xhl = (uint16_t*)ws;
  float* part = (float*)((char*)ws + xprep_bytes(M, K));
  const size_t nx = (size_t)M * Gx;
  hipLaunchKernelGGL(k_w4a8_xprep, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, st, XS, M, G, Gx, Xhl);
  IFD_TRY(check_launch("w4a8_xprep"));
  const int tiles_m = (M + 32 * pl.MT - 1) / (32 * pl.MT), tiles_n = (t64_bands(N) + 7) / 8;
  auto launch = [&](const W4A8TArgs& p, int blocks, int S) {
    return pl.MT == 2 ? launch_w4a8_t_cfg<2>(p, blocks, S, st) : launch_w4a8_t_cfg<4>(p, blocks, S, st);
  };
  // main launch: tiles [0, full), K split pl.S ways (full [S][M][N] partials when S > 1)
  W4A8TArgs p{U, XS, Xhl, Gx, (const uint8_t*)wt, N, K, C, ldc, M, mode, part, pl.gps, tiles_m, tiles_n, 0, 0};
  IFD_TRY(launch(p, pl.full, pl.S));
  if (pl.S > 1) return launch_splitk_reduce(part, pl.S, M, N, C, ldc, mode, st);
  if (!pl.St) return IFD_OK;
  // tail launch: tiles [full, tiles), K split St ways into compact partials, then their reduction
  const int ntail = pl.tiles - pl.full, BM = 32 * pl.MT;
  W4A8TArgs q{U, XS, Xhl, Gx, (const uint8_t*)wt, N, K, C, ldc, M, mode, part, pl.gpt, tiles_m, tiles_n, pl.full,
              ntail};
  IFD_TRY(launch(q, ntail, pl.St));
  const size_t n = (size_t)ntail * BM * 64;
  hipLaunchKernelGGL(k_wa_tail_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, pl.St, ntail,
                     pl.full, tiles_m, tiles_n, BM, M, N, C, ldc, mode);
  return check_launch("w4a8_tail_reduce");
}

}  // namespace ifd
