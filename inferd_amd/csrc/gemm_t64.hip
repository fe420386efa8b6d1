// GEMM on T64 weights for any M (decode batches above 16 rows and prefill): C (mode) = A . W^T.
//
// Replaces the reference's MLX affine_qmm_t_nax (third_party/mlx/.../quantized_nax.h:938-1076, 1206-1267) and its
// split-K variant (engine/kernels/qmm_splitk.metal:14-107) for T64-packed weights.
//
// Block: 8 waves, two per SIMD; block tile BM = 32 MT rows x NBB = 4 NB bands (128 NB columns); grid x = tiles
// (XCD-contiguous runs, bands of kGtBand M tiles walked M-fastest), grid y = K splits.
// K advances in chunks of two 64-groups. The waves form two quads: quad kq (= wave / 4) takes group kq of every
// chunk, and wave wq (= wave % 4) of a quad the bands wq NB .. + NB - 1 over all BM rows. The two waves on a SIMD thus
// work on the same outputs at different K, and their instruction streams interleave (one's dequant VALU and LDS
// reads under the other's MFMAs). At the end quad 1 adds its sums into quad 0's through LDS.
// Chunks flow through an NS-stage LDS ring filled by direct global->LDS DMA (global_load_lds_dwordx4), NS - 1 chunks
// ahead, at no VGPR cost, with one s_barrier per chunk; NS is as deep as 160 KB of LDS allows for the tile height, so
// that the short tiles keep more weight bytes in flight. A stage holds the activation slab [BM][128 bf16]
// (16-byte columns XOR-swizzled by row: conflict-free fragment reads), the code halves of the chunk's 2 NBB T64
// tiles, and their (s, b) dwords [2 groups][1 KB]. Per chunk every wave DMAs MT activation row quads and its own NB
// code tiles; waves 0 and 1 also the (s, b) dwords of group 0 and 1.
// Every DMA is issued by a whole wave under wave-uniform control flow: the LDS destination goes to M0, one value per
// wave, and a DMA under a lane-dependent branch may be merged by the compiler with another one whose destination
// differs, leaving one M0 for both.
//  DEQ = false (affine): codes enter the MFMA as exact bf16 (128 + q); per group the fp32 epilogue adds
//    s P + (b - 128 s) X, with X (the activation group sums) from a second MFMA against ones: the decode GEMV
//    arithmetic (engine/kernels/core.metal:85-171).
//  DEQ = true: codes are dequantized in registers to bf16(s q + b) (MLX qmm rounding, quantized.h:528-535) and
//    accumulate over K; one dequant feeds MT MFMA tiles: the cheaper choice from 4 M tiles up.
//  A8 (with DEQ = false): the reference's W4A8 GEMM with per-(row, 64-group) int8 activations (w4a8.metal:24-98):
//    A holds the int8 codes xq as exact bf16 integers, so the MFMAs give P = sum (128 + q) xq and X = sum xq exactly
//    (every partial sum is an integer below 2^24), and per group acc += sx (s P + (b - 128 s) X) with sx the row's
//    scale for that group, = sx s sum q xq + sx b sum xq: the reference's S sx P + B (sx sum xq). The stage also
//    holds the chunk's sx for the tile's rows (from a transposed copy sxT [G][Mp]), DMAd by waves 2 and 3.
#include <algorithm>

#include "common.h"
#include "dma.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"
#include "t64_dev.h"

namespace ifd {

struct GemmTArgs {
  const uint16_t* A;
  int lda;
  const uint8_t* wt;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;
  int gps;
  int tiles_m, tiles_n;
  const float* sxT;  // A8: the activation scales transposed, [G][Mp] (rows past M zero)
  int Mp;
};

constexpr int kGtBand = 4;  // M tiles per band of the tile order
constexpr int kGtThreads = 512;

// bytes of one pipeline stage, and the stages that fit in 160 KB of LDS; A8 adds [2 groups][256 rows] sx
__host__ __device__ constexpr int gt_stage_bytes(int MT, int NB, bool A8 = false) {
  return MT * 32 * 256 + 2 * 4 * NB * kT64Codes + 2 * 1024 + (A8 ? 2 * 1024 : 0);
}
__host__ __device__ constexpr int gt_stages(int MT, int NB, bool A8 = false) {
  return 160 * 1024 / gt_stage_bytes(MT, NB, A8) < 6 ? 160 * 1024 / gt_stage_bytes(MT, NB, A8) : 6;
}

template <int MT, int NB, bool DEQ, bool A8 = false>
__global__ __launch_bounds__(kGtThreads, 1) void k_gemm_t(GemmTArgs p) {
  constexpr int NS = gt_stages(MT, NB, A8);
  static_assert(NB >= 1 && NB <= 2, "one (s, b) DMA covers a group's NBB <= 8 tiles");
  static_assert(!(A8 && DEQ), "the W4A8 form is the affine arithmetic");
  constexpr int BM = 32 * MT, NBB = 4 * NB;
  constexpr int A_BYTES = BM * 256;             // [BM][128 bf16]
  constexpr int C_BYTES = 2 * NBB * kT64Codes;  // [2 groups][NBB bands][1024]
  constexpr int SX_OFF = A_BYTES + C_BYTES + 2 * 1024;  // A8: [2 groups][256] sx
  constexpr int ST = SX_OFF + (A8 ? 2 * 1024 : 0);  // + [2 groups][1 KB] (s, b)
  static_assert(ST == gt_stage_bytes(MT, NB, A8) && NS >= 3, "stage layout");
  constexpr int VPC = MT + NB;                  // DMA instructions per wave per chunk (waves 0, 1: one more)
  constexpr int NE = MT * NB * 16;              // accumulators per lane
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  // wave-uniform (SGPR) so that every DMA destination, which goes to M0, is computed as a scalar
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = wave >> 2, wq = wave & 3;
  const int j = lane & 31, h = lane >> 5;

  const int ntiles = p.tiles_m * p.tiles_n;
  const int L = xcd_remap(blockIdx.x, ntiles);
  const int per_band = kGtBand * p.tiles_n;
  const int bandi = L / per_band, within = L % per_band;
  const int bm = min(kGtBand, p.tiles_m - bandi * kGtBand);
  const int tm = bandi * kGtBand + within % bm, tn = within / bm;
  const int m0 = tm * BM;
  const int nbands = t64_bands(p.N);
  const int G = p.K / kGroup;
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps);
  const int nch = (g1 - g0) / 2, lastg = g0 + 2 * (nch - 1);

  // activation DMA: instruction i of this wave covers rows 4 (wave MT + i) .. + 3; lane -> LDS slot lane of that
  // 1 KB: row r = 4 (wave MT + i) + lane / 16, physical 16-byte column lane % 16 holding logical column
  // (lane % 16) ^ (r % 16). Rows past M re-read row M - 1 (finite data; their outputs are not stored).
  const uint16_t* asrc[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int r = 4 * (wave * MT + i) + lane / 16;
    const int c = (lane & 15) ^ (r & 15);
    asrc[i] = p.A + (size_t)min(m0 + r, p.M - 1) * p.lda + 8 * c;
  }
  // code DMA: this wave's NB bands of group kq (bands past the end re-read the last band; not stored)
  const size_t gstride = (size_t)nbands * kT64Tile;
  const uint8_t* tb[NB];
#pragma unroll
  for (int b = 0; b < NB; b++)
    tb[b] = p.wt + (size_t)min(tn * NBB + wq * NB + b, nbands - 1) * kT64Tile + (size_t)kq * gstride + 16 * lane;
  // (s, b) DMA (waves 0 and 1, group = wave): lane -> band (lane mod 8 NBB) / 8, 16-byte part lane % 8; lanes from
  // 8 NBB on repeat the first ones
  const uint8_t* sbsrc = p.wt +
                         (size_t)min(tn * NBB + (lane % (8 * NBB)) / 8, nbands - 1) * kT64Tile + kT64Codes +
                         16 * (lane & 7) + (size_t)(wave & 1) * gstride;
  // A8: waves 2 and 3 DMA the sx of rows m0 .. m0 + 255 for group (wave - 2) of the chunk (sxT is padded past them)
  const float* sxsrc = A8 ? p.sxT + (size_t)(wave & 1) * p.Mp + m0 + 4 * lane : nullptr;

  auto issue = [&](int chunk, int stage) {
    const size_t g = (size_t)min(g0 + 2 * chunk, lastg);
    uint8_t* st = lds + stage * ST;
#pragma unroll
    for (int i = 0; i < MT; i++) dma16(asrc[i] + g * kGroup, st + (wave * MT + i) * 1024);
#pragma unroll
    for (int b = 0; b < NB; b++)
      dma16(tb[b] + g * gstride, st + A_BYTES + (kq * NBB + wq * NB + b) * kT64Codes);
    if (wave < 2) dma16(sbsrc + g * gstride, st + A_BYTES + C_BYTES + wave * 1024);
    if constexpr (A8) {
      if (wave >= 2 && wave < 4) dma16(sxsrc + g * (size_t)p.Mp, st + SX_OFF + (wave - 2) * 1024);
    }
  };

  f32x16 acc[MT][NB];
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[a][b] = zero16();
  u32x4 ones;
  ones[0] = ones[1] = ones[2] = ones[3] = 0x3F803F80u;

  // B fragments of band b (of this wave's NB) of group kq in a stage: codes -> bf16 (dequant or 128 + q), and
  // (s, b - 128 s)
  auto load_band = [&](const uint8_t* st, int b, u32x4 (&bf)[4], float& sc, float& bp) {
    const int band = wq * NB + b;
    const u32x4 codes = *(const u32x4*)(st + A_BYTES + (kq * NBB + band) * kT64Codes + 16 * lane);
    const uint32_t sb = *(const uint32_t*)(st + A_BYTES + C_BYTES + kq * 1024 + band * 128 + 4 * j);
    sc = bf2f((uint16_t)(sb & 0xFFFFu));
    const float bi = bf2f((uint16_t)(sb >> 16));
    if (DEQ) {
      const float sa = t64_sa(sc), sbs = t64_sb(sc);
#pragma unroll
      for (int t = 0; t < 4; t++) bf[t] = t64_dequant(codes[t], sa, sbs, bi);
    } else {
      bp = __builtin_fmaf(-128.f, sc, bi);
#pragma unroll
      for (int t = 0; t < 4; t++) bf[t] = t64_off128(codes[t]);
    }
  };
  // activation fragments of M tile a of group kq in a stage
  auto load_a = [&](const uint8_t* st, int a, u32x4 (&af)[4]) {
    const int r = a * 32 + j;
#pragma unroll
    for (int t = 0; t < 4; t++) af[t] = *(const u32x4*)(st + r * 256 + 16 * ((kq * 8 + 4 * h + t) ^ (r & 15)));
  };

  auto compute = [&](int stage) {
    const uint8_t* st = lds + stage * ST;
    if (DEQ) {
      // bands outermost: one band's fragments live at a time, and band b + 1's dequant (VALU) overlaps band b's
      // MFMAs; the activation fragments are re-read per band (LDS has the bandwidth) and double-buffered
      u32x4 bcur[4], bnext[4];
      float sc0, bp0, sc1, bp1;
      load_band(st, 0, bcur, sc0, bp0);
#pragma unroll
      for (int b = 0; b < NB; b++) {
        if (b + 1 < NB) load_band(st, b + 1, bnext, sc1, bp1);
        u32x4 af[2][4];
        load_a(st, 0, af[0]);
#pragma unroll
        for (int a = 0; a < MT; a++) {
          if (a + 1 < MT) load_a(st, a + 1, af[(a + 1) & 1]);
#pragma unroll
          for (int t = 0; t < 4; t++) acc[a][b] = mfma_bf16(af[a & 1][t], bcur[t], acc[a][b]);
        }
        if (b + 1 < NB) {
#pragma unroll
          for (int t = 0; t < 4; t++) bcur[t] = bnext[t];
        }
      }
      (void)sc0, (void)bp0, (void)sc1, (void)bp1;
    } else {
      float sc[NB], bp[NB];
      u32x4 bfr[NB][4];
#pragma unroll
      for (int b = 0; b < NB; b++) load_band(st, b, bfr[b], sc[b], bp[b]);
#pragma unroll
      for (int a = 0; a < MT; a++) {
        u32x4 af[4];
        load_a(st, a, af);
        f32x16 X = zero16();
#pragma unroll
        for (int t = 0; t < 4; t++) X = mfma_bf16(af[t], ones, X);
        // A8: the sx of this lane's 16 rows (a 32 + 8 q + 4 h + 0..3) for group kq
        float sxv[16];
        if constexpr (A8) {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const u32x4 v = *(const u32x4*)(st + SX_OFF + kq * 1024 + (a * 32 + 8 * q + 4 * h) * 4);
#pragma unroll
            for (int e = 0; e < 4; e++) sxv[4 * q + e] = __uint_as_float(v[e]);
          }
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
          f32x16 P = zero16();
#pragma unroll
          for (int t = 0; t < 4; t++) P = mfma_bf16(af[t], bfr[b][t], P);
#pragma unroll
          for (int r2 = 0; r2 < 16; r2++) {
            if constexpr (A8)
              acc[a][b][r2] = __builtin_fmaf(sxv[r2], __builtin_fmaf(sc[b], P[r2], bp[b] * X[r2]), acc[a][b][r2]);
            else
              acc[a][b][r2] = __builtin_fmaf(sc[b], P[r2], __builtin_fmaf(bp[b], X[r2], acc[a][b][r2]));
          }
        }
      }
    }
  };

  // Every iteration issues one chunk (past the end: a re-read of the last chunk into a stage nobody reads again), so
  // each wave's count of outstanding DMA instructions is the same on every iteration: waiting for all but its DMAs of
  // the NS - 2 youngest chunks leaves those in flight. The LDS reads of the previous chunk finish before the barrier
  // that lets any wave overwrite that stage.
#pragma unroll
  for (int s = 0; s < NS - 1; s++) issue(s, s);
  for (int c = 0; c < nch; c++) {
    if (wave < (A8 ? 4 : 2)) wait_vm_barrier<(VPC + 1) * (NS - 2)>();
    else wait_vm_barrier<VPC * (NS - 2)>();
    issue(c + NS - 1, (c + NS - 1) % NS);
    compute(c % NS);
  }
  // no DMA may still target LDS and every wave's fragment reads are done before LDS is reused for the sums
  wait_vm_barrier<0>();

  // quad 1 hands its sums to quad 0 (lane-contiguous dwords: conflict-free)
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
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[a][b][r] += red[((a * NB + b) * 16 + r) * 64];

  const bool split = gridDim.y > 1;
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const int col = (tn * NBB + wq * NB + b) * 32 + j;
      if (col >= p.N) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + a * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        if (row >= p.M) continue;
        if (split) p.part[((size_t)blockIdx.y * p.M + row) * p.N + col] = acc[a][b][r];
        else store_mode(p.C, (size_t)row * p.ldc + col, acc[a][b][r], p.mode);
      }
    }
}

// Tile/split plan: (MT, NB, DEQ) by M; the K split S (whole 2-group chunks) maximises the occupancy of the last
// round of blocks over 256 CUs, with fp32 partials of at most 64 MB.
struct GtPlan {
  int MT, NB, S, gps;
  bool deq;
};
// Mrows: the rows the tiles cover (M, or more when the tile height is chosen for fewer rows)
static GtPlan gemm_t_plan(int M, int N, int K, int Mrows = 0) {
  GtPlan pl{};
  pl.MT = M <= 32 ? 1 : M <= 64 ? 2 : 4;
  pl.NB = 2;
  pl.deq = pl.MT == 4;
  if (Mrows > M) M = Mrows;
  const int G = K / kGroup;
  const long tiles = (long)((M + 32 * pl.MT - 1) / (32 * pl.MT)) * ((t64_bands(N) + 4 * pl.NB - 1) / (4 * pl.NB));
  const long smax = std::max(1L, std::min<long>(G / 8, (64L << 20) / ((long)M * N * 4)));
  long best = 1;
  double best_eff = 0.0;
  for (long S = 1; S <= smax && tiles * (S - 1) < 4 * 256; S++) {
    const long blocks = tiles * S, rounds = (blocks + 255) / 256;
    const double eff = (double)blocks / (rounds * 256.0) - 0.02 * (S - 1);  // small cost per extra split
    if (eff > best_eff + 1e-9) best_eff = eff, best = S;
  }
  int gps = (int)((G + best - 1) / best);
  gps = (gps + 1) / 2 * 2;
  pl.S = (G + gps - 1) / gps;
  pl.gps = gps;
  return pl;
}

// Prefill shapes that fill at least one round of 256 CUs with 256-row tiles go to k_gemm_t8 (gemm_t8.hip): half the
// dequant VALU per MFMA.
static bool use_t8(int M, int N) { return (long)((M + 255) / 256) * ((t64_bands(N) + 7) / 8) >= 256; }

size_t gemm_t_workspace(int M, int N, int K, int mode) {
  if (!use_t8(M, N) && gemm_sk_applies(M, N, K, mode)) return gemm_sk_workspace(M, N, K, mode);
  if (use_t8(M, N))
    return align_up(gemm_t8_workspace(M, N, K), 256) + (mode == kModeSwiglu ? (size_t)M * N * sizeof(uint16_t) : 0);
  return epilogue_ws_bytes(gemm_t_plan(M, N, K).S, M, N, mode);
}

template <int MT, int NB, bool DEQ, bool A8 = false>
static int launch_gemm_t_cfg(const GemmTArgs& p, int S, hipStream_t st) {
  const size_t pipe = (size_t)gt_stages(MT, NB, A8) * gt_stage_bytes(MT, NB, A8);
  const size_t red = (size_t)4 * MT * NB * 16 * 64 * sizeof(float);  // quad 1's sums, after the K loop
  const size_t lds = std::max(pipe, red);
  static bool attr = false;
  if (!attr) {
    hipFuncSetAttribute((const void*)k_gemm_t<MT, NB, DEQ, A8>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)lds);
    attr = true;
  }
  hipLaunchKernelGGL((k_gemm_t<MT, NB, DEQ, A8>), dim3(p.tiles_m * p.tiles_n, S), dim3(kGtThreads), lds, st, p);
  return check_launch("gemm_t64");
}

// W4A8 with per-(row, 64-group) scales on T64 weights past the decode GEMV's rows: Ab = the int8 rows as bf16
// integers [M][K], sxT = their scales transposed [G][Mp] (Mp >= 128 tiles + 256, zero past M); the affine pipeline
// for every tile height. Workspace: the K-split partials (epilogue_ws_bytes of the plan).
// 64-row tiles at most: the affine form has no dequant to share across M tiles, and four tiles' accumulators with
// their row scales spill registers
static GtPlan gemm_t_a8_plan(int M, int N, int K) { return gemm_t_plan(std::min(M, 64), N, K, M); }
size_t gemm_t_a8_workspace(int M, int N, int K, int mode) {
  return epilogue_ws_bytes(gemm_t_a8_plan(M, N, K).S, M, N, mode);
}
int launch_gemm_t_a8(const uint16_t* Ab, const float* sxT, int Mp, const void* wt, int N, int K, void* C, int ldc,
                     int M, int mode, void* ws, size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (K % 128) return fail(IFD_ERR_ARG, "T64 W4A8 needs K %% 128 == 0 (K=%d)", K);
  if (mode == kModeSwiglu) return fail(IFD_ERR_UNSUPPORTED, "T64 W4A8: no SwiGLU mode");
  const GtPlan pl = gemm_t_a8_plan(M, N, K);
  const size_t need = epilogue_ws_bytes(pl.S, M, N, mode);
  if (need > ws_bytes || (need && !ws))
    return fail(IFD_ERR_WORKSPACE, "gemm_t64_w4a8 needs %zu bytes of workspace, got %zu", need, ws_bytes);
  GemmTArgs p{Ab, K, (const uint8_t*)wt, N, K, C, ldc, M, mode, (float*)ws, pl.gps,
              (M + 32 * pl.MT - 1) / (32 * pl.MT), (t64_bands(N) + 4 * pl.NB - 1) / (4 * pl.NB), sxT, Mp};
  const int rc = pl.MT == 1 ? launch_gemm_t_cfg<1, 2, false, true>(p, pl.S, st)
                            : launch_gemm_t_cfg<2, 2, false, true>(p, pl.S, st);
  IFD_TRY(rc);
  return launch_epilogue(ws, pl.S, M, N, C, ldc, mode, st);
}

int launch_gemm_t(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                  void* ws, size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (K % 128) return fail(IFD_ERR_ARG, "T64 GEMM needs K %% 128 == 0 (K=%d)", K);
  // decode batches: the stream-K kernel (every CU streams an equal share of the weights, fixup kernel after)
  if (!use_t8(M, N) && gemm_sk_applies(M, N, K, mode))
    return launch_gemm_sk(A, lda, wt, N, K, C, ldc, M, mode, ws, ws_bytes, st);
  if (use_t8(M, N)) {
    const size_t need = gemm_t_workspace(M, N, K, mode), t8ws = gemm_t8_workspace(M, N, K);
    if (need > ws_bytes || (need && !ws))
      return fail(IFD_ERR_WORKSPACE, "gemm_t64 needs %zu bytes of workspace, got %zu", need, ws_bytes);
    if (mode != kModeSwiglu) return launch_gemm_t8(A, lda, wt, N, K, C, ldc, M, mode, ws, t8ws, st);
    // SwiGLU: the bf16 product into the workspace (after the tail partials), then silu_mul
    uint16_t* gu = (uint16_t*)((char*)ws + align_up(t8ws, 256));
    IFD_TRY(launch_gemm_t8(A, lda, wt, N, K, gu, N, M, 0, ws, t8ws, st));
    return launch_silu_mul(gu, N, (uint16_t*)C, ldc, N / 2, M, st);
  }
  const GtPlan pl = gemm_t_plan(M, N, K);
  const size_t need = epilogue_ws_bytes(pl.S, M, N, mode);
  if (need > ws_bytes || (need && !ws))
    return fail(IFD_ERR_WORKSPACE, "gemm_t64 needs %zu bytes of workspace, got %zu", need, ws_bytes);
  // the SwiGLU mode without a split stores the bf16 product into the workspace for silu_mul
  const bool via_ws = mode == kModeSwiglu && pl.S == 1;
  GemmTArgs p{A, lda, (const uint8_t*)wt, N, K, via_ws ? ws : C, via_ws ? N : ldc, M, via_ws ? 0 : mode, (float*)ws,
              pl.gps, (M + 32 * pl.MT - 1) / (32 * pl.MT), (t64_bands(N) + 4 * pl.NB - 1) / (4 * pl.NB), nullptr, 0};
  int rc;
  if (pl.MT == 1) rc = launch_gemm_t_cfg<1, 2, false>(p, pl.S, st);
  else if (pl.MT == 2) rc = launch_gemm_t_cfg<2, 2, false>(p, pl.S, st);
  else rc = launch_gemm_t_cfg<4, 2, true>(p, pl.S, st);
  IFD_TRY(rc);
  return launch_epilogue(ws, pl.S, M, N, C, ldc, mode, st);
}

}  // namespace ifd
