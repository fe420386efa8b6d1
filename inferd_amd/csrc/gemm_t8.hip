// Prefill GEMM on T64 weights, 256-row tiles: C (mode) = A . W^T with every weight dequantized to bf16(s q + b) (MLX
// qmm rounding, quantized.h:528-535) and fp32 accumulation (reference affine_qmm_t_nax,
// third_party/mlx/.../quantized_nax.h:938-1076, 1206-1267).
//
// Block: 8 waves (two per SIMD), tile 256 rows x 8 bands (256 columns); wave w owns bands 2 (w % 4), 2 (w % 4) + 1
// over M tiles 4 (w / 4) .. + 3 of 32 rows (128 fp32 accumulators per lane). One activation fragment read from LDS
// feeds two MFMAs and one dequantized B fragment four: each band is dequantized by two waves, and the LDS serves
// half the activation bytes of a one-band-per-wave layout (an MFMA reading its whole A operand from LDS would need
// the LDS's full bandwidth).
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
constexpr int kT8NW = 5;   // weight stages in the LDS ring (two steps further ahead)
constexpr int kT8Band = 4;  // M tiles per band of the tile order
constexpr int kT8Row = 256 + 4;  // staged half-tile row stride (floats)

struct GemmT8Args {
  const uint16_t* A;
  int lda;
  const uint8_t* wt;
  uint32_t w_bytes;  // bytes of the T64 weights (buffer bound)
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

// One wave-wide 16-byte-per-lane DMA through a buffer resource: lane l's 16 bytes at voff(l) + soff land at
// lds + 16 l (LDS base in M0, wave-uniform control flow only).
__device__ __forceinline__ void t8_dma(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, (int)voff, (int)soff, 0, 0);
}

// The pipeline of one wave; W0: wave 0, which also issues the (s, b) rows. Step s issues, right after its barrier,
// the activations of group s + 2 and the weights of group s + 4, and waits at its barrier for the activations of s
// (read through the step) and the weights of s + 2 (whose codes it reads for the dequant at step s + 1): both were
// issued two steps earlier, and only the previous step's DMAs are younger. Past the split's end the streams re-read
// its last group into stages nobody reads, so every step issues the same DMAs and every wait is a constant.
template <bool W0>
__device__ __forceinline__ void t8_body(const GemmT8Args& p, uint8_t* lds, const int wave, const int Lrel, int tm,
                                        int tn) {
  constexpr int BM = 256, NBB = 8;
  constexpr int A_BYTES = BM * 128;                     // activation slab [256][64 bf16]
  constexpr int W_BYTES = NBB * kT64Codes + NBB * 128;  // code halves [8][1024] + (s, b) rows [8][128]
  constexpr int D = 4 + 1 + (W0 ? 1 : 0);               // DMAs per step
  uint8_t* const aring = lds;                    // kT8NS slabs
  uint8_t* const wring = lds + kT8NS * A_BYTES;  // kT8NW weight stages
  const int tid = threadIdx.x, lane = tid & 63;
  const int j = lane & 31, h = lane >> 5;
  const int m0 = tm * BM;
  const int nbands = t64_bands(p.N);
  const int G = p.K / kGroup;
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps), Gz = g1 - g0;
  const uint32_t gstride = (uint32_t)nbands * kT64Tile;

  // activation DMA i (0..3) of this wave covers rows 8 (4 wave + i) .. + 7: lane -> row 8 (4 wave + i) + lane / 8,
  // physical 16-byte column lane % 8 holding logical column (lane % 8) ^ ((row / 2) % 8). Rows past M re-read row
  // M - 1 (their outputs are not stored).
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.A, 0, (int)((uint32_t)p.M * p.lda * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)p.wt, 0, (int)p.w_bytes, 0x00020000);
  uint32_t va[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 8 * (4 * wave + i) + lane / 8;
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    va[i] = (uint32_t)min(m0 + r, p.M - 1) * (uint32_t)p.lda * 2u + 16u * c;
  }
  const uint32_t vw = (uint32_t)min(tn * NBB + wave, nbands - 1) * kT64Tile + 16u * lane;
  const uint32_t vs = (uint32_t)min(tn * NBB + lane / 8, nbands - 1) * kT64Tile + kT64Codes + 16u * (lane & 7);

  // the streams: group offsets of the next issue, clamped to the split's last group
  int ga = g0, gw = g0, sa_st = 0, sw_st = 0;
  auto issue_a = [&]() __attribute__((always_inline)) {
    uint8_t* st = aring + sa_st * A_BYTES;
    const uint32_t so = (uint32_t)min(ga, g1 - 1) * 2u * kGroup;
#pragma unroll
    for (int i = 0; i < 4; i++) t8_dma(ra, st + (4 * wave + i) * 1024, va[i], so);
    ga++;
    sa_st = sa_st + 1 == kT8NS ? 0 : sa_st + 1;
  };
  auto issue_w = [&]() __attribute__((always_inline)) {
    uint8_t* st = wring + sw_st * W_BYTES;
    const uint32_t so = (uint32_t)min(gw, g1 - 1) * gstride;
    t8_dma(rw, st + wave * kT64Codes, vw, so);
    if constexpr (W0) t8_dma(rw, st + NBB * kT64Codes, vs, so);
    gw++;
    sw_st = sw_st + 1 == kT8NW ? 0 : sw_st + 1;
  };

  // compute roles: wave w owns bands 2 bp, 2 bp + 1 (bp = w % 4) over M tiles 4 mh .. 4 mh + 3 (mh = w / 4), so one
  // activation fragment read from LDS feeds two MFMAs
  const int mh = wave >> 2, bp = wave & 3;
  f32x16 acc[2][4];
#pragma unroll
  for (int nb = 0; nb < 2; nb++)
#pragma unroll
    for (int a = 0; a < 4; a++) acc[nb][a] = zero16();
  struct Codes {
    u32x4 w[2];
    uint32_t sb[2];
  };
  auto read_codes = [&](int ws, Codes& cd) __attribute__((always_inline)) {  // the wave's two bands of stage ws
    const uint8_t* wst = wring + ws * W_BYTES;
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const int band = 2 * bp + nb;
      cd.w[nb] = *(const u32x4*)(wst + band * kT64Codes + 16 * lane);
      cd.sb[nb] = *(const uint32_t*)(wst + NBB * kT64Codes + band * 128 + 4 * j);
    }
  };
  auto dequant = [&](const Codes& cd, u32x4 (&bf)[2][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const float sc = bf2f((uint16_t)(cd.sb[nb] & 0xFFFFu)), bi = bf2f((uint16_t)(cd.sb[nb] >> 16));
      const float sa = t64_sa(sc), sbs = t64_sb(sc);
#pragma unroll
      for (int t = 0; t < 4; t++) bf[nb][t] = t64_dequant(cd.w[nb][t], sa, sbs, bi);
    }
  };
  // activation fragments of the wave's M tile a: MFMA step t takes k = 32 h + 8 t .. + 7 (logical column 4 h + t)
  auto load_a = [&](const uint8_t* st, int a, u32x4 (&af)[4]) __attribute__((always_inline)) {
    const int r = (4 * mh + a) * 32 + j;
#pragma unroll
    for (int t = 0; t < 4; t++) af[t] = *(const u32x4*)(st + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
  };

  // prologue: A(0), A(1) and W(0) .. W(3); then W(0) dequantized and W(1)'s codes read before step 0
  for (int s = 0; s < 2; s++) {
    issue_a();
    issue_w();
  }
  issue_w();
  issue_w();
  // W(1) landed: the younger DMAs are W(2), W(3)
  if constexpr (W0) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  u32x4 bf0[2][4], bf1[2][4];
  Codes cc;
  read_codes(0, cc);
  dequant(cc, bf0);
  read_codes(1, cc);
  int ca = 0, cw2 = 2;  // stages: activations of step s, weights of step s + 2

  // Step s: bc (B fragments of s) and cc (codes of s + 1) in registers; dequantizes cc into bn, then reads the codes
  // of s + 2 into cc (the next barrier waits for them). Four groups, one per M tile, each closed by a scheduling
  // barrier: the tile's eight MFMAs (two bands), the next tile's activation fragments and a quarter of the dequant.
  auto step = [&](u32x4 (&bc)[2][4], u32x4 (&bn)[2][4]) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(D) : "memory");
    issue_a();
    issue_w();
    const uint8_t* ast = aring + ca * A_BYTES;
    float sa[2], sbs[2], bi[2];
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const float sc = bf2f((uint16_t)(cc.sb[nb] & 0xFFFFu));
      bi[nb] = bf2f((uint16_t)(cc.sb[nb] >> 16)), sa[nb] = t64_sa(sc), sbs[nb] = t64_sb(sc);
    }
    u32x4 af[2][4];
    load_a(ast, 0, af[0]);
#pragma unroll
    for (int a = 0; a < 4; a++) {
      if (a + 1 < 4) load_a(ast, a + 1, af[(a + 1) & 1]);
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const int d = 2 * a + k;  // dequant word d: band d / 4, word d % 4
        bn[d / 4][d % 4] = t64_dequant(cc.w[d / 4][d % 4], sa[d / 4], sbs[d / 4], bi[d / 4]);
      }
#pragma unroll
      for (int nb = 0; nb < 2; nb++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[nb][a] = mfma_bf16(af[a & 1][t], bc[nb][t], acc[nb][a]);
#pragma unroll
      for (int m = 0; m < 8; m++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (m < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int t = 0; t < 4; t++) asm volatile("" : "+v"(bn[nb][t]));
    read_codes(cw2, cc);
    ca = ca + 1 == kT8NS ? 0 : ca + 1;
    cw2 = cw2 + 1 == kT8NW ? 0 : cw2 + 1;
  };
  int s = 0;
  for (; s + 1 < Gz; s += 2) {
    step(bf0, bf1);
    step(bf1, bf0);
  }
  if (s < Gz) step(bf0, bf1);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // The tile leaves through LDS (free after the K loop) in two halves of 128 rows: the four waves holding a half
  // stage it as fp32 [128][kT8Row], then all waves store whole rows, 4 columns per access (a split tail: its compact
  // fp32 partials).
  const bool split = gridDim.y > 1;
  float* const stg = (float*)lds;
#pragma unroll
  for (int hf = 0; hf < 2; hf++) {
    if (mh == hf)
#pragma unroll
      for (int nb = 0; nb < 2; nb++)
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
          for (int r = 0; r < 16; r++)
            stg[(a * 32 + 8 * (r / 4) + 4 * h + (r % 4)) * kT8Row + (2 * bp + nb) * 32 + j] = acc[nb][a][r];
    __syncthreads();
    for (int e = tid; e < 128 * 64; e += 512) {
      const int row = e >> 6, c4 = (e & 63) * 4, lrow = 128 * hf + row, grow = m0 + lrow, gcol = tn * 256 + c4;
      if (grow >= p.M || gcol >= p.N) continue;
      const float4 v = *(const float4*)(stg + row * kT8Row + c4);
      if (split) {
        *(float4*)(p.part + (((size_t)blockIdx.y * p.ntail + Lrel) * BM + lrow) * 256 + c4) = v;
        continue;
      }
      const size_t o = (size_t)grow * p.ldc + gcol;
      if (gcol + 4 <= p.N && (o & 3) == 0 && p.mode != 1) {
        if (p.mode == 2) *(float4*)((float*)p.C + o) = v;
        else *(u32x2*)((uint16_t*)p.C + o) = u32x2{pack_bf2(v.x, v.y), pack_bf2(v.z, v.w)};
      } else {
        const float vv[4] = {v.x, v.y, v.z, v.w};
        for (int k = 0; k < 4 && gcol + k < p.N; k++) store_mode(p.C, o + k, vv[k], p.mode);
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(512, 1) void k_gemm_t8(GemmT8Args p) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int Lrel = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  t8_tile(p.tile0 + Lrel, p.tiles_m, p.tiles_n, tm, tn);
  if (wave == 0) t8_body<true>(p, lds, wave, Lrel, tm, tn);
  else t8_body<false>(p, lds, wave, Lrel, tm, tn);
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
  constexpr size_t ring = (size_t)kT8NS * 256 * 128 + (size_t)kT8NW * (8 * kT64Codes + 8 * 128);
  constexpr size_t lds = ring > (size_t)128 * kT8Row * 4 ? ring : (size_t)128 * kT8Row * 4;  // ring, then half a tile
  static bool attr = false;
  if (!attr) {
    hipFuncSetAttribute((const void*)k_gemm_t8, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr = true;
  }
  const int tiles_m = (M + 255) / 256, tiles_n = (t64_bands(N) + 7) / 8;
  const int G = K / kGroup;
  if (t64_bytes(N, K) >= ((size_t)1 << 31) || (size_t)M * lda * 2 >= ((size_t)1 << 31))
    return fail(IFD_ERR_UNSUPPORTED, "gemm_t8: operands past 2 GiB");
  const uint32_t wb = (uint32_t)t64_bytes(N, K);
  GemmT8Args p{A, lda, (const uint8_t*)wt, wb, N, K, C, ldc, M, mode, (float*)ws, G, tiles_m, tiles_n, 0, 0};
  hipLaunchKernelGGL(k_gemm_t8, dim3(pl.full, 1), dim3(512), lds, st, p);
  IFD_TRY(check_launch("gemm_t8"));
  if (!pl.St) return IFD_OK;
  const int ntail = pl.tiles - pl.full;
  GemmT8Args q{A, lda, (const uint8_t*)wt, wb, N, K, C, ldc, M, mode, (float*)ws, pl.gpt, tiles_m, tiles_n, pl.full,
               ntail};
  hipLaunchKernelGGL(k_gemm_t8, dim3(ntail, pl.St), dim3(512), lds, st, q);
  IFD_TRY(check_launch("gemm_t8 tail"));
  const size_t n = (size_t)ntail * 256 * 64;
  hipLaunchKernelGGL(k_t8_tail_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const float*)ws, pl.St,
                     ntail, pl.full, tiles_m, tiles_n, M, N, C, ldc, mode);
  return check_launch("gemm_t8 tail reduce");
}

}  // namespace ifd
