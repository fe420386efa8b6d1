// Gathered expert GEMM on T64 expert stacks: C[q][n] = bf16(sum_k A_row(q)[k] * bf16(s q + b)[n][k]) over expert-
// sorted rows q, with the SwiGLU of a [gate | up] stack fused (C receives h), for the MoE FFN's gate/up and down
// products (reference affine_gather_qmm_rhs, third_party/mlx/.../quantized_nax.h:1467-1681, scheduled by
// schedule_row_tile, steel/utils.h:502-542; moe_silu_mul, moe.metal:103-111).
//
// Work items are (row tile, column tile) pairs: a row tile is up to BM = 32 MT sorted rows of one expert (the
// dispatch's tile schedule), a column tile 8 bands (256 output columns; with SwiGLU 8 gate bands and the matching 8
// up bands, 256 h columns). Items are numbered row tile-major, so an expert's column tiles are neighbours and share
// its activation rows in L2. The grid is one block per CU; block b streams items [b n / nblk, (b + 1) n / nblk) as one
// continuous sequence of (item, 64-group) steps, so the DMA pipeline runs across item boundaries without draining.
//
// Block: 8 waves; wave w owns band w of the column tile (with SwiGLU, its gate band and its up band) over all MT M
// tiles. Two LDS rings filled by direct global -> LDS DMA: NA activation slabs [BM][64 bf16] (16-byte columns
// XOR-swizzled by row pair), whose rows are gathered through perm by the DMA itself (row q of a tile is token
// perm[q] / div, or row q of A), and NW weight stages (the item's code halves and (s, b) rows of one group). Waves
// 0-3 issue the activation DMAs, waves 4-7 the weight DMAs, each with its own in-order vmcnt stream. Row indices
// come from scalar loads, which do not count in vmcnt. Weights are dequantized to bf16(s q + b) (MLX's gather_qmm
// rounding) one step ahead of their MFMAs; the k order of a lane's MFMA steps is that of k_gqmm, so the sums are
// bit-identical to it.
//
// At the end of an item a wave stages its bf16 outputs in its own LDS tile and writes them as 16-byte buffer
// stores, rows past the segment at an out-of-range offset (dropped by the buffer bounds check, yet issued, so each
// wave's count of outstanding stores is exact). The vmcnt waits count those stores among the younger operations.
#include <algorithm>

#include "common.h"
#include "dma.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"
#include "t64_dev.h"

namespace ifd {

constexpr int kGqThreads = 512;

struct GqArgs {
  const uint16_t* A;
  int lda;
  const int* perm;  // null: sorted row q reads row q of A
  uint32_t div_m;   // perm[q] / div = mulhi(perm[q], div_m) (div_m = ceil(2^32 / div)); 0 when div = 1
  const int* tiles;    // [ntiles][2] = (expert, first sorted row)
  const int* ntiles;   // [1]
  const int* offsets;  // [E + 1] (+ 1 with the shared segment)
  const uint8_t* wt;   // routed experts' T64 stack, expert e at e * ebytes
  size_t ebytes;
  const uint8_t* wsh;  // the shared expert (expert index E), or null
  int E, N, K, G;
  uint16_t* C;
  uint32_t c_bytes;
  int ldc, nct_log2, nblk;
};

// bands per wave: two with SwiGLU (its gate and up band) or in the wide plain form (two 8-band column groups)
__host__ __device__ constexpr int gq_nbw(bool two) { return two ? 2 : 1; }
__host__ __device__ constexpr int gq_abytes(int MT) { return MT * 32 * 128; }
__host__ __device__ constexpr int gq_wbytes(bool two) { return gq_nbw(two) * (8 * kT64Codes + 8 * 128); }
constexpr int kGqStg = 32 * 64;  // a wave's staged output: one M tile [32][32] bf16
__host__ __device__ constexpr int gq_na(int MT, bool two) { return two ? 4 : (MT == 2 ? 6 : 8); }
__host__ __device__ constexpr int gq_nw(int MT, bool two) { return two ? (MT == 2 ? 6 : 7) : (MT == 2 ? 10 : 12); }
__host__ __device__ constexpr size_t gq_lds(int MT, bool two) {
  return (size_t)gq_na(MT, two) * gq_abytes(MT) + (size_t)gq_nw(MT, two) * gq_wbytes(two) + 8 * kGqStg;
}

// A scalar (SMEM) load of a wave-uniform element: it counts in lgkmcnt, not in vmcnt.
__device__ __forceinline__ int sload(const int* p, int i) {
  return *((const __attribute__((address_space(4))) int*)p + __builtin_amdgcn_readfirstlane(i));
}

// WIDE (plain only): each wave owns two bands, 8 apart, so an item is 16 bands (512 columns)
template <int MT, bool SILU, bool WIDE>
__global__ __launch_bounds__(kGqThreads, 1) void k_gqmm_t(GqArgs p) {
  constexpr bool TWO = SILU || WIDE;
  constexpr int BM = 32 * MT, NBW = gq_nbw(TWO), NA = gq_na(MT, TWO), NW = gq_nw(MT, TWO);
  constexpr int A_BYTES = gq_abytes(MT), W_BYTES = gq_wbytes(TWO);
  constexpr int SB_OFF = NBW * 8 * kT64Codes;  // (s, b) rows of a weight stage, after its code tiles
  constexpr int NCW = TWO ? 4 : 2;             // code DMAs per weight wave per step
  static_assert(!(SILU && WIDE), "SwiGLU pairs a gate and an up band per wave");
  static_assert(gq_lds(MT, TWO) <= 160 * 1024, "LDS plan");
  static_assert(MT * (NA - 2) + 8 * MT <= 63 && (NCW + 1) * (NW - 2) + 8 * MT <= 63, "vmcnt range");
  extern __shared__ __align__(16) uint8_t lds[];
  uint8_t* const aring = lds;
  uint8_t* const wring = lds + NA * A_BYTES;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, h = lane >> 5;
  uint16_t* const stg = (uint16_t*)(wring + NW * W_BYTES + wave * kGqStg);

  const int b = xcd_remap(blockIdx.x, p.nblk);
  const int nitems = sload(p.ntiles, 0) << p.nct_log2;
  const int it0 = (int)((long)b * nitems / p.nblk), it1 = (int)((long)(b + 1) * nitems / p.nblk);
  if (it0 >= it1) return;  // block-uniform, before any barrier
  const int G = p.G, n = (it1 - it0) * G;
  const int nbands = t64_bands(p.N);
  const size_t gstride = (size_t)nbands * kT64Tile;
  const int up0 = nbands / 2;  // first up band of a [gate | up] stack

  // weight DMA roles of waves 4-7 (ww = wave - 4): SwiGLU, code tiles [4 ww, 4 ww + 4) of the stage's 16 (8 gate +
  // 8 up bands) and the (s, b) DMA ww for ww < 2; plain, code tiles [2 ww, 2 ww + 2) of 8 and the (s, b) DMA for
  // ww = 3
  const int ww = wave - 4;
  const bool has_sb = TWO ? ww < 2 : ww == 3;
  const int sbj = TWO ? ww : 0;

  // (expert, column tile, rows) of an item; a tile holds at least its first row
  auto item_rows = [&](int item, int& e, int& c, int& q0, int& q1) __attribute__((always_inline)) {
    const int tile = item >> p.nct_log2;
    c = item & ((1 << p.nct_log2) - 1);
    e = min(max(sload(p.tiles, 2 * tile), 0), p.E);
    q0 = sload(p.tiles, 2 * tile + 1);
    q1 = max(min(sload(p.offsets, e + 1), q0 + BM), q0 + 1);
  };
  auto band_of = [&](int c, int ti) __attribute__((always_inline)) {  // physical band of the stage's tile ti
    const int bb = SILU ? (ti < 8 ? 8 * c + ti : up0 + 8 * c + ti - 8) : (WIDE ? 16 * c + ti : 8 * c + ti);
    return min(bb, nbands - 1);
  };

  // ---- DMA streams: (item, group) of the next step to issue
  int s_item = it0, s_g = 0, s_i = 0, s_st = 0;
  const uint16_t* arow[MT];
  const uint8_t* wsrc[NCW + 1];  // the code sources, then the (s, b) source
  auto stream_item = [&](int item) __attribute__((always_inline)) {
    int e, c, q0, q1;
    item_rows(item, e, c, q0, q1);
    if (wave < 4) {
      // the wave's 8 MT row indices: all scalar loads in flight at once, then one wait
      int v[MT][8];
#pragma unroll
      for (int i = 0; i < MT; i++)
#pragma unroll
        for (int rho = 0; rho < 8; rho++) v[i][rho] = min(q0 + 8 * (MT * wave + i) + rho, q1 - 1);
      if (p.perm) {
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
          for (int rho = 0; rho < 8; rho++) v[i][rho] = sload(p.perm, v[i][rho]);
        if (p.div_m)
#pragma unroll
          for (int i = 0; i < MT; i++)
#pragma unroll
            for (int rho = 0; rho < 8; rho++)
              v[i][rho] = (int)__builtin_amdgcn_readfirstlane(__umulhi((uint32_t)v[i][rho], p.div_m));
      }
#pragma unroll
      for (int i = 0; i < MT; i++) {
        const int r0 = 8 * (MT * wave + i);
        int src = 0;
#pragma unroll
        for (int rho = 0; rho < 8; rho++) src = (lane >> 3) == rho ? v[i][rho] : src;
        const int r = r0 + (lane >> 3);
        const int c16 = (lane & 7) ^ ((r >> 1) & 7);
        arow[i] = p.A + (size_t)src * p.lda + 8 * c16;
      }
    } else {
      // expert E is the shared expert; without one the reads stay inside the stack
      const uint8_t* wb = e >= p.E && p.wsh ? p.wsh : p.wt + (size_t)min(e, p.E - 1) * p.ebytes;
#pragma unroll
      for (int i = 0; i < NCW; i++) wsrc[i] = wb + (size_t)band_of(c, NCW * ww + i) * kT64Tile + 16 * lane;
      wsrc[NCW] = wb + (size_t)band_of(c, 8 * sbj + (lane >> 3)) * kT64Tile + kT64Codes + 16 * (lane & 7);
    }
  };
  stream_item(s_item);
  auto issue = [&]() __attribute__((always_inline)) {
    if (wave < 4) {
      uint8_t* st = aring + s_st * A_BYTES;
#pragma unroll
      for (int i = 0; i < MT; i++) dma16(arow[i] + (size_t)s_g * kGroup, st + (MT * wave + i) * 1024);
      s_st = s_st + 1 == NA ? 0 : s_st + 1;
    } else {
      uint8_t* st = wring + s_st * W_BYTES;
      const size_t off = (size_t)s_g * gstride;
#pragma unroll
      for (int i = 0; i < NCW; i++) dma16(wsrc[i] + off, st + (NCW * ww + i) * kT64Codes);
      if (has_sb) dma16(wsrc[NCW] + off, st + SB_OFF + sbj * 1024);
      s_st = s_st + 1 == NW ? 0 : s_st + 1;
    }
    s_i++;
    if (++s_g == G) {
      s_g = 0;
      if (++s_item < it1) stream_item(s_item);
    }
  };

  // this wave's bands of weight stage ws, dequantized
  auto dequant = [&](int ws, u32x4 (&bf)[NBW][4]) __attribute__((always_inline)) {
    const uint8_t* wst = wring + ws * W_BYTES;
#pragma unroll
    for (int nb = 0; nb < NBW; nb++) {
      const int t = 8 * nb + wave;
      const u32x4 codes = *(const u32x4*)(wst + t * kT64Codes + 16 * lane);
      const uint32_t sb = *(const uint32_t*)(wst + SB_OFF + t * 128 + 4 * j);
      const float sc = bf2f((uint16_t)(sb & 0xFFFFu)), bi = bf2f((uint16_t)(sb >> 16)), sa = t64_sa(sc), sbs = t64_sb(sc);
#pragma unroll
      for (int q = 0; q < 4; q++) bf[nb][q] = t64_dequant(codes[q], sa, sbs, bi);
    }
  };
  auto load_a = [&](const uint8_t* st, int a, u32x4 (&af)[4]) __attribute__((always_inline)) {
    const int r = a * 32 + j;
#pragma unroll
    for (int t = 0; t < 4; t++) af[t] = *(const u32x4*)(st + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
  };

  f32x16 acc[NBW][MT];
#pragma unroll
  for (int nb = 0; nb < NBW; nb++)
#pragma unroll
    for (int a = 0; a < MT; a++) acc[nb][a] = zero16();

  // Waits. A wave waits until only younger operations than the DMA it needs are outstanding: its later DMAs and
  // the output stores (NST per item end) of the item ends it issued after that DMA. Every operation of a wave
  // completes in issue order, so the needed DMA has landed. nrec: those item ends (0, 1 or 2).
  constexpr int NST = 2 * MT * (WIDE ? 2 : 1);  // output stores per item end
  auto wait_a = [&](int k, int nrec) __attribute__((always_inline)) { wait_vm_rec<MT, NA - 2, NST>(k, nrec); };
  auto wait_w = [&](int k, int nrec, bool first) __attribute__((always_inline)) {  // k = younger weight steps
    if (first) {
      if (has_sb) wait_vm_dyn<NCW + 1, NW - 2>(k);
      else wait_vm_dyn<NCW, NW - 2>(k);
    } else {
      if (has_sb) wait_vm_rec<NCW + 1, NW - 3, NST>(k, nrec);
      else wait_vm_rec<NCW, NW - 3, NST>(k, nrec);
    }
  };
  {
    const int pre = min(wave < 4 ? NA - 1 : NW - 1, n);
    for (int i = 0; i < pre; i++) issue();
  }
  if (wave >= 4) wait_w(min(NW - 2, n - 1), 0, true);  // W(0) for the first dequant
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  u32x4 bf0[NBW][4], bf1[NBW][4];
  dequant(0, bf0);
  int ca = 0, cw = 1 % NW;

  // step i with the B fragments of step i in bc; dequantizes step i + 1 into bn. Waves 0-3 need A(i), waves 4-7
  // W(i + 1); the stage a DMA issued here overwrites held a step every wave finished before the barrier.
  // Item ends whose stores are younger than the DMA awaited at step i: for A(i), issued at step i - NA + 1, those
  // at the ends of steps i - NA + 1 .. i - 1; for W(i + 1), issued at step i + 2 - NW, those from step i + 2 - NW.
  int d1 = 1 << 20, d2 = 1 << 20;  // steps since the last two item ends
  auto step = [&](int i, u32x4 (&bc)[NBW][4], u32x4 (&bn)[NBW][4]) __attribute__((always_inline)) {
    if (wave < 4) wait_a(min(NA - 2, n - 1 - i), (d1 < NA - 1) + (d2 < NA - 1));
    else if (i + 1 < n) wait_w(min(NW - 3, n - 2 - i), (d1 < NW - 2) + (d2 < NW - 2), false);
    d1++, d2++;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (s_i < n) issue();
    dequant(cw, bn);  // past the run's end a stale stage, never used: one basic block with the MFMAs
    const uint8_t* ast = aring + ca * A_BYTES;
    u32x4 af[2][4];
    load_a(ast, 0, af[0]);
#pragma unroll
    for (int a = 0; a < MT; a++) {
      if (a + 1 < MT) load_a(ast, a + 1, af[(a + 1) & 1]);
#pragma unroll
      for (int nb = 0; nb < NBW; nb++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[nb][a] = mfma_bf16(af[a & 1][t], bc[nb][t], acc[nb][a]);
    }
    ca = ca + 1 == NA ? 0 : ca + 1;
    cw = cw + 1 == NW ? 0 : cw + 1;
  };

  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)p.C, 0, (int)p.c_bytes, 0x00020000);
  // The item's outputs, one M tile at a time: bf16 (SwiGLU: h of the bf16 gate and up sums) into this wave's LDS
  // tile [32][32], then two 16-byte stores of 16 rows x 32 columns; rows past the segment go to an offset past the
  // buffer, which the bounds check drops.
  auto epilogue = [&](int c, int q0, int q1) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < (WIDE ? 2 : 1); nb++) {
      const int col = ((WIDE ? 16 * c + 8 * nb : 8 * c) + wave) * 32 + 8 * (lane & 3);
#pragma unroll
      for (int a = 0; a < MT; a++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float v = acc[nb][a][r];
          if (SILU) v = swiglu_f(bf2f(f2bf(acc[0][a][r])), bf2f(f2bf(acc[NBW - 1][a][r])));
          stg[(8 * (r / 4) + 4 * h + (r % 4)) * 32 + j] = f2bf(v);
        }
        asm volatile("" ::: "memory");  // the 16-byte reads below see the 2-byte writes above (same wave, in order)
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) {
          const int row = 16 * s2 + (lane >> 2);
          const u32x4 v = *(const u32x4*)(stg + row * 32 + 8 * (lane & 3));
          const int q = q0 + 32 * a + row;
          const int off = q < q1 ? (int)(((size_t)q * p.ldc + col) * 2) : 0x7FFFFFF0;
          __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 0);
        }
        asm volatile("" ::: "memory");  // the next tile's writes come after these reads
      }
    }
#pragma unroll
    for (int nb = 0; nb < NBW; nb++)
#pragma unroll
      for (int a = 0; a < MT; a++) acc[nb][a] = zero16();
  };

  int i = 0;
  for (int item = it0; item < it1; item++) {
    int e, c, q0, q1;
    item_rows(item, e, c, q0, q1);
    (void)e;
    for (int g = 0; g < G; g += 2, i += 2) {  // G is even
      step(i, bf0, bf1);
      step(i + 1, bf1, bf0);
    }
    epilogue(c, q0, q1);
    d2 = d1, d1 = 0;
  }
}

// ---- host side

static int gq_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  }
  return n;
}

template <int MT, bool SILU, bool WIDE>
static int launch_gq_cfg(const GqArgs& a, hipStream_t st) {
  constexpr size_t lds = gq_lds(MT, SILU || WIDE);
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)k_gqmm_t<MT, SILU, WIDE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
    attr = true;
  }
  hipLaunchKernelGGL((k_gqmm_t<MT, SILU, WIDE>), dim3(a.nblk), dim3(kGqThreads), lds, st, a);
  return check_launch("moe_gather_qmm_t64");
}

int launch_moe_gather_qmm_t64(const uint16_t* A, int lda, const int* perm, int div, const int* tiles,
                              const int* ntiles, const int* offsets, int tile_rows, const void* wt, const void* wsh,
                              int E, int N, int K, int silu, uint16_t* C, int ldc, int rows, hipStream_t st) {
  if (rows == 0) return IFD_OK;
  if (tile_rows != 32 && tile_rows != 64)
    return fail(IFD_ERR_ARG, "moe_gather_qmm_t64: tile_rows=%d must be 32 or 64", tile_rows);
  if (K % 128) return fail(IFD_ERR_ARG, "moe_gather_qmm_t64: K=%d must be a multiple of 128", K);
  const int NO = silu ? N / 2 : N;
  if (N % 256 || NO % 256)
    return fail(IFD_ERR_ARG, "moe_gather_qmm_t64: N=%d must give output columns in whole 256-column tiles", N);
  const size_t cb = (size_t)rows * ldc * sizeof(uint16_t);
  if (cb >= ((size_t)1 << 31) - 64) return fail(IFD_ERR_UNSUPPORTED, "moe_gather_qmm_t64: output past 2 GiB");
  if (div < 1 || div > 64) return fail(IFD_ERR_ARG, "moe_gather_qmm_t64: div=%d must be in [1, 64]", div);
  // perm[q] / div as a multiply-high: exact for perm values below 2^32 / div (2^26 at div = 64)
  const uint32_t div_m = div == 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + div - 1) / div);
  // plain products with output columns in whole 512-column tiles take the wide form (two bands per wave)
  const bool wide = !silu && NO % 512 == 0;
  const int nct = NO / (wide ? 512 : 256);
  if (nct & (nct - 1)) return fail(IFD_ERR_UNSUPPORTED, "moe_gather_qmm_t64: %d column tiles (not a power of 2)", nct);
  GqArgs a{A, lda, perm, div_m, tiles, ntiles, offsets, (const uint8_t*)wt, t64_bytes(N, K), (const uint8_t*)wsh,
           E, N, K, K / kGroup, C, (uint32_t)cb, ldc, __builtin_ctz(nct), gq_cus()};
  const int MT = tile_rows / 32;
  if (silu) return MT == 2 ? launch_gq_cfg<2, true, false>(a, st) : launch_gq_cfg<1, true, false>(a, st);
  if (wide) return MT == 2 ? launch_gq_cfg<2, false, true>(a, st) : launch_gq_cfg<1, false, true>(a, st);
  return MT == 2 ? launch_gq_cfg<2, false, false>(a, st) : launch_gq_cfg<1, false, false>(a, st);
}

}  // namespace ifd
