// Stream-K GEMM on T64 weights for decode batches (16 < M, below the 256-row prefill tiles): C (mode) = A . W^T with
// every weight dequantized to bf16(s q + b) (MLX qmm rounding, third_party/mlx/.../quantized.h:528-535) and fp32
// accumulation. Serves the reference's affine_qmm_t_nax (quantized_nax.h:938-1076) with its split-K variant
// (engine/kernels/qmm_splitk.metal:14-107) and, in the SwiGLU mode, the gemm -> silu_mul pair of the MLP
// (engine/src/qwen35.h:1693-1700).
//
// Work is the set of units (tile, 64-group); a tile is BM = 32 MT rows x 8 bands (256 columns). Block b (of nblk,
// one or two per CU) takes units [b U / nblk, (b + 1) U / nblk) (stream-K): every CU streams the same weight bytes
// whatever the tile count. A run never covers more than one tile's worth of groups, so it touches at most two tiles
// ("segments"). A segment covering its whole tile is stored by the block; any other segment is a piece of its tile,
// and its fp32 sums go to the block's partial slot (the first segment's as soon as it ends, while the run goes on).
// k_sk_fixup then sums each cut tile's pieces in unit order, in parallel over all CUs, and stores it: the result
// does not depend on timing.
//
// Block: 4 waves (one per SIMD); wave w owns bands 2w and 2w + 1 of the tile over all MT M tiles, so one
// activation fragment read from LDS feeds two MFMAs and one dequantized weight fragment feeds MT. One LDS ring
// filled by direct global -> LDS DMA; a stage holds a step's activation slab [BM][64 bf16] (16-byte columns
// XOR-swizzled by row pair) and its weights (8 code halves + 8 (s, b) rows). Each wave issues its own share of both
// (the activation rows 8 (MT w + q) .. + 7 and its two bands' codes; wave 0 also the (s, b) rows) as one in-order
// vmcnt stream, the activations R - 1 steps ahead and the weights R; the stream positions advance incrementally (no
// per-step division). Within a step the wave reads its activation fragments and the next step's codes from LDS
// first, then runs its MFMAs with the next step's dequant scheduled between them. Every DMA is issued by a whole
// wave under wave-uniform control flow (the LDS base goes to M0). Finished tiles are staged through LDS and leave as
// whole rows.
//
// SwiGLU mode: tile t holds gate bands 4t..4t+3 (waves 0, 1) and the matching up bands (waves 2, 3); the staged tile
// (or the fixup) gives h = silu(bf16(gate)) * bf16(up) (reference silu_mul, core.metal:777-787).
#include <algorithm>

#include "common.h"
#include "dma.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"
#include "t64_dev.h"

namespace ifd {

constexpr int kSkWaves = 4;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkDeqValu = 2 * (4 * 17 + 8);  // VALU of a wave's dequant per step: 2 bands x (4 words, the scales)
constexpr int kSkWBytes = 8 * kT64Codes + 8 * 128;  // weights of a stage: 8 code halves + 8 (s, b) rows
constexpr int kSkLds = 160 * 1024;  // LDS per CU
constexpr int kSkRow = 256 + 4;  // staged tile row stride (floats): rows h = 0, 1 of one store fall in other banks

// 32-row tiles run two blocks per CU (two waves per SIMD hide the latency of their short steps), larger tiles one.
// A stage holds one step's activation slab and weights; the ring is as deep as LDS allows, at most 8 stages.
__host__ __device__ constexpr int sk_bpc(int MT) { return MT == 1 ? 2 : 1; }
__host__ __device__ constexpr int sk_abytes(int MT) { return MT * 32 * 128; }
__host__ __device__ constexpr int sk_stage(int MT) { return sk_abytes(MT) + kSkWBytes; }
__host__ __device__ constexpr int sk_ring(int MT) {
  return (kSkLds / sk_bpc(MT) - 64) / sk_stage(MT) < 8 ? (kSkLds / sk_bpc(MT) - 64) / sk_stage(MT) : 8;
}
// the ring, and after the K loop the staged tile [32 MT][kSkRow] fp32 in the same memory
__host__ __device__ constexpr size_t sk_lds(int MT) {
  return (size_t)sk_ring(MT) * sk_stage(MT) > (size_t)MT * 32 * kSkRow * 4 ? (size_t)sk_ring(MT) * sk_stage(MT)
                                                                             : (size_t)MT * 32 * kSkRow * 4;
}

struct GemmSkArgs {
  const uint16_t* A;
  int lda;
  const uint8_t* wt;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;  // partial slots [2 nblk][8 bands][MT * 16 / 4][64] float4 (MFMA fragment order)
  uint32_t part_bytes;
  int tiles_m, tiles_n, G, nblk;
  int swi;  // SwiGLU mode: bands per half (N / 64); 0 otherwise
};

// the block whose run holds unit u
__host__ __device__ inline int sk_block_of(long u, int nblk, long U) { return (int)((u * nblk + nblk - 1) / U); }

template <int MT>
__global__ __launch_bounds__(kSkThreads, sk_bpc(MT)) void k_gemm_sk(GemmSkArgs p) {
  constexpr int BM = 32 * MT, R = sk_ring(MT), A_BYTES = sk_abytes(MT), STAGE = sk_stage(MT);
  constexpr int NE = MT * 16;  // accumulators per lane and band
  static_assert(R >= 4 && sk_lds(MT) + 64 <= kSkLds / sk_bpc(MT), "LDS plan");
  static_assert((R - 2) * (MT + 3) + 3 <= 63, "vmcnt range");
  extern __shared__ __align__(16) uint8_t lds[];
  float* const stg = (float*)lds;  // staged tile [BM][kSkRow], after the K loop
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, h = lane >> 5;

  const int b = xcd_remap(blockIdx.x, p.nblk);
  const int G = p.G;
  const long U = (long)p.tiles_m * p.tiles_n * G;
  const int u0 = (int)((long)b * U / p.nblk), u1 = (int)((long)(b + 1) * U / p.nblk), n = u1 - u0;
  const int nbands = t64_bands(p.N);
  const size_t gstride = (size_t)nbands * kT64Tile;

  auto phys_band = [&](int tn, int lb) __attribute__((always_inline)) {  // physical band of local band lb (0..7) of column tile tn
    const int bb = p.swi ? (lb < 4 ? 4 * tn + lb : p.swi + 4 * tn + lb - 4) : 8 * tn + lb;
    return min(bb, nbands - 1);
  };

  // ---- this wave's DMA stream. Stage s of the ring holds the activation slab of one step ([BM][64 bf16], 16-byte
  // columns XOR-swizzled by row pair) and its weights (8 code halves, then 8 (s, b) rows). Unit j's activations and
  // weights share stage j % R. At step i the wave issues the activations of step i + R - 1 (its MT DMAs of 8 rows)
  // and the weights of step i + R (the code halves of its two bands; wave 0 also the (s, b) rows of all 8), each
  // stream with its own (tile, group) position.
  const bool has_sb = wave == 0;
  const uint16_t* arow[MT];  // this lane's source row (and 16-byte column) of each activation DMA in the tile
  const uint8_t* wsrc[3];    // this lane's code sources (two bands) and (s, b) source
  auto a_tile_addr = [&](int tile) __attribute__((always_inline)) {
    const int tm = tile % p.tiles_m;
#pragma unroll
    for (int q = 0; q < MT; q++) {
      const int r = 8 * (MT * wave + q) + lane / 8;
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      arow[q] = p.A + (size_t)min(tm * BM + r, p.M - 1) * p.lda + 8 * c;
    }
  };
  auto w_tile_addr = [&](int tile) __attribute__((always_inline)) {
    const int tn = tile / p.tiles_m;
    wsrc[0] = p.wt + (size_t)phys_band(tn, 2 * wave) * kT64Tile + 16 * lane;
    wsrc[1] = p.wt + (size_t)phys_band(tn, 2 * wave + 1) * kT64Tile + 16 * lane;
    wsrc[2] = p.wt + (size_t)phys_band(tn, lane / 8) * kT64Tile + kT64Codes + 16 * (lane & 7);
  };
  int a_tile = u0 / G, a_g = u0 % G, a_i = 0, a_st = 0;
  int w_tile = a_tile, w_g = a_g, w_i = 0, w_st = 0;
  a_tile_addr(a_tile);
  w_tile_addr(w_tile);
  auto issue_a = [&]() __attribute__((always_inline)) {
    uint8_t* st = lds + a_st * STAGE;
#pragma unroll
    for (int q = 0; q < MT; q++) dma16(arow[q] + (size_t)a_g * kGroup, st + (MT * wave + q) * 1024);
    a_st = a_st + 1 == R ? 0 : a_st + 1;
    a_i++;
    if (++a_g == G) {
      a_g = 0;
      if (a_i < n) a_tile_addr(++a_tile);
    }
  };
  auto issue_w = [&]() __attribute__((always_inline)) {
    uint8_t* st = lds + w_st * STAGE + A_BYTES;
    const size_t off = (size_t)w_g * gstride;
    dma16(wsrc[0] + off, st + (2 * wave) * kT64Codes);
    dma16(wsrc[1] + off, st + (2 * wave + 1) * kT64Codes);
    if (has_sb) dma16(wsrc[2] + off, st + 8 * kT64Codes);
    w_st = w_st + 1 == R ? 0 : w_st + 1;
    w_i++;
    if (++w_g == G) {
      w_g = 0;
      if (w_i < n) w_tile_addr(++w_tile);
    }
  };

  // this wave's two bands of the weights in stage s, dequantized
  auto dequant = [&](int s, u32x4 (&bf)[2][4]) __attribute__((always_inline)) {
    const uint8_t* wst = lds + s * STAGE + A_BYTES;
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const int band = 2 * wave + nb;
      const u32x4 codes = *(const u32x4*)(wst + band * kT64Codes + 16 * lane);
      const uint32_t sb = *(const uint32_t*)(wst + 8 * kT64Codes + band * 128 + 4 * j);
      const float sc = bf2f((uint16_t)(sb & 0xFFFFu)), bi = bf2f((uint16_t)(sb >> 16));
      const float sa = t64_sa(sc), sbs = t64_sb(sc);
#pragma unroll
      for (int t = 0; t < 4; t++) bf[nb][t] = t64_dequant(codes[t], sa, sbs, bi);
    }
  };
  // activation fragments of M tile a: MFMA step t takes k = 32 h + 8 t .. + 7 (logical column 4 h + t)
  auto load_a = [&](const uint8_t* st, int a, u32x4 (&af)[4]) __attribute__((always_inline)) {
    const int r = a * 32 + j;
#pragma unroll
    for (int t = 0; t < 4; t++) af[t] = *(const u32x4*)(st + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
  };

  f32x16 acc[2][MT];
#pragma unroll
  for (int nb = 0; nb < 2; nb++)
#pragma unroll
    for (int a = 0; a < MT; a++) acc[nb][a] = zero16();

  // Waits. At step i the wave needs A(i) and W(i + 1), both issued at step i - R + 1 (the prologue for the first
  // steps), W(i + 1) after A(i): it waits until at most the DMAs issued after W(i + 1) are outstanding (every
  // operation of a wave completes in issue order; younger output stores only lengthen the wait). In the last R
  // steps of the run fewer are in flight: wait for all.
  constexpr int nwa = 3, nwo = 2;  // weight DMAs per step of wave 0 / of the others
  auto wait_step = [&](int i) __attribute__((always_inline)) {
    if (i + R > n) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (i < R - 2) {  // the prologue's lone W(R - 1) sits between
      if (has_sb) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((R - 3) * (MT + nwa) + nwa) : "memory");
      else asm volatile("s_waitcnt vmcnt(%0)" ::"n"((R - 3) * (MT + nwo) + nwo) : "memory");
    } else {
      if (has_sb) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((R - 2) * (MT + nwa)) : "memory");
      else asm volatile("s_waitcnt vmcnt(%0)" ::"n"((R - 2) * (MT + nwo)) : "memory");
    }
  };
  // prologue: A(0..R-2) and W(0..R-1) (those of the run), then W(0) for the first dequant
  for (int jj = 0; jj < R - 1; jj++) {
    if (a_i < n) issue_a();
    if (w_i < n) issue_w();
  }
  if (w_i < n) issue_w();
  if (n < R) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    if (has_sb) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((R - 2) * (MT + nwa) + nwa) : "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" ::"n"((R - 2) * (MT + nwo) + nwo) : "memory");
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  u32x4 bf0[2][4], bf1[2][4];
  dequant(0, bf0);
  int ca = 0, cw = 1 % R;  // stage of step i (activations) and of step i + 1 (weights to dequantize)

  // step i with the B fragments of step i in bc; dequantizes step i + 1 into bn
  auto step = [&](int i, u32x4 (&bc)[2][4], u32x4 (&bn)[2][4]) __attribute__((always_inline)) {
    wait_step(i);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (a_i < n) issue_a();
    if (w_i < n) issue_w();
    // One basic block: the step's activation fragments and the next step's codes from LDS, then the MFMAs with the
    // next step's dequant between them, so that the VALU work and the LDS latency overlap the matrix core. Past the
    // run's end the dequant reads a stale stage, never used.
    const uint8_t* ast = lds + ca * STAGE;
    u32x4 af[MT][4];
#pragma unroll
    for (int a = 0; a < MT; a++) load_a(ast, a, af[a]);
    dequant(cw, bn);
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
      for (int nb = 0; nb < 2; nb++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[nb][a] = mfma_bf16(af[a][t], bc[nb][t], acc[nb][a]);
    __builtin_amdgcn_sched_group_barrier(0x100, 4 * MT + 4, 0);  // the LDS reads
#pragma unroll
    for (int k = 0; k < 8 * MT; k++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                    // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, (kSkDeqValu + 8 * MT - 1) / (8 * MT), 0);  // VALU between
    }
    // the next step's fragments are complete in this step (else the compiler may sink the dequant past the next
    // barrier, next to its use)
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int t = 0; t < 4; t++) asm volatile("" : "+v"(bn[nb][t]));
    ca = ca + 1 == R ? 0 : ca + 1;
    cw = cw + 1 == R ? 0 : cw + 1;
  };
  // steps [lo, hi) with the current fragments in bf0 on entry and on exit
  auto run = [&](int lo, int hi) __attribute__((always_inline)) {
    int i = lo;
    for (; i + 1 < hi; i += 2) {
      step(i, bf0, bf1);
      step(i + 1, bf1, bf0);
    }
    if (i < hi) {
      step(i, bf0, bf1);
#pragma unroll
      for (int nb = 0; nb < 2; nb++)
#pragma unroll
        for (int t = 0; t < 4; t++) bf0[nb][t] = bf1[nb][t];
    }
  };

  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.part, 0, (int)p.part_bytes, 0x00020000);
  const size_t slot_floats = (size_t)8 * NE * 64;
  // byte offset of this lane's float4 (band, M tile a, rows 4q..4q+3) in a slot
  auto slot_off = [&](int slot, int band, int a, int q) __attribute__((always_inline)) {
    return (int)((((size_t)slot * slot_floats + (size_t)band * NE * 64) + ((size_t)(a * 4 + q) * 64 + lane) * 4) * 4);
  };
  auto write_slot = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int a = 0; a < MT; a++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const u32x4 x = {__float_as_uint(acc[nb][a][4 * q]), __float_as_uint(acc[nb][a][4 * q + 1]),
                           __float_as_uint(acc[nb][a][4 * q + 2]), __float_as_uint(acc[nb][a][4 * q + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(x, rs, slot_off(slot, 2 * wave + nb, a, q), 0, 0);
        }
  };

  const int tile_first = u0 / G, tile_last = (u1 - 1) / G;
  const bool two = tile_last != tile_first;
  const int n1 = min(n, (tile_first + 1) * G - u0);
  run(0, n1);
  if (two) {
    write_slot(2 * b);  // the first tile's piece, while the run goes on
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int a = 0; a < MT; a++) acc[nb][a] = zero16();
    run(n1, n);
  }
  // every DMA and partial store has landed; LDS is free once all waves are past their reads
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // a whole tile's acc, staged through LDS and stored as rows (SwiGLU: h)
  auto store_tile = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int a = 0; a < MT; a++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          stg[(a * 32 + 8 * (r / 4) + 4 * h + (r % 4)) * kSkRow + 32 * (2 * wave + nb) + j] = acc[nb][a][r];
    __syncthreads();
    const int tm = t % p.tiles_m, tn = t / p.tiles_m;
    if (p.swi) {
      uint16_t* C = (uint16_t*)p.C;
      for (int e = tid; e < BM * 32; e += kSkThreads) {
        const int row = e >> 5, c4 = (e & 31) * 4, grow = tm * BM + row;
        if (grow >= p.M) continue;
        const float4 g = *(const float4*)(stg + row * kSkRow + c4);
        const float4 u = *(const float4*)(stg + row * kSkRow + 128 + c4);
        const uint32_t lo =
            pack_bf2(swiglu_f(bf2f(f2bf(g.x)), bf2f(f2bf(u.x))), swiglu_f(bf2f(f2bf(g.y)), bf2f(f2bf(u.y))));
        const uint32_t hi =
            pack_bf2(swiglu_f(bf2f(f2bf(g.z)), bf2f(f2bf(u.z))), swiglu_f(bf2f(f2bf(g.w)), bf2f(f2bf(u.w))));
        *(u32x2*)(C + (size_t)grow * p.ldc + tn * 128 + c4) = u32x2{lo, hi};
      }
    } else {
      for (int e = tid; e < BM * 64; e += kSkThreads) {
        const int row = e >> 6, c4 = (e & 63) * 4, grow = tm * BM + row, gcol = tn * 256 + c4;
        if (grow >= p.M || gcol >= p.N) continue;
        const float* sv = stg + row * kSkRow + c4;
        const size_t o = (size_t)grow * p.ldc + gcol;
        if (gcol + 4 <= p.N && (o & 3) == 0 && p.mode != 1) {
          if (p.mode == 2) *(float4*)((float*)p.C + o) = *(const float4*)sv;
          else *(u32x2*)((uint16_t*)p.C + o) = u32x2{pack_bf2(sv[0], sv[1]), pack_bf2(sv[2], sv[3])};
        } else {
          for (int k = 0; k < 4 && gcol + k < p.N; k++) store_mode(p.C, o + k, sv[k], p.mode);
        }
      }
    }
  };

  // ---- epilogue: the last segment, stored when it is a whole tile, else a piece of a cut tile
  const int tlo = tile_last * G;
  const bool whole = u0 <= tlo && u1 >= tlo + G;
  if (whole) {
    store_tile(tile_last);
    return;
  }
  write_slot(2 * b + (two ? 1 : 0));  // a piece of a cut tile: k_sk_fixup sums the pieces
}

// Sum of a cut tile's pieces (partial slots, in unit order) and its store. Block (tile, w, f): one wave over the
// float4 fragment f = (a, q) of column band w of the tile (SwiGLU: gate band w with up band w + 4, giving h), the
// loads of up to kFixBatch pieces in flight at once; whole tiles were stored by k_gemm_sk.
constexpr int kFixBatch = 8;
template <int MT>
__global__ __launch_bounds__(64) void k_sk_fixup(GemmSkArgs p) {
  constexpr int BM = 32 * MT, NE = MT * 16;
  const int tile = blockIdx.x, w = blockIdx.y, a = blockIdx.z / 4, q = blockIdx.z % 4;
  const int lane = threadIdx.x, j = lane & 31, h = lane >> 5;
  const int G = p.G;
  const long U = (long)p.tiles_m * p.tiles_n * G;
  const long tlo = (long)tile * G;
  const int bf = sk_block_of(tlo, p.nblk, U), bl = sk_block_of(tlo + G - 1, p.nblk, U);
  if (bf == bl) return;
  const float4* part = (const float4*)p.part;
  auto sum = [&](int wv) __attribute__((always_inline)) {
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int b0 = bf; b0 <= bl; b0 += kFixBatch) {
      float4 x[kFixBatch];
#pragma unroll
      for (int k = 0; k < kFixBatch; k++) {
        const int bb = b0 + k;
        if (bb <= bl) {
          const int slot = 2 * bb + ((long)bb * U / p.nblk < tlo ? 1 : 0);
          x[k] = part[(((size_t)slot * 8 + wv) * NE / 4 + a * 4 + q) * 64 + lane];
        }
      }
#pragma unroll
      for (int k = 0; k < kFixBatch; k++)
        if (b0 + k <= bl) t.x += x[k].x, t.y += x[k].y, t.z += x[k].z, t.w += x[k].w;
    }
    return t;
  };
  const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
  const float4 v = sum(w);
  const float vv[4] = {v.x, v.y, v.z, v.w};
  const int row0 = tm * BM + a * 32 + 8 * q + 4 * h;
  if (p.swi) {
    const float4 u4 = sum(w + 4);
    const float uu[4] = {u4.x, u4.y, u4.z, u4.w};
    const int col = (4 * tn + w) * 32 + j;
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (row0 + e < p.M)
        ((uint16_t*)p.C)[(size_t)(row0 + e) * p.ldc + col] = f2bf(swiglu_f(bf2f(f2bf(vv[e])), bf2f(f2bf(uu[e]))));
  } else {
    const int col = (8 * tn + w) * 32 + j;
    if (col >= p.N) return;
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (row0 + e < p.M) store_mode(p.C, (size_t)(row0 + e) * p.ldc + col, vv[e], p.mode);
  }
}

// ---- host side

static int cu_count() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  }
  return n;
}

struct SkPlan {
  int MT, tiles_m, tiles_n, G, nblk;
};
static SkPlan gemm_sk_plan(int M, int N, int K) {
  SkPlan pl{};
  pl.MT = M <= 32 ? 1 : M <= 64 ? 2 : 4;
  const int bpc = pl.MT == 1 ? 2 : 1;  // sk_bpc
  pl.tiles_m = (M + 32 * pl.MT - 1) / (32 * pl.MT);
  pl.tiles_n = (t64_bands(N) + 7) / 8;
  pl.G = K / kGroup;
  const long tiles = (long)pl.tiles_m * pl.tiles_n, U = tiles * pl.G;
  // the resident blocks, but never more than one tile of groups per block (at most two segments) nor fewer than one
  // unit
  pl.nblk = (int)std::min<long>(std::max<long>((long)cu_count() * bpc, tiles), U);
  return pl;
}

// Shapes with tiles for at least a third of the CUs: there each tile is cut into a few pieces. With fewer tiles (long
// K, narrow N) every tile is cut into many, and the aligned K split (gemm_t64.hip) moves fewer partial bytes; it is
// still the faster kernel at 32-row tiles and with two or more 128-row M tiles over a long K (measured: N = 5120,
// K = 17408, M = 32: 25.9 against 29.5 us; M = 256: 70.8 against 75.4 us). With one 128-row tile (64 < M <= 128)
// stream-K is faster on every narrow shape measured (K = 17408: 45.9 against 47.6 us; N = K = 5120: 26.0 against
// 31.2 us; N = 2048, K = 8192: 23.5 against 31.0 us), and both kernels compute bf16(s*q + b) there.
bool gemm_sk_applies(int M, int N, int K, int mode) {
  if (M <= 16 || K % kGroup) return false;
  if (mode == kModeSwiglu && N % 256) return false;
  const SkPlan pl = gemm_sk_plan(M, N, K);
  return (long)pl.tiles_m * pl.tiles_n * 3 >= cu_count() || (M > 64 && M <= 128);
}

size_t gemm_sk_workspace(int M, int N, int K, int mode) {
  (void)mode;
  const SkPlan pl = gemm_sk_plan(M, N, K);
  return (size_t)2 * pl.nblk * 8 * (16 * pl.MT) * 64 * sizeof(float);
}

template <int MT>
static int launch_sk_cfg(const GemmSkArgs& a, hipStream_t st) {
  constexpr size_t lds = sk_lds(MT);
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)k_gemm_sk<MT>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr = true;
  }
  hipLaunchKernelGGL(k_gemm_sk<MT>, dim3(a.nblk), dim3(kSkThreads), lds, st, a);
  IFD_TRY(check_launch("gemm_sk"));
  hipLaunchKernelGGL(k_sk_fixup<MT>, dim3(a.tiles_m * a.tiles_n, a.swi ? 4 : 8, MT * 4), dim3(64), 0, st, a);
  return check_launch("gemm_sk fixup");
}

int launch_gemm_sk(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                   void* ws, size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (!gemm_sk_applies(M, N, K, mode)) return fail(IFD_ERR_UNSUPPORTED, "gemm_sk: shape M=%d N=%d K=%d", M, N, K);
  const SkPlan pl = gemm_sk_plan(M, N, K);
  const size_t need = gemm_sk_workspace(M, N, K, mode);
  if (need > ws_bytes || !ws)
    return fail(IFD_ERR_WORKSPACE, "gemm_sk needs %zu bytes of workspace, got %zu", need, ws_bytes);
  if (need >= (size_t)1 << 31) return fail(IFD_ERR_UNSUPPORTED, "gemm_sk: partials past 2 GiB");
  GemmSkArgs a{A, lda, (const uint8_t*)wt, N, K, C, ldc, M, mode, (float*)ws, (uint32_t)need,
               pl.tiles_m, pl.tiles_n, pl.G, pl.nblk, mode == kModeSwiglu ? N / 64 : 0};
  if (pl.MT == 1) return launch_sk_cfg<1>(a, st);
  if (pl.MT == 2) return launch_sk_cfg<2>(a, st);
  return launch_sk_cfg<4>(a, st);
}

}  // namespace ifd
