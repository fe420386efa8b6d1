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
// Block: 8 waves; wave w owns band w of the tile over all MT M tiles (one dequantized B fragment feeds MT MFMAs).
// Two LDS rings filled by direct global -> LDS DMA: NA activation slabs [BM][64 bf16] (16-byte columns XOR-swizzled
// by row pair) and NW weight stages (8 code halves + 8 (s, b) rows). Waves 0-3 issue the activation DMAs, waves 4-7
// the weight DMAs, each with its own in-order vmcnt stream; the stream positions advance incrementally (no per-step
// division). The dequant of step i + 1 is issued alongside the MFMAs of step i. Every DMA is issued by a whole wave
// under wave-uniform control flow (the LDS base goes to M0). Finished tiles are staged through LDS and leave as
// whole rows.
//
// SwiGLU mode: tile t holds gate bands 4t..4t+3 (waves 0-3) and the matching up bands (waves 4-7); the staged tile
// (or the fixup) gives h = silu(bf16(gate)) * bf16(up) (reference silu_mul, core.metal:777-787).
#include <algorithm>

#include "common.h"
#include "dma.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"
#include "t64_dev.h"

namespace ifd {

constexpr int kSkThreads = 512;
constexpr int kSkWBytes = 8 * kT64Codes + 8 * 128;  // weight stage: 8 code halves + 8 (s, b) rows
constexpr int kSkLds = 160 * 1024;  // LDS per CU
constexpr int kSkRow = 256 + 4;  // staged tile row stride (floats): rows h = 0, 1 of one store fall in other banks

// 32-row tiles run two blocks per CU (four waves per SIMD hide the latency of their short steps); a ring of four or
// more stages keeps the weight stream at full rate. 128-row tiles favour a deeper activation ring (16 KB slabs) over a
// deeper weight ring (measured).
__host__ __device__ constexpr int sk_bpc(int MT) { return MT == 1 ? 2 : 1; }
__host__ __device__ constexpr int sk_abytes(int MT) { return MT * 32 * 128; }
__host__ __device__ constexpr int sk_na(int MT) { return MT == 1 ? 4 : MT == 2 ? 5 : 6; }
__host__ __device__ constexpr int sk_nw(int MT) {
  return MT == 4 ? 5
         : (kSkLds / sk_bpc(MT) - 64 - sk_na(MT) * sk_abytes(MT)) / kSkWBytes < 15
             ? (kSkLds / sk_bpc(MT) - 64 - sk_na(MT) * sk_abytes(MT)) / kSkWBytes
             : 15;
}
__host__ __device__ constexpr size_t sk_rings(int MT) {
  return (size_t)sk_na(MT) * sk_abytes(MT) + (size_t)sk_nw(MT) * kSkWBytes;
}
// the rings, and after the K loop the staged tile [32 MT][kSkRow] fp32 in the same memory
__host__ __device__ constexpr size_t sk_lds(int MT) {
  return sk_rings(MT) > (size_t)MT * 32 * kSkRow * 4 ? sk_rings(MT) : (size_t)MT * 32 * kSkRow * 4;
}

struct GemmSkArgs {
  const uint16_t* A;
  int lda;
  const uint8_t* wt;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;  // partial slots [2 nblk][8 waves][MT * 16 / 4][64] float4 (MFMA fragment order)
  uint32_t part_bytes;
  int tiles_m, tiles_n, G, nblk;
  int swi;  // SwiGLU mode: bands per half (N / 64); 0 otherwise
};

// the block whose run holds unit u
__host__ __device__ inline int sk_block_of(long u, int nblk, long U) { return (int)((u * nblk + nblk - 1) / U); }

template <int MT>
__global__ __launch_bounds__(kSkThreads, sk_bpc(MT)) void k_gemm_sk(GemmSkArgs p) {
  constexpr int BM = 32 * MT, NA = sk_na(MT), NW = sk_nw(MT), A_BYTES = sk_abytes(MT);
  constexpr int NE = MT * 16;  // accumulators per lane
  static_assert(NA >= 3 && NW >= 4 && sk_lds(MT) + 64 <= kSkLds / sk_bpc(MT), "LDS plan");
  static_assert(3 * (NW - 2) <= 63 && MT * (NA - 2) <= 63, "vmcnt range");
  extern __shared__ __align__(16) uint8_t lds[];
  uint8_t* const aring = lds;
  uint8_t* const wring = lds + NA * A_BYTES;
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

  // ---- DMA streams: waves 0-3 the activations, waves 4-7 the weights; (tile, group) of the next step to issue
  int s_tile = u0 / G, s_g = u0 % G, s_i = 0, s_st = 0;
  const uint16_t* arow[MT];  // waves 0-3: this lane's source row (and 16-byte column) of each DMA in the tile
  const uint8_t* wsrc[3];    // waves 4-7: this lane's code sources (two bands) and (s, b) source (wave 7)
  auto stream_tile = [&](int tile) __attribute__((always_inline)) {
    const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
    if (wave < 4) {
#pragma unroll
      for (int q = 0; q < MT; q++) {
        const int r = 8 * (MT * wave + q) + lane / 8;
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        arow[q] = p.A + (size_t)min(tm * BM + r, p.M - 1) * p.lda + 8 * c;
      }
    } else {
      const int ww = wave - 4;
      wsrc[0] = p.wt + (size_t)phys_band(tn, 2 * ww) * kT64Tile + 16 * lane;
      wsrc[1] = p.wt + (size_t)phys_band(tn, 2 * ww + 1) * kT64Tile + 16 * lane;
      wsrc[2] = p.wt + (size_t)phys_band(tn, lane / 8) * kT64Tile + kT64Codes + 16 * (lane & 7);
    }
  };
  stream_tile(s_tile);
  auto issue = [&]() __attribute__((always_inline)) {
    if (wave < 4) {
      uint8_t* st = aring + s_st * A_BYTES;
#pragma unroll
      for (int q = 0; q < MT; q++) dma16(arow[q] + (size_t)s_g * kGroup, st + (MT * wave + q) * 1024);
      s_st = s_st + 1 == NA ? 0 : s_st + 1;
    } else {
      uint8_t* st = wring + s_st * kSkWBytes;
      const size_t off = (size_t)s_g * gstride;
      const int ww = wave - 4;
      dma16(wsrc[0] + off, st + (2 * ww) * kT64Codes);
      dma16(wsrc[1] + off, st + (2 * ww + 1) * kT64Codes);
      if (wave == 7) dma16(wsrc[2] + off, st + 8 * kT64Codes);
      s_st = s_st + 1 == NW ? 0 : s_st + 1;
    }
    s_i++;
    if (++s_g == G) {
      s_g = 0;
      stream_tile(++s_tile);
    }
  };

  // this wave's band from weight stage ws, dequantized
  auto dequant = [&](int ws, u32x4 (&bf)[4]) __attribute__((always_inline)) {
    const uint8_t* wst = wring + ws * kSkWBytes;
    const u32x4 codes = *(const u32x4*)(wst + wave * kT64Codes + 16 * lane);
    const uint32_t sb = *(const uint32_t*)(wst + 8 * kT64Codes + wave * 128 + 4 * j);
    const float sc = bf2f((uint16_t)(sb & 0xFFFFu)), bi = bf2f((uint16_t)(sb >> 16)), sa = t64_sa(sc), sbs = t64_sb(sc);
#pragma unroll
    for (int t = 0; t < 4; t++) bf[t] = t64_dequant(codes[t], sa, sbs, bi);
  };
  // activation fragments of M tile a: MFMA step t takes k = 32 h + 8 t .. + 7 (logical column 4 h + t)
  auto load_a = [&](const uint8_t* st, int a, u32x4 (&af)[4]) __attribute__((always_inline)) {
    const int r = a * 32 + j;
#pragma unroll
    for (int t = 0; t < 4; t++) af[t] = *(const u32x4*)(st + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
  };

  f32x16 acc[MT], acc0[MT];  // acc0: the first segment, once the run crosses into a second tile
#pragma unroll
  for (int a = 0; a < MT; a++) acc[a] = zero16(), acc0[a] = zero16();

  // Pipeline. Waves 0-3 have issued A(0 .. i + NA - 2) at the top of step i and need A(i); waves 4-7 have issued
  // W(0 .. i + NW - 2) and need W(i + 1) (dequantized during step i). DMAs complete in order per wave: waiting until
  // at most the younger DMAs of this wave's own stream are outstanding leaves exactly those in flight (other
  // outstanding operations, such as partial stores, only lengthen the wait). The stage a DMA overwrites held a step
  // every wave finished before the barrier.
  const int nwv = wave == 7 ? 3 : 2;  // weight DMAs per step of this wave
  {
    const int pre = min(wave < 4 ? NA - 1 : NW - 1, n);
    for (int i = 0; i < pre; i++) issue();
  }
  if (wave >= 4) {  // W(0) for the first dequant
    const int y = min(NW - 2, n - 1);
    if (nwv == 3) wait_vm_dyn<3, NW - 2>(y);
    else wait_vm_dyn<2, NW - 2>(y);
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  u32x4 bf0[4], bf1[4];
  dequant(0, bf0);
  int ca = 0, cw = 1 % NW;  // A stage of step i, weight stage of step i + 1

  // step i with the B fragments of step i in bc; dequantizes step i + 1 into bn
  auto step = [&](int i, u32x4 (&bc)[4], u32x4 (&bn)[4]) __attribute__((always_inline)) {
    if (wave < 4) {
      wait_vm_dyn<MT, NA - 2>(min(NA - 2, n - 1 - i));
    } else if (i + 1 < n) {
      const int y = min(NW - 3, n - 2 - i);
      if (nwv == 3) wait_vm_dyn<3, NW - 3>(y);
      else wait_vm_dyn<2, NW - 3>(y);
    }
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
      for (int t = 0; t < 4; t++) acc[a] = mfma_bf16(af[a & 1][t], bc[t], acc[a]);
    }
    ca = ca + 1 == NA ? 0 : ca + 1;
    cw = cw + 1 == NW ? 0 : cw + 1;
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
      for (int t = 0; t < 4; t++) bf0[t] = bf1[t];
    }
  };

  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.part, 0, (int)p.part_bytes, 0x00020000);
  const size_t slot_floats = (size_t)8 * NE * 64;
  auto slot_off = [&](int slot, int a, int q) __attribute__((always_inline)) {  // byte offset of this lane's float4 (a, rows 4q..4q+3) in a slot
    return (int)((((size_t)slot * slot_floats + (size_t)wave * NE * 64) + ((size_t)(a * 4 + q) * 64 + lane) * 4) * 4);
  };
  auto write_slot = [&](int slot, f32x16 (&v)[MT]) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const u32x4 x = {__float_as_uint(v[a][4 * q]), __float_as_uint(v[a][4 * q + 1]),
                         __float_as_uint(v[a][4 * q + 2]), __float_as_uint(v[a][4 * q + 3])};
        __builtin_amdgcn_raw_buffer_store_b128(x, rs, slot_off(slot, a, q), 0, 0);
      }
  };

  const int tile_first = u0 / G, tile_last = (u1 - 1) / G;
  const bool two = tile_last != tile_first;
  const int n1 = min(n, (tile_first + 1) * G - u0);
  run(0, n1);
  if (two) {
#pragma unroll
    for (int a = 0; a < MT; a++) acc0[a] = acc[a], acc[a] = zero16();
    write_slot(2 * b, acc0);  // the first tile's piece, while the run goes on
    run(n1, n);
  }
  // every DMA and partial store has landed; LDS is free once all waves are past their reads
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // ---- epilogue: the last segment, stored when it is a whole tile, else a piece in slot 2 b + (two ? 1 : 0)
  const int tlo = tile_last * G;
  if (u0 > tlo || u1 < tlo + G) {
    write_slot(2 * b + (two ? 1 : 0), acc);
    return;
  }
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int r = 0; r < 16; r++) stg[(a * 32 + 8 * (r / 4) + 4 * h + (r % 4)) * kSkRow + 32 * wave + j] = acc[a][r];
  __syncthreads();
  const int tm = tile_last % p.tiles_m, tn = tile_last / p.tiles_m;
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
    return;
  }
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
