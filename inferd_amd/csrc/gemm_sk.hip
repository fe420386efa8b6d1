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
// (the activation rows 8 (MT w + q) .. + 7, its two bands' codes and their two (s, b) rows) as one in-order vmcnt
// stream, R units ahead; the stream positions advance by scalar adds, with a branch only at a tile boundary or the
// run's end. All waves run the same code. The step loop is unrolled over the ring, so stages, LDS addresses and
// fragment registers are compile-time constants and a step issues little beyond its MFMAs, dequant, LDS reads and
// DMAs (one wave per SIMD issues about one instruction every 4 cycles, so the count sets the step time). Every DMA
// is issued by a whole wave under wave-uniform control flow (the LDS base goes to M0). Finished tiles are staged
// through LDS and leave as whole rows.
//
// SwiGLU mode: tile t holds gate bands 4t..4t+3 (waves 0, 1) and the matching up bands (waves 2, 3); the staged tile
// (or the fixup) gives h = silu(bf16(gate)) * bf16(up) (reference silu_mul, core.metal:777-787).
//
// The same kernel serves T64x8 (8-bit) weights with BITS = 8: a band's codes are two 1 KB halves per group (two DMAs
// instead of one), dequantized from the stored q - 128 bytes to bf16(s q + b), MLX's 8-bit qmm rounding.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "dma.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"
#include "t64_dev.h"

namespace ifd {

constexpr int kSkWaves = 4;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkLds = 160 * 1024;  // LDS per CU
constexpr int kSkRow = 256 + 4;  // staged tile row stride (floats): rows h = 0, 1 of one store fall in other banks

// BITS = 4: T64 weights; BITS = 8: T64x8 weights (t64.h), whose code tiles are twice as large (two 1 KB halves per
// band and group, each one DMA) and are dequantized from the stored q - 128 bytes.
__host__ __device__ constexpr int sk_codes(int BITS) { return BITS == 8 ? kT64x8Codes : kT64Codes; }
__host__ __device__ constexpr int sk_tileb(int BITS) { return BITS == 8 ? kT64x8Tile : kT64Tile; }
// weights of a stage: 8 bands' codes + 8 (s, b) rows
__host__ __device__ constexpr int sk_wbytes(int BITS) { return 8 * sk_codes(BITS) + 8 * 128; }

// 4-bit 32-row tiles run two blocks per CU (two waves per SIMD hide the latency of their short steps), other tiles
// one (an 8-bit stage is too large for two rings of four). A stage holds one step's activation slab and weights; the
// ring is as deep as LDS allows, at most 8 stages.
__host__ __device__ constexpr int sk_bpc(int MT, int BITS) { return MT == 1 && BITS == 4 ? 2 : 1; }
__host__ __device__ constexpr int sk_abytes(int MT) { return MT * 32 * 128; }
__host__ __device__ constexpr int sk_stage(int MT, int BITS) { return sk_abytes(MT) + sk_wbytes(BITS); }
__host__ __device__ constexpr int sk_ring(int MT, int BITS) {
  return (kSkLds / sk_bpc(MT, BITS) - 64) / sk_stage(MT, BITS) < 8 ? (kSkLds / sk_bpc(MT, BITS) - 64) / sk_stage(MT, BITS)
                                                                   : 8;
}
// the ring, and after the K loop the staged tile [32 MT][kSkRow] fp32 in the same memory
__host__ __device__ constexpr size_t sk_lds(int MT, int BITS) {
  return (size_t)sk_ring(MT, BITS) * sk_stage(MT, BITS) > (size_t)MT * 32 * kSkRow * 4
             ? (size_t)sk_ring(MT, BITS) * sk_stage(MT, BITS)
             : (size_t)MT * 32 * kSkRow * 4;
}

struct GemmSkArgs {
  const uint16_t* A;
  int lda;
  const uint8_t* wt;
  uint32_t w_bytes;  // bytes of the T64 weights (buffer bound)
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;  // partial slots [2 nblk][8 bands][MT * 16 / 4][64] float4 (MFMA fragment order)
  uint32_t part_bytes;
  int tiles_m, tiles_n, G, nblk;
  int swi;  // SwiGLU mode: bands per half (N / 64); 0 otherwise
  // k_sk_fixup only: the stream-K tiles are tiles tile0 .. tile0 + ntiles - 1 of the tile order, and each output row
  // is scaled by rs[row * rs_stride] before its store (rs null: no scale)
  int tile0, ntiles;
  const float* rs;
  int rs_stride;
  int sparse;  // more blocks than units: some runs are empty
};

// the block whose run holds unit u
__host__ __device__ inline int sk_block_of(long u, int nblk, long U) { return (int)((u * nblk + nblk - 1) / U); }

// Wave-wide DMAs through a buffer resource: lane l's 16 (4) bytes at voff(l) + soff land at lds + 16 l (4 l) (LDS
// base in M0, wave-uniform control flow only).
__device__ __forceinline__ void sk_dma(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, (int)voff, (int)soff, 0, 0);
}
__device__ __forceinline__ void sk_dma4(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 4, (int)voff, (int)soff, 0, 0);
}

template <int K>
using sk_ic = std::integral_constant<int, K>;
// f(sk_ic<K>{}) for K = 0 .. N - 1, unrolled at compile time
template <int K, int N, class F>
__device__ __forceinline__ void sk_static_for(F&& f) {
  if constexpr (K < N) {
    f(sk_ic<K>{});
    sk_static_for<K + 1, N>(f);
  }
}

// The pipeline of one wave. A wave issues a step's data as one pair of DMAs per unit: A(j), its 8 MT activation rows
// (8 (MT w + q) .. + 7, q < MT), and W(j), the codes of its two bands and their two (s, b) rows (one 4-byte-per-lane
// DMA). Pair j lands in stage j % R. The prologue issues pairs 0 .. R - 1 and step i pair i + R, past the run's end
// too (re-reading its last unit, L2 hits), so the waits are constants: at step i the wave reads A(i + 1)'s fragments
// and W(i + 2)'s codes, so it waits for pair i + 2, behind which R - 3 younger pairs are in flight. Step i refills
// stage i % R, whose A(i) was last read at step i - 1 and W(i) at step i - 2, both before the barrier that opens step
// i. The loop is unrolled over the ring (twice for an odd depth), so that every stage, LDS address and fragment
// register set is a compile-time constant; a run enters it at its phase (Duff's device). A step issues about 220
// instructions for its 8 MT MFMAs, which a single wave per SIMD issues one every ~4 cycles: the stream's bookkeeping
// is a few scalar adds and one countdown per step.
template <int MT, int BITS>
__device__ __forceinline__ void sk_body(const GemmSkArgs& p, uint8_t* lds, const int wave, const int b) {
  constexpr int BM = 32 * MT, R = sk_ring(MT, BITS), A_BYTES = sk_abytes(MT), STAGE = sk_stage(MT, BITS);
  constexpr int CODES = sk_codes(BITS), TILEB = sk_tileb(BITS);
  constexpr int NE = MT * 16;             // accumulators per lane and band
  constexpr int NH = BITS / 4;            // 1 KB code DMAs per band
  constexpr int NWC = 2 * NH;             // code DMAs per pair (two bands)
  constexpr int PAIR = MT + NWC + 1;      // DMAs per pair: activation rows, codes, the (s, b) rows
  constexpr int UNR = R % 2 ? 2 * R : R;  // steps per unrolled body
  static_assert(R >= 4 && (R - 2) * PAIR <= 63 && UNR <= 16, "ring depth, vmcnt range, unroll");
  float* const stg = (float*)lds;  // staged tile [BM][kSkRow], after the K loop
  const int tid = threadIdx.x, lane = tid & 63;
  const int j = lane & 31, h = lane >> 5;

  const int G = p.G;
  const long U = (long)p.tiles_m * p.tiles_n * G;
  const int u0 = (int)((long)b * U / p.nblk), u1 = (int)((long)(b + 1) * U / p.nblk), n = u1 - u0;
  const int nbands = t64_bands(p.N);
  const uint32_t gstride = (uint32_t)nbands * TILEB;
  const int tile_first = u0 / G, tile_last = (u1 - 1) / G;

  auto phys_band = [&](int tn, int lb) __attribute__((always_inline)) {  // physical band of local band lb (0..7)
    const int bb = p.swi ? (lb < 4 ? 4 * tn + lb : p.swi + 4 * tn + lb - 4) : 8 * tn + lb;
    return min(bb, nbands - 1);
  };
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.A, 0, (int)((uint32_t)p.M * p.lda * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)p.wt, 0, (int)p.w_bytes, 0x00020000);

  // ---- the DMA stream: per-lane offsets of the current tile, the unit's group offsets in scalar registers
  uint32_t va[MT], vw[NWC], vs;
  auto set_tile = [&](int tile) __attribute__((always_inline)) {
    const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
#pragma unroll
    for (int q = 0; q < MT; q++) {
      const int r = 8 * (MT * wave + q) + lane / 8;
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      va[q] = (uint32_t)min(tm * BM + r, p.M - 1) * (uint32_t)p.lda * 2u + 16u * c;
    }
#pragma unroll
    for (int k = 0; k < NWC; k++)
      vw[k] = (uint32_t)phys_band(tn, 2 * wave + k / NH) * TILEB + 1024u * (k % NH) + 16u * lane;
    vs = (uint32_t)phys_band(tn, 2 * wave + h) * TILEB + CODES + 4u * j;  // lane l: band 2 w + l / 32, column l % 32
  };
  // The stream walks units u0 .. u1 - 1 and then stays on u1 - 1. `left` counts the advances to its next event (a
  // tile boundary or the run's last unit); only then does it branch.
  int s_tile = tile_first, to_switch = G - u0 % G, to_end = n - 1;
  uint32_t a_so = (uint32_t)(u0 % G) * 2u * kGroup, w_so = (uint32_t)(u0 % G) * gstride;
  uint32_t a_inc = 2u * kGroup, w_inc = gstride;
  int seg = min(to_switch, to_end), left;
  if (to_end == 0) a_inc = 0, w_inc = 0, seg = 1 << 30;
  left = seg;
  set_tile(s_tile);
  auto advance = [&]() __attribute__((always_inline)) {
    a_so += a_inc;
    w_so += w_inc;
    if (--left == 0) {
      to_switch -= seg;
      to_end -= seg;
      if (to_switch == 0) {  // the next unit opens the next tile
        set_tile(++s_tile);
        a_so = 0, w_so = 0, to_switch = G;
      }
      if (to_end == 0) a_inc = 0, w_inc = 0, seg = 1 << 30;  // on the run's last unit: stay
      else seg = min(to_switch, to_end);
      left = seg;
    }
  };
  // DMA d of the pair bound for stage s: activation rows (d < MT), code halves, then the (s, b) rows
  auto issue_one = [&](int s, int d) __attribute__((always_inline)) {
    uint8_t* st = lds + s * STAGE;
    if (d < MT) sk_dma(ra, st + (MT * wave + d) * 1024, va[d], a_so);
    else if (d - MT < NWC)
      sk_dma(rw, st + A_BYTES + (2 * wave + (d - MT) / NH) * CODES + ((d - MT) % NH) * 1024, vw[d - MT], w_so);
    else sk_dma4(rw, st + A_BYTES + 8 * CODES + 2 * wave * 128, vs, w_so);
  };

  // LDS reads one step ahead of their use
  struct Codes {
    u32x4 w[2][NH];
    uint32_t sb[2];
  };
  auto read_codes = [&](int s, Codes& cd) __attribute__((always_inline)) {  // this wave's two bands of stage s
    const uint8_t* wst = lds + s * STAGE + A_BYTES;
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const int band = 2 * wave + nb;
#pragma unroll
      for (int hh = 0; hh < NH; hh++) cd.w[nb][hh] = *(const u32x4*)(wst + band * CODES + hh * 1024 + 16 * lane);
      cd.sb[nb] = *(const uint32_t*)(wst + 8 * CODES + band * 128 + 4 * j);
    }
  };
  // MFMA step t's B fragment of band nb: column j, k = 32 h + 8 t .. + 7 dequantized to bf16(s q + b). sa, sbs: the
  // scalings of s for t64_dequant (4 bits); 8 bits: sa = s, and q = stored byte ^ 0x80.
  auto deq_step = [&](const Codes& cd, int nb, int t, float sa, float sbs, float bi) __attribute__((always_inline)) {
    if constexpr (BITS == 4) {
      return t64_dequant(cd.w[nb][0][t], sa, sbs, bi);
    } else {
      (void)sbs;
      return dequant8x8_bf16(cd.w[nb][t / 2][2 * (t % 2)] ^ 0x80808080u, cd.w[nb][t / 2][2 * (t % 2) + 1] ^ 0x80808080u,
                             sa, bi);
    }
  };
  auto scales = [&](uint32_t sbw, float& sa, float& sbs, float& bi) __attribute__((always_inline)) {
    const float sc = bf2f((uint16_t)(sbw & 0xFFFFu));
    bi = bf2f((uint16_t)(sbw >> 16));
    sa = BITS == 4 ? t64_sa(sc) : sc;
    sbs = BITS == 4 ? t64_sb(sc) : 0.f;
  };
  auto dequant = [&](const Codes& cd, u32x4 (&bf)[2][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      float sa, sbs, bi;
      scales(cd.sb[nb], sa, sbs, bi);
#pragma unroll
      for (int t = 0; t < 4; t++) bf[nb][t] = deq_step(cd, nb, t, sa, sbs, bi);
    }
  };
  // activation fragments of stage s: M tile a, MFMA step t takes k = 32 h + 8 t .. + 7 (logical column 4 h + t)
  auto load_a = [&](int s, u32x4 (&af)[MT][4]) __attribute__((always_inline)) {
    const uint8_t* st = lds + s * STAGE;
#pragma unroll
    for (int a = 0; a < MT; a++) {
      const int r = a * 32 + j;
#pragma unroll
      for (int t = 0; t < 4; t++) af[a][t] = *(const u32x4*)(st + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
    }
  };

  f32x16 acc[2][MT];
#pragma unroll
  for (int nb = 0; nb < 2; nb++)
#pragma unroll
    for (int a = 0; a < MT; a++) acc[nb][a] = zero16();

  // Fragment sets by step parity: entering step i, set i % 2 holds A(i)'s fragments, W(i) dequantized and W(i + 1)'s
  // codes; the step fills the other set with A(i + 1), W(i + 1) dequantized and W(i + 2)'s codes.
  u32x4 af[2][MT][4], bf[2][2][4];
  Codes cd[2];

  // prologue: pairs 0 .. R - 1; A(0) and W(0), W(1) (pairs 0, 1) are awaited before step 0
#pragma unroll
  for (int s = 0; s < R; s++) {
#pragma unroll
    for (int d = 0; d < PAIR; d++) issue_one(s, d);
    advance();
  }
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((R - 2) * PAIR) : "memory");
  load_a(0, af[0]);
  read_codes(0, cd[0]);
  dequant(cd[0], bf[0]);
  read_codes(1, cd[0]);

  // Step i = K (mod UNR): eight groups, each closed by a scheduling barrier: MT MFMAs of this step (consecutive ones
  // on different accumulators), one 8-code dequant of the next, a share of the LDS reads for the next steps and of
  // the pair's DMAs, so that the matrix core has work through the whole step and the wave's other instructions issue
  // in its shadow.
  auto step = [&](auto KC) __attribute__((always_inline)) {
    constexpr int K = decltype(KC)::value, S = K % R, P = K % 2, S1 = (S + 1) % R, S2 = (S + 2) % R;
    constexpr int NDS = 4 * MT + 2 * (NH + 1), DEQ = BITS == 4 ? 17 : 22;
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((R - 3) * PAIR) : "memory");
    const uint8_t* const ast = lds + S1 * STAGE;           // activation fragments of step i + 1
    const uint8_t* const wst = lds + S2 * STAGE + A_BYTES;  // codes of step i + 2
    float sa[2], sbs[2], bi[2];
#pragma unroll
    for (int nb = 0; nb < 2; nb++) scales(cd[P].sb[nb], sa[nb], sbs[nb], bi[nb]);
#pragma unroll
    for (int g = 0; g < 8; g++) {
#pragma unroll
      for (int d = g * PAIR / 8; d < (g + 1) * PAIR / 8; d++) issue_one(S, d);
#pragma unroll
      for (int d = g * NDS / 8; d < (g + 1) * NDS / 8; d++) {
        if (d < 4 * MT) {
          const int am = d / 4, t = d % 4, r = am * 32 + j;
          af[P ^ 1][am][t] = *(const u32x4*)(ast + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
        } else {
          const int nb = (d - 4 * MT) / (NH + 1), e = (d - 4 * MT) % (NH + 1), band = 2 * wave + nb;
          if (e < NH) cd[P ^ 1].w[nb][e] = *(const u32x4*)(wst + band * CODES + e * 1024 + 16 * lane);
          else cd[P ^ 1].sb[nb] = *(const uint32_t*)(wst + 8 * CODES + band * 128 + 4 * j);
        }
      }
      bf[P ^ 1][g / 4][g % 4] = deq_step(cd[P], g / 4, g % 4, sa[g / 4], sbs[g / 4], bi[g / 4]);
#pragma unroll
      for (int m = g * MT; m < (g + 1) * MT; m++) {
        const int am = m % MT, nb = (m / MT) % 2, t = m / (2 * MT);
        acc[nb][am] = mfma_bf16(af[P][am][t], bf[P][nb][t], acc[nb][am]);
      }
#pragma unroll
      for (int m = 0; m < MT; m++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, DEQ / MT + 1, 0);  // VALU
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int t = 0; t < 4; t++) asm volatile("" : "+v"(bf[P ^ 1][nb][t]));
    advance();
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

  // Steps [lo, hi): the unrolled body starts at phase 0, and its first pass skips the steps before lo (one unsigned
  // compare per step).
  auto run = [&](int lo, int hi) __attribute__((always_inline)) {
    int i = lo - lo % UNR;
    const uint32_t len = (uint32_t)(hi - lo);
    while (i < hi) {
      sk_static_for<0, UNR>([&](auto KC) __attribute__((always_inline)) {
        if ((uint32_t)(i - lo) < len) step(KC);
        i++;
      });
    }
  };
  // the run's one or two segments: the first segment's piece is written as soon as it ends, while the run goes on
  const bool two = tile_last != tile_first;
  const int n1 = min(n, (tile_first + 1) * G - u0);
  int lo = 0, hi = n1;
#pragma clang loop unroll(disable)
  for (int sgi = 0; sgi < 2; sgi++) {
    run(lo, hi);
    if (sgi == 1 || !two) break;
    write_slot(2 * b);
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int a = 0; a < MT; a++) acc[nb][a] = zero16();
    lo = n1, hi = n;
  }
  // every DMA and partial store has landed; LDS is free once all waves are past their reads
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // A tile is staged through LDS ([BM][kSkRow] fp32) and leaves as rows (SwiGLU: h). Lane (wave, j, h) stages
  // acc[nb][a][r] at row a 32 + 8 (r / 4) + 4 h + r % 4, column 32 (2 wave + nb) + j, which are also the entries of its
  // float4s in a piece slot. The caller has passed a barrier since the staging area was last read.
  auto stg_at = [&](int nb, int a, int r) __attribute__((always_inline)) {
    return stg + (a * 32 + 8 * (r / 4) + 4 * h + (r % 4)) * kSkRow + 32 * (2 * wave + nb) + j;
  };
  auto stage_tile = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int a = 0; a < MT; a++)
#pragma unroll
        for (int r = 0; r < 16; r++) *stg_at(nb, a, r) = acc[nb][a][r];
  };
  auto emit_tile = [&](int t) __attribute__((always_inline)) {
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
  auto store_tile = [&](int t) __attribute__((always_inline)) {
    stage_tile();
    emit_tile(t);
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

template <int MT, int BITS>
__global__ __launch_bounds__(kSkThreads, sk_bpc(MT, BITS)) void k_gemm_sk(GemmSkArgs p) {
  static_assert(sk_lds(MT, BITS) + 64 <= kSkLds / sk_bpc(MT, BITS), "LDS plan");
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = xcd_remap(blockIdx.x, p.nblk);
  sk_body<MT, BITS>(p, lds, wave, b);
}

// Sum of a cut tile's pieces (partial slots, in unit order) and its store. Block (tile, w, a), wave q: the float4
// fragment (a, q) of column band w of the tile (SwiGLU: gate band w with up band w + 4, giving h), the
// loads of up to kFixBatch pieces in flight at once; whole tiles were stored by the GEMM kernel. blockIdx.x is the
// tile's index among the stream-K tiles (units [tile G, tile G + G) of their U = ntiles G).
constexpr int kFixBatch = 8;
template <int MT>
__global__ __launch_bounds__(256) void k_sk_fixup(GemmSkArgs p) {
  constexpr int BM = 32 * MT, NE = MT * 16;
  const int tile = blockIdx.x, w = blockIdx.y, a = blockIdx.z, q = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  // run boundaries in 32-bit arithmetic (the host keeps U nblk below 2^32): block bb's run starts at unit
  // bb U / nblk, and unit u lies in the run of block (u nblk + nblk - 1) / U
  const uint32_t G = (uint32_t)p.G, U = (uint32_t)p.ntiles * G, nb = (uint32_t)p.nblk;
  const uint32_t tlo = (uint32_t)tile * G;
  const int bf = (int)((tlo * nb + nb - 1) / U), bl = (int)(((tlo + G - 1) * nb + nb - 1) / U);
  if (bf == bl) return;
  // Block bf holds the tile's first unit: the tile is its second segment (slot 2 bf + 1) when its run starts
  // before the tile, else its first (slot 2 bf). Every later block's run starts inside the tile, which is its first
  // segment (slot 2 bb). With more blocks than units (sparse) some of those runs are empty and hold no piece.
  const uint32_t lo_f = (uint32_t)bf * U / nb;
  const float4* part = (const float4*)p.part;
  const int w1 = p.swi ? w + 4 : w;  // SwiGLU: the up band's pieces, loaded beside the gate band's
  float4 t0 = make_float4(0.f, 0.f, 0.f, 0.f), t1 = t0;
  for (int b0 = bf; b0 <= bl; b0 += kFixBatch) {
    float4 x0[kFixBatch], x1[kFixBatch];
    bool has[kFixBatch];
#pragma unroll
    for (int k = 0; k < kFixBatch; k++) {
      const int bb = b0 + k;
      has[k] = bb <= bl;
      if (has[k] && p.sparse && bb > bf) has[k] = (uint32_t)(bb + 1) * U / nb > (uint32_t)bb * U / nb;
      if (has[k]) {
        const int slot = 2 * bb + (bb == bf && lo_f < tlo ? 1 : 0);
        x0[k] = part[(((size_t)slot * 8 + w) * NE / 4 + a * 4 + q) * 64 + lane];
        if (p.swi) x1[k] = part[(((size_t)slot * 8 + w1) * NE / 4 + a * 4 + q) * 64 + lane];
      }
    }
#pragma unroll
    for (int k = 0; k < kFixBatch; k++)
      if (has[k]) {
        t0.x += x0[k].x, t0.y += x0[k].y, t0.z += x0[k].z, t0.w += x0[k].w;
        if (p.swi) t1.x += x1[k].x, t1.y += x1[k].y, t1.z += x1[k].z, t1.w += x1[k].w;
      }
  }
  const int tm = (p.tile0 + tile) % p.tiles_m, tn = (p.tile0 + tile) / p.tiles_m;
  const float4 v = t0;
  float vv[4] = {v.x, v.y, v.z, v.w};
  const int row0 = tm * BM + a * 32 + 8 * q + 4 * h;
  if (p.rs) {
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (row0 + e < p.M) vv[e] *= p.rs[(size_t)(row0 + e) * p.rs_stride];
  }
  if (p.swi) {
    const float4 u4 = t1;
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

struct SkPlan {
  int MT, tiles_m, tiles_n, G, nblk;
};
static SkPlan gemm_sk_plan(int M, int N, int K, int bits = 4) {
  SkPlan pl{};
  pl.MT = M <= 32 ? 1 : M <= 64 ? 2 : 4;
  const int bpc = pl.MT == 1 && bits == 4 ? 2 : 1;  // sk_bpc
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
  if (M <= 16 || K % kGroup || t64_bytes(N, K) >= ((size_t)1 << 31)) return false;
  if (mode == kModeSwiglu && N % 256) return false;
  const SkPlan pl = gemm_sk_plan(M, N, K);
  if (((uint64_t)pl.tiles_m * pl.tiles_n * pl.G + 1) * (pl.nblk + 1) >= ((uint64_t)1 << 32)) return false;  // fixup
  return (long)pl.tiles_m * pl.tiles_n * 3 >= cu_count() || (M > 64 && M <= 128);
}

static size_t sk_part_bytes(const SkPlan& pl) { return (size_t)2 * pl.nblk * 8 * (16 * pl.MT) * 64 * sizeof(float); }

size_t gemm_sk_workspace(int M, int N, int K, int mode) {
  (void)mode;
  return sk_part_bytes(gemm_sk_plan(M, N, K));
}

size_t gemm_sk8_workspace(int M, int N, int K) { return sk_part_bytes(gemm_sk_plan(M, N, K, 8)); }

template <int MT, int BITS>
static int launch_sk_cfg(const GemmSkArgs& a, bool fixup, hipStream_t st) {
  constexpr size_t lds = sk_lds(MT, BITS);
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)k_gemm_sk<MT, BITS>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr = true;
  }
  hipLaunchKernelGGL((k_gemm_sk<MT, BITS>), dim3(a.nblk), dim3(kSkThreads), lds, st, a);
  IFD_TRY(check_launch("gemm_sk"));
  if (!fixup) return IFD_OK;
  hipLaunchKernelGGL(k_sk_fixup<MT>, dim3(a.ntiles, a.swi ? 4 : 8, MT), dim3(256), 0, st, a);
  return check_launch("gemm_sk fixup");
}

int launch_sk_fixup_rows(const float* part, int tiles_m, int tiles_n, int tile0, int ntiles, int G, int nblk, void* C,
                         int ldc, int M, int N, int mode, const float* rs, int rs_stride, hipStream_t st) {
  GemmSkArgs a{};
  a.part = (float*)part;
  a.tiles_m = tiles_m, a.tiles_n = tiles_n, a.tile0 = tile0, a.ntiles = ntiles, a.G = G, a.nblk = nblk;
  a.C = C, a.ldc = ldc, a.M = M, a.N = N, a.mode = mode, a.rs = rs, a.rs_stride = rs_stride;
  a.sparse = (long)ntiles * G < nblk;
  hipLaunchKernelGGL(k_sk_fixup<4>, dim3(ntiles, 8, 4), dim3(256), 0, st, a);
  return check_launch("sk fixup");
}

template <int BITS>
static int launch_sk_bits(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                          void* ws, size_t ws_bytes, hipStream_t st) {
  const SkPlan pl = gemm_sk_plan(M, N, K, BITS);
  const size_t need = sk_part_bytes(pl), wbytes = BITS == 8 ? t64x8_bytes(N, K) : t64_bytes(N, K);
  if (need > ws_bytes || !ws)
    return fail(IFD_ERR_WORKSPACE, "gemm_sk needs %zu bytes of workspace, got %zu", need, ws_bytes);
  if (need >= (size_t)1 << 31) return fail(IFD_ERR_UNSUPPORTED, "gemm_sk: partials past 2 GiB");
  if (wbytes >= ((size_t)1 << 31) || (size_t)M * lda * 2 >= ((size_t)1 << 31))
    return fail(IFD_ERR_UNSUPPORTED, "gemm_sk: operands past 2 GiB");
  if (((uint64_t)pl.tiles_m * pl.tiles_n * pl.G + 1) * (pl.nblk + 1) >= ((uint64_t)1 << 32))
    return fail(IFD_ERR_UNSUPPORTED, "gemm_sk: too many units");
  // the fixup kernel runs when some tile is cut
  const long tiles = (long)pl.tiles_m * pl.tiles_n, U = tiles * pl.G;
  bool fixup = false;
  for (long t = 0; t < tiles && !fixup; t++)
    fixup = sk_block_of(t * pl.G + pl.G - 1, pl.nblk, U) != sk_block_of(t * pl.G, pl.nblk, U);
  GemmSkArgs a{A, lda, (const uint8_t*)wt, (uint32_t)wbytes, N, K, C, ldc, M, mode, (float*)ws, (uint32_t)need,
               pl.tiles_m, pl.tiles_n, pl.G, pl.nblk, mode == kModeSwiglu ? N / 64 : 0, 0, (int)tiles, nullptr, 0, 0};
  if (pl.MT == 1) return launch_sk_cfg<1, BITS>(a, fixup, st);
  if (pl.MT == 2) return launch_sk_cfg<2, BITS>(a, fixup, st);
  return launch_sk_cfg<4, BITS>(a, fixup, st);
}

int launch_gemm_sk(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                   void* ws, size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (!gemm_sk_applies(M, N, K, mode)) return fail(IFD_ERR_UNSUPPORTED, "gemm_sk: shape M=%d N=%d K=%d", M, N, K);
  return launch_sk_bits<4>(A, lda, wt, N, K, C, ldc, M, mode, ws, ws_bytes, st);
}

int launch_gemm_sk8(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                    void* ws, size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (K % kGroup || (mode == kModeSwiglu && N % 256))
    return fail(IFD_ERR_UNSUPPORTED, "gemm_sk8: shape N=%d K=%d", N, K);
  return launch_sk_bits<8>(A, lda, wt, N, K, C, ldc, M, mode, ws, ws_bytes, st);
}

}  // namespace ifd
