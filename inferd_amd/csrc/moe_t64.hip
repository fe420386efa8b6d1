// Gathered expert GEMM on T64 expert stacks: C[q][n] = bf16(sum_k A_row(q)[k] * bf16(s q + b)[n][k]) over expert-
// sorted rows q, with the SwiGLU of a [gate | up] stack fused (C receives h), for the MoE FFN's gate/up and down
// products (reference affine_gather_qmm_rhs, third_party/mlx/.../quantized_nax.h:1467-1681, scheduled by
// schedule_row_tile, steel/utils.h:502-542; moe_silu_mul, moe.metal:103-111).
//
// Work items are (row tile, column tile) pairs: a row tile is up to BM = 32 MT sorted rows of one expert (the
// dispatch's tile schedule), a column tile 8 bands (256 output columns; with SwiGLU 8 gate bands and the matching 8
// up bands, 256 h columns). Items are numbered row tile-major, so an expert's column tiles are neighbours and share
// its activation rows in L2. The grid is one block per CU; a block streams a contiguous run of (item, group pair)
// units as one continuous sequence of (item, 64-group) steps, so the DMA pipeline runs across item boundaries without
// draining. Without a piece buffer a run is whole items, [b n / nblk, (b + 1) n / nblk). With one (the balanced
// schedule) block b takes units [b U / nblk, (b + 1) U / nblk) of the U = n G / 2: every CU streams the same bytes
// whatever n, and an item cut by a run boundary leaves each contributor's fp32 sums (its rows only) in a piece slot,
// written through to memory. The contributors count themselves in a counter of the workspace header once their run
// is done; the last one sums the item's pieces in unit order and stores the item as a whole item ends. A cut item's
// sum is therefore the sum of its K ranges' sums, in K order, and does not depend on timing.
//
// Block: 8 waves; wave w owns band w of the column tile (with SwiGLU, its gate band and its up band) over all MT M
// tiles. Two LDS rings filled by direct global -> LDS DMA: NA activation slabs [BM][64 bf16] (16-byte columns
// XOR-swizzled by row pair), whose rows are gathered through perm by the DMA itself (row q of a tile is token
// perm[q] / div, or row q of A), and NW weight stages (the item's code halves and (s, b) rows of one group). Waves
// 0-3 issue the activation DMAs, waves 4-7 the weight DMAs, each as buffer loads whose per-lane offsets are set once
// per item and whose group offset is one scalar register, so a step issues no address arithmetic; each role's code
// is compiled on its own, so every wait is a constant. Row indices come from scalar loads, which do not count in
// vmcnt. Weights are dequantized to bf16(s q + b) (MLX's gather_qmm rounding) one step ahead of their MFMAs; the k
// order of a lane's MFMA steps is that of k_gqmm, so the sums are bit-identical to it.
//
// At the end of an item a wave stages its bf16 outputs in its own LDS tile and writes them as 16-byte buffer
// stores, rows past the segment at an out-of-range offset (dropped by the buffer bounds check).
#include <algorithm>
#include <cmath>

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
  uint32_t a_bytes;  // bytes of A that a sorted row may read (buffer bound)
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
  float* part;         // balanced schedule: piece slots [2 nblk][8 waves][NBW][MT][4][64] float4; null: whole items
  uint32_t part_bytes;
  unsigned* cnt;       // [nblk] counters of the cut items (zero between calls), by the block holding the first unit
};

// The balanced schedule runs when whole-item runs would make the longest run at least this many (item, group pair)
// units longer than the even share (config 4: gate/up at T = 16 and 2048, 14.5 and 11.8 units; not down, nor gate/up
// at T = 128, 2-5 units, where the cut items' sums cost more than they save).
constexpr int kGqMinLoss = 8;
// the block whose run of units holds unit u (runs [b U / nblk, (b + 1) U / nblk))
__device__ __forceinline__ int gq_block_of(long u, int nblk, long U) { return (int)((u * nblk + nblk - 1) / U); }

// bands per wave: two with SwiGLU (its gate and up band) or in the wide plain form (two 8-band column groups)
__host__ __device__ constexpr int gq_nbw(bool two) { return two ? 2 : 1; }
__host__ __device__ constexpr int gq_abytes(int MT) { return MT * 32 * 128; }
__host__ __device__ constexpr int gq_wbytes(bool two) { return gq_nbw(two) * (8 * kT64Codes + 8 * 128); }
constexpr int kGqStg = 32 * 64;  // a wave's staged output: one M tile [32][32] bf16
__host__ __device__ constexpr int gq_na(int MT, bool two) { return two ? 4 : (MT == 2 ? 6 : 8); }
__host__ __device__ constexpr int gq_nw(int MT, bool two) { return two ? (MT == 2 ? 6 : 7) : (MT == 2 ? 10 : 12); }
// the rings, the waves' output tiles and one word for the cut items' arrival flag
__host__ __device__ constexpr size_t gq_lds(int MT, bool two) {
  return (size_t)gq_na(MT, two) * gq_abytes(MT) + (size_t)gq_nw(MT, two) * gq_wbytes(two) + 8 * kGqStg + 16;
}
// bytes of one piece slot at 32 MT-row tiles (two bands per wave at most)
__host__ __device__ constexpr size_t gq_slot_bytes(int MT) { return (size_t)8 * 2 * MT * 4 * 64 * 16; }

// A scalar (SMEM) load of a wave-uniform element: it counts in lgkmcnt, not in vmcnt.
__device__ __forceinline__ int sload(const int* p, int i) {
  return *((const __attribute__((address_space(4))) int*)p + __builtin_amdgcn_readfirstlane(i));
}

// One wave-wide 16-byte-per-lane DMA through a buffer resource: lane l's 16 bytes at voff(l) + soff land at
// lds + 16 l (LDS base in M0, wave-uniform control flow only). Out-of-range lanes write zeros.
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, (int)voff, (int)soff, 0, 0);
}
// The same with the non-temporal cache policy, for the expert weights: most are read by one row tile's items only
// (measured on the operator at config 4: T = 16 / 128 / 2048 134.4 / 246.3 / 397.5 -> 128.4 / 243.2 / 373.9 us)
__device__ __forceinline__ void bdma16_nt(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, (int)voff, (int)soff, 0, kNt);
}

// The pipeline of one wave role. ROLE 0: waves 0-3, the activation DMAs (MT per step); ROLE 1 / 2: waves 4-7, the
// weight DMAs (NCW code tiles per step, ROLE 1 also one (s, b) DMA). Each role's DMA stream has a fixed shape, so
// every wait is a compile-time count of the DMAs younger than the one awaited:
// - ROLE 0 needs A(i + 1) at step i (its fragments are read a step ahead), issued NA - 2 steps earlier: the
//   MT (NA - 3) DMAs of the steps between are younger.
// - ROLE 1 / 2 need W(i + 2) at step i (its codes are read two steps ahead), issued NW - 3 steps earlier:
//   D (NW - 4) younger DMAs.
// DMA loads retire from vmcnt in issue order. The output stores of an item end are not counted: a store may retire
// before an older load, so counting it could release a wait early, while an uncounted store still in flight only
// makes the wait longer. The streams run on past the last step (re-reading it) so that the steady counts hold to the
// end; the kernel drains vmcnt before it exits.
// BAL: the balanced schedule's run (cut items possible); otherwise whole items only, compiled without the pieces
template <int MT, bool SILU, bool WIDE, int ROLE, bool BAL>
__device__ __forceinline__ void gq_role(const GqArgs& p, uint8_t* lds, const int wave, const int b, const int nitems,
                                        const int u0, const int u1) {
  constexpr bool TWO = SILU || WIDE;
  constexpr int NBW = gq_nbw(TWO), NA = gq_na(MT, TWO), NW = gq_nw(MT, TWO);
  constexpr int A_BYTES = gq_abytes(MT), W_BYTES = gq_wbytes(TWO);
  constexpr int SB_OFF = NBW * 8 * kT64Codes;  // (s, b) rows of a weight stage, after its code tiles
  constexpr int NCW = TWO ? 4 : 2;             // code DMAs per weight wave per step
  constexpr bool AW = ROLE == 0;
  constexpr int D = AW ? MT : NCW + (ROLE == 1 ? 1 : 0);  // DMAs per step
  constexpr int NR = AW ? NA : NW;                          // the ring this role fills
  constexpr int LAG = AW ? NA - 1 : NW - 1;                 // steps the issue runs ahead
  constexpr int BASE = AW ? D * (NA - 3) : D * (NW - 4);  // younger than A(i + 1) / W(i + 2) at step i
  static_assert(NA >= 3 && NW >= 4 && D * (AW ? NA - 2 : NW - 3) <= 63, "ring depth, vmcnt range");
  uint8_t* const aring = lds;
  uint8_t* const wring = lds + NA * A_BYTES;
  const int tid = threadIdx.x, lane = tid & 63;
  const int j = lane & 31, h = lane >> 5;
  uint16_t* const stg = (uint16_t*)(wring + NW * W_BYTES + wave * kGqStg);
  const int G = p.G, G2 = G / 2;
  const int nbands = t64_bands(p.N);
  const uint32_t gstride = (uint32_t)nbands * kT64Tile;
  const int up0 = nbands / 2;  // first up band of a [gate | up] stack
  // weight roles: SwiGLU / wide, code tiles [4 ww, 4 ww + 4) of the stage's 16 and the (s, b) DMA ww for ww < 2;
  // plain, code tiles [2 ww, 2 ww + 2) of 8 and the (s, b) DMA for ww = 3
  const int ww = wave - 4;
  const int sbj = TWO ? ww : 0;

  // (expert, column tile, rows) of an item; a tile holds at least its first row
  auto item_rows = [&](int item, int& e, int& c, int& q0, int& q1) __attribute__((always_inline)) {
    const int tile = item >> p.nct_log2;
    c = item & ((1 << p.nct_log2) - 1);
    e = min(max(sload(p.tiles, 2 * tile), 0), p.E);
    q0 = sload(p.tiles, 2 * tile + 1);
    q1 = max(min(sload(p.offsets, e + 1), q0 + 32 * MT), q0 + 1);
  };
  auto band_of = [&](int c, int ti) __attribute__((always_inline)) {  // physical band of the stage's tile ti
    const int bb = SILU ? (ti < 8 ? 8 * c + ti : up0 + 8 * c + ti - 8) : (WIDE ? 16 * c + ti : 8 * c + ti);
    return min(bb, nbands - 1);
  };

  // ---- this role's DMA stream: (item, group) of the next issue; per-lane offsets of the item, group offset soff
  // the source base of the stream (A, or the item's expert), as two wave-uniform halves: the buffer resource built
  // from them stays in SGPRs
  uint32_t base_lo = (uint32_t)(uintptr_t)p.A, base_hi = (uint32_t)((uintptr_t)p.A >> 32);
  const uint32_t nrec = AW ? p.a_bytes : (uint32_t)p.ebytes;
  uint32_t voff[D];
  const uint32_t gstep = AW ? 2u * kGroup : gstride;
  int s_item = u0 / G2, s_g = 2 * (u0 - s_item * G2), s_st = 0, s_left = 2 * (u1 - u0) - 1;
  uint32_t soff = (uint32_t)s_g * gstep;
  auto stream_item = [&](int item) __attribute__((always_inline)) {
    int e, c, q0, q1;
    item_rows(item, e, c, q0, q1);
    if constexpr (AW) {
      const uint32_t rowb = 2u * (uint32_t)p.lda;
      if (p.perm) {
        // the wave's 8 MT row indices: all scalar loads in flight at once, then one wait
        int v[MT][8];
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
          for (int rho = 0; rho < 8; rho++) v[i][rho] = sload(p.perm, min(q0 + 8 * (MT * wave + i) + rho, q1 - 1));
        if (p.div_m)
#pragma unroll
          for (int i = 0; i < MT; i++)
#pragma unroll
            for (int rho = 0; rho < 8; rho++)
              v[i][rho] = (int)__builtin_amdgcn_readfirstlane(__umulhi((uint32_t)v[i][rho], p.div_m));
#pragma unroll
        for (int i = 0; i < MT; i++) {
          int src = 0;
#pragma unroll
          for (int rho = 0; rho < 8; rho++) src = (lane >> 3) == rho ? v[i][rho] : src;
          const int r = 8 * (MT * wave + i) + (lane >> 3);
          voff[i] = (uint32_t)src * rowb + 16u * (uint32_t)((lane & 7) ^ ((r >> 1) & 7));
        }
      } else {
#pragma unroll
        for (int i = 0; i < MT; i++) {
          const int r = 8 * (MT * wave + i) + (lane >> 3);
          voff[i] = (uint32_t)min(q0 + r, q1 - 1) * rowb + 16u * (uint32_t)((lane & 7) ^ ((r >> 1) & 7));
        }
      }
    } else {
      // expert E is the shared expert; without one the reads stay inside the stack
      const uint8_t* wb = e >= p.E && p.wsh ? p.wsh : p.wt + (size_t)min(e, p.E - 1) * p.ebytes;
      base_lo = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)wb);
      base_hi = __builtin_amdgcn_readfirstlane((uint32_t)((uintptr_t)wb >> 32));
#pragma unroll
      for (int i = 0; i < NCW; i++) voff[i] = (uint32_t)band_of(c, NCW * ww + i) * kT64Tile + 16u * lane;
      if constexpr (ROLE == 1)
        voff[NCW] = (uint32_t)band_of(c, 8 * sbj + (lane >> 3)) * kT64Tile + kT64Codes + 16u * (lane & 7);
    }
  };
  stream_item(s_item);
  auto issue = [&]() __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(((uint64_t)base_hi << 32) | base_lo), 0, (int)nrec, 0x00020000);
    if constexpr (AW) {
      uint8_t* st = aring + s_st * A_BYTES;
#pragma unroll
      for (int i = 0; i < MT; i++) bdma16(rsrc, st + (MT * wave + i) * 1024, voff[i], soff);
    } else {
      uint8_t* st = wring + s_st * W_BYTES;
#pragma unroll
      for (int i = 0; i < NCW; i++) bdma16_nt(rsrc, st + (NCW * ww + i) * kT64Codes, voff[i], soff);
      if constexpr (ROLE == 1) bdma16_nt(rsrc, st + SB_OFF + sbj * 1024, voff[NCW], soff);
    }
    s_st = s_st + 1 == NR ? 0 : s_st + 1;
    if (s_left <= 0) return;  // past the run's last step: re-read it (L2 hits), never new bytes
    s_left--;
    soff += gstep;
    if (++s_g == G) {  // next item
      s_g = 0;
      soff = 0;
      stream_item(++s_item);
    }
  };

  // LDS reads run one step ahead of their use: at step i the wave reads the activation fragments of step i + 1 and
  // the weight codes of step i + 2 while its MFMAs (step i) and dequant (step i + 1) work on registers, so neither
  // waits on LDS.
  struct Codes {
    u32x4 w[NBW];
    uint32_t sb[NBW];
  };
  auto read_codes = [&](int ws, Codes& cd) __attribute__((always_inline)) {  // this wave's bands of weight stage ws
    const uint8_t* wst = wring + ws * W_BYTES;
#pragma unroll
    for (int nb = 0; nb < NBW; nb++) {
      const int t = 8 * nb + wave;
      cd.w[nb] = *(const u32x4*)(wst + t * kT64Codes + 16 * lane);
      cd.sb[nb] = *(const uint32_t*)(wst + SB_OFF + t * 128 + 4 * j);
    }
  };
  auto dequant = [&](const Codes& cd, u32x4 (&bf)[NBW][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NBW; nb++) {
      const float sc = bf2f((uint16_t)(cd.sb[nb] & 0xFFFFu)), bi = bf2f((uint16_t)(cd.sb[nb] >> 16));
      const float sa = t64_sa(sc), sbs = t64_sb(sc);
#pragma unroll
      for (int q = 0; q < 4; q++) bf[nb][q] = t64_dequant(cd.w[nb][q], sa, sbs, bi);
    }
  };
  // activation fragments of stage st: M tile a, MFMA step t takes k = 32 h + 8 t .. + 7 (logical column 4 h + t)
  auto load_a = [&](const uint8_t* st, u32x4 (&af)[MT][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < MT; a++) {
      const int r = a * 32 + j;
#pragma unroll
      for (int t = 0; t < 4; t++) af[a][t] = *(const u32x4*)(st + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
    }
  };

  f32x16 acc[NBW][MT];
#pragma unroll
  for (int nb = 0; nb < NBW; nb++)
#pragma unroll
    for (int a = 0; a < MT; a++) acc[nb][a] = zero16();

  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)p.C, 0, (int)p.c_bytes, 0x00020000);
  // prologue: LAG steps of this role's stream; then A(0) and W(0), W(1) into registers
  for (int i = 0; i < LAG; i++) issue();
  if constexpr (AW) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(D * (NA - 2)) : "memory");  // A(0)
  else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(D * (NW - 3)) : "memory");               // W(0), W(1)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  u32x4 bf0[NBW][4], bf1[NBW][4], af0[MT][4], af1[MT][4];
  Codes cd0, cd1;
  load_a(aring, af0);
  read_codes(0, cd0);
  dequant(cd0, bf0);
  read_codes(1 % NW, cd0);
  int ca1 = 1 % NA, cw2 = 2 % NW;  // stages read at step i: activations of step i + 1, codes of step i + 2

  // Step i: B fragments bc and activation fragments afc of step i, codes cc of step i + 1 in registers; reads the
  // activations of step i + 1 into afn and the codes of step i + 2 into cn, dequantizes cc into bn. The waits are
  // for A(i + 1) (ROLE 0) and W(i + 2) (ROLE 1 / 2); the stage a DMA issued here overwrites was read two steps ago.
  auto step = [&](u32x4 (&bc)[NBW][4], u32x4 (&bn)[NBW][4], u32x4 (&afc)[MT][4], u32x4 (&afn)[MT][4], Codes& cc,
                  Codes& cn) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(BASE) : "memory");
    issue();
    // Eight groups, each closed by a scheduling barrier: 4 NBW MT / 8 MFMAs of this step, one 8-code dequant of the
    // next (17 VALU) and a share of the LDS reads for the next steps, so that the matrix core has work through the
    // whole step and the VALU issues in its shadow.
    constexpr int NMF = 4 * NBW * MT, NDS = 4 * MT + 2 * NBW, NDQ = 4 * NBW;
    const uint8_t* const ast = aring + ca1 * A_BYTES;  // activation fragments of step i + 1
    const uint8_t* const wst = wring + cw2 * W_BYTES;  // codes of step i + 2
    float sa[NBW], sbs[NBW], bi[NBW];
#pragma unroll
    for (int nb = 0; nb < NBW; nb++) {
      const float sc = bf2f((uint16_t)(cc.sb[nb] & 0xFFFFu));
      bi[nb] = bf2f((uint16_t)(cc.sb[nb] >> 16)), sa[nb] = t64_sa(sc), sbs[nb] = t64_sb(sc);
    }
#pragma unroll
    for (int g = 0; g < NDQ; g++) {
#pragma unroll
      for (int d = g * NDS / NDQ; d < (g + 1) * NDS / NDQ; d++) {
        if (d < 4 * MT) {
          const int am = d / 4, t = d % 4, r = am * 32 + j;
          afn[am][t] = *(const u32x4*)(ast + r * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7)));
        } else {
          const int nb = (d - 4 * MT) / 2, tt = 8 * nb + wave;
          if ((d - 4 * MT) % 2 == 0) cn.w[nb] = *(const u32x4*)(wst + tt * kT64Codes + 16 * lane);
          else cn.sb[nb] = *(const uint32_t*)(wst + SB_OFF + tt * 128 + 4 * j);
        }
      }
      bn[g / 4][g % 4] = t64_dequant(cc.w[g / 4][g % 4], sa[g / 4], sbs[g / 4], bi[g / 4]);
#pragma unroll
      for (int m = g * NMF / NDQ; m < (g + 1) * NMF / NDQ; m++) {  // MFMA order: M tile, band, k step
        const int am = m / (4 * NBW), nb = (m / 4) % NBW, t = m % 4;
        acc[nb][am] = mfma_bf16(afc[am][t], bc[nb][t], acc[nb][am]);
      }
#pragma unroll
      for (int m = 0; m < NMF / NDQ; m++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 17 * NDQ / NMF + 1, 0);  // VALU
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int nb = 0; nb < NBW; nb++)
#pragma unroll
      for (int t = 0; t < 4; t++) asm volatile("" : "+v"(bn[nb][t]));
    ca1 = ca1 + 1 == NA ? 0 : ca1 + 1;
    cw2 = cw2 + 1 == NW ? 0 : cw2 + 1;
  };

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

  if constexpr (!BAL) {
    for (int item = u0 / G2; item < u1 / G2; item++) {
      for (int g = 0; g < G; g += 2) {  // G is even
        step(bf0, bf1, af0, af1, cd0, cd1);
        step(bf1, bf0, af1, af0, cd1, cd0);
      }
      int e, c, q0, q1;
      item_rows(item, e, c, q0, q1);
      (void)e;
      epilogue(c, q0, q1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA lands in LDS after the block ends
    return;
  }
  // a cut item's piece: this wave's sums of the item's rows (fragment rows past them are never read), written through
  // to memory; float4 k of a lane holds rows 8 k + 4 h .. + 3 of its M tile
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc((void*)p.part, 0, (int)p.part_bytes, 0x00020000);
  auto piece_off = [&](int slot, int nb, int a, int k4) __attribute__((always_inline)) {
    return (int)((((((size_t)slot * 8 + wave) * NBW + nb) * MT + a) * 4 + k4) * 64 + lane) * 16;
  };
  auto store_piece = [&](int slot, int nrows) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NBW; nb++)
#pragma unroll
      for (int a = 0; a < MT; a++)
#pragma unroll
        for (int k4 = 0; k4 < 4; k4++) {
          if (a * 32 + 8 * k4 + 4 * h >= nrows) continue;
          const u32x4 v = {__float_as_uint(acc[nb][a][4 * k4]), __float_as_uint(acc[nb][a][4 * k4 + 1]),
                           __float_as_uint(acc[nb][a][4 * k4 + 2]), __float_as_uint(acc[nb][a][4 * k4 + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, rp, piece_off(slot, nb, a, k4), 0, kSc1);
        }
  };
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NBW; nb++)
#pragma unroll
      for (int a = 0; a < MT; a++) acc[nb][a] = zero16();
  };

  // the run: segments of items; a whole item is stored at its end, a cut one leaves a piece (slot 2 b for the run's
  // first segment, 2 b + 1 for its last)
  const long U = (long)nitems * G2;
  int u = u0, ncut = 0, cut0 = 0, cut1 = 0;
  bool seeded = false;  // acc still holds the run's last segment, the first piece of its cut item (its sum's seed)
  while (u < u1) {
    const int item = u / G2, ga = u - item * G2, gb = min(G2, u1 - item * G2);
    for (int g = ga; g < gb; g++) {  // a unit is two groups
      step(bf0, bf1, af0, af1, cd0, cd1);
      step(bf1, bf0, af1, af0, cd1, cd0);
    }
    int e, c, q0, q1;
    item_rows(item, e, c, q0, q1);
    (void)e;
    if (ga == 0 && gb == G2) {
      epilogue(c, q0, q1);
    } else {
      store_piece(2 * b + (u == u0 ? 0 : 1), q1 - q0);
      if (ncut == 0) cut0 = item;
      else cut1 = item;
      ncut++;
      // the item's first piece is this block's when the item starts in this run, which leaves it the run's last
      // segment: keep the sums for the item's total
      seeded = item * G2 + gb == u1 && gq_block_of((long)item * G2, p.nblk, U) == b;
      if (!seeded) zero_acc();
    }
    u = item * G2 + gb;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA lands in LDS after this; the pieces are in memory
  if (ncut == 0) return;
  // arrivals at the cut items, one counter round trip for both: the last contributor of an item sums its pieces in
  // unit order and stores it
  unsigned* const s_last = (unsigned*)(wring + NW * W_BYTES + 8 * kGqStg);
  auto contributors = [&](int item, int& bf, int& bl) __attribute__((always_inline)) {
    const long us = (long)item * G2;
    bf = gq_block_of(us, p.nblk, U), bl = gq_block_of(us + G2 - 1, p.nblk, U);
    int n = 0;
    for (int bb = bf; bb <= bl; bb++) n += (long)(bb + 1) * U / p.nblk > (long)bb * U / p.nblk;
    return n;
  };
  __syncthreads();  // every wave's pieces are complete
  if (threadIdx.x == 0) {
    unsigned old[2];
#pragma unroll
    for (int ci = 0; ci < 2; ci++)
      if (ci < ncut) {
        int bf, bl;
        (void)contributors(ci == 0 ? cut0 : cut1, bf, bl);
        old[ci] = __hip_atomic_fetch_add(p.cnt + bf, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
    for (int ci = 0; ci < 2; ci++)
      if (ci < ncut) {
        int bf, bl;
        const bool last = old[ci] + 1 == (unsigned)contributors(ci == 0 ? cut0 : cut1, bf, bl);
        if (last) __hip_atomic_store(p.cnt + bf, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
        s_last[ci] = last;
      }
  }
  __syncthreads();
  const bool last0 = s_last[0] != 0, last1 = ncut > 1 && s_last[1] != 0;
  // the run's last cut first, while acc may still hold its seed
  for (int r = ncut - 1; r >= 0; r--) {
    const bool seed = seeded && r == ncut - 1;
    if (!(r == 0 ? last0 : last1)) {
      if (seed) zero_acc();
      continue;
    }
    const int item = r == 0 ? cut0 : cut1;
    int bf, bl;
    (void)contributors(item, bf, bl);
    const long lo_f = (long)bf * U / p.nblk, us = (long)item * G2;
    int e, c, q0, q1;
    item_rows(item, e, c, q0, q1);
    (void)e;
    const int nrows = q1 - q0;
    // the pieces in unit order (the seed, when held, is the first), a batch of contributors' loads in flight
    constexpr int FB = MT == 2 ? 2 : 4;
    for (int b0 = seed ? bf + 1 : bf; b0 <= bl; b0 += FB) {
      u32x4 v[FB][NBW][MT][4];
#pragma unroll
      for (int z = 0; z < FB; z++) {
        const int bb = b0 + z;
        const bool has = bb <= bl && (long)(bb + 1) * U / p.nblk > (long)bb * U / p.nblk;
        const int slot = bb == bf && lo_f < us ? 2 * bf + 1 : 2 * bb;
#pragma unroll
        for (int nb = 0; nb < NBW; nb++)
#pragma unroll
          for (int a = 0; a < MT; a++)
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++)
              v[z][nb][a][k4] = has && a * 32 + 8 * k4 + 4 * h < nrows
                                    ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                    rp, piece_off(slot, nb, a, k4), 0, kSc1))
                                    : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int z = 0; z < FB; z++) {
        const int bb = b0 + z;
        if (bb > bl || (long)(bb + 1) * U / p.nblk <= (long)bb * U / p.nblk) continue;  // no piece
#pragma unroll
        for (int nb = 0; nb < NBW; nb++)
#pragma unroll
          for (int a = 0; a < MT; a++)
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++)
#pragma unroll
              for (int x = 0; x < 4; x++) acc[nb][a][4 * k4 + x] += __uint_as_float(v[z][nb][a][k4][x]);
      }
    }
    epilogue(c, q0, q1);  // stores the item and zeroes acc
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// WIDE (plain only): each wave owns two bands, 8 apart, so an item is 16 bands (512 columns)
// BALK: compiled with the balanced schedule (launched when a piece buffer is given and a whole-item run can fall
// kGqMinLoss units behind, K >= 128 kGqMinLoss); otherwise whole items only
template <int MT, bool SILU, bool WIDE, bool BALK>
__global__ __launch_bounds__(kGqThreads, 1) void k_gqmm_t(GqArgs p) {
  constexpr bool TWO = SILU || WIDE;
  static_assert(!(SILU && WIDE), "SwiGLU pairs a gate and an up band per wave");
  static_assert(gq_lds(MT, TWO) <= 160 * 1024, "LDS plan");
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = xcd_remap(blockIdx.x, p.nblk);
  const int nitems = sload(p.ntiles, 0) << p.nct_log2;
  const int G2 = p.G / 2;
  int u0, u1;  // this block's run of (item, group pair) units
  // the balanced schedule where whole-item runs would leave the longest at least kGqMinLoss units past the even
  // share (the fixed cost of the cut items' sums is a few steps); the same decision in every block
  const int per = (nitems + p.nblk - 1) / p.nblk;
  const bool bal = BALK && p.part && (long)per * G2 * p.nblk - (long)nitems * G2 >= (long)kGqMinLoss * p.nblk;
  if (bal) {
    const long U = (long)nitems * G2;
    u0 = (int)((long)b * U / p.nblk), u1 = (int)((long)(b + 1) * U / p.nblk);
  } else {
    u0 = (int)((long)b * nitems / p.nblk) * G2, u1 = (int)((long)(b + 1) * nitems / p.nblk) * G2;
  }
  if (u0 >= u1) return;  // block-uniform, before any barrier
  const bool has_sb = TWO ? wave - 4 < 2 : wave == 7;
  if (BALK && bal) {
    if (wave < 4) gq_role<MT, SILU, WIDE, 0, BALK>(p, lds, wave, b, nitems, u0, u1);
    else if (has_sb) gq_role<MT, SILU, WIDE, 1, BALK>(p, lds, wave, b, nitems, u0, u1);
    else gq_role<MT, SILU, WIDE, 2, BALK>(p, lds, wave, b, nitems, u0, u1);
  } else {
    if (wave < 4) gq_role<MT, SILU, WIDE, 0, false>(p, lds, wave, b, nitems, u0, u1);
    else if (has_sb) gq_role<MT, SILU, WIDE, 1, false>(p, lds, wave, b, nitems, u0, u1);
    else gq_role<MT, SILU, WIDE, 2, false>(p, lds, wave, b, nitems, u0, u1);
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

template <int MT, bool SILU, bool WIDE, bool BALK>
static int launch_gq_kernel(const GqArgs& a, hipStream_t st) {
  constexpr size_t lds = gq_lds(MT, SILU || WIDE);
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)k_gqmm_t<MT, SILU, WIDE, BALK>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr = true;
  }
  hipLaunchKernelGGL((k_gqmm_t<MT, SILU, WIDE, BALK>), dim3(a.nblk), dim3(kGqThreads), lds, st, a);
  return check_launch("moe_gather_qmm_t64");
}
// The units by which the longest whole-item run is expected to exceed the even share, for `rows` sorted rows spread
// uniformly over E experts (Poisson rows per expert, one tile per tile_rows of an expert's rows), nct column tiles
// and G2 group pairs per item, on nblk blocks. The kernel decides on the dispatch's actual item count; this estimate
// only picks which compiled form to launch.
static double gq_expected_loss(int rows, int E, int tile_rows, int nct, int G2, int nblk) {
  const double lam = (double)rows / E;
  double tiles = 0.0, pr = std::exp(-lam);  // P(x) for x = 0, 1, ...
  const int xmax = (int)(lam + 12.0 * std::sqrt(lam) + 30.0);
  for (int x = 0; x <= xmax; x++) {
    tiles += pr * ((x + tile_rows - 1) / tile_rows);
    pr *= lam / (x + 1);
  }
  const double n = tiles * E * nct;
  return std::ceil(n / nblk) * G2 - n * G2 / nblk;
}

template <int MT, bool SILU, bool WIDE>
static int launch_gq_cfg(const GqArgs& a, int rows, hipStream_t st) {
  // the form compiled with the balanced schedule where the kernel is expected to take it (its whole-item path runs
  // slower there than in the form compiled without it); with fewer than kGqMinLoss group pairs per item no
  // whole-item run falls that far behind the even share
  if (a.part && a.G / 2 >= kGqMinLoss &&
      gq_expected_loss(rows, a.E + (a.wsh ? 1 : 0), 32 * MT, 1 << a.nct_log2, a.G / 2, a.nblk) >= kGqMinLoss - 2)
    return launch_gq_kernel<MT, SILU, WIDE, true>(a, st);
  return launch_gq_kernel<MT, SILU, WIDE, false>(a, st);
}

size_t moe_gather_t64_part_bytes(int tile_rows) { return 2 * (size_t)gq_cus() * gq_slot_bytes(tile_rows / 32); }

int launch_moe_gather_qmm_t64(const uint16_t* A, int lda, const int* perm, int div, const int* tiles,
                              const int* ntiles, const int* offsets, int tile_rows, const void* wt, const void* wsh,
                              int E, int N, int K, int silu, uint16_t* C, int ldc, int rows, float* part,
                              size_t part_bytes, unsigned* cnt, hipStream_t st) {
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
  // plain products with output columns in whole 512-column tiles take the wide form (two bands per wave) on 64-row
  // tiles; 32-row tiles (few rows per expert) keep 256-column items, twice as many, which spread more evenly over
  // the CUs (config 4 at T = 128: 238 against 244 us, same box)
  const bool wide = !silu && NO % 512 == 0 && tile_rows == 64;
  const int nct = NO / (wide ? 512 : 256);
  if (nct & (nct - 1)) return fail(IFD_ERR_UNSUPPORTED, "moe_gather_qmm_t64: %d column tiles (not a power of 2)", nct);
  // every perm value is a routed slot below rows, so a sorted row reads one of the first (rows - 1) / div + 1 rows
  const size_t ab = (size_t)(perm ? (rows - 1) / div + 1 : rows) * lda * sizeof(uint16_t);
  if (ab >= ((size_t)1 << 31)) return fail(IFD_ERR_UNSUPPORTED, "moe_gather_qmm_t64: activations past 2 GiB");
  if (t64_bytes(N, K) >= ((size_t)1 << 31)) return fail(IFD_ERR_UNSUPPORTED, "moe_gather_qmm_t64: expert past 2 GiB");
  if (part) {  // the balanced schedule: a piece slot pair per block, a header counter per block
    if (!cnt || part_bytes < moe_gather_t64_part_bytes(tile_rows) || gq_cus() > kWsCounters)
      return fail(IFD_ERR_WORKSPACE, "moe_gather_qmm_t64: %zu bytes of pieces and the counter header needed",
                  moe_gather_t64_part_bytes(tile_rows));
  }
  GqArgs a{A, lda, (uint32_t)ab, perm, div_m, tiles, ntiles, offsets, (const uint8_t*)wt, t64_bytes(N, K),
           (const uint8_t*)wsh, E, N, K, K / kGroup, C, (uint32_t)cb, ldc, __builtin_ctz(nct), gq_cus(),
           part, (uint32_t)(part ? moe_gather_t64_part_bytes(tile_rows) : 0), cnt};
  const int MT = tile_rows / 32;
  if (silu) return MT == 2 ? launch_gq_cfg<2, true, false>(a, rows, st) : launch_gq_cfg<1, true, false>(a, rows, st);
  if (wide) return MT == 2 ? launch_gq_cfg<2, false, true>(a, rows, st) : launch_gq_cfg<1, false, true>(a, rows, st);
  return MT == 2 ? launch_gq_cfg<2, false, false>(a, rows, st) : launch_gq_cfg<1, false, false>(a, rows, st);
}

}  // namespace ifd
