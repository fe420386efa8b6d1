// W8A8 on T64x8 weights (t64.h) with per-token int8 activations, on int8 MFMA; and the T64x8 repack.
//
// Replaces the reference's w4a8_gemm instantiated with BITS = 8 (engine/kernels/w4a8.metal:43-98; the 8-bit offset
// 128 at :57, the identity :8 and epilogue :78-87):
//   y[m][n] = sx[m] * sum_g ( s_g[n] * P_g[m][n] + b'_g[n] * X_g[m] ),  P_g = sum_{k in g} (q - 128) xq,
//   b' = b + 128 s,  X_g = sum_{k in g} xq
// with q the unflipped 8-bit code, xq the int8 activation and sx the row's scale. T64x8 stores q - 128 as int8, so
// the codes are B fragments as they stand: no unpack.
//
// The kernel is stream-K over units (128-row x 256-column tile, 64-group), one block per CU, as the 4-bit W4A8
// stream-K kernel (w4a8_t64.hip) with single-group steps: the first q nblk = (T / nblk) nblk tiles are whole-tile
// work (block b takes tiles b q .. b q + q - 1); the other nsk = T % nblk tiles are split: block b takes their units
// [b U / nblk, (b + 1) U / nblk), U = nsk G, first. Pieces of cut tiles go to the block's two partial slots
// (unscaled fp32 sums in MFMA fragment order) and k_sk_fixup (gemm_sk.hip) sums each cut tile's pieces in unit order,
// applies sx and stores it.
//
// Block: 8 waves, two per SIMD; wave w owns band w (32 columns) over the 4 M tiles of 32 rows. Per step and M tile:
// two v_mfma_i32_32x32x32_i8 give the group's exact P, acc += s float(P) (two VALU per accumulator), and b' X_g
// enters acc through one bf16 MFMA whose only non-zero k slots are (X_hi, X_lo, X_hi, X_lo) against
// (b'_hi, b'_hi, b'_lo, b'_lo): X = X_hi + X_lo and b' = b'_hi + b'_lo are exact / near-exact bf16 pairs.
// One LDS ring of kW8R stages filled by direct global -> LDS DMA; a stage holds a group's activation slab [128][64]
// (16-byte columns XOR-swizzled by row quad), the 8 bands' code tiles, their (s, b) rows and the X pairs of the 128
// rows (16-byte slots from k_w8a8_xprep). Every wave issues its slab rows and its band's two code halves; wave 0 also
// the (s, b) rows and the first 64 rows' X slots, wave 1 the other 64 rows' X slots. They are buffer loads with a
// scalar group offset, and each role's code is compiled on its own, so every wait is a constant. Past the run's last
// unit the stream re-issues that unit (bytes already in L2) so that the count holds to the last step.
#include <algorithm>

#include "common.h"
#include "dma.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"

namespace ifd {

// ---- repack ------------------------------------------------------------------------------------------------------
// One thread per (group, band, lane): two 16-byte code fragments (q ^ 0x80 of the unflipped codes) and, for h == 0,
// the row's (s, b) dword. xr is the source's flip mask (0, or 0x80808080 for flipped 8-bit weights).
__global__ __launch_bounds__(256) void k_pack_t64x8(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ s,
                                                    const uint16_t* __restrict__ b, int N, int K, int ldk,
                                                    uint32_t xr, uint8_t* __restrict__ out) {
  const int G = K / kGroup, nb = t64_bands(N), ldw = ldk / 4, ldg = ldk / kGroup;
  const size_t total = (size_t)G * nb * 64;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i % 64), band = (int)(i / 64 % nb), g = (int)(i / 64 / nb);
  const int j = lane & 31, h = lane >> 5, n = band * 32 + j;
  uint8_t* tile = out + ((size_t)g * nb + band) * kT64x8Tile;
  u32x4 v[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
  uint32_t sb = 0;
  if (n < N) {
    const uint32_t* src = wq + (size_t)n * ldw + (size_t)g * 16 + 8 * h;
    const uint32_t x = xr ^ 0x80808080u;
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
      for (int t = 0; t < 4; t++) v[s2][t] = src[4 * s2 + t] ^ x;
    sb = (uint32_t)s[(size_t)n * ldg + g] | ((uint32_t)b[(size_t)n * ldg + g] << 16);
  }
  *(u32x4*)(tile + 16 * lane) = v[0];
  *(u32x4*)(tile + 1024 + 16 * lane) = v[1];
  if (h == 0) *(uint32_t*)(tile + kT64x8Codes + 4 * j) = sb;
}

int launch_pack_t64x8(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr,
                      void* out, hipStream_t st) {
  const size_t total = (size_t)(K / kGroup) * t64_bands(N) * 64;
  if (total == 0) return IFD_OK;
  hipLaunchKernelGGL(k_pack_t64x8, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, wq, s, b, N, K, ldk, xr,
                     (uint8_t*)out);
  return check_launch("pack_t64x8");
}

// ---- W8A8 stream-K -----------------------------------------------------------------------------------------------
constexpr int kW8R = 5;
constexpr int kW8A = 128 * 64;
constexpr int kW8C = 8 * kT64x8Codes;
constexpr int kW8SB = 1024;
constexpr int kW8X = 2048;
constexpr int kW8Stage = kW8A + kW8C + kW8SB + kW8X;
constexpr int kW8Row = 256 + 4;  // staged tile row stride (floats)
constexpr size_t kW8Lds = (size_t)kW8R * kW8Stage > (size_t)128 * kW8Row * 4 ? (size_t)kW8R * kW8Stage
                                                                             : (size_t)128 * kW8Row * 4;
static_assert(kW8Lds <= 160 * 1024, "LDS plan");

struct W8A8SkArgs {
  const int8_t* U;       // [M][K]
  const float* XS;       // [M][G][2]
  const u32x4* Xt;       // [G][Mx]: (pair, pair, 0, 0), pair = bf16 X_hi | bf16 X_lo << 16; rows past M zero
  int Mx;
  const uint8_t* wt;
  uint32_t w_bytes, u_bytes, x_bytes;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;
  uint32_t part_bytes;
  int tiles_m, tiles_n, G, nblk;
  int q, tile0, nsk;  // whole tiles per block; the stream-K tiles tile0 .. tile0 + nsk - 1
};

// X_g of (row, group) recovered exactly from XS = (sx, sx X_g) and split as X_hi = 256 floor(X / 256), X_lo =
// X - X_hi (both exact in bf16, |X| <= 8192); Xt[g][m] = (pair, pair, 0, 0), zero for m >= M.
__global__ __launch_bounds__(256) void k_w8a8_xprep(const float* __restrict__ XS, int M, int G, int Mx,
                                                    u32x4* __restrict__ Xt) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)G * Mx) return;
  const int g = (int)(i / Mx), m = (int)(i % Mx);
  uint32_t v = 0;
  if (m < M) {
    const float x = rintf(XS[((size_t)m * G + g) * 2 + 1] / XS[((size_t)m * G + g) * 2]);
    const float hi = floorf(x * (1.f / 256.f)) * 256.f;
    v = (uint32_t)f2bf(hi) | (uint32_t)f2bf(x - hi) << 16;
  }
  Xt[i] = u32x4{v, v, 0u, 0u};
}

__device__ __forceinline__ void w8_dma(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, (int)voff, (int)soff, 0, 0);
}

// ROLE 0: wave 0 (also the (s, b) rows and the X slots of rows 0-63), 1: wave 1 (X slots of rows 64-127),
// 2: waves 2-7.
template <int ROLE>
__device__ __forceinline__ void w8_body(const W8A8SkArgs& p, uint8_t* lds, const int wave, const int b) {
  constexpr int R = kW8R, D = ROLE == 0 ? 5 : ROLE == 1 ? 4 : 3;
  static_assert(R >= 4 && (R - 2) * D <= 63, "ring depth, vmcnt range");
  float* const stg = (float*)lds;  // staged tile [128][kW8Row], after the K loop
  const int tid = threadIdx.x, lane = tid & 63;
  const int j = lane & 31, h = lane >> 5;
  const int G = p.G;
  const long Usk = (long)p.nsk * G;
  const int ur0 = (int)((long)b * Usk / p.nblk), ur1 = (int)((long)(b + 1) * Usk / p.nblk);
  const int nr = ur1 - ur0, n = nr + p.q * G;
  const int nbands = t64_bands(p.N);
  const uint32_t gstride = (uint32_t)nbands * kT64x8Tile;

  // unit i of the run -> (tile, group)
  auto unit = [&](int i, int& tile, int& g) __attribute__((always_inline)) {
    if (i < nr) {
      tile = p.tile0 + (ur0 + i) / G, g = (ur0 + i) % G;
    } else {
      tile = b * p.q + (i - nr) / G, g = (i - nr) % G;
    }
  };

  const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc((void*)p.U, 0, (int)p.u_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)p.wt, 0, (int)p.w_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)p.Xt, 0, (int)p.x_bytes, 0x00020000);

  // ---- the DMA stream: per-lane offsets of the current tile, the group in a scalar
  uint32_t va, vw, v3 = 0, vx = 0;
  auto set_tile = [&](int tile) __attribute__((always_inline)) {
    const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
    const int r = 16 * wave + lane / 4;  // slab row of this lane's 16 bytes
    va = (uint32_t)min(tm * 128 + r, p.M - 1) * (uint32_t)p.K + 16u * ((lane & 3) ^ ((r >> 2) & 3));
    vw = (uint32_t)min(8 * tn + wave, nbands - 1) * kT64x8Tile + 16u * lane;
    if constexpr (ROLE == 0)
      v3 = (uint32_t)min(8 * tn + lane / 8, nbands - 1) * kT64x8Tile + kT64x8Codes + 16u * (lane & 7);
    vx = (uint32_t)(tm * 128 + 64 * ROLE) * 16u + 16u * lane;
  };
  int s_i = 0, s_tile, s_g;
  unit(0, s_tile, s_g);
  set_tile(s_tile);
  auto issue = [&](int slot) __attribute__((always_inline)) {
    uint8_t* st = lds + slot * kW8Stage;
    const uint32_t w_so = (uint32_t)s_g * gstride;
    w8_dma(ru, st + wave * 1024, va, (uint32_t)s_g * 64u);
    w8_dma(rw, st + kW8A + wave * kT64x8Codes, vw, w_so);
    w8_dma(rw, st + kW8A + wave * kT64x8Codes + 1024, vw + 1024u, w_so);
    if constexpr (ROLE == 0) w8_dma(rw, st + kW8A + kW8C, v3, w_so);
    if constexpr (ROLE < 2)
      w8_dma(rx, st + kW8A + kW8C + kW8SB + ROLE * 1024, vx, (uint32_t)s_g * (uint32_t)p.Mx * 16u);
  };
  auto advance = [&]() __attribute__((always_inline)) {
    if (s_i >= n - 1) return;  // past the run's last unit the stream re-reads it
    s_i++;
    if (++s_g == G || s_i == nr) {
      unit(s_i, s_tile, s_g);
      set_tile(s_tile);
    }
  };

  f32x16 acc[4];
#pragma unroll
  for (int a = 0; a < 4; a++) acc[a] = zero16();

  // The operands of one step, read from its stage one step ahead of their use.
  struct Ops {
    u32x4 a[4][2];  // activation fragments of the 4 M tiles (k = 32 h + 16 s2 + 0..15 at index s2)
    u32x4 bq[2];    // the band's B fragments, as stored
    float sc;       // the column's scale
    u32x4 xb;       // (b'_hi, b'_hi, b'_lo, b'_lo) in k slots 0..3 for the lanes h = 0, else 0
    u32x4 xv[4];    // the X slot of row a 32 + j
  };
  auto read_a = [&](const uint8_t* st, int a, Ops& o) __attribute__((always_inline)) {
    const int r = a * 32 + j;
    o.a[a][0] = *(const u32x4*)(st + r * 64 + 16 * ((2 * h) ^ ((r >> 2) & 3)));
    o.a[a][1] = *(const u32x4*)(st + r * 64 + 16 * ((2 * h + 1) ^ ((r >> 2) & 3)));
    o.xv[a] = *(const u32x4*)(st + kW8A + kW8C + kW8SB + 16 * r);
  };
  // b' = b + 128 s in fp32 (the reference's bw), split as b'_hi = bf16(b'), b'_lo = bf16(b' - b'_hi)
  auto finish = [&](const uint32_t sb, Ops& o) __attribute__((always_inline)) {
    const float sc = bf2f((uint16_t)(sb & 0xFFFFu));
    const float bw = bf2f((uint16_t)(sb >> 16)) + 128.f * sc;
    const uint32_t hi = f2bf(bw), lo = f2bf(bw - bf2f((uint16_t)hi));
    o.sc = sc;
    o.xb = h ? u32x4{0u, 0u, 0u, 0u} : u32x4{hi | hi << 16, lo | lo << 16, 0u, 0u};
  };
  auto read_w = [&](const uint8_t* st, Ops& o, uint32_t& sb) __attribute__((always_inline)) {
    o.bq[0] = *(const u32x4*)(st + kW8A + wave * kT64x8Codes + 16 * lane);
    o.bq[1] = *(const u32x4*)(st + kW8A + wave * kT64x8Codes + 1024 + 16 * lane);
    sb = *(const uint32_t*)(st + kW8A + kW8C + wave * 128 + 4 * j);
  };
  auto read_all = [&](int slot, Ops& o) __attribute__((always_inline)) {
    const uint8_t* st = lds + slot * kW8Stage;
    uint32_t sb;
    read_w(st, o, sb);
#pragma unroll
    for (int a = 0; a < 4; a++) read_a(st, a, o);
    finish(sb, o);
  };

  // Step i: cu holds step i's operands. Waits for stage i + 1 (R - 3 younger stages in flight), issues stage
  // i + R - 1 into the stage read at step i - 1, then per M tile a: the two i8 MFMAs of P, the bias MFMA, step
  // i + 1's fragments of tile a, and the epilogue of tile a - 1 (P double-buffered).
  auto step = [&](int i, Ops& cu, Ops& nx) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((R - 3) * D) : "memory");
    const int slot = i % R;
    issue(slot == 0 ? R - 1 : slot - 1);
    advance();
    const uint8_t* st = lds + (slot + 1 == R ? 0 : slot + 1) * kW8Stage;
    uint32_t sb;
    read_w(st, nx, sb);
    i32x16 P[2];
#pragma unroll
    for (int a = 0; a < 4; a++) {
      P[a & 1] = mfma_i8(cu.a[a][0], cu.bq[0], izero16());
      P[a & 1] = mfma_i8(cu.a[a][1], cu.bq[1], P[a & 1]);
      acc[a] = mfma_bf16(cu.xv[a], cu.xb, acc[a]);
      read_a(st, a, nx);
      if (a > 0) {
#pragma unroll
        for (int e = 0; e < 16; e++) acc[a - 1][e] = __builtin_fmaf(cu.sc, (float)P[(a - 1) & 1][e], acc[a - 1][e]);
      }
    }
#pragma unroll
    for (int e = 0; e < 16; e++) acc[3][e] = __builtin_fmaf(cu.sc, (float)P[1][e], acc[3][e]);
    finish(sb, nx);
  };

  // prologue: stages 0 .. R - 2 issued, stage 0 read
#pragma unroll
  for (int k = 0; k < R - 1; k++) {
    issue(k);
    advance();
  }
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((R - 2) * D) : "memory");
  Ops o0, o1;
  read_all(0, o0);

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
    const int len = i < nr ? min(G - g, nr - i) : G;
    int k = i;
    for (; k + 1 < i + len; k += 2) {
      step(k, o0, o1);
      step(k + 1, o1, o0);
    }
    if (k < i + len) {
      step(k, o0, o1);
      o0 = o1;
    }
    i += len;
    whole = len == G;
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
    for (int e = 0; e < 16; e++) stg[(a * 32 + 8 * (e / 4) + 4 * h + (e % 4)) * kW8Row + 32 * wave + j] = acc[a][e];
  __syncthreads();
  const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
  for (int e = tid; e < 128 * 64; e += 512) {
    const int row = e >> 6, c4 = (e & 63) * 4, grow = tm * 128 + row, gcol = tn * 256 + c4;
    if (grow >= p.M || gcol >= p.N) continue;
    const float sx = p.XS[(size_t)grow * G * 2];
    const float4 v4 = *(const float4*)(stg + row * kW8Row + c4);
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

__global__ __launch_bounds__(512, 1) void k_w8a8_sk(W8A8SkArgs p) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = xcd_remap(blockIdx.x, p.nblk);
  if (wave == 0) w8_body<0>(p, lds, wave, b);
  else if (wave == 1) w8_body<1>(p, lds, wave, b);
  else w8_body<2>(p, lds, wave, b);
}

// Stream-K plan: q whole tiles per block, the last T % nblk tiles split over the blocks
struct W8Plan {
  int tiles_m, tiles_n, G, nblk, q, tile0, nsk, Mx;
};
static W8Plan w8a8_plan(int M, int N, int K) {
  W8Plan pl{};
  pl.tiles_m = (M + 127) / 128;
  pl.tiles_n = (t64_bands(N) + 7) / 8;
  pl.G = K / kGroup;
  pl.Mx = pl.tiles_m * 128;
  const int tiles = pl.tiles_m * pl.tiles_n, cus = cu_count();
  pl.q = tiles / cus;
  pl.nsk = tiles - pl.q * cus;
  pl.tile0 = pl.q * cus;
  // with no whole tiles, never more blocks than units
  pl.nblk = pl.q ? cus : std::min(cus, pl.nsk * pl.G);
  return pl;
}
static size_t w8_xt_bytes(const W8Plan& pl) { return align_up((size_t)pl.G * pl.Mx * 16, 256); }
static size_t w8_part_bytes(const W8Plan& pl) { return pl.nsk ? (size_t)2 * pl.nblk * 8 * 16 * 64 * 16 : 0; }

size_t w8a8_t_workspace(int M, int N, int K) {
  const W8Plan pl = w8a8_plan(M, N, K);
  return w8_xt_bytes(pl) + w8_part_bytes(pl);
}

int launch_w8a8_t(const int8_t* U, const float* XS, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                  void* ws, size_t ws_bytes, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (K % kGroup) return fail(IFD_ERR_ARG, "T64x8 W8A8 needs K %% 64 == 0 (K=%d)", K);
  const W8Plan pl = w8a8_plan(M, N, K);
  const size_t need = w8_xt_bytes(pl) + w8_part_bytes(pl);
  if (need > ws_bytes || !ws)
    return fail(IFD_ERR_WORKSPACE, "w8a8_t64x8 needs %zu bytes of workspace, got %zu", need, ws_bytes);
  if (t64x8_bytes(N, K) >= ((size_t)1 << 31) || (size_t)M * K >= ((size_t)1 << 31) ||
      w8_xt_bytes(pl) >= ((size_t)1 << 31) || w8_part_bytes(pl) >= ((size_t)1 << 31) ||
      ((uint64_t)pl.nsk * pl.G + 1) * (pl.nblk + 1) >= ((uint64_t)1 << 32))
    return fail(IFD_ERR_UNSUPPORTED, "w8a8_t64x8: operands past 2 GiB");
  u32x4* Xt = (u32x4*)ws;
  float* part = (float*)((char*)ws + w8_xt_bytes(pl));
  const size_t nx = (size_t)pl.G * pl.Mx;
  hipLaunchKernelGGL(k_w8a8_xprep, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, st, XS, M, pl.G, pl.Mx, Xt);
  IFD_TRY(check_launch("w8a8_xprep"));
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)k_w8a8_sk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kW8Lds);
    attr = true;
  }
  W8A8SkArgs a{U, XS, Xt, pl.Mx, (const uint8_t*)wt, (uint32_t)t64x8_bytes(N, K), (uint32_t)((size_t)M * K),
               (uint32_t)(nx * 16), N, K, C, ldc, M, mode, part, (uint32_t)w8_part_bytes(pl), pl.tiles_m, pl.tiles_n,
               pl.G, pl.nblk, pl.q, pl.tile0, pl.nsk};
  hipLaunchKernelGGL(k_w8a8_sk, dim3(pl.nblk), dim3(512), kW8Lds, st, a);
  IFD_TRY(check_launch("w8a8_sk"));
  if (!pl.nsk) return IFD_OK;
  // the fixup runs when some stream-K tile is cut between blocks
  const long U2 = (long)pl.nsk * pl.G;
  bool cut = false;
  for (long t = 0; t < pl.nsk && !cut; t++)
    cut = (t * pl.G * pl.nblk + pl.nblk - 1) / U2 != ((t * pl.G + pl.G - 1) * pl.nblk + pl.nblk - 1) / U2;
  if (!cut) return IFD_OK;
  return launch_sk_fixup_rows(part, pl.tiles_m, pl.tiles_n, pl.tile0, pl.nsk, pl.G, pl.nblk, C, ldc, M, N, mode, XS,
                              2 * pl.G, st);
}

}  // namespace ifd
