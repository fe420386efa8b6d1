// T64-layout kernels: the repack from the reference layout and the decode GEMV on T64 weights (and, with BITS = 8,
// on T64x8 weights).
//
// The decode kernel computes what the reference's qmv4 computes (engine/kernels/core.metal:85-171): per 64-group
// s * sum q x + b * sum x in fp32, here with the products on bf16 MFMA (codes enter as exact bf16 (128 + q)) and the
// group epilogue s * P + (b - 128 s) * X in fp32.
#include "common.h"
#include "host.h"
#include "kernels.h"
#include "t64.h"

namespace ifd {

// ---- repack ------------------------------------------------------------------------------------------------------
// One thread per (expert, group, band, lane): 16 bytes of codes (unflipped, T64 nibble order) and, for h == 0, the
// row's (s, b) dword.
__global__ __launch_bounds__(256) void k_pack_t64(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ s,
                                                  const uint16_t* __restrict__ b, int N, int K, int ldk, uint32_t xr,
                                                  int E, uint8_t* __restrict__ out) {
  const int G = K / kGroup, nb = t64_bands(N), ldw = ldk / 8, ldg = ldk / kGroup;
  const size_t total = (size_t)E * G * nb * 64;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i % 64), band = (int)(i / 64 % nb), g = (int)(i / 64 / nb % G), e = (int)(i / 64 / nb / G);
  const int j = lane & 31, h = lane >> 5, n = band * 32 + j;
  uint8_t* tile = out + (size_t)e * t64_bytes(N, K) + ((size_t)g * nb + band) * kT64Tile;
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  uint32_t sb = 0;
  if (n < N) {
    const size_t row = (size_t)e * N + n;
    const uint32_t* src = wq + row * ldw + (size_t)g * 8 + 4 * h;
#pragma unroll
    for (int t = 0; t < 4; t++) v[t] = t64_word(src[t] ^ xr);
    sb = (uint32_t)s[row * ldg + g] | ((uint32_t)b[row * ldg + g] << 16);
  }
  *(u32x4*)(tile + 16 * lane) = v;
  if (h == 0) *(uint32_t*)(tile + kT64Codes + 4 * j) = sb;
}

int launch_pack_t64(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int ldk, uint32_t xr,
                    int E, void* out, hipStream_t st) {
  const size_t total = (size_t)E * (K / kGroup) * t64_bands(N) * 64;
  if (total == 0) return IFD_OK;
  hipLaunchKernelGGL(k_pack_t64, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, wq, s, b, N, K, ldk, xr, E,
                     (uint8_t*)out);
  return check_launch("pack_t64");
}

// ---- decode GEMV, M <= 16 --------------------------------------------------------------------------------------
// Block: 256 threads = 4 waves = 4 bands (128 output columns) x one K split. The activation rows of the split are
// staged once in LDS (natural order) with their 64-group sums; then each wave streams its band's tiles in
// ping-pong blocks of kTB groups (one 16-byte code load + one (s, b) dword per lane per group) and reads
// activations from LDS. Prefetch loads are unconditional (the last block is re-read past the end) so every path
// leaves the same number of loads outstanding and the waits stay one block behind.
// With a K split the blocks store fp32 partials [S][M][N]; given completion counters (the workspace header), the
// last block to finish a 128-column tile sums its S partials in split order and stores the result (SwiGLU mode:
// gate tile t and up tile t + sw_half share one counter, and the last of their 2 S blocks writes h), so no
// reduction kernel follows. The sums are those of k_splitk_reduce / k_splitk_swiglu, bit for bit.
// MULTI: several linears that share A and K in one launch. Linear l owns the global bands band0[l] ..
// band0[l + 1] - 1, each linear's count rounded up to whole blocks of 4, so a block never spans two linears. The
// split partials and the fixup's counters run over the global columns (N = 32 band0[n]); the stores go to each
// linear's own output.
constexpr int kQmvMulti = 8;
struct QmvTMulti {
  int n;
  int band0[kQmvMulti + 1];
  const uint8_t* wt[kQmvMulti];
  void* C[kQmvMulti];
  int ldc[kQmvMulti], N[kQmvMulti];
};

struct QmvTArgs {
  const uint16_t* A;
  int lda;
  const uint8_t* wt;
  int N, K;
  void* C;
  int ldc, M, mode;
  float* part;
  uint32_t part_bytes;
  unsigned* cnt;  // null: partials only, a reduction kernel follows
  int sw_half;    // SwiGLU fixup: number of gate column tiles (0: plain store mode)
  int gps;
  const float* XS;  // A8: the rows' (sx, sx sum xq) per 64-group [M][K / 64][2] (A holds xq as bf16 integers)
  QmvTMulti mt;     // MULTI only
};

constexpr int kTB = 2;     // groups per pipeline block
constexpr int kMaxS = 16;  // K splits at most
#ifndef QMV_FIXB
#define QMV_FIXB 8
#endif
constexpr int kFixB = QMV_FIXB;  // partial loads in flight per thread in the split-K fixup

__device__ __forceinline__ u32x4 t64_bf16_off128(uint32_t w) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; i++) r[i] = ((w >> (4 * i)) & 0x000F000Fu) | 0x43004300u;  // (q_2i, q_2i+1) + 128
  return r;
}


// BITS = 8: T64x8 tiles (two 1 KB code halves per lane group; the exact q as bf16 and the bias b, the reference's
// qmv8 arithmetic s * sum q x + b * sum x, core.metal:175-248).
// A8: the reference's W4A8 GEMM with per-(row, 64-group) int8 activations (w4a8.metal:24-98): A holds xq as exact
// bf16 integers, so P and the group sums X are exact integers, and per group acc += sx (s P + (b - 128 s) X), the
// row's group scale sx staged beside X.
template <int RACT, int BITS, bool A8 = false, bool MULTI = false>
__global__ __launch_bounds__(256, 2) void k_qmv_t(QmvTArgs p) {
  constexpr int NH = BITS / 4, TILEB = BITS == 8 ? kT64x8Tile : kT64Tile, CODES = BITS == 8 ? kT64x8Codes : kT64Codes;
  extern __shared__ __align__(16) uint16_t lds[];
  __shared__ unsigned s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  // this block's linear (MULTI): its weights, output and column count; gb0 its first global band
  const uint8_t* wbase = p.wt;
  void* Cl = p.C;
  int ldcl = p.ldc, Nl = p.N, gb0 = 0;
  if constexpr (MULTI) {
    int lin = 0;
    for (int l = 1; l < p.mt.n; l++) lin += (int)blockIdx.x * 4 >= p.mt.band0[l];
    wbase = p.mt.wt[lin], Cl = p.mt.C[lin], ldcl = p.mt.ldc[lin], Nl = p.mt.N[lin], gb0 = p.mt.band0[lin];
  }
  const int G = p.K / kGroup, nb = t64_bands(Nl);
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps), Gz = g1 - g0;
  const int Kz = Gz * kGroup, ldA = Kz + 8, M = p.M;
  uint16_t* As = lds;
  float* Xs = (float*)((char*)lds + ((size_t)M * ldA * 2 + 15) / 16 * 16);  // [Gz][16]
  float* Ss = Xs + (size_t)Gz * 16;                                          // A8: [Gz][16] sx

  // this wave's band; its first block of tiles is requested before the activations are staged, so the weight
  // stream starts one memory latency earlier
  const int band = blockIdx.x * 4 + wave - gb0;  // the linear's band
  const bool live = band < nb;
  const uint8_t* tcol = wbase + (size_t)(live ? band : 0) * TILEB;  // + g * nb * TILEB
  const size_t gstride = (size_t)nb * TILEB;
  struct Blk {
    u32x4 w[kTB][NH];
    uint32_t sb[kTB];
  };
  auto load_blk = [&](Blk& B, int g) {
#pragma unroll
    for (int i = 0; i < kTB; i++) {
      const uint8_t* t = tcol + (size_t)(g + i) * gstride;
#pragma unroll
      // streamed once: non-temporal loads (measured 2-3% faster on the gate_up and down shapes at M = 1)
      for (int hh = 0; hh < NH; hh++) B.w[i][hh] = __builtin_nontemporal_load((const u32x4*)(t + 1024 * hh + 16 * lane));
      B.sb[i] = __builtin_nontemporal_load((const uint32_t*)(t + CODES + 4 * j));
    }
  };
  Blk b0, b1;
  if (live) load_blk(b0, g0);

  // ---- stage A[0:M][g0*64 : g1*64] and the 64-group sums; kStageU 16-byte chunks per thread are loaded before any
  // is used (one memory latency per kStageU passes); 8 consecutive threads hold one row's 64-group
  constexpr int kStageU = 4;
  const int cpr = Kz / 8, total = M * cpr;
  for (int c0 = 0; c0 < total; c0 += 256 * kStageU) {
    u32x4 v[kStageU];
#pragma unroll
    for (int u = 0; u < kStageU; u++) {
      const int c = c0 + 256 * u + tid;
      v[u] = u32x4{0u, 0u, 0u, 0u};
      if (c < total) v[u] = *(const u32x4*)(p.A + (size_t)(c / cpr) * p.lda + (size_t)g0 * kGroup + 8 * (c % cpr));
    }
#pragma unroll
    for (int u = 0; u < kStageU; u++) {
      const int c = c0 + 256 * u + tid;
      const bool ok = c < total;
      const int m = ok ? c / cpr : 0, kc = ok ? c % cpr : 0;
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 4; e++) sum += bf2f((uint16_t)(v[u][e] & 0xFFFFu)) + bf2f((uint16_t)(v[u][e] >> 16));
      sum += __shfl_xor(sum, 1, 64);
      sum += __shfl_xor(sum, 2, 64);
      sum += __shfl_xor(sum, 4, 64);
      if (ok) {
        *(u32x4*)(As + (size_t)m * ldA + 8 * kc) = v[u];
        if ((kc & 7) == 0) Xs[(kc >> 3) * 16 + m] = sum;
      }
    }
  }
  for (int i = tid; i < Gz * 16; i += 256) {
    const int m = i & 15, gl = i >> 4;
    if (m >= M) Xs[i] = 0.f;
    if constexpr (A8) Ss[i] = m < M ? p.XS[((size_t)m * G + g0 + gl) * 2] : 0.f;
  }
  __syncthreads();

  const bool aok = j < M;
  const uint16_t* arow = As + (size_t)(aok ? j : 0) * ldA + 32 * h;

  f32x16 acc = zero16();
  auto compute_blk = [&](const Blk& B, int g) {
#pragma unroll
    for (int i = 0; i < kTB; i++) {
      const int gl = g + i - g0;
      u32x4 af[4];
      const uint16_t* ag = arow + (size_t)gl * 64;
#pragma unroll
      for (int t = 0; t < 4; t++) af[t] = aok ? *(const u32x4*)(ag + 8 * t) : u32x4{0u, 0u, 0u, 0u};
      const float4 x0 = *(const float4*)(Xs + gl * 16 + 4 * h);
      float4 x1 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (RACT > 4) x1 = *(const float4*)(Xs + gl * 16 + 8 + 4 * h);
      f32x16 P = zero16();
#pragma unroll
      for (int t = 0; t < 4; t++) {
        // MFMA step t: codes of k = 32 h + 8 t .. + 7 as exact bf16, 128 + q (4 bits) or q (8 bits: byte ^ 0x80)
        const u32x4 bq = BITS == 4 ? t64_bf16_off128(B.w[i][0][t])
                                   : codes8_bf16(B.w[i][t / 2 % NH][2 * (t % 2)] ^ 0x80808080u,
                                                 B.w[i][t / 2 % NH][2 * (t % 2) + 1] ^ 0x80808080u);
        P = mfma_bf16(af[t], bq, P);
      }
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      const float sc = bf2f((uint16_t)(B.sb[i] & 0xFFFFu)), bi = bf2f((uint16_t)(B.sb[i] >> 16));
      const float bp = BITS == 4 ? __builtin_fmaf(-128.f, sc, bi) : bi;
      if constexpr (A8) {
        const float4 s0 = *(const float4*)(Ss + gl * 16 + 4 * h);
        float4 s1 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (RACT > 4) s1 = *(const float4*)(Ss + gl * 16 + 8 + 4 * h);
        const float ss[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int r = 0; r < RACT; r++) acc[r] = __builtin_fmaf(ss[r], __builtin_fmaf(sc, P[r], bp * xs[r]), acc[r]);
      } else {
#pragma unroll
        for (int r = 0; r < RACT; r++) acc[r] = __builtin_fmaf(sc, P[r], __builtin_fmaf(bp, xs[r], acc[r]));
      }
    }
  };
  if (live) {  // waves past the last band skip the stream but take part in the fixup's barriers
    const int glast = g1 - kTB;
    for (int g = g0;; g += 2 * kTB) {
      load_blk(b1, min(g + kTB, glast));
      compute_blk(b0, g);
      if (g + kTB >= g1) break;
      load_blk(b0, min(g + 2 * kTB, glast));
      compute_blk(b1, g + kTB);
      if (g + 2 * kTB >= g1) break;
    }
  }
  const int col = band * 32 + j, gcol = (gb0 + band) * 32 + j;  // the linear's column, the global column
  if (gridDim.y == 1) {
    if (!live || col >= Nl) return;
#pragma unroll
    for (int r = 0; r < RACT; r++) {
      const int row = 8 * (r / 4) + 4 * h + (r % 4);
      if (row < M) store_mode(Cl, (size_t)row * ldcl + col, acc[r], p.mode);
    }
    return;
  }

  // ---- K split: partials, then (with counters) the fixup by the tile's last block
  const __amdgpu_buffer_rsrc_t rs = part_rsrc(p.part, p.part_bytes);
  if (live && col < Nl) {
#pragma unroll
    for (int r = 0; r < RACT; r++) {
      const int row = 8 * (r / 4) + 4 * h + (r % 4);
      if (row < M)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[r]),  rs,
                                              (int)((((size_t)blockIdx.y * M + row) * p.N + gcol) * 4), 0, kSc1);
    }
  }
  if (!p.cnt) return;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are complete (written through)
  __syncthreads();
  const int tile = p.sw_half ? (int)blockIdx.x % p.sw_half : (int)blockIdx.x;
  const unsigned arrivals = (p.sw_half ? 2u : 1u) * gridDim.y;
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(p.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == arrivals;
    if (last) __hip_atomic_store(p.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next call
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  const int S = (int)gridDim.y;
  const size_t mn = (size_t)M * p.N;
  // four columns of one row per thread and pass (16-byte partial loads, N % 4 == 0), the loads of kFixB splits in
  // flight at once (their registers count against the occupancy the stream needs), summed in split order
  auto sum4 = [&](size_t o) {
    float4 acc4 = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z0 = 0; z0 < S; z0 += kFixB) {
      u32x4 v[kFixB];
#pragma unroll
      for (int z = 0; z < kFixB; z++)
        if (z0 + z < S)
          v[z] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rs, (int)(((z0 + z) * mn + o) * 4), 0, kSc1));
#pragma unroll
      for (int z = 0; z < kFixB; z++)
        if (z0 + z < S) {
          acc4.x += __uint_as_float(v[z][0]);
          acc4.y += __uint_as_float(v[z][1]);
          acc4.z += __uint_as_float(v[z][2]);
          acc4.w += __uint_as_float(v[z][3]);
        }
    }
    return acc4;
  };
  for (int e = tid; e < M * 32; e += 256) {
    const int row = e >> 5, c4 = (e & 31) * 4;
    if (!p.sw_half) {
      const int c = (int)blockIdx.x * 128 + c4, cl = c - 32 * gb0;  // global, and the linear's column
      if (cl >= Nl) continue;
      const float4 v = sum4((size_t)row * p.N + c);
      const size_t o = (size_t)row * ldcl + cl;
      // a linear of the multi-linear launch may end inside the quad (its N need not be a multiple of 4)
      store_mode(Cl, o, v.x, p.mode);
      if (cl + 1 < Nl) store_mode(Cl, o + 1, v.y, p.mode);
      if (cl + 2 < Nl) store_mode(Cl, o + 2, v.z, p.mode);
      if (cl + 3 < Nl) store_mode(Cl, o + 3, v.w, p.mode);
    } else {
      const int I = p.N / 2, c = tile * 128 + c4;
      const float4 g = sum4((size_t)row * p.N + c), u = sum4((size_t)row * p.N + I + c);
      uint16_t* o = (uint16_t*)p.C + (size_t)row * p.ldc + c;
      o[0] = f2bf(swiglu_f(bf2f(f2bf(g.x)), bf2f(f2bf(u.x))));
      o[1] = f2bf(swiglu_f(bf2f(f2bf(g.y)), bf2f(f2bf(u.y))));
      o[2] = f2bf(swiglu_f(bf2f(f2bf(g.z)), bf2f(f2bf(u.z))));
      o[3] = f2bf(swiglu_f(bf2f(f2bf(g.w)), bf2f(f2bf(u.w))));
    }
  }
}

// Split plan: enough waves for the bytes in flight (the stream is latency-bound): about 6 per SIMD for weights past
// 64 MB, 2 below, where each split's fixed costs (its activation staging, partial store and the last block's reads)
// outweigh the extra waves (measured: K = N = 5120, 10.2 -> 9.5 us; the 50 MB down, 15.5 -> 14.7 us; the 100 MB
// gate_up is fastest at 6); whole kTB-group blocks of at least two per split, at most kMaxS splits, <= ~40 KB of
// staged activations per block.
struct TPlan {
  int S, gps;
};
static TPlan qmv_t_plan(int M, int N, int K, int bits = 4) {
  const int G = K / kGroup, waves = 4 * ((t64_bands(N) + 3) / 4);
  const long target = (long)N * K / 8 * bits <= (64l << 20) ? 2048 : 6144;
  long S = (target + waves - 1) / waves;
  S = std::max<long>(S, ((long)M * K * 2 + 40959) / 40960);
  S = std::min<long>(S, std::max(1, G / (2 * kTB)));
  S = std::min<long>(S, kMaxS);
  int gps = (int)((G + S - 1) / S);
  gps = (gps + kTB - 1) / kTB * kTB;
  return TPlan{(G + gps - 1) / gps, gps};
}

// The in-kernel fixup applies with counters for every tile and rows of whole 16-byte partial quads (N % 4 == 0); the
// SwiGLU pairing needs gate and up halves of whole 128-column tiles.
static bool qmv_t_fixup(int N, int mode, int S) {
  const int tiles = (t64_bands(N) + 3) / 4;
  if (S <= 1 || tiles > kWsCounters || N % 4) return false;
  return mode != kModeSwiglu || (N % 256 == 0);
}

size_t qmv_t_workspace(int M, int N, int K, int mode, int bits) {
  if (M > 16) return 0;
  return epilogue_ws_bytes(qmv_t_plan(M, N, K, bits).S, M, N, mode);
}

template <int BITS, bool A8 = false>
static int launch_qmv_t_bits(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M,
                             int mode, unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st,
                             const float* XS = nullptr) {
  if (M == 0) return IFD_OK;
  if (M > 16) return fail(IFD_ERR_UNSUPPORTED, "T64 decode kernel takes M <= 16");
  if (K % (kGroup * kTB)) return fail(IFD_ERR_ARG, "T64 decode needs K %% %d == 0 (K=%d)", kGroup * kTB, K);
  const TPlan pl = qmv_t_plan(M, N, K, BITS);
  const size_t need = epilogue_ws_bytes(pl.S, M, N, mode);
  if (need > ws_bytes || (need && !ws))
    return fail(IFD_ERR_WORKSPACE, "qmv_t64 needs %zu bytes of workspace, got %zu", need, ws_bytes);
  const bool fix = cnt && qmv_t_fixup(N, mode, pl.S);
  // the SwiGLU mode without a split stores the bf16 product into the workspace for silu_mul
  const bool via_ws = mode == kModeSwiglu && pl.S == 1;
  QmvTArgs p{A,
             lda,
             (const uint8_t*)wt,
             N,
             K,
             via_ws ? ws : C,
             via_ws ? N : ldc,
             M,
             via_ws ? 0 : mode,
             (float*)ws,
             (uint32_t)(pl.S > 1 ? need : 0),
             fix ? cnt : nullptr,
             fix && mode == kModeSwiglu ? (t64_bands(N) + 3) / 4 / 2 : 0,
             pl.gps,
             XS,
             {}};
  const int Kz = pl.gps * kGroup;
  const size_t lds =
      ((size_t)M * (Kz + 8) * 2 + 15) / 16 * 16 + (size_t)pl.gps * 16 * sizeof(float) * (A8 ? 2 : 1);
  if (lds > 64 * 1024) return fail(IFD_ERR_UNSUPPORTED, "qmv_t64: %zu bytes of LDS needed", lds);
  dim3 grid((t64_bands(N) + 3) / 4, pl.S), block(256);
  if (M <= 8) hipLaunchKernelGGL((k_qmv_t<4, BITS, A8>), grid, block, lds, st, p);
  else hipLaunchKernelGGL((k_qmv_t<8, BITS, A8>), grid, block, lds, st, p);
  IFD_TRY(check_launch("qmv_t64"));
  if (fix) return IFD_OK;
  return launch_epilogue(ws, pl.S, M, N, C, ldc, mode, st);
}

// Several linears sharing A and K (M <= 16, modes 0-2): the decode GEMV over their concatenated bands in one launch.
// Its K split is planned for the concatenated width and summed in-kernel (counters required when it splits).
size_t qmv_t_multi_workspace(int M, int n, const int* Ns, int K) {
  int bands = 0;
  for (int l = 0; l < n; l++) bands += (t64_bands(Ns[l]) + 3) / 4 * 4;
  return qmv_t_workspace(M, 32 * bands, K, 0);
}
int launch_qmv_t_multi(const uint16_t* A, int lda, int n, const void* const* wts, const int* Ns, int K,
                       void* const* Cs, const int* ldcs, int M, int mode, unsigned* cnt, void* ws, size_t ws_bytes,
                       hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (M > 16) return fail(IFD_ERR_UNSUPPORTED, "T64 multi-linear GEMV takes M <= 16");
  if (n < 1 || n > kQmvMulti) return fail(IFD_ERR_ARG, "T64 multi-linear GEMV: n=%d linears (1 to %d)", n, kQmvMulti);
  if (K % (kGroup * kTB)) return fail(IFD_ERR_ARG, "T64 decode needs K %% %d == 0 (K=%d)", kGroup * kTB, K);
  if (mode == kModeSwiglu) return fail(IFD_ERR_UNSUPPORTED, "T64 multi-linear GEMV: modes 0-2");
  QmvTMulti mt{};
  mt.n = n;
  int bands = 0;
  for (int l = 0; l < n; l++) {
    mt.band0[l] = bands;
    mt.wt[l] = (const uint8_t*)wts[l], mt.C[l] = Cs[l], mt.ldc[l] = ldcs[l], mt.N[l] = Ns[l];
    bands += (t64_bands(Ns[l]) + 3) / 4 * 4;
  }
  mt.band0[n] = bands;
  const int Ntot = 32 * bands;
  const TPlan pl = qmv_t_plan(M, Ntot, K);
  const size_t need = epilogue_ws_bytes(pl.S, M, Ntot, mode);
  if (need > ws_bytes || (need && !ws))
    return fail(IFD_ERR_WORKSPACE, "qmv_t64 multi needs %zu bytes of workspace, got %zu", need, ws_bytes);
  if (pl.S > 1 && !(cnt && qmv_t_fixup(Ntot, mode, pl.S)))
    return fail(IFD_ERR_WORKSPACE, "qmv_t64 multi: a split launch needs the workspace's counter header");
  QmvTArgs p{A, lda, nullptr, Ntot, K, nullptr, 0, M, mode, (float*)ws, (uint32_t)(pl.S > 1 ? need : 0),
             pl.S > 1 ? cnt : nullptr, 0, pl.gps, nullptr, mt};
  const size_t lds = ((size_t)M * (pl.gps * kGroup + 8) * 2 + 15) / 16 * 16 + (size_t)pl.gps * 16 * sizeof(float);
  if (lds > 64 * 1024) return fail(IFD_ERR_UNSUPPORTED, "qmv_t64 multi: %zu bytes of LDS needed", lds);
  dim3 grid(bands / 4, pl.S), block(256);
  if (M <= 8) hipLaunchKernelGGL((k_qmv_t<4, 4, false, true>), grid, block, lds, st, p);
  else hipLaunchKernelGGL((k_qmv_t<8, 4, false, true>), grid, block, lds, st, p);
  return check_launch("qmv_t64 multi");
}

int launch_qmv_t(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                 unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st) {
  return launch_qmv_t_bits<4>(A, lda, wt, N, K, C, ldc, M, mode, cnt, ws, ws_bytes, st);
}

int launch_qmv_t8(const uint16_t* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                  unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st) {
  return launch_qmv_t_bits<8>(A, lda, wt, N, K, C, ldc, M, mode, cnt, ws, ws_bytes, st);
}

// The W4A8 form of the decode GEMV (per-group int8 activations): Ab = xq as bf16 integers [M][K], XS their
// (sx, sx sum xq) per group.
int launch_qmv_t_a8(const uint16_t* Ab, const float* XS, const void* wt, int N, int K, void* C, int ldc, int M,
                    int mode, unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st) {
  if (mode == kModeSwiglu) return fail(IFD_ERR_UNSUPPORTED, "T64 W4A8: no SwiGLU mode");
  return launch_qmv_t_bits<4, true>(Ab, K, wt, N, K, C, ldc, M, mode, cnt, ws, ws_bytes, st, XS);
}

}  // namespace ifd
