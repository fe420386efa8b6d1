// Decode path (M <= 128 rows of concurrent agents): 4- and 8-bit GEMV/skinny GEMM on bf16 MFMA.
//
// Replaces the reference's qmv4 / qmv8 (engine/kernels/core.metal:85-171, 175-248) and its split-K neighbours (qmm_splitk +
// splitk_reduce, engine/kernels/qmm_splitk.metal:14-107; host choice engine/src/qwen35.h:1520-1556).
//
// Layout per wave: 32 output columns (weight rows n) x a K range; lane l owns column l % 32 and half h = l / 32 of
// every 64-group's codes: 16 bytes (4 bits, words 4h..4h+3 of the group) or 2 x 16 bytes (8 bits, words 4h..4h+3
// and 8+4h..8+4h+3), one or two global_load_dwordx4 per group, each covering 32 contiguous bytes of every row across
// the wave. A 64-group is four 32x32x16 bf16 MFMA steps; in step t the lane supplies eight codes of the group
// (GroupCodes::kofs) and the activation fragment of row m at the same k (16 bytes), so every MFMA stays inside one
// group.
//
// Two variants:
//  * affine (M <= 32): codes enter the MFMA as exact bf16 values, 128 + q (4 bits) or q (8 bits), a second MFMA
//    against ones gives the activation group sums X, and the group epilogue adds s * P + (b - 128 s) * X (4 bits) or
//    s * P + b * X (8 bits) in fp32: the qmv4 / qmv8 arithmetic (s * sum q x + b * sum x, fp32) with fp32 MFMA
//    accumulation.
//  * dequant (32 < M <= 128): codes are dequantized in registers to bf16(s q + b), MLX's qmm rounding
//    (quantized.h:528-535), and accumulate over the whole K range; one dequant feeds all 32-row M tiles.
// Narrow outputs split K over blockIdx.y and write fp32 partials [S][M][N]; k_splitk_reduce applies the store mode.
#include "common.h"
#include "host.h"
#include "kernels.h"

namespace ifd {

struct QmvArgs {
  const uint16_t* A;
  int lda;
  const uint32_t* wq;
  const uint16_t* s;
  const uint16_t* b;
  int N, K, ldk;
  uint32_t xr;
  void* C;
  int ldc, M, mode;
  float* part;  // split partials (gridDim.y > 1)
  int gps;      // 64-groups per split
};

constexpr int kQmvPF = 4;  // groups of weights in flight per lane

template <int RACT, int BITS>
__global__ __launch_bounds__(256) void k_qmv_affine(QmvArgs p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 128 + wave * 32;
  if (n0 >= p.N) return;
  const int n = min(n0 + j, p.N - 1);
  const int G = p.K / kGroup, ldw = p.ldk * BITS / 32, ldg = p.ldk / kGroup;
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps);
  const uint32_t* wrow = p.wq + (size_t)n * ldw + 4 * h;
  const uint16_t* srow = p.s + (size_t)n * ldg;
  const uint16_t* brow = p.b + (size_t)n * ldg;
  const bool aok = j < p.M;
  const uint16_t* arow = p.A + (size_t)(aok ? j : 0) * p.lda;
  const uint32_t xr = p.xr;
  u32x4 ones;
  ones[0] = ones[1] = ones[2] = ones[3] = 0x3F803F80u;  // bf16 1.0 pairs

  f32x16 acc = zero16();
  GroupCodes<BITS> wbuf[kQmvPF];
  uint16_t sbuf[kQmvPF], bbuf[kQmvPF];  // raw bf16 bits: converted at use so the loads stay in flight
#pragma unroll
  for (int i = 0; i < kQmvPF; i++) {
    const int g = g0 + i;
    if (g < g1) {
      wbuf[i].load(wrow, g);
      sbuf[i] = srow[g];
      bbuf[i] = brow[g];
    }
  }
  for (int gb = g0; gb < g1; gb += kQmvPF) {
#pragma unroll
    for (int i = 0; i < kQmvPF; i++) {
      const int g = gb + i;
      if (g >= g1) break;
      const GroupCodes<BITS> wv = wbuf[i];
      const uint16_t sraw = sbuf[i], braw = bbuf[i];
      if (g + kQmvPF < g1) {
        wbuf[i].load(wrow, g + kQmvPF);
        sbuf[i] = srow[g + kQmvPF];
        bbuf[i] = brow[g + kQmvPF];
      }
      u32x4 af[4];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        if (aok) af[t] = *(const u32x4*)(arow + (size_t)g * 64 + GroupCodes<BITS>::kofs(t, h));
        else af[t] = u32x4{0u, 0u, 0u, 0u};
      }
      f32x16 P = zero16(), X = zero16();
#pragma unroll
      for (int t = 0; t < 4; t++) {
        P = mfma_bf16(af[t], wv.step_affine(t, xr), P);
        X = mfma_bf16(af[t], ones, X);
      }
      const float sc = bf2f(sraw), bi = bf2f(braw);
      const float bp = affine_bias<BITS>(sc, bi);
#pragma unroll
      for (int r = 0; r < RACT; r++) acc[r] = __builtin_fmaf(sc, P[r], __builtin_fmaf(bp, X[r], acc[r]));
    }
  }
  const int col = n0 + j;
  if (col >= p.N) return;
  const bool split = gridDim.y > 1;
#pragma unroll
  for (int r = 0; r < RACT; r++) {
    const int row = 8 * (r / 4) + 4 * h + (r % 4);
    if (row >= p.M) continue;
    if (split) p.part[((size_t)blockIdx.y * p.M + row) * p.N + col] = acc[r];
    else store_mode(p.C, (size_t)row * p.ldc + col, acc[r], p.mode);
  }
}

template <int MT, int BITS>
__global__ __launch_bounds__(256) void k_qmv_deq(QmvArgs p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 128 + wave * 32;
  if (n0 >= p.N) return;
  const int n = min(n0 + j, p.N - 1);
  const int G = p.K / kGroup, ldw = p.ldk * BITS / 32, ldg = p.ldk / kGroup;
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps);
  const uint32_t* wrow = p.wq + (size_t)n * ldw + 4 * h;
  const uint16_t* srow = p.s + (size_t)n * ldg;
  const uint16_t* brow = p.b + (size_t)n * ldg;
  const uint16_t* arow[MT];
  bool aok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int m = 32 * mt + j;
    aok[mt] = m < p.M;
    arow[mt] = p.A + (size_t)(aok[mt] ? m : 0) * p.lda;
  }
  const uint32_t xr = p.xr;

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = zero16();
  GroupCodes<BITS> wbuf[kQmvPF];
  uint16_t sbuf[kQmvPF], bbuf[kQmvPF];  // raw bf16 bits: converted at use so the loads stay in flight
#pragma unroll
  for (int i = 0; i < kQmvPF; i++) {
    const int g = g0 + i;
    if (g < g1) {
      wbuf[i].load(wrow, g);
      sbuf[i] = srow[g];
      bbuf[i] = brow[g];
    }
  }
  for (int gb = g0; gb < g1; gb += kQmvPF) {
#pragma unroll
    for (int i = 0; i < kQmvPF; i++) {
      const int g = gb + i;
      if (g >= g1) break;
      const GroupCodes<BITS> wv = wbuf[i];
      const uint16_t sraw = sbuf[i], braw = bbuf[i];
      if (g + kQmvPF < g1) {
        wbuf[i].load(wrow, g + kQmvPF);
        sbuf[i] = srow[g + kQmvPF];
        bbuf[i] = brow[g + kQmvPF];
      }
      const float sc = bf2f(sraw), bi = bf2f(braw);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const u32x4 bfr = wv.step_dequant(t, xr, sc, bi);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
          u32x4 af = u32x4{0u, 0u, 0u, 0u};
          if (aok[mt]) af = *(const u32x4*)(arow[mt] + (size_t)g * 64 + GroupCodes<BITS>::kofs(t, h));
          acc[mt] = mfma_bf16(af, bfr, acc[mt]);
        }
      }
    }
  }
  const int col = n0 + j;
  if (col >= p.N) return;
  const bool split = gridDim.y > 1;
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = 32 * mt + 8 * (r / 4) + 4 * h + (r % 4);
      if (row >= p.M) continue;
      if (split) p.part[((size_t)blockIdx.y * p.M + row) * p.N + col] = acc[mt][r];
      else store_mode(p.C, (size_t)row * p.ldc + col, acc[mt][r], p.mode);
    }
}

// Small-M decode (M <= 16): the block's activation rows for its K range are staged once in LDS together with their
// 64-group sums X; for 4-bit codes the rows are reordered to the (0,4,1,5,2,6,3,7) pair order of
// codes_bf16_off128_p04 (one and-or per code pair), 8-bit codes keep the natural order. Afterwards each wave only
// streams its weights (two 8-group blocks in flight per lane, with the blocks' scales and biases as one 16 B load
// each) and reads activations from LDS, so the weight loads are the only vector-memory traffic in the main loop.
// Requires K % 512 == 0, ldk % 512 == 0, 16-byte aligned scales/biases and splits of whole 8-group blocks.

__device__ __forceinline__ size_t small_lds_x_offset(int M, int Kz) {
  return ((size_t)M * (Kz + 8) * 2 + 15) / 16 * 16;  // bytes: A rows (Kz + 8 bf16 each), then X
}

template <int RACT, int BITS>
__global__ __launch_bounds__(256, 2) void k_qmv_small(QmvArgs p) {
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int G = p.K / kGroup, ldw = p.ldk * BITS / 32, ldg = p.ldk / kGroup;
  const int g0 = blockIdx.y * p.gps, g1 = min(G, g0 + p.gps), Gz = g1 - g0;
  const int Kz = Gz * kGroup, ldA = Kz + 8, M = p.M;
  uint16_t* As = lds;
  float* Xs = (float*)((char*)lds + small_lds_x_offset(M, Kz));  // [Gz][16]

  // ---- stage A[0:M][g0*64 : g1*64] (pair-ordered for 4 bits) and the group sums
  const int cpr = Kz / 8, total = M * cpr;  // 16-byte chunks; a multiple of 8 (one group = 8 chunks)
  for (int c0 = 0; c0 < total; c0 += 256) {
    const int c = c0 + tid;
    const bool ok = c < total;
    const int m = ok ? c / cpr : 0, kc = ok ? c % cpr : 0;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (ok) v = *(const u32x4*)(p.A + (size_t)m * p.lda + (size_t)g0 * kGroup + 8 * kc);
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) sum += bf2f((uint16_t)(v[e] & 0xFFFFu)) + bf2f((uint16_t)(v[e] >> 16));
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    if (ok) {
      *(u32x4*)(As + (size_t)m * ldA + 8 * kc) = BITS == 4 ? perm_pairs04(v) : v;
      if ((kc & 7) == 0) Xs[(kc >> 3) * 16 + m] = sum;
    }
  }
  for (int i = tid; i < Gz * 16; i += 256)
    if ((i & 15) >= M) Xs[i] = 0.f;
  __syncthreads();

  const int n0 = blockIdx.x * 128 + wave * 32;
  if (n0 >= p.N) return;  // no barrier follows
  const int n = min(n0 + j, p.N - 1);
  const uint32_t* wrow = p.wq + (size_t)n * ldw + 4 * h;
  const uint16_t* srow = p.s + (size_t)n * ldg;
  const uint16_t* brow = p.b + (size_t)n * ldg;
  const bool aok = j < M;
  const uint16_t* arow = As + (size_t)(aok ? j : 0) * ldA;
  const uint32_t xr = p.xr;

  f32x16 acc = zero16();
  // Ping-pong register blocks of 8 groups: the lane's codes of 8 groups plus the 8 scales and 8 biases of this
  // column as one 16 B vector each (ldg % 8 == 0, g0 % 8 == 0: checked by the host). Loads land where they are used,
  // so the only waits are for a block issued one block earlier.
  struct Blk {
    GroupCodes<BITS> w[8];
    u32x4 s, b;
  };
  auto load_blk = [&](Blk& B, int g) {
#pragma unroll
    for (int i = 0; i < 8; i++) B.w[i].load(wrow, g + i);
    B.s = *(const u32x4*)(srow + g);
    B.b = *(const u32x4*)(brow + g);
  };
  auto compute_blk = [&](const Blk& B, int g) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int gl = g + i - g0;
      u32x4 af[4];
      const uint16_t* ag = arow + (size_t)gl * 64;
#pragma unroll
      for (int t = 0; t < 4; t++)
        af[t] = aok ? *(const u32x4*)(ag + GroupCodes<BITS>::kofs(t, h)) : u32x4{0u, 0u, 0u, 0u};
      const float4 x0 = *(const float4*)(Xs + gl * 16 + 4 * h);
      float4 x1 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (RACT > 4) x1 = *(const float4*)(Xs + gl * 16 + 8 + 4 * h);
      f32x16 P = zero16();
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const u32x4 bop = BITS == 4 ? codes_bf16_off128_p04(B.w[i].word(t) ^ xr) : B.w[i].step_affine(t, xr);
        P = mfma_bf16(af[t], bop, P);
      }
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      const float sc = bf2f((uint16_t)(B.s[i / 2] >> (16 * (i & 1))));
      const float bi = bf2f((uint16_t)(B.b[i / 2] >> (16 * (i & 1))));
      const float bp = affine_bias<BITS>(sc, bi);
#pragma unroll
      for (int r = 0; r < RACT; r++) acc[r] = __builtin_fmaf(sc, P[r], __builtin_fmaf(bp, xs[r], acc[r]));
    }
  };
  // The prefetches are unconditional (the last block is re-read past the end) so that every path leaves the same
  // number of loads outstanding and the waits can stay one block behind.
  const int glast = g1 - 8;
  Blk b0, b1;
  load_blk(b0, g0);
  for (int g = g0;; g += 16) {
    load_blk(b1, min(g + 8, glast));
    compute_blk(b0, g);
    if (g + 8 >= g1) break;
    load_blk(b0, min(g + 16, glast));
    compute_blk(b1, g + 8);
    if (g + 16 >= g1) break;
  }
  const int col = n0 + j;
  if (col >= p.N) return;
  const bool split = gridDim.y > 1;
#pragma unroll
  for (int r = 0; r < RACT; r++) {
    const int row = 8 * (r / 4) + 4 * h + (r % 4);
    if (row >= M) continue;
    if (split) p.part[((size_t)blockIdx.y * M + row) * p.N + col] = acc[r];
    else store_mode(p.C, (size_t)row * p.ldc + col, acc[r], p.mode);
  }
}

// Sum of the S partials [S][M][N] of V consecutive columns n .. n + V - 1 of row m, in split order.
template <int V>
__device__ __forceinline__ void splitk_sum(const float* __restrict__ part, int S, size_t mn, size_t o, float (&v)[V]) {
#pragma unroll
  for (int e = 0; e < V; e++) v[e] = 0.f;
  for (int z = 0; z < S; z++) {
    const float* q = part + (size_t)z * mn + o;
    if (V == 4) {
      const float4 t = *(const float4*)q;
      v[0] += t.x, v[1] += t.y, v[2] += t.z, v[3] += t.w;
    } else {
#pragma unroll
      for (int e = 0; e < V; e++) v[e] += q[e];
    }
  }
}

// C (mode 0-2) = the split sum; V = 4 columns per thread when N, ldc and C allow vector accesses, else 1.
template <int V>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, int S, int M, int N, void* C,
                                                       int ldc, int mode) {
  const int nv = N / V;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, mn = (size_t)M * N;
  if (i >= (size_t)M * nv) return;
  const int m = (int)(i / nv), n = (int)(i % nv) * V;
  float v[V];
  splitk_sum<V>(part, S, mn, (size_t)m * N + n, v);
  const size_t o = (size_t)m * ldc + n;
  if (V == 4 && mode == 2) {
    *(float4*)((float*)C + o) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (V == 4 && mode == 0) {
    *(uint2*)((uint16_t*)C + o) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
  } else {
#pragma unroll
    for (int e = 0; e < V; e++) store_mode(C, o + e, v[e], mode);
  }
}

// SwiGLU epilogue: N = 2 I partial columns [gate | up]; h[m][i] = swiglu(bf16(sum gate), bf16(sum up)), the bf16
// rounding of each sum being the mode-0 store of the unfused GEMM.
template <int V>
__global__ __launch_bounds__(256) void k_splitk_swiglu(const float* __restrict__ part, int S, int M, int I,
                                                       uint16_t* __restrict__ H, int ldh) {
  const int iv = I / V;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, mn = (size_t)M * 2 * I;
  if (i >= (size_t)M * iv) return;
  const int m = (int)(i / iv), c = (int)(i % iv) * V;
  float g[V], u[V];
  splitk_sum<V>(part, S, mn, (size_t)m * 2 * I + c, g);
  splitk_sum<V>(part, S, mn, (size_t)m * 2 * I + I + c, u);
  float h[V];
#pragma unroll
  for (int e = 0; e < V; e++) h[e] = swiglu_f(bf2f(f2bf(g[e])), bf2f(f2bf(u[e])));
  uint16_t* o = H + (size_t)m * ldh + c;
  if (V == 4) {
    *(uint2*)o = make_uint2(pack_bf2(h[0], h[1]), pack_bf2(h[2], h[3]));
  } else {
#pragma unroll
    for (int e = 0; e < V; e++) o[e] = f2bf(h[e]);
  }
}

int launch_splitk_reduce(const float* part, int S, int M, int N, void* C, int ldc, int mode, hipStream_t st) {
  if (M == 0) return IFD_OK;
  if (mode == kModeSwiglu) {
    const int I = N / 2;
    const bool vec = I % 4 == 0 && ldc % 4 == 0 && ((uintptr_t)C & 7) == 0;
    const size_t n = (size_t)M * (vec ? I / 4 : I);
    if (vec)
      hipLaunchKernelGGL(k_splitk_swiglu<4>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, S, M, I,
                         (uint16_t*)C, ldc);
    else
      hipLaunchKernelGGL(k_splitk_swiglu<1>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, S, M, I,
                         (uint16_t*)C, ldc);
    return check_launch("splitk_swiglu");
  }
  const bool vec = N % 4 == 0 && ldc % 4 == 0 && mode != 1 && ((uintptr_t)C & (mode == 2 ? 15 : 7)) == 0;
  const size_t n = (size_t)M * (vec ? N / 4 : N);
  if (vec)
    hipLaunchKernelGGL(k_splitk_reduce<4>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, S, M, N, C, ldc,
                       mode);
  else
    hipLaunchKernelGGL(k_splitk_reduce<1>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, S, M, N, C, ldc,
                       mode);
  return check_launch("splitk_reduce");
}

size_t epilogue_ws_bytes(int S, int M, int N, int mode) {
  if (S > 1) return (size_t)S * M * N * sizeof(float);
  return mode == kModeSwiglu ? (size_t)M * N * sizeof(uint16_t) : 0;
}

int launch_epilogue(const void* ws, int S, int M, int N, void* C, int ldc, int mode, hipStream_t st) {
  if (S > 1) return launch_splitk_reduce((const float*)ws, S, M, N, C, ldc, mode, st);
  if (mode == kModeSwiglu) return launch_silu_mul((const uint16_t*)ws, N, (uint16_t*)C, ldc, N / 2, M, st);
  return IFD_OK;
}

// K splits for a decode GEMM: enough blocks (~2 per CU on 256 CUs) while every split keeps >= 4 groups and the
// partials stay small (S * M <= 1024 rows, the reference's kSplitRows, qwen35.h:77).
// K split plan for a decode GEMM: enough blocks (~2 per CU on 256 CUs) while every split keeps >= 4 groups and the
// partials stay small (S * M <= 1024 rows, the reference's kSplitRows, qwen35.h:77). With M <= 16 the staged
// activations take at most ~40 KB of LDS per block, and when G % 8 == 0 splits hold whole 8-group blocks.
struct QmvPlan {
  int S, gps;
};
static QmvPlan qmv_plan(int M, int N, int K) {
  const int G = K / kGroup, bx = (N + 127) / 128;
  long S = (512 + bx - 1) / bx;
  if (M <= 16) S = std::max<long>(S, ((long)M * K * 2 + 40959) / 40960);
  S = std::min<long>(S, std::max(1, G / 4));
  S = std::min<long>(S, std::max(1, 1024 / std::max(M, 1)));
  int gps = (int)((G + S - 1) / S);
  if (M <= 16 && G % 8 == 0) gps = (gps + 7) / 8 * 8;
  return QmvPlan{(G + gps - 1) / gps, gps};
}

size_t qmv_workspace(int M, int N, int K) {
  const QmvPlan pl = qmv_plan(M, N, K);
  return pl.S > 1 ? (size_t)pl.S * M * N * sizeof(float) : 0;
}

int launch_qmv(const W4Gemm& g, void* ws, size_t ws_bytes, hipStream_t st) {
  if (g.M == 0) return IFD_OK;
  if (g.M > 128) return fail(IFD_ERR_ARG, "qmv path takes M <= 128 (M=%d)", g.M);
  const QmvPlan pl = qmv_plan(g.M, g.N, g.K);
  const int S = pl.S, gps = pl.gps;
  const size_t need = S > 1 ? (size_t)S * g.M * g.N * sizeof(float) : 0;
  if (need > ws_bytes || (need && !ws))
    return fail(IFD_ERR_WORKSPACE, "qmv needs %zu bytes of workspace, got %zu", need, ws_bytes);
  QmvArgs p{(const uint16_t*)g.A, g.lda, g.wq, g.s, g.b, g.N, g.K, g.ldk, g.xr, g.C, g.ldc, g.M, g.mode,
            (float*)ws, gps};
  dim3 grid((g.N + 127) / 128, S), block(256);
  const bool small_ok = g.M <= 16 && g.K % 512 == 0 && g.ldk % 512 == 0 && gps % 8 == 0 && aligned(g.s, 16) &&
                        aligned(g.b, 16);
  if (small_ok) {
    const int Kz = gps * kGroup;
    const size_t lds = ((size_t)g.M * (Kz + 8) * 2 + 15) / 16 * 16 + (size_t)gps * 16 * sizeof(float);
    if (lds > 64 * 1024) return fail(IFD_ERR_UNSUPPORTED, "qmv: %zu bytes of LDS needed", lds);
    if (g.bits == 8) {
      if (g.M <= 8) hipLaunchKernelGGL((k_qmv_small<4, 8>), grid, block, lds, st, p);
      else hipLaunchKernelGGL((k_qmv_small<8, 8>), grid, block, lds, st, p);
    } else {
      if (g.M <= 8) hipLaunchKernelGGL((k_qmv_small<4, 4>), grid, block, lds, st, p);
      else hipLaunchKernelGGL((k_qmv_small<8, 4>), grid, block, lds, st, p);
    }
  } else if (g.bits == 8) {
    if (g.M <= 8) hipLaunchKernelGGL((k_qmv_affine<4, 8>), grid, block, 0, st, p);
    else if (g.M <= 16) hipLaunchKernelGGL((k_qmv_affine<8, 8>), grid, block, 0, st, p);
    else if (g.M <= 32) hipLaunchKernelGGL((k_qmv_affine<16, 8>), grid, block, 0, st, p);
    else if (g.M <= 64) hipLaunchKernelGGL((k_qmv_deq<2, 8>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((k_qmv_deq<4, 8>), grid, block, 0, st, p);
  } else if (g.M <= 8) {
    hipLaunchKernelGGL((k_qmv_affine<4, 4>), grid, block, 0, st, p);
  } else if (g.M <= 16) {
    hipLaunchKernelGGL((k_qmv_affine<8, 4>), grid, block, 0, st, p);
  } else if (g.M <= 32) {
    hipLaunchKernelGGL((k_qmv_affine<16, 4>), grid, block, 0, st, p);
  } else if (g.M <= 64) {
    hipLaunchKernelGGL((k_qmv_deq<2, 4>), grid, block, 0, st, p);
  } else {
    hipLaunchKernelGGL((k_qmv_deq<4, 4>), grid, block, 0, st, p);
  }
  IFD_TRY(check_launch("qmv"));
  if (S > 1) return launch_splitk_reduce((const float*)ws, S, g.M, g.N, g.C, g.ldc, g.mode, st);
  return IFD_OK;
}

}  // namespace ifd
