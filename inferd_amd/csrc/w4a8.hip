// W4A8 / W8A8: int8 activations x the checkpoint's 4- or 8-bit weights on int8 MFMA, plus the elementwise kernels of
// the path (activation quantizer, in-place flip, SwiGLU).
//
// Replaces the reference's a8_quant + w4a8_gemm (engine/kernels/w4a8.metal:24-98; host w4a8,
// engine/src/qwen35.h:1323-1366), w_flip (w4a8.metal:19-22) and silu_mul (engine/kernels/core.metal:777-787).
//
// Per 64-group g the GEMM forms the exact int32 P = sum_k q[n,k] xq[m,k] (q unsigned 0..15 after undoing a flip)
// on v_mfma_i32_32x32x32_i8, then applies the affine correction in fp32:
//   y[m,n] += s[n,g] sx[m,g] P + b[n,g] (sx[m,g] sum_k xq[m,k])
// which is the reference's identity (w4a8.metal:7-8) written with unsigned codes. With per-token scales (sx constant
// along the row) sx is factored out of the group loop.
// Block: 256 threads (2 x 2 waves), tile 128 x 128, one group per step, int8 tiles and the group's (s, b) / XS
// staged in LDS, double-buffered.
#include "common.h"
#include "host.h"
#include "kernels.h"

namespace ifd {

// ---- activation quantizer --------------------------------------------------------------------------------------
// One block of 256 threads per row. form 1: amax over the row; 0: per 64-group. sx = amax / 127 (1 if 0),
// xq = rint(x / sx) (IEEE division and round-half-even: bit-identical to the CPU reference), XS = (sx, sx * sum xq).
// form 2 (the reference's qa8_quant, qa8.metal:30-49): per 64-group, xq = clamp(rint(x * (127 / amax)), +-127) (0
// when amax == 0), XS = (amax / 127, amax / 127 * sum xq); stored in natural K order.
// Lane layout: a lane takes 8 consecutive elements (one 16-byte load), so 8 consecutive lanes hold one 64-group and
// a wave 8 groups per pass. The group max and sum are three DPP steps within those 8 lanes (quad swaps, then the
// half-row mirror). The group max is exact in any order, and so is the fp32 sum of 64 integer codes (|sum| <= 8128):
// the bits do not depend on the layout. (One element per lane and a 64-lane shuffle reduction per group left each
// wave bound by the reductions' latency.)
template <class Op>
__device__ __forceinline__ float dpp_reduce8_f(float v, Op op) {
  v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false)));  // quad_perm 1,0,3,2
  v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false)));  // quad_perm 2,3,0,1
  v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false)));  // row_half_mirror
  return v;
}
__global__ __launch_bounds__(256) void k_a8_quant(const uint16_t* __restrict__ A, int lda, int K, int form,
                                                  int8_t* __restrict__ U, float* __restrict__ XS) {
  const int per_token = form == 1;
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* a = A + (size_t)m * lda;
  const int G = K / kGroup, nc = K / 8;  // 16-byte chunks; chunk c is part c % 8 of group c / 8
  auto fmax_op = [](float x, float y) { return fmaxf(x, y); };
  auto add_op = [](float x, float y) { return x + y; };
  auto unpack = [](const u32x4& w, float (&x)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      x[2 * e] = __uint_as_float(w[e] << 16);
      x[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
    }
  };
  float row_sx = 1.f;
  if (per_token) {
    float mx = 0.f;
    for (int c = tid; c < nc; c += 256) {
      float x[8];
      unpack(*(const u32x4*)(a + 8 * c), x);
#pragma unroll
      for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(x[e]));
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    row_sx = mx > 0.f ? mx / 127.f : 1.f;
  }
  // a pass covers 256 chunks = 32 groups; the 8 lanes of a group are live or not together (nc % 8 == 0)
  for (int c = tid; c < nc; c += 256) {
    float x[8];
    unpack(*(const u32x4*)(a + 8 * c), x);
    float sx = row_sx, q[8];
    if (form == 2) {
      float amax = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(x[e]));
      amax = dpp_reduce8_f(amax, fmax_op);
      const float inv = amax > 0.f ? 127.f / amax : 0.f;
#pragma unroll
      for (int e = 0; e < 8; e++) q[e] = fminf(fmaxf(rintf(x[e] * inv), -127.f), 127.f);
      sx = amax / 127.f;
    } else {
      if (!per_token) {
        float amax = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(x[e]));
        amax = dpp_reduce8_f(amax, fmax_op);
        sx = amax > 0.f ? amax / 127.f : 1.f;
      }
#pragma unroll
      for (int e = 0; e < 8; e++) q[e] = rintf(x[e] / sx);
    }
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      lo |= ((uint32_t)(int)q[e] & 0xFFu) << (8 * e);
      hi |= ((uint32_t)(int)q[4 + e] & 0xFFu) << (8 * e);
    }
    *(uint2*)(U + (size_t)m * K + 8 * c) = make_uint2(lo, hi);
    float qs = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) qs += q[e];
    qs = dpp_reduce8_f(qs, add_op);
    if ((c & 7) == 0) {
      const int g = c >> 3;
      XS[((size_t)m * G + g) * 2] = sx;
      XS[((size_t)m * G + g) * 2 + 1] = sx * qs;
    }
  }
}

int launch_a8_quant(const uint16_t* A, int lda, int M, int K, int form, int8_t* U, float* XS, hipStream_t st) {
  if (M == 0) return IFD_OK;
  hipLaunchKernelGGL(k_a8_quant, dim3(M), dim3(256), 0, st, A, lda, K, form, U, XS);
  return check_launch("a8_quant");
}

// ---- flip / SwiGLU ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_flip(uint32_t* wq, size_t n32, uint32_t mask) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n32) wq[i] ^= mask;
}
int launch_flip(uint32_t* wq, size_t n32, uint32_t mask, hipStream_t st) {
  if (n32 == 0) return IFD_OK;
  hipLaunchKernelGGL(k_flip, dim3((unsigned)((n32 + 255) / 256)), dim3(256), 0, st, wq, n32, mask);
  return check_launch("flip");
}

// h = bf16(float(bf16(g / (1 + exp(-g)))) * u), 8 values per thread; rows of gu are ldgu apart (gate at 0, up at I),
// rows of h ldh apart (I, ldgu and ldh multiples of 8).
__global__ __launch_bounds__(256) void k_silu_mul(const uint16_t* __restrict__ gu, int ldgu, uint16_t* __restrict__ h,
                                                  int ldh, int I, int rows) {
  const int per_row = I / 8;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)rows * per_row) return;
  const int r = (int)(i / per_row), c = (int)(i % per_row) * 8;
  const u32x4 gv = *(const u32x4*)(gu + (size_t)r * ldgu + c);
  const u32x4 uv = *(const u32x4*)(gu + (size_t)r * ldgu + I + c);
  u32x4 o;
#pragma unroll
  for (int t = 0; t < 4; t++)
    o[t] = pack_bf2(swiglu_f(bf2f((uint16_t)gv[t]), bf2f((uint16_t)uv[t])),
                    swiglu_f(bf2f((uint16_t)(gv[t] >> 16)), bf2f((uint16_t)(uv[t] >> 16))));
  *(u32x4*)(h + (size_t)r * ldh + c) = o;
}
int launch_silu_mul(const uint16_t* gu, int ldgu, uint16_t* h, int ldh, int I, int rows, hipStream_t st) {
  if (rows == 0) return IFD_OK;
  const size_t n = (size_t)rows * (I / 8);
  hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, gu, ldgu, h, ldh, I, rows);
  return check_launch("silu_mul");
}

// RMS norm, one block per row: out = bf16(float(x) * rsqrt(sum x^2 / D + eps) * float(w)), fp32 sum of squares
// (reference rmsnorm, core.metal:486-500).
__global__ __launch_bounds__(256) void k_rmsnorm(const uint16_t* __restrict__ x, int in_stride,
                                                 const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                 int out_stride, int D, float eps) {
  __shared__ float red[4];
  const uint16_t* xr = x + (size_t)blockIdx.x * in_stride;
  const float ss = wave_sum(row_sumsq256(xr, D));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float r = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
  row_norm_store256(xr, w, out + (size_t)blockIdx.x * out_stride, D, r);
}
int launch_rmsnorm(const uint16_t* x, int in_stride, const uint16_t* w, uint16_t* out, int out_stride, int rows,
                   int D, float eps, hipStream_t st) {
  if (rows == 0) return IFD_OK;
  hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, st, x, in_stride, w, out, out_stride, D, eps);
  return check_launch("rmsnorm");
}

// ---- W4A8 GEMM -------------------------------------------------------------------------------------------------
constexpr int kA8BM = 128, kA8BN = 128, kA8Ld = 80;  // LDS row: 64 int8 + 16 pad
constexpr int kA8Band = 4;

struct W4A8Args {
  const int8_t* U;
  const float* XS;
  const uint32_t* wq;
  const uint16_t* s;
  const uint16_t* b;
  int N, K, ldk;
  uint32_t xr;
  void* C;
  int ldc, M, mode;
  int tiles_m, tiles_n;
};

// BITS 4: codes 0..15 enter the int8 MFMA as they are; BITS 8: as signed q - 128 (the stored byte ^ 0x80 once the
// flip is undone), with the bias b + 128 s (reference w4a8_gemm BITS = 8, w4a8.metal:57, 78-87).
template <bool PT, int BITS>
__global__ __launch_bounds__(256) void k_w4a8(W4A8Args p) {
  __shared__ __align__(16) int8_t Us[2][kA8BM * kA8Ld];
  __shared__ __align__(16) int8_t Ws[2][kA8BN * kA8Ld];
  __shared__ __align__(16) float Sb[2][kA8BN][2];   // (s, b) of the group per column
  __shared__ __align__(16) float Xq[2][kA8BM][2];   // (sx, sx * sum xq) of the group per row
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;

  const int ntiles = p.tiles_m * p.tiles_n;
  const int L = xcd_remap(blockIdx.x, ntiles);
  const int per_band = kA8Band * p.tiles_n;
  const int band = L / per_band, within = L % per_band;
  const int bm = min(kA8Band, p.tiles_m - band * kA8Band);
  const int tm = band * kA8Band + within % bm, tn = within / bm;
  const int m0 = tm * kA8BM, n0 = tn * kA8BN;
  const int G = p.K / kGroup, ldw = p.ldk * BITS / 32, ldg = p.ldk / kGroup;

  // activation tile: 128 rows x 64 B, two 16 B chunks per thread: c = tid + 256 i -> row c / 4, part c % 4
  const int8_t* uptr[2];
  bool uok[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int c = tid + 256 * i, m = m0 + (c >> 2);
    uok[i] = m < p.M;
    uptr[i] = p.U + (size_t)(uok[i] ? m : 0) * p.K + 16 * (c & 3);
  }
  // weight tile: row tid / 2, half tid % 2 (32 codes = BITS words)
  const int wr = tid >> 1, wh = tid & 1;
  const int nw = min(n0 + wr, p.N - 1);
  const uint32_t* wptr = p.wq + (size_t)nw * ldw + 4 * wh;
  const uint16_t* sptr = p.s + (size_t)nw * ldg;
  const uint16_t* bptr = p.b + (size_t)nw * ldg;
  const int xm = min(m0 + (tid & 127), max(p.M - 1, 0));

  u32x4 ureg[2];
  GroupCodes<BITS> wreg;
  uint32_t sbreg = 0;
  float xsreg[2] = {0.f, 0.f};
  auto gload = [&](int g) {
#pragma unroll
    for (int i = 0; i < 2; i++) ureg[i] = uok[i] ? *(const u32x4*)(uptr[i] + (size_t)g * 64) : u32x4{0u, 0u, 0u, 0u};
    wreg.load(wptr, g);
    if (wh == 0) sbreg = (uint32_t)sptr[g] | ((uint32_t)bptr[g] << 16);
    if (tid < 128) {
      xsreg[0] = p.XS[((size_t)xm * G + g) * 2];
      xsreg[1] = p.XS[((size_t)xm * G + g) * 2 + 1];
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int c = tid + 256 * i;
      *(u32x4*)(&Us[buf][(c >> 2) * kA8Ld + 16 * (c & 3)]) = ureg[i];
    }
    int8_t* ws = &Ws[buf][wr * kA8Ld];
    if (BITS == 4) {
#pragma unroll
      for (int t = 0; t < 4; t++) *(u32x2*)(ws + 32 * wh + 8 * t) = codes_i8(wreg.word(t) ^ p.xr);
    } else {
      const uint32_t sx = p.xr ^ 0x80808080u;  // stored byte -> q - 128 as int8
#pragma unroll
      for (int i = 0; i < 2; i++) *(u32x4*)(ws + 32 * i + 16 * wh) = wreg.w[i % (BITS / 4)] ^ u32x4{sx, sx, sx, sx};
    }
    if (wh == 0) {
      Sb[buf][wr][0] = bf2f((uint16_t)(sbreg & 0xFFFFu));
      Sb[buf][wr][1] = bf2f((uint16_t)(sbreg >> 16));
    }
    if (tid < 128) {
      Xq[buf][tid][0] = xsreg[0];
      // per-token: the exact integer sum xq (|sum| <= 8128), sx is applied once after the loop
      Xq[buf][tid][1] = PT ? rintf(xsreg[1] / xsreg[0]) : xsreg[1];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int c = 0; c < 2; c++) acc[a][c] = zero16();

  gload(0);
  lstore(0);
  __syncthreads();
  for (int g = 0; g < G; g++) {
    const int buf = g & 1;
    if (g + 1 < G) gload(g + 1);
    const int8_t* us = &Us[buf][(wm * 64 + j) * kA8Ld + 16 * h];
    const int8_t* ws = &Ws[buf][(wn * 64 + j) * kA8Ld + 16 * h];
    i32x16 P[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
      for (int c = 0; c < 2; c++) P[a][c] = izero16();
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      u32x4 af[2], bf[2];
#pragma unroll
      for (int a = 0; a < 2; a++) af[a] = *(const u32x4*)(us + a * 32 * kA8Ld + 32 * kk);
#pragma unroll
      for (int c = 0; c < 2; c++) bf[c] = *(const u32x4*)(ws + c * 32 * kA8Ld + 32 * kk);
#pragma unroll
      for (int a = 0; a < 2; a++)
#pragma unroll
        for (int c = 0; c < 2; c++) P[a][c] = mfma_i8(af[a], bf[c], P[a][c]);
    }
    // epilogue of the group
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const float sc = Sb[buf][wn * 64 + 32 * c + j][0];
      const float bi = BITS == 4 ? Sb[buf][wn * 64 + 32 * c + j][1] : __builtin_fmaf(128.f, sc, Sb[buf][wn * 64 + 32 * c + j][1]);
#pragma unroll
      for (int a = 0; a < 2; a++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
          const int row = wm * 64 + 32 * a + 8 * r4 + 4 * h;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float sx = Xq[buf][row + e][0], sq = Xq[buf][row + e][1];
            const float pf = (float)P[a][c][4 * r4 + e];
            float v = acc[a][c][4 * r4 + e];
            if (PT) v = __builtin_fmaf(sc, pf, v);  // y / sx = sum_g s P + b sum xq
            else v = __builtin_fmaf(sx, sc * pf, v);
            acc[a][c][4 * r4 + e] = __builtin_fmaf(bi, sq, v);
          }
        }
    }
    if (g + 1 < G) lstore(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m0 + wm * 64 + 32 * a + 8 * (r / 4) + 4 * h + (r % 4);
      if (row >= p.M) continue;
      const float sx = PT ? p.XS[(size_t)row * G * 2] : 1.f;
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int col = n0 + wn * 64 + 32 * c + j;
        if (col >= p.N) continue;
        store_mode(p.C, (size_t)row * p.ldc + col, PT ? sx * acc[a][c][r] : acc[a][c][r], p.mode);
      }
    }
}

size_t w4a8_workspace(int, int, int) { return 0; }

int launch_w4a8(const W4Gemm& g, int per_token, void*, size_t, hipStream_t st) {
  if (g.M == 0) return IFD_OK;
  W4A8Args p{(const int8_t*)g.A, g.XS, g.wq, g.s, g.b, g.N, g.K, g.ldk, g.xr, g.C, g.ldc, g.M, g.mode,
             (g.M + kA8BM - 1) / kA8BM, (g.N + kA8BN - 1) / kA8BN};
  const dim3 grid(p.tiles_m * p.tiles_n);
  if (g.bits == 8) {
    if (per_token) hipLaunchKernelGGL((k_w4a8<true, 8>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((k_w4a8<false, 8>), grid, dim3(256), 0, st, p);
  } else {
    if (per_token) hipLaunchKernelGGL((k_w4a8<true, 4>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((k_w4a8<false, 4>), grid, dim3(256), 0, st, p);
  }
  return check_launch("w4a8");
}

}  // namespace ifd
