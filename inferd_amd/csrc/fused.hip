// Fused producers around the GEMMs of the decode step: the norm or activation that feeds a W4A8 GEMM also writes its
// int8 activations, and a deferred split-K residual reduce runs inside the next norm. Each is bit-identical to its
// unfused sequence of this library's kernels (k_splitk_reduce, k_rmsnorm, k_silu_mul, k_a8_quant).
//
// One block of 256 threads per row (per 2048-column chunk of a row for the per-group silu_mul_a8). Thread t takes
// elements t + 256 k (as k_rmsnorm), so wave w of pass k covers the 64 consecutive elements of group 4 k + w: the
// per-group amax and code sums of the W4A8 quantization stay inside one wave, and no thread reads an element another
// thread wrote.
#include "common.h"
#include "host.h"
#include "kernels.h"

namespace ifd {

// Block-wide sum / max over the 4 waves of a 256-thread block (wave order, as k_rmsnorm / k_a8_quant).
__device__ __forceinline__ float block_sum4(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float s = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return s;
}
__device__ __forceinline__ float block_max4(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return m;
}

// W4A8 activation quantization of one row (reference a8_quant, engine/kernels/w4a8.metal:24-41): value(i) gives the
// bf16-rounded activation of element i (as fp32). Per group: sx = amax / 127 (1 when 0), q = rint(v / sx), XS = (sx,
// sx * sum q); per token: one amax over the row.
template <bool PT, class F>
__device__ __forceinline__ void quant_row(F value, int D, float* red, int8_t* U, float* XS) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // 8 elements' values per thread at a time, at clamped indices, ahead of the reductions, which use DPP (as
  // k_a8_quant: the group max and the fp32 sum of 64 integer codes are exact in any order)
  float row_sx = 1.f;
  if (PT) {
    float mx = 0.f;
    for (int i0 = 0; i0 < D; i0 += 256 * 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = value(min(i0 + 256 * j + tid, D - 1));
#pragma unroll
      for (int j = 0; j < 8; j++)
        if (i0 + 256 * j + tid < D) mx = fmaxf(mx, fabsf(v[j]));
    }
    mx = block_max4(mx, red);
    row_sx = mx > 0.f ? mx / 127.f : 1.f;
  }
  for (int i00 = 0; i00 < D; i00 += 256 * 8) {
    float vv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) vv[j] = value(min(i00 + 256 * j + tid, D - 1));
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int i0 = i00 + 256 * j, i = i0 + tid;
      if (i0 + 64 * wave >= D) break;  // wave-uniform; whole groups: D % 64 == 0
      const float v = vv[j];
      float sx = row_sx;
      if (!PT) {
        const float amax = dpp_max_f(fabsf(v));
        sx = amax > 0.f ? amax / 127.f : 1.f;
      }
      const float q = rintf(v / sx);
      U[i] = (int8_t)q;
      const float qs = dpp_sum_f(q);
      if (lane == 0) {
        const int g = i / kGroup;
        XS[2 * g] = sx;
        XS[2 * g + 1] = sx * qs;
      }
    }
  }
}

// rmsnorm (k_rmsnorm; reference core.metal:486-500) with the quantization of its bf16 output (reference rmsnorm_a8,
// core.metal:502-537, per group there).
template <bool PT>
__global__ __launch_bounds__(256) void k_rmsnorm_a8(const uint16_t* __restrict__ x, int in_stride,
                                                    const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                    int out_stride, int D, float eps, int8_t* __restrict__ U,
                                                    float* __restrict__ XS) {
  __shared__ float red[4];
  const size_t row = blockIdx.x;
  const uint16_t* xr = x + row * in_stride;
  const float r = rsqrtf(block_sum4(row_sumsq256(xr, D), red) / (float)D + eps);
  row_norm_store256(xr, w, out + row * out_stride, D, r);
  auto value = [&](int i) { return bf2f(f2bf(bf2f(xr[i]) * r * bf2f(w[i]))); };
  quant_row<PT>(value, D, red, U + row * D, XS + row * (D / kGroup) * 2);
}

// silu_mul (k_silu_mul; reference core.metal:777-787) quantized without writing h (reference silu_mul_a8,
// core.metal:789-814, per group there). gu rows [gate (I) | up (I)], ldgu apart. Per group, block (row, c) takes
// columns [c kSmChunk, (c + 1) kSmChunk): the groups are independent, so a row spreads over blocks; per token the
// row's amax needs the whole row in one block (gridDim.y = 1).
constexpr int kSmChunk = 256 * 8;
template <bool PT>
__global__ __launch_bounds__(256) void k_silu_mul_a8(const uint16_t* __restrict__ gu, int ldgu, int I,
                                                     int8_t* __restrict__ U, float* __restrict__ XS) {
  __shared__ float red[4];
  const size_t row = blockIdx.x;
  const int c0 = PT ? 0 : (int)blockIdx.y * kSmChunk, n = PT ? I : min(kSmChunk, I - c0);
  const uint16_t* g = gu + row * ldgu + c0;
  auto value = [&](int i) { return bf2f(f2bf(swiglu_f(bf2f(g[i]), bf2f(g[I + i])))); };
  quant_row<PT>(value, n, red, U + row * I + c0, XS + (row * (I / kGroup) + c0 / kGroup) * 2);
}

// A deferred split-K residual reduce inside the next rmsnorm (reference splitk_res_norm, core.metal:539-595):
// x[row] = bf16(sum_z part[z][row] + x[row]) in split order (k_splitk_reduce, mode 1), then out = rmsnorm(x) and,
// with U, its quantization. Each thread uses only the elements it wrote (a load clamped past the row's end reads
// element D - 1 and discards it).
template <int A8>  // 0: none, 1: per group, 2: per token
__global__ __launch_bounds__(256) void k_splitk_res_norm(const float* __restrict__ part, int S, int M, uint16_t* x,
                                                         int ldx, const uint16_t* __restrict__ w,
                                                         uint16_t* __restrict__ out, int out_stride, int D, float eps,
                                                         int8_t* __restrict__ U, float* __restrict__ XS) {
  __shared__ float red[4];
  const size_t row = blockIdx.x, mn = (size_t)M * D;
  uint16_t* xr = x + row * ldx;
  float ss = 0.f;
  // 8 elements per thread at a time, their loads at clamped indices issued before the sums (as row_sumsq256); each
  // element's partials summed in split order, then the residual
  for (int i0 = threadIdx.x; i0 < D; i0 += 256 * 8) {
    float acc[8];
    uint16_t xu[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      acc[k] = 0.f;
      xu[k] = xr[min(i0 + 256 * k, D - 1)];
    }
    for (int z = 0; z < S; z++) {
      float pv[8];
#pragma unroll
      for (int k = 0; k < 8; k++) pv[k] = part[z * mn + row * D + min(i0 + 256 * k, D - 1)];
#pragma unroll
      for (int k = 0; k < 8; k++) acc[k] += pv[k];
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = i0 + 256 * k;
      if (i < D) {
        const uint16_t v = f2bf(acc[k] + bf2f(xu[k]));
        xr[i] = v;
        const float f = bf2f(v);
        ss = __builtin_fmaf(f, f, ss);
      }
    }
  }
  const float r = rsqrtf(block_sum4(ss, red) / (float)D + eps);
  row_norm_store256(xr, w, out + row * out_stride, D, r);
  if (A8) {
    auto value = [&](int i) { return bf2f(f2bf(bf2f(xr[i]) * r * bf2f(w[i]))); };
    if (A8 == 2) quant_row<true>(value, D, red, U + row * D, XS + row * (D / kGroup) * 2);
    else quant_row<false>(value, D, red, U + row * D, XS + row * (D / kGroup) * 2);
  }
}

int launch_rmsnorm_a8(const uint16_t* x, int in_stride, const uint16_t* w, uint16_t* out, int out_stride, int rows,
                      int D, float eps, int per_token, int8_t* U, float* XS, hipStream_t st) {
  if (rows == 0) return IFD_OK;
  if (per_token)
    hipLaunchKernelGGL(k_rmsnorm_a8<true>, dim3(rows), dim3(256), 0, st, x, in_stride, w, out, out_stride, D, eps, U,
                       XS);
  else
    hipLaunchKernelGGL(k_rmsnorm_a8<false>, dim3(rows), dim3(256), 0, st, x, in_stride, w, out, out_stride, D, eps,
                       U, XS);
  return check_launch("rmsnorm_a8");
}

int launch_silu_mul_a8(const uint16_t* gu, int ldgu, int I, int rows, int per_token, int8_t* U, float* XS,
                       hipStream_t st) {
  if (rows == 0) return IFD_OK;
  if (per_token) hipLaunchKernelGGL(k_silu_mul_a8<true>, dim3(rows), dim3(256), 0, st, gu, ldgu, I, U, XS);
  else
    hipLaunchKernelGGL(k_silu_mul_a8<false>, dim3(rows, (I + kSmChunk - 1) / kSmChunk), dim3(256), 0, st, gu, ldgu, I,
                       U, XS);
  return check_launch("silu_mul_a8");
}

int launch_splitk_res_norm(const float* part, int S, uint16_t* x, int ldx, const uint16_t* w, uint16_t* out,
                           int out_stride, int rows, int D, float eps, int a8, int8_t* U, float* XS, hipStream_t st) {
  if (rows == 0) return IFD_OK;
  if (a8 == 2)
    hipLaunchKernelGGL(k_splitk_res_norm<2>, dim3(rows), dim3(256), 0, st, part, S, rows, x, ldx, w, out, out_stride,
                       D, eps, U, XS);
  else if (a8 == 1)
    hipLaunchKernelGGL(k_splitk_res_norm<1>, dim3(rows), dim3(256), 0, st, part, S, rows, x, ldx, w, out, out_stride,
                       D, eps, U, XS);
  else
    hipLaunchKernelGGL(k_splitk_res_norm<0>, dim3(rows), dim3(256), 0, st, part, S, rows, x, ldx, w, out, out_stride,
                       D, eps, U, XS);
  return check_launch("splitk_res_norm");
}

}  // namespace ifd
