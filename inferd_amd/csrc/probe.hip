// Measurement probes: the HBM read and MFMA ceilings the benchmark reports beside the datasheet peaks, measured on
// the same GPU in the same process. They play the role of the reference's micro-benchmarks (bw_read,
// micro/kernels.metal:8-16, printed as results/micro-2026-10-29-r2.txt:2-4; fma_rate, micro/fma_rate.mm), which
// measure the ceilings its kernels are judged against. Not part of the operator path.
#include "common.h"
#include "host.h"
#include "kernels.h"

namespace ifd {

// Stream read: every wave reads kProbeUnroll contiguous 1 KB lines per iteration (16 B per lane), the waves of the
// grid walking the buffer in interleaved 1 KB lines (each load instruction is one coalesced 1 KB request). The XOR
// of everything read is stored only if it equals a value it cannot equal, so no load is dead to the compiler.
constexpr int kProbeUnroll = 8;
__global__ __launch_bounds__(256) void k_probe_read(const u32x4* __restrict__ src, size_t n16, uint32_t never,
                                                    u32x4* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  u32x4 acc = u32x4{0u, 0u, 0u, 0u};
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; u++) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; u++) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= src[i];
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == never) sink[threadIdx.x] = acc;
}

// MFMA only: each wave runs kProbeChains independent accumulator chains of one MFMA shape for `iters` rounds on
// register operands (no memory traffic in the loop), then stores one value per lane.
constexpr int kProbeChains = 8;
template <bool INT8>
__global__ __launch_bounds__(256) void k_probe_mfma(int iters, float* __restrict__ out) {
  const uint32_t lane = threadIdx.x & 63;
  const u32x4 a = u32x4{0x3F803F80u ^ lane, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u ^ (lane << 1)};
  const u32x4 b = u32x4{0x3C003C00u, 0x3C003C00u ^ lane, 0x3C003C00u, 0x3C003C00u};
  float s = 0.f;
  if (INT8) {
    i32x16 acc[kProbeChains];
#pragma unroll
    for (int c = 0; c < kProbeChains; c++) acc[c] = izero16();
    for (int it = 0; it < iters; it++)
#pragma unroll
      for (int c = 0; c < kProbeChains; c++) acc[c] = mfma_i8(a, b, acc[c]);
#pragma unroll
    for (int c = 0; c < kProbeChains; c++) s += (float)acc[c][c];
  } else {
    f32x16 acc[kProbeChains];
#pragma unroll
    for (int c = 0; c < kProbeChains; c++) acc[c] = zero16();
    for (int it = 0; it < iters; it++)
#pragma unroll
      for (int c = 0; c < kProbeChains; c++) acc[c] = mfma_bf16(a, b, acc[c]);
#pragma unroll
    for (int c = 0; c < kProbeChains; c++) s += acc[c][c];
  }
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

int launch_probe_read(const void* src, size_t bytes, void* sink, int blocks, hipStream_t st) {
  hipLaunchKernelGGL(k_probe_read, dim3(blocks), dim3(256), 0, st, (const u32x4*)src, bytes / 16, 0x9E3779B9u,
                     (u32x4*)sink);
  return check_launch("probe_read");
}

int launch_probe_mfma(int int8, int iters, int blocks, float* out, hipStream_t st) {
  if (int8) hipLaunchKernelGGL(k_probe_mfma<true>, dim3(blocks), dim3(256), 0, st, iters, out);
  else hipLaunchKernelGGL(k_probe_mfma<false>, dim3(blocks), dim3(256), 0, st, iters, out);
  return check_launch("probe_mfma");
}

}  // namespace ifd
