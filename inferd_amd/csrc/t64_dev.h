// Device-side decoding of T64 code words (t64.h) into MFMA B fragments.
#pragma once
#include "common.h"

namespace ifd {

__device__ __forceinline__ u32x4 t64_off128(uint32_t w) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; i++) r[i] = ((w >> (4 * i)) & 0x000F000Fu) | 0x43004300u;
  return r;
}
// Eight T64 codes (one word) -> bf16(s q + b) in natural k order. Code 2i sits in nibble i, code 2i + 1 in nibble
// i + 4 (t64.h), so each 16-bit half of the word holds four codes, the pair (2i, 2i + 1) at the same place in the
// two halves. Masking the word (and the word shifted by 8) with 0x000F000F / 0x00F000F0 leaves two f16 subnormals
// q 2^-24 or 16 q 2^-24 = q 2^-20 per 32 bits, which v_fma_mix_f32 widens exactly; with sa = s 2^24 and sb = s 2^20
// (exact power-of-two scalings of a bf16) each fma computes s q exactly and rounds s q + b once in fp32, as the
// bf16(fp32(s q + b)) of the MLX loader. 17 VALU instructions per 8 codes (5 integer, 8 fma_mix, 4 conversions).
// The scalings are exact for |s| < 2^103; larger scales overflow (a 4-bit scale is a weight range / 15).
__device__ __forceinline__ float h16_lo(uint32_t p) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(p & 0xFFFFu)); }
__device__ __forceinline__ float h16_hi(uint32_t p) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(p >> 16)); }
__device__ __forceinline__ u32x4 t64_dequant(uint32_t w, float sa, float sb, float b) {
  const uint32_t p01 = w & 0x000F000Fu, p23 = w & 0x00F000F0u, w8 = w >> 8;
  const uint32_t p45 = w8 & 0x000F000Fu, p67 = w8 & 0x00F000F0u;
  return u32x4{pack_bf2(__builtin_fmaf(sa, h16_lo(p01), b), __builtin_fmaf(sa, h16_hi(p01), b)),
               pack_bf2(__builtin_fmaf(sb, h16_lo(p23), b), __builtin_fmaf(sb, h16_hi(p23), b)),
               pack_bf2(__builtin_fmaf(sa, h16_lo(p45), b), __builtin_fmaf(sa, h16_hi(p45), b)),
               pack_bf2(__builtin_fmaf(sb, h16_lo(p67), b), __builtin_fmaf(sb, h16_hi(p67), b))};
}
// The two scalings of a group's bf16 scale s for t64_dequant.
__device__ __forceinline__ float t64_sa(float s) { return s * 16777216.f; }
__device__ __forceinline__ float t64_sb(float s) { return s * 1048576.f; }

}  // namespace ifd
