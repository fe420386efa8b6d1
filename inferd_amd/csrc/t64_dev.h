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
// i + 4 (t64.h), so the low nibbles of the four bytes hold codes 0, 4, 1, 5 and the high nibbles codes 2, 6, 3, 7.
// Two masks split the word into bytes; one byte -> fp32 conversion per code (v_cvt_f32_ubyte0..3) gives q, or 16 q for
// the high nibbles, which take s / 16 (exact: a power-of-two scaling of a bf16); fma rounds s q + b once in fp32, as
// the bf16(fp32(s q + b)) of the MLX loader. 22 VALU instructions per 8 codes, two of them integer ops: integer VALU
// co-issues poorly beside MFMA, conversions and fma well. The masks go through opaque moves so that the compiler
// selects the byte conversions instead of folding the masks into bitfield extracts.
__device__ __forceinline__ u32x4 t64_dequant(uint32_t w, float s, float s16, float b) {
  uint32_t lo, hi;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(w));
  asm("v_and_b32 %0, 0xf0f0f0f0, %1" : "=v"(hi) : "v"(w));
  const float c0 = __builtin_fmaf(s, (float)(lo & 0xFFu), b), c4 = __builtin_fmaf(s, (float)((lo >> 8) & 0xFFu), b);
  const float c1 = __builtin_fmaf(s, (float)((lo >> 16) & 0xFFu), b), c5 = __builtin_fmaf(s, (float)(lo >> 24), b);
  const float c2 = __builtin_fmaf(s16, (float)(hi & 0xFFu), b), c6 = __builtin_fmaf(s16, (float)((hi >> 8) & 0xFFu), b);
  const float c3 = __builtin_fmaf(s16, (float)((hi >> 16) & 0xFFu), b), c7 = __builtin_fmaf(s16, (float)(hi >> 24), b);
  return u32x4{pack_bf2(c0, c1), pack_bf2(c2, c3), pack_bf2(c4, c5), pack_bf2(c6, c7)};
}

}  // namespace ifd
