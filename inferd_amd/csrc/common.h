// Shared device helpers for the gfx950 (CDNA4) kernels of the W4 quantized-matmul path.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ifd {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) int32_t i32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(16))) int32_t i32x16;

constexpr int kGroup = 64;  // MLX affine group size along K

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;
// two fp32 -> packed bf16 pair (lo in bits 0-15), round to nearest even: one two-input v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}
// SwiGLU of one bf16 (gate, up) pair: bf16(float(bf16(g / (1 + exp(-g)))) * u) (reference silu_mul,
// engine/kernels/core.metal:777-787)
__device__ __forceinline__ float swiglu_f(float g, float u) { return bf2f(f2bf(g / (1.f + expf(-g)))) * u; }

// D(32x32 fp32) += A(32x16 bf16) * B(16x32 bf16). Lane l holds A row (l % 32), B column (l % 32), eight consecutive
// k values 8 * (l / 32) .. +7 of the 16; D row 8 * (r / 4) + 4 * (l / 32) + (r % 4), column l % 32, for r = 0..15.
__device__ __forceinline__ f32x16 mfma_bf16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
// D(32x32 int32) += A(32x32 int8) * B(32x32 int8); lane l: sixteen consecutive k values 16 * (l / 32) .. +15.
__device__ __forceinline__ i32x16 mfma_i8(u32x4 a, u32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                               0);
}

// Eight 4-bit codes of one word (k order 0..7, low nibble first) as eight bf16 values (off + q) in natural k order:
// bf16 0x4300 | q == 128 + q exactly. The caller corrects with bias' = bias - 128 * scale.
__device__ __forceinline__ u32x4 codes_bf16_off128(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;  // bytes: q0 q2 q4 q6 / q1 q3 q5 q7
  u32x4 r;
  // v_perm_b32(S0 = hi, S1 = lo): selector bytes 0-3 pick lo, 4-7 pick hi, 0x0c gives 0
  r[0] = __builtin_amdgcn_perm(hi, lo, 0x0c040c00u) | 0x43004300u;  // (q0, q1)
  r[1] = __builtin_amdgcn_perm(hi, lo, 0x0c050c01u) | 0x43004300u;  // (q2, q3)
  r[2] = __builtin_amdgcn_perm(hi, lo, 0x0c060c02u) | 0x43004300u;  // (q4, q5)
  r[3] = __builtin_amdgcn_perm(hi, lo, 0x0c070c03u) | 0x43004300u;  // (q6, q7)
  return r;
}

// Eight 4-bit codes of one word as eight bf16 values (128 + q) in the paired k order (0,4,1,5,2,6,3,7): one
// v_and_or_b32 (+ one shift) per pair. The activation fragment must use the same order (see perm_pairs04).
__device__ __forceinline__ u32x4 codes_bf16_off128_p04(uint32_t w) {
  u32x4 r;
  r[0] = (w & 0x000F000Fu) | 0x43004300u;          // (q0, q4)
  r[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;   // (q1, q5)
  r[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;   // (q2, q6)
  r[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;  // (q3, q7)
  return r;
}
// Eight consecutive bf16 values (x0..x7) reordered to (x0,x4,x1,x5,x2,x6,x3,x7).
__device__ __forceinline__ u32x4 perm_pairs04(u32x4 v) {
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
  r[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
  r[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
  r[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
  return r;
}

// Eight 4-bit codes of one word as eight int8 values 0..15 in natural k order (two dwords).
__device__ __forceinline__ u32x2 codes_i8(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  u32x2 r;
  r[0] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // q0 q1 q2 q3
  r[1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // q4 q5 q6 q7
  return r;
}

// Dequantize eight codes to bf16(s * q + b) in natural k order (MLX's qmm loader rounding, quantized.h:528-535).
__device__ __forceinline__ u32x4 dequant8_bf16(uint32_t w, float s, float b) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float q0 = (float)((lo >> (8 * i)) & 0xFFu), q1 = (float)((hi >> (8 * i)) & 0xFFu);
    r[i] = pack_bf2(__builtin_fmaf(s, q0, b), __builtin_fmaf(s, q1, b));
  }
  return r;
}

// ---- 8-bit codes (MLX affine 8-bit: byte i of a row is element i) ----
// Eight 8-bit codes of two words (k order 0..7) as eight bf16 values q (exact: every integer 0..255 is a bf16):
// v_cvt_f32_ubyte per code, then the high halves of two floats packed by one v_perm_b32.
__device__ __forceinline__ u32x4 codes8_bf16(uint32_t w0, uint32_t w1) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const uint32_t w = i ? w1 : w0;
    const uint32_t f0 = __float_as_uint((float)(w & 0xFFu)), f1 = __float_as_uint((float)((w >> 8) & 0xFFu));
    const uint32_t f2 = __float_as_uint((float)((w >> 16) & 0xFFu)), f3 = __float_as_uint((float)(w >> 24));
    r[2 * i] = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
    r[2 * i + 1] = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
  }
  return r;
}
// Eight 8-bit codes of two words dequantized to bf16(s * q + b) in natural k order.
__device__ __forceinline__ u32x4 dequant8x8_bf16(uint32_t w0, uint32_t w1, float s, float b) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const uint32_t w = i ? w1 : w0;
    const float q0 = (float)(w & 0xFFu), q1 = (float)((w >> 8) & 0xFFu);
    const float q2 = (float)((w >> 16) & 0xFFu), q3 = (float)(w >> 24);
    r[2 * i] = pack_bf2(__builtin_fmaf(s, q0, b), __builtin_fmaf(s, q1, b));
    r[2 * i + 1] = pack_bf2(__builtin_fmaf(s, q2, b), __builtin_fmaf(s, q3, b));
  }
  return r;
}

// The codes one lane holds for one 64-group in the MLX layout: 32 codes = BITS words, loaded as one (4 bits) or two
// (8 bits) 16 B pieces at word offsets 4 h (+ 8) of the group, so that each load instruction of a wave covers 32
// contiguous bytes of every row. Step t of the four 32x32x16 MFMA steps takes the eight codes at k = kofs(t, h) + 0..7:
// 32 h + 8 t for 4 bits (one 16 B piece = 32 codes), 32 (t / 2) + 16 h + 8 (t % 2) for 8 bits (a piece = 16 codes).
// The activation fragment of a step is read at the same k.
template <int BITS>
struct GroupCodes {
  u32x4 w[BITS / 4];
  static __device__ __forceinline__ int kofs(int t, int h) {
    return BITS == 4 ? 32 * h + 8 * t : 32 * (t >> 1) + 16 * h + 8 * (t & 1);
  }
  // the row's words for group g from `row` (already offset to this lane's first piece: 4 h words)
  __device__ __forceinline__ void load(const uint32_t* row, int g) {
#pragma unroll
    for (int i = 0; i < BITS / 4; i++) w[i] = *(const u32x4*)(row + (size_t)g * 2 * BITS + 8 * i);
  }
  __device__ __forceinline__ uint32_t word(int i) const { return w[i / 4][i % 4]; }
  // step t as bf16 MFMA operand, offset so that it is exact: 128 + q (4 bits) or q (8 bits)
  __device__ __forceinline__ u32x4 step_affine(int t, uint32_t xr) const {
    if (BITS == 4) return codes_bf16_off128(word(t) ^ xr);
    return codes8_bf16(word(2 * t) ^ xr, word(2 * t + 1) ^ xr);
  }
  // step t dequantized to bf16(s q + b)
  __device__ __forceinline__ u32x4 step_dequant(int t, uint32_t xr, float s, float b) const {
    if (BITS == 4) return dequant8_bf16(word(t) ^ xr, s, b);
    return dequant8x8_bf16(word(2 * t) ^ xr, word(2 * t + 1) ^ xr, s, b);
  }
};
// the bias correction of step_affine's offset: b - 128 s (4 bits) or b (8 bits)
template <int BITS>
__device__ __forceinline__ float affine_bias(float s, float b) {
  return BITS == 4 ? __builtin_fmaf(-128.f, s, b) : b;
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; i++) z[i] = 0.f;
  return z;
}
__device__ __forceinline__ i32x16 izero16() {
  i32x16 z;
#pragma unroll
  for (int i = 0; i < 16; i++) z[i] = 0;
  return z;
}

// Store one fp32 result with the GEMM store mode (0 bf16, 1 bf16 residual add, 2 fp32).
__device__ __forceinline__ void store_mode(void* C, size_t o, float v, int mode) {
  if (mode == 2) {
    ((float*)C)[o] = v;
  } else if (mode == 1) {
    uint16_t* c = (uint16_t*)C + o;
    *c = f2bf(v + bf2f(*c));
  } else {
    ((uint16_t*)C)[o] = f2bf(v);
  }
}

// Wave64 reductions.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// Wave-wide max / min / sum with DPP: an inclusive scan within rows of 16 lanes (row_shr 1, 2, 4, 8), then across
// rows (row_bcast 15 into rows 1 and 3, row_bcast 31 into rows 2 and 3), so lane 63 holds the result, which
// readlane makes wave-uniform. Lanes a step has no source for keep the identity. About a tenth of the latency of the
// LDS-permute shuffles, which matters in the serial top-k loop.
template <class Op>
__device__ __forceinline__ int dpp_reduce_i(int v, int id, Op op) {
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x118, 0xf, 0xf, false));  // row_shr:8
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ float dpp_max_f(float v) {
  return __int_as_float(dpp_reduce_i(__float_as_int(v), __float_as_int(-INFINITY), [](int a, int b) {
    return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b)));
  }));
}
__device__ __forceinline__ float dpp_sum_f(float v) {
  return __int_as_float(dpp_reduce_i(__float_as_int(v), 0, [](int a, int b) {
    return __float_as_int(__int_as_float(a) + __int_as_float(b));
  }));
}
__device__ __forceinline__ int dpp_min_i(int v) {
  return dpp_reduce_i(v, 0x7fffffff, [](int a, int b) { return min(a, b); });
}

// The two row passes of rmsnorm for a 256-thread block: thread t takes elements t + 256 k, in k order, with 8
// elements' loads issued before their arithmetic. The loads are unconditional, at an index clamped to the row, and
// the select comes after them: a load under the bound check became a branch with its own wait, and the serial load
// latency made a 5120-wide row take about 9 us. An element past D contributes fma(0, 0, ss) = ss (ss >= +0).
__device__ __forceinline__ float row_sumsq256(const uint16_t* __restrict__ xr, int D) {
  float ss = 0.f;
  for (int i0 = (int)threadIdx.x; i0 < D; i0 += 256 * 8) {
    uint16_t u[8];
#pragma unroll
    for (int k = 0; k < 8; k++) u[k] = xr[min(i0 + 256 * k, D - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float v = i0 + 256 * k < D ? bf2f(u[k]) : 0.f;
      ss = __builtin_fmaf(v, v, ss);
    }
  }
  return ss;
}
// o[i] = bf16(x[i] r w[i]); each thread writes only the elements it read (o may be x)
__device__ __forceinline__ void row_norm_store256(const uint16_t* xr, const uint16_t* __restrict__ w, uint16_t* o,
                                                  int D, float r) {
  for (int i0 = (int)threadIdx.x; i0 < D; i0 += 256 * 8) {
    uint16_t xu[8], wu[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = min(i0 + 256 * k, D - 1);
      xu[k] = xr[i];
      wu[k] = w[i];
    }
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (i0 + 256 * k < D) o[i0 + 256 * k] = f2bf(bf2f(xu[k]) * r * bf2f(wu[k]));
  }
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}

// Device-coherent (sc1) buffer accesses to data that blocks on different XCDs (separate L2s) exchange within one
// kernel: stores write through to memory, loads do not hit a stale line of the local L2. Plain loads batch, unlike
// atomic loads, which the compiler orders one after another.
constexpr int kSc1 = 16;  // cache-policy operand: SC1
constexpr int kNt = 2;    // cache-policy operand: NT (non-temporal)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const void* part, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)part, 0, (int)bytes, 0x00020000);
}

// Bijective remap of a 1-D block id so that each XCD (blocks are dealt round-robin over 8 XCDs) runs a contiguous
// range of logical tiles: neighbouring tiles then share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int X = 8;
  const int per = nblocks / X, rem = nblocks % X, x = bid % X, i = bid / X;
  return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

}  // namespace ifd
