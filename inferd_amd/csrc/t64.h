// The T64 weight layout: the MI355X-native arrangement of an MLX affine 4-bit group-64 linear [N, K].
//
// A repack of the reference layout (wq uint32 [N][K/8], s/b bf16 [N][K/64]) made once at load, like the
// reference's in-place flip (engine/src/qwen35.h:1306-1322). Same size (0.5625 B per weight); codes are stored
// unflipped.
//
//   nb = ceil(N / 32) bands of 32 output columns (weight rows); rows past N are zero.
//   tile(g, b) = 1152 bytes at ((g * nb) + b) * 1152, for 64-group g and band b  (group-major: all bands of a group
//   are contiguous, so a grid that walks K in step streams one contiguous window of HBM)
//     bytes [0, 1024): 64 lanes x 16 bytes. Lane l = j + 32 h (row 32 b + j, half h) holds four words; word t
//                      carries the codes of k = 64 g + 32 h + 8 t + e, e = 0..7, with code e in nibble
//                      kT64Nib[e] = (0, 4, 1, 5, 2, 6, 3, 7)[e]: then (word >> 4 i) & 0x000F000F puts codes (2i, 2i+1)
//                      in the two 16-bit halves (one and-or builds a bf16 pair in natural k order).
//     bytes [1024, 1152): 32 dwords, dword j = s | (b << 16) (bf16 bits) of row 32 b + j.
// The 16-byte load of lane l at tile + 16 l is exactly that lane's B-operand fragment for the four 32x32x16 bf16 MFMA
// steps of the group (column j, k slots 32 h + 8 t .. + 7), so one wave-wide load instruction reads 1 KB contiguous.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace ifd {

constexpr int kT64Tile = 1152;
constexpr int kT64Codes = 1024;

__host__ __device__ inline int t64_bands(int N) { return (N + 31) / 32; }
__host__ __device__ inline size_t t64_bytes(int N, int K) { return (size_t)(K / 64) * t64_bands(N) * kT64Tile; }

// codes of one word in natural order (nibble e = code e) -> T64 nibble order
__host__ __device__ inline uint32_t t64_word(uint32_t w) {
  uint32_t o = 0;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int nib = (e & 1) ? 4 + (e >> 1) : (e >> 1);
    o |= ((w >> (4 * e)) & 15u) << (4 * nib);
  }
  return o;
}

// ---- T64x8: the same arrangement for an MLX affine 8-bit group-64 linear (wq uint32 [N][K/4]) -------------------
//
//   tile(g, b) = 2176 bytes at ((g * nb) + b) * 2176 (group-major, as above)
//     bytes [0, 2048): [s2 = 0, 1][64 lanes][16 bytes]. Lane l = j + 32 h (row 32 b + j) holds, at s2 * 1024 + 16 l,
//                      the codes of k = 64 g + 32 h + 16 s2 + 0..15 in natural order, each stored as the int8
//                      q - 128 (the byte q ^ 0x80): exactly the lane's B fragment of v_mfma_i32_32x32x32_i8 step s2.
//     bytes [2048, 2176): 32 dwords, dword j = s | (b << 16) (bf16 bits) of row 32 b + j.
// 1.0625 B per weight, the size of the MLX layout.
constexpr int kT64x8Tile = 2176;
constexpr int kT64x8Codes = 2048;

__host__ __device__ inline size_t t64x8_bytes(int N, int K) { return (size_t)(K / 64) * t64_bands(N) * kT64x8Tile; }

}  // namespace ifd
