// Prefill path: 4- or 8-bit weights x bf16 activations on bf16 MFMA, for any M (used above 128 rows).
//
// Replaces MLX's affine_qmm_t_nax (third_party/mlx/.../quantized_nax.h:938-1076, 1206-1267; instances
// engine/kernels/mlx_qmm.metal:9-14; host mlx_qmm, engine/src/qwen35.h:1427-1462), with the same numerics: every
// weight is dequantized once per block tile to bf16(s q + b) (quantized.h:528-535), activations stay bf16, the
// product accumulates in fp32 and is stored by mode (0 bf16, 1 bf16 residual add, 2 fp32).
//
// Block: 256 threads (4 waves as 2 x 2), tile 256 (M) x 128 (N), one 64-group of K per step. Each step stages the
// activation tile (32 KB) and the dequantized weight tile (16 KB) in LDS, double-buffered (one barrier per step);
// each wave then runs a 128 x 64 sub-tile as 4 x 2 MFMA 32x32x16 tiles. The dequant of a weight tile (32 codes per
// thread) is shared by all 256 rows of the block. Block ids are remapped so that each XCD walks a contiguous run of
// tiles in bands of 4 M tiles, so a weight tile and an activation tile are fetched into that XCD's L2 once per band.
#include "common.h"
#include "host.h"
#include "kernels.h"

namespace ifd {

constexpr int kQmmBM = 256, kQmmBN = 128, kQmmLd = 72;  // LDS row: 64 bf16 + 8 pad (144 B)
constexpr int kQmmBand = 4;

struct QmmArgs {
  const uint16_t* A;
  int lda;
  const uint32_t* wq;
  const uint16_t* s;
  const uint16_t* b;
  int N, K, ldk;
  uint32_t xr;
  void* C;
  int ldc, M, mode;
  int tiles_m, tiles_n;
};

template <int BITS>
__global__ __launch_bounds__(256) void k_qmm(QmmArgs p) {
  extern __shared__ __align__(16) uint16_t smem[];
  uint16_t* As = smem;                         // [2][256][72]
  uint16_t* Ws = smem + 2 * kQmmBM * kQmmLd;   // [2][128][72]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;

  // tile order: XCD-contiguous, then bands of kQmmBand M tiles walked M-fastest
  const int ntiles = p.tiles_m * p.tiles_n;
  const int L = xcd_remap(blockIdx.x, ntiles);
  const int per_band = kQmmBand * p.tiles_n;
  const int band = L / per_band, within = L % per_band;
  const int bm = min(kQmmBand, p.tiles_m - band * kQmmBand);
  const int tm = band * kQmmBand + within % bm, tn = within / bm;
  const int m0 = tm * kQmmBM, n0 = tn * kQmmBN;

  const int G = p.K / kGroup, ldw = p.ldk * BITS / 32, ldg = p.ldk / kGroup;
  // activation loads: 8 chunks of 16 B per thread, chunk c = tid + 256 i -> row c / 8, column 8 (c % 8)
  const uint16_t* aptr[8];
  bool aok[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int c = tid + 256 * i, row = c >> 3, m = m0 + row;
    aok[i] = m < p.M;
    aptr[i] = p.A + (size_t)(aok[i] ? m : 0) * p.lda + 8 * (c & 7);
  }
  // weight loads: row tid / 2, half tid % 2 (32 codes = BITS words)
  const int wr = tid >> 1, wh = tid & 1;
  const int nw = min(n0 + wr, p.N - 1);
  const uint32_t* wptr = p.wq + (size_t)nw * ldw + 4 * wh;
  const uint16_t* sptr = p.s + (size_t)nw * ldg;
  const uint16_t* bptr = p.b + (size_t)nw * ldg;

  u32x4 areg[8];
  GroupCodes<BITS> wreg;
  uint32_t sbreg;
  auto gload = [&](int g) {
#pragma unroll
    for (int i = 0; i < 8; i++) areg[i] = aok[i] ? *(const u32x4*)(aptr[i] + (size_t)g * 64) : u32x4{0u, 0u, 0u, 0u};
    wreg.load(wptr, g);
    sbreg = (uint32_t)sptr[g] | ((uint32_t)bptr[g] << 16);
  };
  auto lstore = [&](int buf) {
    uint16_t* as = As + buf * kQmmBM * kQmmLd;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int c = tid + 256 * i;
      *(u32x4*)(as + (c >> 3) * kQmmLd + 8 * (c & 7)) = areg[i];
    }
    const float sc = bf2f((uint16_t)(sbreg & 0xFFFFu)), bi = bf2f((uint16_t)(sbreg >> 16));
    uint16_t* ws = Ws + buf * kQmmBN * kQmmLd + wr * kQmmLd;
#pragma unroll
    for (int t = 0; t < 4; t++)
      *(u32x4*)(ws + GroupCodes<BITS>::kofs(t, wh)) = wreg.step_dequant(t, p.xr, sc, bi);
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int c = 0; c < 2; c++) acc[a][c] = zero16();

  gload(0);
  lstore(0);
  __syncthreads();
  for (int g = 0; g < G; g++) {
    const int buf = g & 1;
    if (g + 1 < G) gload(g + 1);
    const uint16_t* as = As + buf * kQmmBM * kQmmLd + (wm * 128 + j) * kQmmLd + 8 * h;
    const uint16_t* ws = Ws + buf * kQmmBN * kQmmLd + (wn * 64 + j) * kQmmLd + 8 * h;
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      u32x4 af[4], bf[2];
#pragma unroll
      for (int a = 0; a < 4; a++) af[a] = *(const u32x4*)(as + a * 32 * kQmmLd + 16 * kk);
#pragma unroll
      for (int c = 0; c < 2; c++) bf[c] = *(const u32x4*)(ws + c * 32 * kQmmLd + 16 * kk);
#pragma unroll
      for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 2; c++) acc[a][c] = mfma_bf16(af[a], bf[c], acc[a][c]);
    }
    if (g + 1 < G) lstore(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int col = n0 + wn * 64 + 32 * c + j;
      if (col >= p.N) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * 128 + 32 * a + 8 * (r / 4) + 4 * h + (r % 4);
        if (row < p.M) store_mode(p.C, (size_t)row * p.ldc + col, acc[a][c][r], p.mode);
      }
    }
}

size_t qmm_workspace(int, int, int) { return 0; }

int launch_qmm(const W4Gemm& g, void*, size_t, hipStream_t st) {
  if (g.M == 0) return IFD_OK;
  QmmArgs p{(const uint16_t*)g.A, g.lda, g.wq, g.s, g.b, g.N, g.K, g.ldk, g.xr, g.C, g.ldc, g.M, g.mode,
            (g.M + kQmmBM - 1) / kQmmBM, (g.N + kQmmBN - 1) / kQmmBN};
  const size_t lds = (size_t)2 * (kQmmBM + kQmmBN) * kQmmLd * sizeof(uint16_t);
  static bool attr = false;
  if (!attr) {
    hipFuncSetAttribute((const void*)k_qmm<4>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipFuncSetAttribute((const void*)k_qmm<8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr = true;
  }
  if (g.bits == 8) hipLaunchKernelGGL(k_qmm<8>, dim3(p.tiles_m * p.tiles_n), dim3(256), lds, st, p);
  else hipLaunchKernelGGL(k_qmm<4>, dim3(p.tiles_m * p.tiles_n), dim3(256), lds, st, p);
  return check_launch("qmm");
}

}  // namespace ifd
