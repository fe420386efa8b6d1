// Decode MoE for T <= 16 tokens in three launches, each distinct expert's weights read once for every token that
// picked it.
//
// Replaces the reference's four-launch decode MoE (engine/kernels/moe.metal:267-293 router, 326-368 moe_plan,
// 370-488 moe_gu2, 490-551 moe_dn2; host engine/src/qwen35.h:1876-1908) up to 8 tokens, and its per-row expert GEMVs
// for fewer than moe_sort_min = 128 routed rows beyond them (moe_qmv4 + moe_silu_mul + moe_qmv4 + moe_combine,
// moe.metal:6-58, 103-111, 113-187; host qwen35.h:1801-1807, 1947-1955): the same qmv4 arithmetic per row, with each
// distinct expert read once. Tokens are the MFMA's A rows: a lane holds rows 8 (r / 4) + 4 h + r % 4 of its RT
// accumulators (RT = 4 up to 8 tokens, 8 up to 16).
//  1. k_mdec_router: router logits (bf16 router [E1][H] x bf16 tokens) as K-split fp32 partials [KS][T][E1]. One
//     32-expert tile x a K range per wave (32x32x16 bf16 MFMA, tokens in the A rows), the block's eight waves summed
//     in wave order. The last block to finish (a counter in the workspace header) then routes: wave w sums token
//     w's partials in split order and routes it (route_token, as k_moe_route); one thread per pick lists the
//     distinct experts in pick order: plan = [nuniq, expert[T k], pick[T k][16]] (pick[u][t] = token t's pick index
//     of unique expert u, or -1).
//  2. k_mdec_gu: one block per (32 gate/up column pairs, unique expert or the shared expert). Its four waves split K;
//     each stages the token rows of its K range in LDS and streams the 32 gate and 32 up rows of its expert (16 B
//     of codes per lane and group, all loads of a chunk issued before the first wait), runs the qmv4 arithmetic on
//     bf16 MFMA (codes as 128 + q, the group sums X from the staged rows, s P + (b - 128 s) X in fp32), and the waves'
//     sums are added in wave order. The SwiGLU of the bf16-rounded gate and up goes to act[t][j] for every token t
//     that picked the expert as its j-th (j = k: the shared expert).
//  3. k_mdec_dn: one block per (128 output columns, unique expert or the shared expert): the down rows of the expert
//     against act of the tokens that picked it (same arithmetic), d[t][j] = bf16(result), stored write-through. The
//     last block of each 128-column chunk (a counter in the workspace header) combines:
//     out[t][h] = bf16(acc) or bf16(out + bf16(acc)), acc = sum_j wt[t][j] d[t][j][h] + sg[t] d[t][k][h], in j order.
// Every sum runs in a fixed order, so results do not depend on block timing.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "host.h"
#include "kernels.h"
#include "moe_dev.h"
#include "t64.h"
#include "t64_dev.h"

namespace ifd {

constexpr int kMdecMaxT = 16, kMdecMaxK = 16, kMdecKG = 8;  // tokens, picks, groups per wave and chunk
// the MFMA output row (token) of accumulator r of a lane in half h
__device__ __forceinline__ int mdec_row(int r, int h) { return 8 * (r / 4) + 4 * h + (r % 4); }
constexpr int kMdecMaxKS = 4;                                 // K splits of the router
constexpr int kMdecCmbB = 12;  // slots whose 16-byte loads a combining thread has in flight at once
constexpr int kMdecStageU = 4;  // token-row chunks a staging thread loads before using any

struct MdecArgs {
  const uint16_t* x;       // normalised tokens [T][H]
  const uint16_t* router;  // bf16 [E1][H]
  int T, H, E, E1, k, I, norm, shared_gate, assign, KS;
  const uint32_t* egu_wq;  // routed experts [E][2I][H] (gate rows, then up rows), MLX affine 4-bit
  const uint16_t* egu_s;
  const uint16_t* egu_b;
  const uint32_t* edn_wq;  // [E][H][I]
  const uint16_t* edn_s;
  const uint16_t* edn_b;
  const uint32_t* sgu_wq;  // shared expert [2I][H] and [H][I], or null
  const uint16_t* sgu_s;
  const uint16_t* sgu_b;
  const uint32_t* sdn_wq;
  const uint16_t* sdn_s;
  const uint16_t* sdn_b;
  uint16_t* out;           // [T][H]
  int* idx;                // routing outputs [T][k], [T][k], [T]
  float* wt;
  float* sg;
  float* logits;           // optional [T][E1]: the summed logits the routing used
  float* part;             // [KS][T][E1]
  int* plan;               // [1 + T k + T k 16]
  uint16_t* act;           // [T][k + 1][I]
  uint16_t* d;             // [T][k + 1][H]
  uint32_t d_bytes;
  unsigned* cnt;           // H / 128 counters, zero between calls
  int sb16_gu, sb16_dn;    // a wave's 8 scales (biases) of a row are one aligned 16 B load
  int sh_bits;             // the shared expert's width: 4, or 8 (the reference's moe_gu2_4_8 / moe_dn2_4_8)
  int routed;              // idx / wt / sg hold the caller's routing (no router, no routing here)
  const uint16_t* ys;      // with routed: the shared expert's output rows [T][H] for the combine, or null
  int out16;               // out and ys 16-byte aligned: the combine loads and stores 8 columns at a time
  int has_sh;              // a shared expert (either layout)
  // the T64 path: routed experts packed by ifd_pack_t64 with E (expert e at e gu_eb, e dn_eb bytes), the
  // shared expert's T64 copies or null; the gate/up K split (gS splits of gps groups) and its partials
  const uint8_t* egu_t;
  const uint8_t* edn_t;
  const uint8_t* sgu_t;
  const uint8_t* sdn_t;
  size_t gu_eb, dn_eb;
  float* gpart;
  uint32_t gpart_bytes;
  int gS, gps;
};

// The 8 bf16 values at v (16-byte aligned) as 8 raw halves.
__device__ __forceinline__ void load8h(const uint16_t* v, uint16_t (&o)[kMdecKG]) {
  const u32x4 w = *(const u32x4*)v;
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = (uint16_t)(w[i / 2] >> (16 * (i & 1)));
}

// ---- 1 + 2. router logits, then (the last block) routing and the distinct-expert plan -----------------------------
// Routing and the plan, by one block of NTHR threads: wave w routes tokens w, w + NTHR / 64, ... from the K-split
// partials (summed in split order; device-coherent loads: other blocks, maybe on other XCDs, wrote them), then one
// thread per pick numbers the distinct experts in pick order.
template <int NTHR>
__device__ __forceinline__ void mdec_plan_block(const MdecArgs& p) {
  __shared__ int tidx[kMdecMaxT * kMdecMaxK], urank[kMdecMaxT * kMdecMaxK], firstpick[512], wcount[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int T = p.T, k = p.k, NU = T * k;
  int* upick = p.plan + 1 + NU;
  for (int i = tid; i < NU * kMdecMaxT; i += NTHR) upick[i] = -1;
  for (int i = tid; i < p.E; i += NTHR) firstpick[i] = 0x7fffffff;
  const __amdgpu_buffer_rsrc_t rp = part_rsrc(p.part, (uint32_t)((size_t)p.KS * T * p.E1 * 4));
  for (int t = wave; t < T; t += NTHR / 64) {
    if (p.routed) {  // the caller's routing
      if (lane == 0)
        for (int jj = 0; jj < k; jj++) tidx[t * k + jj] = p.idx[t * k + jj];
      continue;
    }
    // token t's logits: every load issued before the first add
    float part[kMdecMaxKS][9];
#pragma unroll
    for (int z = 0; z < kMdecMaxKS; z++)
#pragma unroll
      for (int i = 0; i < 9; i++) {
        const int c = i < 8 ? i * 64 + lane : p.E;  // slot 8: the shared expert's gate logit
        part[z][i] = z < p.KS && c < p.E1
                         ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                               rp, (int)((((size_t)z * T + t) * p.E1 + c) * 4), 0, kSc1))
                         : 0.f;
      }
    float v[9];
#pragma unroll
    for (int i = 0; i < 9; i++) {
      v[i] = part[0][i];
#pragma unroll
      for (int z = 1; z < kMdecMaxKS; z++)
        if (z < p.KS) v[i] += part[z][i];
    }
    if (p.logits) {
#pragma unroll
      for (int i = 0; i < 8; i++)
        if (i * 64 + lane < p.E1) p.logits[(size_t)t * p.E1 + i * 64 + lane] = v[i];
      if (p.shared_gate && lane == 0) p.logits[(size_t)t * p.E1 + p.E] = v[8];
    }
    const float gate = v[8];
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = v[i];
    int who;
    float pw;
    route_token(r, p.E, k, p.norm, who, pw);
    if (lane < k) tidx[t * k + lane] = who, p.idx[t * k + lane] = who, p.wt[t * k + lane] = pw;
    if (lane == 0) p.sg[t] = p.shared_gate ? 1.f / (1.f + expf(-gate)) : 1.f;
  }
  __syncthreads();
  // The distinct experts in pick order, one thread per pick q (q < T k <= 256, waves 0-3): its expert's first pick
  // (an LDS atomic min), then that first pick's rank among the first picks (ballot counts): the unique slot u.
  static_assert(NTHR >= kMdecMaxT * kMdecMaxK, "one thread per pick");
  if (tid < NU) atomicMin(&firstpick[tidx[tid]], tid);
  __syncthreads();
  const int f = tid < NU ? firstpick[tidx[tid]] : 0;
  const bool first = tid < NU && f == tid;
  int rank = 0;
  if (wave < 4) {
    const unsigned long long m = __ballot(first);
    if (lane == 0) wcount[wave] = __popcll(m);
    rank = __popcll(m & ((1ull << lane) - 1));
  }
  __syncthreads();
  if (first) {
    int u = rank;
    for (int w = 0; w < wave; w++) u += wcount[w];
    urank[tid] = u;
    p.plan[1 + u] = tidx[tid];
  }
  __syncthreads();
  if (tid < NU) upick[urank[f] * kMdecMaxT + tid / k] = tid % k;
  if (tid == 0) p.plan[0] = wcount[0] + wcount[1] + wcount[2] + wcount[3];
}

template <int RT>
__global__ __launch_bounds__(512) void k_mdec_router(MdecArgs p) {
  __shared__ float red[8][64][RT];
  __shared__ unsigned s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 31, h = lane >> 5;
  const int e0 = blockIdx.x * 32, ks = blockIdx.y;
  const int Kc = p.H / (8 * p.KS), k0 = (ks * 8 + wave) * Kc;
  const bool tok = j < p.T, eok = e0 + j < p.E1;
  const uint16_t* xa = p.x + (size_t)(tok ? j : 0) * p.H + k0 + 32 * h;
  const uint16_t* wb = p.router + (size_t)(eok ? e0 + j : 0) * p.H + k0 + 32 * h;
  f32x16 acc = zero16();
  for (int kb = 0; kb < Kc; kb += 64) {
    u32x4 a[4], b[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      a[t] = tok ? *(const u32x4*)(xa + kb + 8 * t) : u32x4{0u, 0u, 0u, 0u};
      b[t] = eok ? *(const u32x4*)(wb + kb + 8 * t) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int t = 0; t < 4; t++) acc = mfma_bf16(a[t], b[t], acc);
  }
  // D row mdec_row(r, h) (r < RT) is that token, column j is expert e0 + j; the waves' K ranges summed in wave
  // order and written through for the block that routes
#pragma unroll
  for (int r = 0; r < RT; r++) red[wave][lane][r] = acc[r];
  __syncthreads();
  if (wave == 0) {
    const __amdgpu_buffer_rsrc_t rp = part_rsrc(p.part, (uint32_t)((size_t)p.KS * p.T * p.E1 * 4));
#pragma unroll
    for (int r = 0; r < RT; r++) {
      float v = red[0][lane][r];
#pragma unroll
      for (int w = 1; w < 8; w++) v += red[w][lane][r];
      const int t = mdec_row(r, h), e = e0 + j;
      if (t < p.T && e < p.E1)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rp, (int)((((size_t)ks * p.T + t) * p.E1 + e) * 4),
                                              0, kSc1);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const unsigned arrivals = gridDim.x * gridDim.y;
    unsigned* c = p.cnt + (kWsCounters - 1);
    const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == arrivals;
    if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (s_last) mdec_plan_block<512>(p);
}

// Routing and the plan from logits the caller computed (p.part = those logits, one split)
__global__ __launch_bounds__(512) void k_mdec_plan(MdecArgs p) { mdec_plan_block<512>(p); }

// The slot of block row u: a distinct routed expert (u < nuniq), the shared expert (u == T k), or nothing.
struct MdecSlot {
  int e;       // expert, or -1 for the shared expert
  bool live;
};
__device__ __forceinline__ MdecSlot mdec_slot(const MdecArgs& p, int u) {
  const int NU = p.T * p.k;
  if (u == NU) return MdecSlot{-1, p.has_sh != 0};
  return MdecSlot{u < p.plan[0] ? p.plan[1 + u] : 0, u < p.plan[0]};
}
// token t's pick index of slot u (k for the shared expert), or -1
__device__ __forceinline__ int mdec_pick(const MdecArgs& p, int u, int t) {
  const int NU = p.T * p.k;
  if (t >= p.T) return -1;
  return u == NU ? p.k : p.plan[1 + NU + u * kMdecMaxT + t];
}

// Stage rows [T][ng * 64] (row t from src(t), null = zeros) into LDS As (row stride lda) and their 64-group sums into
// Xs[g][t] (kMdecMaxT per group). nthr threads starting at thread `first`; every 8 consecutive chunks are one group, so the
// group sum is a reduction over 8 consecutive lanes.
// U chunks per thread are loaded before any is used (one memory latency per U passes, not per pass).
template <int U, class Src>
__device__ __forceinline__ void mdec_stage(Src src, int T, int ng, uint16_t* As, int lda, float* Xs, int first,
                                           int nthr) {
  const int cpr = ng * 8, total = T * cpr, me = (int)threadIdx.x - first;
  for (int c0 = 0; c0 < total; c0 += U * nthr) {
    u32x4 v[U];
#pragma unroll
    for (int q = 0; q < U; q++) {
      const int c = c0 + q * nthr + me;
      const bool ok = c < total;
      const uint16_t* s = ok ? src(c / cpr) : nullptr;
      v[q] = s ? *(const u32x4*)(s + 8 * (c % cpr)) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < U; q++) {
      const int c = c0 + q * nthr + me;
      const bool ok = c < total;
      const int t = ok ? c / cpr : 0, kc = ok ? c % cpr : 0;
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 4; e++) sum += bf2f((uint16_t)(v[q][e] & 0xFFFFu)) + bf2f((uint16_t)(v[q][e] >> 16));
      sum += __shfl_xor(sum, 1, 64);
      sum += __shfl_xor(sum, 2, 64);
      sum += __shfl_xor(sum, 4, 64);
      if (ok) {
        *(u32x4*)(As + (size_t)t * lda + 8 * kc) = v[q];
        if ((kc & 7) == 0) Xs[(kc >> 3) * kMdecMaxT + t] = sum;
      }
    }
  }
}

// One wave's share of a qmv4-arithmetic product: 32 weight rows (wrow: the lane's row, offset 4 h words) over ng
// groups starting at group g0 of the row, against the staged token rows As (row j of the MFMA A operand = token j,
// zero past T). Adds s P + (b - 128 s) X of each group into acc[r] (rows mdec_row(r, h), r < RT).
struct MdecW {
  const uint32_t* w;  // row words + 4 h
  const uint16_t* s;  // row scales
  const uint16_t* b;  // row biases
};

// ---- 3. gate/up + SwiGLU -------------------------------------------------------------------------------------------
// LDS of k_mdec_gu for T tokens: per wave its staged rows [T][kMdecKG * 64 + 8] and group sums [kMdecKG][kMdecMaxT]
// (then the waves' sums [4][64][2 RT])
constexpr int kMdecGuRow = kMdecKG * 64 + 8;
__host__ __device__ constexpr size_t mdec_gu_lds(int T, int RT) {
  return (size_t)4 * T * kMdecGuRow * 2 + (size_t)4 * kMdecKG * kMdecMaxT * 4 + (size_t)4 * 64 * 2 * RT * 4;
}

// SB: the shared expert's width (8: the reference's moe_gu2_4_8, a kernel of its own, so that the 4-bit form keeps its
// registers)
// three waves per SIMD up to 8 tokens (three blocks of 8 staged rows fit the LDS), two beyond
template <int RT, int SB>
__global__ __launch_bounds__(256, RT == 4 ? 3 : 2) void k_mdec_gu(MdecArgs p) {
  extern __shared__ __align__(16) uint8_t glds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 31, h = lane >> 5;
  const int u = blockIdx.y, T = p.T, I = p.I, H = p.H, G = H / kGroup, Gw = G / 4;
  uint16_t* const As = (uint16_t*)glds + (size_t)wave * T * kMdecGuRow;
  float* const Xs = (float*)(glds + (size_t)4 * T * kMdecGuRow * 2) + wave * kMdecKG * kMdecMaxT;
  float* const red = (float*)(glds + (size_t)4 * T * kMdecGuRow * 2 + (size_t)4 * kMdecKG * kMdecMaxT * 4);
  auto RED = [&](int w, int l, int r) -> float& { return red[((size_t)w * 64 + l) * 2 * RT + r]; };
  const MdecSlot sl = mdec_slot(p, u);
  if (!sl.live) return;  // block-uniform, before any barrier
  const int n0 = blockIdx.x * 32;
  const size_t rows0 = sl.e < 0 ? 0 : (size_t)sl.e * 2 * I;
  const uint32_t* wq = sl.e < 0 ? p.sgu_wq : p.egu_wq;
  const uint16_t* ws = sl.e < 0 ? p.sgu_s : p.egu_s;
  const uint16_t* wb = sl.e < 0 ? p.sgu_b : p.egu_b;
  const size_t rg = rows0 + n0 + j, ru = rg + I;
  const bool aok = j < T;

  float ag[RT], au[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) ag[r] = au[r] = 0.f;
  // the product for codes of B bits (4: the routed experts and a 4-bit shared expert; 8: an 8-bit shared expert,
  // the qmv8 arithmetic s P + b X)
  auto run = [&](auto bits_c) __attribute__((always_inline)) {
  constexpr int B = decltype(bits_c)::value;
  // groups per chunk: 8-bit chunks hold half the groups, so that the code registers are those of a 4-bit chunk
  constexpr int KG = B == 8 ? kMdecKG / 2 : kMdecKG;
  const size_t wpr = (size_t)H * B / 32;  // words per row
  const MdecW Wg{wq + rg * wpr + 4 * h, ws + rg * G, wb + rg * G};
  const MdecW Wu{wq + ru * wpr + 4 * h, ws + ru * G, wb + ru * G};
  for (int c0 = 0; c0 < Gw; c0 += KG) {
    const int gb = wave * Gw + c0, ng = min(KG, Gw - c0);
    // every load of the chunk first (clamped re-reads past ng keep the count fixed), then the token rows
    GroupCodes<B> cg[KG], cu[KG];
    uint16_t sgr[kMdecKG], bgr[kMdecKG], sur[kMdecKG], bur[kMdecKG];
#pragma unroll
    for (int i = 0; i < KG; i++) {
      const int g = gb + min(i, ng - 1);
      cg[i].load(Wg.w, g);
      cu[i].load(Wu.w, g);
    }
    if (B == 4 && p.sb16_gu) {  // whole chunks of 8 groups at 16-byte aligned offsets (block-uniform)
      load8h(Wg.s + gb, sgr), load8h(Wg.b + gb, bgr), load8h(Wu.s + gb, sur), load8h(Wu.b + gb, bur);
    } else {
#pragma unroll
      for (int i = 0; i < KG; i++) {
        const int g = gb + min(i, ng - 1);
        sgr[i] = Wg.s[g], bgr[i] = Wg.b[g], sur[i] = Wu.s[g], bur[i] = Wu.b[g];
      }
    }
    if (c0 > 0) __syncthreads();  // the previous chunk's reads of As are done (every wave runs the same chunks)
    mdec_stage<kMdecStageU>([&](int t) { return p.x + (size_t)t * H + (size_t)gb * 64; }, T, ng, As, kMdecGuRow, Xs,
                            wave * 64, 64);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KG; i++) {
      if (i >= ng) break;
      f32x16 Pg = zero16(), Pu = zero16();
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const u32x4 af = aok ? *(const u32x4*)(As + (size_t)j * kMdecGuRow + 64 * i + GroupCodes<B>::kofs(t, h))
                             : u32x4{0u, 0u, 0u, 0u};
        Pg = mfma_bf16(af, cg[i].step_affine(t, 0u), Pg);
        Pu = mfma_bf16(af, cu[i].step_affine(t, 0u), Pu);
      }
      const float sgf = bf2f(sgr[i]), bgf = affine_bias<B>(sgf, bf2f(bgr[i]));
      const float suf = bf2f(sur[i]), buf = affine_bias<B>(suf, bf2f(bur[i]));
#pragma unroll
      for (int r = 0; r < RT; r++) {
        const float X = Xs[i * kMdecMaxT + mdec_row(r, h)];
        ag[r] = __builtin_fmaf(sgf, Pg[r], __builtin_fmaf(bgf, X, ag[r]));
        au[r] = __builtin_fmaf(suf, Pu[r], __builtin_fmaf(buf, X, au[r]));
      }
    }
  }
  };
  if constexpr (SB == 8) {
    if (sl.e < 0) run(std::integral_constant<int, 8>{});  // block-uniform
    else run(std::integral_constant<int, 4>{});
  } else {
    run(std::integral_constant<int, 4>{});
  }
#pragma unroll
  for (int r = 0; r < RT; r++) RED(wave, lane, r) = ag[r], RED(wave, lane, RT + r) = au[r];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    const int t = mdec_row(r, h), pk = mdec_pick(p, u, t);
    if (pk < 0) continue;
    const float g = RED(0, lane, r) + RED(1, lane, r) + RED(2, lane, r) + RED(3, lane, r);
    const float v = RED(0, lane, RT + r) + RED(1, lane, RT + r) + RED(2, lane, RT + r) + RED(3, lane, RT + r);
    p.act[((size_t)t * (p.k + 1) + pk) * I + n0 + j] = f2bf(swiglu_f(bf2f(f2bf(g)), bf2f(f2bf(v))));
  }
}

// The combine of 128-column chunk blockIdx.x, by the last down block of that chunk: out[t][h] = bf16(acc) or
// bf16(out + bf16(acc)), acc = sum_j wt[t][j] d[t][j][h] + sg[t] d[t][k][h] in slot order (rd: d, written through).
template <int CB = kMdecCmbB, int CW = 128>
__device__ __forceinline__ void mdec_combine(const MdecArgs& p, __amdgpu_buffer_rsrc_t rd) {
  const int tid = threadIdx.x, T = p.T, H = p.H, k = p.k;
  const int nj = k + (p.has_sh || p.ys ? 1 : 0);
  if (p.out16) {
    // eight columns per thread (16-byte loads and stores; out and ys 16-byte aligned), CB slots' loads in
    // flight at once, summed in slot order
    for (int i = tid; i < T * (CW / 8); i += 256) {
      const int t = i / (CW / 8), hc = blockIdx.x * CW + (i % (CW / 8)) * 8;
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; e++) a[e] = 0.f;
      for (int j0 = 0; j0 < nj; j0 += CB) {
        u32x4 dv[CB];
        float wv[CB];
#pragma unroll
        for (int z = 0; z < CB; z++) {
          const int jj = j0 + z;
          if (jj < nj) {
            dv[z] = jj == k && p.ys ? *(const u32x4*)(p.ys + (size_t)t * H + hc)
                                    : __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                    rd, (int)((((size_t)t * (k + 1) + jj) * H + hc) * 2),
                                                                    0, kSc1));
            wv[z] = jj < k ? p.wt[t * k + jj] : p.sg[t];
          }
        }
#pragma unroll
        for (int z = 0; z < CB; z++)
          if (j0 + z < nj)
#pragma unroll
            for (int e = 0; e < 8; e++)
              a[e] = __builtin_fmaf(wv[z], bf2f((uint16_t)(dv[z][e / 2] >> (16 * (e & 1)))), a[e]);
      }
      u32x4* o = (u32x4*)(p.out + (size_t)t * H + hc);
      const u32x4 ov = p.assign ? u32x4{0u, 0u, 0u, 0u} : *o;
      u32x4 res;
#pragma unroll
      for (int e2 = 0; e2 < 4; e2++) {
        float v[2];
#pragma unroll
        for (int f = 0; f < 2; f++) {
          const int e = 2 * e2 + f;
          v[f] = p.assign ? a[e] : bf2f((uint16_t)(ov[e2] >> (16 * f))) + bf2f(f2bf(a[e]));
        }
        res[e2] = pack_bf2(v[0], v[1]);
      }
      *o = res;
    }
    return;
  }
  for (int i = tid; i < T * CW; i += 256) {
    const int t = i / CW, hc = blockIdx.x * CW + (i % CW);
    // every slot's value and weight requested before the first is used, then summed in slot order
    uint16_t dv[kMdecMaxK + 1];
    float wv[kMdecMaxK + 1];
#pragma unroll
    for (int jj = 0; jj <= kMdecMaxK; jj++)
      if (jj < nj) {
        dv[jj] = jj == k && p.ys ? p.ys[(size_t)t * H + hc]
                                 : __builtin_amdgcn_raw_buffer_load_b16(
                                       rd, (int)((((size_t)t * (k + 1) + jj) * H + hc) * 2), 0, kSc1);
        wv[jj] = jj < k ? p.wt[t * k + jj] : p.sg[t];
      }
    float a = 0.f;
#pragma unroll
    for (int jj = 0; jj <= kMdecMaxK; jj++)
      if (jj < nj) a = __builtin_fmaf(wv[jj], bf2f(dv[jj]), a);
    uint16_t* o = p.out + (size_t)t * H + hc;
    *o = p.assign ? f2bf(a) : f2bf(bf2f(*o) + bf2f(f2bf(a)));
  }
}

// ---- 4. down + combine ---------------------------------------------------------------------------------------------
template <int RT, int SB>
__global__ __launch_bounds__(256) void k_mdec_dn(MdecArgs p) {
  extern __shared__ __align__(16) uint16_t lds[];  // As [T][I + 8], then Xs [I / 64][kMdecMaxT]
  __shared__ unsigned s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 31, h = lane >> 5;
  const int u = blockIdx.y, T = p.T, I = p.I, H = p.H, Gi = I / kGroup, k = p.k;
  const MdecSlot sl = mdec_slot(p, u);
  if (!sl.live) return;  // block-uniform, before any barrier
  const int lda = I + 8;
  uint16_t* As = lds;
  float* Xs = (float*)(lds + (size_t)T * lda + 8);  // 16-byte aligned: T lda + 8 is a multiple of 8
  const int h0 = blockIdx.x * 128 + wave * 32;
  const size_t row = (sl.e < 0 ? 0 : (size_t)sl.e * H) + h0 + j;
  const uint16_t* ws = (sl.e < 0 ? p.sdn_s : p.edn_s) + row * Gi;
  const uint16_t* wb = (sl.e < 0 ? p.sdn_b : p.edn_b) + row * Gi;
  const bool aok = j < T;

  float acc[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) acc[r] = 0.f;
  // codes of B bits, as in k_mdec_gu
  auto run = [&](auto bits_c) __attribute__((always_inline)) {
  constexpr int B = decltype(bits_c)::value;
  constexpr int KG = B == 8 ? kMdecKG / 2 : kMdecKG;  // as in k_mdec_gu
  const uint32_t* wq = (sl.e < 0 ? p.sdn_wq : p.edn_wq) + row * ((size_t)I * B / 32) + 4 * h;
  for (int c0 = 0; c0 < Gi; c0 += KG) {
    const int ng = min(KG, Gi - c0);
    GroupCodes<B> cw[KG];
    uint16_t sr[kMdecKG], br[kMdecKG];
#pragma unroll
    for (int i = 0; i < KG; i++) {
      const int g = c0 + min(i, ng - 1);
      cw[i].load(wq, g);
    }
    if (B == 4 && p.sb16_dn) {
      load8h(ws + c0, sr), load8h(wb + c0, br);
    } else {
#pragma unroll
      for (int i = 0; i < KG; i++) {
        const int g = c0 + min(i, ng - 1);
        sr[i] = ws[g], br[i] = wb[g];
      }
    }
    if (c0 == 0) {  // the activation rows of the tokens that picked this slot (zero rows for the others)
      mdec_stage<2>(  // T / 4 passes of 256 threads at most: two in flight
          [&](int t) -> const uint16_t* {
            const int pk = mdec_pick(p, u, t);
            return pk < 0 ? nullptr : p.act + ((size_t)t * (k + 1) + pk) * I;
          },
          T, Gi, As, lda, Xs, 0, 256);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < KG; i++) {
      if (i >= ng) break;
      const int g = c0 + i;
      f32x16 P = zero16();
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const u32x4 af = aok ? *(const u32x4*)(As + (size_t)j * lda + 64 * g + GroupCodes<B>::kofs(t, h))
                             : u32x4{0u, 0u, 0u, 0u};
        P = mfma_bf16(af, cw[i].step_affine(t, 0u), P);
      }
      const float sf = bf2f(sr[i]), bf = affine_bias<B>(sf, bf2f(br[i]));
#pragma unroll
      for (int r = 0; r < RT; r++)
        acc[r] = __builtin_fmaf(sf, P[r], __builtin_fmaf(bf, Xs[g * kMdecMaxT + mdec_row(r, h)], acc[r]));
    }
  }
  };
  if constexpr (SB == 8) {
    if (sl.e < 0) run(std::integral_constant<int, 8>{});  // block-uniform
    else run(std::integral_constant<int, 4>{});
  } else {
    run(std::integral_constant<int, 4>{});
  }
  // d[t][pick][h] = bf16(result), written through for the combining block
  const __amdgpu_buffer_rsrc_t rd = part_rsrc(p.d, p.d_bytes);
#pragma unroll
  for (int r = 0; r < RT; r++) {
    const int t = mdec_row(r, h), pk = mdec_pick(p, u, t);
    if (pk >= 0)
      __builtin_amdgcn_raw_buffer_store_b16(f2bf(acc[r]), rd, (int)((((size_t)t * (k + 1) + pk) * H + h0 + j) * 2), 0,
                                            kSc1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const unsigned arrivals = (unsigned)p.plan[0] + (p.has_sh ? 1u : 0u);
    const unsigned old = __hip_atomic_fetch_add(p.cnt + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == arrivals;
    if (last) __hip_atomic_store(p.cnt + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  mdec_combine(p, rd);
}

// ---- the T64 path: expert stacks in the T64 layout, each wave streaming one band -----------------------------------
// A wave streams its band's 1152-byte (group, band) tiles, 16 bytes per lane of one tile per group, in ping-pong
// blocks of kMdtTB groups with the next block requested before the current one is used (non-temporal loads: each
// tile is read once). The arithmetic is the qmv4 arithmetic of the MLX-layout kernels: codes as exact bf16 128 + q,
// P = sum x (128 + q) by bf16 MFMA, s P + (b - 128 s) X per group with the group sums X of the staged token rows.
constexpr int kMdtTB = 2;
constexpr int kMdtMaxT = kMdecMaxT;  // tokens per launch: RT = 4 accumulator rows up to 8, 8 up to 16
struct MdtBlk {
  u32x4 w[kMdtTB];
  uint32_t sb[kMdtTB];
};
// Stage rows [T][ng 64] of this slot's tokens (row t from src(t), zeros for null) into As (row stride lda) and their
// 64-group sums into Xs[g][16] (rows past T zero), by the block's 256 threads.
template <class Src>
__device__ __forceinline__ void mdt_stage(Src src, int T, int ng, uint16_t* As, int lda, float* Xs) {
  mdec_stage<kMdecStageU>(src, T, ng, As, lda, Xs, 0, 256);
  for (int i = threadIdx.x; i < ng * kMdecMaxT; i += 256)
    if ((i & (kMdecMaxT - 1)) >= T) Xs[i] = 0.f;
}
// One wave's product over groups [g0, g1) of NB bands, streamed as one sequence band by band (with NB > 1, g1 - g0
// is a multiple of kMdtTB, so that a ping-pong block never spans two bands): tcol = the first band's first tile,
// bstride = bytes
// between the bands, gstride = bytes between groups; As / Xs staged from group g0 on. acc[b][r] (r < RT): token row
// mdec_row(r, h), column j of band b.
template <int NB, int RT>
__device__ __forceinline__ void mdt_band(const uint8_t* tcol, size_t bstride, size_t gstride, int g0, int g1,
                                         const uint16_t* As, int lda, const float* Xs, int T, f32x16 (&acc)[NB]) {
  const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  const bool aok = j < T;
  const uint16_t* arow = As + (size_t)(aok ? j : 0) * lda + 32 * h;
  const int ng = g1 - g0, n = NB * ng;  // steps: (band, group) band-major
  auto load_blk = [&](MdtBlk& B, int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kMdtTB; i++) {
      const int q = min(s + i, n - 1), b = q / ng;
      const uint8_t* t = tcol + (size_t)b * bstride + (size_t)(g0 + q - b * ng) * gstride;
      B.w[i] = __builtin_nontemporal_load((const u32x4*)(t + 16 * lane));
      B.sb[i] = __builtin_nontemporal_load((const uint32_t*)(t + kT64Codes + 4 * j));
    }
  };
  auto compute_blk = [&](const MdtBlk& B, int s) __attribute__((always_inline)) {
    const int b = NB == 1 ? 0 : s / ng;  // the block's band
#pragma unroll
    for (int i = 0; i < kMdtTB; i++) {
      if (s + i >= n) break;
      const int gl = s + i - b * ng;
      u32x4 af[4];
#pragma unroll
      for (int t = 0; t < 4; t++) af[t] = aok ? *(const u32x4*)(arow + (size_t)gl * 64 + 8 * t) : u32x4{0u, 0u, 0u, 0u};
      const float4 x0 = *(const float4*)(Xs + gl * kMdecMaxT + 4 * h);
      float4 x1 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (RT > 4) x1 = *(const float4*)(Xs + gl * kMdecMaxT + 8 + 4 * h);
      f32x16 P = zero16();
#pragma unroll
      for (int t = 0; t < 4; t++) P = mfma_bf16(af[t], t64_off128(B.w[i][t]), P);
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      const float sc = bf2f((uint16_t)(B.sb[i] & 0xFFFFu)), bi = bf2f((uint16_t)(B.sb[i] >> 16));
      const float bp = __builtin_fmaf(-128.f, sc, bi);
#pragma unroll
      for (int bb = 0; bb < NB; bb++)
        if (bb == b)
#pragma unroll
          for (int r = 0; r < RT; r++) acc[bb][r] = __builtin_fmaf(sc, P[r], __builtin_fmaf(bp, xs[r], acc[bb][r]));
    }
  };
  MdtBlk b0, b1;
  load_blk(b0, 0);
  for (int s = 0;; s += 2 * kMdtTB) {
    load_blk(b1, min(s + kMdtTB, n - 1));
    compute_blk(b0, s);
    if (s + kMdtTB >= n) break;
    load_blk(b0, min(s + 2 * kMdtTB, n - 1));
    compute_blk(b1, s + kMdtTB);
    if (s + 2 * kMdtTB >= n) break;
  }
}

// Gate/up + SwiGLU: block = (64 h columns c, slot u, K split z). Waves 0, 1 stream gate bands 2c, 2c + 1 of the
// slot's expert, waves 2, 3 the matching up bands I / 32 + 2c, + 1, over groups [z gps, (z + 1) gps). With one split
// the block pairs gate and up through LDS and writes h; with several each block writes its fp32 sums (write-through)
// and the last of a (slot, c)'s splits (a counter in the workspace header) sums them in split order and writes h.
template <int RT>
__global__ __launch_bounds__(256) void k_mdt_gu(MdecArgs p) {
  extern __shared__ __align__(16) uint16_t lds[];
  __shared__ float red[4][64][RT];
  __shared__ unsigned s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 31, h = lane >> 5;
  const int c = blockIdx.x, u = blockIdx.y, z = blockIdx.z, T = p.T, H = p.H, I = p.I, nct = I / 64;
  const MdecSlot sl = mdec_slot(p, u);
  if (!sl.live) return;  // block-uniform, before any barrier
  const int G = H / kGroup, g0 = z * p.gps, g1 = min(G, g0 + p.gps), ng = g1 - g0, lda = ng * 64 + 8;
  uint16_t* As = lds;
  float* Xs = (float*)(lds + (size_t)T * lda + 8);  // 16-byte aligned: T lda + 8 is a multiple of 8
  mdt_stage([&](int t) { return p.x + (size_t)t * H + (size_t)g0 * 64; }, T, ng, As, lda, Xs);
  __syncthreads();
  const uint8_t* stack = sl.e < 0 ? p.sgu_t : p.egu_t + (size_t)sl.e * p.gu_eb;
  const int band = wave < 2 ? 2 * c + wave : I / 32 + 2 * c + wave - 2, nb = 2 * I / 32;
  f32x16 accs[1] = {zero16()};
  mdt_band<1, RT>(stack + (size_t)band * kT64Tile, 0, (size_t)nb * kT64Tile, g0, g1, As, lda, Xs, T, accs);
  f32x16& acc = accs[0];
  if (p.gS > 1) {  // this split's sums, then the (slot, c) tile's last split sums them all
    const __amdgpu_buffer_rsrc_t rg = part_rsrc(p.gpart, p.gpart_bytes);
    // a split's sums: [4 waves][RT / 4 quads][64 lanes] 16-byte quads
    constexpr int NQ = RT / 4;
    const int slot = (u * nct + c) * p.gS + z;
#pragma unroll
    for (int q4 = 0; q4 < NQ; q4++) {
      const u32x4 v = {__float_as_uint(acc[4 * q4]), __float_as_uint(acc[4 * q4 + 1]), __float_as_uint(acc[4 * q4 + 2]),
                       __float_as_uint(acc[4 * q4 + 3])};
      __builtin_amdgcn_raw_buffer_store_b128(v, rg, (int)(((((size_t)slot * 4 + wave) * NQ + q4) * 64 + lane) * 16),
                                             0, kSc1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      unsigned* ctr = p.cnt + u * nct + c;
      const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old + 1 == (unsigned)p.gS;
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next call
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    float a[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) a[r] = 0.f;
    for (int z0 = 0; z0 < p.gS; z0 += 4) {  // four splits' loads in flight, summed in split order
      u32x4 w[4][NQ];
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (z0 + q < p.gS)
#pragma unroll
          for (int q4 = 0; q4 < NQ; q4++)
            w[q][q4] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           rg, (int)((((((size_t)(u * nct + c) * p.gS + z0 + q) * 4 + wave) * NQ + q4) * 64 + lane) *
                                     16), 0, kSc1));
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (z0 + q < p.gS)
#pragma unroll
          for (int r = 0; r < RT; r++) a[r] += __uint_as_float(w[q][r / 4][r % 4]);
    }
#pragma unroll
    for (int r = 0; r < RT; r++) acc[r] = a[r];
  }
  // gate (waves 0, 1) with up (waves 2, 3): h = silu(bf16(gate)) bf16(up) for the tokens that picked the slot
#pragma unroll
  for (int r = 0; r < RT; r++) red[wave][lane][r] = acc[r];
  __syncthreads();
  if (wave >= 2) return;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    const int t = mdec_row(r, h), pk = mdec_pick(p, u, t);
    if (pk < 0) continue;
    const float g = red[wave][lane][r], v = red[wave + 2][lane][r];
    p.act[((size_t)t * (p.k + 1) + pk) * I + 64 * c + 32 * wave + j] = f2bf(swiglu_f(bf2f(f2bf(g)), bf2f(f2bf(v))));
  }
}

// Down + combine: block = (128 NB output columns, slot u); wave w streams bands NB (4 x + w) .. + NB - 1
// of the slot's down rows over all I / 64 groups against the act rows of the tokens that picked it (the staging and
// the block's fixed costs shared by more weight bytes), d[t][pick][h] = bf16(result) written through; the last block
// of a chunk (a counter in the workspace header) combines its columns, as k_mdec_dn.
template <int NB, int RT>
__global__ __launch_bounds__(256) void k_mdt_dn(MdecArgs p) {
  extern __shared__ __align__(16) uint16_t lds[];
  __shared__ unsigned s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 31, h = lane >> 5;
  const int u = blockIdx.y, T = p.T, I = p.I, H = p.H, Gi = I / kGroup, k = p.k;
  const MdecSlot sl = mdec_slot(p, u);
  if (!sl.live) return;  // block-uniform, before any barrier
  const int lda = I + 8;
  uint16_t* As = lds;
  float* Xs = (float*)(lds + (size_t)T * lda + 8);
  mdt_stage(
      [&](int t) -> const uint16_t* {
        const int pk = mdec_pick(p, u, t);
        return pk < 0 ? nullptr : p.act + ((size_t)t * (k + 1) + pk) * I;
      },
      T, Gi, As, lda, Xs);
  __syncthreads();
  const uint8_t* stack = sl.e < 0 ? p.sdn_t : p.edn_t + (size_t)sl.e * p.dn_eb;
  const int band = (blockIdx.x * 4 + wave) * NB, nb = H / 32;
  f32x16 acc[NB];
#pragma unroll
  for (int bb = 0; bb < NB; bb++) acc[bb] = zero16();
  mdt_band<NB, RT>(stack + (size_t)band * kT64Tile, kT64Tile, (size_t)nb * kT64Tile, 0, Gi, As, lda, Xs, T, acc);
  const __amdgpu_buffer_rsrc_t rd = part_rsrc(p.d, p.d_bytes);
#pragma unroll
  for (int bb = 0; bb < NB; bb++) {
    const int h0 = (band + bb) * 32;
#pragma unroll
    for (int r = 0; r < RT; r++) {
      const int t = mdec_row(r, h), pk = mdec_pick(p, u, t);
      if (pk >= 0)
        __builtin_amdgcn_raw_buffer_store_b16(f2bf(acc[bb][r]), rd,
                                              (int)((((size_t)t * (k + 1) + pk) * H + h0 + j) * 2), 0, kSc1);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const unsigned arrivals = (unsigned)p.plan[0] + (p.has_sh ? 1u : 0u);
    const unsigned old = __hip_atomic_fetch_add(p.cnt + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == arrivals;
    if (last) __hip_atomic_store(p.cnt + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  mdec_combine<4, 128 * NB>(p, rd);  // a small batch: fewer registers, more of this kernel's waves in flight
}

// ---- host ------------------------------------------------------------------------------------------------------------
// K splits of the router: each of a block's 8 waves takes H / (8 KS) columns, a multiple of 64
static int mdec_ks(int H) {
  for (int ks : {4, 2, 1})
    if (H % (512 * ks) == 0) return ks;
  return 0;
}

// The T64 path's gate/up K split: about 6 waves per SIMD over the T k + 1 slots (most of them live), whole blocks of
// kMdtTB groups and at least two per split, and a counter per (slot, 64-column tile) below the router's.
static void mdt_split(int T, int H, int I, int k, int& S, int& gps) {
  const int slots = T * k + 1, nct = I / 64, G = H / kGroup;
  S = (int)std::min<long>((6144l + (long)slots * nct * 4 - 1) / ((long)slots * nct * 4), G / (2 * kMdtTB));
  if (S < 1 || (long)slots * nct > kWsCounters - 2) S = 1;
  gps = (G + S - 1) / S;
  gps = (gps + kMdtTB - 1) / kMdtTB * kMdtTB;
  S = (G + gps - 1) / gps;
}

MdecLayout mdec_layout(int T, int H, int I, int E, int k, bool t64) {
  MdecLayout L{};
  auto take = [&](size_t& off, size_t bytes) {
    off = L.total;
    L.total = align_up(L.total + bytes, 256);
  };
  const int E1 = E + 1, KS = mdec_ks(H);
  take(L.part, (size_t)KS * T * E1 * 4);
  take(L.plan, (size_t)(1 + (1 + kMdecMaxT) * T * k) * 4);
  take(L.act, (size_t)T * (k + 1) * I * 2);
  take(L.d, (size_t)T * (k + 1) * H * 2);
  take(L.idx, (size_t)T * k * 4);
  take(L.wt, (size_t)T * k * 4);
  take(L.sg, (size_t)T * 4);
  L.gS = 1, L.gps = H / kGroup;
  if (t64) {
    mdt_split(T, H, I, k, L.gS, L.gps);
    take(L.gpart, L.gS > 1 ? (size_t)(T * k + 1) * (I / 64) * L.gS * 4 * 64 * 16 * (T > 8 ? 2 : 1) : 0);
  }
  return L;
}

template <int RT>
static int launch_mdec(const MdecArgs& p, const MdecCall& c, hipStream_t st) {
  const int slots = c.T * c.k + 1;
  if (c.logits_in || c.routed) hipLaunchKernelGGL(k_mdec_plan, dim3(1), dim3(512), 0, st, p);
  else hipLaunchKernelGGL(k_mdec_router<RT>, dim3((p.E1 + 31) / 32, p.KS), dim3(512), 0, st, p);
  IFD_TRY(check_launch("moe_decode router"));
  // up to 16 tokens the staged rows can take more than the default 64 KB of dynamic LDS
  auto allow_lds = [](const void* k, size_t bytes, const char* what) -> int {
    if (bytes <= 64 * 1024) return IFD_OK;
    if (bytes > 150 * 1024) return fail(IFD_ERR_UNSUPPORTED, "moe_decode %s: %zu bytes of LDS", what, bytes);
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) {
      (void)hipGetLastError();
      return fail(IFD_ERR_LAUNCH, "moe_decode %s: %zu bytes of LDS refused", what, bytes);
    }
    return IFD_OK;
  };
  if (p.egu_t) {  // the T64 path
    const size_t glds = ((size_t)c.T * (p.gps * 64 + 8) + 8) * 2 + (size_t)p.gps * kMdecMaxT * 4;
    IFD_TRY(allow_lds((const void*)k_mdt_gu<RT>, glds, "gate_up"));
    hipLaunchKernelGGL(k_mdt_gu<RT>, dim3(c.I / 64, slots, p.gS), dim3(256), glds, st, p);
    IFD_TRY(check_launch("moe_decode gate_up"));
    const size_t dlds = ((size_t)c.T * (c.I + 8) + 8) * 2 + (size_t)(c.I / kGroup) * kMdecMaxT * 4;
    // two bands per wave when one per wave would give more than four blocks per CU (config 4 at T = 8: 61.3 against
    // 66.1 us for the whole decode; at T <= 4 one band per wave keeps more blocks in flight: T = 1 / 2 / 4 32.9 /
    // 37.1 / 46.6 against 36.0 / 39.9 / 47.6 us) and a band's groups fill whole ping-pong blocks
    if ((long)slots * (c.H / 128) > 4l * cu_count() && (c.I / kGroup) % kMdtTB == 0) {
      IFD_TRY(allow_lds((const void*)k_mdt_dn<2, RT>, dlds, "down"));
      hipLaunchKernelGGL((k_mdt_dn<2, RT>), dim3(c.H / 256, slots), dim3(256), dlds, st, p);
    } else {
      IFD_TRY(allow_lds((const void*)k_mdt_dn<1, RT>, dlds, "down"));
      hipLaunchKernelGGL((k_mdt_dn<1, RT>), dim3(c.H / 128, slots), dim3(256), dlds, st, p);
    }
    return check_launch("moe_decode down");
  }
  const size_t glds = mdec_gu_lds(c.T, RT);
  const void* gu = p.sh_bits == 8 ? (const void*)k_mdec_gu<RT, 8> : (const void*)k_mdec_gu<RT, 4>;
  IFD_TRY(allow_lds(gu, glds, "gate_up"));
  if (p.sh_bits == 8) hipLaunchKernelGGL((k_mdec_gu<RT, 8>), dim3(c.I / 32, slots), dim3(256), glds, st, p);
  else hipLaunchKernelGGL((k_mdec_gu<RT, 4>), dim3(c.I / 32, slots), dim3(256), glds, st, p);
  IFD_TRY(check_launch("moe_decode gate_up"));
  const size_t lds = ((size_t)c.T * (c.I + 8) + 8) * 2 + (size_t)(c.I / kGroup) * kMdecMaxT * 4;
  const void* dn = p.sh_bits == 8 ? (const void*)k_mdec_dn<RT, 8> : (const void*)k_mdec_dn<RT, 4>;
  IFD_TRY(allow_lds(dn, lds, "down"));
  if (p.sh_bits == 8) hipLaunchKernelGGL((k_mdec_dn<RT, 8>), dim3(c.H / 128, slots), dim3(256), lds, st, p);
  else hipLaunchKernelGGL((k_mdec_dn<RT, 4>), dim3(c.H / 128, slots), dim3(256), lds, st, p);
  return check_launch("moe_decode down");
}

int launch_moe_decode(const MdecCall& c, unsigned* cnt, void* ws, size_t ws_bytes, hipStream_t st) {
  if (c.T == 0) return IFD_OK;
  // the caller's routing: every token's result depends on its own row only, so the launches take 16 tokens (8 on
  // T64 stacks) at a time on the one workspace (stream-ordered)
  const int group = c.egu_t64 ? kMdtMaxT : kMdecMaxT;
  if (c.routed && c.T > group) {
    for (int t0 = 0; t0 < c.T; t0 += group) {
      MdecCall cc = c;
      cc.T = std::min(group, c.T - t0);
      cc.xn = (const uint16_t*)c.xn + (size_t)t0 * c.H;
      cc.out = (uint16_t*)c.out + (size_t)t0 * c.H;
      cc.idx = c.idx + (size_t)t0 * c.k, cc.wt = c.wt + (size_t)t0 * c.k, cc.sg = c.sg ? c.sg + t0 : nullptr;
      cc.ys = c.ys ? (const uint16_t*)c.ys + (size_t)t0 * c.H : nullptr;
      IFD_TRY(launch_moe_decode(cc, cnt, ws, ws_bytes, st));
    }
    return IFD_OK;
  }
  if (c.T > kMdecMaxT) return fail(IFD_ERR_UNSUPPORTED, "moe_decode takes at most %d tokens", kMdecMaxT);
  const bool t64 = c.egu_t64 != nullptr;
  if (t64 && (c.T > kMdtMaxT || c.sh_bits != 4 || (c.sgu_t64 == nullptr) != (c.sdn_t64 == nullptr)))
    return fail(IFD_ERR_UNSUPPORTED, "moe_decode on T64 stacks: up to %d tokens, 4-bit shared expert", kMdtMaxT);
  const MdecLayout L = mdec_layout(c.T, c.H, c.I, c.E, c.k, t64);
  if (!ws || ws_bytes < L.total || !cnt)
    return fail(IFD_ERR_WORKSPACE, "moe_decode needs %zu bytes of workspace after the header, got %zu", L.total,
                ws_bytes);
  char* w = (char*)ws;
  MdecArgs p{};
  p.x = (const uint16_t*)c.xn;
  p.router = (const uint16_t*)c.router;
  p.T = c.T, p.H = c.H, p.E = c.E, p.E1 = c.E + (c.shared_gate ? 1 : 0), p.k = c.k, p.I = c.I;
  p.norm = c.norm, p.shared_gate = c.shared_gate, p.assign = c.assign, p.KS = mdec_ks(c.H);
  p.egu_wq = c.egu_wq, p.egu_s = c.egu_s, p.egu_b = c.egu_b;
  p.edn_wq = c.edn_wq, p.edn_s = c.edn_s, p.edn_b = c.edn_b;
  p.sgu_wq = c.sgu_wq, p.sgu_s = c.sgu_s, p.sgu_b = c.sgu_b;
  p.sdn_wq = c.sdn_wq, p.sdn_s = c.sdn_s, p.sdn_b = c.sdn_b;
  p.sh_bits = c.sh_bits;
  p.has_sh = c.sgu_wq || c.sgu_t64 ? 1 : 0;
  p.routed = c.routed, p.ys = (const uint16_t*)c.ys;
  p.out16 = ((uintptr_t)c.out % 16 == 0 && (uintptr_t)c.ys % 16 == 0) ? 1 : 0;
  p.out = (uint16_t*)c.out;
  p.idx = c.idx ? c.idx : (int*)(w + L.idx);
  p.wt = c.wt ? c.wt : (float*)(w + L.wt);
  p.sg = c.sg ? c.sg : (float*)(w + L.sg);
  p.logits = c.logits;
  p.part = c.logits_in ? (float*)c.logits_in : (float*)(w + L.part);
  if (c.logits_in) p.KS = 1;
  p.plan = (int*)(w + L.plan);
  p.act = (uint16_t*)(w + L.act);
  p.d = (uint16_t*)(w + L.d);
  p.d_bytes = (uint32_t)((size_t)c.T * (c.k + 1) * c.H * 2);
  p.cnt = cnt;
  if (t64) {
    p.egu_t = (const uint8_t*)c.egu_t64, p.edn_t = (const uint8_t*)c.edn_t64;
    p.sgu_t = (const uint8_t*)c.sgu_t64, p.sdn_t = (const uint8_t*)c.sdn_t64;
    p.gu_eb = t64_bytes(2 * c.I, c.H), p.dn_eb = t64_bytes(c.H, c.I);
    p.gS = L.gS, p.gps = L.gps;
    p.gpart = (float*)(w + L.gpart);
    p.gpart_bytes = (uint32_t)((size_t)(c.T * c.k + 1) * (c.I / 64) * L.gS * 4 * 64 * 16 * (c.T > 8 ? 2 : 1));
  }
  // vector scale / bias loads: every chunk holds 8 groups (the wave's group count a multiple of 8) and rows start
  // 16-byte aligned
  const bool shared = c.sgu_wq != nullptr;
  const int G = c.H / kGroup, Gi = c.I / kGroup;
  p.sb16_gu = (G / 4) % 8 == 0 && aligned(c.egu_s, 16) && aligned(c.egu_b, 16) &&
              (!shared || (aligned(c.sgu_s, 16) && aligned(c.sgu_b, 16)));
  p.sb16_dn = Gi % 8 == 0 && aligned(c.edn_s, 16) && aligned(c.edn_b, 16) &&
              (!shared || (aligned(c.sdn_s, 16) && aligned(c.sdn_b, 16)));
  if (c.T <= 8) return launch_mdec<4>(p, c, st);
  return launch_mdec<8>(p, c, st);
}

}  // namespace ifd
