// Device routing shared by the sorted MoE path (k_moe_route) and the decode MoE (k_mdec_plan): one wave routes one
// token. Softmax over E <= 512 logits in fp32 as exp(l - max) (8 per lane), top-k by repeated max scan (a tie goes
// to the lowest expert index), weights p / sum, renormalised over the k picks when norm != 0 (reference moe_route /
// moe_topk, engine/kernels/moe.metal:60-101, 295-324).
#pragma once
#include "common.h"

namespace ifd {

// v[i]: logit i * 64 + lane of the token (lanes past E: anything). On return lane j < k <= 16 holds pick j: its
// expert who and weight p.
// Each round takes the largest remaining value: its lowest index comes from a ballot when one lane holds it (a tie
// within the lane goes to the lower i by the strict compare), and from a min-reduction over the tied lanes'
// indices when several do. The weights are divided after the rounds, pick j in lane j, all in one instruction: the
// same quotients m / sum, and their total in pick order, as a division per round.
__device__ __forceinline__ void route_token(float (&v)[8], int E, int k, int norm, int& who, float& p) {
  const int lane = threadIdx.x & 63;
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    if (i * 64 + lane >= E) v[i] = -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
  mx = dpp_max_f(mx);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const bool ok = i * 64 + lane < E;
    const float ex = ok ? expf(v[i] - mx) : 0.f;
    sum += ex;
    v[i] = ok ? ex : -2.f;  // padding never wins a pick (picks need v > -1)
  }
  sum = dpp_sum_f(sum);
  float m_l = 0.f;
  int w_l = 0;
  for (int jj = 0; jj < k; jj++) {
    float best = -1.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (v[i] > best) best = v[i], bi = i * 64 + lane;  // strict >: lowest index of this lane wins a tie
    const float m = dpp_max_f(best);
    const unsigned long long hit = __ballot(best == m);
    const int w = __popcll(hit) == 1 ? __builtin_amdgcn_readlane(bi, __ffsll((long long)hit) - 1)
                                     : dpp_min_i(best == m ? bi : 0x7fffffff);
    if ((w & 63) == lane) {
#pragma unroll
      for (int i = 0; i < 8; i++)
        if (i == w / 64) v[i] = -1.f;
    }
    if (lane == jj) m_l = m, w_l = w;
  }
  p = m_l / sum;
  float tot = 0.f;
  for (int jj = 0; jj < k; jj++) tot += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), jj));
  if (norm) p = p / tot;
  who = w_l;
}

}  // namespace ifd
