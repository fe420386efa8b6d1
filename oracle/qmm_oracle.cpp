// CPU oracle for the W4 quantized-matmul hot path: a plain C++ restatement of the reference's semantics.
//
// TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
// library, and only as the checker or the timed CPU comparator. The product path (inferd_amd/) never calls it.
//
// Weight format (MLX affine, group 64; reference engine/src/weights.h:226-236, engine/kernels/core.metal:13-15):
//   Wq uint32 [N, K/8], element j of a little-endian word at bits 4j (low nibble first);
//   S, B bf16 [N, K/64];  w[n,k] = S[n,k/64] * q[n,k] + B[n,k/64],  q in 0..15.
//   "flipped" weights store q ^ 8 in every nibble (engine/kernels/w4a8.metal:17-22); xr = 0x88888888 undoes it.
// bf16 values are passed as uint16_t bit patterns; float<->bf16 is round-to-nearest-even (engine/src/weights.h:342-347).
//
// Every function runs over `nthreads` std::threads (0 = all hardware threads) and is deterministic: each output
// element's sum runs in a fixed order whatever the thread count.
//
// Pinning (tests/test_oracle.py): nibble unpack is checked exhaustively and against a hand-built vector; dequant by a
// one-hot activation probe and the all-8 (b = -8s) zero case; qmv/qmm/w4a8 against float64 textbook GEMMs in numpy
// and exact-rational known answers (tests/golden/); routing against a brute-force lexsort; dispatch against numpy's
// stable argsort; SwiGLU and combine against their closed forms; RMS norm against constant, one-hot and
// power-of-two-scaled rows whose outputs are exact.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
// round to nearest even, as engine/src/weights.h:343-347 (no NaN special case, like the reference)
inline uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
inline float bfround(float f) { return bf2f(f2bf(f)); }

template <class F>
void parallel_for(int n, int nthreads, F fn) {
  if (n <= 0) return;
  int T = nthreads > 0 ? nthreads : (int)std::max(1u, std::thread::hardware_concurrency());
  T = std::min(T, n);
  if (T == 1) {
    for (int i = 0; i < n; i++) fn(i);
    return;
  }
  std::vector<std::thread> th;
  th.reserve(T);
  for (int t = 0; t < T; t++)
    th.emplace_back([=, &fn] {
      // static block partition: which thread runs an index never changes a result
      const int lo = (int)((int64_t)n * t / T), hi = (int)((int64_t)n * (t + 1) / T);
      for (int i = lo; i < hi; i++) fn(i);
    });
  for (auto& x : th) x.join();
}

inline int code_at(const uint32_t* wrow, int k, uint32_t xr) { return (int)(((wrow[k >> 3] ^ xr) >> (4 * (k & 7))) & 15u); }
// 8-bit: byte k % 4 of word k / 4 (MLX affine 8-bit; reference qmv8, engine/kernels/core.metal:173-174, 224-228)
inline int code8_at(const uint32_t* wrow, int k, uint32_t xr) { return (int)(((wrow[k >> 2] ^ xr) >> (8 * (k & 3))) & 255u); }
inline int code_b(const uint32_t* wrow, int k, uint32_t xr, int bits) {
  return bits == 8 ? code8_at(wrow, k, xr) : code_at(wrow, k, xr);
}

}  // namespace

extern "C" {

int orc_version(void) { return 1; }

void orc_f32_to_bf16(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = f2bf(x[i]);
}
void orc_bf16_to_f32(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = bf2f(x[i]);
}

// codes uint8 [N, K] (values 0..15) -> Wq uint32 [N, K/8], low nibble first (engine/src/weights.h:398-400).
void orc_pack_w4(const uint8_t* codes, uint32_t* wq, int N, int K) {
  const int kw = K / 8;
  for (int n = 0; n < N; n++)
    for (int w = 0; w < kw; w++) {
      uint32_t v = 0;
      for (int j = 0; j < 8; j++) v |= (uint32_t)(codes[(size_t)n * K + w * 8 + j] & 15) << (4 * j);
      wq[(size_t)n * kw + w] = v;
    }
}
// Wq -> codes, undoing a flip with xr (0 or 0x88888888) (engine/kernels/core.metal:132-133).
void orc_unpack_w4(const uint32_t* wq, uint8_t* codes, int N, int K, uint32_t xr) {
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) codes[(size_t)n * K + k] = (uint8_t)code_at(wq + (size_t)n * (K / 8), k, xr);
}
// codes uint8 [N, K] (0..255) -> Wq uint32 [N, K/4], byte j of a word = element j (MLX affine 8-bit).
void orc_pack_w8(const uint8_t* codes, uint32_t* wq, int N, int K) {
  for (int n = 0; n < N; n++)
    for (int w = 0; w < K / 4; w++) {
      uint32_t v = 0;
      for (int j = 0; j < 4; j++) v |= (uint32_t)codes[(size_t)n * K + 4 * w + j] << (8 * j);
      wq[(size_t)n * (K / 4) + w] = v;
    }
}
void orc_unpack_w8(const uint32_t* wq, uint8_t* codes, int N, int K, uint32_t xr) {
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) codes[(size_t)n * K + k] = (uint8_t)code8_at(wq + (size_t)n * (K / 4), k, xr);
}
// In-place flip, engine/kernels/w4a8.metal:19-22 (mask 0x88888888 for 4-bit, 0x80808080 for 8-bit).
void orc_flip(uint32_t* wq, int64_t n32, uint32_t mask) {
  for (int64_t i = 0; i < n32; i++) wq[i] ^= mask;
}
// Dequantize to float: w = S*q + B in fp32 (the qmv semantics; the product S*q is exact in fp32).
void orc_dequant_f32(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, uint32_t xr, float* w) {
  const int kg = K / 64;
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) {
      const float sc = bf2f(s[(size_t)n * kg + k / 64]), bi = bf2f(b[(size_t)n * kg + k / 64]);
      w[(size_t)n * K + k] = sc * (float)code_at(wq + (size_t)n * (K / 8), k, xr) + bi;
    }
}
// Either width: w = S*q + B in fp32 (bits 4 or 8).
void orc_dequant_f32_b(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, int bits, uint32_t xr,
                       float* w) {
  const int kg = K / 64, kw = K * bits / 32;
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) {
      const float sc = bf2f(s[(size_t)n * kg + k / 64]), bi = bf2f(b[(size_t)n * kg + k / 64]);
      w[(size_t)n * K + k] = sc * (float)code_b(wq + (size_t)n * kw, k, xr, bits) + bi;
    }
}
// Dequantize to bf16 as MLX's qmm loader does: bf16(fp32(S*q + B)) (third_party/mlx/.../quantized.h:528-535).
void orc_dequant_bf16(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K, uint32_t xr, uint16_t* w) {
  const int kg = K / 64;
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) {
      const float sc = bf2f(s[(size_t)n * kg + k / 64]), bi = bf2f(b[(size_t)n * kg + k / 64]);
      w[(size_t)n * K + k] = f2bf(sc * (float)code_at(wq + (size_t)n * (K / 8), k, xr) + bi);
    }
}

// Decode GEMV semantics (engine/kernels/core.metal:85-171 qmv4, 175-248 qmv8): per 64-group g,
//   y[m,n] += S[n,g] * sum_{k in g} q[n,k] x[m,k] + B[n,g] * sum_{k in g} x[m,k], fp32 throughout.
// A bf16 [M, lda], Y fp32 [M, N] (the value before the bf16 store; see orc_store). bits 4 or 8.
void orc_qmv_b(const uint16_t* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
               int bits, uint32_t xr, float* Y, int M, int nthreads) {
  const int kg = K / 64, kw = K * bits / 32;
  std::vector<float> xf((size_t)M * K);
  for (int m = 0; m < M; m++)
    for (int k = 0; k < K; k++) xf[(size_t)m * K + k] = bf2f(A[(size_t)m * lda + k]);
  parallel_for(N, nthreads, [&](int n) {
    const uint32_t* wr = wq + (size_t)n * kw;
    for (int m = 0; m < M; m++) {
      const float* x = xf.data() + (size_t)m * K;
      float acc = 0.f;
      for (int g = 0; g < kg; g++) {
        float qx = 0.f, sx = 0.f;
        for (int k = g * 64; k < g * 64 + 64; k++) {
          qx += (float)code_b(wr, k, xr, bits) * x[k];
          sx += x[k];
        }
        acc += bf2f(s[(size_t)n * kg + g]) * qx + bf2f(b[(size_t)n * kg + g]) * sx;
      }
      Y[(size_t)m * N + n] = acc;
    }
  });
}
void orc_qmv(const uint16_t* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
             uint32_t xr, float* Y, int M, int nthreads) {
  orc_qmv_b(A, lda, wq, s, b, N, K, 4, xr, Y, M, nthreads);
}

// Prefill GEMM semantics (MLX affine_qmm_t: third_party/mlx/.../quantized_nax.h:938-1076 with the dequant of
// quantized.h:528-535): every weight is dequantized to bf16(S*q + B), activations are bf16, fp32 accumulation over K.
// bits 4 or 8 (MLX instantiates the same loader for both, quantized.h:486-576).
void orc_qmm_b(const uint16_t* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
               int bits, uint32_t xr, float* Y, int M, int nthreads) {
  const int kg = K / 64, kw = K * bits / 32;
  std::vector<float> xf((size_t)M * K);
  for (int m = 0; m < M; m++)
    for (int k = 0; k < K; k++) xf[(size_t)m * K + k] = bf2f(A[(size_t)m * lda + k]);
  parallel_for(N, nthreads, [&](int n) {
    const uint32_t* wr = wq + (size_t)n * kw;
    std::vector<float> wrow(K);
    for (int k = 0; k < K; k++)
      wrow[k] = bfround(bf2f(s[(size_t)n * kg + k / 64]) * (float)code_b(wr, k, xr, bits) +
                        bf2f(b[(size_t)n * kg + k / 64]));
    for (int m = 0; m < M; m++) {
      const float* x = xf.data() + (size_t)m * K;
      float acc = 0.f;
      for (int k = 0; k < K; k++) acc += x[k] * wrow[k];
      Y[(size_t)m * N + n] = acc;
    }
  });
}
void orc_qmm(const uint16_t* A, int lda, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
             uint32_t xr, float* Y, int M, int nthreads) {
  orc_qmm_b(A, lda, wq, s, b, N, K, 4, xr, Y, M, nthreads);
}

// Store epilogue shared by every GEMM (engine/kernels/core.metal:14-15): mode 0 C = bf16(y), 1 C = bf16(y + C),
// 2 C = y (fp32). C rows are ldc elements apart.
void orc_store(const float* Y, void* C, int ldc, int M, int N, int mode) {
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      const float y = Y[(size_t)m * N + n];
      if (mode == 2) ((float*)C)[(size_t)m * ldc + n] = y;
      else if (mode == 1) {
        uint16_t* c = (uint16_t*)C + (size_t)m * ldc + n;
        *c = f2bf(y + bf2f(*c));
      } else ((uint16_t*)C)[(size_t)m * ldc + n] = f2bf(y);
    }
}

// Activation quantizer (engine/kernels/w4a8.metal:24-41): per row and 64-group, sx = amax/127 (1 if amax == 0),
// xq = rint(x / sx) (no clamp), XS = (sx, sx * sum xq). per_token != 0: one amax over the whole row of K (the
// per-token scale BASELINE config 3 asks for); XS still holds one (sx, sx * sum_g xq) pair per group.
// per_token == 2: the int8 prefill's quantizer (engine/kernels/qa8.metal:30-49): per 64-group,
// xq = clamp(rint(x * (127 / amax)), -127, 127) (inv = 0 when amax == 0), XS = (amax / 127, amax / 127 * sum xq).
void orc_a8_quant(const uint16_t* A, int lda, int M, int K, int per_token, int8_t* U, float* XS) {
  const int kg = K / 64;
  if (per_token == 2) {
    for (int m = 0; m < M; m++)
      for (int g = 0; g < kg; g++) {
        const uint16_t* a = A + (size_t)m * lda + g * 64;
        float amax = 0.f;
        for (int k = 0; k < 64; k++) amax = std::max(amax, std::fabs(bf2f(a[k])));
        const float inv = amax > 0.f ? 127.f / amax : 0.f;
        float qs = 0.f;
        for (int k = 0; k < 64; k++) {
          const float q = std::min(std::max(std::rint(bf2f(a[k]) * inv), -127.f), 127.f);
          U[(size_t)m * K + g * 64 + k] = (int8_t)q;
          qs += q;
        }
        XS[((size_t)m * kg + g) * 2 + 0] = amax / 127.f;
        XS[((size_t)m * kg + g) * 2 + 1] = amax / 127.f * qs;
      }
    return;
  }
  for (int m = 0; m < M; m++) {
    const uint16_t* a = A + (size_t)m * lda;
    float row_amax = 0.f;
    if (per_token)
      for (int k = 0; k < K; k++) row_amax = std::max(row_amax, std::fabs(bf2f(a[k])));
    for (int g = 0; g < kg; g++) {
      float amax = row_amax;
      if (!per_token)
        for (int k = g * 64; k < g * 64 + 64; k++) amax = std::max(amax, std::fabs(bf2f(a[k])));
      const float sx = amax > 0.f ? amax / 127.f : 1.f;
      float qs = 0.f;
      for (int k = g * 64; k < g * 64 + 64; k++) {
        const float q = std::rint(bf2f(a[k]) / sx);
        U[(size_t)m * K + k] = (int8_t)q;
        qs += q;
      }
      XS[((size_t)m * kg + g) * 2 + 0] = sx;
      XS[((size_t)m * kg + g) * 2 + 1] = sx * qs;
    }
  }
}

// W4A8 / W8A8 GEMM (engine/kernels/w4a8.metal:7-8, 57, 78-87): per group g, P = sum (q - off) xq exactly (integers,
// off = 8 for 4 bits, 128 for 8 bits), then
//   y += S sx P + (B + off S) (sx sum xq)   in fp32, in group order.
void orc_wxa8(const int8_t* U, const float* XS, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
              int bits, uint32_t xr, float* Y, int M, int nthreads) {
  const int kg = K / 64, kw = K * bits / 32;
  const int off = bits == 8 ? 128 : 8;
  parallel_for(N, nthreads, [&](int n) {
    const uint32_t* wr = wq + (size_t)n * kw;
    std::vector<int8_t> qs(K);
    for (int k = 0; k < K; k++) qs[k] = (int8_t)(code_b(wr, k, xr, bits) - off);
    for (int m = 0; m < M; m++) {
      const int8_t* u = U + (size_t)m * K;
      float acc = 0.f;
      for (int g = 0; g < kg; g++) {
        int32_t P = 0;
        for (int k = g * 64; k < g * 64 + 64; k++) P += (int32_t)qs[k] * (int32_t)u[k];
        const float sw = bf2f(s[(size_t)n * kg + g]), bw = bf2f(b[(size_t)n * kg + g]) + (float)off * sw;
        const float sx = XS[((size_t)m * kg + g) * 2], sq = XS[((size_t)m * kg + g) * 2 + 1];
        acc += sw * sx * (float)P + bw * sq;
      }
      Y[(size_t)m * N + n] = acc;
    }
  });
}
void orc_w4a8(const int8_t* U, const float* XS, const uint32_t* wq, const uint16_t* s, const uint16_t* b, int N, int K,
              uint32_t xr, float* Y, int M, int nthreads) {
  orc_wxa8(U, XS, wq, s, b, N, K, 4, xr, Y, M, nthreads);
}

// SwiGLU on rows of [gate (I) | up (I)] (engine/kernels/core.metal:777-787, moe.metal:103-111):
//   h = bf16(float(bf16(g * sigmoid(g))) * u), computed as g / (1 + exp(-g)).
void orc_silu_mul(const uint16_t* gu, uint16_t* h, int I, int rows) {
  for (int r = 0; r < rows; r++)
    for (int i = 0; i < I; i++) {
      const float g = bf2f(gu[(size_t)r * 2 * I + i]), u = bf2f(gu[(size_t)r * 2 * I + I + i]);
      h[(size_t)r * I + i] = f2bf(bfround(g / (1.f + std::exp(-g))) * u);
    }
}

// RMS norm (engine/kernels/core.metal:486-500): out = bf16(float(x) * r * float(w)), r = rsqrt(sum x^2 / D + eps).
// The sum of squares is taken in double (the reference sums in fp32 in an unspecified order); r is rounded to fp32
// and the products are fp32, left to right, as the reference writes them.
void orc_rmsnorm(const uint16_t* x, int in_stride, const uint16_t* w, uint16_t* out, int out_stride, int rows, int D,
                 float eps) {
  for (int r = 0; r < rows; r++) {
    const uint16_t* xr = x + (size_t)r * in_stride;
    double ss = 0.0;
    for (int i = 0; i < D; i++) ss += (double)bf2f(xr[i]) * bf2f(xr[i]);
    const float rs = (float)(1.0 / std::sqrt(ss / D + (double)eps));
    for (int i = 0; i < D; i++) out[(size_t)r * out_stride + i] = f2bf(bf2f(xr[i]) * rs * bf2f(w[i]));
  }
}

// bf16 x bf16 GEMM with fp32 accumulation (router logits, engine/kernels/moe.metal:198-213 / qwen35.h:1919-1929):
// Y[m, n] = sum_k A[m, k] W[n, k]; W bf16 [N, K].
void orc_gemm_bf16(const uint16_t* A, const uint16_t* W, float* Y, int M, int N, int K, int nthreads) {
  std::vector<float> wf((size_t)N * K);
  for (size_t i = 0; i < wf.size(); i++) wf[i] = bf2f(W[i]);
  parallel_for(M, nthreads, [&](int m) {
    std::vector<float> x(K);
    for (int k = 0; k < K; k++) x[k] = bf2f(A[(size_t)m * K + k]);
    for (int n = 0; n < N; n++) {
      float acc = 0.f;
      const float* w = wf.data() + (size_t)n * K;
      for (int k = 0; k < K; k++) acc += x[k] * w[k];
      Y[(size_t)m * N + n] = acc;
    }
  });
}

// Router (engine/kernels/moe.metal:60-101; moe_route_bf qwen4.metal:1462-1503 reads bf16 logits): softmax over the
// first E logits in fp32 as exp(l - max); top-k by repeated max scan over the exponentials, ties -> lowest expert
// index; weights p/sum, renormalised over the k picks when norm != 0. Shared gate: sg = sigmoid(l[E]) when
// shared_gate == 1 (the reference), sg = 1 when shared_gate == 0 (an always-on shared expert).
// logits: fp32 (logits_bf16 == 0) or bf16 bit patterns, row stride `stride` elements.
void orc_moe_route(const void* logits, int logits_bf16, int T, int E, int k, int stride, int norm, int shared_gate,
                   int* idx, float* wt, float* sg) {
  std::vector<float> v(E);
  for (int t = 0; t < T; t++) {
    auto L = [&](int c) {
      return logits_bf16 ? bf2f(((const uint16_t*)logits)[(size_t)t * stride + c]) : ((const float*)logits)[(size_t)t * stride + c];
    };
    float mx = -INFINITY;
    for (int c = 0; c < E; c++) mx = std::max(mx, L(c));
    float sum = 0.f;
    for (int c = 0; c < E; c++) {
      v[c] = std::exp(L(c) - mx);
      sum += v[c];
    }
    float tot = 0.f;
    for (int j = 0; j < k; j++) {
      float best = -1.f;
      int bi = 0;
      for (int c = 0; c < E; c++)
        if (v[c] > best) best = v[c], bi = c;  // strict >: the lowest index wins a tie
      v[bi] = -1.f;
      idx[t * k + j] = bi;
      wt[t * k + j] = best / sum;
      tot += best / sum;
    }
    if (norm)
      for (int j = 0; j < k; j++) wt[t * k + j] /= tot;
    sg[t] = shared_gate ? 1.f / (1.f + std::exp(-L(E))) : 1.f;
  }
}

// Dispatch: counting sort of routed rows r = t*k + j by expert (engine/kernels/moe.metal:130-161), made stable
// (rows keep their order inside an expert's segment; the reference's atomic scatter order is unspecified).
// offsets [E + 1] (offsets[E] = R), perm [R] sorted position -> r, inv [R] r -> sorted position.
void orc_moe_dispatch(const int* idx, int R, int E, int* offsets, int* perm, int* inv) {
  std::vector<int> cnt(E, 0);
  for (int r = 0; r < R; r++) cnt[idx[r]]++;
  int acc = 0;
  for (int e = 0; e < E; e++) {
    offsets[e] = acc;
    acc += cnt[e];
    cnt[e] = 0;
  }
  offsets[E] = acc;
  for (int r = 0; r < R; r++) {
    const int e = idx[r], q = offsets[e] + cnt[e]++;
    perm[q] = r;
    inv[r] = q;
  }
}

// Gathered expert GEMM (MLX affine_gather_qmm_rhs: quantized_nax.h:1467-1681): sorted row q belongs to expert e with
// offsets[e] <= q < offsets[e+1]; its activation row is A[perm[q] / div] (div = k for token rows, or A[q] when
// perm == nullptr); y[q, n] = sum_k A_row[k] * bf16(S_e[n,g] q_e[n,k] + B_e[n,g]) with fp32 accumulation.
// W stacked [E, N, K/8], S/B [E, N, K/64].
void orc_moe_gather_qmm(const uint16_t* A, const int* perm, int div, const int* offsets, const uint32_t* wq,
                        const uint16_t* s, const uint16_t* b, int E, int N, int K, float* Y, int R, int nthreads) {
  const int kg = K / 64, kw = K / 8;
  parallel_for(E, nthreads, [&](int e) {
    const int q0 = offsets[e], q1 = offsets[e + 1];
    if (q0 >= q1) return;
    std::vector<float> wrow(K), x(K);
    for (int n = 0; n < N; n++) {
      const size_t row = (size_t)e * N + n;
      for (int k = 0; k < K; k++)
        wrow[k] = bfround(bf2f(s[row * kg + k / 64]) * (float)code_at(wq + row * kw, k, 0) + bf2f(b[row * kg + k / 64]));
      for (int q = q0; q < q1; q++) {
        const uint16_t* a = A + (size_t)(perm ? perm[q] / div : q) * K;
        float acc = 0.f;
        for (int k = 0; k < K; k++) acc += bf2f(a[k]) * wrow[k];
        Y[(size_t)q * N + n] = acc;
      }
    }
  });
  (void)R;
}

// Gathered expert GEMM on int8 activations (reference qa8g_gemm, engine/kernels/qa8.metal:212-397): sorted row q
// of expert e reads quantized row r = perm[q] / div (or q); y[q, n] = sum_g sx[r,g] (S_e[n,g] sum_k q_e[n,k] U[r,k]) +
// B_e[n,g] (sx sum xq)[r,g], the integer sums exact, fp32 in group order (the W4A8 identity on unflipped codes).
void orc_moe_gather_w4a8(const int8_t* U, const float* XS, const int* perm, int div, const int* offsets,
                         const uint32_t* wq, const uint16_t* s, const uint16_t* b, int E, int N, int K, float* Y,
                         int nthreads) {
  const int kg = K / 64, kw = K / 8;
  parallel_for(E, nthreads, [&](int e) {
    const int q0 = offsets[e], q1 = offsets[e + 1];
    std::vector<int> codes(K);
    for (int n = 0; n < N && q0 < q1; n++) {
      const size_t row = (size_t)e * N + n;
      for (int k = 0; k < K; k++) codes[k] = code_at(wq + row * kw, k, 0);
      for (int q = q0; q < q1; q++) {
        const size_t r = (size_t)(perm ? perm[q] / div : q);
        float acc = 0.f;
        for (int g = 0; g < kg; g++) {
          int32_t P = 0;
          for (int k = g * 64; k < g * 64 + 64; k++) P += codes[k] * (int32_t)U[r * K + k];
          const float sx = XS[(r * kg + g) * 2], sq = XS[(r * kg + g) * 2 + 1];
          acc += bf2f(s[row * kg + g]) * sx * (float)P + bf2f(b[row * kg + g]) * sq;
        }
        Y[(size_t)q * N + n] = acc;
      }
    }
  });
}

// Weighted combine over sorted expert outputs (engine/kernels/moe.metal:172-187):
//   acc = sum_j w[t,j] yd[inv[t*k+j], h] + sg[t] ys[t,h] in fp32 over bf16 inputs;
//   out = bf16(acc) (assign) or bf16(x + bf16(acc)) (residual). ys may be null (no shared expert).
void orc_moe_combine(uint16_t* x, const uint16_t* yd, const float* wt, const uint16_t* ys, const float* sg, const int* inv,
                     int T, int H, int k, int assign) {
  for (int t = 0; t < T; t++)
    for (int h = 0; h < H; h++) {
      float acc = 0.f;
      for (int j = 0; j < k; j++) acc += wt[t * k + j] * bf2f(yd[(size_t)inv[t * k + j] * H + h]);
      if (ys) acc += sg[t] * bf2f(ys[(size_t)t * H + h]);
      uint16_t* o = x + (size_t)t * H + h;
      *o = assign ? f2bf(acc) : f2bf(bf2f(*o) + bfround(acc));
    }
}

// The MoE FFN composition (engine/src/qwen35.h:1869-1980, sorted path): given routing (idx, wt, sg) for T tokens,
// shared expert (dense gate_up [2I, H] and down [H, I], through Qwen35::gemm: the decode GEMV semantics when
// shared_qmv != 0, else qmm's) -> ys; dispatch; gathered gate/up qmm -> SwiGLU -> gathered down qmm -> combine.
// Writes out bf16 [T, H] (assign) or adds into it (assign == 0). Shared weights may be null (no shared expert).
void orc_moe_experts(const uint16_t* xn, int T, int H, int I, int E, int k, const int* idx, const float* wt,
                     const float* sg, const uint32_t* gu_wq, const uint16_t* gu_s, const uint16_t* gu_b,
                     const uint32_t* dn_wq, const uint16_t* dn_s, const uint16_t* dn_b, const uint32_t* sh_gu_wq,
                     const uint16_t* sh_gu_s, const uint16_t* sh_gu_b, const uint32_t* sh_dn_wq, const uint16_t* sh_dn_s,
                     const uint16_t* sh_dn_b, int shared_qmv, uint16_t* out, int assign, int nthreads) {
  const int R = T * k;
  std::vector<uint16_t> ys;
  if (sh_gu_wq) {
    auto dense = shared_qmv ? orc_qmv : orc_qmm;
    std::vector<float> y((size_t)T * 2 * I);
    dense(xn, H, sh_gu_wq, sh_gu_s, sh_gu_b, 2 * I, H, 0, y.data(), T, nthreads);
    std::vector<uint16_t> gu((size_t)T * 2 * I), act((size_t)T * I);
    for (size_t i = 0; i < y.size(); i++) gu[i] = f2bf(y[i]);
    orc_silu_mul(gu.data(), act.data(), I, T);
    std::vector<float> yd((size_t)T * H);
    dense(act.data(), I, sh_dn_wq, sh_dn_s, sh_dn_b, H, I, 0, yd.data(), T, nthreads);
    ys.resize((size_t)T * H);
    for (size_t i = 0; i < yd.size(); i++) ys[i] = f2bf(yd[i]);
  }
  std::vector<int> offsets(E + 1), perm(R), inv(R);
  orc_moe_dispatch(idx, R, E, offsets.data(), perm.data(), inv.data());
  std::vector<float> y1((size_t)R * 2 * I);
  orc_moe_gather_qmm(xn, perm.data(), k, offsets.data(), gu_wq, gu_s, gu_b, E, 2 * I, H, y1.data(), R, nthreads);
  std::vector<uint16_t> egu((size_t)R * 2 * I), eact((size_t)R * I);
  for (size_t i = 0; i < y1.size(); i++) egu[i] = f2bf(y1[i]);
  orc_silu_mul(egu.data(), eact.data(), I, R);
  std::vector<float> y2((size_t)R * H);
  orc_moe_gather_qmm(eact.data(), nullptr, 1, offsets.data(), dn_wq, dn_s, dn_b, E, H, I, y2.data(), R, nthreads);
  std::vector<uint16_t> edn((size_t)R * H);
  for (size_t i = 0; i < y2.size(); i++) edn[i] = f2bf(y2[i]);
  orc_moe_combine(out, edn.data(), wt, ys.empty() ? nullptr : ys.data(), sg, inv.data(), T, H, k, assign);
}

// Decode MoE, T <= 8 (reference moe_plan / moe_gu2 / moe_dn2, engine/kernels/moe.metal:326-551; host
// engine/src/qwen35.h:1876-1908): every pick j of token t (expert e = idx[t][j]) and, as pick k, the shared expert
// (when its weights are given) run per token with the decode GEMV arithmetic (qmv4: fp32 s sum q x + b sum x):
//   g, u = qmv(x_t, [gate | up]_e); a = bf16(float(bf16(silu(bf16 g))) * bf16 u); d_j = bf16(qmv(a, down_e));
//   acc = sum_{j < k} wt[t][j] d_j + sg[t] d_k in fp32 (j order); out = bf16(acc) (assign) or bf16(x + bf16(acc)).
// Deduplicating the experts across tokens (moe_plan) changes which weights are read once, not these values.
// sh_bits: the shared expert's width, 4 or 8 (the reference's moe_gu2_4_8 / moe_dn2_4_8, moe.metal:465-476, 544-547:
// the same arithmetic with the qmv8 dot, core.metal:175-248)
void orc_moe_decode_b(const uint16_t* xn, int T, int H, int I, int k, const int* idx, const float* wt, const float* sg,
                      const uint32_t* gu_wq, const uint16_t* gu_s, const uint16_t* gu_b, const uint32_t* dn_wq,
                      const uint16_t* dn_s, const uint16_t* dn_b, const uint32_t* sh_gu_wq, const uint16_t* sh_gu_s,
                      const uint16_t* sh_gu_b, const uint32_t* sh_dn_wq, const uint16_t* sh_dn_s,
                      const uint16_t* sh_dn_b, int sh_bits, uint16_t* out, int assign) {
  const size_t gw = (size_t)2 * I * (H / 8), gs = (size_t)2 * I * (H / 64), dw = (size_t)H * (I / 8),
               ds = (size_t)H * (I / 64);
  std::vector<float> y(2 * I), yd(H);
  std::vector<uint16_t> gu(2 * I), act(I);
  auto expert = [&](const uint16_t* x, const uint32_t* gwq, const uint16_t* gsc, const uint16_t* gbi,
                    const uint32_t* dwq, const uint16_t* dsc, const uint16_t* dbi, std::vector<uint16_t>& d,
                    int bits) {
    orc_qmv_b(x, H, gwq, gsc, gbi, 2 * I, H, bits, 0, y.data(), 1, 1);
    for (int i = 0; i < 2 * I; i++) gu[i] = f2bf(y[i]);
    orc_silu_mul(gu.data(), act.data(), I, 1);
    orc_qmv_b(act.data(), I, dwq, dsc, dbi, H, I, bits, 0, yd.data(), 1, 1);
    d.resize(H);
    for (int h = 0; h < H; h++) d[h] = f2bf(yd[h]);
  };
  std::vector<std::vector<uint16_t>> dj(k + 1);
  for (int t = 0; t < T; t++) {
    const uint16_t* x = xn + (size_t)t * H;
    for (int j = 0; j < k; j++) {
      const size_t e = (size_t)idx[t * k + j];
      expert(x, gu_wq + e * gw, gu_s + e * gs, gu_b + e * gs, dn_wq + e * dw, dn_s + e * ds, dn_b + e * ds, dj[j], 4);
    }
    if (sh_gu_wq) expert(x, sh_gu_wq, sh_gu_s, sh_gu_b, sh_dn_wq, sh_dn_s, sh_dn_b, dj[k], sh_bits);
    for (int h = 0; h < H; h++) {
      float acc = 0.f;
      for (int j = 0; j < k; j++) acc += wt[t * k + j] * bf2f(dj[j][h]);
      if (sh_gu_wq) acc += sg[t] * bf2f(dj[k][h]);
      uint16_t* o = out + (size_t)t * H + h;
      *o = assign ? f2bf(acc) : f2bf(bf2f(*o) + bfround(acc));
    }
  }
}
void orc_moe_decode(const uint16_t* xn, int T, int H, int I, int k, const int* idx, const float* wt, const float* sg,
                    const uint32_t* gu_wq, const uint16_t* gu_s, const uint16_t* gu_b, const uint32_t* dn_wq,
                    const uint16_t* dn_s, const uint16_t* dn_b, const uint32_t* sh_gu_wq, const uint16_t* sh_gu_s,
                    const uint16_t* sh_gu_b, const uint32_t* sh_dn_wq, const uint16_t* sh_dn_s, const uint16_t* sh_dn_b,
                    uint16_t* out, int assign) {
  orc_moe_decode_b(xn, T, H, I, k, idx, wt, sg, gu_wq, gu_s, gu_b, dn_wq, dn_s, dn_b, sh_gu_wq, sh_gu_s, sh_gu_b,
                   sh_dn_wq, sh_dn_s, sh_dn_b, 4, out, assign);
}

}  // extern "C"
