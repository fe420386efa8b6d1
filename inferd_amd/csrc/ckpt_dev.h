// Device-side loaders: the reference's load_qlinear / load_qlinear_bf16_q8 / load_moe (engine/src/weights.h:271-406,
// engine/src/moe.h:14-87), which read a checkpoint into GPU buffers, over the host loader of ckpt.h and the shim's
// QLinear / MoeW (qwen35_ops.h). Each layer is one device allocation [wq | s | b] (as the reference's one buffer per
// layer); a 4-bit linear whose K is a multiple of 256 also gets its T64 copy, packed once here, which gemm() reads.
//
// Errors in the checkpoint keep the reference's loader behaviour: a message on stderr and exit(1).
#pragma once
#include <string>
#include <vector>

#include "ckpt.h"
#include "qwen35_ops.h"

namespace inferd {

// The allocator and stream the loaders upload with (the role of the reference's Gpu& at load).
struct Gpu {
  hipStream_t stream = nullptr;
  std::vector<void*> owned;  // every buffer the loaders allocated; freed by release()
  void* alloc(size_t bytes) {
    void* p = nullptr;
    hip_ok(hipMalloc(&p, std::max<size_t>(bytes, 256)), "load");
    owned.push_back(p);
    return p;
  }
  void release() {
    hip_ok(hipStreamSynchronize(stream), "release");
    for (void* p : owned) (void)hipFree(p);
    owned.clear();
  }
};

namespace detail {
template <class F>
auto or_exit(const char* op, F&& f) -> decltype(f()) {
  try {
    return f();
  } catch (CkptError& e) {
    fprintf(stderr, "%s: %s\n", op, e.what());
    exit(1);
  }
}
inline void upload(Gpu& g, void* dst, const void* src, size_t bytes) {
  if (bytes) hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g.stream), "load");
}
}  // namespace detail

// A host linear on the device: [wq | s | b] in one buffer (bits 16: the bf16 rows), plus the T64 copy when t64 and the
// shape allows it (4-bit with K % 256 == 0: T64; 8-bit: T64x8). The upload is synchronous with respect to the host
// arrays.
inline QLinear upload_qlinear(Gpu& g, const HostQLinear& h, bool t64 = true) {
  QLinear q;
  q.N = h.N, q.K = h.K, q.bits = h.bits;
  if (h.bits == 16) {
    q.wq = BufRef(g.alloc(h.w16.size() * 2));
    detail::upload(g, q.wq.ptr<void>(), h.w16.data(), h.w16.size() * 2);
    q.s = q.b = q.wq;
  } else {
    const size_t wb = h.wq.size() * 4, sb = h.s.size() * 2;
    void* buf = g.alloc(wb + 2 * sb);
    q.wq = BufRef(buf, 0), q.s = BufRef(buf, wb), q.b = BufRef(buf, wb + sb);
    detail::upload(g, q.wq.ptr<void>(), h.wq.data(), wb);
    detail::upload(g, q.s.ptr<void>(), h.s.data(), sb);
    detail::upload(g, q.b.ptr<void>(), h.b.data(), sb);
    if (t64 && h.bits == 4 && h.K % 256 == 0) {
      void* t = g.alloc(ifd_t64_bytes(h.N, h.K, 1));
      ok(ifd_pack_t64(q.wq.ptr<uint32_t>(), q.s.ptr<uint16_t>(), q.b.ptr<uint16_t>(), h.N, h.K, 0, 0u, 1, t, g.stream),
         "load");
      q.t64 = BufRef(t);
    }
    if (t64 && h.bits == 8 && h.K % 64 == 0) {
      void* t = g.alloc(ifd_t64x8_bytes(h.N, h.K));
      ok(ifd_pack_t64x8(q.wq.ptr<uint32_t>(), q.s.ptr<uint16_t>(), q.b.ptr<uint16_t>(), h.N, h.K, 0, 0u, t, g.stream),
         "load");
      q.t64 = BufRef(t);
    }
  }
  hip_ok(hipStreamSynchronize(g.stream), "load");
  return q;
}

// A host expert stack on the device: [wq | s | b] in one buffer, plus the E experts' T64 copy (ifd_pack_t64 with E)
// when t64 and the stack is 4-bit with K and N multiples of 256, which encode_moe's sorted route then reads.
inline MoeW upload_moe(Gpu& g, const HostMoeW& h, bool t64 = true) {
  MoeW m;
  m.E = h.E, m.N = h.N, m.K = h.K, m.bits = h.bits;
  const size_t wb = h.wq.size() * 4, sb = h.s.size() * 2;
  void* buf = g.alloc(wb + 2 * sb);
  m.wq = BufRef(buf, 0), m.s = BufRef(buf, wb), m.b = BufRef(buf, wb + sb);
  detail::upload(g, m.wq.ptr<void>(), h.wq.data(), wb);
  detail::upload(g, m.s.ptr<void>(), h.s.data(), sb);
  detail::upload(g, m.b.ptr<void>(), h.b.data(), sb);
  if (t64 && h.bits == 4 && h.K % 256 == 0 && h.N % 256 == 0) {
    void* t = g.alloc(ifd_t64_bytes(h.N, h.K, h.E));
    ok(ifd_pack_t64(m.wq.ptr<uint32_t>(), m.s.ptr<uint16_t>(), m.b.ptr<uint16_t>(), h.N, h.K, 0, 0u, h.E, t, g.stream),
       "load");
    m.t64 = BufRef(t);
  }
  hip_ok(hipStreamSynchronize(g.stream), "load");
  return m;
}

// reference load_qlinear (weights.h:271-340): quantized or bf16 linears sharing K, fused by rows.
inline QLinear load_qlinear(Gpu& g, const Checkpoint& ck, const std::vector<std::string>& prefixes, bool t64 = true) {
  return upload_qlinear(g, detail::or_exit("load_qlinear", [&] { return load_qlinear(ck, prefixes); }), t64);
}
// reference load_qlinear_bf16_q8 (weights.h:349-406): bf16 linears quantized at load to 8 (or 4) bits, group 64.
inline QLinear load_qlinear_bf16_q8(Gpu& g, const Checkpoint& ck, const std::vector<std::string>& names, int bits = 8,
                                    bool t64 = true) {
  return upload_qlinear(g, detail::or_exit("load_qlinear_bf16_q8", [&] { return load_qlinear_bf16(ck, names, bits); }),
                        t64);
}
// reference load_moe (moe.h:14-87): stacked expert matrices fused along N per expert, groups expanded to 64.
inline MoeW load_moe(Gpu& g, const Checkpoint& ck, const std::vector<std::string>& prefixes, bool t64 = true) {
  return upload_moe(g, detail::or_exit("load_moe", [&] { return load_moe(ck, prefixes); }), t64);
}

}  // namespace inferd
