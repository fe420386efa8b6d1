// Test driver for the checkpoint loader (inferd_amd/csrc/ckpt.h): loads what the command names and writes the
// host arrays to a raw file that tests/test_ckpt.py compares with its expectations. Host only (no GPU).
//
//   ckpt_test qlinear DIR OUT PREFIX...      load_qlinear (fused rows)
//   ckpt_test moe     DIR OUT PREFIX...      load_moe (fused along N per expert)
//   ckpt_test bf16q   DIR OUT BITS NAME...   load_qlinear_bf16 (quantized at load)
//   ckpt_test quant   IN  OUT BITS N K       quantize_affine of raw bf16 rows read from IN
//
// OUT: int32 {bits, E, N, K}, then wq (uint32), s, b (bf16), w16 (bf16) as present. A loader error prints
// "ckpt error: <message>" to stderr and exits with status 2.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <vector>

#include "ckpt.h"

using namespace inferd;

template <class T>
static void put(std::ofstream& f, const std::vector<T>& v) {
  f.write((const char*)v.data(), (std::streamsize)(v.size() * sizeof(T)));
}

static void write_out(const std::string& path, int bits, int E, int N, int K, const std::vector<uint32_t>& wq,
                      const std::vector<uint16_t>& s, const std::vector<uint16_t>& b, const std::vector<uint16_t>& w16) {
  std::ofstream f(path, std::ios::binary);
  const int32_t h[4] = {bits, E, N, K};
  f.write((const char*)h, sizeof h);
  put(f, wq), put(f, s), put(f, b), put(f, w16);
  if (!f) throw CkptError("cannot write " + path);
}

int main(int argc, char** argv) {
  if (argc < 5) {
    fprintf(stderr, "usage: ckpt_test qlinear|moe|bf16q|quant ...\n");
    return 64;
  }
  const std::string cmd = argv[1], src = argv[2], out = argv[3];
  try {
    if (cmd == "qlinear" || cmd == "moe") {
      Checkpoint ck(src);
      const std::vector<std::string> names(argv + 4, argv + argc);
      if (cmd == "qlinear") {
        const HostQLinear q = load_qlinear(ck, names);
        write_out(out, q.bits, 1, q.N, q.K, q.wq, q.s, q.b, q.w16);
      } else {
        const HostMoeW m = load_moe(ck, names);
        write_out(out, m.bits, m.E, m.N, m.K, m.wq, m.s, m.b, {});
      }
    } else if (cmd == "bf16q") {
      Checkpoint ck(src);
      const int bits = atoi(argv[4]);
      const std::vector<std::string> names(argv + 5, argv + argc);
      const HostQLinear q = load_qlinear_bf16(ck, names, bits);
      write_out(out, q.bits, 1, q.N, q.K, q.wq, q.s, q.b, {});
    } else if (cmd == "quant" && argc == 7) {
      const int bits = atoi(argv[4]), N = atoi(argv[5]), K = atoi(argv[6]);
      std::vector<uint16_t> w((size_t)N * K);
      std::ifstream f(src, std::ios::binary);
      f.read((char*)w.data(), (std::streamsize)(w.size() * 2));
      if (!f) throw CkptError("short input " + src);
      const HostQLinear q = quantize_affine(w.data(), N, K, bits);
      write_out(out, q.bits, 1, q.N, q.K, q.wq, q.s, q.b, {});
    } else {
      fprintf(stderr, "unknown command %s\n", cmd.c_str());
      return 64;
    }
  } catch (CkptError& e) {
    fprintf(stderr, "ckpt error: %s\n", e.what());
    return 2;
  }
  return 0;
}
