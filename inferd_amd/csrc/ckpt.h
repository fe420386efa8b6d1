// MLX safetensors checkpoints -> the affine weight layout the kernels read (host only, no GPU calls).
//
// Replaces the reference's loader (engine/src/weights.h: Checkpoint :54-224, load_qlinear :271-340, the load-time
// quantizer load_qlinear_bf16_q8 :349-406; engine/src/moe.h: load_moe :14-87; the per-module quantization spec,
// qwen4.h:11-29). A checkpoint is a directory of *.safetensors files and an optional config.json whose
// "quantization" object gives bits and group_size, globally and per module prefix.
//
// Every header is untrusted: its length is checked against the file, and each tensor's dtype, shape and
// data_offsets against each other and the data section before anything is sized from them or read. Every read names
// its destination's capacity. Errors throw CkptError naming the file or tensor.
//
// Layout produced (QLinear, [N, K]): wq uint32 [N][K bits / 32] (element j of a word at bits bits*j, low first),
// scales and biases bf16 [N][K / 64]. Several tensors sharing K are fused by concatenating rows (gate | up). A
// quantization group wider than 64 becomes 64-groups that repeat its scale and bias (exact; codes unchanged).
#pragma once
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace inferd {

struct CkptError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// ---- a small JSON reader (objects, arrays, strings, numbers, literals): enough for safetensors headers and config
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const std::string& k) const {
    if (kind != Obj) return nullptr;
    for (auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
  // an integer-valued number within [lo, hi]
  int64_t integer(int64_t lo, int64_t hi) const {
    if (kind != Num || num != std::floor(num) || num < (double)lo || num > (double)hi)
      throw CkptError("expected an integer in [" + std::to_string(lo) + ", " + std::to_string(hi) + "]");
    return (int64_t)num;
  }

  static Json parse(const std::string& text) {
    size_t i = 0;
    Json v = value(text, i, 0);
    ws(text, i);
    if (i != text.size()) throw CkptError("JSON: trailing characters at " + std::to_string(i));
    return v;
  }

 private:
  static void ws(const std::string& t, size_t& i) {
    while (i < t.size() && (t[i] == ' ' || t[i] == '\n' || t[i] == '\r' || t[i] == '\t')) i++;
  }
  static void expect(const std::string& t, size_t& i, char c) {
    ws(t, i);
    if (i >= t.size() || t[i] != c) throw CkptError(std::string("JSON: expected '") + c + "' at " + std::to_string(i));
    i++;
  }
  static std::string string(const std::string& t, size_t& i) {
    expect(t, i, '"');
    std::string s;
    while (i < t.size() && t[i] != '"') {
      char c = t[i++];
      if (c == '\\') {
        if (i >= t.size()) break;
        const char e = t[i++];
        switch (e) {
          case 'n': s += '\n'; break;
          case 't': s += '\t'; break;
          case 'r': s += '\r'; break;
          case 'b': s += '\b'; break;
          case 'f': s += '\f'; break;
          case 'u': {  // kept as UTF-8 for the BMP; names in headers are ASCII in practice
            if (i + 4 > t.size()) throw CkptError("JSON: short \\u escape");
            const unsigned cp = (unsigned)std::stoul(t.substr(i, 4), nullptr, 16);
            i += 4;
            if (cp < 0x80) s += (char)cp;
            else if (cp < 0x800) s += (char)(0xC0 | (cp >> 6)), s += (char)(0x80 | (cp & 0x3F));
            else s += (char)(0xE0 | (cp >> 12)), s += (char)(0x80 | ((cp >> 6) & 0x3F)), s += (char)(0x80 | (cp & 0x3F));
            break;
          }
          default: s += e;
        }
      } else {
        s += c;
      }
    }
    if (i >= t.size()) throw CkptError("JSON: unterminated string");
    i++;
    return s;
  }
  static Json value(const std::string& t, size_t& i, int depth) {
    if (depth > 64) throw CkptError("JSON: nested too deeply");
    ws(t, i);
    if (i >= t.size()) throw CkptError("JSON: unexpected end");
    Json v;
    const char c = t[i];
    if (c == '{') {
      v.kind = Obj;
      i++;
      ws(t, i);
      if (i < t.size() && t[i] == '}') return i++, v;
      for (;;) {
        std::string k = string(t, i);
        expect(t, i, ':');
        v.obj.emplace_back(std::move(k), value(t, i, depth + 1));
        ws(t, i);
        if (i < t.size() && t[i] == ',') { i++; continue; }
        expect(t, i, '}');
        return v;
      }
    }
    if (c == '[') {
      v.kind = Arr;
      i++;
      ws(t, i);
      if (i < t.size() && t[i] == ']') return i++, v;
      for (;;) {
        v.arr.push_back(value(t, i, depth + 1));
        ws(t, i);
        if (i < t.size() && t[i] == ',') { i++; continue; }
        expect(t, i, ']');
        return v;
      }
    }
    if (c == '"') {
      v.kind = Str;
      v.str = string(t, i);
      return v;
    }
    if (t.compare(i, 4, "true") == 0) return i += 4, v.kind = Bool, v.b = true, v;
    if (t.compare(i, 5, "false") == 0) return i += 5, v.kind = Bool, v;
    if (t.compare(i, 4, "null") == 0) return i += 4, v;
    size_t n = 0;
    try {
      v.num = std::stod(t.substr(i, 40), &n);
    } catch (std::exception&) {
      throw CkptError("JSON: bad value at " + std::to_string(i));
    }
    if (n == 0) throw CkptError("JSON: bad value at " + std::to_string(i));
    i += n;
    v.kind = Num;
    return v;
  }
};

struct TensorInfo {
  std::string dtype, file;
  std::vector<int64_t> shape;
  uint64_t off = 0, nbytes = 0;  // absolute offset of the data in file
  int fd = -1;
};

inline size_t dtype_bytes(const std::string& d) {
  static const std::map<std::string, size_t> sz = {{"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E4M3", 1}, {"F8_E5M2", 1},
                                                    {"U16", 2},  {"I16", 2}, {"F16", 2}, {"BF16", 2},    {"U32", 4},
                                                    {"I32", 4},  {"F32", 4}, {"U64", 8}, {"I64", 8},     {"F64", 8}};
  auto it = sz.find(d);
  return it == sz.end() ? 0 : it->second;
}

class Checkpoint {
 public:
  // dir: a directory of *.safetensors files (and config.json, optional); or one .safetensors file
  explicit Checkpoint(const std::string& path) {
    struct stat st;
    if (stat(path.c_str(), &st) != 0) throw CkptError("cannot open " + path + ": " + strerror(errno));
    if (S_ISDIR(st.st_mode)) {
      dir_ = path;
      const std::string cfg = path + "/config.json";
      if (access(cfg.c_str(), R_OK) == 0) config_ = Json::parse(slurp(cfg));
      DIR* dp = opendir(path.c_str());
      if (!dp) throw CkptError("cannot list " + path);
      std::vector<std::string> files;
      while (dirent* de = readdir(dp)) {
        const std::string n = de->d_name;
        if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) files.push_back(path + "/" + n);
      }
      closedir(dp);
      for (auto& f : files) index(f);
    } else {
      dir_ = path;
      index(path);
    }
  }
  ~Checkpoint() {
    for (int fd : fds_) close(fd);
  }
  Checkpoint(const Checkpoint&) = delete;
  Checkpoint& operator=(const Checkpoint&) = delete;

  bool has(const std::string& name) const { return t_.count(name) > 0; }
  const TensorInfo& info(const std::string& name) const {
    auto it = t_.find(name);
    if (it == t_.end()) throw CkptError("checkpoint " + dir_ + ": missing tensor " + name);
    return it->second;
  }
  const Json& config() const { return config_; }
  [[noreturn]] void reject(const std::string& name, const std::string& what) const {
    throw CkptError("checkpoint " + dir_ + ": tensor " + name + ": " + what);
  }
  void need_dtype(const std::string& name, const char* dt) const {
    if (info(name).dtype != dt) reject(name, std::string("expected ") + dt + ", got " + info(name).dtype);
  }
  // dimension `axis` of a tensor of rank `rank`, within [lo, hi]
  int dim(const std::string& name, int rank, int axis, int64_t lo = 1, int64_t hi = 1 << 30) const {
    const TensorInfo& ti = info(name);
    if ((int)ti.shape.size() != rank)
      reject(name, "expected rank " + std::to_string(rank) + ", got " + std::to_string(ti.shape.size()));
    const int64_t v = ti.shape[axis];
    if (v < lo || v > hi) reject(name, "dimension " + std::to_string(axis) + " is " + std::to_string(v));
    return (int)v;
  }
  // the tensor's bytes into dst (capacity cap): a tensor larger than its destination is refused before any copy
  void read_into(const TensorInfo& ti, void* dst, size_t cap) const {
    if (ti.nbytes > cap)
      throw CkptError("checkpoint " + dir_ + ": a " + std::to_string(ti.nbytes) + "-byte tensor does not fit its " +
                      std::to_string(cap) + "-byte destination");
    if (!pread_all(ti.fd, dst, ti.nbytes, ti.off)) throw CkptError(ti.file + ": short read (truncated file?)");
  }

  // Quantization spec of a module prefix (reference qspec, qwen4.h:11-29): config "quantization" {bits, group_size}
  // and per-prefix overrides; without a config, bits come from the shapes and the group is 64.
  struct QSpec {
    int bits = 0, gs = 64;
  };
  QSpec qspec(const std::string& prefix) const {
    QSpec s;
    const Json* q = config_.get("quantization");
    try {
      if (q) {
        if (const Json* b = q->get("bits")) s.bits = (int)b->integer(2, 8);
        if (const Json* g = q->get("group_size")) s.gs = (int)g->integer(32, 1 << 16);
        if (const Json* o = q->get(prefix); o && o->kind == Json::Obj) {  // an override names both
          const Json *b = o->get("bits"), *g = o->get("group_size");
          if (!b || !g) throw CkptError("an override needs bits and group_size");
          s.bits = (int)b->integer(2, 8);
          s.gs = (int)g->integer(32, 1 << 16);
        }
      }
    } catch (CkptError& e) {
      reject(prefix, std::string("quantization config: ") + e.what());
    }
    if (s.gs % 64) reject(prefix, "group size " + std::to_string(s.gs) + " is not a multiple of 64");
    return s;
  }

 private:
  static std::string slurp(const std::string& p) {
    int fd = open(p.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw CkptError("cannot read " + p);
    std::string s;
    char buf[1 << 16];
    for (;;) {
      const ssize_t r = read(fd, buf, sizeof buf);
      if (r < 0 && errno == EINTR) continue;
      if (r <= 0) break;
      s.append(buf, (size_t)r);
    }
    close(fd);
    return s;
  }
  static bool pread_all(int fd, void* dst, size_t n, uint64_t off) {
    for (size_t done = 0; done < n;) {
      const ssize_t r = pread(fd, (char*)dst + done, std::min<size_t>(n - done, (size_t)1 << 28), (off_t)(off + done));
      if (r < 0 && errno == EINTR) continue;
      if (r <= 0) return false;
      done += (size_t)r;
    }
    return true;
  }
  [[noreturn]] static void bad(const std::string& f, const std::string& what) {
    throw CkptError("invalid safetensors file " + f + ": " + what);
  }
  void index(const std::string& f) {
    const int fd = open(f.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) bad(f, strerror(errno));
    fds_.push_back(fd);
    struct stat st;
    if (fstat(fd, &st) != 0) bad(f, strerror(errno));
    const uint64_t size = (uint64_t)st.st_size;
    uint64_t hlen = 0;
    if (size < 8 || !pread_all(fd, &hlen, 8, 0)) bad(f, "shorter than its 8-byte header length");
    if (hlen < 2 || hlen > ((uint64_t)100 << 20) || hlen > size - 8)
      bad(f, "header length " + std::to_string(hlen) + " does not fit the " + std::to_string(size) + "-byte file");
    std::string h(hlen, '\0');
    if (!pread_all(fd, h.data(), hlen, 8)) bad(f, "short header");
    Json hv;
    try {
      hv = Json::parse(h);
    } catch (CkptError& e) {
      bad(f, std::string("header: ") + e.what());
    }
    if (hv.kind != Json::Obj) bad(f, "header is not a JSON object");
    const uint64_t data = size - 8 - hlen;
    for (auto& [name, v] : hv.obj) {
      if (name == "__metadata__") continue;
      const Json *dt = v.get("dtype"), *sh = v.get("shape"), *off = v.get("data_offsets");
      if (!dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off || off->kind != Json::Arr ||
          off->arr.size() != 2)
        bad(f, "tensor " + name + ": needs dtype, shape and two data_offsets");
      TensorInfo ti;
      ti.dtype = dt->str;
      ti.file = f;
      ti.fd = fd;
      uint64_t elems = 1;
      try {
        for (auto& d : sh->arr) {
          const int64_t n = d.integer(0, (int64_t)1 << 40);
          if (n && elems > UINT64_MAX / (uint64_t)n) throw CkptError("shape overflows");
          ti.shape.push_back(n);
          elems *= (uint64_t)n;
        }
        const uint64_t b = (uint64_t)off->arr[0].integer(0, (int64_t)1 << 50);
        const uint64_t e = (uint64_t)off->arr[1].integer(0, (int64_t)1 << 50);
        if (b > e || e > data)
          throw CkptError("data_offsets [" + std::to_string(b) + ", " + std::to_string(e) + ") outside the " +
                          std::to_string(data) + "-byte data section");
        const size_t es = dtype_bytes(ti.dtype);
        if (!es) throw CkptError("unsupported dtype " + ti.dtype);
        if (elems > UINT64_MAX / es || elems * es != e - b)
          throw CkptError(ti.dtype + " shape holds " + std::to_string(elems) + " elements but the range is " +
                          std::to_string(e - b) + " bytes");
        ti.off = 8 + hlen + b;
        ti.nbytes = e - b;
      } catch (CkptError& ex) {
        bad(f, "tensor " + name + ": " + ex.what());
      }
      t_[name] = std::move(ti);
    }
  }

  std::string dir_;
  Json config_;
  std::map<std::string, TensorInfo> t_;
  std::vector<int> fds_;
};

// ---- affine weights on the host, ready for upload ------------------------------------------------------------------
struct HostQLinear {
  std::vector<uint32_t> wq;    // [N][K bits / 32]
  std::vector<uint16_t> s, b;  // bf16 [N][K / 64]
  std::vector<uint16_t> w16;   // bits == 16 (an unquantized checkpoint): the bf16 rows [N][K]; wq, s, b empty
  int N = 0, K = 0, bits = 4;
};
struct HostMoeW {  // E stacked [N, K] affine matrices (parts fused along N per expert)
  std::vector<uint32_t> wq;
  std::vector<uint16_t> s, b;
  int E = 0, N = 0, K = 0, bits = 4;
};

// s / b rows of G source groups of gs values -> G gs / 64 groups of 64 (each repeated gs / 64 times)
inline void expand_groups(const uint16_t* src, size_t rows, int G, int f, uint16_t* dst) {
  for (size_t r = 0; r < rows; r++)
    for (int g = 0; g < G; g++)
      for (int k = 0; k < f; k++) dst[(r * G + g) * f + k] = src[r * G + g];
}

// Quantized linears sharing K, fused by rows (reference load_qlinear, weights.h:271-340): U32 weights [n, K bits/32],
// BF16 scales / biases [n, K / gs]; bits 4 or 8. BF16 weights (an unquantized checkpoint) load as bits 16, as there.
// The group size comes from the quantization spec (64 without a config, where the reference assumes 64 for every
// linear; it reads the spec for MoE stacks only).
inline HostQLinear load_qlinear(const Checkpoint& ck, const std::vector<std::string>& prefixes) {
  HostQLinear q;
  if (prefixes.empty()) throw CkptError("load_qlinear: no tensors named");
  if (ck.info(prefixes[0] + ".weight").dtype == "BF16") {
    q.bits = 16;
    for (auto& p : prefixes) {
      const std::string wn = p + ".weight";
      ck.need_dtype(wn, "BF16");
      const int n = ck.dim(wn, 2, 0), k = ck.dim(wn, 2, 1);
      if (q.K && q.K != k) ck.reject(wn, "fused parts differ in K");
      if ((int64_t)q.N + n > (1 << 30)) ck.reject(wn, "fused rows overflow");
      q.K = k, q.N += n;
    }
    q.w16.resize((size_t)q.N * q.K);
    size_t r0 = 0;
    for (auto& p : prefixes) {
      const TensorInfo& ti = ck.info(p + ".weight");
      ck.read_into(ti, q.w16.data() + r0 * q.K, (q.w16.size() - r0 * q.K) * 2);
      r0 += (size_t)ti.shape[0];
    }
    return q;
  }
  struct Part {
    int n, G, f;
    const TensorInfo *w, *s, *b;
  };
  std::vector<Part> parts;
  for (auto& p : prefixes) {
    const std::string wn = p + ".weight", sn = p + ".scales", bn = p + ".biases";
    ck.need_dtype(wn, "U32");
    ck.need_dtype(sn, "BF16");
    ck.need_dtype(bn, "BF16");
    const auto sp = ck.qspec(p);
    const int n = ck.dim(wn, 2, 0), wk = ck.dim(wn, 2, 1, 1, (1 << 30) / 32);
    const int G = ck.dim(sn, 2, 1, 1, (1 << 30) / sp.gs);
    if (ck.dim(sn, 2, 0) != n || ck.info(bn).shape != ck.info(sn).shape)
      ck.reject(sn, "scales / biases do not match the weight's rows");
    const int K = G * sp.gs;
    const int bits = (int)((int64_t)wk * 32 / K);
    if ((bits != 4 && bits != 8) || (int64_t)wk * 32 != (int64_t)K * bits || (sp.bits && sp.bits != bits))
      ck.reject(wn, "not a 4- or 8-bit quantized [" + std::to_string(n) + ", " + std::to_string(K) + "] at group " +
                        std::to_string(sp.gs));
    if (q.K && (q.K != K || q.bits != bits)) ck.reject(wn, "fused parts differ in K or bits");
    if ((int64_t)q.N + n > (1 << 30)) ck.reject(wn, "fused rows overflow");
    q.K = K, q.bits = bits, q.N += n;
    parts.push_back({n, G, sp.gs / 64, &ck.info(wn), &ck.info(sn), &ck.info(bn)});
  }
  const size_t wrow = (size_t)q.K * q.bits / 32, G64 = (size_t)q.K / 64;
  q.wq.resize((size_t)q.N * wrow);
  q.s.resize((size_t)q.N * G64);
  q.b.resize((size_t)q.N * G64);
  size_t r0 = 0;
  for (auto& pt : parts) {
    ck.read_into(*pt.w, q.wq.data() + r0 * wrow, (q.wq.size() - r0 * wrow) * 4);
    std::vector<uint16_t> tmp((size_t)pt.n * pt.G);
    for (int which = 0; which < 2; which++) {
      ck.read_into(which ? *pt.b : *pt.s, tmp.data(), tmp.size() * 2);
      expand_groups(tmp.data(), (size_t)pt.n, pt.G, pt.f, (which ? q.b : q.s).data() + r0 * G64);
    }
    r0 += (size_t)pt.n;
  }
  return q;
}

// MoE stacks (reference load_moe, moe.h:14-87): 3-D [E, n, K bits/32] weights (2-D counts as E = 1) with scales /
// biases [E, n, K / gs], fused along N per expert; the group size from the spec, expanded to 64-groups.
inline HostMoeW load_moe(const Checkpoint& ck, const std::vector<std::string>& prefixes) {
  HostMoeW m;
  if (prefixes.empty()) throw CkptError("load_moe: no tensors named");
  struct Part {
    int n, G, f;
    const TensorInfo *w, *s, *b;
  };
  std::vector<Part> parts;
  int gs0 = 0;
  for (auto& p : prefixes) {
    const std::string wn = p + ".weight", sn = p + ".scales", bn = p + ".biases";
    ck.need_dtype(wn, "U32");
    ck.need_dtype(sn, "BF16");
    ck.need_dtype(bn, "BF16");
    const int rank = (int)ck.info(wn).shape.size();
    if (rank != 2 && rank != 3) ck.reject(wn, "expected rank 2 or 3");
    const auto sp = ck.qspec(p);
    const int E = rank == 3 ? ck.dim(wn, 3, 0, 1, 1 << 16) : 1, n = ck.dim(wn, rank, rank - 2);
    const int wk = ck.dim(wn, rank, rank - 1, 1, (1 << 30) / 32);
    const int G = ck.dim(sn, rank, rank - 1, 1, (1 << 30) / sp.gs);
    if (ck.dim(sn, rank, rank - 2) != n || (rank == 3 && ck.dim(sn, 3, 0) != E) || ck.info(bn).shape != ck.info(sn).shape)
      ck.reject(sn, "scales / biases do not match the weight");
    const int K = G * sp.gs, bits = (int)((int64_t)wk * 32 / K);
    if ((bits != 4 && bits != 8) || (int64_t)wk * 32 != (int64_t)K * bits) ck.reject(wn, "unsupported width");
    if ((m.E && m.E != E) || (m.K && (m.K != K || m.bits != bits))) ck.reject(wn, "MoE stack mismatch");
    if (gs0 && gs0 != sp.gs) ck.reject(sn, "MoE stack mixes group sizes");
    if ((int64_t)m.N + n > (1 << 30) || (int64_t)E * (m.N + n) > ((int64_t)1 << 34)) ck.reject(wn, "stack too large");
    gs0 = sp.gs;
    m.E = E, m.K = K, m.bits = bits, m.N += n;
    parts.push_back({n, G, sp.gs / 64, &ck.info(wn), &ck.info(sn), &ck.info(bn)});
  }
  const size_t wrow = (size_t)m.K * m.bits / 32, G64 = (size_t)m.K / 64;
  m.wq.resize((size_t)m.E * m.N * wrow);
  m.s.resize((size_t)m.E * m.N * G64);
  m.b.resize((size_t)m.E * m.N * G64);
  int n0 = 0;
  for (auto& pt : parts) {
    std::vector<uint32_t> w((size_t)m.E * pt.n * wrow);
    ck.read_into(*pt.w, w.data(), w.size() * 4);
    for (int e = 0; e < m.E; e++)
      memcpy(m.wq.data() + ((size_t)e * m.N + n0) * wrow, w.data() + (size_t)e * pt.n * wrow, (size_t)pt.n * wrow * 4);
    std::vector<uint16_t> tmp((size_t)m.E * pt.n * pt.G);
    for (int which = 0; which < 2; which++) {
      ck.read_into(which ? *pt.b : *pt.s, tmp.data(), tmp.size() * 2);
      for (int e = 0; e < m.E; e++)
        expand_groups(tmp.data() + (size_t)e * pt.n * pt.G, (size_t)pt.n, pt.G, pt.f,
                      (which ? m.b : m.s).data() + ((size_t)e * m.N + n0) * G64);
    }
    n0 += pt.n;
  }
  return m;
}

inline float ckpt_bf2f(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
inline uint16_t ckpt_f2bf(float f) {  // round to nearest even
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Load-time affine quantization of bf16 rows [N, K] to `bits` (4 or 8), group 64 (reference load_qlinear_bf16_q8,
// weights.h:349-406): per group, lo / hi the min / max, scale = (hi - lo) / (2^bits - 1) (1e-8 when 0), both rounded
// to bf16; q = clamp(round((w - lo_bf16) / scale_bf16), 0, 2^bits - 1).
inline HostQLinear quantize_affine(const uint16_t* w, int N, int K, int bits) {
  if ((bits != 4 && bits != 8) || K % 64 || N < 0) throw CkptError("quantize_affine: bits 4 or 8, K a multiple of 64");
  HostQLinear q;
  q.N = N, q.K = K, q.bits = bits;
  const float levels = (float)((1 << bits) - 1);
  const int G = K / 64, per = 32 / bits;
  q.wq.assign((size_t)N * K / per, 0u);
  q.s.resize((size_t)N * G);
  q.b.resize((size_t)N * G);
  for (int r = 0; r < N; r++)
    for (int g = 0; g < G; g++) {
      const uint16_t* x = w + (size_t)r * K + g * 64;
      float lo = INFINITY, hi = -INFINITY;
      for (int i = 0; i < 64; i++) lo = std::fmin(lo, ckpt_bf2f(x[i])), hi = std::fmax(hi, ckpt_bf2f(x[i]));
      float sc = (hi - lo) / levels;
      if (sc == 0.f) sc = 1e-8f;
      const uint16_t sb = ckpt_f2bf(sc), bb = ckpt_f2bf(lo);
      q.s[(size_t)r * G + g] = sb;
      q.b[(size_t)r * G + g] = bb;
      const float scr = ckpt_bf2f(sb), lor = ckpt_bf2f(bb);
      for (int i = 0; i < 64; i++) {
        const float v = (ckpt_bf2f(x[i]) - lor) / scr;
        const uint32_t u = (uint32_t)std::fmin(levels, std::fmax(0.f, std::round(v)));
        const size_t e = (size_t)r * K + g * 64 + i;
        q.wq[e / per] |= u << (bits * (e % per));
      }
    }
  return q;
}

// BF16 linears [n_i, K] fused by rows and quantized at load (the reference's path for unquantized checkpoints).
inline HostQLinear load_qlinear_bf16(const Checkpoint& ck, const std::vector<std::string>& names, int bits) {
  if (names.empty()) throw CkptError("load_qlinear_bf16: no tensors named");
  if (bits != 4 && bits != 8) throw CkptError(std::to_string(bits) + "-bit quantization is not supported");
  int N = 0, K = 0;
  for (auto& n : names) {
    ck.need_dtype(n, "BF16");
    const int r = ck.dim(n, 2, 0), k = ck.dim(n, 2, 1);
    if (k % 64) ck.reject(n, "K is not a multiple of 64");
    if (K && K != k) ck.reject(n, "fused parts differ in K");
    if ((int64_t)N + r > (1 << 30)) ck.reject(n, "fused rows overflow");
    K = k, N += r;
  }
  std::vector<uint16_t> w((size_t)N * K);
  size_t r0 = 0;
  for (auto& n : names) {
    const TensorInfo& ti = ck.info(n);
    ck.read_into(ti, w.data() + r0 * K, (w.size() - r0 * K) * 2);
    r0 += (size_t)ti.shape[0];
  }
  return quantize_affine(w.data(), N, K, bits);
}

}  // namespace inferd
