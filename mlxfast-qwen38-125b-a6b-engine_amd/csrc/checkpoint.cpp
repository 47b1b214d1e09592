// Safetensors checkpoints on the host: the header reader (the validation rules of
// Sources/MLXFastCore/Safetensors.swift:75-176) over a read-only mapping of each file, and the loader
// that turns an MLX affine-4-bit checkpoint of the 125B-A6B family into a target and its MTP head
// through mtpx_target_adopt / mtpx_head_adopt.  The tensor names and the load-time transforms follow
// the reference's binding of the loaded module (Runner/FastModel/TrackFastModel.swift:365-575:
// hyper-connection norm scale times 1/hc, the GDN in-projection rows qkv | z | b | a, q_proj rows
// regrouped as every head's query then every head's gate, the indexer's key rows; the head,
// Runner/FastModel/TrackFastHead.swift:56-61) and the checkpoint inventory of
// Sources/MLXFastTransform/Qwen4ExpCheckpointValidation.swift:312-510 (dtypes and shapes checked per
// tensor).  The reference adopts a module that mlx-swift-lm loaded (Runner/Qwen4ExpRunner.swift:135-229,
// 324-342); here the library reads the files itself and the target/head own the device copies.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mtpx.h"
#include "abi_internal.h"

namespace {

using mtpx::set_error;

// ---------------------------------------------------------------------------------------------
// A minimal JSON reader (objects, arrays, strings with escapes, numbers, literals) for headers.
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool is_int = false;
  int64_t i = 0;
  double d = 0.0;
  std::string s;
  std::vector<JVal> a;
  std::vector<std::pair<std::string, JVal>> o;
};

struct JParser {
  const char* p;
  const char* e;
  std::string err;

  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail(const char* m) {
    if (err.empty()) err = m;
    return false;
  }
  static void utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (e - p < 4) return fail("short \\u escape");
    v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool str(std::string& out) {
    if (p >= e || *p != '"') return fail("expected a string");
    ++p;
    while (p < e && *p != '"') {
      const unsigned char c = (unsigned char)*p++;
      if (c < 0x20) return fail("control character in a string");
      if (c != '\\') {
        out += (char)c;
        continue;
      }
      if (p >= e) return fail("unterminated escape");
      const char x = *p++;
      switch (x) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // a surrogate pair
            uint32_t lo;
            if (e - p < 6 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
            p += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= e) return fail("unterminated string");
    ++p;
    return true;
  }
  bool num(JVal& v) {
    const char* s0 = p;
    if (p < e && *p == '-') ++p;
    bool integral = true;
    while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
      if (*p == '.' || *p == 'e' || *p == 'E') integral = false;
      ++p;
    }
    const std::string t(s0, p);
    if (t.empty() || t == "-") return fail("bad number");
    v.kind = JVal::NUM;
    char* end = nullptr;
    v.d = strtod(t.c_str(), &end);
    if (!end || *end) return fail("bad number");
    if (integral) {
      errno = 0;
      const long long ll = strtoll(t.c_str(), &end, 10);
      v.is_int = errno == 0 && end && !*end;
      v.i = ll;
    }
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("unexpected end");
    const char c = *p;
    if (c == '{') {
      ++p;
      v.kind = JVal::OBJ;
      ws();
      if (p < e && *p == '}') {
        ++p;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail("expected ':'");
        ++p;
        v.o.emplace_back(std::move(k), JVal());
        if (!value(v.o.back().second, depth + 1)) return false;
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == '}') {
          ++p;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p;
      v.kind = JVal::ARR;
      ws();
      if (p < e && *p == ']') {
        ++p;
        return true;
      }
      for (;;) {
        v.a.emplace_back();
        if (!value(v.a.back(), depth + 1)) return false;
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == ']') {
          ++p;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = JVal::STR;
      return str(v.s);
    }
    if (c == 't' && e - p >= 4 && !strncmp(p, "true", 4)) {
      p += 4;
      v.kind = JVal::BOOL;
      return true;
    }
    if (c == 'f' && e - p >= 5 && !strncmp(p, "false", 5)) {
      p += 5;
      v.kind = JVal::BOOL;
      return true;
    }
    if (c == 'n' && e - p >= 4 && !strncmp(p, "null", 4)) {
      p += 4;
      v.kind = JVal::NUL;
      return true;
    }
    return num(v);
  }
};

// ---------------------------------------------------------------------------------------------
// One safetensors file: header parsed and checked, the file mapped read-only.
constexpr uint64_t MAX_HEADER = 100000000;  // the reference implementation's header limit

struct StTensor {
  std::string name, dtype;
  std::vector<int64_t> shape;
  int64_t start = 0, end = 0;  // byte range within the data section
};

struct StFile {
  std::string path;
  int fd = -1;
  size_t size = 0;
  const uint8_t* map = nullptr;
  uint64_t header_len = 0;
  std::map<std::string, std::string> meta;
  std::vector<StTensor> tensors;  // sorted by name
  std::unordered_map<std::string, size_t> index;

  const uint8_t* data(const StTensor& t) const { return map + 8 + header_len + t.start; }
  ~StFile() {
    if (map) munmap(const_cast<uint8_t*>(map), size);
    if (fd >= 0) close(fd);
  }
};

int64_t dtype_bytes(const std::string& d) {
  static const std::map<std::string, int64_t> sz = {
      {"BOOL", 1}, {"U8", 1}, {"I8", 1}, {"F8_E4M3", 1}, {"F8_E5M2", 1}, {"I16", 2}, {"U16", 2}, {"F16", 2},
      {"BF16", 2}, {"I32", 4}, {"U32", 4}, {"F32", 4}, {"I64", 8}, {"U64", 8}, {"F64", 8}};
  const auto it = sz.find(d);
  return it == sz.end() ? 0 : it->second;
}

int fail_st(const std::string& m) { return set_error(MTPX_ERR_ARG, m.c_str()); }

bool int_array(const JVal& v, std::vector<int64_t>& out) {
  if (v.kind != JVal::ARR) return false;
  for (const JVal& x : v.a) {
    if (x.kind != JVal::NUM || !x.is_int) return false;
    out.push_back(x.i);
  }
  return true;
}

int st_open(const std::string& path, StFile** out) {
  StFile* f = new StFile();
  f->path = path;
  auto bad = [&](const std::string& m) {
    delete f;
    return fail_st(m + ": " + path);
  };
  f->fd = open(path.c_str(), O_RDONLY);
  if (f->fd < 0) return bad("cannot open safetensors file");
  struct stat sb;
  if (fstat(f->fd, &sb) != 0) return bad("cannot stat safetensors file");
  f->size = (size_t)sb.st_size;
  if (f->size < 8) return bad("safetensors file is too small");
  uint8_t pre[8];
  if (pread(f->fd, pre, 8, 0) != 8) return bad("safetensors file is too small");
  uint64_t hl = 0;
  for (int k = 7; k >= 0; --k) hl = (hl << 8) | pre[k];  // little endian
  if (hl == 0) return bad("safetensors header is empty");
  if (hl > MAX_HEADER) return bad("safetensors header exceeds 100000000 bytes");
  if (hl > f->size - 8) return bad("truncated safetensors header");
  f->header_len = hl;
  std::string hdr(hl, '\0');
  if (pread(f->fd, &hdr[0], hl, 8) != (ssize_t)hl) return bad("truncated safetensors header");
  JParser jp{hdr.data(), hdr.data() + hdr.size(), {}};
  JVal root;
  if (!jp.value(root, 0)) return bad("invalid safetensors header JSON (" + jp.err + ")");
  jp.ws();
  if (jp.p != jp.e) return bad("invalid safetensors header JSON (trailing data)");
  if (root.kind != JVal::OBJ) return bad("safetensors header must be a JSON object");
  const int64_t data_bytes = (int64_t)(f->size - 8 - hl);
  for (const auto& kv : root.o) {
    const std::string& name = kv.first;
    const JVal& v = kv.second;
    if (name == "__metadata__") {
      if (v.kind == JVal::OBJ) {  // a string map; anything else is ignored
        bool all = true;
        for (const auto& m : v.o) all = all && m.second.kind == JVal::STR;
        if (all)
          for (const auto& m : v.o) f->meta[m.first] = m.second.s;
      }
      continue;
    }
    if (v.kind != JVal::OBJ) continue;
    const JVal *dt = nullptr, *sh = nullptr, *off = nullptr;
    for (const auto& m : v.o) {
      if (m.first == "dtype") dt = &m.second;
      if (m.first == "shape") sh = &m.second;
      if (m.first == "data_offsets") off = &m.second;
    }
    if (!dt || dt->kind != JVal::STR) return bad("invalid tensor header for " + name);
    StTensor t;
    t.name = name;
    t.dtype = dt->s;
    std::vector<int64_t> o;
    if (!sh || !int_array(*sh, t.shape)) return bad("invalid shape for " + name);
    for (int64_t d : t.shape)
      if (d < 0) return bad("invalid shape for " + name);
    if (!off || !int_array(*off, o) || o.size() != 2) return bad("invalid tensor header for " + name);
    if (o[0] < 0 || o[1] < o[0]) return bad("invalid data_offsets for " + name);
    if (o[1] > data_bytes) return bad("data_offsets for " + name + " exceed safetensors file size");
    t.start = o[0];
    t.end = o[1];
    if (f->index.count(name)) return bad("tensor " + name + " appears twice");
    f->index[name] = 0;
    f->tensors.push_back(std::move(t));
  }
  std::sort(f->tensors.begin(), f->tensors.end(), [](const StTensor& a, const StTensor& b) { return a.name < b.name; });
  for (size_t i = 0; i < f->tensors.size(); ++i) f->index[f->tensors[i].name] = i;
  void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
  if (m == MAP_FAILED) return bad("cannot map safetensors file");
  f->map = static_cast<const uint8_t*>(m);
  *out = f;
  return MTPX_OK;
}

// The byte count the dtype and shape call for (-1: unknown dtype or overflow).
int64_t expected_bytes(const StTensor& t) {
  int64_t n = dtype_bytes(t.dtype);
  if (!n) return -1;
  for (int64_t d : t.shape) {
    if (d && n > INT64_MAX / d) return -1;
    n *= d;
  }
  return n;
}

// ---------------------------------------------------------------------------------------------
// A checkpoint: several files, one name space.
struct Checkpoint {
  std::vector<StFile*> files;
  std::unordered_map<std::string, std::pair<StFile*, size_t>> where;
  ~Checkpoint() {
    for (StFile* f : files) delete f;
  }
  const StTensor* find(const std::string& n, StFile** f) const {
    const auto it = where.find(n);
    if (it == where.end()) return nullptr;
    *f = it->second.first;
    return &it->second.first->tensors[it->second.second];
  }
};

bool ends_with(const std::string& s, const char* suf) {
  const size_t n = strlen(suf);
  return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

// ---------------------------------------------------------------------------------------------
// The loader: device copies of the checkpoint's tensors, transformed where the binding transforms them.
struct Loader {
  mtpx_ctx ctx;
  const Checkpoint* ck;
  std::vector<void*> allocs;  // device buffers, handed to the target/head on success
  std::string err;
  int code = MTPX_OK;

  void release() {
    for (void* q : allocs) (void)hipFree(q);
    allocs.clear();
  }
  bool fail(int c, const std::string& m) {
    if (code == MTPX_OK) {
      code = c;
      err = m;
    }
    return false;
  }
  void* dalloc(size_t n) {
    void* p = nullptr;
    if (hipMalloc(&p, n ? n : 4) != hipSuccess) {
      fail(MTPX_ERR_OOM, "checkpoint: device allocation of " + std::to_string(n) + " bytes failed");
      return nullptr;
    }
    allocs.push_back(p);
    return p;
  }
  // The tensor `name` with this dtype and shape (a -1 entry: any extent), or null after an error.
  const StTensor* get(const std::string& name, const char* dtype, std::vector<int64_t> shape, StFile** f) {
    if (code) return nullptr;
    const StTensor* t = ck->find(name, f);
    if (!t) return fail(MTPX_ERR_ARG, "checkpoint: tensor " + name + " is missing"), nullptr;
    bool ok = t->dtype == dtype && t->shape.size() == shape.size();
    for (size_t k = 0; ok && k < shape.size(); ++k) ok = shape[k] < 0 || shape[k] == t->shape[k];
    if (!ok) {
      std::string want = std::string(dtype) + " [";
      for (size_t k = 0; k < shape.size(); ++k) want += (k ? ", " : "") + std::to_string(shape[k]);
      std::string got = t->dtype + " [";
      for (size_t k = 0; k < t->shape.size(); ++k) got += (k ? ", " : "") + std::to_string(t->shape[k]);
      return fail(MTPX_ERR_ARG, "checkpoint: tensor " + name + " is " + got + "], expected " + want + "]"), nullptr;
    }
    if (expected_bytes(*t) != t->end - t->start)
      return fail(MTPX_ERR_ARG, "checkpoint: tensor " + name + ": data size does not match its dtype and shape"),
             nullptr;
    return t;
  }
  bool upload(void* dst, const void* src, size_t n) {
    if (!n) return true;
    if (hipMemcpy(dst, src, n, hipMemcpyHostToDevice) != hipSuccess)
      return fail(MTPX_ERR_HIP, "checkpoint: host to device copy failed");
    return true;
  }
  // A tensor as one device buffer.
  const void* tensor(const std::string& name, const char* dtype, std::vector<int64_t> shape) {
    StFile* f = nullptr;
    const StTensor* t = get(name, dtype, shape, &f);
    if (!t) return nullptr;
    void* d = dalloc((size_t)(t->end - t->start));
    if (!d || !upload(d, f->data(*t), (size_t)(t->end - t->start))) return nullptr;
    return d;
  }
  // Host bytes of a small tensor.
  std::vector<uint8_t> host(const std::string& name, const char* dtype, std::vector<int64_t> shape) {
    StFile* f = nullptr;
    const StTensor* t = get(name, dtype, shape, &f);
    if (!t) return {};
    const uint8_t* p = f->data(*t);
    return std::vector<uint8_t>(p, p + (t->end - t->start));
  }

  // An affine-4-bit matrix (stem.weight U32 [lead.., K/8], .scales / .biases BF16 [lead.., K/gs]).
  bool q4(const std::string& stem, std::vector<int64_t> lead, int64_t K, int gs, mtpx_q4* q) {
    std::vector<int64_t> ws = lead, ss = lead;
    ws.push_back(K / 8);
    ss.push_back(K / gs);
    q->w = static_cast<const uint32_t*>(tensor(stem + ".weight", "U32", ws));
    q->s = static_cast<const uint16_t*>(tensor(stem + ".scales", "BF16", ss));
    q->b = static_cast<const uint16_t*>(tensor(stem + ".biases", "BF16", ss));
    q->sb = nullptr;
    return code == MTPX_OK;
  }

  // Several affine-4-bit matrices over the same K, stacked by rows into one matrix.  `parts`:
  // (stem, rows, first row, row count) -- rows [first, first + count) of a stem of `rows` rows;
  // `order` (optional, for one part): a row permutation applied to that part.
  struct Part {
    std::string stem;
    int64_t rows, first, count;
    const std::vector<int64_t>* order;
  };
  bool q4_rows(const std::vector<Part>& parts, int64_t K, int gs, mtpx_q4* q) {
    int64_t N = 0;
    for (const Part& p : parts) N += p.count;
    const int64_t wb = K / 2, sbb = 2 * (K / gs);  // bytes per row
    uint8_t* dw = static_cast<uint8_t*>(dalloc((size_t)(N * wb)));
    uint8_t* ds = static_cast<uint8_t*>(dalloc((size_t)(N * sbb)));
    uint8_t* db = static_cast<uint8_t*>(dalloc((size_t)(N * sbb)));
    if (code) return false;
    int64_t at = 0;
    for (const Part& p : parts) {
      StFile *fw = nullptr, *fs = nullptr, *fb = nullptr;
      const StTensor* tw = get(p.stem + ".weight", "U32", {p.rows, K / 8}, &fw);
      const StTensor* ts = get(p.stem + ".scales", "BF16", {p.rows, K / gs}, &fs);
      const StTensor* tb = get(p.stem + ".biases", "BF16", {p.rows, K / gs}, &fb);
      if (code) return false;
      struct {
        const uint8_t* src;
        uint8_t* dst;
        int64_t rb;
      } m[3] = {{fw->data(*tw), dw, wb}, {fs->data(*ts), ds, sbb}, {fb->data(*tb), db, sbb}};
      for (auto& x : m) {
        if (p.order) {  // a permuted part: gathered on the host, copied once
          std::vector<uint8_t> tmp((size_t)(p.count * x.rb));
          for (int64_t r = 0; r < p.count; ++r)
            memcpy(&tmp[(size_t)(r * x.rb)], x.src + (size_t)((*p.order)[r] * x.rb), (size_t)x.rb);
          if (!upload(x.dst + at * x.rb, tmp.data(), tmp.size())) return false;
        } else if (!upload(x.dst + at * x.rb, x.src + p.first * x.rb, (size_t)(p.count * x.rb))) {
          return false;
        }
      }
      at += p.count;
    }
    q->w = reinterpret_cast<const uint32_t*>(dw);
    q->s = reinterpret_cast<const uint16_t*>(ds);
    q->b = reinterpret_cast<const uint16_t*>(db);
    q->sb = nullptr;
    return true;
  }

  // A bf16 vector scaled by a bf16 factor in bf16 arithmetic (the product of two bf16 values in float,
  // rounded to nearest even): the hyper-connection norm scale = hc_norm.weight * (1 / hc).
  const uint16_t* bf16_scaled(const std::string& name, int64_t n, float factor) {
    std::vector<uint8_t> h = host(name, "BF16", {n});
    if (code) return nullptr;
    auto to_f = [](uint16_t v) {
      uint32_t u = (uint32_t)v << 16;
      float f;
      memcpy(&f, &u, 4);
      return f;
    };
    auto to_bf = [](float f) {
      uint32_t u;
      memcpy(&u, &f, 4);
      if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // NaN stays NaN
      u += 0x7fffu + ((u >> 16) & 1u);
      return (uint16_t)(u >> 16);
    };
    const float fb = to_f(to_bf(factor));
    std::vector<uint16_t> out((size_t)n);
    for (int64_t i = 0; i < n; ++i) {
      uint16_t v;
      memcpy(&v, &h[(size_t)(2 * i)], 2);
      out[(size_t)i] = to_bf(to_f(v) * fb);
    }
    void* d = dalloc(2 * (size_t)n);
    if (!d || !upload(d, out.data(), 2 * (size_t)n)) return nullptr;
    return static_cast<const uint16_t*>(d);
  }

  bool hc(const std::string& stem, int H, int hcn, int LW, int gs, bool inject, mtpx_hc_weights* m) {
    const int W = hcn * H;
    memset(m, 0, sizeof(*m));
    m->norm_scale = bf16_scaled(stem + ".hc_norm.weight", W, 1.0f / (float)hcn);
    q4(stem + ".input_mix_weight_down", {LW}, W, gs, &m->down);
    q4(stem + ".input_mix_weight_up", {W}, LW, gs, &m->up);
    if (inject) q4(stem + ".block_inject_weight", {hcn}, W, gs, &m->inject);
    return code == MTPX_OK;
  }

  // The MoE block (mlp.*): bf16 router, stacked routed experts, shared expert, q4 shared gate.
  bool moe(const std::string& p, const mtpx_layer_config& lc, mtpx_moe_weights* m) {
    const int H = lc.hidden, E = lc.experts, F = lc.expert_width, gs = lc.group_size;
    memset(m, 0, sizeof(*m));
    m->hidden = H;
    m->experts = E;
    m->top_k = lc.top_k;
    m->expert_width = F;
    m->group_size = gs;
    m->router = static_cast<const uint16_t*>(tensor(p + "mlp.gate.weight", "BF16", {E, H}));
    mtpx_q4 q;
    q4(p + "mlp.switch_mlp.gate_proj", {E, F}, H, gs, &q);
    m->gate_w = q.w, m->gate_s = q.s, m->gate_b = q.b;
    q4(p + "mlp.switch_mlp.up_proj", {E, F}, H, gs, &q);
    m->up_w = q.w, m->up_s = q.s, m->up_b = q.b;
    q4(p + "mlp.switch_mlp.down_proj", {E, H}, F, gs, &q);
    m->down_w = q.w, m->down_s = q.s, m->down_b = q.b;
    q4(p + "mlp.shared_expert.gate_proj", {F}, H, gs, &q);
    m->sh_gate_w = q.w, m->sh_gate_s = q.s, m->sh_gate_b = q.b;
    q4(p + "mlp.shared_expert.up_proj", {F}, H, gs, &q);
    m->sh_up_w = q.w, m->sh_up_s = q.s, m->sh_up_b = q.b;
    q4(p + "mlp.shared_expert.down_proj", {H}, F, gs, &q);
    m->sh_down_w = q.w, m->sh_down_s = q.s, m->sh_down_b = q.b;
    q4(p + "mlp.shared_expert_gate", {1}, H, gs, &q);
    m->shared_gate_w = q.w, m->shared_gate_s = q.s, m->shared_gate_b = q.b;
    return code == MTPX_OK;
  }

  // An attention layer's weights (self_attn.*) and its MoE.
  bool attention(const std::string& p, const mtpx_layer_config& lc, mtpx_layer_weights* w) {
    const int H = lc.hidden, HQ = lc.heads, HK = lc.kv_heads, D = lc.head_dim, gs = lc.group_size;
    memset(w, 0, sizeof(*w));
    // q_proj rows per head [query (D) | gate (D)] -> every head's query, then every head's gate
    std::vector<int64_t> order;
    for (int h = 0; h < HQ; ++h)
      for (int i = 0; i < D; ++i) order.push_back((int64_t)h * 2 * D + i);
    for (int h = 0; h < HQ; ++h)
      for (int i = 0; i < D; ++i) order.push_back((int64_t)h * 2 * D + D + i);
    // the indexer projection's rows: its query heads, then the key rows the cache keeps (the last index_dim)
    StFile* f = nullptr;
    const StTensor* ix = ck->find(p + "self_attn.indexer.index_qk_proj.weight", &f);
    if (!ix || ix->shape.size() != 2) return fail(MTPX_ERR_ARG, "checkpoint: tensor " + p +
                                                                     "self_attn.indexer.index_qk_proj.weight is missing");
    const int64_t irows = ix->shape[0];
    if (irows < lc.index_dim) return fail(MTPX_ERR_ARG, "checkpoint: the indexer projection has fewer rows than index_dim");
    mtpx_q4 qkv;
    q4_rows({{p + "self_attn.q_proj", 2LL * HQ * D, 0, 2LL * HQ * D, &order},
             {p + "self_attn.k_proj", (int64_t)HK * D, 0, (int64_t)HK * D, nullptr},
             {p + "self_attn.v_proj", (int64_t)HK * D, 0, (int64_t)HK * D, nullptr},
             {p + "self_attn.indexer.index_qk_proj", irows, irows - lc.index_dim, lc.index_dim, nullptr}},
            H, gs, &qkv);
    w->qkv_w = qkv.w, w->qkv_s = qkv.s, w->qkv_b = qkv.b;
    w->qkv_rows = 2 * HQ * D + 2 * HK * D + lc.index_dim;
    w->q_norm = static_cast<const uint16_t*>(tensor(p + "self_attn.q_norm.weight", "BF16", {D}));
    w->k_norm = static_cast<const uint16_t*>(tensor(p + "self_attn.k_norm.weight", "BF16", {D}));
    mtpx_q4 o;
    q4(p + "self_attn.o_proj", {H}, (int64_t)HQ * D, gs, &o);
    w->o_w = o.w, w->o_s = o.s, w->o_b = o.b;
    return moe(p, lc, &w->moe);
  }

  // A GDN layer's linear_attn.* weights.
  bool gdn(const std::string& p, const mtpx_target_config& cfg, mtpx_gdn_weights* g) {
    const int H = cfg.layer.hidden, gs = cfg.layer.group_size, hk = cfg.key_heads, hv = cfg.value_heads;
    const int kc = cfg.conv_kernel;
    const int64_t cd = (2LL * hk + hv) * 128, vd = (int64_t)hv * 128;
    memset(g, 0, sizeof(*g));
    q4_rows({{p + "linear_attn.in_proj_qkv", cd, 0, cd, nullptr},
             {p + "linear_attn.in_proj_z", vd, 0, vd, nullptr},
             {p + "linear_attn.in_proj_b", hv, 0, hv, nullptr},
             {p + "linear_attn.in_proj_a", hv, 0, hv, nullptr}},
            H, gs, &g->in_proj);
    g->conv_w = static_cast<const uint16_t*>(tensor(p + "linear_attn.conv1d.weight", "BF16", {cd, kc, 1}));
    // -exp(A_log) in float32 (TrackFastModel.swift:418-419)
    std::vector<uint8_t> al = host(p + "linear_attn.A_log", "BF16", {hv});
    if (code) return false;
    std::vector<float> nea((size_t)hv);
    for (int i = 0; i < hv; ++i) {
      uint16_t v;
      memcpy(&v, &al[(size_t)(2 * i)], 2);
      uint32_t u = (uint32_t)v << 16;
      float a;
      memcpy(&a, &u, 4);
      nea[(size_t)i] = (float)-exp((double)a);  // exp in double, rounded once to float
    }
    void* d = dalloc(4 * (size_t)hv);
    if (!d || !upload(d, nea.data(), 4 * (size_t)hv)) return false;
    g->neg_exp_alog = static_cast<const float*>(d);
    g->dt_bias = static_cast<const uint16_t*>(tensor(p + "linear_attn.dt_bias", "BF16", {hv}));
    g->norm_w = static_cast<const uint16_t*>(tensor(p + "linear_attn.norm.weight", "BF16", {128}));
    q4(p + "linear_attn.out_proj", {H}, vd, gs, &g->out_proj);
    return code == MTPX_OK;
  }

  // The PLE block (ple.*) with its table assembled from the checkpoint's shards.
  bool ple(const std::string& p, const mtpx_ple_config& pc, mtpx_ple_weights* w) {
    const int W = pc.hc * pc.hidden, Ed = pc.embed_dim, gs = pc.group_size, rgs = pc.row_group_size;
    const int nh = (pc.ngram_size - 1) * pc.heads_per_ngram;
    const int64_t rd = Ed / nh;
    memset(w, 0, sizeof(*w));
    q4(p + "key_proj", {W}, Ed, gs, &w->key_proj);
    q4(p + "value_proj", {pc.hidden}, Ed, gs, &w->value_proj);
    w->norm_key = static_cast<const uint16_t*>(tensor(p + "norm_key.weight", "BF16", {W}));
    w->norm_query = static_cast<const uint16_t*>(tensor(p + "norm_query.weight", "BF16", {W}));
    w->norm_conv = static_cast<const uint16_t*>(tensor(p + "norm_conv.weight", "BF16", {W}));
    w->conv_w = static_cast<const uint16_t*>(tensor(p + "conv1d.weight", "BF16", {W, pc.conv_kernel, 1}));
    // the table: shard_0, shard_1, ... in order, rows stacked
    std::vector<Part> parts;
    for (int j = 0;; ++j) {
      StFile* f = nullptr;
      const std::string stem = p + "ple_embedding.ngram_embedding.shard_" + std::to_string(j);
      const StTensor* t = ck->find(stem + ".weight", &f);
      if (!t) break;
      if (t->shape.size() != 2) return fail(MTPX_ERR_ARG, "checkpoint: tensor " + stem + ".weight is not 2-D");
      parts.push_back({stem, t->shape[0], 0, t->shape[0], nullptr});
    }
    if (parts.empty()) return fail(MTPX_ERR_ARG, "checkpoint: no n-gram table shards under " + p);
    mtpx_q4 tab;
    if (!q4_rows(parts, rd, rgs, &tab)) return false;
    int64_t rows = 0;
    for (const Part& x : parts) rows += x.count;
    w->table.w = tab.w, w->table.s = tab.s, w->table.b = tab.b;
    w->table.rows = rows;
    std::vector<uint8_t> mult = host(p + "ple_embedding.layer_multipliers", "I64", {pc.ngram_size});
    if (code) return false;
    for (int k = 0; k < pc.ngram_size && k < MTPX_PLE_MAX_NGRAM; ++k)
      memcpy(&w->table.multiplier[k], &mult[(size_t)(8 * k)], 8);
    return code == MTPX_OK;
  }
};

std::string text_prefix(const char* prefix) { return prefix ? std::string(prefix) : std::string("language_model."); }

}  // namespace

extern "C" {

int mtpx_st_open(const char* path, mtpx_st* out) {
  if (!path || !out) return set_error(MTPX_ERR_ARG, "st_open: null argument");
  StFile* f = nullptr;
  const int rc = st_open(path, &f);
  if (rc) return rc;
  out->ctx = f;
  return MTPX_OK;
}

int mtpx_st_free(mtpx_st st) {
  delete static_cast<StFile*>(st.ctx);
  return MTPX_OK;
}

int mtpx_st_count(mtpx_st st, int64_t* n) {
  StFile* f = static_cast<StFile*>(st.ctx);
  if (!f || !n) return set_error(MTPX_ERR_ARG, "st_count: null argument");
  *n = (int64_t)f->tensors.size();
  return MTPX_OK;
}

int mtpx_st_tensor(mtpx_st st, int64_t i, const char** name, const char** dtype, int* ndim, const int64_t** shape,
                   int64_t* nbytes) {
  StFile* f = static_cast<StFile*>(st.ctx);
  if (!f) return set_error(MTPX_ERR_ARG, "st_tensor: null file");
  if (i < 0 || i >= (int64_t)f->tensors.size()) return set_error(MTPX_ERR_ARG, "st_tensor: index out of range");
  const StTensor& t = f->tensors[(size_t)i];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype.c_str();
  if (ndim) *ndim = (int)t.shape.size();
  if (shape) *shape = t.shape.data();
  if (nbytes) *nbytes = t.end - t.start;
  return MTPX_OK;
}

int mtpx_st_find(mtpx_st st, const char* name, int64_t* i) {
  StFile* f = static_cast<StFile*>(st.ctx);
  if (!f || !name || !i) return set_error(MTPX_ERR_ARG, "st_find: null argument");
  const auto it = f->index.find(name);
  if (it == f->index.end()) {
    *i = -1;
    return set_error(MTPX_ERR_ARG, (std::string("st_find: no tensor ") + name).c_str());
  }
  *i = (int64_t)it->second;
  return MTPX_OK;
}

int mtpx_st_metadata(mtpx_st st, const char* key, const char** value) {
  StFile* f = static_cast<StFile*>(st.ctx);
  if (!f || !key || !value) return set_error(MTPX_ERR_ARG, "st_metadata: null argument");
  const auto it = f->meta.find(key);
  *value = it == f->meta.end() ? nullptr : it->second.c_str();
  return MTPX_OK;
}

int mtpx_st_read(mtpx_st st, int64_t i, void* dst, int64_t nbytes) {
  StFile* f = static_cast<StFile*>(st.ctx);
  if (!f || !dst) return set_error(MTPX_ERR_ARG, "st_read: null argument");
  if (i < 0 || i >= (int64_t)f->tensors.size()) return set_error(MTPX_ERR_ARG, "st_read: index out of range");
  const StTensor& t = f->tensors[(size_t)i];
  if (nbytes != t.end - t.start) return set_error(MTPX_ERR_ARG, "st_read: byte count differs from the tensor's");
  memcpy(dst, f->data(t), (size_t)nbytes);
  return MTPX_OK;
}

int mtpx_checkpoint_open(const char* const* paths, int n, mtpx_checkpoint* out) {
  if (!paths || n < 1 || !out) return set_error(MTPX_ERR_ARG, "checkpoint_open: bad argument");
  std::vector<std::string> files;
  for (int k = 0; k < n; ++k) {
    if (!paths[k]) return set_error(MTPX_ERR_ARG, "checkpoint_open: null path");
    struct stat sb;
    if (stat(paths[k], &sb) == 0 && S_ISDIR(sb.st_mode)) {  // every *.safetensors file of the directory
      DIR* d = opendir(paths[k]);
      if (!d) return set_error(MTPX_ERR_ARG, "checkpoint_open: cannot read the directory");
      std::vector<std::string> in;
      while (dirent* e = readdir(d))
        if (ends_with(e->d_name, ".safetensors")) in.push_back(std::string(paths[k]) + "/" + e->d_name);
      closedir(d);
      std::sort(in.begin(), in.end());
      files.insert(files.end(), in.begin(), in.end());
    } else {
      files.push_back(paths[k]);
    }
  }
  if (files.empty()) return set_error(MTPX_ERR_ARG, "checkpoint_open: no safetensors files");
  Checkpoint* ck = new Checkpoint();
  for (const std::string& p : files) {
    StFile* f = nullptr;
    const int rc = st_open(p, &f);
    if (rc) {
      delete ck;
      return rc;
    }
    ck->files.push_back(f);
    for (size_t i = 0; i < f->tensors.size(); ++i) {
      const std::string& nm = f->tensors[i].name;
      if (ck->where.count(nm)) {
        const std::string m = "checkpoint_open: tensor " + nm + " is in two files";
        delete ck;
        return set_error(MTPX_ERR_ARG, m.c_str());
      }
      ck->where[nm] = {f, i};
    }
  }
  out->ctx = ck;
  return MTPX_OK;
}

int mtpx_checkpoint_free(mtpx_checkpoint ck) {
  delete static_cast<Checkpoint*>(ck.ctx);
  return MTPX_OK;
}

int mtpx_checkpoint_count(mtpx_checkpoint ck, int64_t* n) {
  Checkpoint* c = static_cast<Checkpoint*>(ck.ctx);
  if (!c || !n) return set_error(MTPX_ERR_ARG, "checkpoint_count: null argument");
  *n = (int64_t)c->where.size();
  return MTPX_OK;
}

int mtpx_target_load(mtpx_ctx ctx, const mtpx_target_config* cfg, mtpx_checkpoint ck, const char* prefix, int pack_sb,
                     mtpx_target* out) {
  const Checkpoint* c = static_cast<const Checkpoint*>(ck.ctx);
  if (!ctx.ctx || !cfg || !c || !out) return set_error(MTPX_ERR_ARG, "target_load: null argument");
  if (cfg->num_layers < 1 || cfg->num_layers > 4096 || cfg->full_attention_interval < 1)
    return set_error(MTPX_ERR_ARG, "target_load: bad layer schedule");
  if (hipSetDevice(mtpx::ctx_device(ctx)) != hipSuccess) return set_error(MTPX_ERR_HIP, "target_load: hipSetDevice");
  const mtpx_layer_config& lc = cfg->layer;
  const int H = lc.hidden, gs = lc.group_size;
  const std::string tp = text_prefix(prefix), mp = tp + "model.";
  Loader ld{ctx, c, {}, {}, MTPX_OK};
  mtpx_target_weights tw;
  memset(&tw, 0, sizeof(tw));
  ld.q4(mp + "embed_tokens", {cfg->vocab}, H, gs, &tw.embed);
  ld.q4(tp + "lm_head", {cfg->vocab}, H, gs, &tw.lm_head);
  ld.hc(mp + "hyper_connection_mixer", H, cfg->hc, cfg->lowrank, gs, false, &tw.final_hc);
  std::vector<mtpx_target_layer_weights> layers((size_t)cfg->num_layers);
  for (int i = 0; i < cfg->num_layers && !ld.code; ++i) {
    mtpx_target_layer_weights& L = layers[(size_t)i];
    memset(&L, 0, sizeof(L));
    const std::string p = mp + "layers." + std::to_string(i) + ".";
    L.kind = (i + 1) % cfg->full_attention_interval == 0 ? MTPX_LAYER_ATTENTION : MTPX_LAYER_GDN;
    ld.hc(p + "attn_hyper_connection", H, cfg->hc, cfg->lowrank, gs, true, &L.attn_hc);
    ld.hc(p + "mlp_hyper_connection", H, cfg->hc, cfg->lowrank, gs, true, &L.mlp_hc);
    if (L.kind == MTPX_LAYER_ATTENTION) {
      ld.attention(p, lc, &L.attn);
    } else {
      ld.gdn(p, *cfg, &L.gdn);
      ld.moe(p, lc, &L.attn.moe);
    }
    if (i == cfg->ple_layer) ld.ple(p + "ple.", cfg->ple, &L.ple);
  }
  if (ld.code) {
    ld.release();
    return set_error(ld.code, ld.err.c_str());
  }
  mtpx_target t{nullptr};
  const int rc = mtpx_target_adopt(ctx, cfg, &tw, layers.data(), pack_sb, &t);
  if (rc) {
    ld.release();
    return rc;
  }
  // the checkpoint's n-gram head geometry must be the one the config derives
  if (cfg->ple_layer >= 0) {
    const int nh = (cfg->ple.ngram_size - 1) * cfg->ple.heads_per_ngram;
    const std::string p = mp + "layers." + std::to_string(cfg->ple_layer) + ".ple.ple_embedding.";
    std::vector<uint8_t> voc = ld.host(p + "ngram_heads_vocab_sizes", "I64", {nh});
    std::vector<uint8_t> off = ld.host(p + "ngram_heads_offsets", "I64", {nh});
    mtpx_target_layer_weights got;
    if (!ld.code && mtpx_target_layer_weights_get(t, cfg->ple_layer, &got) == MTPX_OK) {
      for (int k = 0; k < nh; ++k) {
        int64_t v, o;
        memcpy(&v, &voc[(size_t)(8 * k)], 8);
        memcpy(&o, &off[(size_t)(8 * k)], 8);
        if (v != got.ple.table.vocab[k] || o != got.ple.table.offset[k]) {
          ld.fail(MTPX_ERR_ARG, "checkpoint: the n-gram head vocabularies/offsets differ from the config's");
          break;
        }
      }
    }
    if (ld.code) {
      mtpx_target_free(t);
      ld.release();
      return set_error(ld.code, ld.err.c_str());
    }
  }
  for (void* q : ld.allocs) mtpx::target_own(t, q);
  *out = t;
  return MTPX_OK;
}

int mtpx_head_load(mtpx_ctx ctx, const mtpx_head_config* cfg, mtpx_checkpoint ck, mtpx_target target,
                   const char* prefix, int pack_sb, mtpx_head* out) {
  const Checkpoint* c = static_cast<const Checkpoint*>(ck.ctx);
  if (!ctx.ctx || !cfg || !c || !target.ctx || !out) return set_error(MTPX_ERR_ARG, "head_load: null argument");
  if (hipSetDevice(mtpx::ctx_device(ctx)) != hipSuccess) return set_error(MTPX_ERR_HIP, "head_load: hipSetDevice");
  const mtpx_layer_config& lc = cfg->layer;
  const int H = lc.hidden, gs = lc.group_size, W = cfg->hc * H;
  const std::string hp = text_prefix(prefix) + "mtp.";
  mtpx_target_weights tw;
  int rc = mtpx_target_weights_get(target, &tw);
  if (rc) return rc;
  int64_t tv = 0;
  int tW = 0;
  mtpx::target_dims(target, &tv, &tW);
  if (tv != cfg->vocab || tW != W) return set_error(MTPX_ERR_ARG, "head_load: the target's vocabulary or width differs");
  Loader ld{ctx, c, {}, {}, MTPX_OK};
  mtpx_head_weights w;
  memset(&w, 0, sizeof(w));
  w.embed = tw.embed;  // the target's embed_tokens: the head has none of its own
  w.pre_norm_embedding = static_cast<const uint16_t*>(ld.tensor(hp + "pre_fc_norm_embedding.weight", "BF16", {H}));
  w.pre_norm_hidden = static_cast<const uint16_t*>(ld.tensor(hp + "pre_fc_norm_hidden.weight", "BF16", {W}));
  ld.q4(hp + "fc_embedding", {H}, H, gs, &w.fc_embedding);
  ld.q4(hp + "fc_hidden", {H}, H, gs, &w.fc_hidden);
  ld.hc(hp + "hyper_connection_mixer", H, cfg->hc, cfg->lowrank, gs, false, &w.final_hc);
  const std::string lp = hp + "layers.0.";
  ld.hc(lp + "attn_hyper_connection", H, cfg->hc, cfg->lowrank, gs, true, &w.attn_hc);
  ld.hc(lp + "mlp_hyper_connection", H, cfg->hc, cfg->lowrank, gs, true, &w.mlp_hc);
  ld.attention(lp, lc, &w.layer);
  // the shortlist: rows of the target's lm_head (ids 0..low-1 then the special ids), copied on the device
  const std::vector<int32_t> ids = mtpx::head_shortlist_ids(cfg);
  const int64_t n = (int64_t)ids.size(), wb = H / 2, sbb = 2 * (H / gs);
  uint8_t* dw = static_cast<uint8_t*>(ld.dalloc((size_t)(n * wb)));
  uint8_t* ds = static_cast<uint8_t*>(ld.dalloc((size_t)(n * sbb)));
  uint8_t* db = static_cast<uint8_t*>(ld.dalloc((size_t)(n * sbb)));
  int32_t* did = static_cast<int32_t*>(ld.dalloc(4 * (size_t)n));
  if (!ld.code) {
    struct {
      const uint8_t* src;
      uint8_t* dst;
      int64_t rb;
    } m[3] = {{reinterpret_cast<const uint8_t*>(tw.lm_head.w), dw, wb},
              {reinterpret_cast<const uint8_t*>(tw.lm_head.s), ds, sbb},
              {reinterpret_cast<const uint8_t*>(tw.lm_head.b), db, sbb}};
    for (auto& x : m)
      for (int64_t r = 0; r < n && !ld.code;) {  // runs of consecutive ids: one copy each
        int64_t e = r + 1;
        while (e < n && ids[(size_t)e] == ids[(size_t)e - 1] + 1) ++e;
        if (hipMemcpy(x.dst + r * x.rb, x.src + (int64_t)ids[(size_t)r] * x.rb, (size_t)((e - r) * x.rb),
                      hipMemcpyDeviceToDevice) != hipSuccess)
          ld.fail(MTPX_ERR_HIP, "head_load: shortlist row copy failed");
        r = e;
      }
    if (!ld.code && !ld.upload(did, ids.data(), 4 * (size_t)n)) {
    }
  }
  w.shortlist.w = reinterpret_cast<const uint32_t*>(dw);
  w.shortlist.s = reinterpret_cast<const uint16_t*>(ds);
  w.shortlist.b = reinterpret_cast<const uint16_t*>(db);
  w.shortlist_ids = did;
  w.shortlist_rows = (int)n;
  if (ld.code) {
    ld.release();
    return set_error(ld.code, ld.err.c_str());
  }
  mtpx_head hd{nullptr};
  rc = mtpx_head_adopt(ctx, cfg, &w, pack_sb, &hd);
  if (rc) {
    ld.release();
    return rc;
  }
  for (void* q : ld.allocs) mtpx::head_own(hd, q);
  *out = hd;
  return MTPX_OK;
}

}  // extern "C"
