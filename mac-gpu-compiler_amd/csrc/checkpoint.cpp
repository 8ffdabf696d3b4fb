// Safetensors/config.json reader and seeded random-init checkpoint writer.
// File contract: metal_infrence_engine/src/cpu_inference.rs:58-96.
#include "checkpoint.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <thread>

namespace qe {
namespace {

// ---------------------------------------------------------------------------------------------
// A small JSON reader: enough for the safetensors header and HF config.json.
// ---------------------------------------------------------------------------------------------
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  bool integral = false;  // written without fraction or exponent, and fits in int64
  int64_t i64 = 0;
  std::string str;
  std::vector<Json> items;
  std::vector<std::string> keys;  // for Obj, parallel to items

  const Json* get(const std::string& k) const {
    const Json* r = nullptr;
    for (size_t i = 0; i < keys.size(); i++)
      if (keys[i] == k) r = &items[i];  // a later duplicate key wins, like a map insert
    return r;
  }
};

class JsonParser {
 public:
  JsonParser(const char* s, size_t n) : s_(s), n_(n) {}
  bool parse(Json& out) {
    if (!value(out, 0)) return false;
    ws();
    return i_ == n_;
  }

 private:
  const char* s_;
  size_t n_, i_ = 0;

  void ws() {
    while (i_ < n_ && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) i_++;
  }
  static int hex(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }
  bool hex4(unsigned& v) {
    if (i_ + 4 > n_) return false;
    v = 0;
    for (int k = 0; k < 4; k++) {
      int h = hex(s_[i_++]);
      if (h < 0) return false;
      v = v * 16 + unsigned(h);
    }
    return true;
  }
  static void utf8(std::string& o, unsigned cp) {
    if (cp < 0x80) {
      o += char(cp);
    } else if (cp < 0x800) {
      o += char(0xC0 | (cp >> 6));
      o += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      o += char(0xE0 | (cp >> 12));
      o += char(0x80 | ((cp >> 6) & 0x3F));
      o += char(0x80 | (cp & 0x3F));
    } else {
      o += char(0xF0 | (cp >> 18));
      o += char(0x80 | ((cp >> 12) & 0x3F));
      o += char(0x80 | ((cp >> 6) & 0x3F));
      o += char(0x80 | (cp & 0x3F));
    }
  }
  bool string(std::string& o) {
    if (i_ >= n_ || s_[i_] != '"') return false;
    i_++;
    while (true) {
      if (i_ >= n_) return false;
      unsigned char c = (unsigned char)s_[i_++];
      if (c == '"') return true;
      if (c < 0x20) return false;
      if (c != '\\') {
        o += char(c);
        continue;
      }
      if (i_ >= n_) return false;
      char e = s_[i_++];
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          unsigned cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {
            unsigned lo;
            if (i_ + 2 > n_ || s_[i_] != '\\' || s_[i_ + 1] != 'u') return false;
            i_ += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return false;
          }
          utf8(o, cp);
          break;
        }
        default: return false;
      }
    }
  }
  bool digits() {
    size_t st = i_;
    while (i_ < n_ && s_[i_] >= '0' && s_[i_] <= '9') i_++;
    return i_ > st;
  }
  bool value(Json& v, int depth) {
    if (depth > 64) return false;
    ws();
    if (i_ >= n_) return false;
    char c = s_[i_];
    if (c == '{' || c == '[') {
      bool obj = c == '{';
      v.kind = obj ? Json::Obj : Json::Arr;
      i_++;
      ws();
      if (i_ < n_ && s_[i_] == (obj ? '}' : ']')) { i_++; return true; }
      while (true) {
        ws();
        if (obj) {
          std::string k;
          if (!string(k)) return false;
          ws();
          if (i_ >= n_ || s_[i_] != ':') return false;
          i_++;
          v.keys.push_back(std::move(k));
        }
        v.items.emplace_back();
        if (!value(v.items.back(), depth + 1)) return false;
        ws();
        if (i_ >= n_) return false;
        if (s_[i_] == ',') { i_++; continue; }
        if (s_[i_] == (obj ? '}' : ']')) { i_++; return true; }
        return false;
      }
    }
    if (c == '"') {
      v.kind = Json::Str;
      return string(v.str);
    }
    auto lit = [&](const char* w) {
      size_t l = strlen(w);
      if (n_ - i_ >= l && memcmp(s_ + i_, w, l) == 0) { i_ += l; return true; }
      return false;
    };
    if (lit("true")) { v.kind = Json::Bool; v.b = true; return true; }
    if (lit("false")) { v.kind = Json::Bool; v.b = false; return true; }
    if (lit("null")) { v.kind = Json::Null; return true; }
    if (c == '-' || (c >= '0' && c <= '9')) {
      size_t st = i_;
      bool integral = true;
      if (s_[i_] == '-') i_++;
      if (!digits()) return false;
      if (i_ < n_ && s_[i_] == '.') { integral = false; i_++; if (!digits()) return false; }
      if (i_ < n_ && (s_[i_] == 'e' || s_[i_] == 'E')) {
        integral = false;
        i_++;
        if (i_ < n_ && (s_[i_] == '+' || s_[i_] == '-')) i_++;
        if (!digits()) return false;
      }
      std::string t(s_ + st, i_ - st);
      v.kind = Json::Num;
      v.num = strtod(t.c_str(), nullptr);
      if (integral) {
        errno = 0;
        long long x = strtoll(t.c_str(), nullptr, 10);
        if (errno == 0) { v.integral = true; v.i64 = x; }
      }
      return true;
    }
    return false;
  }
};

bool json_u64(const Json& o, const char* k, uint64_t& out) {
  const Json* v = o.get(k);
  if (!v || v->kind != Json::Num || !v->integral || v->i64 < 0) return false;
  out = uint64_t(v->i64);
  return true;
}
bool json_f32(const Json& o, const char* k, float& out) {
  const Json* v = o.get(k);
  if (!v || v->kind != Json::Num) return false;
  out = float(v->num);  // serde_json: parse as f64, then `as f32`
  return true;
}
bool fits_i32(const Json& v) {
  return v.kind == Json::Num && v.integral && v.i64 >= INT32_MIN && v.i64 <= INT32_MAX;
}

std::string sibling_config(const std::string& path) {
  size_t slash = path.rfind('/');
  return slash == std::string::npos ? std::string("config.json") : path.substr(0, slash + 1) + "config.json";
}

bool read_file(const std::string& path, std::string& out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[65536];
  size_t n;
  while ((n = fread(buf, 1, sizeof(buf), f)) > 0) out.append(buf, n);
  bool ok = !ferror(f);
  fclose(f);
  return ok;
}

}  // namespace

Checkpoint::~Checkpoint() {
  if (map_) munmap(map_, len_);
}

int Checkpoint::open(const std::string& path, std::string& err) {
  int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) {
    err = "cannot open " + path + ": " + strerror(errno);
    return QE_ERR_IO;
  }
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    ::close(fd);
    err = "cannot stat " + path;
    return QE_ERR_IO;
  }
  len_ = size_t(sb.st_size);
  if (len_ > 0) {
    void* m = mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      ::close(fd);
      len_ = 0;
      err = "cannot mmap " + path;
      return QE_ERR_IO;
    }
    map_ = m;
  }
  ::close(fd);
  const uint8_t* b = static_cast<const uint8_t*>(map_);
  // cpu_inference.rs:62-64
  if (len_ < 8) {
    err = "file is shorter than the 8-byte header length";
    return QE_ERR_FORMAT;
  }
  uint64_t hl = 0;
  for (int i = 7; i >= 0; i--) hl = (hl << 8) | b[i];
  if (hl > len_ - 8) {
    err = "header length " + std::to_string(hl) + " exceeds the file size";
    return QE_ERR_FORMAT;
  }
  Json root;
  JsonParser jp(reinterpret_cast<const char*>(b + 8), size_t(hl));
  if (!jp.parse(root) || root.kind != Json::Obj) {
    err = "safetensors header is not a JSON object";
    return QE_ERR_FORMAT;
  }
  // cpu_inference.rs:67-73
  for (size_t i = 0; i < root.items.size(); i++) {
    if (root.keys[i] == "__metadata__") continue;
    const Json& tv = root.items[i];
    const Json* dt = tv.get("dtype");
    const Json* sh = tv.get("shape");
    const Json* of = tv.get("data_offsets");
    bool bad = !dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !of || of->kind != Json::Arr ||
               of->items.size() != 2;
    if (!bad) {
      for (auto& d : sh->items) bad |= !fits_i32(d);
      for (auto& d : of->items) bad |= !fits_i32(d);
    }
    if (bad) {
      err = "tensor " + root.keys[i] + ": malformed header entry";
      return QE_ERR_FORMAT;
    }
    TensorInfo t;
    t.name = root.keys[i];
    t.dtype = dt->str;
    for (auto& d : sh->items) t.shape.push_back(d.i64);
    t.off0 = of->items[0].i64;
    t.off1 = of->items[1].i64;
    auto it = index_.find(t.name);
    if (it != index_.end()) {
      tensors_[it->second] = std::move(t);
    } else {
      index_[t.name] = tensors_.size();
      tensors_.push_back(std::move(t));
    }
  }
  // cpu_inference.rs:74-76
  data_ = b + 8 + hl;
  data_len_ = len_ - 8 - size_t(hl);
  if (reinterpret_cast<uintptr_t>(data_) % 2 != 0) {
    err = "safetensors data section is not 2-byte aligned";
    return QE_ERR_FORMAT;
  }
  // every entry's byte range must lie in the data section, also for tensors the engine never
  // loads: the byte formula (bench.rs:106-116) sums off1 - off0 over all of them
  for (const auto& t : tensors_) {
    if (t.off0 < 0 || t.off1 < t.off0 || uint64_t(t.off1) > data_len_) {
      err = "tensor " + t.name + ": data_offsets [" + std::to_string(t.off0) + ", " + std::to_string(t.off1) +
            ") are not a range inside the " + std::to_string(data_len_) + "-byte data section";
      return QE_ERR_FORMAT;
    }
  }
  // cpu_inference.rs:80-81
  std::string cpath = sibling_config(path), text;
  if (!read_file(cpath, text)) {
    err = "cannot read " + cpath;
    return QE_ERR_IO;
  }
  Json cj;
  JsonParser cp(text.data(), text.size());
  if (!cp.parse(cj) || cj.kind != Json::Obj) {
    err = cpath + " is not a JSON object";
    return QE_ERR_FORMAT;
  }
  uint64_t eos = 0;
  bool ok = json_u64(cj, "hidden_size", cfg_.hidden_size) && json_u64(cj, "intermediate_size", cfg_.intermediate_size) &&
            json_u64(cj, "num_hidden_layers", cfg_.num_hidden_layers) &&
            json_u64(cj, "num_attention_heads", cfg_.num_attention_heads) &&
            json_u64(cj, "num_key_value_heads", cfg_.num_key_value_heads) && json_u64(cj, "head_dim", cfg_.head_dim) &&
            json_u64(cj, "vocab_size", cfg_.vocab_size) && json_f32(cj, "rms_norm_eps", cfg_.rms_norm_eps) &&
            json_f32(cj, "rope_theta", cfg_.rope_theta) && json_u64(cj, "eos_token_id", eos) && eos <= 0xFFFFFFFFull;
  if (!ok) {
    err = cpath + ": a required field is missing or has the wrong type";
    return QE_ERR_FORMAT;
  }
  cfg_.eos_token_id = uint32_t(eos);
  return QE_OK;
}

const uint16_t* Checkpoint::bf16(const std::string& name, uint64_t numel, std::string& err) const {
  auto it = index_.find(name);
  if (it == index_.end()) {
    err = "missing tensor " + name;
    return nullptr;
  }
  const TensorInfo& t = tensors_[it->second];
  if (t.dtype != "BF16") {
    err = name + ": only BF16 is supported, got " + t.dtype;
    return nullptr;
  }
  uint64_t n = 1;
  bool wrapped = false;
  for (int64_t d : t.shape) wrapped |= __builtin_mul_overflow(n, uint64_t(d < 0 ? 0 : d), &n);
  if (wrapped) {
    err = name + ": the shape's element count overflows 64 bits";
    return nullptr;
  }
  if (t.off0 < 0 || t.off1 < t.off0 || uint64_t(t.off1 - t.off0) / 2 != n || n != numel) {
    err = name + ": expected " + std::to_string(numel) + " elements";
    return nullptr;
  }
  if (uint64_t(t.off1) > data_len_) {
    err = name + ": data offsets run past the end of the file";
    return nullptr;
  }
  // the reference views the bytes in place as u16 (cpu_inference.rs:95), which needs an even
  // offset into the (2-byte aligned) data section
  if (t.off0 % 2) {
    err = name + ": data offset " + std::to_string(t.off0) + " is not 2-byte aligned";
    return nullptr;
  }
  return reinterpret_cast<const uint16_t*>(data_ + t.off0);
}

uint64_t Checkpoint::weight_bytes_per_token() const {
  uint64_t bytes = 0;
  for (const auto& t : tensors_)
    if (t.name != "model.embed_tokens.weight") bytes += uint64_t(t.off1 - t.off0);
  return bytes + cfg_.hidden_size * 2;
}

std::string layer_tensor(uint64_t l, const char* suffix) {
  return "model.layers." + std::to_string(l) + "." + suffix;
}

// ---------------------------------------------------------------------------------------------
// Seeded random-init checkpoint.
//   element stream of tensor t: key_t = mix(seed ^ mix(t + G)), u_i = mix(key_t + (i + 1) * G)
//   pairs (2j, 2j+1) from Box-Muller on (u_2j, u_2j+1); w = bf16_rne(float(0.02 * z)).
// mix() is the splitmix64 finalizer, G = 0x9E3779B97F4A7C15.
// ---------------------------------------------------------------------------------------------
namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return uint16_t((u >> 16) | 0x40);  // quiet NaN
  uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);
  return uint16_t(r >> 16);
}

struct Spec {
  std::string name;
  std::vector<uint64_t> shape;
  int kind;  // 0 random matrix, 1 norm gain (1.0), 2 copy of tensor 0 (tied lm_head)
  uint64_t numel() const {
    uint64_t n = 1;
    for (auto d : shape) n *= d;
    return n;
  }
};

// Box-Muller in f32 (the result is rounded to bf16 anyway): u1 in (0, 1], u2 in [0, 1) from the
// top 24 bits of two counter hashes; z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), r = sqrt(-2 ln u1).
void fill_random(uint16_t* dst, uint64_t numel, uint64_t key) {
  const float two_pi = 6.28318530717958647692f;
  for (uint64_t j = 0; 2 * j < numel; j++) {
    uint64_t a = mix64(key + (2 * j + 1) * kGolden);
    uint64_t b = mix64(key + (2 * j + 2) * kGolden);
    float u1 = float((a >> 40) + 1) * 0x1.0p-24f;
    float u2 = float(b >> 40) * 0x1.0p-24f;
    float r = 0.02f * sqrtf(-2.0f * logf(u1));
    float sn, cs;
    sincosf(two_pi * u2, &sn, &cs);
    dst[2 * j] = f32_to_bf16_rne(r * cs);
    if (2 * j + 1 < numel) dst[2 * j + 1] = f32_to_bf16_rne(r * sn);
  }
}

// shortest decimal that reads back (via f64, then `as f32`) to exactly f
std::string float_json(float f) {
  char buf[64];
  if (std::isfinite(f) && std::fabs(f) < 1e15f && std::floor(f) == f) {
    snprintf(buf, sizeof(buf), "%.1f", double(f));
    return buf;
  }
  for (int p = 1; p <= 9; p++) {
    snprintf(buf, sizeof(buf), "%.*g", p, double(f));
    if (float(strtod(buf, nullptr)) == f) break;
  }
  std::string s(buf);
  if (s.find_first_of(".eE") == std::string::npos && s.find("inf") == std::string::npos && s.find("nan") == std::string::npos)
    s += ".0";
  return s;
}

}  // namespace

void random_prompt(uint64_t seed, uint64_t n, uint32_t vocab, uint32_t* out) {
  uint64_t key = mix64(seed ^ 0x70726F6D70744944ull);
  for (uint64_t i = 0; i < n; i++) {
    uint64_t r = mix64(key + (i + 1) * kGolden);
    out[i] = uint32_t(((r >> 32) * uint64_t(vocab)) >> 32);
  }
}

int write_random_checkpoint(const std::string& dir, uint64_t seed, const qe_config& c, std::string& err) {
  const uint64_t H = c.hidden_size, I = c.intermediate_size, L = c.num_hidden_layers;
  const uint64_t QD = c.num_attention_heads * c.head_dim, KD = c.num_key_value_heads * c.head_dim;
  const uint64_t V = c.vocab_size, D = c.head_dim;
  if (!H || !I || !L || !QD || !KD || !V || !D) {
    err = "config has a zero dimension";
    return QE_ERR_ARG;
  }
  std::vector<Spec> specs;
  specs.push_back({"model.embed_tokens.weight", {V, H}, 0});
  for (uint64_t l = 0; l < L; l++) {
    specs.push_back({layer_tensor(l, "input_layernorm.weight"), {H}, 1});
    specs.push_back({layer_tensor(l, "self_attn.q_proj.weight"), {QD, H}, 0});
    specs.push_back({layer_tensor(l, "self_attn.k_proj.weight"), {KD, H}, 0});
    specs.push_back({layer_tensor(l, "self_attn.v_proj.weight"), {KD, H}, 0});
    specs.push_back({layer_tensor(l, "self_attn.q_norm.weight"), {D}, 1});
    specs.push_back({layer_tensor(l, "self_attn.k_norm.weight"), {D}, 1});
    specs.push_back({layer_tensor(l, "self_attn.o_proj.weight"), {H, QD}, 0});
    specs.push_back({layer_tensor(l, "post_attention_layernorm.weight"), {H}, 1});
    specs.push_back({layer_tensor(l, "mlp.gate_proj.weight"), {I, H}, 0});
    specs.push_back({layer_tensor(l, "mlp.up_proj.weight"), {I, H}, 0});
    specs.push_back({layer_tensor(l, "mlp.down_proj.weight"), {H, I}, 0});
  }
  specs.push_back({"model.norm.weight", {H}, 1});
  specs.push_back({"lm_head.weight", {V, H}, 2});

  // header JSON, padded with spaces so the data section starts 8-byte aligned
  std::vector<uint64_t> offs(specs.size() + 1, 0);
  std::string hdr = "{\"__metadata__\":{\"format\":\"pt\"}";
  for (size_t t = 0; t < specs.size(); t++) {
    offs[t + 1] = offs[t] + specs[t].numel() * 2;
    hdr += ",\"" + specs[t].name + "\":{\"dtype\":\"BF16\",\"shape\":[";
    for (size_t k = 0; k < specs[t].shape.size(); k++) hdr += (k ? "," : "") + std::to_string(specs[t].shape[k]);
    hdr += "],\"data_offsets\":[" + std::to_string(offs[t]) + "," + std::to_string(offs[t + 1]) + "]}";
  }
  hdr += "}";
  while ((8 + hdr.size()) % 8) hdr += ' ';
  if (offs.back() > 0x7FFFFFFFull) {
    err = "checkpoint data exceeds the i32 offsets the reference loader reads";
    return QE_ERR_ARG;
  }
  const uint64_t total = 8 + hdr.size() + offs.back();

  std::string path = dir + "/model.safetensors";
  int fd = ::open(path.c_str(), O_RDWR | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) {
    err = "cannot create " + path + ": " + strerror(errno);
    return QE_ERR_IO;
  }
  if (ftruncate(fd, off_t(total)) != 0) {
    ::close(fd);
    err = "cannot size " + path;
    return QE_ERR_IO;
  }
  const uint64_t hl = hdr.size();
  std::string head(8, '\0');
  for (int i = 0; i < 8; i++) head[i] = char(uint8_t(hl >> (8 * i)));
  head += hdr;
  auto pwrite_all = [&](const void* buf, size_t n, uint64_t at) -> bool {
    const char* p = static_cast<const char*>(buf);
    while (n) {
      ssize_t w = pwrite(fd, p, n, off_t(at));
      if (w <= 0) return false;
      p += w;
      n -= size_t(w);
      at += uint64_t(w);
    }
    return true;
  };
  bool ok = pwrite_all(head.data(), head.size(), 0);
  const uint64_t data0 = 8 + hl;

  // work items: (tensor, element range) in 4M-element blocks; each thread fills a private
  // buffer and writes it at its file offset (the tied lm_head gets the embedding blocks too)
  struct Item { size_t t; uint64_t begin, end; };
  std::vector<Item> items;
  const uint64_t block = uint64_t(1) << 22;  // even, so Box-Muller pairs never straddle items
  for (size_t t = 0; t < specs.size(); t++) {
    if (specs[t].kind == 2) continue;
    uint64_t n = specs[t].numel();
    for (uint64_t b = 0; b < n; b += block) items.push_back({t, b, std::min(n, b + block)});
  }
  const size_t tied = specs.size() - 1;
  std::atomic<size_t> next{0};
  std::atomic<bool> write_ok{true};
  auto worker = [&]() {
    std::vector<uint16_t> buf(block);
    while (true) {
      size_t k = next.fetch_add(1);
      if (k >= items.size()) break;
      const Item& it = items[k];
      uint64_t cnt = it.end - it.begin;
      if (specs[it.t].kind == 1) {
        std::fill(buf.begin(), buf.begin() + cnt, uint16_t(0x3F80));
      } else {
        uint64_t key = mix64(seed ^ mix64(uint64_t(it.t) + kGolden));
        // element i of the tensor uses counters 2*(i/2)+1, 2*(i/2)+2: shift the key by begin
        fill_random(buf.data(), cnt, key + it.begin * kGolden);
      }
      bool w = pwrite_all(buf.data(), cnt * 2, data0 + offs[it.t] + it.begin * 2);
      if (it.t == 0) w = w && pwrite_all(buf.data(), cnt * 2, data0 + offs[tied] + it.begin * 2);
      if (!w) write_ok = false;
    }
  };
  unsigned nt = std::max(1u, std::min(64u, std::thread::hardware_concurrency()));
  std::vector<std::thread> th;
  for (unsigned i = 0; i < nt; i++) th.emplace_back(worker);
  for (auto& x : th) x.join();
  ok = ok && write_ok && ::close(fd) == 0;
  if (!ok) {
    err = "cannot write " + path;
    return QE_ERR_IO;
  }

  std::string cfg = "{\n  \"architectures\": [\"Qwen3ForCausalLM\"],\n  \"model_type\": \"qwen3\",\n";
  char buf[1024];
  snprintf(buf, sizeof(buf),
           "  \"hidden_size\": %llu,\n  \"intermediate_size\": %llu,\n  \"num_hidden_layers\": %llu,\n"
           "  \"num_attention_heads\": %llu,\n  \"num_key_value_heads\": %llu,\n  \"head_dim\": %llu,\n"
           "  \"vocab_size\": %llu,\n  \"rms_norm_eps\": %s,\n  \"rope_theta\": %s,\n  \"eos_token_id\": %u,\n"
           "  \"tie_word_embeddings\": true,\n  \"hidden_act\": \"silu\",\n  \"torch_dtype\": \"bfloat16\",\n"
           "  \"attention_bias\": false,\n  \"max_position_embeddings\": 40960,\n  \"init_seed\": %llu\n}\n",
           (unsigned long long)H, (unsigned long long)I, (unsigned long long)L,
           (unsigned long long)c.num_attention_heads, (unsigned long long)c.num_key_value_heads,
           (unsigned long long)D, (unsigned long long)V, float_json(c.rms_norm_eps).c_str(), float_json(c.rope_theta).c_str(),
           c.eos_token_id, (unsigned long long)seed);
  cfg += buf;
  std::string cpath = dir + "/config.json";
  FILE* f = fopen(cpath.c_str(), "wb");
  if (!f || fwrite(cfg.data(), 1, cfg.size(), f) != cfg.size()) {
    if (f) fclose(f);
    err = "cannot write " + cpath;
    return QE_ERR_IO;
  }
  fclose(f);
  return QE_OK;
}

}  // namespace qe
