// Host-only robustness check of the engine's safetensors / config.json reader
// (csrc/checkpoint.cpp), built with ASan and UBSan by tests/test_parser_sanitizers.py.
// Writes a small valid checkpoint, then opens ITERS mutated copies of its header and of its
// config.json: truncations, garbled bytes, bogus header lengths, structural characters, long
// digit runs. Every accepted file has each of its tensor views read at both ends.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <random>
#include <string>
#include <vector>

#include "../../mac-gpu-compiler_amd/csrc/checkpoint.h"

static std::string slurp(const std::string& p) {
  std::ifstream f(p, std::ios::binary);
  return std::string((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

static void spit(const std::string& p, const std::string& s) {
  std::ofstream o(p, std::ios::binary | std::ios::trunc);
  o.write(s.data(), std::streamsize(s.size()));
}

static int try_open(const std::string& path) {
  qe::Checkpoint ck;
  std::string e;
  if (ck.open(path, e) != QE_OK) return 0;
  for (const auto& t : ck.tensors()) {
    uint64_t numel = 1;
    for (auto d : t.shape) numel *= uint64_t(d < 0 ? 0 : d);
    const uint16_t* p = ck.bf16(t.name, numel, e);
    if (p && numel) {
      volatile uint16_t a = p[0], b = p[numel - 1];
      (void)a;
      (void)b;
    }
  }
  (void)ck.weight_bytes_per_token();
  return 1;
}

int main(int argc, char** argv) {
  if (argc < 3) return 2;
  const std::string dir = argv[1];
  const int iters = atoi(argv[2]);
  const qe_config cfg{256, 512, 2, 4, 2, 128, 1000, 1e-6f, 1e6f, 999};
  std::string err;
  if (qe::write_random_checkpoint(dir, 1234, cfg, err)) {
    printf("write failed: %s\n", err.c_str());
    return 1;
  }
  const std::string st = dir + "/model.safetensors", cj = dir + "/config.json";
  const std::string orig = slurp(st), ocfg = slurp(cj);
  uint64_t hl;
  memcpy(&hl, orig.data(), 8);
  std::mt19937_64 rng(7);
  int ok = 0;
  for (int it = 0; it < iters; it++) {
    std::string s = orig;
    switch (it % 6) {
      case 0: s.resize(rng() % (8 + hl + 64)); break;
      case 1: for (int k = 0; k < 8; k++) s[8 + rng() % hl] = char(rng()); break;
      case 2: { const uint64_t v = rng(); memcpy(&s[0], &v, 8); break; }
      case 3: { const uint64_t v = hl + rng() % 64 - 32; memcpy(&s[0], &v, 8); break; }
      case 4: for (int k = 0; k < 4; k++) { const size_t i = 8 + rng() % hl; if (s[i] >= '0' && s[i] <= '9') s[i] = char('0' + rng() % 10); } break;
      default: s[8 + rng() % hl] = "{}[]\":,"[rng() % 7]; break;
    }
    spit(st, s);
    ok += try_open(st);
  }
  spit(st, orig);
  for (int it = 0; it < iters; it++) {
    std::string c = ocfg;
    switch (it % 4) {
      case 0: c.resize(rng() % c.size()); break;
      case 1: for (int k = 0; k < 3; k++) c[rng() % c.size()] = char(rng()); break;
      case 2: c[rng() % c.size()] = "{}[]\":,-0123456789eE."[rng() % 21]; break;
      default: c.insert(rng() % c.size(), std::string(rng() % 40, "9-e"[rng() % 3])); break;
    }
    spit(cj, c);
    ok += try_open(st);
  }
  spit(cj, ocfg);
  if (!try_open(st)) return 3;  // the restored file still opens
  printf("accepted %d of %d mutated files\n", ok, 2 * iters);
  return 0;
}
