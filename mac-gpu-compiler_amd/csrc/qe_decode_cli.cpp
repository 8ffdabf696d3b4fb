// qe_decode: command-line greedy decode over the C ABI of include/qe.h, the shape of the
// reference's bench loop (metal_infrence_engine/src/bin/bench.rs:165-191): prompt prefill, then
// greedy decode steps, tokens printed at the end. It links only libqe.so and the HIP runtime, so
// tools that cannot attach to a Python process (counter collection) can run the real step.
//
//   qe_decode [--dir DIR] [--seed S] [--prompt-len P] [--steps K] [--kv f32|bf16] [--copy-mib N]
//
// DIR (default /tmp/qe_bench/qwen3_0_6b_seed<S>) gets a seeded random-init checkpoint of the
// Qwen3-0.6B architecture if it has none. --copy-mib N first runs one N MiB device-to-device
// copy, a kernel of known traffic (N MiB read, N MiB written) for scaling memory counters.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <sys/stat.h>
#include <vector>

#include "../../include/qe.h"

namespace {

int die(const char* what, int rc) {
  std::fprintf(stderr, "qe_decode: %s failed (%d): %s\n", what, rc, qe_last_error());
  return 1;
}

void on_token(void* user, uint32_t tok) { static_cast<std::vector<uint32_t>*>(user)->push_back(tok); }

// mkdir -p
bool make_dirs(const std::string& path) {
  for (size_t i = 1; i <= path.size(); i++) {
    if (i == path.size() || path[i] == '/') {
      const std::string part = path.substr(0, i);
      if (mkdir(part.c_str(), 0755) != 0 && errno != EEXIST) return false;
    }
  }
  return true;
}

}  // namespace

int main(int argc, char** argv) {
  uint64_t seed = 20260101, prompt_len = 130, steps = 128, copy_mib = 0;
  int kv_dtype = QE_KV_F32;
  std::string dir;
  for (int i = 1; i < argc; i++) {
    const char* a = argv[i];
    const char* v = i + 1 < argc ? argv[i + 1] : nullptr;
    if (!strcmp(a, "--dir") && v) { dir = v; i++; }
    else if (!strcmp(a, "--seed") && v) { seed = strtoull(v, nullptr, 10); i++; }
    else if (!strcmp(a, "--prompt-len") && v) { prompt_len = strtoull(v, nullptr, 10); i++; }
    else if (!strcmp(a, "--steps") && v) { steps = strtoull(v, nullptr, 10); i++; }
    else if (!strcmp(a, "--copy-mib") && v) { copy_mib = strtoull(v, nullptr, 10); i++; }
    else if (!strcmp(a, "--kv") && v) { kv_dtype = !strcmp(v, "bf16") ? QE_KV_BF16 : QE_KV_F32; i++; }
    else {
      std::fprintf(stderr, "usage: %s [--dir DIR] [--seed S] [--prompt-len P] [--steps K] [--kv f32|bf16] [--copy-mib N]\n", argv[0]);
      return 2;
    }
  }
  if (prompt_len == 0) prompt_len = 1;
  if (dir.empty()) dir = "/tmp/qe_bench/qwen3_0_6b_seed" + std::to_string(seed);

  if (copy_mib) {
    const size_t bytes = size_t(copy_mib) << 20;
    void *src = nullptr, *dst = nullptr;
    if (hipMalloc(&src, bytes) != hipSuccess || hipMalloc(&dst, bytes) != hipSuccess) {
      std::fprintf(stderr, "qe_decode: hipMalloc of %llu MiB failed\n", (unsigned long long)copy_mib);
      return 1;
    }
    if (hipMemset(src, 0, bytes) != hipSuccess || hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
      std::fprintf(stderr, "qe_decode: calibration copy failed\n");
      return 1;
    }
    (void)hipFree(src);
    (void)hipFree(dst);
    std::printf("calibration copy: %llu MiB device to device\n", (unsigned long long)copy_mib);
  }

  const std::string ckpt = dir + "/model.safetensors";
  struct stat sb;
  if (stat(ckpt.c_str(), &sb) != 0) {
    if (!make_dirs(dir)) {
      std::fprintf(stderr, "qe_decode: cannot create %s\n", dir.c_str());
      return 1;
    }
    const qe_config cfg = {1024, 3072, 28, 16, 8, 128, 151936, 1e-6f, 1e6f, 151645};
    int rc = qe_write_random_checkpoint(dir.c_str(), seed, &cfg);
    if (rc) return die("qe_write_random_checkpoint", rc);
  }
  qe_model* m = nullptr;
  int rc = qe_model_load(ckpt.c_str(), &m);
  if (rc) return die("qe_model_load", rc);
  qe_config cfg;
  qe_model_config(m, &cfg);
  qe_kv* kv = nullptr;
  if ((rc = qe_kv_new(m, prompt_len + steps + 1, kv_dtype, &kv))) return die("qe_kv_new", rc);

  std::vector<uint32_t> prompt(prompt_len);
  qe_random_prompt(7, prompt_len, uint32_t(cfg.vocab_size), prompt.data());
  std::vector<float> logits(cfg.vocab_size);
  if ((rc = qe_prefill(m, prompt.data(), prompt_len, 0, kv, logits.data()))) return die("qe_prefill", rc);
  uint32_t first = 0;  // first maximum wins (main.rs:37-42)
  for (uint32_t i = 1; i < uint32_t(cfg.vocab_size); i++)
    if (logits[i] > logits[first]) first = i;

  std::vector<uint32_t> toks;
  const auto t0 = std::chrono::steady_clock::now();
  if ((rc = qe_decode(m, first, prompt_len, steps, kv, on_token, &toks, nullptr))) return die("qe_decode", rc);
  const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  std::printf("decode: %llu steps at positions %llu..%llu in %.3f ms (%.1f tok/s)\n", (unsigned long long)steps,
              (unsigned long long)prompt_len, (unsigned long long)(prompt_len + steps - 1), s * 1e3,
              steps ? double(steps) / s : 0.0);
  std::printf("tokens: %u", first);
  for (uint32_t t : toks) std::printf(" %u", t);
  std::printf("\n");
  qe_kv_free(kv);
  qe_model_free(m);
  return 0;
}
