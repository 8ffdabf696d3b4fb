// qe_op_attention_static: the isolated decode attention of qe_op_attention with its partial-sum
// work area in device memory the library owns from load time, so that a caller that cannot
// allocate (code under HIP graph capture, serving loops that forbid hipMalloc) can run it with
// only its inputs and outputs. No reference counterpart.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <mutex>

#include "../../include/qe.h"
#include "kernels.h"
#include "status.h"

namespace {

// Partials of one call: kStaticAttnRows rows of kPartStride floats, one row per (q head, position
// run), i.e. calls with n_heads x runs <= 2048 (16 q heads at the op's largest 128 runs). 1 MiB
// per GPU, held until the process ends. Every call on a GPU uses that GPU's one array: each call
// writes every row it reads (runs past the last position write empty partials), so nothing needs
// clearing between calls, but calls that overlap on one GPU (two streams, two threads) race.
constexpr uint32_t kStaticAttnRows = 2048;
static __device__ __align__(256) float scratch[size_t(kStaticAttnRows) * qe::kPartStride];

// `scratch` names the array in host code but is not its device address: kernels get the address
// hipGetSymbolAddress returns on each device, looked up once per device with it current, on the
// first call there (which therefore must not be under stream capture; later calls launch only).
constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_ptr[kMaxDevices] = {};

int scratch_on_current_device(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return qe::set_error(QE_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return qe::set_error(QE_ERR_UNSUPPORTED, "device index %d above %d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return qe::set_error(QE_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    g_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_ptr[dev];
  return QE_OK;
}

}  // namespace

extern "C" int qe_op_attention_static(const float* q, const float* k, const float* v, float* out, uint64_t n_pos,
                                      uint64_t kv_stride, uint64_t n_heads, uint64_t n_kv_heads, uint32_t n_splits,
                                      void* stream) {
  if (!q || !k || !v || !out) return qe::set_error(QE_ERR_ARG, "null argument");
  if (n_pos == 0 || n_pos > kv_stride || kv_stride > 0xFFFFFFFFull)
    return qe::set_error(QE_ERR_ARG, "need 0 < n_pos <= kv_stride");
  if (!n_kv_heads || n_heads % n_kv_heads) return qe::set_error(QE_ERR_ARG, "n_heads must be a multiple of n_kv_heads");
  const uint64_t G = n_heads / n_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return qe::set_error(QE_ERR_UNSUPPORTED, "q heads per KV head must be 1, 2, 4 or 8");
  if (n_splits > uint32_t(qe::kAttnMaxSplits)) return qe::set_error(QE_ERR_ARG, "n_splits above %d", qe::kAttnMaxSplits);
  // the run count qe_op_attention picks: n_splits, or runs of 64 positions, at most kAttnMaxSplits
  uint64_t splits = n_splits ? n_splits : (n_pos + 63) / 64;
  splits = std::min<uint64_t>(std::max<uint64_t>(splits, 1), qe::kAttnMaxSplits);
  if (n_heads * splits > kStaticAttnRows)
    return qe::set_error(QE_ERR_ARG, "n_heads x runs = %llu x %llu is above the %u partial rows of the static work area",
                         (unsigned long long)n_heads, (unsigned long long)splits, kStaticAttnRows);
  float* work = nullptr;
  if (int rc = scratch_on_current_device(&work)) return rc;
  qe::AttnParams a{};
  a.qkv = q;
  a.k_cache = const_cast<float*>(k);
  a.v_cache = const_cast<float*>(v);
  a.partial = work;
  a.n_heads = uint32_t(n_heads);
  a.n_kv = uint32_t(n_kv_heads);
  a.max_seq = uint32_t(kv_stride);
  a.scale = 1.0f / sqrtf(float(qe::kHeadDim));
  a.n_pos_fixed = uint32_t(n_pos);
  const hipError_t e = qe::launch_attention_op(a, uint32_t(splits), out, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return qe::set_error(QE_ERR_HIP, "attention launch failed: %s", hipGetErrorString(e));
  return QE_OK;
}
