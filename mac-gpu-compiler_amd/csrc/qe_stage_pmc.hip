// qe_stage_pmc: launches each decode-step kernel of the Qwen3-0.6B shapes on synthetic inputs,
// eight times per stage with the weights rotating over four copies (past the 4 MB L2), after a
// 1 GiB device copy of known traffic. Meant to run under `rocprofv3 --pmc FETCH_SIZE` and
// `--pmc WRITE_SIZE`: the counters per dispatch, scaled by the copy's, give each stage's HBM
// bytes per launch. Stage order and kernels are those of the engine's decode step, including
// the attention launch's L2 prefetch of the layer's gate/up and down weights.
//
//   qe_stage_pmc [--pos P] [--no-prefetch]   (attention attends positions 0..P, default 193)
//   qe_stage_pmc --fused [--pos P]   the two-launch layer instead: 8 x (attention block, MLP
//                         block) in step order with the engine's attention shape for P + 1
//                         positions (runs of 64 positions, 4 / 8 / 16 / 32 of them), then
//                         2 x (final reduce, lm_head, argmax); exits with status 2 if this
//                         device does not deal a launch's workgroups to its XCDs round-robin
//   qe_stage_pmc --l2-persist   no counters: times, as graphs of 64 launches, a launch whose
//                         workgroup (XCD x, slot s) reads 64 KiB of XCD x's 2 MiB share of a
//                         16 MiB chunk, for the same chunk every launch, 8 rotating chunks
//                         (128 MiB, within the MALL) and 48 (768 MiB): whether L2 keeps lines
//                         from one launch to the next
//   qe_stage_pmc --gemm   the chunked prefill's GEMM instead (launch_gemm, no norm, plain store),
//                         3 launches at each of M x N x K = 2048 x 4096 x 1024 (q|k|v of a
//                         2048-token chunk: k_gemm_tile), 512 x 6144 x 1024 and 512 x 4096 x 1024
//                         (gate|up and q|k|v of a 512-token chunk: k_gemm_rows8), for the
//                         matrix-core counters (SQ_INSTS_MFMA, SQ_VALU_MFMA_BUSY_CYCLES, ...);
//                         --reps R launches per shape instead of 3, --random fills A and W with
//                         hashed values in [-1, 1) and [-1/64, 1/64) instead of constants (the
//                         same work; what changes is how many bits the operands toggle)
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "batch.h"
#include "kernels.h"
#include "l2_prefetch.h"

namespace {

#define CK(x)                                                                                  \
  do {                                                                                         \
    hipError_t e_ = (x);                                                                       \
    if (e_ != hipSuccess) {                                                                    \
      std::fprintf(stderr, "qe_stage_pmc: %s failed: %s\n", #x, hipGetErrorString(e_));        \
      std::exit(1);                                                                            \
    }                                                                                          \
  } while (0)

__global__ void k_copy(const float4* __restrict__ s, float4* __restrict__ d, size_t n) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256) d[i] = s[i];
}

// every workgroup reads all of p[0..n): each XCD's L2 misses on the buffer once per launch, unless
// the lines are still in it from an earlier launch (the sum only feeds a never-taken store)
__global__ void k_reread(const float4* __restrict__ p, size_t n, float* sink) {
  float a = 0.f;
  for (size_t i = threadIdx.x; i < n; i += 256) {
    const float4 v = p[i];
    a += v.x + v.y + v.z + v.w;
  }
  if (a == -1.25f) sink[threadIdx.x] = a;
}

// bf16 ~ small values, so sums stay finite
__global__ void k_fill_bf16(uint16_t* p, size_t n, uint32_t seed) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256) {
    uint32_t h = uint32_t(i) * 2654435761u ^ seed;
    h ^= h >> 15;
    p[i] = uint16_t(0x3C00u | (h & 0x7Fu));  // 2^-7 .. ~2^-6, positive
  }
}

__global__ void k_fill_f32(float* p, size_t n, float v) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256) p[i] = v;
}

// p[i] = scale x (a hash of i mapped to [-1, 1)); bf16: the upper halves of such floats
__device__ __forceinline__ float hash_unit(uint32_t i) {
  uint32_t h = i * 2654435761u;
  h ^= h >> 16;
  h *= 2246822519u;
  h ^= h >> 13;
  return float(h >> 8) * (2.0f / 16777216.0f) - 1.0f;
}
__global__ void k_fill_hash_f32(float* p, size_t n, float scale) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256)
    p[i] = scale * hash_unit(uint32_t(i));
}
__global__ void k_fill_hash_bf16(uint16_t* p, size_t n, float scale) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256)
    p[i] = uint16_t(__float_as_uint(scale * hash_unit(uint32_t(i) ^ 0x9E3779B9u)) >> 16);
}

// workgroup (XCD x, slot blockIdx / 8) reads 64 KiB of XCD x's 2 MiB share of 16 MiB chunk `chunk`
__global__ __launch_bounds__(256) void k_read_xcd_share(const float4* __restrict__ base, uint32_t chunk, float* sink) {
  const uint32_t x = qe::xcc_id() & 7, slot = blockIdx.x >> 3;
  const float4* p = base + (size_t(chunk) * (16u << 20) + size_t(x) * (2u << 20) + size_t(slot) * (64u << 10)) / 16;
  float a = 0.f;
#pragma unroll 4
  for (uint32_t i = threadIdx.x; i < (64u << 10) / 16; i += 256) {
    const float4 v = p[i];
    a += v.x + v.y + v.z + v.w;
  }
  if (a == -1.25f) sink[threadIdx.x] = a;
}

template <typename T>
T* dalloc(size_t n) {
  T* p = nullptr;
  CK(hipMalloc(&p, n * sizeof(T)));
  return p;
}

}  // namespace

int main(int argc, char** argv) {
  uint32_t pos = 193;
  bool prefetch = true, gemm = false, random = false, fused = false, persist = false, pf_idle = false;
  int reps = 3;
  for (int i = 1; i < argc; i++) {
    if (!strcmp(argv[i], "--pos") && i + 1 < argc) pos = uint32_t(strtoul(argv[++i], nullptr, 10));
    else if (!strcmp(argv[i], "--no-prefetch")) prefetch = false;
    else if (!strcmp(argv[i], "--gemm")) gemm = true;
    else if (!strcmp(argv[i], "--fused")) fused = true;
    else if (!strcmp(argv[i], "--l2-persist")) persist = true;
    else if (!strcmp(argv[i], "--pf-idle")) pf_idle = true;
    else if (!strcmp(argv[i], "--random")) random = true;
    else if (!strcmp(argv[i], "--reps") && i + 1 < argc) reps = std::max(1, atoi(argv[++i]));
  }
  if (persist) {
    CK(hipSetDevice(0));
    hipStream_t ps;
    CK(hipStreamCreate(&ps));
    const uint32_t NCH = 48;  // 16 MiB chunks
    float4* buf = dalloc<float4>(size_t(NCH) * (16u << 20) / 16);
    float* sink = dalloc<float>(256);
    k_fill_f32<<<8192, 256, 0, ps>>>(reinterpret_cast<float*>(buf), size_t(NCH) * (16u << 20) / 4, 1.f);
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    const uint32_t rot[3] = {1, 8, NCH};
    const char* what[3] = {"the same 16 MiB chunk every launch", "8 chunks in turn (128 MiB)", "48 chunks in turn (768 MiB)"};
    for (int v = 0; v < 3; v++) {
      hipGraph_t g;
      hipGraphExec_t ge;
      CK(hipStreamBeginCapture(ps, hipStreamCaptureModeGlobal));
      for (uint32_t i = 0; i < 64; i++) hipLaunchKernelGGL(k_read_xcd_share, dim3(256), dim3(256), 0, ps, buf, i % rot[v], sink);
      CK(hipStreamEndCapture(ps, &g));
      CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
      CK(hipGraphLaunch(ge, ps));
      CK(hipStreamSynchronize(ps));
      float best = 1e30f;
      for (int t = 0; t < 5; t++) {
        CK(hipEventRecord(e0, ps));
        CK(hipGraphLaunch(ge, ps));
        CK(hipEventRecord(e1, ps));
        CK(hipEventSynchronize(e1));
        float ms = 0.f;
        CK(hipEventElapsedTime(&ms, e0, e1));
        best = std::min(best, ms);
      }
      const double us = best * 1e3 / 64;
      std::printf("l2-persist: %-36s %.3f us per launch, %.0f GB/s\n", what[v], us, 16.0 * 1048576 / (us * 1e-6) / 1e9);
      CK(hipGraphExecDestroy(ge));
      CK(hipGraphDestroy(g));
    }
    return 0;
  }
  if (gemm) {
    CK(hipSetDevice(0));
    hipStream_t gs;
    CK(hipStreamCreate(&gs));
    const uint32_t shapes[3][3] = {{2048, 4096, 1024}, {512, 6144, 1024}, {512, 4096, 1024}};
    for (const auto& sh : shapes) {
      const uint32_t M = sh[0], N = sh[1], K = sh[2];
      float* A = dalloc<float>(size_t(M) * K);
      uint16_t* W = dalloc<uint16_t>(size_t(N) * K);
      float* C = dalloc<float>(size_t(M) * N);
      if (random) {
        k_fill_hash_f32<<<1024, 256, 0, gs>>>(A, size_t(M) * K, 1.0f);
        k_fill_hash_bf16<<<1024, 256, 0, gs>>>(W, size_t(N) * K, 1.0f / 64);
      } else {
        k_fill_f32<<<1024, 256, 0, gs>>>(A, size_t(M) * K, 0.5f);
        // bf16 pairs (0, 0.0078125): any finite values give the same matrix-core work
        k_fill_f32<<<1024, 256, 0, gs>>>(reinterpret_cast<float*>(W), size_t(N) * K / 2, 0.0078125f);
      }
      const qe::GemmParams g{A, K, nullptr, nullptr, W, M, N, K, C, N, 1e-6f};
      for (int r = 0; r < reps; r++) CK(qe::launch_gemm(g, false, qe::kGemmStore, gs));
      CK(hipStreamSynchronize(gs));
      CK(hipFree(A));
      CK(hipFree(W));
      CK(hipFree(C));
      std::printf("gemm %u x %u x %u: %d launches%s\n", M, N, K, reps, random ? " (hashed operands)" : "");
    }
    return 0;
  }
  const uint32_t H = 1024, I = 3072, V = 151936, NH = 16, NKV = 8, D = qe::kHeadDim, G = NH / NKV;
  const uint32_t QD = NH * D, KD = NKV * D, max_seq = 258;
  if (pos >= max_seq) pos = max_seq - 1;
  CK(hipSetDevice(0));
  hipStream_t s;
  CK(hipStreamCreate(&s));

  // 1 GiB copy: 1 GiB read, 1 GiB written
  {
    const size_t n4 = (size_t(1) << 30) / 16;
    float4* a = dalloc<float4>(n4);
    float4* b = dalloc<float4>(n4);
    k_fill_f32<<<4096, 256, 0, s>>>(reinterpret_cast<float*>(a), n4 * 4, 1.f);
    hipLaunchKernelGGL(k_copy, dim3(8192), dim3(256), 0, s, a, b, n4);
    CK(hipStreamSynchronize(s));
    // L2 persistence between dispatches: two launches that each read a 2 MiB buffer (under one
    // XCD's 4 MB L2) from all 256 workgroups; the second fetches ~nothing if L2 keeps the lines
    const size_t r4 = (size_t(2) << 20) / 16;
    for (int r = 0; r < 2; r++) hipLaunchKernelGGL(k_reread, dim3(256), dim3(256), 0, s, a, r4, reinterpret_cast<float*>(b));
    CK(hipStreamSynchronize(s));
    CK(hipFree(a));
    CK(hipFree(b));
  }

  // weights: four copies of each per-layer matrix, one lm_head
  const size_t n_qkv = size_t(QD + 2 * KD) * H, n_o = size_t(H) * QD, n_gu = size_t(2) * I * H, n_dn = size_t(H) * I;
  const size_t per_copy = n_qkv + n_o + n_gu + n_dn;
  uint16_t* W = dalloc<uint16_t>(per_copy * 4);
  uint16_t* LM = dalloc<uint16_t>(size_t(V) * H);
  uint16_t* gains = dalloc<uint16_t>(H);
  k_fill_bf16<<<8192, 256, 0, s>>>(W, per_copy * 4, 1u);
  k_fill_bf16<<<8192, 256, 0, s>>>(LM, size_t(V) * H, 2u);
  k_fill_bf16<<<4, 256, 0, s>>>(gains, H, 3u);
  // activations and attention state
  float* x = dalloc<float>(H);
  float* qkv = dalloc<float>(QD + 2 * KD);
  float* h = dalloc<float>(I);
  float* logits = dalloc<float>(V);
  const uint32_t n_cand = qe::matvec_num_blocks(V, H, qe::kLogits);
  qe::ArgCand* cand = dalloc<qe::ArgCand>(n_cand);
  float* kc = dalloc<float>(size_t(NKV) * max_seq * D);
  float* vc = dalloc<float>(size_t(NKV) * max_seq * D);
  const uint32_t splits = (max_seq + 63) / 64;
  float* part = dalloc<float>(size_t(NKV) * splits * G * qe::kPartStride);
  float* rope = dalloc<float>(size_t(max_seq) * D);
  float* rope_cur = dalloc<float>(D);
  qe::StepState* st = dalloc<qe::StepState>(1);
  uint32_t* tokens = dalloc<uint32_t>(max_seq + 2);
  uint32_t* err = dalloc<uint32_t>(1);
  k_fill_f32<<<4, 256, 0, s>>>(x, H, 0.5f);
  k_fill_f32<<<16, 256, 0, s>>>(qkv, QD + 2 * KD, 0.25f);
  k_fill_f32<<<16, 256, 0, s>>>(h, I, 0.125f);
  k_fill_f32<<<512, 256, 0, s>>>(kc, size_t(NKV) * max_seq * D, 0.01f);
  k_fill_f32<<<512, 256, 0, s>>>(vc, size_t(NKV) * max_seq * D, 0.02f);
  k_fill_f32<<<64, 256, 0, s>>>(rope, size_t(max_seq) * D, 0.5f);
  k_fill_f32<<<1, 256, 0, s>>>(rope_cur, D, 0.5f);
  const qe::StepState st_h{pos, 0u, max_seq, max_seq + 2};
  CK(hipMemcpyAsync(st, &st_h, sizeof(st_h), hipMemcpyHostToDevice, s));
  CK(hipMemsetAsync(tokens, 0, (max_seq + 2) * 4, s));
  CK(hipMemsetAsync(err, 0, 4, s));
  CK(hipStreamSynchronize(s));

  if (fused) {
    // the launches need the round-robin workgroup -> XCD placement the engine checks at load
    uint32_t* place = dalloc<uint32_t>(qe::kFusedXcds * qe::kFusedSlots);
    uint32_t* host_ids = nullptr;
    CK(hipHostMalloc(&host_ids, qe::kFusedXcds * qe::kFusedSlots * 4, hipHostMallocDefault));
    bool ok = false;
    CK(qe::fused_placement_check(place, host_ids, &ok, s));
    CK(hipHostFree(host_ids));
    if (!ok) {
      std::fprintf(stderr, "qe_stage_pmc: workgroups are not dealt to the XCDs round-robin; no fused launches\n");
      return 2;
    }
    // the engine's step shape (step_shape): runs of 32 positions up to 256 cached positions, then
    // runs of 64 (4, 8, 16 or 32 per KV head), then 32 runs of a whole number of 64-position tiles
    const uint32_t NX = qe::kFusedXcds, n = pos + 1, R = qe::kFusedMaxRuns;
    uint32_t run, fsplits;
    if (n <= 256) {
      run = 32;
      const uint32_t active = (n + 31) / 32;
      fsplits = active <= 4 ? 4 : active <= 8 ? 8 : 16;
    } else {
      run = 64 * ((n + 64 * R - 1) / (64 * R));
      const uint32_t active = (n + run - 1) / run;
      fsplits = run > 64 ? R : active <= 4 ? 4 : active <= 8 ? 8 : active <= 16 ? 16 : R;
    }
    float* res0 = dalloc<float>(H);
    float* res1 = dalloc<float>(H);
    float* part_attn = dalloc<float>(size_t(NX) * H);
    float* part_mlp = dalloc<float>(size_t(NX) * H);
    uint2* fqkv = dalloc<uint2>(qe::kFusedQkvPairs + qe::kFusedAttPairs);
    uint2* fpart = dalloc<uint2>(qe::kFusedPartPairs);
    uint2* fh = dalloc<uint2>(qe::kFusedHPairs);
    uint32_t* fsync = dalloc<uint32_t>(qe::kFusedSyncWords);
    k_fill_f32<<<4, 256, 0, s>>>(res0, H, 0.5f);
    CK(hipMemsetAsync(part_mlp, 0, size_t(NX) * H * 4, s));
    CK(hipMemsetAsync(fqkv, 0, (qe::kFusedQkvPairs + qe::kFusedAttPairs) * 8, s));
    CK(hipMemsetAsync(fpart, 0, qe::kFusedPartPairs * 8, s));
    CK(hipMemsetAsync(fh, 0, qe::kFusedHPairs * 8, s));
    CK(hipMemsetAsync(fsync, 0, qe::kFusedSyncWords * 4, s));
    CK(hipStreamSynchronize(s));
    qe::FusedLayerParams f{};
    f.rows = 1;
    f.w_in = gains; f.q_norm = gains; f.k_norm = gains; f.w_post = gains;
    f.qkv = fqkv; f.attn_part = fpart; f.h = fh;
    f.tokens = tokens; f.vocab = V; f.state = st;
    f.k_cache = kc; f.v_cache = vc; f.kv_bf16 = 0; f.max_seq = max_seq; f.rope_cur = rope_cur;
    f.splits = fsplits; f.run = run; f.eps = 1e-6f; f.scale = 0.08838834764f;
    f.sync = fsync; f.err = err;
    for (int it = 0; it < 8; it++) {
      const uint16_t* Wc = W + per_copy * (it % 4);
      f.w_qkv = Wc; f.w_o = Wc + n_qkv; f.w_gu = Wc + n_qkv + n_o; f.w_down = Wc + n_qkv + n_o + n_gu;
      f.res_in = res0; f.part_in = part_mlp; f.res_out = res1; f.part_out = part_attn;
      f.qkv_next = nullptr;
      if (pf_idle && fsplits < 16) {  // the engine's rule: the attention block's idle slots load the
        // first 2 (16 - runs) of each MLP workgroup's 24 gate|up rows of their XCD, the run slots
        // the rest once their partials are out
        const uint8_t* gu = reinterpret_cast<const uint8_t*>(f.w_gu);
        const uint32_t rows = std::min(2 * (16 - fsplits), 24u);
        f.pf[0] = qe::FusedPrefetch{gu, 2 * I / NX * H * 2, rows * H * 2, 24 * H * 2, qe::kFusedSlots};
        f.pf_idle = 1;
        if (rows < 24) {
          f.pf[1] = qe::FusedPrefetch{gu + size_t(rows) * H * 2, 2 * I / NX * H * 2, (24 - rows) * H * 2, 24 * H * 2,
                                      qe::kFusedSlots};
          f.pf_run = 1;
        }
        // ... and its o_proj workgroups the down columns of their XCD
        f.pf[2] = qe::FusedPrefetch{reinterpret_cast<const uint8_t*>(f.w_down), I / NX * 2, I / NX * 2, I * 2, H};
      }
      CK(qe::launch_fused_attn(f, false, s));
      f.pf_idle = 0;
      f.pf_run = 0;
      for (auto& r : f.pf) r = qe::FusedPrefetch{};
      // ... and the MLP block loads the next layer's q|k|v rows (the next weight copy's)
      if (pf_idle) f.qkv_next = W + per_copy * ((it + 1) % 4);
      f.res_in = res1; f.part_in = part_attn; f.res_out = res0; f.part_out = part_mlp;
      CK(qe::launch_fused_mlp(f, s));
      CK(hipStreamSynchronize(s));
    }
    for (int it = 0; it < 2; it++) {
      CK(qe::launch_fused_reduce(res0, part_mlp, x, 1, nullptr, 0.f, s));
      qe::MatvecParams p{};
      p.eps = 1e-6f; p.w = LM; p.x = x; p.nw = gains; p.rows = V; p.cols = H; p.out = logits; p.cand = cand;
      CK(qe::launch_matvec(p, qe::kNorm, qe::kLogits, s));
      CK(qe::launch_argmax(cand, n_cand, logits, st, tokens, nullptr, err, nullptr, nullptr, 0, s));
      CK(hipStreamSynchronize(s));
    }
    uint32_t e = 0;
    CK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
    std::printf("qe_stage_pmc: 8 x (attention block at pos %u in %u runs of %u, MLP block), 2 x (final reduce, "
                "lm_head, argmax); error bits 0x%x\n", pos, fsplits, run, e);
    return e ? 1 : 0;
  }

  for (int it = 0; it < 8; it++) {
    const uint16_t* Wc = W + per_copy * (it % 4);
    qe::MatvecParams p{};
    p.eps = 1e-6f;
    // q|k|v with the input RMSNorm
    p.w = Wc; p.x = x; p.nw = gains; p.rows = QD + 2 * KD; p.cols = H; p.out = qkv;
    CK(qe::launch_matvec_wide(p, qe::kNorm, qe::kStore, s));
    // attention: q/k norm + RoPE, K/V append at pos, split partials
    qe::AttnParams a{};
    a.qkv = qkv; a.q_norm = gains; a.k_norm = gains; a.rope = rope; a.rope_cur = rope_cur;
    a.k_cache = kc; a.v_cache = vc; a.partial = part; a.state = st; a.err = err;
    a.n_heads = NH; a.n_kv = NKV; a.max_seq = max_seq; a.eps = 1e-6f; a.scale = 0.08838834764f;
    if (prefetch) {
      a.pf[0] = qe::l2_prefetch_target(Wc + n_qkv + n_o, 2 * I, H, qe::kNorm, qe::kSiluPair);
      a.pf[1] = qe::l2_prefetch_target(Wc + n_qkv + n_o + n_gu, H, I, qe::kCopy, qe::kResAdd);
      a.pf_slots = qe::l2_prefetch_slots(a.pf, qe::kMaxPrefetch);
      // the engine's rule: prefetch while one layer's K/V (f32 here) is below half its bytes
      a.pf_max_pos = uint32_t(0.5 * (3.0 * I * H * 2) / (2.0 * NKV * D * 4));
    }
    CK(qe::launch_attention_split(a, splits, s));
    // merge + o_proj + residual
    p = qe::MatvecParams{};
    p.w = Wc + n_qkv; p.rows = H; p.cols = QD; p.out = x;
    p.attn_part = part; p.attn_splits = splits; p.attn_group = G;
    CK(qe::launch_matvec_wide(p, qe::kAttnMerge, qe::kResAdd, s));
    // post-attention RMSNorm + gate|up + silu*up
    p = qe::MatvecParams{};
    p.eps = 1e-6f; p.w = Wc + n_qkv + n_o; p.x = x; p.nw = gains; p.rows = 2 * I; p.cols = H; p.out = h;
    CK(qe::launch_matvec_wide(p, qe::kNorm, qe::kSiluPair, s));
    // down + residual
    p = qe::MatvecParams{};
    p.w = Wc + n_qkv + n_o + n_gu; p.x = h; p.rows = H; p.cols = I; p.out = x;
    CK(qe::launch_matvec_wide(p, qe::kCopy, qe::kResAdd, s));
    CK(hipStreamSynchronize(s));
  }
  for (int it = 0; it < 2; it++) {
    qe::MatvecParams p{};
    p.eps = 1e-6f; p.w = LM; p.x = x; p.nw = gains; p.rows = V; p.cols = H; p.out = logits; p.cand = cand;
    CK(qe::launch_matvec(p, qe::kNorm, qe::kLogits, s));
    CK(qe::launch_argmax(cand, n_cand, logits, st, tokens, nullptr, err, nullptr, nullptr, 0, s));
    CK(hipStreamSynchronize(s));
  }
  uint32_t e = 0;
  CK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
  std::printf("qe_stage_pmc: 8 x (qkv, attention at pos %u%s, o_proj, gate_up, down), 2 x (lm_head, argmax); error bits 0x%x\n",
              pos, prefetch ? " with the L2 prefetch" : "", e);
  return 0;
}
