// gfx950 kernels of the batch-1 decode step: one kernel per dependent stage.
//
// Stage map (reference: metal_infrence_engine/src/shaders/inference.metal, cpu_inference.rs):
//   embed + rmsnorm + q|k|v  -> k_mv_wide<.., kEmbedNorm, kStore>   (inference.metal:98-130, 143-186)
//   rmsnorm + matvec         -> k_mv_wide<.., kNorm, ..>            (inference.metal:113-130, 143-186)
//   qk_norm_rope + attention + K/V append -> k_attn_split (attention.hip, inference.metal:194-296)
//   attention merge + o_proj + add_inplace -> k_mv_wide<.., kAttnMerge, kResAdd>
//   silu_mul                 -> k_mv_wide epilogue kSiluPair          (inference.metal:325-334)
//   add_inplace              -> k_mv_wide epilogue kResAdd            (inference.metal:338-346)
//   final rmsnorm + lm_head  -> k_matvec<.., kNorm, kLogits>          (inference.metal:113-186)
//   argmax                   -> kLogits candidates + k_argmax         (inference.metal:300-321)
// All arithmetic is f32 with bf16 weights widened exactly (u16 << 16).
#include "kernels.h"

#include <algorithm>
#include <cmath>

#include "device_common.h"

namespace qe {
namespace {

// ---------------------------------------------------------------------------------------------
// matvec: out[r] = sum_c bf16(W[r,c]) * xin[c]   (cpu_inference.rs:225-257, inference.metal:143-186)
// 256 threads = 4 waves; each wave owns R consecutive rows; lane l reads 16-byte chunks
// l, l+64, ... of each row (CPL chunks per lane), so one wave-wide load covers 1 KB of a row.
// All weight loads are issued before the x prologue so they are in flight during it.
// Prologue kNorm: xin = (x * s) * gain with s = 1/sqrt(mean(x^2) + eps)  (cpu_inference.rs:189-194)
// ---------------------------------------------------------------------------------------------
// w and x are also leading arguments, preloaded into scalar registers at wave launch (the build's
// -amdgpu-kernarg-preload-count), so the weight loads do not wait for a load of the argument block.
template <int R, int CPL, int PRO, int EPI>
__global__ __launch_bounds__(256) void k_matvec(const uint16_t* w, const float* xv, uint32_t rows, uint32_t cols,
                                                MatvecParams p) {
  extern __shared__ __align__(16) float xs[];
  __shared__ float red[4];
  __shared__ ArgCand cbest[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t nch = cols >> 3;
  const uint32_t row0 = (blockIdx.x * 4u + uint32_t(wave)) * R;
  const uint4* W = reinterpret_cast<const uint4*>(w);

  // unconditional loads (a load behind a divergent branch is waited for on the spot): chunk
  // indexes past the row end re-read the last chunk and are skipped in the dot product. The
  // weights are streamed with the non-temporal hint: read once per step, 311.8 MB at the lm_head
  // shape, they then bypass the MALL (53.2 -> 48.9 us per lm_head, 2372 -> 2394 tok/s).
  uint4 wv[R][CPL];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint32_t row = min(row0 + uint32_t(r), rows - 1);  // past the end: re-read the last row
    const uint4* wr = W + size_t(row) * nch;
#pragma unroll
    for (int k = 0; k < CPL; k++) wv[r][k] = ld_stream(&wr[min(uint32_t(lane) + 64u * k, nch - 1)]);
  }

  const float4* x4 = reinterpret_cast<const float4*>(xv);
  float4* xs4 = reinterpret_cast<float4*>(xs);
  float ss = 0.f;
  for (uint32_t i = tid; i < cols / 4; i += 256) {
    float4 v = x4[i];
    xs4[i] = v;
    if (PRO == kNorm) ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  if (PRO == kNorm) {
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float s = 1.0f / sqrtf(tot / float(cols) + p.eps);
    for (uint32_t i = tid; i < cols; i += 256) xs[i] = xs[i] * s * bf16f(p.nw[i]);
  }
  __syncthreads();

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; k++) {
    const uint32_t c = uint32_t(lane) + 64u * k;
    if (c < nch) {
      const float4 a = xs4[2 * c], b = xs4[2 * c + 1];
#pragma unroll
      for (int r = 0; r < R; r++) acc[r] = dot8(wv[r][k], a, b, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);

  if (EPI == kStore || EPI == kResAdd) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t row = row0 + r;
        if (row < rows) {
          if (EPI == kStore) p.out[row] = acc[r];
          else p.out[row] += acc[r];
        }
      }
    }
  } else if (EPI == kSiluPair) {
    // rows 2i, 2i+1 are gate_i, up_i: out[i] = silu(gate_i) * up_i  (cpu_inference.rs:170)
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r + 1 < R; r += 2) {
        const uint32_t row = row0 + r;
        if (row + 1 < rows) {
          const float g = acc[r];
          p.out[row >> 1] = g / (1.0f + expf(-g)) * acc[r + 1];
        }
      }
    }
  } else if (EPI == kLogits) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t row = row0 + r;
      if (row < rows) {
        if (lane == 0) p.out[row] = acc[r];
        const float v = acc[r];
        if (!isnan(v) && cand_better(v, row, bv, bi)) { bv = v; bi = row; }
      }
    }
    if (lane == 0) cbest[wave] = ArgCand{bv, bi};
    __syncthreads();
    if (tid == 0) {
      ArgCand b = cbest[0];
      for (int w = 1; w < 4; w++)
        if (cand_better(cbest[w].v, cbest[w].i, b.v, b.i)) b = cbest[w];
      p.cand[blockIdx.x] = b;
    }
  }
}

// Any cols (multiple of 8): one wave per row, x read straight from global memory.
__global__ __launch_bounds__(256) void k_matvec_generic(MatvecParams p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t row = blockIdx.x * 4u + uint32_t(wave);
  if (row >= p.rows) return;
  const uint32_t nch = p.cols >> 3;
  const uint4* wr = reinterpret_cast<const uint4*>(p.w) + size_t(row) * nch;
  const float4* x4 = reinterpret_cast<const float4*>(p.x);
  float acc = 0.f;
  for (uint32_t c = lane; c < nch; c += 64) acc = dot8(wr[c], x4[2 * c], x4[2 * c + 1], acc);
  acc = wave_sum(acc);
  if (lane == 0) p.out[row] = acc;
}

// ---------------------------------------------------------------------------------------------
// matvec for the per-layer projections (q|k|v, o, gate|up, down). A batch-1 projection is only
// 4-13 MB, so a launch is latency-bound unless many workgroups have their loads in flight at
// once: TPR threads share a row (thread t reads 16-byte chunks t, t+TPR, ...), a 256-thread
// workgroup holds 256/TPR row groups of RR rows, giving ~1000 workgroups per launch. Each thread
// reads only the x chunks it multiplies, straight from global memory (no LDS staging).
// Prologue kNorm: every row group computes sum(x^2) over its own chunks (which cover the whole
// row) and normalizes them, (x * s) * gain (cpu_inference.rs:189-194).
// Prologue kEmbedNorm: x is the bf16 embedding row of the step's token (inference.metal:98-107),
// which workgroup 0 also stores to x_out for the residual stream.
// Prologue kAttnMerge: x[h*128 + d] is the attention output merged from the split partials
// [n_kv][splits][group][kPartStride] of the split attention kernel; each thread merges exactly
// the 8 dims of its own chunks, so no LDS is involved (SM >= splits partials are loaded).
// Every load is unconditional (chunk indexes past the row end re-read the last chunk and get
// x = 0) and all of them are issued before the first use: a load behind a divergent branch
// makes the compiler wait for it before issuing the next one. Inputs that come from L2 (x,
// gains, partials) are issued before the weights, which stream from HBM, so that prologue
// arithmetic overlaps the weight transfer; the embedding row depends on the token and goes last.
// ---------------------------------------------------------------------------------------------
template <int TPR, int CPT, int RR, int PRO, int EPI, int SM = 1>
__global__ __launch_bounds__(256) void k_mv_wide(MatvecParams p) {
  constexpr int NG = 256 / TPR;          // row groups per workgroup
  constexpr int WPG = TPR / 64;          // waves per row group
  constexpr bool NORM = PRO == kNorm || PRO == kEmbedNorm;
  __shared__ float red[4][RR + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = tid / TPR, t = tid % TPR;
  const uint32_t nch = p.cols >> 3;
  const uint32_t row0 = (blockIdx.x * NG + uint32_t(grp)) * RR;
  const uint4* W = reinterpret_cast<const uint4*>(p.w);
  uint32_t cc[CPT];  // clamped chunk index
#pragma unroll
  for (int k = 0; k < CPT; k++) cc[k] = min(uint32_t(t) + uint32_t(TPR) * k, nch - 1);

  uint4 wv[RR][CPT];
  auto load_weights = [&]() {
#pragma unroll
    for (int r = 0; r < RR; r++) {
      const uint32_t row = min(row0 + uint32_t(r), p.rows - 1);
#pragma unroll
      for (int k = 0; k < CPT; k++) wv[r][k] = W[size_t(row) * nch + cc[k]];
    }
  };
  uint4 gains[CPT];
  auto load_gains = [&]() {
    const uint4* NWv = reinterpret_cast<const uint4*>(p.nw);
#pragma unroll
    for (int k = 0; k < CPT; k++) gains[k] = NWv[cc[k]];
  };

  // residual rows (epilogue kResAdd: out += acc), read up front instead of after the reduction
  float res[RR];
  auto load_res = [&]() {
    if constexpr (EPI == kResAdd) {
#pragma unroll
      for (int r = 0; r < RR; r++) res[r] = p.out[min(row0 + uint32_t(r), p.rows - 1)];
    }
  };

  // Loads first, then a scheduling barrier: without it the scheduler sinks loads towards their
  // uses (to save registers), behind waits for the earlier ones.
  float4 xa[CPT], xb[CPT];
  if constexpr (PRO == kEmbedNorm) {
    load_weights();
    load_gains();
    load_res();
    uint32_t tok = p.tokens[p.state->tok_idx];
    if (tok >= p.vocab) {
      if (blockIdx.x == 0 && tid == 0) atomicOr(p.err, kErrToken);
      tok = 0;
    }
    const uint4* E = reinterpret_cast<const uint4*>(p.embed) + size_t(tok) * nch;
    uint4 e[CPT];
#pragma unroll
    for (int k = 0; k < CPT; k++) e[k] = E[cc[k]];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      xa[k] = make_float4(__uint_as_float(e[k].x << 16), __uint_as_float(e[k].x & 0xFFFF0000u),
                          __uint_as_float(e[k].y << 16), __uint_as_float(e[k].y & 0xFFFF0000u));
      xb[k] = make_float4(__uint_as_float(e[k].z << 16), __uint_as_float(e[k].z & 0xFFFF0000u),
                          __uint_as_float(e[k].w << 16), __uint_as_float(e[k].w & 0xFFFF0000u));
      const uint32_t c = uint32_t(t) + uint32_t(TPR) * k;
      if (blockIdx.x == 0 && grp == 0 && c < nch) {
        float4* xo = reinterpret_cast<float4*>(p.x_out);
        xo[2 * c] = xa[k];
        xo[2 * c + 1] = xb[k];
      }
    }
  } else if constexpr (PRO == kAttnMerge) {
    // out_h = sum_s e_s acc_s / sum_s e_s l_s with e_s = exp(m_s - max m); empty runs (m = -inf)
    // and loads past the last split (s >= splits re-read the last one) weigh 0
    const uint32_t G = p.attn_group, S = p.attn_splits;
    float2 ml[CPT][SM];
    float4 a0[CPT][SM], a1[CPT][SM];
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      const uint32_t h = cc[k] >> 4, d0 = (cc[k] & 15) * 8, g = h / G, j = h % G;
      const float* base = p.attn_part + (size_t(g) * S * G + j) * kPartStride;
#pragma unroll
      for (int s = 0; s < SM; s++) {
        const float* q = base + size_t(min(uint32_t(s), S - 1)) * G * kPartStride;
        ml[k][s] = *reinterpret_cast<const float2*>(q);
        a0[k][s] = *reinterpret_cast<const float4*>(q + 4 + d0);
        a1[k][s] = *reinterpret_cast<const float4*>(q + 8 + d0);
      }
    }
    load_res();
    load_weights();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      float M = -INFINITY;
#pragma unroll
      for (int s = 0; s < SM; s++) M = uint32_t(s) < S ? fmaxf(M, ml[k][s].x) : M;
      float L = 0.f;
      float4 A0 = make_float4(0.f, 0.f, 0.f, 0.f), A1 = A0;
#pragma unroll
      for (int s = 0; s < SM; s++) {
        const float e = (uint32_t(s) < S && ml[k][s].x != -INFINITY) ? expf(ml[k][s].x - M) : 0.f;
        L += e * ml[k][s].y;
        A0.x += e * a0[k][s].x; A0.y += e * a0[k][s].y; A0.z += e * a0[k][s].z; A0.w += e * a0[k][s].w;
        A1.x += e * a1[k][s].x; A1.y += e * a1[k][s].y; A1.z += e * a1[k][s].z; A1.w += e * a1[k][s].w;
      }
      const float inv = 1.0f / L;
      xa[k] = make_float4(A0.x * inv, A0.y * inv, A0.z * inv, A0.w * inv);
      xb[k] = make_float4(A1.x * inv, A1.y * inv, A1.z * inv, A1.w * inv);
    }
  } else {
    const float4* x4 = reinterpret_cast<const float4*>(p.x);
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      xa[k] = x4[2 * cc[k]];
      xb[k] = x4[2 * cc[k] + 1];
    }
    if constexpr (NORM) load_gains();
    load_res();
    load_weights();
    __builtin_amdgcn_sched_barrier(0);
  }
  if (uint32_t(TPR) * CPT > nch) {  // chunks past the row end contribute 0
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      const bool in = uint32_t(t) + uint32_t(TPR) * k < nch;
      const float z = 0.f;
      xa[k] = make_float4(in ? xa[k].x : z, in ? xa[k].y : z, in ? xa[k].z : z, in ? xa[k].w : z);
      xb[k] = make_float4(in ? xb[k].x : z, in ? xb[k].y : z, in ? xb[k].z : z, in ? xb[k].w : z);
    }
  }
  // RMSNorm: the scale s is a scalar, so sum_c W[r,c] * ((x_c * s) * g_c) is evaluated as
  // s * sum_c W[r,c] * (x_c * g_c): the sum of squares then reduces alongside the dot products
  // instead of in front of them (a reassociation of the reference's f32 product, well inside
  // the logit tolerance)
  float ss = 0.f;
  if constexpr (NORM) {
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      ss += (xa[k].x * xa[k].x + xa[k].y * xa[k].y + xa[k].z * xa[k].z + xa[k].w * xa[k].w) +
            (xb[k].x * xb[k].x + xb[k].y * xb[k].y + xb[k].z * xb[k].z + xb[k].w * xb[k].w);
      const uint4 g = gains[k];
      xa[k].x *= __uint_as_float(g.x << 16);
      xa[k].y *= __uint_as_float(g.x & 0xFFFF0000u);
      xa[k].z *= __uint_as_float(g.y << 16);
      xa[k].w *= __uint_as_float(g.y & 0xFFFF0000u);
      xb[k].x *= __uint_as_float(g.z << 16);
      xb[k].y *= __uint_as_float(g.z & 0xFFFF0000u);
      xb[k].z *= __uint_as_float(g.w << 16);
      xb[k].w *= __uint_as_float(g.w & 0xFFFF0000u);
    }
  }

  float acc[RR];
#pragma unroll
  for (int r = 0; r < RR; r++) {
    acc[r] = 0.f;
#pragma unroll
    for (int k = 0; k < CPT; k++) acc[r] = dot8(wv[r][k], xa[k], xb[k], acc[r]);
    acc[r] = wave_sum(acc[r]);
  }
  if constexpr (NORM) ss = wave_sum(ss);
  if (WPG > 1) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RR; r++) red[wave][r] = acc[r];
      red[wave][RR] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r <= RR; r++) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < WPG; w++) v += red[grp * WPG + w][r];
      if (r < RR) acc[r] = v;
      else ss = v;
    }
  }
  if constexpr (NORM) {
    const float s = 1.0f / sqrtf(ss / float(p.cols) + p.eps);
#pragma unroll
    for (int r = 0; r < RR; r++) acc[r] *= s;
  }
  if (t != 0) return;
  if (EPI == kStore || EPI == kResAdd) {
#pragma unroll
    for (int r = 0; r < RR; r++) {
      const uint32_t row = row0 + r;
      if (row < p.rows) {
        if (EPI == kStore) p.out[row] = acc[r];
        else p.out[row] = res[r] + acc[r];
      }
    }
  } else if (EPI == kSiluPair) {
#pragma unroll
    for (int r = 0; r + 1 < RR; r += 2) {
      const uint32_t row = row0 + r;
      if (row + 1 < p.rows) {
        const float g = acc[r];
        p.out[row >> 1] = g / (1.0f + expf(-g)) * acc[r + 1];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// argmax over the per-workgroup candidates; first maximum wins; a NaN logits[0] gives 0 (the
// sequential scan of main.rs:37-42 can never move off index 0 then). Feeds the next step.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_argmax(const ArgCand* __restrict__ cand, uint32_t n_cand,
                                                 const float* __restrict__ logits, StepState* st,
                                                 uint32_t* tokens, uint32_t* host_tokens, uint32_t* err,
                                                 const float* __restrict__ rope, float* rope_cur, uint32_t half) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the RoPE row of the next position, which the next step's attention reads as rope_cur
  const uint32_t next = st->pos + 1, max_seq = st->max_seq;
  float2 rc = make_float2(0.f, 0.f);
  if (rope) {
    rc = reinterpret_cast<const float2*>(rope)[size_t(min(next, max_seq - 1)) * half + min(uint32_t(tid), half - 1)];
  }
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  // candidates per thread loaded together, so their latencies overlap; indexes past the end
  // re-read the last candidate, which cannot change the result
  constexpr int U = 16;
  for (uint32_t base = 0; base < n_cand; base += 1024u * U) {
    ArgCand c[U];
#pragma unroll
    for (int u = 0; u < U; u++) c[u] = cand[min(base + uint32_t(tid) + 1024u * u, n_cand - 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; u++)
      if (cand_better(c[u].v, c[u].i, bv, bi)) { bv = c[u].v; bi = c[u].i; }
  }
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(bv, o);
    const uint32_t oi = __shfl_xor(bi, o);
    if (cand_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 16; w++)
      if (cand_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    const uint32_t tok = (isnan(logits[0]) || bi == 0xFFFFFFFFu) ? 0u : bi;
    const uint32_t k = st->tok_idx + 1;
    if (k < st->tok_cap) {
      tokens[k] = tok;
      if (host_tokens) host_tokens[k] = tok;
    } else {
      atomicOr(err, kErrRing);
    }
    st->pos = next;
    st->tok_idx = k;
  }
  if (rope_cur && uint32_t(tid) < half && next < max_seq) reinterpret_cast<float2*>(rope_cur)[tid] = rc;
}

// streaming read (tests/read_bandwidth.rs:16-54): grid-stride float4, 4 accumulators
__global__ __launch_bounds__(256) void k_read_sum(const float4* __restrict__ src, uint64_t n4, float* partial) {
  const uint64_t grid = uint64_t(gridDim.x) * 256;
  uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
  float4 a0 = make_float4(0, 0, 0, 0), a1 = a0, a2 = a0, a3 = a0;
  for (; i + 3 * grid < n4; i += 4 * grid) {
    const float4 v0 = src[i], v1 = src[i + grid], v2 = src[i + 2 * grid], v3 = src[i + 3 * grid];
    a0.x += v0.x; a0.y += v0.y; a0.z += v0.z; a0.w += v0.w;
    a1.x += v1.x; a1.y += v1.y; a1.z += v1.z; a1.w += v1.w;
    a2.x += v2.x; a2.y += v2.y; a2.z += v2.z; a2.w += v2.w;
    a3.x += v3.x; a3.y += v3.y; a3.z += v3.z; a3.w += v3.w;
  }
  for (; i < n4; i += grid) {
    const float4 v = src[i];
    a0.x += v.x; a0.y += v.y; a0.z += v.z; a0.w += v.w;
  }
  float s = ((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w)) +
            ((a2.x + a2.y) + (a2.z + a2.w)) + ((a3.x + a3.y) + (a3.z + a3.w));
  s = wave_sum(s);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

// The same read with non-temporal loads, workgroup b summing the contiguous float4s
// [n4 b / grid, n4 (b + 1) / grid): the streaming form that reads fastest on gfx950.
__global__ __launch_bounds__(256) void k_read_sum_nt(const float4* __restrict__ src, uint64_t n4, float* partial) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  const f32x4_t* s4 = reinterpret_cast<const f32x4_t*>(src);
  const uint64_t b1 = n4 * (blockIdx.x + 1) / gridDim.x;
  uint64_t i = n4 * blockIdx.x / gridDim.x + threadIdx.x;
  f32x4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0, a3 = a0;
  for (; i + 3 * 256 < b1; i += 4 * 256) {
    const f32x4_t v0 = __builtin_nontemporal_load(s4 + i), v1 = __builtin_nontemporal_load(s4 + i + 256),
                  v2 = __builtin_nontemporal_load(s4 + i + 512), v3 = __builtin_nontemporal_load(s4 + i + 768);
    a0 += v0;
    a1 += v1;
    a2 += v2;
    a3 += v3;
  }
  for (; i < b1; i += 256) a0 += __builtin_nontemporal_load(s4 + i);
  float s = ((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w)) +
            ((a2.x + a2.y) + (a2.z + a2.w)) + ((a3.x + a3.y) + (a3.z + a3.w));
  s = wave_sum(s);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

// rows per workgroup for a given chunks-per-lane
constexpr int rows_per_wave(int cpl, int epi) {
  return epi == kSiluPair ? (cpl <= 2 ? 4 : 2) : (cpl <= 1 ? 8 : cpl <= 2 ? 4 : cpl <= 4 ? 2 : 1);
}

template <int CPL, int PRO, int EPI>
hipError_t launch_mv(const MatvecParams& p, hipStream_t s) {
  constexpr int R = rows_per_wave(CPL, EPI);
  const uint32_t blocks = ceil_div(p.rows, 4u * R);
  hipLaunchKernelGGL((k_matvec<R, CPL, PRO, EPI>), dim3(blocks), dim3(256), size_t(p.cols) * 4, s, p.w, p.x, p.rows,
                     p.cols, p);
  return hipGetLastError();
}

template <int TPR, int CPT, int RR, int PRO, int EPI, int SM = 1>
hipError_t launch_wide(const MatvecParams& p, hipStream_t s) {
  constexpr int rows_per_block = (256 / TPR) * RR;
  const uint32_t blocks = ceil_div(p.rows, rows_per_block);
  hipLaunchKernelGGL((k_mv_wide<TPR, CPT, RR, PRO, EPI, SM>), dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

// rows per row group: silu needs the (gate, up) pair; one-chunk rows of <= 128 threads take two
template <int TPR, int CPT, int PRO, int EPI>
hipError_t launch_wide_rr(const MatvecParams& p, hipStream_t s) {
  // two rows per row group also for the 3-chunk rows of down (measured +0.8% per decode step)
  constexpr int RR = (EPI == kSiluPair || (TPR <= 128 && CPT == 1) || (TPR == 128 && CPT == 3)) ? 2 : 1;
  return launch_wide<TPR, CPT, RR, PRO, EPI>(p, s);
}

// threads per row x chunks per thread: an exact fit where one exists, so no lane idles
template <int PRO, int EPI>
hipError_t launch_wide_cols(const MatvecParams& p, hipStream_t s) {
  const uint32_t nch = p.cols / 8;
  if (nch <= 64) return launch_wide_rr<64, 1, PRO, EPI>(p, s);
  // gate|up (the silu pair, usually on weights the attention launch prefetched into L2) runs
  // faster on twice the rows per workgroup: 64 threads x 2 chunks per row group (measured +1.3%
  // per decode step)
  if (nch <= 128) return EPI == kSiluPair ? launch_wide_rr<64, 2, PRO, EPI>(p, s) : launch_wide_rr<128, 1, PRO, EPI>(p, s);
  if (nch <= 256) return launch_wide_rr<256, 1, PRO, EPI>(p, s);
  if (nch == 384) return launch_wide_rr<128, 3, PRO, EPI>(p, s);
  if (nch <= 512) return launch_wide_rr<256, 2, PRO, EPI>(p, s);
  return hipErrorInvalidValue;
}

// attention merge + o_proj + residual: four rows per workgroup amortize the merge, which every
// workgroup repeats for the whole input
template <int SM>
hipError_t launch_merge_cols(const MatvecParams& p, hipStream_t s) {
  const uint32_t nch = p.cols / 8;
  if (nch <= 128) return launch_wide<128, 1, 4, kAttnMerge, kResAdd, SM>(p, s);
  if (nch <= 256) return launch_wide<256, 1, 4, kAttnMerge, kResAdd, SM>(p, s);
  if (nch <= 512) return launch_wide<256, 2, 4, kAttnMerge, kResAdd, SM>(p, s);
  return hipErrorInvalidValue;
}

template <int PRO, int EPI>
hipError_t launch_mv_cpl(const MatvecParams& p, hipStream_t s) {
  const uint32_t nch = p.cols / 8;
  if (nch <= 64) return launch_mv<1, PRO, EPI>(p, s);
  if (nch <= 128) return launch_mv<2, PRO, EPI>(p, s);
  if (nch <= 256) return launch_mv<4, PRO, EPI>(p, s);
  if (nch <= 384) return launch_mv<6, PRO, EPI>(p, s);
  if (nch <= 512) return launch_mv<8, PRO, EPI>(p, s);
  return hipErrorInvalidValue;
}

}  // namespace

uint32_t matvec_num_blocks(uint32_t rows, uint32_t cols, int epilogue) {
  const uint32_t nch = cols / 8;
  const int cpl = nch <= 64 ? 1 : nch <= 128 ? 2 : nch <= 256 ? 4 : nch <= 384 ? 6 : nch <= 512 ? 8 : 0;
  if (!cpl) return ceil_div(rows, 4);
  return ceil_div(rows, 4u * uint32_t(rows_per_wave(cpl, epilogue)));
}

hipError_t launch_matvec(const MatvecParams& p, int prologue, int epilogue, hipStream_t s) {
  if (p.cols % 8 || p.rows == 0 || p.cols == 0) return hipErrorInvalidValue;
  if (p.cols / 8 > 512) {
    if (prologue != kCopy || epilogue != kStore) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_matvec_generic, dim3(ceil_div(p.rows, 4)), dim3(256), 0, s, p);
    return hipGetLastError();
  }
  if (prologue == kCopy && epilogue == kStore) return launch_mv_cpl<kCopy, kStore>(p, s);
  if (prologue == kCopy && epilogue == kResAdd) return launch_mv_cpl<kCopy, kResAdd>(p, s);
  if (prologue == kNorm && epilogue == kStore) return launch_mv_cpl<kNorm, kStore>(p, s);
  if (prologue == kNorm && epilogue == kSiluPair) return launch_mv_cpl<kNorm, kSiluPair>(p, s);
  if (prologue == kNorm && epilogue == kLogits) return launch_mv_cpl<kNorm, kLogits>(p, s);
  if (prologue == kCopy && epilogue == kLogits) return launch_mv_cpl<kCopy, kLogits>(p, s);
  return hipErrorInvalidValue;
}

// rows one workgroup of launch_matvec_wide covers: (256 / TPR) row groups of RR rows, with the
// TPR / CPT / RR that launch_wide_cols and launch_merge_cols pick for this shape
uint32_t matvec_wide_rows_per_block(uint32_t cols, int prologue, int epilogue) {
  const uint32_t nch = cols / 8;
  if (prologue == kAttnMerge) return nch <= 128 ? 8 : 4;  // RR 4 with TPR 128, else TPR 256
  const bool silu = epilogue == kSiluPair;
  if (nch <= 64) return 4 * 2;                // TPR 64, CPT 1: RR 2
  if (nch <= 128) return silu ? 4 * 2 : 2 * 2;  // silu: TPR 64, CPT 2, RR 2; else TPR 128, CPT 1, RR 2
  if (nch <= 256) return silu ? 2 : 1;        // TPR 256
  if (nch == 384) return 2 * 2;               // TPR 128, CPT 3: RR 2
  return silu ? 2 : 1;                        // TPR 256, CPT 2
}

L2Prefetch l2_prefetch_target(const uint16_t* w, uint32_t rows, uint32_t cols, int prologue, int epilogue) {
  const uint32_t rpb = matvec_wide_rows_per_block(cols, prologue, epilogue);
  return L2Prefetch{w, rows * (cols / 8), rpb * (cols / 8), ceil_div(rows, rpb)};
}

uint32_t l2_prefetch_slots(const L2Prefetch* pf, int n) {
  uint64_t chunks = 0;
  for (int i = 0; i < n; i++) chunks += pf[i].w ? pf[i].n_chunks : 0;
  if (!chunks) return 0;
  // 8 XCDs x slots workgroups x 256 threads x 16 chunks, with headroom for uneven splits
  return uint32_t(std::min<uint64_t>(64, ceil_div(uint32_t(chunks), 8u * 256u * 12u)));
}

hipError_t launch_matvec_wide(const MatvecParams& p, int prologue, int epilogue, hipStream_t s) {
  if (p.cols % 8 || p.rows == 0 || p.cols == 0 || p.cols / 8 > 512) return hipErrorInvalidValue;
  if (epilogue == kSiluPair && p.rows % 2) return hipErrorInvalidValue;
  if (prologue == kCopy && epilogue == kStore) return launch_wide_cols<kCopy, kStore>(p, s);
  if (prologue == kCopy && epilogue == kResAdd) return launch_wide_cols<kCopy, kResAdd>(p, s);
  if (prologue == kNorm && epilogue == kStore) return launch_wide_cols<kNorm, kStore>(p, s);
  if (prologue == kEmbedNorm && epilogue == kStore) return launch_wide_cols<kEmbedNorm, kStore>(p, s);
  if (prologue == kNorm && epilogue == kSiluPair) return launch_wide_cols<kNorm, kSiluPair>(p, s);
  if (prologue == kAttnMerge && epilogue == kResAdd) {
    if (!p.attn_part || p.attn_splits == 0 || p.attn_splits > uint32_t(kAttnMaxMergeSplits) ||
        p.attn_group == 0 || p.cols % kHeadDim)
      return hipErrorInvalidValue;
    if (p.attn_splits <= 4) return launch_merge_cols<4>(p, s);
    if (p.attn_splits <= 8) return launch_merge_cols<8>(p, s);
    return launch_merge_cols<16>(p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_argmax(const ArgCand* cand, uint32_t n_cand, const float* logits, StepState* st, uint32_t* tokens,
                         uint32_t* host_tokens, uint32_t* err, const float* rope, float* rope_cur, uint32_t half,
                         hipStream_t s) {
  if (n_cand == 0 || (rope && (half == 0 || half > 1024))) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, cand, n_cand, logits, st, tokens, host_tokens, err, rope,
                     rope_cur, half);
  return hipGetLastError();
}

hipError_t launch_read_sum(const float* src, uint64_t n, float* partial, uint32_t grid, bool nt, hipStream_t s) {
  if (n % 4 || grid == 0) return hipErrorInvalidValue;
  if (nt)
    hipLaunchKernelGGL(k_read_sum_nt, dim3(grid), dim3(256), 0, s, reinterpret_cast<const float4*>(src), n / 4,
                       partial);
  else
    hipLaunchKernelGGL(k_read_sum, dim3(grid), dim3(256), 0, s, reinterpret_cast<const float4*>(src), n / 4, partial);
  return hipGetLastError();
}

}  // namespace qe
