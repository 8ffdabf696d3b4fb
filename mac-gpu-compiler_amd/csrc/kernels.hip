// gfx950 kernels of the batch-1 decode step: one kernel per dependent stage.
//
// Stage map (reference: metal_infrence_engine/src/shaders/inference.metal, cpu_inference.rs):
//   embed            -> k_embed                        (inference.metal:98-107)
//   rmsnorm + matvec -> k_matvec<.., kNorm, ..>          (inference.metal:113-130, 143-186)
//   qk_norm_rope + attention + K/V append -> k_attention (inference.metal:194-296)
//   silu_mul         -> k_matvec epilogue kSiluPair      (inference.metal:325-334)
//   add_inplace      -> k_matvec epilogue kResAdd        (inference.metal:338-346)
//   argmax           -> k_matvec epilogue kLogits + k_argmax (inference.metal:300-321)
// All arithmetic is f32 with bf16 weights widened exactly (u16 << 16).
#include "kernels.h"

#include <cmath>

namespace qe {
namespace {

__device__ __forceinline__ float bf16f(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return uint16_t((u >> 16) | 0x40);
  return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Cross-lane move through DPP. Lanes the control does not write keep 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes of a wave, returned to every lane (wave-uniform).
// quad xor1, quad xor2, half-row mirror, row mirror, row_bcast15 (rows 1,3), row_bcast31 (rows 2,3):
// lane 63 then holds the total.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  v += dpp<0x142, 0xA>(v);
  v += dpp<0x143, 0xC>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// a beats b: larger value, or equal value and lower index (first maximum wins, main.rs:37-42)
__device__ __forceinline__ bool cand_better(float av, uint32_t ai, float bv, uint32_t bi) {
  return av > bv || (av == bv && ai < bi);
}

// acc += sum of the 8 bf16 weights in u times the 8 floats a, b (f32 FMA)
__device__ __forceinline__ float dot8(uint4 u, float4 a, float4 b, float acc) {
  acc = fmaf(__uint_as_float(u.x << 16), a.x, acc);
  acc = fmaf(__uint_as_float(u.x & 0xFFFF0000u), a.y, acc);
  acc = fmaf(__uint_as_float(u.y << 16), a.z, acc);
  acc = fmaf(__uint_as_float(u.y & 0xFFFF0000u), a.w, acc);
  acc = fmaf(__uint_as_float(u.z << 16), b.x, acc);
  acc = fmaf(__uint_as_float(u.z & 0xFFFF0000u), b.y, acc);
  acc = fmaf(__uint_as_float(u.w << 16), b.z, acc);
  acc = fmaf(__uint_as_float(u.w & 0xFFFF0000u), b.w, acc);
  return acc;
}

__host__ __device__ __forceinline__ uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------------------------
// embed: x = bf16 row of the token read from the device token ring (inference.metal:98-107)
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed(const uint16_t* __restrict__ table, uint32_t hidden, uint32_t vocab,
                                               const uint32_t* __restrict__ tokens, const StepState* __restrict__ st,
                                               float* __restrict__ x, uint32_t* err) {
  uint32_t tok = tokens[st->tok_idx];
  if (tok >= vocab) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, kErrToken);
    tok = 0;
  }
  uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < hidden) x[i] = bf16f(table[size_t(tok) * hidden + i]);
}

// ---------------------------------------------------------------------------------------------
// matvec: out[r] = sum_c bf16(W[r,c]) * xin[c]   (cpu_inference.rs:225-257, inference.metal:143-186)
// 256 threads = 4 waves; each wave owns R consecutive rows; lane l reads 16-byte chunks
// l, l+64, ... of each row (CPL chunks per lane), so one wave-wide load covers 1 KB of a row.
// All weight loads are issued before the x prologue so they are in flight during it.
// Prologue kNorm: xin = (x * s) * gain with s = 1/sqrt(mean(x^2) + eps)  (cpu_inference.rs:189-194)
// ---------------------------------------------------------------------------------------------
template <int R, int CPL, int PRO, int EPI>
__global__ __launch_bounds__(256) void k_matvec(MatvecParams p) {
  extern __shared__ __align__(16) float xs[];
  __shared__ float red[4];
  __shared__ ArgCand cbest[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t nch = p.cols >> 3;
  const uint32_t row0 = (blockIdx.x * 4u + uint32_t(wave)) * R;
  const uint4* W = reinterpret_cast<const uint4*>(p.w);

  uint4 wv[R][CPL];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint32_t row = min(row0 + uint32_t(r), p.rows - 1);  // past the end: re-read the last row
    const uint4* wr = W + size_t(row) * nch;
#pragma unroll
    for (int k = 0; k < CPL; k++) {
      const uint32_t c = uint32_t(lane) + 64u * k;
      wv[r][k] = c < nch ? wr[c] : make_uint4(0, 0, 0, 0);
    }
  }

  const float4* x4 = reinterpret_cast<const float4*>(p.x);
  float4* xs4 = reinterpret_cast<float4*>(xs);
  float ss = 0.f;
  for (uint32_t i = tid; i < p.cols / 4; i += 256) {
    float4 v = x4[i];
    xs4[i] = v;
    if (PRO == kNorm) ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  if (PRO == kNorm) {
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float s = 1.0f / sqrtf(tot / float(p.cols) + p.eps);
    for (uint32_t i = tid; i < p.cols; i += 256) xs[i] = xs[i] * s * bf16f(p.nw[i]);
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
        if (row < p.rows) {
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
        if (row + 1 < p.rows) {
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
      if (row < p.rows) {
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
// attention for one new token: GQA, split-K over positions with an online softmax per split,
// merged by the last split to finish (inference.metal:194-296, cpu_inference.rs:134-162).
// grid (n_kv, grid_splits); one workgroup serves all G q heads of its KV head from one read of
// K/V. Lane l holds head dims (2l, 2l+1). With norm_rope, the workgroup first applies the
// per-head q RMSNorm + RoPE, and the split that owns `pos` also normalizes/rotates the new k
// and appends k and v to the cache (cpu_inference.rs:137-141).
// ---------------------------------------------------------------------------------------------
template <int G, bool KV_BF16>
__global__ __launch_bounds__(256) void k_attention(AttnParams p) {
  constexpr int D = kHeadDim;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t g = blockIdx.x;
  uint32_t n, pos;
  if (p.norm_rope) {
    pos = p.state->pos;
    if (pos >= p.max_seq) {
      if (g == 0 && blockIdx.y == 0 && tid == 0) atomicOr(p.err, kErrPos);
      return;
    }
    n = pos + 1;
  } else {
    n = p.n_pos_fixed;
    pos = n - 1;
  }
  uint32_t nsplit = p.force_splits ? min(p.force_splits, gridDim.y) : min(gridDim.y, ceil_div(n, kAttnMinChunk));
  const uint32_t chunk = ceil_div(n, nsplit);
  nsplit = ceil_div(n, chunk);
  const uint32_t s = blockIdx.y;
  if (s >= nsplit) return;
  const uint32_t t0 = s * chunk, t1 = min(n, t0 + chunk);
  const bool owns_new = p.norm_rope && t1 == n;

  __shared__ float qs[G][D];
  __shared__ float knew[D], vnew[D], ktmp[D];
  __shared__ float wm[4][G], wl[4][G];
  __shared__ float wacc[4][G][D];
  __shared__ int is_last;

  for (int i = tid; i < G * D; i += 256) qs[i / D][i % D] = p.qkv[size_t(g) * G * D + i];
  __syncthreads();
  if (p.norm_rope) {
    for (int j = wave; j < G; j += 4) {
      const float a = qs[j][2 * lane], b = qs[j][2 * lane + 1];
      const float ssum = wave_sum(a * a + b * b);
      const float sc = 1.0f / sqrtf(ssum / float(D) + p.eps);
      qs[j][2 * lane] = a * sc * bf16f(p.q_norm[2 * lane]);
      qs[j][2 * lane + 1] = b * sc * bf16f(p.q_norm[2 * lane + 1]);
    }
    if (owns_new && wave == 0) {
      const float* kr = p.qkv + size_t(p.n_heads) * D + size_t(g) * D;
      const float* vr = p.qkv + size_t(p.n_heads) * D + size_t(p.n_kv) * D + size_t(g) * D;
      const float a = kr[2 * lane], b = kr[2 * lane + 1];
      const float ssum = wave_sum(a * a + b * b);
      const float sc = 1.0f / sqrtf(ssum / float(D) + p.eps);
      ktmp[2 * lane] = a * sc * bf16f(p.k_norm[2 * lane]);
      ktmp[2 * lane + 1] = b * sc * bf16f(p.k_norm[2 * lane + 1]);
      vnew[2 * lane] = vr[2 * lane];
      vnew[2 * lane + 1] = vr[2 * lane + 1];
    }
    __syncthreads();
    const float2* rope = reinterpret_cast<const float2*>(p.rope) + size_t(pos) * (D / 2);
    for (int i = tid; i < G * (D / 2); i += 256) {
      const int j = i / (D / 2), d = i % (D / 2);
      const float2 cs = rope[d];
      const float a = qs[j][d], b = qs[j][d + D / 2];
      qs[j][d] = a * cs.x - b * cs.y;
      qs[j][d + D / 2] = b * cs.x + a * cs.y;
    }
    if (owns_new && tid < D / 2) {
      const float2 cs = rope[tid];
      const float a = ktmp[tid], b = ktmp[tid + D / 2];
      knew[tid] = a * cs.x - b * cs.y;
      knew[tid + D / 2] = b * cs.x + a * cs.y;
    }
    __syncthreads();
    if (owns_new && tid < D) {
      const size_t slot = (size_t(g) * p.max_seq + pos) * D + tid;
      if (KV_BF16) {
        const uint16_t kb = f32_to_bf16(knew[tid]), vb = f32_to_bf16(vnew[tid]);
        static_cast<uint16_t*>(p.k_cache)[slot] = kb;
        static_cast<uint16_t*>(p.v_cache)[slot] = vb;
        knew[tid] = bf16f(kb);  // attend with what later steps will read back
        vnew[tid] = bf16f(vb);
      } else {
        static_cast<float*>(p.k_cache)[slot] = knew[tid];
        static_cast<float*>(p.v_cache)[slot] = vnew[tid];
      }
    }
    __syncthreads();
  }

  // per-wave online softmax over positions t0 + wave, t0 + wave + 4, ...
  float2 q2[G];
#pragma unroll
  for (int j = 0; j < G; j++) q2[j] = make_float2(qs[j][2 * lane], qs[j][2 * lane + 1]);
  float m[G], l[G];
  float2 acc[G];
#pragma unroll
  for (int j = 0; j < G; j++) { m[j] = -INFINITY; l[j] = 0.f; acc[j] = make_float2(0.f, 0.f); }

  const size_t head_base = size_t(g) * p.max_seq * D;
  // positions that come from the cache; with owns_new the last one (pos) comes from LDS
  const uint32_t tc1 = owns_new ? t1 - 1 : t1;
  constexpr int U = 4;
  uint32_t t = t0 + wave;
  for (; t + 4 * (U - 1) < tc1; t += 4 * U) {
    float2 kk[U], vv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const size_t off = head_base + size_t(t + 4 * u) * D + 2 * lane;
      if (KV_BF16) {
        const uint32_t kb = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.k_cache) + off);
        const uint32_t vb = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.v_cache) + off);
        kk[u] = make_float2(__uint_as_float(kb << 16), __uint_as_float(kb & 0xFFFF0000u));
        vv[u] = make_float2(__uint_as_float(vb << 16), __uint_as_float(vb & 0xFFFF0000u));
      } else {
        kk[u] = *reinterpret_cast<const float2*>(static_cast<const float*>(p.k_cache) + off);
        vv[u] = *reinterpret_cast<const float2*>(static_cast<const float*>(p.v_cache) + off);
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
#pragma unroll
      for (int j = 0; j < G; j++) {
        const float sc = wave_sum(q2[j].x * kk[u].x + q2[j].y * kk[u].y) * p.scale;
        const float mn = fmaxf(m[j], sc);
        const float co = expf(m[j] - mn), pe = expf(sc - mn);
        l[j] = l[j] * co + pe;
        acc[j].x = acc[j].x * co + pe * vv[u].x;
        acc[j].y = acc[j].y * co + pe * vv[u].y;
        m[j] = mn;
      }
    }
  }
  for (; t < tc1 + (owns_new ? 1u : 0u); t += 4) {
    float2 kk, vv;
    if (owns_new && t == tc1) {
      kk = make_float2(knew[2 * lane], knew[2 * lane + 1]);
      vv = make_float2(vnew[2 * lane], vnew[2 * lane + 1]);
    } else {
      const size_t off = head_base + size_t(t) * D + 2 * lane;
      if (KV_BF16) {
        const uint32_t kb = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.k_cache) + off);
        const uint32_t vb = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.v_cache) + off);
        kk = make_float2(__uint_as_float(kb << 16), __uint_as_float(kb & 0xFFFF0000u));
        vv = make_float2(__uint_as_float(vb << 16), __uint_as_float(vb & 0xFFFF0000u));
      } else {
        kk = *reinterpret_cast<const float2*>(static_cast<const float*>(p.k_cache) + off);
        vv = *reinterpret_cast<const float2*>(static_cast<const float*>(p.v_cache) + off);
      }
    }
#pragma unroll
    for (int j = 0; j < G; j++) {
      const float sc = wave_sum(q2[j].x * kk.x + q2[j].y * kk.y) * p.scale;
      const float mn = fmaxf(m[j], sc);
      const float co = expf(m[j] - mn), pe = expf(sc - mn);
      l[j] = l[j] * co + pe;
      acc[j].x = acc[j].x * co + pe * vv.x;
      acc[j].y = acc[j].y * co + pe * vv.y;
      m[j] = mn;
    }
  }

  // combine the 4 waves
#pragma unroll
  for (int j = 0; j < G; j++) {
    if (lane == 0) { wm[wave][j] = m[j]; wl[wave][j] = l[j]; }
    wacc[wave][j][2 * lane] = acc[j].x;
    wacc[wave][j][2 * lane + 1] = acc[j].y;
  }
  __syncthreads();
  const uint32_t nsplit_f = nsplit;
  float* part = p.partial + (size_t(g) * kAttnMaxSplits + s) * G * (2 + D);
  for (int i = tid; i < G * D; i += 256) {
    const int j = i / D, d = i % D;
    float M = -INFINITY;
    for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][j]);
    float L = 0.f, A = 0.f;
    for (int w = 0; w < 4; w++) {
      const float e = wm[w][j] == -INFINITY ? 0.f : expf(wm[w][j] - M);
      L += e * wl[w][j];
      A += e * wacc[w][j][d];
    }
    if (nsplit_f == 1) {
      p.att[(size_t(g) * G + j) * D + d] = A / L;
    } else {
      if (d == 0) { part[j * (2 + D)] = M; part[j * (2 + D) + 1] = L; }
      part[j * (2 + D) + 2 + d] = A;
    }
  }
  if (nsplit_f == 1) return;

  // last split to arrive merges (release/acquire through device-scope fences)
  __threadfence();
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(&p.counter[g], 1u) == nsplit_f - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* pg = p.partial + size_t(g) * kAttnMaxSplits * G * (2 + D);
  for (int i = tid; i < G * D; i += 256) {
    const int j = i / D, d = i % D;
    float M = -INFINITY;
    for (uint32_t q = 0; q < nsplit_f; q++) M = fmaxf(M, pg[(q * G + j) * (2 + D)]);
    float L = 0.f, A = 0.f;
    for (uint32_t q = 0; q < nsplit_f; q++) {
      const float* pq = pg + (q * G + j) * (2 + D);
      const float e = pq[0] == -INFINITY ? 0.f : expf(pq[0] - M);
      L += e * pq[1];
      A += e * pq[2 + d];
    }
    p.att[(size_t(g) * G + j) * D + d] = A / L;
  }
  if (tid == 0) atomicExch(&p.counter[g], 0u);
}

// ---------------------------------------------------------------------------------------------
// argmax over the per-workgroup candidates; first maximum wins; a NaN logits[0] gives 0 (the
// sequential scan of main.rs:37-42 can never move off index 0 then). Feeds the next step.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_argmax(const ArgCand* __restrict__ cand, uint32_t n_cand,
                                                 const float* __restrict__ logits, StepState* st,
                                                 uint32_t* tokens, uint32_t* host_tokens, uint32_t* err) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint32_t i = tid; i < n_cand; i += 1024) {
    const ArgCand c = cand[i];
    if (cand_better(c.v, c.i, bv, bi)) { bv = c.v; bi = c.i; }
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
    st->pos += 1;
    st->tok_idx = k;
  }
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

// rows per workgroup for a given chunks-per-lane
constexpr int rows_per_wave(int cpl, int epi) {
  return epi == kSiluPair ? (cpl <= 2 ? 4 : 2) : (cpl <= 1 ? 8 : cpl <= 2 ? 4 : cpl <= 4 ? 2 : 1);
}

template <int CPL, int PRO, int EPI>
hipError_t launch_mv(const MatvecParams& p, hipStream_t s) {
  constexpr int R = rows_per_wave(CPL, EPI);
  const uint32_t blocks = ceil_div(p.rows, 4u * R);
  hipLaunchKernelGGL((k_matvec<R, CPL, PRO, EPI>), dim3(blocks), dim3(256), size_t(p.cols) * 4, s, p);
  return hipGetLastError();
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

hipError_t launch_embed(const uint16_t* table, uint32_t hidden, uint32_t vocab, const uint32_t* tokens,
                        const StepState* st, float* x, uint32_t* err, hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3(ceil_div(hidden, 256)), dim3(256), 0, s, table, hidden, vocab, tokens, st, x, err);
  return hipGetLastError();
}

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
  return hipErrorInvalidValue;
}

hipError_t launch_attention(const AttnParams& p, uint32_t grid_splits, hipStream_t s) {
  const uint32_t G = p.n_kv ? p.n_heads / p.n_kv : 0;
  if (!p.n_kv || p.n_heads % p.n_kv || grid_splits == 0 || grid_splits > uint32_t(kAttnMaxSplits))
    return hipErrorInvalidValue;
  dim3 grid(p.n_kv, grid_splits);
#define QE_ATT(GG)                                                                     \
  if (G == GG) {                                                                       \
    if (p.kv_bf16) hipLaunchKernelGGL((k_attention<GG, true>), grid, dim3(256), 0, s, p);  \
    else hipLaunchKernelGGL((k_attention<GG, false>), grid, dim3(256), 0, s, p);           \
    return hipGetLastError();                                                          \
  }
  QE_ATT(1)
  QE_ATT(2)
  QE_ATT(4)
  QE_ATT(8)
#undef QE_ATT
  return hipErrorInvalidValue;
}

hipError_t launch_argmax(const ArgCand* cand, uint32_t n_cand, const float* logits, StepState* st, uint32_t* tokens,
                         uint32_t* host_tokens, uint32_t* err, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, cand, n_cand, logits, st, tokens, host_tokens, err);
  return hipGetLastError();
}

hipError_t launch_read_sum(const float* src, uint64_t n, float* partial, uint32_t grid, hipStream_t s) {
  if (n % 4 || grid == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_read_sum, dim3(grid), dim3(256), 0, s, reinterpret_cast<const float4*>(src), n / 4, partial);
  return hipGetLastError();
}

}  // namespace qe
