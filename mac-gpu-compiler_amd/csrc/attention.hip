// GQA decode attention for one new token (inference.metal:194-296, cpu_inference.rs:134-162).
//
// grid (n_kv, splits): one workgroup per (KV head, run of positions) serves all G q heads of
// that KV head from a single read of K and V. Lane l of a wave holds head dims (2l, 2l+1); wave w
// of NW takes positions t0 + w, t0 + w + NW, ... in batches of U whose K/V loads are all issued
// before any is used, with an online softmax (running max m, sum l, accumulator) per wave.
// With norm_rope, the workgroup first applies the per-head q RMSNorm and RoPE, and the workgroup
// whose run holds the new position also normalizes/rotates the new k and appends k and v to the
// cache (cpu_inference.rs:134-141). One split writes att directly; several splits write
// (m, l, acc) partials and the last split to finish merges them.
#include "kernels.h"

#include <cmath>

#include "device_common.h"

namespace qe {
namespace {

template <bool KV_BF16>
__device__ __forceinline__ void load_kv(const AttnParams& p, size_t off, float2& k, float2& v) {
  if (KV_BF16) {
    const uint32_t kb = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.k_cache) + off);
    const uint32_t vb = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.v_cache) + off);
    k = make_float2(__uint_as_float(kb << 16), __uint_as_float(kb & 0xFFFF0000u));
    v = make_float2(__uint_as_float(vb << 16), __uint_as_float(vb & 0xFFFF0000u));
  } else {
    k = *reinterpret_cast<const float2*>(static_cast<const float*>(p.k_cache) + off);
    v = *reinterpret_cast<const float2*>(static_cast<const float*>(p.v_cache) + off);
  }
}

template <int G>
__device__ __forceinline__ void online_update(const float2 (&q2)[G], float2 k, float2 v, float scale, float (&m)[G],
                                              float (&l)[G], float2 (&acc)[G]) {
#pragma unroll
  for (int j = 0; j < G; j++) {
    const float sc = wave_sum(q2[j].x * k.x + q2[j].y * k.y) * scale;  // dot(q, k) * scale
    const float mn = fmaxf(m[j], sc);
    const float co = expf(m[j] - mn), pe = expf(sc - mn);
    l[j] = l[j] * co + pe;
    acc[j].x = acc[j].x * co + pe * v.x;
    acc[j].y = acc[j].y * co + pe * v.y;
    m[j] = mn;
  }
}

template <int G, int NW, bool KV_BF16>
__global__ __launch_bounds__(NW * 64) void k_attention(AttnParams p, uint32_t chunk_min) {
  constexpr int D = kHeadDim, NT = NW * 64, U = 8;
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
  uint32_t nsplit = p.force_splits ? min(p.force_splits, gridDim.y) : min(gridDim.y, ceil_div(n, chunk_min));
  const uint32_t chunk = ceil_div(n, nsplit);
  nsplit = ceil_div(n, chunk);  // every split below nsplit starts before n
  const uint32_t s = blockIdx.y;
  if (s >= nsplit) return;
  const uint32_t t0 = s * chunk, t1 = min(n, t0 + chunk);
  const bool owns_new = p.norm_rope && t1 == n;
  // positions read from the cache; with owns_new the last one (pos) comes from LDS instead
  const uint32_t tc1 = owns_new ? t1 - 1 : t1;
  const size_t head_base = size_t(g) * p.max_seq * D;

  __shared__ float qs[G][D];
  __shared__ float knew[D], vnew[D], ktmp[D];
  __shared__ float wm[NW][G], wl[NW][G];
  __shared__ float wacc[NW][G][D];
  __shared__ int is_last;

  // the first K/V batch does not depend on q: issue it before the q/k prologue
  float2 kk[U], vv[U];
  uint32_t t = t0 + wave;
  bool preloaded = t + NW * (U - 1) < tc1;
  if (preloaded) {
#pragma unroll
    for (int u = 0; u < U; u++) load_kv<KV_BF16>(p, head_base + size_t(t + NW * u) * D + 2 * lane, kk[u], vv[u]);
  }

  for (int i = tid; i < G * D; i += NT) qs[i / D][i % D] = p.qkv[size_t(g) * G * D + i];
  __syncthreads();
  if (p.norm_rope) {
    for (int j = wave; j < G; j += NW) {
      const float a = qs[j][2 * lane], b = qs[j][2 * lane + 1];
      const float ssum = wave_sum(a * a + b * b);
      const float sc = 1.0f / sqrtf(ssum / float(D) + p.eps);
      qs[j][2 * lane] = a * sc * bf16f(p.q_norm[2 * lane]);
      qs[j][2 * lane + 1] = b * sc * bf16f(p.q_norm[2 * lane + 1]);
    }
    if (owns_new && wave == NW - 1) {
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
    // rotate-half RoPE from the table row of pos (metal_inference.rs:140-154)
    const float2* rope = reinterpret_cast<const float2*>(p.rope) + size_t(pos) * (D / 2);
    for (int i = tid; i < G * (D / 2); i += NT) {
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
        knew[tid] = bf16f(kb);  // attend with the values later steps read back
        vnew[tid] = bf16f(vb);
      } else {
        static_cast<float*>(p.k_cache)[slot] = knew[tid];
        static_cast<float*>(p.v_cache)[slot] = vnew[tid];
      }
    }
    __syncthreads();
  }

  float2 q2[G];
#pragma unroll
  for (int j = 0; j < G; j++) q2[j] = make_float2(qs[j][2 * lane], qs[j][2 * lane + 1]);
  float m[G], l[G];
  float2 acc[G];
#pragma unroll
  for (int j = 0; j < G; j++) { m[j] = -INFINITY; l[j] = 0.f; acc[j] = make_float2(0.f, 0.f); }

  for (; t + NW * (U - 1) < tc1; t += NW * U) {
    if (!preloaded) {
#pragma unroll
      for (int u = 0; u < U; u++) load_kv<KV_BF16>(p, head_base + size_t(t + NW * u) * D + 2 * lane, kk[u], vv[u]);
    }
    preloaded = false;
#pragma unroll
    for (int u = 0; u < U; u++) online_update<G>(q2, kk[u], vv[u], p.scale, m, l, acc);
  }
  for (; t < t1; t += NW) {
    float2 k1, v1;
    if (owns_new && t == tc1) {
      k1 = make_float2(knew[2 * lane], knew[2 * lane + 1]);
      v1 = make_float2(vnew[2 * lane], vnew[2 * lane + 1]);
    } else {
      load_kv<KV_BF16>(p, head_base + size_t(t) * D + 2 * lane, k1, v1);
    }
    online_update<G>(q2, k1, v1, p.scale, m, l, acc);
  }

  // combine the NW waves
#pragma unroll
  for (int j = 0; j < G; j++) {
    if (lane == 0) { wm[wave][j] = m[j]; wl[wave][j] = l[j]; }
    wacc[wave][j][2 * lane] = acc[j].x;
    wacc[wave][j][2 * lane + 1] = acc[j].y;
  }
  __syncthreads();
  float* part = p.partial + (size_t(g) * kAttnMaxSplits + s) * G * (2 + D);
  for (int i = tid; i < G * D; i += NT) {
    const int j = i / D, d = i % D;
    float M = -INFINITY;
    for (int w = 0; w < NW; w++) M = fmaxf(M, wm[w][j]);
    float L = 0.f, A = 0.f;
    for (int w = 0; w < NW; w++) {
      const float e = wm[w][j] == -INFINITY ? 0.f : expf(wm[w][j] - M);  // a wave with no positions adds 0
      L += e * wl[w][j];
      A += e * wacc[w][j][d];
    }
    if (nsplit == 1) {
      p.att[(size_t(g) * G + j) * D + d] = A / L;
    } else {
      if (d == 0) { part[j * (2 + D)] = M; part[j * (2 + D) + 1] = L; }
      part[j * (2 + D) + 2 + d] = A;
    }
  }
  if (nsplit == 1) return;

  // the last split to arrive merges (release/acquire through device-scope fences)
  __threadfence();
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(&p.counter[g], 1u) == nsplit - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* pg = p.partial + size_t(g) * kAttnMaxSplits * G * (2 + D);
  for (int i = tid; i < G * D; i += NT) {
    const int j = i / D, d = i % D;
    float M = -INFINITY;
    for (uint32_t q = 0; q < nsplit; q++) M = fmaxf(M, pg[(q * G + j) * (2 + D)]);
    float L = 0.f, A = 0.f;
    for (uint32_t q = 0; q < nsplit; q++) {
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
// Decode-step attention over a fixed split of the cache: workgroup (g, s) covers positions
// [s*chunk, (s+1)*chunk) of KV head g, in tiles of 64 positions:
//   scores: lane j of every wave takes position tile+j; wave w multiplies head dims
//           [32w, 32w+32) (eight 16-byte K loads per lane), partial dots meet in LDS;
//   softmax: wave h reduces head h's 64 scores once per tile (max, exp, sum) -- no per-position
//            cross-lane reduction;
//   PV:     thread (d, half) accumulates dim d over its half of the tile for all G heads, with V
//           loaded in the same batch as K.
// The workgroup writes its (m, l, acc) partial per q head; runs past pos write m = -inf.
// The o_proj matvec merges the partials in its prologue (kAttnMerge).
// ---------------------------------------------------------------------------------------------
template <int G, bool KV_BF16>
__global__ __launch_bounds__(256) void k_attn_split(AttnParams p, uint32_t chunk) {
  constexpr int D = kHeadDim, T = 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t g = blockIdx.x, s = blockIdx.y;
  float* part = p.partial + (size_t(g) * gridDim.y + s) * G * kPartStride;
  const uint32_t pos = p.state->pos;
  if (pos >= p.max_seq) {
    if (g == 0 && s == 0 && tid == 0) atomicOr(p.err, kErrPos);
    return;
  }
  const uint32_t n = pos + 1, t0 = s * chunk;
  if (t0 >= n) {  // nothing cached here yet: an empty partial
    if (tid < G) { part[tid * kPartStride] = -INFINITY; part[tid * kPartStride + 1] = 0.f; }
    return;
  }
  const uint32_t t1 = min(n, t0 + chunk);
  const bool owns_new = t1 == n;
  const size_t head_base = size_t(g) * p.max_seq * D;

  __shared__ float qs[G][D];
  __shared__ float knew[D], vnew[D], ktmp[D];
  __shared__ float sp[4][G][T];
  __shared__ float pes[G][T];
  __shared__ float Ms[G], Ls[G], Cs[G];
  __shared__ float accx[G][D];

  // ---- q/k RMSNorm + RoPE, K/V append (cpu_inference.rs:134-141) ----
  for (int i = tid; i < G * D; i += 256) qs[i / D][i % D] = p.qkv[size_t(g) * G * D + i];
  if (tid < G) { Ms[tid] = -INFINITY; Ls[tid] = 0.f; }
  __syncthreads();
  for (int j = wave; j < G; j += 4) {
    const float a = qs[j][2 * lane], b = qs[j][2 * lane + 1];
    const float ssum = wave_sum(a * a + b * b);
    const float sc = 1.0f / sqrtf(ssum / float(D) + p.eps);
    qs[j][2 * lane] = a * sc * bf16f(p.q_norm[2 * lane]);
    qs[j][2 * lane + 1] = b * sc * bf16f(p.q_norm[2 * lane + 1]);
  }
  if (owns_new && wave == 3) {
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
    const size_t slot = head_base + size_t(pos) * D + tid;
    if (KV_BF16) {
      const uint16_t kb = f32_to_bf16(knew[tid]), vb = f32_to_bf16(vnew[tid]);
      static_cast<uint16_t*>(p.k_cache)[slot] = kb;
      static_cast<uint16_t*>(p.v_cache)[slot] = vb;
      knew[tid] = bf16f(kb);  // attend with the values later steps read back
      vnew[tid] = bf16f(vb);
    } else {
      static_cast<float*>(p.k_cache)[slot] = knew[tid];
      static_cast<float*>(p.v_cache)[slot] = vnew[tid];
    }
  }
  __syncthreads();

  const int d = tid & (D - 1), half = tid >> 7;
  float acc[G];
#pragma unroll
  for (int j = 0; j < G; j++) acc[j] = 0.f;

  for (uint32_t tile = t0; tile < t1; tile += T) {
    const uint32_t tl = min(uint32_t(T), t1 - tile);
    // K: lane -> position tile + lane, wave -> dims [32 wave, 32 wave + 32)
    const uint32_t tk0 = tile + lane;
    const bool k_cached = lane < int(tl) && !(owns_new && tk0 == pos);
    const uint32_t tk = k_cached ? tk0 : t0;  // lanes without a cached position address a valid row
    float4 kr[8];
    if (KV_BF16) {
      const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.k_cache) + head_base + size_t(tk) * D + 32 * wave);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint4 u = k_cached ? src[i] : make_uint4(0, 0, 0, 0);
        kr[2 * i] = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u),
                                __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xFFFF0000u));
        kr[2 * i + 1] = make_float4(__uint_as_float(u.z << 16), __uint_as_float(u.z & 0xFFFF0000u),
                                    __uint_as_float(u.w << 16), __uint_as_float(u.w & 0xFFFF0000u));
      }
    } else {
      const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(p.k_cache) + head_base + size_t(tk) * D + 32 * wave);
#pragma unroll
      for (int i = 0; i < 8; i++) kr[i] = k_cached ? src[i] : make_float4(0, 0, 0, 0);
    }
    // V: thread (d, half) -> positions tile + 32 half + i
    float vr[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const uint32_t tv = tile + 32 * half + i;
      const bool v_cached = 32 * half + i < int(tl) && !(owns_new && tv == pos);
      const size_t off = head_base + size_t(v_cached ? tv : t0) * D + d;
      if (KV_BF16) vr[i] = v_cached ? bf16f(static_cast<const uint16_t*>(p.v_cache)[off]) : 0.f;
      else vr[i] = v_cached ? static_cast<const float*>(p.v_cache)[off] : 0.f;
      if (owns_new && tv == pos) vr[i] = vnew[d];
    }
    if (owns_new && tk0 == pos) {
#pragma unroll
      for (int i = 0; i < 8; i++)
        kr[i] = make_float4(knew[32 * wave + 4 * i], knew[32 * wave + 4 * i + 1], knew[32 * wave + 4 * i + 2], knew[32 * wave + 4 * i + 3]);
    }
#pragma unroll
    for (int j = 0; j < G; j++) {
      float sdot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float4 q4 = *reinterpret_cast<const float4*>(&qs[j][32 * wave + 4 * i]);
        sdot += kr[i].x * q4.x + kr[i].y * q4.y + kr[i].z * q4.z + kr[i].w * q4.w;
      }
      sp[wave][j][lane] = sdot;
    }
    __syncthreads();
    for (int j = wave; j < G; j += 4) {
      const bool valid = lane < int(tl);
      const float sc = valid ? ((sp[0][j][lane] + sp[1][j][lane]) + (sp[2][j][lane] + sp[3][j][lane])) * p.scale : -INFINITY;
      const float m_old = Ms[j];
      const float m_new = fmaxf(m_old, wave_max(sc));
      const float pe = valid ? expf(sc - m_new) : 0.f;
      const float tsum = wave_sum(pe);
      const float c = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
      pes[j][lane] = pe;
      if (lane == 0) { Ls[j] = Ls[j] * c + tsum; Ms[j] = m_new; Cs[j] = c; }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < G; j++) {
      float a = acc[j] * Cs[j];
#pragma unroll
      for (int i = 0; i < 32; i++) a += pes[j][32 * half + i] * vr[i];
      acc[j] = a;
    }
    __syncthreads();  // sp / pes / Cs are rewritten by the next tile
  }

  // the two halves of the tile meet; half 0 writes the partial
  if (half == 1) {
#pragma unroll
    for (int j = 0; j < G; j++) accx[j][d] = acc[j];
  }
  __syncthreads();
  if (half == 0) {
#pragma unroll
    for (int j = 0; j < G; j++) {
      part[j * kPartStride + 4 + d] = acc[j] + accx[j][d];
      if (d == 0) { part[j * kPartStride] = Ms[j]; part[j * kPartStride + 1] = Ls[j]; }
    }
  }
}

template <int NW>
hipError_t launch_nw(const AttnParams& p, uint32_t grid_splits, uint32_t chunk_min, hipStream_t s) {
  const uint32_t G = p.n_heads / p.n_kv;
  dim3 grid(p.n_kv, grid_splits);
#define QE_ATT(GG)                                                                                       \
  if (G == GG) {                                                                                         \
    if (p.kv_bf16) hipLaunchKernelGGL((k_attention<GG, NW, true>), grid, dim3(NW * 64), 0, s, p, chunk_min);  \
    else hipLaunchKernelGGL((k_attention<GG, NW, false>), grid, dim3(NW * 64), 0, s, p, chunk_min);           \
    return hipGetLastError();                                                                            \
  }
  QE_ATT(1)
  QE_ATT(2)
  QE_ATT(4)
  QE_ATT(8)
#undef QE_ATT
  return hipErrorInvalidValue;
}

bool attn_args_ok(const AttnParams& p, uint32_t grid_splits) {
  if (!p.n_kv || p.n_heads % p.n_kv) return false;
  const uint32_t G = p.n_heads / p.n_kv;
  return (G == 1 || G == 2 || G == 4 || G == 8) && grid_splits > 0 && grid_splits <= uint32_t(kAttnMaxSplits);
}

}  // namespace

// 4-wave workgroups, splits of at least kAttnMinChunk positions (the isolated op's default)
hipError_t launch_attention(const AttnParams& p, uint32_t grid_splits, hipStream_t s) {
  if (!attn_args_ok(p, grid_splits)) return hipErrorInvalidValue;
  return launch_nw<4>(p, grid_splits, kAttnMinChunk, s);
}

hipError_t launch_attention_split(const AttnParams& p, uint32_t splits, uint32_t chunk, hipStream_t s) {
  if (!attn_args_ok(p, splits) || splits > uint32_t(kAttnMaxMergeSplits) || chunk == 0 || !p.norm_rope)
    return hipErrorInvalidValue;
  const uint32_t G = p.n_heads / p.n_kv;
  dim3 grid(p.n_kv, splits);
#define QE_ATT(GG)                                                                                   \
  if (G == GG) {                                                                                     \
    if (p.kv_bf16) hipLaunchKernelGGL((k_attn_split<GG, true>), grid, dim3(256), 0, s, p, chunk);   \
    else hipLaunchKernelGGL((k_attn_split<GG, false>), grid, dim3(256), 0, s, p, chunk);            \
    return hipGetLastError();                                                                        \
  }
  QE_ATT(1)
  QE_ATT(2)
  QE_ATT(4)
  QE_ATT(8)
#undef QE_ATT
  return hipErrorInvalidValue;
}

// 16-wave workgroups (fewer for wide GQA groups, to bound LDS), splits of kAttnBlockPositions:
// a single workgroup per KV head up to 512 positions, so no merge round trip at short context
hipError_t launch_attention_wide(const AttnParams& p, uint32_t grid_splits, hipStream_t s) {
  if (!attn_args_ok(p, grid_splits)) return hipErrorInvalidValue;
  const uint32_t G = p.n_heads / p.n_kv;
  if (G <= 2) return launch_nw<16>(p, grid_splits, kAttnBlockPositions, s);
  if (G == 4) return launch_nw<8>(p, grid_splits, kAttnBlockPositions, s);
  return launch_nw<4>(p, grid_splits, kAttnBlockPositions, s);
}

}  // namespace qe
