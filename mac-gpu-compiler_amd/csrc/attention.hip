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
// [s*chunk, (s+1)*chunk) of KV head g, in tiles of T = 64 positions, for all G q heads of g.
// Every global load of a tile is issued before any of its values is used, and no load sits
// behind a divergent branch (the compiler waits for such a load on the spot): positions past
// the run or the cache are clamped to a valid row and masked where the values are consumed.
// The first tile, the q/k/v rows, the norm gains and the RoPE row of the current position
// (rope_cur, advanced by k_argmax) do not depend on pos, so they are in flight together with
// the read of pos itself.
//   prologue: wave w prepares rows w, w+4, ... of [q_0 .. q_{G-1}, k_new, v_new]; lane l holds
//             dims l and l+64, the pair RoPE rotates together (cpu_inference.rs:134-141)
//   scores:   thread (pg = tid/8, dc = tid%8) takes positions tile+pg and tile+pg+32 over dims
//             [16dc, 16dc+16); the 8 lanes of a position meet through DPP
//   softmax:  wave j reduces head j's 64 scores once per tile (online max, exp, sum)
//   PV:       thread (dg = tid%32, pp = tid/32) accumulates dims [4dg, 4dg+4) over positions
//             tile+8pp .. tile+8pp+7; the 8 position groups meet in LDS at the end
// The workgroup writes its (m, l, acc) partial per q head; a run past pos writes an empty one
// (m = -inf, l = 0, acc = 0). The o_proj matvec merges the partials in its prologue.
// ---------------------------------------------------------------------------------------------
template <bool KV_BF16>
struct KVTile;
template <>
struct KVTile<false> {
  float4 k[2][4];  // scores layout: 2 positions x 16 dims
  float4 v[8];     // PV layout: 8 positions x 4 dims
};
template <>
struct KVTile<true> {
  uint4 k[2][2];
  uint2 v[8];
};

// component-wise select (a ternary on float4 objects selects between their addresses, which
// keeps them out of registers)
__device__ __forceinline__ float4 sel4(bool c, float4 a, float4 b) {
  return make_float4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

__device__ __forceinline__ float4 bf16x4(uint32_t a, uint32_t b) {
  return make_float4(__uint_as_float(a << 16), __uint_as_float(a & 0xFFFF0000u), __uint_as_float(b << 16),
                     __uint_as_float(b & 0xFFFF0000u));
}

// K/V rows of positions tile.. in this thread's two layouts; rows past the cache end are clamped
template <bool KV_BF16>
__device__ __forceinline__ void load_tile(KVTile<KV_BF16>& X, const AttnParams& p, size_t head_base, uint32_t tile,
                                          int tid) {
  constexpr int D = kHeadDim;
  const uint32_t last = p.max_seq - 1;
  const int pg = tid >> 3, dc = tid & 7, dg = tid & 31, pp = tid >> 5;
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const size_t row = head_base + size_t(min(tile + uint32_t(pg + 32 * u), last)) * D + 16 * dc;
    if constexpr (KV_BF16) {
      const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.k_cache) + row);
      X.k[u][0] = src[0];
      X.k[u][1] = src[1];
    } else {
      const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(p.k_cache) + row);
#pragma unroll
      for (int i = 0; i < 4; i++) X.k[u][i] = src[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const size_t row = head_base + size_t(min(tile + uint32_t(8 * pp + i), last)) * D + 4 * dg;
    if constexpr (KV_BF16) {
      X.v[i] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.v_cache) + row);
    } else {
      X.v[i] = *reinterpret_cast<const float4*>(static_cast<const float*>(p.v_cache) + row);
    }
  }
}

template <bool KV_BF16>
__device__ __forceinline__ void tile_k(const KVTile<KV_BF16>& X, int u, float4 (&k4)[4]) {
  if constexpr (KV_BF16) {
    k4[0] = bf16x4(X.k[u][0].x, X.k[u][0].y);
    k4[1] = bf16x4(X.k[u][0].z, X.k[u][0].w);
    k4[2] = bf16x4(X.k[u][1].x, X.k[u][1].y);
    k4[3] = bf16x4(X.k[u][1].z, X.k[u][1].w);
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) k4[i] = X.k[u][i];
  }
}

template <bool KV_BF16>
__device__ __forceinline__ float4 tile_v(const KVTile<KV_BF16>& X, int i) {
  if constexpr (KV_BF16) {
    return bf16x4(X.v[i].x, X.v[i].y);
  } else {
    return X.v[i];
  }
}

template <int G, bool KV_BF16>
__global__ __launch_bounds__(256) void k_attn_split(AttnParams p, uint32_t chunk) {
  constexpr int D = kHeadDim, T = 64, NR = G + 2, RPW = (NR + 3) / 4;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, so branches on it are scalar
  const int pg = tid >> 3, dc = tid & 7, dg = tid & 31, pp = tid >> 5;
  const uint32_t g = blockIdx.x, s = blockIdx.y, t0 = s * chunk;
  const size_t head_base = size_t(g) * p.max_seq * D;

  __shared__ __align__(16) float qs[G][D];
  __shared__ __align__(16) float knew[D];
  __shared__ __align__(16) float vnew[D];
  __shared__ float sc[G][T], pes[G][T];
  __shared__ float Ms[G], Ls[G], Cs[G];
  __shared__ __align__(16) float red[8][G][D];

  // ---- loads that do not depend on pos (no early exit follows them: the compiler would sink a
  // load that an exit path does not use past the exit test, behind the read of pos) ----
  float ra[RPW], rb[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const int r = min(wave + 4 * i, NR - 1);
    const size_t off = r < G ? (size_t(g) * G + r) * D
                             : size_t(p.n_heads) * D + (r == G ? 0 : size_t(p.n_kv) * D) + size_t(g) * D;
    ra[i] = p.qkv[off + lane];
    rb[i] = p.qkv[off + lane + 64];
  }
  const float gqa = bf16f(p.q_norm[lane]), gqb = bf16f(p.q_norm[lane + 64]);
  const float gka = bf16f(p.k_norm[lane]), gkb = bf16f(p.k_norm[lane + 64]);
  const float2 cs = reinterpret_cast<const float2*>(p.rope_cur)[lane];
  KVTile<KV_BF16> A, B;
  load_tile<KV_BF16>(A, p, head_base, t0, tid);
  __builtin_amdgcn_sched_barrier(0);  // keep the scheduler from sinking these loads to their uses

  const uint32_t pos = p.state->pos;
  const bool bad = pos >= p.max_seq;
  if (bad && g == 0 && s == 0 && tid == 0) atomicOr(p.err, kErrPos);
  // a run with no cached position (t1 <= t0) goes through one all-masked tile and writes the
  // empty partial m = -inf, l = 0, acc = 0
  const uint32_t n = bad ? 0u : pos + 1;
  const uint32_t t1 = min(n, t0 + chunk);
  const bool owns_new = !bad && pos >= t0 && pos < t0 + chunk;  // this run holds the new position
  float* part = p.partial + (size_t(g) * gridDim.y + s) * G * kPartStride;

  // ---- q/k RMSNorm (cpu_inference.rs:189-194) + rotate-half RoPE (cpu_inference.rs:203-215) ----
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const int r = wave + 4 * i;
    if (r < NR) {
      float a = ra[i], b = rb[i];
      if (r <= G) {
        const float ss = wave_sum(a * a + b * b);
        const float scl = 1.0f / sqrtf(ss / float(D) + p.eps);
        a = a * scl * (r < G ? gqa : gka);
        b = b * scl * (r < G ? gqb : gkb);
        const float ar = a * cs.x - b * cs.y, br = b * cs.x + a * cs.y;
        a = ar;
        b = br;
      }
      if (KV_BF16 && r >= G) {  // attend with the values later steps read back
        a = bf16f(f32_to_bf16(a));
        b = bf16f(f32_to_bf16(b));
      }
      float* dst = r < G ? qs[r] : (r == G ? knew : vnew);
      dst[lane] = a;
      dst[lane + 64] = b;
    }
  }
  if (tid < G) { Ms[tid] = -INFINITY; Ls[tid] = 0.f; }
  __syncthreads();
  if (owns_new) {  // append the new K/V row (cpu_inference.rs:140-141)
    const size_t slot = head_base + size_t(pos) * D + (tid & (D - 1));
    const float val = tid < D ? knew[tid] : vnew[tid - D];
    void* cache = tid < D ? p.k_cache : p.v_cache;
    if (KV_BF16) static_cast<uint16_t*>(cache)[slot] = f32_to_bf16(val);
    else static_cast<float*>(cache)[slot] = val;
  }

  float4 acc[G];
#pragma unroll
  for (int j = 0; j < G; j++) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);

  auto process = [&](const KVTile<KV_BF16>& X, uint32_t tile) __attribute__((always_inline)) {
    // scores s_t = (q . k_t) * scale (cpu_inference.rs:144-152); the new position's k is knew
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const uint32_t t = tile + uint32_t(pg + 32 * u);
      float4 k4[4];
      tile_k<KV_BF16>(X, u, k4);
      const bool sub = owns_new && t == pos;
      const float4* kn = reinterpret_cast<const float4*>(knew) + 4 * dc;
#pragma unroll
      for (int i = 0; i < 4; i++) k4[i] = sel4(sub, kn[i], k4[i]);
      float sv[G];
#pragma unroll
      for (int j = 0; j < G; j++) {
        const float4* qj = reinterpret_cast<const float4*>(qs[j]) + 4 * dc;
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float4 qv = qj[i];
          d += k4[i].x * qv.x + k4[i].y * qv.y + k4[i].z * qv.z + k4[i].w * qv.w;
        }
        sv[j] = sum8(d);
      }
      if (dc == 0) {
#pragma unroll
        for (int j = 0; j < G; j++) sc[j][pg + 32 * u] = t < t1 ? sv[j] * p.scale : -INFINITY;
      }
    }
    __syncthreads();
    // softmax (cpu_inference.rs:217-223) as an online update: running max, rescaled sum
    for (int j = wave; j < G; j += 4) {
      const float x = sc[j][lane];
      const float m_old = Ms[j];
      const float m_new = fmaxf(m_old, wave_max(x));
      const float pe = x == -INFINITY ? 0.f : expf(x - m_new);
      const float c = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
      const float tsum = wave_sum(pe);
      pes[j][lane] = pe;
      if (lane == 0) { Ls[j] = Ls[j] * c + tsum; Ms[j] = m_new; Cs[j] = c; }
    }
    __syncthreads();
    // out += p_t * v_t (cpu_inference.rs:153-160); positions past the run add 0
    float4 v4[8];
    const float4 vn = reinterpret_cast<const float4*>(vnew)[dg];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t t = tile + uint32_t(8 * pp + i);
      v4[i] = sel4(owns_new && t == pos, vn, tile_v<KV_BF16>(X, i));
      v4[i] = sel4(t < t1, v4[i], make_float4(0.f, 0.f, 0.f, 0.f));
    }
#pragma unroll
    for (int j = 0; j < G; j++) {
      const float c = Cs[j];
      float4 a = make_float4(acc[j].x * c, acc[j].y * c, acc[j].z * c, acc[j].w * c);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float pe = pes[j][8 * pp + i];
        a.x += pe * v4[i].x;
        a.y += pe * v4[i].y;
        a.z += pe * v4[i].z;
        a.w += pe * v4[i].w;
      }
      acc[j] = a;
    }
  };

  // tiles alternate between two register sets, so the next tile's loads are in flight while
  // this one is computed (sc / pes / Cs are only rewritten after the next tile's first barrier)
  for (uint32_t tile = t0;; tile += 2 * T) {
    const bool more = tile + T < t1;
    if (more) load_tile<KV_BF16>(B, p, head_base, tile + T, tid);
    __builtin_amdgcn_sched_barrier(0);
    process(A, tile);
    if (!more) break;
    const bool more2 = tile + 2 * T < t1;
    if (more2) load_tile<KV_BF16>(A, p, head_base, tile + 2 * T, tid);
    __builtin_amdgcn_sched_barrier(0);
    process(B, tile + T);
    if (!more2) break;
  }

  // the 8 position groups meet; m and l are the softmax state
#pragma unroll
  for (int j = 0; j < G; j++) reinterpret_cast<float4*>(red[pp][j])[dg] = acc[j];
  __syncthreads();
  for (int o = tid; o < G * D; o += 256) {
    const int j = o / D, d = o % D;
    float a = 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) a += red[q][j][d];
    part[j * kPartStride + 4 + d] = a;
    if (d == 0) { part[j * kPartStride] = Ms[j]; part[j * kPartStride + 1] = Ls[j]; }
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
  if (!attn_args_ok(p, splits) || splits > uint32_t(kAttnMaxMergeSplits) || chunk == 0 || !p.norm_rope ||
      !p.rope_cur || uint64_t(splits) * chunk < p.max_seq)
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
