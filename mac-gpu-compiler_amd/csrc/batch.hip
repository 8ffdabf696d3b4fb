// Multi-token forward (chunked prefill and k-token verify) on bf16 MFMA.
//
// The reference runs its prompt one token at a time (metal_infrence_engine/src/bin/bench.rs:174-176
// calls forward per position); these kernels run a chunk of M tokens through a layer at once, so
// every weight is read once per chunk and the projections become GEMMs on the matrix cores:
//   rownorm        s[m] = 1/sqrt(mean(x_m^2) + eps)                  (cpu_inference.rs:189-194)
//   k_gemm         C[m][n] = sum_k A'[m][k] W[n][k], A' = f32 A (x s[m] x gain[k] with a norm),
//                  split into hi + lo bf16 so the products keep ~16 mantissa bits; epilogues
//                  store / residual add / silu(gate)*up                 (cpu_inference.rs:225-257)
//   k_qk_rope      per token and head: q/k RMSNorm + RoPE, K/V append   (cpu_inference.rs:134-141)
//   k_attn_causal  token m attends positions 0..start+m               (cpu_inference.rs:144-162)
#include "batch.h"

#include <algorithm>
#include <cmath>

#include "device_common.h"

namespace qe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// f32 -> bf16 bits, round to nearest even (NaN kept quiet)
__device__ __forceinline__ uint32_t bf16_bits(float f) { return f32_to_bf16(f); }

// 8 floats -> (hi, lo) bf16x8 with hi = bf16(v), lo = bf16(v - hi)
__device__ __forceinline__ void split8(const float (&v)[8], bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t h0 = bf16_bits(v[2 * e]), h1 = bf16_bits(v[2 * e + 1]);
    const float r0 = v[2 * e] - __uint_as_float(h0 << 16), r1 = v[2 * e + 1] - __uint_as_float(h1 << 16);
    h[e] = h0 | (h1 << 16);
    l[e] = bf16_bits(r0) | (bf16_bits(r1) << 16);
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

// ---------------------------------------------------------------------------------------------
// s[m] = 1 / sqrt(mean_k x[m][k]^2 + eps): one wave per row
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rownorm(const float* __restrict__ x, uint32_t M, uint32_t K, float eps,
                                                 float* __restrict__ s) {
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const float4* xr = reinterpret_cast<const float4*>(x + size_t(row) * K);
  float acc = 0.f;
  for (uint32_t i = lane; i < K / 4; i += 64) {
    const float4 v = xr[i];
    acc += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
  }
  acc = wave_sum(acc);
  if (lane == 0) s[row] = 1.0f / sqrtf(acc / float(K) + eps);
}

// ---------------------------------------------------------------------------------------------
// GEMM C = A' W^T on v_mfma_f32_16x16x32_bf16. Workgroup tile 64 (m) x 64 (n), 4 waves; wave w
// owns rows [16w, 16w+16) of the tile and all four 16-column blocks. Per 32-wide k step, lane l
// loads row (l % 16) of its A block at k = 8 (l / 16) .. +7 (two float4) and the same k range of
// W rows n0 + 16 j + (l % 16) (one 16-byte load per block), all straight from global memory,
// four k steps per iteration (the next iteration's loads are issued before this one's MFMAs);
// A is split into hi + lo bf16 and
// both halves multiply the same W fragment. Output lane layout: rows 4 (l / 16) + r, column l % 16.
// Rows past M and columns past N are clamped on load and skipped on store.
// ---------------------------------------------------------------------------------------------
template <bool NORM, int EPI, int KU>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kg = lane >> 4;
  const uint32_t m0 = blockIdx.y * 64 + wave * 16, n0 = blockIdx.x * 64;
  const uint32_t arow = min(m0 + uint32_t(li), p.M - 1);
  const float* Ar = p.A + size_t(arow) * p.lda;
  const float rs = NORM ? p.rowscale[arow] : 1.0f;
  const uint16_t* Wr[4];
#pragma unroll
  for (int j = 0; j < 4; j++) Wr[j] = p.W + size_t(min(n0 + 16 * j + li, p.N - 1)) * p.K;  // rows past N clamped

  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // KU k-steps of 32 per iteration, held in registers; the next iteration's are loaded before
  // this one's MFMAs issue
  float4 a0[KU], a1[KU];
  uint4 g[KU], w[KU][4];
  auto load = [&](uint32_t k0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const uint32_t k = k0 + 32 * u + 8 * kg;
      a0[u] = *reinterpret_cast<const float4*>(Ar + k);
      a1[u] = *reinterpret_cast<const float4*>(Ar + k + 4);
      if constexpr (NORM) g[u] = *reinterpret_cast<const uint4*>(p.gain + k);
#pragma unroll
      for (int j = 0; j < 4; j++) w[u][j] = *reinterpret_cast<const uint4*>(Wr[j] + k);
    }
  };
  load(0);
  for (uint32_t k0 = 0; k0 < p.K; k0 += 32 * KU) {
    bf16x8 hi[KU], lo[KU];
    uint4 wc[KU][4];
#pragma unroll
    for (int u = 0; u < KU; u++) {
      float v[8] = {a0[u].x, a0[u].y, a0[u].z, a0[u].w, a1[u].x, a1[u].y, a1[u].z, a1[u].w};
      if constexpr (NORM) {
        const uint32_t gg[4] = {g[u].x, g[u].y, g[u].z, g[u].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[2 * e] = (v[2 * e] * rs) * __uint_as_float(gg[e] << 16);
          v[2 * e + 1] = (v[2 * e + 1] * rs) * __uint_as_float(gg[e] & 0xFFFF0000u);
        }
      }
      split8(v, hi[u], lo[u]);
#pragma unroll
      for (int j = 0; j < 4; j++) wc[u][j] = w[u][j];
    }
    if (k0 + 32 * KU < p.K) load(k0 + 32 * KU);
#pragma unroll
    for (int u = 0; u < KU; u++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const bf16x8 b = __builtin_bit_cast(bf16x8, u32x4{wc[u][j].x, wc[u][j].y, wc[u][j].z, wc[u][j].w});
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi[u], b, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo[u], b, acc[j], 0, 0, 0);
      }
    }
  }

  // epilogue: lane holds C[m0 + 4 kg + r][n0 + 16 j + li]
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t n = n0 + 16 * j + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t m = m0 + 4 * kg + r;
      const float c = acc[j][r];
      if constexpr (EPI == kGemmSiluPair) {
        // columns 2i (gate) and 2i+1 (up) sit in neighbouring lanes (cpu_inference.rs:170)
        const float up = __shfl_xor(c, 1);
        if (m < p.M && n < p.N && (li & 1) == 0) p.C[size_t(m) * p.ldc + (n >> 1)] = c / (1.0f + expf(-c)) * up;
      } else if constexpr (EPI == kGemmResAdd) {
        if (m < p.M && n < p.N) p.C[size_t(m) * p.ldc + n] += c;
      } else {
        if (m < p.M && n < p.N) p.C[size_t(m) * p.ldc + n] = c;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Skinny GEMM for M <= 16 MT rows (verify, the last chunk of a prefill): the weights are the
// whole cost, so the work is spread over K as well as N. Workgroup = NW waves on 16 columns
// n0 .. n0+15; wave w covers the k steps [w KPW, (w+1) KPW) with KPW = ceil(K / 32 / NW), two
// per iteration (loads clamped to the last step, steps past the range masked by a zero W
// fragment), MT m-tiles per W fragment, A split hi + lo as in k_gemm. The NW partial tiles are
// summed in LDS in wave order. With the norm, each lane also sums x^2 of its row over the
// steps it loads, so C = s[m] sum_k (x g)[m][k] W[n][k] with s[m] = 1 / sqrt(mean x^2 + eps)
// (the scale applied after the sum, a reassociation of the reference's f32 product).
// ---------------------------------------------------------------------------------------------
template <bool NORM, int EPI, int MT, int NW>
__global__ __launch_bounds__(64 * NW) void k_gemm_skinny(GemmParams p) {
  constexpr int KU = 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kg = lane >> 4;
  const uint32_t n0 = blockIdx.x * 16;
  const uint32_t KS = p.K / 32, KPW = (KS + NW - 1) / NW, s0 = uint32_t(wave) * KPW;
  const uint16_t* Wr = p.W + size_t(min(n0 + uint32_t(li), p.N - 1)) * p.K;
  const float* Ar[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) Ar[t] = p.A + size_t(min(uint32_t(16 * t + li), p.M - 1)) * p.lda;

  f32x4 acc[MT];
  float ss[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) {
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    ss[t] = 0.f;
  }
  float4 a0[KU][MT], a1[KU][MT];
  uint4 g[KU], w[KU];
  auto load = [&](uint32_t it) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const uint32_t k = 32 * min(s0 + it + uint32_t(u), KS - 1) + 8 * kg;
      w[u] = *reinterpret_cast<const uint4*>(Wr + k);
#pragma unroll
      for (int t = 0; t < MT; t++) {
        a0[u][t] = *reinterpret_cast<const float4*>(Ar[t] + k);
        a1[u][t] = *reinterpret_cast<const float4*>(Ar[t] + k + 4);
      }
      if constexpr (NORM) g[u] = *reinterpret_cast<const uint4*>(p.gain + k);
    }
  };
  load(0);
  for (uint32_t it = 0; it < KPW; it += KU) {
    bf16x8 hi[KU][MT], lo[KU][MT];
    uint4 wc[KU];
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const bool ok = it + u < KPW && s0 + it + u < KS;
      wc[u] = make_uint4(ok ? w[u].x : 0u, ok ? w[u].y : 0u, ok ? w[u].z : 0u, ok ? w[u].w : 0u);
#pragma unroll
      for (int t = 0; t < MT; t++) {
        float v[8] = {a0[u][t].x, a0[u][t].y, a0[u][t].z, a0[u][t].w,
                      a1[u][t].x, a1[u][t].y, a1[u][t].z, a1[u][t].w};
        if constexpr (NORM) {
          float q = 0.f;
#pragma unroll
          for (int e = 0; e < 8; e++) q += v[e] * v[e];
          ss[t] += ok ? q : 0.f;
          const uint32_t gg[4] = {g[u].x, g[u].y, g[u].z, g[u].w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            v[2 * e] *= __uint_as_float(gg[e] << 16);
            v[2 * e + 1] *= __uint_as_float(gg[e] & 0xFFFF0000u);
          }
        }
        split8(v, hi[u][t], lo[u][t]);
      }
    }
    if (it + KU < KPW) load(it + KU);
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const bf16x8 b = __builtin_bit_cast(bf16x8, u32x4{wc[u].x, wc[u].y, wc[u].z, wc[u].w});
#pragma unroll
      for (int t = 0; t < MT; t++) {
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi[u][t], b, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo[u][t], b, acc[t], 0, 0, 0);
      }
    }
  }

  // partial tiles: lane holds rows 16 t + 4 kg + r, column li
  __shared__ float part[NW][MT * 16][17];
  __shared__ float ssp[NW][MT * 16];
#pragma unroll
  for (int t = 0; t < MT; t++) {
#pragma unroll
    for (int r = 0; r < 4; r++) part[wave][16 * t + 4 * kg + r][li] = acc[t][r];
    if constexpr (NORM) {
      float q = ss[t];
      q += __shfl_xor(q, 16);
      q += __shfl_xor(q, 32);
      if (kg == 0) ssp[wave][16 * t + li] = q;
    }
  }
  __syncthreads();
  if (tid >= MT * 256) return;  // whole waves
  const uint32_t row = uint32_t(tid) >> 4, col = uint32_t(tid) & 15;
  float c = 0.f;
#pragma unroll
  for (int v = 0; v < NW; v++) c += part[v][row][col];
  if constexpr (NORM) {
    float q = 0.f;
#pragma unroll
    for (int v = 0; v < NW; v++) q += ssp[v][row];
    c *= 1.0f / sqrtf(q / float(p.K) + p.eps);
  }
  const uint32_t m = row, n = n0 + col;
  if constexpr (EPI == kGemmSiluPair) {
    const float up = __shfl_xor(c, 1);  // column n ^ 1 of the same row
    if (m < p.M && n < p.N && (col & 1) == 0) p.C[size_t(m) * p.ldc + (n >> 1)] = c / (1.0f + expf(-c)) * up;
  } else if constexpr (EPI == kGemmResAdd) {
    if (m < p.M && n < p.N) p.C[size_t(m) * p.ldc + n] += c;
  } else {
    if (m < p.M && n < p.N) p.C[size_t(m) * p.ldc + n] = c;
  }
}

// ---------------------------------------------------------------------------------------------
// Per token m and row r of [q heads, k heads, v heads]: q/k RMSNorm + RoPE with the table row of
// position start + m; q goes to Q [M][n_heads][128], k and v to the cache slot (f32 or bf16).
// One wave per (token, row); lane l holds dims l and l + 64.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_qk_rope(BatchAttnParams p) {
  const uint32_t item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const uint32_t rows = p.n_heads + 2 * p.n_kv;
  if (item >= p.M * rows) return;
  const uint32_t m = item / rows, r = item % rows, pos = p.start + m;
  const float* src = p.qkv + size_t(m) * rows * kHeadDim + size_t(r) * kHeadDim;
  float a = src[lane], b = src[lane + 64];
  if (r < p.n_heads + p.n_kv) {
    const uint16_t* gain = r < p.n_heads ? p.q_norm : p.k_norm;
    const float ss = wave_sum(a * a + b * b);
    const float sc = 1.0f / sqrtf(ss / float(kHeadDim) + p.eps);
    a = a * sc * bf16f(gain[lane]);
    b = b * sc * bf16f(gain[lane + 64]);
    const float2 cs = reinterpret_cast<const float2*>(p.rope)[size_t(pos) * (kHeadDim / 2) + lane];
    const float ar = a * cs.x - b * cs.y, br = b * cs.x + a * cs.y;
    a = ar;
    b = br;
  }
  if (r < p.n_heads) {
    float* q = p.q + (size_t(m) * p.n_heads + r) * kHeadDim;
    q[lane] = a;
    q[lane + 64] = b;
  } else {
    const uint32_t kvh = r < p.n_heads + p.n_kv ? r - p.n_heads : r - p.n_heads - p.n_kv;
    void* cache = r < p.n_heads + p.n_kv ? p.k_cache : p.v_cache;
    const size_t slot = (size_t(kvh) * p.max_seq + pos) * kHeadDim;
    if (p.kv_bf16) {
      static_cast<uint16_t*>(cache)[slot + lane] = f32_to_bf16(a);
      static_cast<uint16_t*>(cache)[slot + lane + 64] = f32_to_bf16(b);
    } else {
      static_cast<float*>(cache)[slot + lane] = a;
      static_cast<float*>(cache)[slot + lane + 64] = b;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Causal attention of a chunk: workgroup (KV head g, block of QB = 16 / G tokens, key run s)
// serves its 16 query vectors (token mb + v / G, head g G + v % G) over the positions of run s,
// [s key_run, (s+1) key_run) cut at start + the block's last token, in LDS tiles of T = 32
// positions, with an online softmax per query vector. Thread (v = tid / 16, kk = tid % 16):
// scores for keys kk and kk + 16 of the tile (K rows padded to 129 floats, so the 16 keys sit in
// 16 banks), then dims kk + 16 i (i < 8) of the output. With one run the output is normalized
// into att [M][n_heads][128]; with several, each writes its (m, l, acc) partial to
// part [M][n_heads][runs][kPartStride] (a query vector with no visible key in the run writes
// m = -inf, l = 0) and k_attn_merge_rows combines them.
// ---------------------------------------------------------------------------------------------
template <int G, bool KV_BF16>
__global__ __launch_bounds__(256) void k_attn_causal(BatchAttnParams p) {
  constexpr int D = kHeadDim, T = 32, NQ = 16, QB = NQ / G, KP = D + 1;
  const uint32_t g = blockIdx.x, mb = blockIdx.y * QB, run = blockIdx.z, runs = gridDim.z;
  const int tid = threadIdx.x, qv = tid >> 4, kk = tid & 15;
  __shared__ __align__(16) float qs[NQ][D];
  __shared__ float ks[T][KP];
  __shared__ __align__(16) float vs[T][D];
  __shared__ float ps[NQ][T];
  {
    const int d4 = (tid & 31) * 4;  // 8 rows of 128 per pass, float4 each
#pragma unroll
    for (int pass = 0; pass < NQ / 8; pass++) {
      const int v = pass * 8 + (tid >> 5);
      const uint32_t m = min(mb + uint32_t(v / G), p.M - 1);
      const float4 q4 = *reinterpret_cast<const float4*>(p.q + (size_t(m) * p.n_heads + g * G + v % G) * D + d4);
      qs[v][d4] = q4.x; qs[v][d4 + 1] = q4.y; qs[v][d4 + 2] = q4.z; qs[v][d4 + 3] = q4.w;
    }
  }
  const uint32_t my_m = mb + uint32_t(qv / G);
  const uint32_t my_pos = p.start + min(my_m, p.M - 1);
  const uint32_t last = p.start + min(mb + QB - 1, p.M - 1);  // positions 0..last are needed
  const uint32_t k_begin = run * p.key_run;
  const uint32_t k_end = min(last + 1, k_begin + p.key_run);  // this run: positions [k_begin, k_end)
  float m_run = -INFINITY, l_run = 0.f;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = 0.f;
  const size_t head = size_t(g) * p.max_seq * D;
  const int lr = tid >> 5, ld = (tid & 31) * 4;  // tile loads: rows lr + 8 j, dims ld .. ld + 3
  for (uint32_t t0 = k_begin; t0 < k_end; t0 += T) {
    float4 kv4[T / 8], vv4[T / 8];
#pragma unroll
    for (int j = 0; j < T / 8; j++) {
      const size_t off = head + size_t(min(t0 + uint32_t(lr + 8 * j), k_end - 1)) * D + ld;
      if constexpr (KV_BF16) {
        const uint2 kb = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.k_cache) + off);
        const uint2 vb = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.v_cache) + off);
        kv4[j] = make_float4(__uint_as_float(kb.x << 16), __uint_as_float(kb.x & 0xFFFF0000u),
                             __uint_as_float(kb.y << 16), __uint_as_float(kb.y & 0xFFFF0000u));
        vv4[j] = make_float4(__uint_as_float(vb.x << 16), __uint_as_float(vb.x & 0xFFFF0000u),
                             __uint_as_float(vb.y << 16), __uint_as_float(vb.y & 0xFFFF0000u));
      } else {
        kv4[j] = *reinterpret_cast<const float4*>(static_cast<const float*>(p.k_cache) + off);
        vv4[j] = *reinterpret_cast<const float4*>(static_cast<const float*>(p.v_cache) + off);
      }
    }
    __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
    for (int j = 0; j < T / 8; j++) {
      const int r = lr + 8 * j;
      ks[r][ld] = kv4[j].x; ks[r][ld + 1] = kv4[j].y; ks[r][ld + 2] = kv4[j].z; ks[r][ld + 3] = kv4[j].w;
      vs[r][ld] = vv4[j].x; vs[r][ld + 1] = vv4[j].y; vs[r][ld + 2] = vv4[j].z; vs[r][ld + 3] = vv4[j].w;
    }
    __syncthreads();
    float sc[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int key = kk + 16 * j;
      float dot = 0.f;
#pragma unroll 16
      for (int d = 0; d < D; d++) dot += qs[qv][d] * ks[key][d];
      const uint32_t t = t0 + uint32_t(key);
      sc[j] = t <= my_pos && t < k_end ? dot * p.scale : -INFINITY;
    }
    float tmax = fmaxf(sc[0], sc[1]);
    for (int o = 1; o < 16; o <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o));
    const float m_new = fmaxf(m_run, tmax);  // -inf while no key of the run is visible to this vector
    const float corr = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
    const float e0 = sc[0] == -INFINITY ? 0.f : expf(sc[0] - m_new);
    const float e1 = sc[1] == -INFINITY ? 0.f : expf(sc[1] - m_new);
    ps[qv][kk] = e0;
    ps[qv][kk + 16] = e1;
    float tsum = e0 + e1;
    for (int o = 1; o < 16; o <<= 1) tsum += __shfl_xor(tsum, o);
    l_run = l_run * corr + tsum;
    m_run = m_new;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] *= corr;
    for (int key = 0; key < T; key++) {
      const float pe = ps[qv][key];
#pragma unroll
      for (int i = 0; i < 8; i++) acc[i] += pe * vs[key][kk + 16 * i];
    }
  }
  if (my_m >= p.M) return;
  const size_t vec = size_t(my_m) * p.n_heads + g * G + qv % G;
  if (runs == 1) {
    float* o = p.att + vec * D;
#pragma unroll
    for (int i = 0; i < 8; i++) o[kk + 16 * i] = acc[i] / l_run;
  } else {
    float* o = p.part + (vec * runs + run) * kPartStride;
    if (kk == 0) { o[0] = m_run; o[1] = l_run; }
#pragma unroll
    for (int i = 0; i < 8; i++) o[4 + kk + 16 * i] = acc[i];
  }
}

// att[v] = sum_s e_s acc_s / sum_s e_s l_s over the runs of query vector v = (token, head),
// e_s = exp(m_s - max m); runs without a visible key (m = -inf) weigh 0. One workgroup of 128
// threads (one per dim) per query vector; all of its run loads are issued at once.
__global__ __launch_bounds__(kHeadDim) void k_attn_merge_rows(const float* __restrict__ part, uint32_t runs,
                                                              float* __restrict__ att) {
  constexpr int U = kBatchMaxRuns;
  const size_t v = blockIdx.x;
  const uint32_t d = threadIdx.x;
  const float* base = part + v * runs * kPartStride;
  float mv[U], lv[U], av[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const float* q = base + size_t(min(uint32_t(u), runs - 1)) * kPartStride;
    mv[u] = q[0];
    lv[u] = q[1];
    av[u] = q[4 + d];
  }
  __builtin_amdgcn_sched_barrier(0);
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; u++) M = uint32_t(u) < runs ? fmaxf(M, mv[u]) : M;
  float L = 0.f, A = 0.f;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const float e = (uint32_t(u) < runs && mv[u] != -INFINITY) ? expf(mv[u] - M) : 0.f;
    L += e * lv[u];
    A += e * av[u];
  }
  att[v * kHeadDim + d] = A / L;
}

// x[m] = bf16 embedding row of ids[m] (cpu_inference.rs:109-111)
__global__ __launch_bounds__(256) void k_embed_rows(const uint16_t* __restrict__ table, const uint32_t* __restrict__ ids,
                                                    uint32_t M, uint32_t H, float* __restrict__ x) {
  const uint32_t m = blockIdx.y;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < H; i += gridDim.x * 256)
    x[size_t(m) * H + i] = bf16f(table[size_t(ids[m]) * H + i]);
}

}  // namespace

hipError_t launch_rownorm(const float* x, uint32_t M, uint32_t K, float eps, float* s, hipStream_t st) {
  if (M == 0 || K % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rownorm, dim3(ceil_div(M, 4)), dim3(256), 0, st, x, M, K, eps, s);
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmParams& p, bool norm, int epi, hipStream_t st) {
  if (p.M == 0 || p.N == 0 || p.N % 2 || p.K % 32 || p.K == 0 || p.lda % 4 || !p.A || !p.W || !p.C)
    return hipErrorInvalidValue;
  if (norm && !p.gain) return hipErrorInvalidValue;
  if (p.M <= kGemmSkinnyMaxM) {
    // one m-tile: 16 waves per workgroup when there are few 16-column blocks, so the chip still
    // fills; two m-tiles: 8 waves (their registers do not fit 16)
    const uint32_t blocks = ceil_div(p.N, 16);
    const bool wide = blocks < 256;
#define QE_SKINNY_EPI(NRM, E)                                                                           \
  do {                                                                                                  \
    if (p.M > 16) hipLaunchKernelGGL((k_gemm_skinny<NRM, E, 2, 8>), dim3(blocks), dim3(512), 0, st, p); \
    else if (wide) hipLaunchKernelGGL((k_gemm_skinny<NRM, E, 1, 16>), dim3(blocks), dim3(1024), 0, st, p); \
    else hipLaunchKernelGGL((k_gemm_skinny<NRM, E, 1, 8>), dim3(blocks), dim3(512), 0, st, p);          \
  } while (0)
    if (norm && epi == kGemmStore) QE_SKINNY_EPI(true, kGemmStore);
    else if (norm && epi == kGemmSiluPair) QE_SKINNY_EPI(true, kGemmSiluPair);
    else if (!norm && epi == kGemmStore) QE_SKINNY_EPI(false, kGemmStore);
    else if (!norm && epi == kGemmResAdd) QE_SKINNY_EPI(false, kGemmResAdd);
    else return hipErrorInvalidValue;
#undef QE_SKINNY_EPI
    return hipGetLastError();
  }
  if (norm && !p.rowscale) return hipErrorInvalidValue;
  const dim3 grid(ceil_div(p.N, 64), ceil_div(p.M, 64));
  // four 32-wide k steps per iteration when K allows, else one
#define QE_GEMM(NRM, E)                                                                         \
  do {                                                                                          \
    if (p.K % 128 == 0) hipLaunchKernelGGL((k_gemm<NRM, E, 4>), grid, dim3(256), 0, st, p);     \
    else hipLaunchKernelGGL((k_gemm<NRM, E, 1>), grid, dim3(256), 0, st, p);                    \
  } while (0)
  if (norm && epi == kGemmStore) QE_GEMM(true, kGemmStore);
  else if (norm && epi == kGemmSiluPair) QE_GEMM(true, kGemmSiluPair);
  else if (!norm && epi == kGemmStore) QE_GEMM(false, kGemmStore);
  else if (!norm && epi == kGemmResAdd) QE_GEMM(false, kGemmResAdd);
  else return hipErrorInvalidValue;
#undef QE_GEMM
  return hipGetLastError();
}

hipError_t launch_qk_rope(const BatchAttnParams& p, hipStream_t st) {
  const uint32_t items = p.M * (p.n_heads + 2 * p.n_kv);
  hipLaunchKernelGGL(k_qk_rope, dim3(ceil_div(items, 4)), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_attn_causal(const BatchAttnParams& p, uint32_t runs, hipStream_t st) {
  if (!p.n_kv || p.n_heads % p.n_kv || runs == 0 || runs > uint32_t(kBatchMaxRuns) || (runs > 1 && !p.part))
    return hipErrorInvalidValue;
  const uint32_t G = p.n_heads / p.n_kv;
  BatchAttnParams q = p;
  // runs of whole 32-position tiles covering positions 0 .. start + M - 1, none of them empty
  const uint32_t tiles = ceil_div(p.start + p.M, 32), per_run = ceil_div(tiles, runs);
  runs = ceil_div(tiles, per_run);
  q.key_run = 32 * per_run;
  const dim3 grid(p.n_kv, ceil_div(p.M, 16 / G), runs);
  hipError_t e = hipErrorInvalidValue;
#define QE_ATT(GG)                                                                                         \
  if (G == GG) {                                                                                           \
    if (p.kv_bf16) hipLaunchKernelGGL((k_attn_causal<GG, true>), grid, dim3(256), 0, st, q);               \
    else hipLaunchKernelGGL((k_attn_causal<GG, false>), grid, dim3(256), 0, st, q);                        \
    e = hipGetLastError();                                                                                 \
  }
  QE_ATT(1)
  QE_ATT(2)
  QE_ATT(4)
  QE_ATT(8)
#undef QE_ATT
  if (e != hipSuccess || runs == 1) return e;
  hipLaunchKernelGGL(k_attn_merge_rows, dim3(p.M * p.n_heads), dim3(kHeadDim), 0, st, p.part, runs, p.att);
  return hipGetLastError();
}

uint32_t attn_causal_runs(uint32_t M, uint32_t start, uint32_t n_heads, uint32_t n_kv) {
  if (!M || !n_kv || n_heads % n_kv || n_heads / n_kv > 16) return 1;
  const uint32_t wgs = n_kv * ceil_div(M, 16 / (n_heads / n_kv));
  uint32_t runs = std::min(ceil_div(1024, wgs), uint32_t(kBatchMaxRuns));
  return std::max(1u, std::min(runs, ceil_div(start + M, 64)));
}

hipError_t launch_embed_rows(const uint16_t* table, const uint32_t* ids, uint32_t M, uint32_t H, float* x,
                             hipStream_t st) {
  hipLaunchKernelGGL(k_embed_rows, dim3(ceil_div(H, 256), M), dim3(256), 0, st, table, ids, M, H, x);
  return hipGetLastError();
}

}  // namespace qe
