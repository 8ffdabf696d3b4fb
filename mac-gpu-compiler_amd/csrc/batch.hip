// Multi-token forward (chunked prefill and k-token verify) on bf16 MFMA.
//
// The reference runs its prompt one token at a time (metal_infrence_engine/src/bin/bench.rs:174-176
// calls forward per position); these kernels run a chunk of M tokens through a layer at once, so
// every weight is read once per chunk and the projections become GEMMs on the matrix cores:
//   rownorm        s[m] = 1/sqrt(mean(x_m^2) + eps)                  (cpu_inference.rs:189-194)
//   GEMMs          C[m][n] = sum_k A'[m][k] W[n][k], A' = f32 A (x s[m] x gain[k] with a norm),
//                  split into hi + lo bf16 so the products keep ~16 mantissa bits; epilogues
//                  store / residual add / silu(gate)*up / q-k norm + RoPE + K/V append
//                  (cpu_inference.rs:225-257): k_gemm_skinny (<= 32 rows), k_gemm_lds / k_gemm (<= 64),
//                  k_gemm_rows8 (<= 1024), k_gemm_tile (more); k_mv_rows (<= 4 rows, f32 FMA)
//   k_qk_rope      per token and head: q/k RMSNorm + RoPE, K/V append   (cpu_inference.rs:134-141)
//   k_attn_causal_bf  token m attends positions 0..start+m, split bf16 MFMA (cpu_inference.rs:144-162)
//   k_row_argmax_*    greedy token per logit row (main.rs:37-42)
#include "batch.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "device_common.h"
#include "l2_prefetch.h"

namespace qe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 8 floats -> (hi, lo) bf16x8 with hi = bf16(v), lo = bf16(v - hi), both rounded to nearest
// even by the hardware pair conversion (v_cvt_pk_bf16_f32); hi + lo keeps ~16 mantissa bits
__device__ __forceinline__ void split8(const float (&v)[8], bf16x8& hi, bf16x8& lo) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  u32x4 h, l;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{v[2 * e], v[2 * e + 1]}), bf16x2));
    const float r0 = v[2 * e] - __uint_as_float(hb << 16), r1 = v[2 * e + 1] - __uint_as_float(hb & 0xFFFF0000u);
    h[e] = hb;
    l[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{r0, r1}), bf16x2));
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
// Tiled GEMM, K % 64 == 0: workgroup tile 64 (m) x 64 (n), 4 waves; wave w owns rows
// [16 w, 16 w + 16) and all four 16-column blocks. The W tile of each 64-deep stage is loaded
// once per workgroup into LDS (three buffers, rows padded to 72 bf16 so that the 16 rows a
// fragment read touches land in distinct banks) and shared by the four waves; each wave's A
// rows go straight to registers, split hi + lo. Loads run two stages ahead of the MFMAs.
// gridDim.z > 1 splits K: split z covers K / gridDim.z and writes
// its partial sums (kGemmPartial) to C + z M ldc.
// ---------------------------------------------------------------------------------------------
template <bool NORM, int EPI>
__global__ __launch_bounds__(256) void k_gemm_lds(GemmParams p) {
  constexpr int BK = 64, WP = BK + 8;
  __shared__ __align__(16) uint16_t ws[3][64][WP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kg = lane >> 4;
  const uint32_t m0 = blockIdx.y * 64 + wave * 16, n0 = blockIdx.x * 64;
  const uint32_t kz = p.K / gridDim.z, kbeg = blockIdx.z * kz, nst = kz / BK;
  const uint32_t arow = min(m0 + uint32_t(li), p.M - 1);
  const float* Ar = p.A + size_t(arow) * p.lda + kbeg + 8 * kg;
  const float rs = NORM ? p.rowscale[arow] : 1.0f;
  const uint16_t* gp = NORM ? p.gain + kbeg + 8 * kg : nullptr;
  // W stage: 64 rows x 8 chunks of 16 B; thread t moves chunks t and t + 256
  const uint16_t* Wsrc[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int c = tid + 256 * i;
    Wsrc[i] = p.W + size_t(min(n0 + uint32_t(c >> 3), p.N - 1)) * p.K + kbeg + 8 * (c & 7);
  }
  // one stage in registers: its W chunks (bound for LDS), A fragments and gains
  struct Stage {
    u32x4 w[2];
    f32x4 a[2][2];
    u32x4 g[2];
  };
  auto load = [&](Stage& r, uint32_t stg) __attribute__((always_inline)) {
    const uint32_t k = stg * BK;
#pragma unroll
    for (int i = 0; i < 2; i++) r.w[i] = *reinterpret_cast<const u32x4*>(Wsrc[i] + k);
#pragma unroll
    for (int u = 0; u < 2; u++) {
      r.a[u][0] = *reinterpret_cast<const f32x4*>(Ar + k + 32 * u);
      r.a[u][1] = *reinterpret_cast<const f32x4*>(Ar + k + 32 * u + 4);
      if constexpr (NORM) r.g[u] = *reinterpret_cast<const u32x4*>(gp + k + 32 * u);
    }
  };
  auto store_w = [&](const Stage& r, uint32_t buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4*>(&ws[buf][c >> 3][8 * (c & 7)]) = r.w[i];
    }
  };
  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Software pipeline over three LDS buffers: at step s the W tile of stage s is in buffer
  // s % 3, stage s + 1's W (loaded one step earlier) goes to buffer (s + 1) % 3, whose last
  // readers were at step s - 2, and stage s + 2 is loaded into the registers stage s vacates.
  auto step = [&](Stage& cur, Stage& nxt, uint32_t s) __attribute__((always_inline)) {
    store_w(nxt, (s + 1) % 3);
    bf16x8 hi[2], lo[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      float v[8] = {cur.a[u][0][0], cur.a[u][0][1], cur.a[u][0][2], cur.a[u][0][3],
                    cur.a[u][1][0], cur.a[u][1][1], cur.a[u][1][2], cur.a[u][1][3]};
      if constexpr (NORM) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[2 * e] = (v[2 * e] * rs) * __uint_as_float(cur.g[u][e] << 16);
          v[2 * e + 1] = (v[2 * e + 1] * rs) * __uint_as_float(cur.g[u][e] & 0xFFFF0000u);
        }
      }
      split8(v, hi[u], lo[u]);
    }
    load(cur, min(s + 2, nst - 1));  // unconditional: the last stages reload the last one
    if (s < nst) {                   // an odd stage count ends with one empty step
      const uint32_t buf = s % 3;
#pragma unroll
      for (int u = 0; u < 2; u++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const bf16x8 b = *reinterpret_cast<const bf16x8*>(&ws[buf][16 * j + li][32 * u + 8 * kg]);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi[u], b, acc[j], 0, 0, 0);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo[u], b, acc[j], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  };
  Stage r0, r1;
  load(r0, 0);
  load(r1, min(1u, nst - 1));
  store_w(r0, 0);
  __syncthreads();
  for (uint32_t s = 0; s < nst; s += 2) {
    step(r0, r1, s);
    step(r1, r0, s + 1);
  }

  // epilogue: lane holds C[m0 + 4 kg + r][n0 + 16 j + li]
  float* C = p.C + (EPI == kGemmPartial ? size_t(blockIdx.z) * p.M * p.ldc : 0);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t n = n0 + 16 * j + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t m = m0 + 4 * kg + r;
      const float c = acc[j][r];
      if constexpr (EPI == kGemmSiluPair) {
        const float up = __shfl_xor(c, 1);  // columns 2i (gate) and 2i+1 (up) in neighbouring lanes
        if (m < p.M && n < p.N && (li & 1) == 0) C[size_t(m) * p.ldc + (n >> 1)] = c / (1.0f + expf(-c)) * up;
      } else if constexpr (EPI == kGemmResAdd) {
        if (m < p.M && n < p.N) C[size_t(m) * p.ldc + n] += c;
      } else {
        if (m < p.M && n < p.N) C[size_t(m) * p.ldc + n] = c;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Tiled GEMM for M > 64: workgroup tile 128 (m) x BN (n), BN = 128 or 64, k stages of 32. Four
// waves as 2 x 2: wave (wm, wn) owns rows 64 wm .. 64 wm + 63 and columns (BN / 2) wn .. + BN / 2
// - 1, i.e. 4 x BN / 32 MFMA tiles of 16 x 16, so each fragment read from LDS feeds BN / 32 (A)
// or 8 (W) MFMAs. Both operands are staged in LDS: the thread that loads an f32 A element
// applies the norm scale and splits it into hi + lo bf16 once for the whole workgroup; W rows go
// in as they are. Two LDS buffers and D register stages (stage t in register slot t % D): while
// stage s is computed from one buffer, stage s + 1 goes from its slot to the other buffer and the
// slot is refilled with stage s + 1 + D, so each load has D steps of MFMA work to arrive in (one
// step is short next to the L2 / MALL latency). The stage count K / 32 (per split) is a multiple
// of D (the launcher checks). gridDim.z > 1 splits K as in k_gemm_lds.
// ---------------------------------------------------------------------------------------------
template <bool NORM, int EPI, int BN, int D>
__global__ __launch_bounds__(256) void k_gemm_tile(GemmParams p) {
  constexpr int BM = 128, BK = 32, NT = BN / 32, KP = BK + 8;
  constexpr int WCH = BN * BK / 8 / 256;  // 16-byte W chunks per thread per stage
  static_assert(WCH >= 1 && NT >= 2, "tile");
  __shared__ __align__(16) uint16_t as[2][2][BM][KP];  // [buffer][hi, lo][m][k]
  __shared__ __align__(16) uint16_t bs[2][BN][KP];     // [buffer][n][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, kg = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const uint32_t kz = p.K / gridDim.z, kbeg = blockIdx.z * kz, nst = kz / BK;
  // A staging: float4 f = tid + 256 i (i < 4) is row tid / 8 + 32 i, k (tid % 8) * 4
  const int ar = tid >> 3, ak = (tid & 7) * 4;
  const float* Asrc[4];
  float rs[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t row = min(m0 + uint32_t(ar + 32 * i), p.M - 1);
    Asrc[i] = p.A + size_t(row) * p.lda + kbeg + ak;
    rs[i] = NORM ? p.rowscale[row] : 1.0f;
  }
  const uint16_t* gsrc = NORM ? p.gain + kbeg + ak : nullptr;
  // W staging: chunk c = tid + 256 i is row c / 4, k (c % 4) * 8
  const uint16_t* Wsrc[WCH];
#pragma unroll
  for (int i = 0; i < WCH; i++) {
    const int c = tid + 256 * i;
    Wsrc[i] = p.W + size_t(min(n0 + uint32_t(c >> 2), p.N - 1)) * p.K + kbeg + 8 * (c & 3);
  }
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  struct Stage {
    f32x4 a[4];
    u32x4 w[WCH];
    u32x2 g;
  };
  auto load = [&](Stage& r, uint32_t stg) __attribute__((always_inline)) {
    const uint32_t k = stg * BK;
#pragma unroll
    for (int i = 0; i < 4; i++) r.a[i] = *reinterpret_cast<const f32x4*>(Asrc[i] + k);
#pragma unroll
    for (int i = 0; i < WCH; i++) r.w[i] = *reinterpret_cast<const u32x4*>(Wsrc[i] + k);
    if constexpr (NORM) r.g = *reinterpret_cast<const u32x2*>(gsrc + k);
  };
  auto pk = [](float a, float b) __attribute__((always_inline)) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
  };
  auto store = [&](const Stage& r, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float v[4] = {r.a[i][0], r.a[i][1], r.a[i][2], r.a[i][3]};
      if constexpr (NORM) {
        v[0] = (v[0] * rs[i]) * __uint_as_float(r.g[0] << 16);
        v[1] = (v[1] * rs[i]) * __uint_as_float(r.g[0] & 0xFFFF0000u);
        v[2] = (v[2] * rs[i]) * __uint_as_float(r.g[1] << 16);
        v[3] = (v[3] * rs[i]) * __uint_as_float(r.g[1] & 0xFFFF0000u);
      }
      const uint32_t h0 = pk(v[0], v[1]), h1 = pk(v[2], v[3]);
      const uint32_t l0 = pk(v[0] - __uint_as_float(h0 << 16), v[1] - __uint_as_float(h0 & 0xFFFF0000u));
      const uint32_t l1 = pk(v[2] - __uint_as_float(h1 << 16), v[3] - __uint_as_float(h1 & 0xFFFF0000u));
      *reinterpret_cast<u32x2*>(&as[buf][0][ar + 32 * i][ak]) = u32x2{h0, h1};
      *reinterpret_cast<u32x2*>(&as[buf][1][ar + 32 * i][ak]) = u32x2{l0, l1};
    }
#pragma unroll
    for (int i = 0; i < WCH; i++) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4*>(&bs[buf][c >> 2][8 * (c & 3)]) = r.w[i];
    }
  };
  f32x4 acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // All fragments of the stage are read before the first MFMA, so the LDS latency is paid once
  // per stage; then the hi products, then the lo products (each accumulator still adds hi . w
  // before lo . w).
  auto compute = [&](int buf) __attribute__((always_inline)) {
    bf16x8 b[NT], hi[4], lo[4];
#pragma unroll
    for (int j = 0; j < NT; j++)
      b[j] = *reinterpret_cast<const bf16x8*>(&bs[buf][wn * (BN / 2) + 16 * j + li][8 * kg]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = wm * 64 + 16 * i + li;
      hi[i] = *reinterpret_cast<const bf16x8*>(&as[buf][0][row][8 * kg]);
      lo[i] = *reinterpret_cast<const bf16x8*>(&as[buf][1][row][8 * kg]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < NT; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi[i], b[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < NT; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo[i], b[j], acc[i][j], 0, 0, 0);
  };
  Stage r[D];
#pragma unroll
  for (int i = 0; i < D; i++) load(r[i], min(uint32_t(i), nst - 1));
  store(r[0], 0);
  load(r[0], min(uint32_t(D), nst - 1));
  __syncthreads();
  // Every step is unconditional: the loads past the last stage re-read the last stage (in
  // bounds), and the last step's store goes to the buffer no later step reads.
  for (uint32_t s0 = 0; s0 < nst; s0 += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      const uint32_t s = s0 + uint32_t(i);
      compute(int(s & 1));
      __builtin_amdgcn_sched_barrier(0);
      store(r[(i + 1) % D], int((s + 1) & 1));
      load(r[(i + 1) % D], min(s + 1 + D, nst - 1));
      __syncthreads();
    }
  }

  // epilogue: lane holds C[m0 + 64 wm + 16 i + 4 kg + r][n0 + (BN / 2) wn + 16 j + li]
  float* C = p.C + (EPI == kGemmPartial ? size_t(blockIdx.z) * p.M * p.ldc : 0);
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const uint32_t n = n0 + uint32_t(wn * (BN / 2) + 16 * j + li);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = m0 + uint32_t(wm * 64 + 16 * i + 4 * kg + r);
        const float c = acc[i][j][r];
        if constexpr (EPI == kGemmSiluPair) {
          const float up = __shfl_xor(c, 1);  // columns 2i (gate) and 2i+1 (up) in neighbouring lanes
          if (m < p.M && n < p.N && (li & 1) == 0) C[size_t(m) * p.ldc + (n >> 1)] = c / (1.0f + expf(-c)) * up;
        } else if constexpr (EPI == kGemmResAdd) {
          if (m < p.M && n < p.N) C[size_t(m) * p.ldc + n] += c;
        } else {
          if (m < p.M && n < p.N) C[size_t(m) * p.ldc + n] = c;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Tiled GEMM for chunks of up to kGemmRowsMaxM rows, A straight to registers: workgroup tile 64
// (m) x BN (n), k steps of 64, eight waves. Wave w owns the 16-row block w % 4 and the k half w / 4
// of every step (k 64 s + 32 (w / 4) .. + 31). An A row belongs to one wave pair only, so each lane
// loads its own f32 A fragment (row li of its block, k 8 kg .. 8 kg + 7), applies the norm scale
// and splits it into hi + lo bf16 in registers; only the W tile, which all eight waves read, goes
// through LDS (two buffers, rows staged 128 bytes = 64 k at a time). A 64 x 128 tile keeps the
// bytes each CU pulls per MFMA lower than the 128-row tile does at these sizes, where the loads
// from L2 and not the matrix cores set the pace, and still gives one tile per CU at 512 rows.
// D steps in flight: A of step s + D is loaded as soon as step s is computed, W of step s + 1 + D
// as soon as step s + 1 is in LDS. At the end the k-half-1 waves hand their sums to the k-half-0
// waves through LDS: C = (sum over the even 32-k blocks) + (sum over the odd ones). The step
// count K / 64 (per split) is a multiple of D. gridDim.z > 1 splits K as in k_gemm_lds.
// ---------------------------------------------------------------------------------------------
template <bool NORM, int EPI, int BN, int D>
__global__ __launch_bounds__(512) void k_gemm_rows8(GemmParams p, BatchAttnParams qa) {
  constexpr int BK = 64, KP = BK + 8, NT = BN / 16;
  constexpr int WCH = BN * BK / 8 / 512;  // 16-byte W chunks per thread per step
  static_assert(WCH >= 1, "tile");
  static_assert(2 * BN * KP * 2 >= 4 * 64 * NT * 16, "the reduction reuses the W buffers");
  __shared__ __align__(16) uint16_t bs[2][BN][KP];  // [buffer][n][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, kg = lane >> 4;
  const int wr = wave & 3, kh = wave >> 2;
  const uint32_t m0 = blockIdx.y * 64 + uint32_t(wr) * 16, n0 = blockIdx.x * BN;
  const uint32_t kz = p.K / gridDim.z, kbeg = blockIdx.z * kz, nst = kz / BK;
  const uint32_t row = min(m0 + uint32_t(li), p.M - 1);
  const float* Ar = p.A + size_t(row) * p.lda + kbeg + 32 * kh + 8 * kg;
  const float rs = NORM ? p.rowscale[row] : 1.0f;
  const uint16_t* gsrc = NORM ? p.gain + kbeg + 32 * kh + 8 * kg : nullptr;
  // W staging: chunk c = tid + 512 i is row c / 8, k (c % 8) * 8
  const uint16_t* Wsrc[WCH];
#pragma unroll
  for (int i = 0; i < WCH; i++) {
    const int c = tid + 512 * i;
    Wsrc[i] = p.W + size_t(min(n0 + uint32_t(c >> 3), p.N - 1)) * p.K + kbeg + 8 * (c & 7);
  }
  struct AStage {
    f32x4 a[2];
    u32x4 g;
  };
  struct WStage {
    u32x4 w[WCH];
  };
  auto load_a = [&](AStage& r, uint32_t stg) __attribute__((always_inline)) {
    const uint32_t k = stg * BK;
    r.a[0] = *reinterpret_cast<const f32x4*>(Ar + k);
    r.a[1] = *reinterpret_cast<const f32x4*>(Ar + k + 4);
    if constexpr (NORM) r.g = *reinterpret_cast<const u32x4*>(gsrc + k);
  };
  auto load_w = [&](WStage& r, uint32_t stg) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < WCH; i++) r.w[i] = *reinterpret_cast<const u32x4*>(Wsrc[i] + stg * BK);
  };
  auto store_w = [&](const WStage& r, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < WCH; i++) {
      const int c = tid + 512 * i;
      *reinterpret_cast<u32x4*>(&bs[buf][c >> 3][8 * (c & 7)]) = r.w[i];
    }
  };
  f32x4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const AStage& r, int buf) __attribute__((always_inline)) {
    bf16x8 b[NT], hi, lo;
#pragma unroll
    for (int j = 0; j < NT; j++) b[j] = *reinterpret_cast<const bf16x8*>(&bs[buf][16 * j + li][32 * kh + 8 * kg]);
    float v[8] = {r.a[0][0], r.a[0][1], r.a[0][2], r.a[0][3], r.a[1][0], r.a[1][1], r.a[1][2], r.a[1][3]};
    if constexpr (NORM) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[2 * e] = (v[2 * e] * rs) * __uint_as_float(r.g[e] << 16);
        v[2 * e + 1] = (v[2 * e + 1] * rs) * __uint_as_float(r.g[e] & 0xFFFF0000u);
      }
    }
    split8(v, hi, lo);
#pragma unroll
    for (int j = 0; j < NT; j++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b[j], acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < NT; j++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b[j], acc[j], 0, 0, 0);
  };
  AStage ra[D];
  WStage rw[D];
#pragma unroll
  for (int i = 0; i < D; i++) {
    load_a(ra[i], min(uint32_t(i), nst - 1));
    load_w(rw[i], min(uint32_t(i), nst - 1));
  }
  store_w(rw[0], 0);
  load_w(rw[0], min(uint32_t(D), nst - 1));
  __syncthreads();
  // Every step is unconditional: loads past the last step re-read the last step (in bounds), and
  // the last step's W store goes to the buffer no later step reads.
  for (uint32_t s0 = 0; s0 < nst; s0 += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      const uint32_t s = s0 + uint32_t(i);
      compute(ra[i], int(s & 1));
      load_a(ra[i], min(s + D, nst - 1));
      store_w(rw[(i + 1) % D], int((s + 1) & 1));
      load_w(rw[(i + 1) % D], min(s + 1 + D, nst - 1));
      __syncthreads();
    }
  }
  // the k-half-1 waves' sums, lane-major per (row block, column block), through the W buffers
  f32x4* red = reinterpret_cast<f32x4*>(&bs[0][0][0]);
  if (kh == 1) {
#pragma unroll
    for (int j = 0; j < NT; j++) red[(wr * NT + j) * 64 + lane] = acc[j];
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int j = 0; j < NT; j++) acc[j] += red[(wr * NT + j) * 64 + lane];

  // epilogue: lane holds C[m0 + 4 kg + r][n0 + 16 j + li]
  if constexpr (EPI == kGemmQkRope) {
    // the tile's 128 columns are one head (BN == 128 == head_dim): head hh of [q | k | v]. A row's
    // 128 values sit in the 16 lanes of its kg group (8 each), and the RoPE pair (d, d + 64) is
    // (j, j + 4) of one lane (cpu_inference.rs:134-141, 189-215).
    static_assert(BN == kHeadDim && NT == 8, "one head per tile");
    const uint32_t hh = n0 / kHeadDim;
    const bool isq = hh < qa.n_heads, isk = !isq && hh < qa.n_heads + qa.n_kv;
    float gn[NT];
    const uint16_t* gsrc = isq ? qa.q_norm : qa.k_norm;
#pragma unroll
    for (int j = 0; j < NT; j++) gn[j] = isq || isk ? bf16f(gsrc[16 * j + li]) : 1.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t m = m0 + uint32_t(4 * kg + r), pos = qa.start + min(m, p.M - 1);
      float v[NT];
#pragma unroll
      for (int j = 0; j < NT; j++) v[j] = acc[j][r];
      if (isq || isk) {  // uniform over the workgroup
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NT; j++) ss += v[j] * v[j];
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        ss += __shfl_xor(ss, 8);
        const float sc = 1.0f / sqrtf(ss / float(kHeadDim) + qa.eps);
#pragma unroll
        for (int j = 0; j < NT; j++) v[j] = v[j] * sc * gn[j];
        const float2* rope = reinterpret_cast<const float2*>(qa.rope) + size_t(pos) * (kHeadDim / 2);
#pragma unroll
        for (int j = 0; j < NT / 2; j++) {
          const float2 cs = rope[16 * j + li];
          const float a = v[j], b = v[j + NT / 2];
          v[j] = a * cs.x - b * cs.y;
          v[j + NT / 2] = b * cs.x + a * cs.y;
        }
      }
      if (m < p.M) {
        if (isq) {
          float* q = qa.q + (size_t(m) * qa.n_heads + hh) * kHeadDim;
#pragma unroll
          for (int j = 0; j < NT; j++) q[16 * j + li] = v[j];
        } else {
          const uint32_t kvh = isk ? hh - qa.n_heads : hh - qa.n_heads - qa.n_kv;
          void* cache = isk ? qa.k_cache : qa.v_cache;
          const size_t slot = (size_t(kvh) * qa.max_seq + pos) * kHeadDim;
#pragma unroll
          for (int j = 0; j < NT; j++) {
            if (qa.kv_bf16) static_cast<uint16_t*>(cache)[slot + 16 * j + li] = f32_to_bf16(v[j]);
            else static_cast<float*>(cache)[slot + 16 * j + li] = v[j];
          }
        }
      }
    }
    return;
  }
  float* C = p.C + (EPI == kGemmPartial ? size_t(blockIdx.z) * p.M * p.ldc : 0);
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const uint32_t n = n0 + uint32_t(16 * j + li);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t m = m0 + uint32_t(4 * kg + r);
      const float c = acc[j][r];
      if constexpr (EPI == kGemmSiluPair) {
        const float up = __shfl_xor(c, 1);  // columns 2i (gate) and 2i+1 (up) in neighbouring lanes
        if (m < p.M && n < p.N && (li & 1) == 0) C[size_t(m) * p.ldc + (n >> 1)] = c / (1.0f + expf(-c)) * up;
      } else if constexpr (EPI == kGemmResAdd) {
        if (m < p.M && n < p.N) C[size_t(m) * p.ldc + n] += c;
      } else {
        if (m < p.M && n < p.N) C[size_t(m) * p.ldc + n] = c;
      }
    }
  }
}

// x[m] += sum_z part[z][m] (in z order), then s[m] = 1 / sqrt(mean x[m]^2 + eps); one workgroup
// per row, float4 per thread per pass
__global__ __launch_bounds__(256) void k_resadd_partials(float* __restrict__ x, const float* __restrict__ part,
                                                         uint32_t splits, uint32_t M, uint32_t N, float eps,
                                                         float* __restrict__ s) {
  __shared__ float red[4];
  const uint32_t m = blockIdx.x, tid = threadIdx.x;
  float ss = 0.f;
  for (uint32_t c = tid; c < N / 4; c += 256) {
    float4 acc = reinterpret_cast<const float4*>(part + size_t(m) * N)[c];
    for (uint32_t z = 1; z < splits; z++) {
      const float4 v = reinterpret_cast<const float4*>(part + (size_t(z) * M + m) * N)[c];
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    float4* xr = reinterpret_cast<float4*>(x + size_t(m) * N) + c;
    float4 xv = *xr;
    xv.x += acc.x; xv.y += acc.y; xv.z += acc.z; xv.w += acc.w;
    *xr = xv;
    ss += (xv.x * xv.x + xv.y * xv.y) + (xv.z * xv.z + xv.w * xv.w);
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  if (tid == 0) s[m] = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / float(N) + eps);
}

// ---------------------------------------------------------------------------------------------
// Skinny GEMM for M <= 16 MT rows (verify, the last chunk of a prefill): the weights are the
// whole cost, so the work is spread over K as well as N. Workgroup = NW waves on 16 columns
// n0 .. n0+15 and the K range of split blockIdx.y (gridDim.y > 1: kGemmPartial sums to
// C + split M ldc); wave w covers the k steps [w KPW, (w+1) KPW) with KPW = ceil(K / 32 / NW),
// KMAX at a time with every load of the batch issued before any use (clamped to the last step;
// steps past the range masked by a zero W fragment), MT m-tiles per W fragment, A split
// hi + lo as in k_gemm. The NW partial tiles are summed in LDS in wave order. With the norm,
// each lane also sums x^2 of its row over the steps it loads, so
// C = s[m] sum_k (x g)[m][k] W[n][k] with s[m] = 1 / sqrt(mean x^2 + eps) (the scale applied
// after the sum, a reassociation of the reference's f32 product).
// ---------------------------------------------------------------------------------------------
template <bool NORM, int EPI, int MT, int NW, int KMAX>
__global__ __launch_bounds__(64 * NW) void k_gemm_skinny(GemmParams p) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kg = lane >> 4;
  const uint32_t n0 = blockIdx.x * 16;
  const uint32_t kz = p.K / gridDim.y, kbeg = blockIdx.y * kz;  // this split's k range
  const uint32_t KS = kz / 32, KPW = (KS + NW - 1) / NW, s0 = uint32_t(wave) * KPW;
  const uint16_t* Wr = p.W + size_t(min(n0 + uint32_t(li), p.N - 1)) * p.K + kbeg + 8 * kg;
  const float* Ar[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) Ar[t] = p.A + size_t(min(uint32_t(16 * t + li), p.M - 1)) * p.lda + kbeg + 8 * kg;
  const uint16_t* gp = NORM ? p.gain + kbeg + 8 * kg : nullptr;

  f32x4 acc[MT];
  float ss[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) {
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    ss[t] = 0.f;
  }
  for (uint32_t base = 0; base < KPW; base += KMAX) {
    u32x4 w[KMAX], g[KMAX];
    f32x4 a0[KMAX][MT], a1[KMAX][MT];
#pragma unroll
    for (int u = 0; u < KMAX; u++) {
      const uint32_t k = 32 * min(s0 + base + uint32_t(u), KS - 1);
      w[u] = *reinterpret_cast<const u32x4*>(Wr + k);
#pragma unroll
      for (int t = 0; t < MT; t++) {
        a0[u][t] = *reinterpret_cast<const f32x4*>(Ar[t] + k);
        a1[u][t] = *reinterpret_cast<const f32x4*>(Ar[t] + k + 4);
      }
      if constexpr (NORM) g[u] = *reinterpret_cast<const u32x4*>(gp + k);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < KMAX; u++) {
      const bool ok = base + u < KPW && s0 + base + u < KS;
      const u32x4 wc = ok ? w[u] : u32x4{0u, 0u, 0u, 0u};
      const bf16x8 b = __builtin_bit_cast(bf16x8, wc);
#pragma unroll
      for (int t = 0; t < MT; t++) {
        float v[8] = {a0[u][t][0], a0[u][t][1], a0[u][t][2], a0[u][t][3],
                      a1[u][t][0], a1[u][t][1], a1[u][t][2], a1[u][t][3]};
        if constexpr (NORM) {
          float q = 0.f;
#pragma unroll
          for (int e = 0; e < 8; e++) q += v[e] * v[e];
          ss[t] += ok ? q : 0.f;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            v[2 * e] *= __uint_as_float(g[u][e] << 16);
            v[2 * e + 1] *= __uint_as_float(g[u][e] & 0xFFFF0000u);
          }
        }
        bf16x8 hi, lo;
        split8(v, hi, lo);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b, acc[t], 0, 0, 0);
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
  float* C = p.C + (EPI == kGemmPartial ? size_t(blockIdx.y) * p.M * p.ldc : 0);
  // MT * 256 outputs over the workgroup's threads; each pass covers whole waves
  for (uint32_t o = uint32_t(tid); o < uint32_t(MT * 256); o += uint32_t(64 * NW)) {
    const uint32_t row = o >> 4, col = o & 15;
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
      if (m < p.M && n < p.N && (col & 1) == 0) C[size_t(m) * p.ldc + (n >> 1)] = c / (1.0f + expf(-c)) * up;
    } else if constexpr (EPI == kGemmResAdd) {
      if (m < p.M && n < p.N) C[size_t(m) * p.ldc + n] += c;
    } else {
      if (m < p.M && n < p.N) C[size_t(m) * p.ldc + n] = c;
    }
  }
}

// skinny launch: MT m-tiles, NW waves (4 when K is split over workgroups, else 8), and the
// batch of k steps loaded at once sized to the steps per wave
template <bool NORM, int EPI>
void launch_skinny(const GemmParams& p, uint32_t splits, hipStream_t st) {
  const uint32_t NW = splits > 1 ? 4 : 8, KPW = ceil_div(p.K / splits / 32, NW);
  const dim3 grid(ceil_div(p.N, 16), splits);
  const bool two = p.M > 16, wide_k = KPW > 4;
#define QE_SK(MT, W, KM) hipLaunchKernelGGL((k_gemm_skinny<NORM, EPI, MT, W, KM>), grid, dim3(64 * W), 0, st, p)
  // two m-tiles always load four steps at a time (eight do not fit their registers)
  if (NW == 4) {
    if (two) QE_SK(2, 4, 4);
    else if (wide_k) QE_SK(1, 4, 8);
    else QE_SK(1, 4, 4);
  } else {
    if (two) QE_SK(2, 8, 4);
    else if (wide_k) QE_SK(1, 8, 8);
    else QE_SK(1, 8, 4);
  }
#undef QE_SK
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
// Causal attention of a chunk on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16) with split
// operands: q, and f32 K / V, are split into hi + lo bf16 (K and V once, when a tile is staged
// in LDS), and each product keeps the hi*hi, hi*lo and lo*hi terms (lo*lo is below 2^-16 of the
// product); a bf16 cache is exact in hi, so its tiles take two terms.
// Workgroup (KV head g, block of TOK = 64 RB / G tokens, key run s) serves 64 RB query rows,
// row r = token mb + r / G of head g G + r % G; wave w owns RB blocks of 16 rows (rows 16 (RB w
// + b) .. + 15) and lane l the row l % 16 of each. Keys come in LDS tiles of 64 positions (the
// next tile's K is loaded into registers during this tile's scores, its V during P V), and every fragment a wave reads
// from LDS feeds the MFMAs of all its RB row blocks. Per tile a wave computes the transposed
// scores S^T[key][row] (A = K rows: lane has key 16 j + l % 16, dims 32 s + 8 kg .. +7 with
// kg = l / 16; B = q of row l % 16, same dims). In the 16 x 16 output layout a lane then holds
// keys 16 j + 4 kg + r (j, r < 4) of its own row, so the online softmax (max, rescale, sum)
// stays in the lane plus two shuffles across kg, with no LDS round trip for P. Next
// O^T[d][row] += V^T P^T, with the k index of a 32-key step mapped so that lane kg's eight B
// values are its own probabilities for keys 4 kg + r and 16 + 4 kg + r (r < 4); the A side
// reads those keys from a transposed V tile whose key slots are permuted to match (Vt[d][slot],
// key 32 s + 16 h + 4 kg + r in slot 32 s + 8 kg + 4 h + r), so a lane's eight keys are one
// 16-byte read, and O^T's column is again the lane's row. Rows with no visible key in the run keep m = -inf,
// l = 0. One run: normalized output to att [M][n_heads][128]; several: (m, l, acc) partials to
// part [M][n_heads][runs][kPartStride], combined by k_attn_merge_rows.
// ---------------------------------------------------------------------------------------------
template <int G, bool KV_BF16, int RB>
__global__ __launch_bounds__(256) void k_attn_causal_bf(BatchAttnParams p) {
  constexpr int D = kHeadDim, BK = 64, TOK = 64 * RB / G, KP = D + 8, VP = BK + 8, NL = KV_BF16 ? 1 : 2;
  __shared__ __align__(16) uint16_t ks[NL][BK][KP];  // [hi, lo][key][dim]
  __shared__ __align__(16) uint16_t vt[NL][D][VP];   // [hi, lo][dim][key slot]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, kg = lane >> 4;
  const uint32_t g = blockIdx.x, mb = blockIdx.y * TOK, run = blockIdx.z, runs = p.runs;
  if (run >= runs) {  // a prefetch workgroup (whole workgroup, before any load)
    l2_prefetch_tiles(p.pf.pf, (run - runs) * gridDim.x * gridDim.y + blockIdx.y * gridDim.x + g,
                      reinterpret_cast<uint32_t*>(p.att));
    return;
  }
  uint32_t tok[RB], head[RB], my_pos[RB];
#pragma unroll
  for (int b = 0; b < RB; b++) {
    const uint32_t row = uint32_t(wave * RB + b) * 16 + uint32_t(li);
    tok[b] = mb + row / G;
    head[b] = g * G + row % G;
    my_pos[b] = p.start + min(tok[b], p.M - 1);
  }
  const uint32_t last = p.start + min(mb + TOK - 1, p.M - 1);  // positions 0..last are needed
  const uint32_t k_begin = run * p.key_run;
  const uint32_t k_end = min(last + 1, k_begin + p.key_run);  // this run: positions [k_begin, k_end)
  // scores in base-2 units: softmax weights are 2^(s log2(e) scale - m), m and the partials' m
  // in the same units
  const float sl2 = p.scale * 1.44269504088896341f;

  bf16x8 qh[RB][4], ql[RB][4];
#pragma unroll
  for (int b = 0; b < RB; b++) {
    const float* qp = p.q + (size_t(min(tok[b], p.M - 1)) * p.n_heads + head[b]) * D + 8 * kg;
#pragma unroll
    for (int st = 0; st < 4; st++) {
      const float4 x = *reinterpret_cast<const float4*>(qp + 32 * st);
      const float4 y = *reinterpret_cast<const float4*>(qp + 32 * st + 4);
      const float v[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
      split8(v, qh[b][st], ql[b][st]);
    }
  }
  f32x4 o[RB][8];
  float m_run[RB], l_run[RB];
#pragma unroll
  for (int b = 0; b < RB; b++) {
#pragma unroll
    for (int i = 0; i < 8; i++) o[b][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[b] = -INFINITY;
    l_run[b] = 0.f;
  }

  // staging: K rows lr + 8 i (i < 8) at dims ld .. ld + 3 (coalesced rows); V key pair
  // 2 vk, 2 vk + 1 at dims 4 vb + 32 i .. +3 (i < 4), so that Vt gets (key, key + 1) words
  const size_t hbase = size_t(g) * p.max_seq * D;
  const int lr = tid >> 5, ld = (tid & 31) * 4, vk = tid & 31, vb = tid >> 5;
  // Vt slot of keys 2 vk, 2 vk + 1 (adjacent slots): key 32 s + 16 h + 4 c + r -> 32 s + 8 c + 4 h + r
  const int vslot = (2 * vk & 32) | ((2 * vk >> 2) & 3) << 3 | ((2 * vk >> 4) & 1) << 2 | (2 * vk & 3);
  using Pre = typename std::conditional<KV_BF16, uint2, float4>::type;
  Pre kp[8], vp[8];
  auto load_k = [&](uint32_t t0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const size_t ko = hbase + size_t(min(t0 + uint32_t(lr + 8 * i), k_end - 1)) * D + ld;
      if constexpr (KV_BF16) kp[i] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.k_cache) + ko);
      else kp[i] = *reinterpret_cast<const float4*>(static_cast<const float*>(p.k_cache) + ko);
    }
  };
  auto load_v = [&](uint32_t t0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const size_t vo = hbase + size_t(min(t0 + uint32_t(2 * vk + (i & 1)), k_end - 1)) * D + 4 * vb + 32 * (i >> 1);
      if constexpr (KV_BF16) vp[i] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.v_cache) + vo);
      else vp[i] = *reinterpret_cast<const float4*>(static_cast<const float*>(p.v_cache) + vo);
    }
  };
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  auto pk = [](float x, float y) __attribute__((always_inline)) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{x, y}), bf16x2));
  };
  auto store_k = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      if constexpr (KV_BF16) {
        *reinterpret_cast<uint2*>(&ks[0][lr + 8 * i][ld]) = kp[i];
      } else {
        const float4 v = kp[i];
        const uint32_t h0 = pk(v.x, v.y), h1 = pk(v.z, v.w);
        *reinterpret_cast<uint2*>(&ks[0][lr + 8 * i][ld]) = make_uint2(h0, h1);
        *reinterpret_cast<uint2*>(&ks[NL - 1][lr + 8 * i][ld]) =
            make_uint2(pk(v.x - __uint_as_float(h0 << 16), v.y - __uint_as_float(h0 & 0xFFFF0000u)),
                       pk(v.z - __uint_as_float(h1 << 16), v.w - __uint_as_float(h1 & 0xFFFF0000u)));
      }
    }
  };
  auto store_v = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; i += 2) {  // vp[i]: key 2 vk, vp[i + 1]: key 2 vk + 1, dims 4 vb + 16 i ..
      const int d0 = 4 * vb + 16 * i;
      if constexpr (KV_BF16) {
        const uint2 x = vp[i], y = vp[i + 1];
        const uint32_t w[4] = {(x.x & 0xFFFFu) | (y.x << 16), (x.x >> 16) | (y.x & 0xFFFF0000u),
                               (x.y & 0xFFFFu) | (y.y << 16), (x.y >> 16) | (y.y & 0xFFFF0000u)};
#pragma unroll
        for (int c = 0; c < 4; c++) *reinterpret_cast<uint32_t*>(&vt[0][d0 + c][vslot]) = w[c];
      } else {
        const float x[4] = {vp[i].x, vp[i].y, vp[i].z, vp[i].w};
        const float y[4] = {vp[i + 1].x, vp[i + 1].y, vp[i + 1].z, vp[i + 1].w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const uint32_t h = pk(x[c], y[c]);
          *reinterpret_cast<uint32_t*>(&vt[0][d0 + c][vslot]) = h;
          *reinterpret_cast<uint32_t*>(&vt[NL - 1][d0 + c][vslot]) =
              pk(x[c] - __uint_as_float(h << 16), y[c] - __uint_as_float(h & 0xFFFF0000u));
        }
      }
    }
  };
  // K and V of the next tile are staged apart, each into its LDS tile as soon as the current
  // tile's last read of it is done (after the scores; after P V), so only one of them is held in
  // registers at a time (-5% against both held across the whole tile)
  if (k_begin < k_end) {
    load_k(k_begin);
    store_k();
    load_v(k_begin);
    store_v();
  }
  for (uint32_t t0 = k_begin; t0 < k_end; t0 += BK) {
    const bool more = t0 + BK < k_end;
    __syncthreads();  // K and V of this tile are in LDS
    if (more) load_k(t0 + BK);

    f32x4 s[RB][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int b = 0; b < RB; b++) s[b][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; st++) {
        const bf16x8 kh = *reinterpret_cast<const bf16x8*>(&ks[0][16 * j + li][32 * st + 8 * kg]);
        bf16x8 kl;
        if constexpr (!KV_BF16) kl = *reinterpret_cast<const bf16x8*>(&ks[NL - 1][16 * j + li][32 * st + 8 * kg]);
#pragma unroll
        for (int b = 0; b < RB; b++) {
          s[b][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[b][st], s[b][j], 0, 0, 0);
          s[b][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[b][st], s[b][j], 0, 0, 0);
          if constexpr (!KV_BF16) s[b][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[b][st], s[b][j], 0, 0, 0);
        }
      }
    }
    bf16x8 ph[RB][2], pl[RB][2];
#pragma unroll
    for (int b = 0; b < RB; b++) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t t = t0 + uint32_t(16 * j + 4 * kg + r);
          const float v = t <= my_pos[b] && t < k_end ? s[b][j][r] * sl2 : -INFINITY;
          s[b][j][r] = v;
          mx = fmaxf(mx, v);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run[b], mx);  // -inf while no key of the run is visible to this row
      // 2^(-inf) = 0 on the hardware exp2: masked keys and a first visible tile weigh 0 with no
      // test per key; m_use keeps -inf - -inf out while nothing is visible
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float corr = __builtin_amdgcn_exp2f(m_run[b] - m_use);
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float e = __builtin_amdgcn_exp2f(s[b][j][r] - m_use);
          s[b][j][r] = e;
          sum += e;
        }
      }
      sum += __shfl_xor(sum, 16);
      sum += __shfl_xor(sum, 32);
      l_run[b] = l_run[b] * corr + sum;
      m_run[b] = m_new;
#pragma unroll
      for (int i = 0; i < 8; i++) o[b][i] *= corr;
#pragma unroll
      for (int st = 0; st < 2; st++) {
        const float pv[8] = {s[b][2 * st][0], s[b][2 * st][1], s[b][2 * st][2], s[b][2 * st][3],
                             s[b][2 * st + 1][0], s[b][2 * st + 1][1], s[b][2 * st + 1][2], s[b][2 * st + 1][3]};
        split8(pv, ph[b][st], pl[b][st]);
      }
    }
    __syncthreads();  // every wave's reads of ks are done
    if (more) {
      store_k();
      load_v(t0 + BK);
    }
#pragma unroll
    for (int st = 0; st < 2; st++) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const bf16x8 vh = *reinterpret_cast<const bf16x8*>(&vt[0][16 * i + li][32 * st + 8 * kg]);
        bf16x8 vl;
        if constexpr (!KV_BF16) vl = *reinterpret_cast<const bf16x8*>(&vt[NL - 1][16 * i + li][32 * st + 8 * kg]);
#pragma unroll
        for (int b = 0; b < RB; b++) {
          o[b][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph[b][st], o[b][i], 0, 0, 0);
          o[b][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl[b][st], o[b][i], 0, 0, 0);
          if constexpr (!KV_BF16) o[b][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph[b][st], o[b][i], 0, 0, 0);
        }
      }
    }
    __syncthreads();  // every wave's reads of vt are done
    if (more) store_v();
  }
  // lane holds O^T[16 i + 4 kg + r][row], r < 4
#pragma unroll
  for (int b = 0; b < RB; b++) {
    if (tok[b] >= p.M) continue;
    const size_t vec = size_t(tok[b]) * p.n_heads + head[b];
    if (runs == 1) {
      const float inv = 1.0f / l_run[b];
      float* out = p.att + vec * D + 4 * kg;
#pragma unroll
      for (int i = 0; i < 8; i++)
        *reinterpret_cast<float4*>(out + 16 * i) =
            make_float4(o[b][i][0] * inv, o[b][i][1] * inv, o[b][i][2] * inv, o[b][i][3] * inv);
    } else {
      float* out = p.part + (vec * runs + run) * kPartStride;
      if (kg == 0) {
        out[0] = m_run[b];
        out[1] = l_run[b];
      }
#pragma unroll
      for (int i = 0; i < 8; i++)
        *reinterpret_cast<float4*>(out + 4 + 16 * i + 4 * kg) = make_float4(o[b][i][0], o[b][i][1], o[b][i][2], o[b][i][3]);
    }
  }
}

// att[v] = sum_s e_s acc_s / sum_s e_s l_s over the runs of query vector v = (token, head),
// e_s = 2^(m_s - max m) (m in base-2 units); runs without a visible key (m = -inf) weigh 0. Two query vectors per
// workgroup of 256 threads (one per dim); all U >= runs run loads are issued at once.
template <int U>
__global__ __launch_bounds__(256) void k_attn_merge_rows(const float* __restrict__ part, uint32_t runs,
                                                         uint32_t n_vec, float* __restrict__ att) {
  const size_t v = min(blockIdx.x * 2 + (threadIdx.x >> 7), n_vec - 1);  // odd count: the last one twice
  const uint32_t d = threadIdx.x & (kHeadDim - 1);
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
  for (int u = 0; u < U; u++) {  // m in base-2 units (k_attn_causal_bf)
    const float e = (uint32_t(u) < runs && mv[u] != -INFINITY) ? exp2f(mv[u] - M) : 0.f;
    L += e * lv[u];
    A += e * av[u];
  }
  att[v * kHeadDim + d] = A / L;
}

// tokens[r] = the greedy token of logits row r by the reference's scan (bench.rs:98-103,
// main.rs:37-42): the largest non-NaN value, lowest index on ties, and 0 when the row starts
// with NaN (or has nothing above -inf). Two launches: kArgParts workgroups per row each reduce
// one slice of the row to a (value, index) candidate, then one wave per row reduces the
// candidates. The comparison is a total order on (value, index) among non-NaN values, so the
// result does not depend on how the row is cut.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_row_argmax_part(const float* __restrict__ logits, uint32_t V, uint32_t S,
                                                         ArgCand* __restrict__ cand) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* x = logits + size_t(blockIdx.y) * V;
  const uint32_t beg = blockIdx.x * S, end = min(V, beg + S);
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  constexpr int U = 4;
  for (uint32_t base = beg; base < end; base += 256u * U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = x[min(base + uint32_t(tid) + 256u * u, V - 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t i = base + uint32_t(tid) + 256u * u;
      if (i < end && cand_better(v[u], i, bv, bi)) { bv = v[u]; bi = i; }  // NaN never wins
    }
  }
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(bv, o);
    const uint32_t oi = __shfl_xor(bi, o);
    if (cand_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; w++)
      if (cand_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    cand[size_t(blockIdx.y) * kArgParts + blockIdx.x] = ArgCand{bv, bi};
  }
}

// err_in / err_out (optional): workgroup 0 also copies the error word to err_out, so a host that
// waits for tokens (and err_out) in pinned memory learns of a failed pass without synchronizing
__global__ __launch_bounds__(64) void k_row_argmax_final(const ArgCand* __restrict__ cand,
                                                         const float* __restrict__ logits, uint32_t V,
                                                         uint32_t* __restrict__ tokens, const uint32_t* err_in,
                                                         uint32_t* err_out) {
  static_assert(kArgParts == 64, "one candidate per lane");
  const uint32_t row = blockIdx.x, lane = threadIdx.x;
  const ArgCand c = cand[size_t(row) * kArgParts + lane];
  const bool nan0 = isnan(logits[size_t(row) * V]);
  float bv = c.v;
  uint32_t bi = c.i;
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(bv, o);
    const uint32_t oi = __shfl_xor(bi, o);
    if (cand_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane == 0) tokens[row] = (nan0 || bi == 0xFFFFFFFFu) ? 0u : bi;
  if (err_out && row == 0 && lane == 0) __atomic_store_n(err_out, *err_in, __ATOMIC_RELAXED);
}

// x[m] = bf16 embedding row of ids[m] (cpu_inference.rs:109-111)
__global__ __launch_bounds__(256) void k_embed_rows(const uint16_t* __restrict__ table, const uint32_t* __restrict__ ids,
                                                    uint32_t M, uint32_t H, float* __restrict__ x) {
  const uint32_t m = blockIdx.y;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < H; i += gridDim.x * 256)
    x[size_t(m) * H + i] = bf16f(table[size_t(ids[m]) * H + i]);
}

// the same with the ids in the kernel argument
__global__ __launch_bounds__(256) void k_embed_rows_v(const uint16_t* __restrict__ table, TokenIds ids, uint32_t H,
                                                      float* __restrict__ x) {
  const uint32_t m = blockIdx.y;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < H; i += gridDim.x * 256)
    x[size_t(m) * H + i] = bf16f(table[size_t(ids.id[m]) * H + i]);
}

// column tile of k_gemm_tile: 128 when that alone gives a tile per CU, else 64
uint32_t tile_bn(uint32_t M, uint32_t N) { return ceil_div(M, 128) * ceil_div(N, 128) >= 256 ? 128 : 64; }

// register prefetch depth of k_gemm_tile: stages in flight per thread
constexpr int kTileDepth = 2;

// k_gemm_rows8 serves M rows of a K-deep product
bool rows_kernel(uint32_t M, uint32_t K) { return M > kGemmTileMinM && M <= kGemmRowsMaxM && K % 64 == 0; }

// k_gemm_rows8 over `splits` K splits (K % (64 splits) == 0, checked by the callers)
// Column tile of k_gemm_rows8 for an unsplit launch. The kernel is bound by what a CU pulls from
// L2 (A 16 KB and W BN x 128 B per 64-deep step), so the tile is the one with the fewest bytes
// on the busiest CU: rounds of 256 workgroups x bytes per step. For gate|up at 512 rows
// (N = 6144) 192 columns give 256 workgroups at 40 KB a step against 384 at 32 KB (half the CUs
// running two).
uint32_t rows_bn(uint32_t M, uint32_t N, uint32_t splits) {
  if (splits != 1 || N % 192) return 128;
  const uint64_t rounds128 = ceil_div(ceil_div(N, 128) * ceil_div(M, 64), 256u);
  const uint64_t rounds192 = ceil_div(ceil_div(N, 192) * ceil_div(M, 64), 256u);
  return rounds192 * (16 + 24) < rounds128 * (16 + 16) ? 192 : 128;
}

template <bool NRM, int E>
void launch_rows(const GemmParams& p, uint32_t splits, hipStream_t st) {
  if constexpr (E == kGemmStore || E == kGemmSiluPair || E == kGemmResAdd) {
    if (rows_bn(p.M, p.N, splits) == 192) {
      // two steps in flight where the step count allows (-1% on the 2048-token prefill; the
      // 128-column tile gains nothing from it)
      const dim3 g(ceil_div(p.N, 192), ceil_div(p.M, 64), splits);
      if ((p.K / splits / 64) % 2 == 0)
        hipLaunchKernelGGL((k_gemm_rows8<NRM, E, 192, 2>), g, dim3(512), 0, st, p, BatchAttnParams{});
      else
        hipLaunchKernelGGL((k_gemm_rows8<NRM, E, 192, 1>), g, dim3(512), 0, st, p, BatchAttnParams{});
      return;
    }
  }
  const dim3 g(ceil_div(p.N, 128), ceil_div(p.M, 64), splits);
  hipLaunchKernelGGL((k_gemm_rows8<NRM, E, 128, 1>), g, dim3(512), 0, st, p, BatchAttnParams{});
}

// k_gemm_tile over `splits` K splits (K % (32 splits) == 0, checked by the callers), with the
// deepest register prefetch that divides the stage count
template <bool NRM, int E>
void launch_tile(const GemmParams& p, uint32_t splits, hipStream_t st) {
  const uint32_t bn = tile_bn(p.M, p.N), nst = p.K / splits / 32;
  const dim3 tg(ceil_div(p.N, bn), ceil_div(p.M, 128), splits);
#define QE_TILE_D(D)                                                                             \
  do {                                                                                           \
    if (bn == 128) hipLaunchKernelGGL((k_gemm_tile<NRM, E, 128, D>), tg, dim3(256), 0, st, p);   \
    else hipLaunchKernelGGL((k_gemm_tile<NRM, E, 64, D>), tg, dim3(256), 0, st, p);              \
  } while (0)
  if (nst % kTileDepth == 0) QE_TILE_D(kTileDepth);
  else if (nst % 2 == 0) QE_TILE_D(2);
  else QE_TILE_D(1);
#undef QE_TILE_D
}

// ---------------------------------------------------------------------------------------------
// Matvec over the NV = M token rows of a short verify pass or chunk (M <= kMvRowsMaxM): the
// decode step's matvec layout. A row group of TPR threads covers one weight row in 8-column
// chunks (CPT per thread) and RR rows per group; each weight chunk is loaded once (128-bit) and
// multiplied by the NV token rows in f32 FMA, so the weights stream once per pass as in a decode
// step. With NORM every row group computes the sum of squares of each token row over its own
// chunks (which cover the row) and scales the dot products, s * sum_c W[r,c] (x_c * g_c)
// (cpu_inference.rs:189-194, 225-257). All loads are issued before the first use. Each token row
// costs every wave its own products and lane reductions, so past a few rows the matrix cores
// (k_gemm_skinny) are faster.
// ---------------------------------------------------------------------------------------------
template <int TPR, int CPT, int RR, int NV, bool NORM, int EPI, int SM = 0>
__global__ __launch_bounds__(256) void k_mv_rows(MvRowsParams p) {
  constexpr int NG = 256 / TPR, WPG = TPR / 64, NS = NV * (RR + 1);
  __shared__ float red[4][NS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = tid / TPR, t = tid % TPR;
  const uint32_t nch = p.cols >> 3;
  const uint32_t row0 = (blockIdx.x * NG + uint32_t(grp)) * RR;
  uint32_t cc[CPT];
#pragma unroll
  for (int k = 0; k < CPT; k++) cc[k] = min(uint32_t(t) + uint32_t(TPR) * k, nch - 1);

  // SM > 0: x is merged from the attention's partials (SM slots per chunk, the split kernel's
  // layout), loaded before the weights as the decode step's o_proj does
  float2 ml[SM > 0 ? NV : 1][CPT][SM > 0 ? SM : 1];
  float4 a0[SM > 0 ? NV : 1][CPT][SM > 0 ? SM : 1], a1[SM > 0 ? NV : 1][CPT][SM > 0 ? SM : 1];
  if constexpr (SM > 0) {
    const uint32_t S = p.attn_splits, th = p.tok_heads, GT = uint32_t(NV) * th;
#pragma unroll
    for (int v = 0; v < NV; v++) {
#pragma unroll
      for (int k = 0; k < CPT; k++) {
        const uint32_t h = cc[k] >> 4, d0 = (cc[k] & 15) * 8, g = h / th, j = uint32_t(v) * th + h % th;
#pragma unroll
        for (int s = 0; s < SM; s++) {
          const float* q = p.attn_part + ((size_t(g) * S + min(uint32_t(s), S - 1)) * GT + j) * kPartStride;
          ml[v][k][s] = *reinterpret_cast<const float2*>(q);
          a0[v][k][s] = *reinterpret_cast<const float4*>(q + 4 + d0);
          a1[v][k][s] = *reinterpret_cast<const float4*>(q + 8 + d0);
        }
      }
    }
  }
  const uint4* W = reinterpret_cast<const uint4*>(p.w);
  uint4 wv[RR][CPT];
#pragma unroll
  for (int r = 0; r < RR; r++) {
    const size_t row = min(row0 + uint32_t(r), p.rows - 1);
#pragma unroll
    for (int k = 0; k < CPT; k++) wv[r][k] = W[row * nch + cc[k]];
  }
  const float4* X = reinterpret_cast<const float4*>(p.x);
  float4 xa[NV][CPT], xb[NV][CPT];
  if constexpr (SM == 0) {
#pragma unroll
    for (int v = 0; v < NV; v++) {
#pragma unroll
      for (int k = 0; k < CPT; k++) {
        xa[v][k] = X[size_t(v) * (p.cols >> 2) + 2 * cc[k]];
        xb[v][k] = X[size_t(v) * (p.cols >> 2) + 2 * cc[k] + 1];
      }
    }
  }
  uint4 gains[CPT];
  if constexpr (NORM) {
#pragma unroll
    for (int k = 0; k < CPT; k++) gains[k] = reinterpret_cast<const uint4*>(p.gain)[cc[k]];
  }
  float res[NV][RR];
  if constexpr (EPI == kGemmResAdd) {
#pragma unroll
    for (int v = 0; v < NV; v++)
#pragma unroll
      for (int r = 0; r < RR; r++) res[v][r] = p.out[size_t(v) * p.ldo + min(row0 + uint32_t(r), p.rows - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (SM > 0) {
    // x = sum_s e_s acc_s / sum_s e_s l_s, e_s = exp(m_s - max m) (cpu_inference.rs:153-160 over
    // the runs); empty runs (m = -inf) and slots past the last run weigh 0
    const uint32_t S = p.attn_splits;
#pragma unroll
    for (int v = 0; v < NV; v++) {
#pragma unroll
      for (int k = 0; k < CPT; k++) {
        float M = -INFINITY;
#pragma unroll
        for (int s = 0; s < SM; s++) M = uint32_t(s) < S ? fmaxf(M, ml[v][k][s].x) : M;
        float L = 0.f;
        float4 A0 = make_float4(0.f, 0.f, 0.f, 0.f), A1 = A0;
#pragma unroll
        for (int s = 0; s < SM; s++) {
          const float e = (uint32_t(s) < S && ml[v][k][s].x != -INFINITY) ? expf(ml[v][k][s].x - M) : 0.f;
          L += e * ml[v][k][s].y;
          A0.x += e * a0[v][k][s].x; A0.y += e * a0[v][k][s].y; A0.z += e * a0[v][k][s].z; A0.w += e * a0[v][k][s].w;
          A1.x += e * a1[v][k][s].x; A1.y += e * a1[v][k][s].y; A1.z += e * a1[v][k][s].z; A1.w += e * a1[v][k][s].w;
        }
        const float inv = 1.0f / L;
        xa[v][k] = make_float4(A0.x * inv, A0.y * inv, A0.z * inv, A0.w * inv);
        xb[v][k] = make_float4(A1.x * inv, A1.y * inv, A1.z * inv, A1.w * inv);
      }
    }
  }

  if (uint32_t(TPR) * CPT > nch) {  // chunks past the row end contribute 0
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      // component-wise: a ternary between float4 objects selects their addresses and sends the
      // arrays to scratch memory
      const bool in = uint32_t(t) + uint32_t(TPR) * k < nch;
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const float4 a = xa[v][k], b = xb[v][k];
        xa[v][k] = make_float4(in ? a.x : 0.f, in ? a.y : 0.f, in ? a.z : 0.f, in ? a.w : 0.f);
        xb[v][k] = make_float4(in ? b.x : 0.f, in ? b.y : 0.f, in ? b.z : 0.f, in ? b.w : 0.f);
      }
    }
  }
  float ss[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) {
    ss[v] = 0.f;
    if constexpr (NORM) {
#pragma unroll
      for (int k = 0; k < CPT; k++) {
        const float4 a = xa[v][k], b = xb[v][k];
        ss[v] += (a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w) + (b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w);
        const uint4 g = gains[k];
        xa[v][k] = make_float4(a.x * __uint_as_float(g.x << 16), a.y * __uint_as_float(g.x & 0xFFFF0000u),
                               a.z * __uint_as_float(g.y << 16), a.w * __uint_as_float(g.y & 0xFFFF0000u));
        xb[v][k] = make_float4(b.x * __uint_as_float(g.z << 16), b.y * __uint_as_float(g.z & 0xFFFF0000u),
                               b.z * __uint_as_float(g.w << 16), b.w * __uint_as_float(g.w & 0xFFFF0000u));
      }
      ss[v] = wave_sum(ss[v]);
    }
  }
  float acc[NV][RR];
#pragma unroll
  for (int v = 0; v < NV; v++)
#pragma unroll
    for (int r = 0; r < RR; r++) {
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < CPT; k++) a = dot8(wv[r][k], xa[v][k], xb[v][k], a);
      acc[v][r] = wave_sum(a);
    }
  if constexpr (WPG > 1) {
    if (lane == 0) {
#pragma unroll
      for (int v = 0; v < NV; v++) {
#pragma unroll
        for (int r = 0; r < RR; r++) red[wave][v * (RR + 1) + r] = acc[v][r];
        red[wave][v * (RR + 1) + RR] = ss[v];
      }
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < NV; v++)
#pragma unroll
      for (int r = 0; r <= RR; r++) {
        float a = 0.f;
#pragma unroll
        for (int w = 0; w < WPG; w++) a += red[grp * WPG + w][v * (RR + 1) + r];
        if (r < RR) acc[v][r] = a;
        else ss[v] = a;
      }
  }
  if (t != 0) return;
#pragma unroll
  for (int v = 0; v < NV; v++) {
    float sc = 1.f;
    if constexpr (NORM) sc = 1.0f / sqrtf(ss[v] / float(p.cols) + p.eps);
    float* o = p.out + size_t(v) * p.ldo;
    if constexpr (EPI == kGemmSiluPair) {
#pragma unroll
      for (int r = 0; r + 1 < RR; r += 2) {
        const uint32_t row = row0 + uint32_t(r);
        if (row + 1 < p.rows) {
          const float g = acc[v][r] * sc;
          o[row >> 1] = g / (1.0f + expf(-g)) * (acc[v][r + 1] * sc);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < RR; r++) {
        const uint32_t row = row0 + uint32_t(r);
        if (row < p.rows) o[row] = EPI == kGemmResAdd ? res[v][r] + acc[v][r] * sc : acc[v][r] * sc;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// final RMSNorm + lm_head over the NV token rows of a short verify pass: the decode step's lm_head
// matvec (k_matvec<R, CPL, kNorm, ..>: each wave R rows, lane l the 16-byte chunks l, l + 64, ..)
// with the NV normalized rows staged in LDS, so the 311 MB of weights stream once for all rows.
// Each row's norm and dot products are summed in the decode step's order, so a row's logits equal
// that step's bit for bit. out[v][row] = logits, ldo per token row.
// ---------------------------------------------------------------------------------------------
template <int R, int CPL, int NV>
__global__ __launch_bounds__(256) void k_lm_head_rows(MvRowsParams p) {
  extern __shared__ __align__(16) float xs[];  // [NV][cols]
  __shared__ float red[NV][4];
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
    for (int k = 0; k < CPL; k++) wv[r][k] = ld_stream(&wr[min(uint32_t(lane) + 64u * k, nch - 1)]);  // (as k_matvec)
  }
  const float4* x4 = reinterpret_cast<const float4*>(p.x);
  float4* xs4 = reinterpret_cast<float4*>(xs);
  const uint32_t c4 = p.cols / 4;
  // no gain: the rows come normalized (the fused verify pass's final reduce applied the norm)
  const bool norm = p.gain != nullptr;
#pragma unroll
  for (int v = 0; v < NV; v++) {
    float ss = 0.f;
    for (uint32_t i = tid; i < c4; i += 256) {
      const float4 a = x4[size_t(v) * c4 + i];
      xs4[v * c4 + i] = a;
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    if (norm) {
      ss = wave_sum(ss);
      if (lane == 0) red[v][wave] = ss;
    }
  }
  __syncthreads();
  if (norm) {
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const float tot = (red[v][0] + red[v][1]) + (red[v][2] + red[v][3]);
      const float sc = 1.0f / sqrtf(tot / float(p.cols) + p.eps);
      for (uint32_t i = tid; i < p.cols; i += 256) xs[v * p.cols + i] = xs[v * p.cols + i] * sc * bf16f(p.gain[i]);
    }
    __syncthreads();
  }
  float acc[NV][R];
#pragma unroll
  for (int v = 0; v < NV; v++)
#pragma unroll
    for (int r = 0; r < R; r++) acc[v][r] = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; k++) {
    const uint32_t c = uint32_t(lane) + 64u * k;
    if (c < nch) {
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const float4 a = xs4[v * c4 + 2 * c], b = xs4[v * c4 + 2 * c + 1];
#pragma unroll
        for (int r = 0; r < R; r++) acc[v][r] = dot8(wv[r][k], a, b, acc[v][r]);
      }
    }
  }
#pragma unroll
  for (int v = 0; v < NV; v++)
#pragma unroll
    for (int r = 0; r < R; r++) acc[v][r] = wave_sum(acc[v][r]);
  if (lane == 0) {
#pragma unroll
    for (int v = 0; v < NV; v++)
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t row = row0 + uint32_t(r);
        if (row < p.rows) p.out[size_t(v) * p.ldo + row] = acc[v][r];
      }
  }
  if (p.cand) {  // each token row's best (value, row) of this workgroup, NaN never (k_matvec kLogits)
    __shared__ ArgCand cb[NV][4];
#pragma unroll
    for (int v = 0; v < NV; v++) {
      float bv = -INFINITY;
      uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t row = row0 + uint32_t(r);
        if (row < p.rows && !isnan(acc[v][r]) && cand_better(acc[v][r], row, bv, bi)) {
          bv = acc[v][r];
          bi = row;
        }
      }
      if (lane == 0) cb[v][wave] = ArgCand{bv, bi};
    }
    __syncthreads();
    if (tid < NV) {
      ArgCand b = cb[tid][0];
      for (int w = 1; w < 4; w++)
        if (cand_better(cb[tid][w].v, cb[tid][w].i, b.v, b.i)) b = cb[tid][w];
      p.cand[size_t(tid) * gridDim.x + blockIdx.x] = b;
    }
  }
}

// tokens[row] from the row's candidates: the first maximum, NaN never wins, a NaN first logit or
// no candidate above -inf gives 0 (main.rs:37-42; k_argmax's reduction, one workgroup per row)
__global__ __launch_bounds__(1024) void k_cand_argmax(const ArgCand* __restrict__ cand, uint32_t n_cand,
                                                      const float* __restrict__ logits, uint32_t V,
                                                      uint32_t* __restrict__ tokens, const uint32_t* err_in,
                                                      uint32_t* err_out) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t row = blockIdx.x;
  cand += size_t(row) * n_cand;
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
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
    tokens[row] = (isnan(logits[size_t(row) * V]) || bi == 0xFFFFFFFFu) ? 0u : bi;
    if (err_out && row == 0) __atomic_store_n(err_out, *err_in, __ATOMIC_RELAXED);
  }
}

template <int TPR, int CPT, int RR, int NV, bool NORM, int EPI>
hipError_t launch_mv_rows_t(const MvRowsParams& p, hipStream_t st) {
  constexpr int rows_per_block = (256 / TPR) * RR;
  hipLaunchKernelGGL((k_mv_rows<TPR, CPT, RR, NV, NORM, EPI>), dim3(ceil_div(p.rows, rows_per_block)), dim3(256), 0,
                     st, p);
  return hipGetLastError();
}

// the decode matvec's shapes: an exact fit of threads x chunks where one exists; silu rows pair up
template <int NV, bool NORM, int EPI>
hipError_t launch_mv_rows_cols(const MvRowsParams& p, hipStream_t st) {
  const uint32_t nch = p.cols / 8;
  constexpr bool SILU = EPI == kGemmSiluPair;
  if (nch <= 64) return launch_mv_rows_t<64, 1, 2, NV, NORM, EPI>(p, st);
  if (nch <= 128) {
    if (SILU) return launch_mv_rows_t<64, 2, 2, NV, NORM, EPI>(p, st);
    return launch_mv_rows_t<128, 1, 2, NV, NORM, EPI>(p, st);
  }
  if (nch <= 256) return launch_mv_rows_t<256, 1, SILU ? 2 : 1, NV, NORM, EPI>(p, st);
  if (nch == 384) return launch_mv_rows_t<128, 3, 2, NV, NORM, EPI>(p, st);
  if (nch <= 512) return launch_mv_rows_t<256, 2, SILU ? 2 : 1, NV, NORM, EPI>(p, st);
  return hipErrorInvalidValue;
}

template <int NV>
hipError_t launch_mv_rows_nv(const MvRowsParams& p, bool norm, int epi, hipStream_t st) {
  if (norm && epi == kGemmStore) return launch_mv_rows_cols<NV, true, kGemmStore>(p, st);
  if (norm && epi == kGemmSiluPair) return launch_mv_rows_cols<NV, true, kGemmSiluPair>(p, st);
  if (!norm && epi == kGemmResAdd) return launch_mv_rows_cols<NV, false, kGemmResAdd>(p, st);
  if (!norm && epi == kGemmStore) return launch_mv_rows_cols<NV, false, kGemmStore>(p, st);
  return hipErrorInvalidValue;
}

// o_proj with the attention merge: four rows per workgroup amortize the merge, which every
// workgroup repeats for all heads of its token rows
template <int NV, int SM>
hipError_t launch_mv_merge_t(const MvRowsParams& p, hipStream_t st) {
  const uint32_t nch = p.cols / 8;
  if (nch <= 128) {
    hipLaunchKernelGGL((k_mv_rows<128, 1, 4, NV, false, kGemmResAdd, SM>), dim3(ceil_div(p.rows, 8u)), dim3(256), 0,
                       st, p);
  } else {
    hipLaunchKernelGGL((k_mv_rows<256, 1, 4, NV, false, kGemmResAdd, SM>), dim3(ceil_div(p.rows, 4u)), dim3(256), 0,
                       st, p);
  }
  return hipGetLastError();
}

uint32_t mv_merge_slots(uint32_t splits) { return splits <= 4 ? 4 : splits <= 8 ? 8 : 16; }

template <int NV>
hipError_t launch_mv_merge_nv(const MvRowsParams& p, hipStream_t st) {
  const uint32_t sm = mv_merge_slots(p.attn_splits);
  if (sm == 4) return launch_mv_merge_t<NV, 4>(p, st);
  if constexpr (NV <= 2) {
    if (sm == 8) return launch_mv_merge_t<NV, 8>(p, st);
  }
  if constexpr (NV == 1) return launch_mv_merge_t<NV, 16>(p, st);
  return hipErrorNotSupported;
}

}  // namespace

bool mv_rows_merge_fits(uint32_t M, uint32_t splits) {
  return M >= 1 && M <= kMvRowsMaxM && splits >= 1 && splits <= uint32_t(kAttnMaxMergeSplits) &&
         M * mv_merge_slots(splits) <= 16;
}

hipError_t launch_mv_rows_merge(const MvRowsParams& p, hipStream_t st) {
  if (!p.w || !p.out || !p.attn_part || p.M == 0 || p.M > kMvRowsMaxM || p.rows == 0 || p.cols == 0 ||
      p.ldo < p.rows || p.attn_splits == 0 || p.tok_heads == 0)
    return hipErrorInvalidValue;
  if (p.cols % kHeadDim || p.cols / 8 > 256 || !mv_rows_merge_fits(p.M, p.attn_splits)) return hipErrorNotSupported;
  switch (p.M) {
    case 1: return launch_mv_merge_nv<1>(p, st);
    case 2: return launch_mv_merge_nv<2>(p, st);
    case 3: return launch_mv_merge_nv<3>(p, st);
    default: return launch_mv_merge_nv<4>(p, st);
  }
}

uint32_t lm_head_rows_workgroups(uint32_t rows) { return ceil_div(rows, 4u * 4u); }

hipError_t launch_cand_argmax(const ArgCand* cand, uint32_t n_cand, const float* logits, uint32_t rows, uint32_t V,
                              uint32_t* tokens, hipStream_t st, const uint32_t* err_in, uint32_t* err_out) {
  if (!cand || !logits || !tokens || n_cand == 0 || rows == 0 || V == 0 || rows > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_cand_argmax, dim3(rows), dim3(1024), 0, st, cand, n_cand, logits, V, tokens, err_in, err_out);
  return hipGetLastError();
}

hipError_t launch_lm_head_rows(const MvRowsParams& p, hipStream_t st) {
  if (!p.w || !p.x || !p.out || p.M == 0 || p.M > kMvRowsMaxM || p.rows == 0 || p.cols == 0 ||
      p.cols % 8 || p.ldo < p.rows)
    return hipErrorInvalidValue;
  if (p.cols / 8 > 128) return hipErrorNotSupported;  // the decode lm_head's shape: 2 chunks per lane
  constexpr int CPL = 2, R = 4;
  const dim3 grid(ceil_div(p.rows, 4u * R));
  const size_t lds = size_t(p.M) * p.cols * 4;
  switch (p.M) {
    case 1: hipLaunchKernelGGL((k_lm_head_rows<R, CPL, 1>), grid, dim3(256), lds, st, p); break;
    case 2: hipLaunchKernelGGL((k_lm_head_rows<R, CPL, 2>), grid, dim3(256), lds, st, p); break;
    case 3: hipLaunchKernelGGL((k_lm_head_rows<R, CPL, 3>), grid, dim3(256), lds, st, p); break;
    default: hipLaunchKernelGGL((k_lm_head_rows<R, CPL, 4>), grid, dim3(256), lds, st, p); break;
  }
  return hipGetLastError();
}

hipError_t launch_mv_rows(const MvRowsParams& p, bool norm, int epi, hipStream_t st) {
  if (!p.w || !p.x || !p.out || (norm && !p.gain) || p.M == 0 || p.M > kMvRowsMaxM || p.rows == 0 || p.cols == 0 ||
      p.cols % 8 || p.cols / 8 > 512 || (epi == kGemmSiluPair ? p.rows % 2 || p.ldo < p.rows / 2 : p.ldo < p.rows))
    return hipErrorInvalidValue;
  switch (p.M) {
    case 1: return launch_mv_rows_nv<1>(p, norm, epi, st);
    case 2: return launch_mv_rows_nv<2>(p, norm, epi, st);
    case 3: return launch_mv_rows_nv<3>(p, norm, epi, st);
    default: return launch_mv_rows_nv<4>(p, norm, epi, st);
  }
}

L2Prefetch skinny_prefetch_target(const uint16_t* W, uint32_t N, uint32_t K) {
  return L2Prefetch{W, N * (K / 8), 16 * (K / 8), ceil_div(N, 16u)};
}

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
    if (norm && epi == kGemmStore) launch_skinny<true, kGemmStore>(p, 1, st);
    else if (norm && epi == kGemmSiluPair) launch_skinny<true, kGemmSiluPair>(p, 1, st);
    else if (!norm && epi == kGemmStore) launch_skinny<false, kGemmStore>(p, 1, st);
    else if (!norm && epi == kGemmResAdd) launch_skinny<false, kGemmResAdd>(p, 1, st);
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
  if (norm && !p.rowscale) return hipErrorInvalidValue;
  if (rows_kernel(p.M, p.K)) {
    if (norm && epi == kGemmStore) launch_rows<true, kGemmStore>(p, 1, st);
    else if (norm && epi == kGemmSiluPair) launch_rows<true, kGemmSiluPair>(p, 1, st);
    else if (!norm && epi == kGemmStore) launch_rows<false, kGemmStore>(p, 1, st);
    else if (!norm && epi == kGemmResAdd) launch_rows<false, kGemmResAdd>(p, 1, st);
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
  if (p.M > kGemmTileMinM) {
    if (norm && epi == kGemmStore) launch_tile<true, kGemmStore>(p, 1, st);
    else if (norm && epi == kGemmSiluPair) launch_tile<true, kGemmSiluPair>(p, 1, st);
    else if (!norm && epi == kGemmStore) launch_tile<false, kGemmStore>(p, 1, st);
    else if (!norm && epi == kGemmResAdd) launch_tile<false, kGemmResAdd>(p, 1, st);
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
  const dim3 grid(ceil_div(p.N, 64), ceil_div(p.M, 64));
  if (p.K % 64 == 0) {
    if (norm && epi == kGemmStore) hipLaunchKernelGGL((k_gemm_lds<true, kGemmStore>), grid, dim3(256), 0, st, p);
    else if (norm && epi == kGemmSiluPair) hipLaunchKernelGGL((k_gemm_lds<true, kGemmSiluPair>), grid, dim3(256), 0, st, p);
    else if (!norm && epi == kGemmStore) hipLaunchKernelGGL((k_gemm_lds<false, kGemmStore>), grid, dim3(256), 0, st, p);
    else if (!norm && epi == kGemmResAdd) hipLaunchKernelGGL((k_gemm_lds<false, kGemmResAdd>), grid, dim3(256), 0, st, p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
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

uint32_t gemm_splits(uint32_t M, uint32_t N, uint32_t K) {
  // tiles of the kernel that runs M rows, and the depth one split must stay a multiple of
  uint32_t tiles, unit;
  if (M <= kGemmSkinnyMaxM) {
    tiles = ceil_div(N, 16);
    unit = 32;
  } else if (M <= kGemmTileMinM) {
    tiles = ceil_div(N, 64) * ceil_div(M, 64);
    unit = 64;
  } else if (rows_kernel(M, K)) {
    tiles = ceil_div(N, 128) * ceil_div(M, 64);
    unit = 64;
  } else {
    tiles = ceil_div(N, tile_bn(M, N)) * ceil_div(M, 128);
    unit = 32;
  }
  uint32_t z = 1;
  while (z < 8 && tiles * z < 256 && K % (2 * unit * z) == 0) z *= 2;
  return z;
}

hipError_t launch_gemm_split(const GemmParams& p, uint32_t splits, hipStream_t st) {
  if (p.M == 0 || p.N == 0 || p.N % 2 || p.lda % 4 || !p.A || !p.W || !p.C || splits == 0)
    return hipErrorInvalidValue;
  if (p.M <= kGemmSkinnyMaxM) {
    if (p.K % (32 * splits)) return hipErrorInvalidValue;
    launch_skinny<false, kGemmPartial>(p, splits, st);
    return hipGetLastError();
  }
  if (rows_kernel(p.M, p.K) && p.K % (64 * splits) == 0) {
    launch_rows<false, kGemmPartial>(p, splits, st);
    return hipGetLastError();
  }
  if (p.M > kGemmTileMinM) {
    if (p.K % (32 * splits)) return hipErrorInvalidValue;
    launch_tile<false, kGemmPartial>(p, splits, st);
    return hipGetLastError();
  }
  if (p.K % (64 * splits)) return hipErrorInvalidValue;
  const dim3 grid(ceil_div(p.N, 64), ceil_div(p.M, 64), splits);
  hipLaunchKernelGGL((k_gemm_lds<false, kGemmPartial>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

L2Prefetch gemm_prefetch_target(const uint16_t* W, uint32_t M, uint32_t N, uint32_t K, int epi) {
  if (!W || !rows_kernel(M, K)) return L2Prefetch{};
  const uint32_t bn = epi == kGemmQkRope || epi == kGemmPartial ? 128 : rows_bn(M, N, 1);
  const uint32_t tiles = ceil_div(N, bn);
  // workgroup (j, y, z) runs on XCD (j + tiles (y + gridDim.y z)) % 8: j % 8 when tiles is a
  // multiple of 8 or the grid is one row of tiles
  if (tiles % 8 && (ceil_div(M, 64) > 1 || epi == kGemmPartial)) return L2Prefetch{};
  return L2Prefetch{W, N * (K / 8), bn * (K / 8), tiles};
}

uint32_t tile_prefetch_slots(const L2Prefetch* pf, int n) {
  uint64_t tot = 0;  // XCD 0 has the most consumers
  for (int i = 0; i < n; i++)
    if (pf[i].w && pf[i].n_cwg) tot += uint64_t(ceil_div(pf[i].n_cwg, 8u)) * pf[i].cw_chunks;
  return uint32_t(std::min<uint64_t>(64, (tot + 4095) / 4096));
}

hipError_t launch_resadd_partials(float* x, const float* part, uint32_t splits, uint32_t M, uint32_t N, float eps,
                                  float* s, hipStream_t st) {
  if (!M || N % 4 || !splits) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_resadd_partials, dim3(M), dim3(256), 0, st, x, part, splits, M, N, eps, s);
  return hipGetLastError();
}

hipError_t launch_gemm_qk_rope(const GemmParams& g, const BatchAttnParams& a, hipStream_t st) {
  if (!rows_kernel(g.M, g.K) || g.M != a.M || g.N != (a.n_heads + 2 * a.n_kv) * kHeadDim || !g.rowscale || !g.gain ||
      !a.q || !a.q_norm || !a.k_norm || !a.rope || !a.k_cache || !a.v_cache || g.lda % 4 || !g.A || !g.W)
    return hipErrorNotSupported;
  if (uint64_t(a.start) + a.M > a.max_seq) return hipErrorInvalidValue;  // the K/V rows must fit the cache
  const dim3 grid(g.N / 128, ceil_div(g.M, 64), 1);
  hipLaunchKernelGGL((k_gemm_rows8<true, kGemmQkRope, 128, 1>), grid, dim3(512), 0, st, g, a);
  return hipGetLastError();
}

hipError_t launch_qk_rope(const BatchAttnParams& p, hipStream_t st) {
  const uint32_t items = p.M * (p.n_heads + 2 * p.n_kv);
  hipLaunchKernelGGL(k_qk_rope, dim3(ceil_div(items, 4)), dim3(256), 0, st, p);
  return hipGetLastError();
}

// Row blocks per wave of k_attn_causal_bf. One: at 2048 tokens in chunks of 512, two (half the
// workgroups, each LDS fragment feeding twice the MFMAs) took 15.1 ms against 13.9, and eight
// waves of one block (twice the LDS reads per tile) 14.6.
constexpr uint32_t kAttnCausalRB = 1;

hipError_t launch_attn_causal(const BatchAttnParams& p, uint32_t runs, hipStream_t st) {
  if (!p.n_kv || p.n_heads % p.n_kv || runs == 0 || runs > uint32_t(kBatchMaxRuns) || (runs > 1 && !p.part))
    return hipErrorInvalidValue;
  const uint32_t G = p.n_heads / p.n_kv;
  BatchAttnParams q = p;
  // runs of whole 64-position tiles covering positions 0 .. start + M - 1, none of them empty
  const uint32_t tiles = ceil_div(p.start + p.M, 64), per_run = ceil_div(tiles, runs);
  runs = ceil_div(tiles, per_run);
  q.key_run = 64 * per_run;
  q.runs = runs;
  if (q.pf.slots > 64) return hipErrorInvalidValue;
  constexpr uint32_t RB = kAttnCausalRB;
  const uint32_t gy = ceil_div(p.M, 64 * RB / G);
  // prefetch workgroups: whole planes after the runs' (8 x slots of them at consecutive ids)
  const uint32_t planes = q.pf.slots ? ceil_div(8 * q.pf.slots, p.n_kv * gy) : 0;
  const dim3 grid(p.n_kv, gy, runs + planes);
  hipError_t e = hipErrorInvalidValue;
#define QE_ATT(GG)                                                                                         \
  if (G == GG) {                                                                                           \
    if (p.kv_bf16) hipLaunchKernelGGL((k_attn_causal_bf<GG, true, RB>), grid, dim3(256), 0, st, q);        \
    else hipLaunchKernelGGL((k_attn_causal_bf<GG, false, RB>), grid, dim3(256), 0, st, q);                 \
    e = hipGetLastError();                                                                                 \
  }
  QE_ATT(1)
  QE_ATT(2)
  QE_ATT(4)
  QE_ATT(8)
#undef QE_ATT
  if (e != hipSuccess || runs == 1) return e;
  const uint32_t n_vec = p.M * p.n_heads;
  const dim3 mg(ceil_div(n_vec, 2));
  if (runs <= 4) hipLaunchKernelGGL((k_attn_merge_rows<4>), mg, dim3(256), 0, st, p.part, runs, n_vec, p.att);
  else if (runs <= 8) hipLaunchKernelGGL((k_attn_merge_rows<8>), mg, dim3(256), 0, st, p.part, runs, n_vec, p.att);
  else if (runs <= 16) hipLaunchKernelGGL((k_attn_merge_rows<16>), mg, dim3(256), 0, st, p.part, runs, n_vec, p.att);
  else hipLaunchKernelGGL((k_attn_merge_rows<32>), mg, dim3(256), 0, st, p.part, runs, n_vec, p.att);
  return hipGetLastError();
}

uint32_t attn_causal_runs(uint32_t M, uint32_t start, uint32_t n_heads, uint32_t n_kv) {
  if (!M || !n_kv || n_heads % n_kv || n_heads / n_kv > 16) return 1;
  const uint32_t wgs = n_kv * ceil_div(M, 64 * kAttnCausalRB / (n_heads / n_kv));
  // at least 4 runs, more while that leaves under 512 workgroups (measured: 4 runs beat 2 and 8
  // at M = 512 and 1 and 2 at M = 2048); at most kBatchMaxRuns
  uint32_t runs = std::min(std::max(ceil_div(512, wgs), 4u), uint32_t(kBatchMaxRuns));
  return std::max(1u, std::min(runs, ceil_div(start + M, 128)));
}

hipError_t launch_row_argmax(const float* logits, uint32_t rows, uint32_t V, uint32_t* tokens, ArgCand* cand,
                             hipStream_t st, const uint32_t* err_in, uint32_t* err_out) {
  if (!rows || !V || !cand || rows > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_row_argmax_part, dim3(kArgParts, rows), dim3(256), 0, st, logits, V, ceil_div(V, kArgParts),
                     cand);
  hipLaunchKernelGGL(k_row_argmax_final, dim3(rows), dim3(64), 0, st, cand, logits, V, tokens, err_in, err_out);
  return hipGetLastError();
}

hipError_t launch_embed_rows(const uint16_t* table, const uint32_t* ids, uint32_t M, uint32_t H, float* x,
                             hipStream_t st) {
  hipLaunchKernelGGL(k_embed_rows, dim3(ceil_div(H, 256), M), dim3(256), 0, st, table, ids, M, H, x);
  return hipGetLastError();
}

hipError_t launch_embed_rows(const uint16_t* table, const TokenIds& ids, uint32_t M, uint32_t H, float* x,
                             hipStream_t st) {
  if (M == 0 || M > kIdsByValue) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_embed_rows_v, dim3(ceil_div(H, 256), M), dim3(256), 0, st, table, ids, H, x);
  return hipGetLastError();
}

}  // namespace qe
