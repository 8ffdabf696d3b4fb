// GQA decode attention for one new token (inference.metal:194-296, cpu_inference.rs:134-162).
//
// grid (n_kv, splits): workgroup (g, s) serves all G q heads of KV head g over the run of
// positions [s*chunk, (s+1)*chunk) from a single read of that run's K and V, and writes one
// (m, l, acc) partial per q head. In the decode step the workgroups also apply the per-head q/k
// RMSNorm and RoPE, and the one whose run holds the new position appends k and v to the cache
// (cpu_inference.rs:134-141); the o_proj matvec merges the partials in its prologue. The
// isolated op (qe_op_attention) runs the same kernel on a final q and a complete cache, then
// k_attn_merge.
#include "kernels.h"

#include <cmath>

#include "attn_tile.h"
#include "device_common.h"
#include "l2_prefetch.h"

namespace qe {
namespace {

// ---------------------------------------------------------------------------------------------
// Attention over a fixed split of the cache: workgroup (g, s) covers positions
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
// The workgroup writes its (m, l, acc) partial per q head; a run past the last position writes
// an empty one (m = -inf, l = 0, acc = 0).
// ---------------------------------------------------------------------------------------------
template <int G, bool KV_BF16, bool DECODE>
__global__ __launch_bounds__(256) void k_attn_split(AttnParams p, uint32_t chunk) {
  if (blockIdx.y >= p.splits) {  // a prefetch workgroup (whole workgroup, before any load)
    const uint32_t q = (blockIdx.y - p.splits) * gridDim.x + blockIdx.x;
    if (q < 8 * p.pf_slots && (!DECODE || p.state->pos < p.pf_max_pos)) l2_prefetch(p.pf, p.pf_slots, q, p.err);
    return;
  }
  // DECODE: q/k RMSNorm + RoPE on the raw q|k|v rows, append of the new K/V row, positions
  // 0..state->pos; otherwise (the isolated op) q is final and positions are 0..n_pos_fixed-1
  constexpr int D = kHeadDim, T = 64, NR = DECODE ? G + 2 : G, RPW = (NR + 3) / 4;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, so branches on it are scalar
  const int pg = tid >> 3, dc = tid & 7, dg = tid & 31, pp = tid >> 5;
  // rows of several tokens may be split over row_split workgroups per KV head: this one serves
  // rows rbase .. rbase + G - 1 of the GT rows of KV head g
  const uint32_t rsplit = !DECODE && p.row_split > 1 ? p.row_split : 1u;
  const uint32_t g = blockIdx.x / rsplit, rbase = (blockIdx.x % rsplit) * G, GT = G * rsplit, s = blockIdx.y;
  const size_t head_base = size_t(g) * p.max_seq * D;
  // Decode sizes the runs from the current length (below); the first tile is loaded up front
  // for runs of a single tile, which is what every step up to 64 * splits positions has.
  // the first run start: known at launch unless the decode step has no run length from the host
  const uint32_t t0_first = DECODE ? s * (p.run ? p.run : uint32_t(T)) : s * chunk;

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
    size_t off = r < G ? (size_t(g) * G + r) * D
                       : size_t(p.n_heads) * D + (r == G ? 0 : size_t(p.n_kv) * D) + size_t(g) * D;
    if (!DECODE && p.tok_heads) {  // rows of several tokens: token r / tok_heads, head g tok_heads + r % tok_heads
      const uint32_t rr = rbase + uint32_t(r);
      off = size_t(rr / p.tok_heads) * p.q_tok_stride + (size_t(g) * p.tok_heads + rr % p.tok_heads) * D;
    }
    ra[i] = p.qkv[off + lane];
    rb[i] = p.qkv[off + lane + 64];
  }
  float gqa = 0.f, gqb = 0.f, gka = 0.f, gkb = 0.f;
  float2 cs = make_float2(0.f, 0.f);
  if constexpr (DECODE) {
    gqa = bf16f(p.q_norm[lane]);
    gqb = bf16f(p.q_norm[lane + 64]);
    gka = bf16f(p.k_norm[lane]);
    gkb = bf16f(p.k_norm[lane + 64]);
    cs = reinterpret_cast<const float2*>(p.rope_cur)[lane];
  }
  KVTile<KV_BF16> A, B;
  load_tile<KV_BF16>(A, p.k_cache, p.v_cache, p.max_seq, head_base, t0_first, tid);
  __builtin_amdgcn_sched_barrier(0);  // keep the scheduler from sinking these loads to their uses

  // a run with no cached position (t1 <= t0) goes through one all-masked tile and writes the
  // empty partial m = -inf, l = 0, acc = 0
  uint32_t pos, n, run, t0;
  bool owns_new = false;  // this run holds the new position
  if constexpr (DECODE) {
    pos = p.state->pos;
    const bool bad = pos >= p.max_seq;
    if (bad && g == 0 && s == 0 && tid == 0) atomicOr(p.err, kErrPos);
    n = bad ? 0u : pos + 1;
    if (p.run) {
      // runs of the host's length; positions they do not cover would be skipped: flag that
      run = p.run;
      if (n > p.splits * run) {
        if (g == 0 && s == 0 && tid == 0) atomicOr(p.err, kErrShape);
        n = 0;
      }
    } else {
      // the n positions in p.splits runs of a whole number of tiles
      run = T * ceil_div(max(n, 1u), T * p.splits);
    }
    t0 = s * run;
    owns_new = n != 0 && pos >= t0 && pos < t0 + run;
    if (!p.run && run != T) load_tile<KV_BF16>(A, p.k_cache, p.v_cache, p.max_seq, head_base, t0, tid);  // longer runs start elsewhere
  } else {
    n = p.n_pos_fixed;
    pos = n - 1;
    run = chunk;
    t0 = t0_first;
  }
  const uint32_t t1 = min(n, t0 + run);
  float* part = p.partial + ((size_t(g) * p.splits + s) * GT + rbase) * kPartStride;
  // per-row causal limit: with rows of several tokens, token i of T sees positions < n - (T - 1 - i)
  uint32_t lim[G];
#pragma unroll
  for (int j = 0; j < G; j++) {
    lim[j] = n;
    if (!DECODE && p.tok_heads) lim[j] = n - (GT / p.tok_heads - 1u - (rbase + uint32_t(j)) / p.tok_heads);
  }

  // ---- q/k RMSNorm (cpu_inference.rs:189-194) + rotate-half RoPE (cpu_inference.rs:203-215) ----
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const int r = wave + 4 * i;
    if (r < NR) {
      float a = ra[i], b = rb[i];
      if (DECODE && r <= G) {
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
        for (int j = 0; j < G; j++) sc[j][pg + 32 * u] = t < t1 && t < lim[j] ? sv[j] * p.scale : -INFINITY;
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
    if (more) load_tile<KV_BF16>(B, p.k_cache, p.v_cache, p.max_seq, head_base, tile + T, tid);
    __builtin_amdgcn_sched_barrier(0);
    process(A, tile);
    if (!more) break;
    const bool more2 = tile + 2 * T < t1;
    if (more2) load_tile<KV_BF16>(A, p.k_cache, p.v_cache, p.max_seq, head_base, tile + 2 * T, tid);
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


// ---------------------------------------------------------------------------------------------
// The merge of the split partials: out[h*128 + d] = sum_s e_s acc_s[d] / sum_s e_s l_s over the
// runs of q head h, e_s = exp(m_s - max m); empty runs (m = -inf) weigh 0. Workgroup (h, dim
// slice y) of 8 x DW threads: group j (thread = dim y DW + t) takes runs j, j+8, ..., j + 8(U-1),
// all of its loads issued at once (indexes past the last run re-read it and weigh 0; the launch
// picks the least U with 8U >= splits: at 33 runs, U = 16 instead of 5 cost 1.4 us per launch);
// the 8 groups meet in LDS.
// ---------------------------------------------------------------------------------------------
template <int U, int DW>
__global__ __launch_bounds__(8 * DW) void k_attn_merge(const float* __restrict__ part, uint32_t splits, uint32_t G,
                                                      float* __restrict__ out, uint32_t tok_heads,
                                                      uint32_t q_tok_stride) {
  constexpr int PS = kPartStride;
  const uint32_t h = blockIdx.x, g = h / G, j = h % G, t = threadIdx.x % DW, grp = threadIdx.x / DW;
  const uint32_t d = blockIdx.y * DW + t;
  const float* base = part + (size_t(g) * splits * G + j) * PS;
  float mv[U], lv[U], av[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const float* q = base + size_t(min(grp + 8u * u, splits - 1)) * G * PS;
    mv[u] = q[0];
    lv[u] = q[1];
    av[u] = q[4 + d];
  }
  __builtin_amdgcn_sched_barrier(0);
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; u++) M = grp + 8u * u < splits ? fmaxf(M, mv[u]) : M;
  float L = 0.f, A = 0.f;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const float e = (grp + 8u * u < splits && mv[u] != -INFINITY) ? expf(mv[u] - M) : 0.f;
    L += e * lv[u];
    A += e * av[u];
  }
  __shared__ float gm[8], gl[8], ga[8][DW];
  if (t == 0) { gm[grp] = M; gl[grp] = L; }
  ga[grp][t] = A;
  __syncthreads();
  if (grp != 0) return;
  float MM = -INFINITY;
#pragma unroll
  for (int k = 0; k < 8; k++) MM = fmaxf(MM, gm[k]);
  float LL = 0.f, AA = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const float e = gm[k] == -INFINITY ? 0.f : expf(gm[k] - MM);  // a group with no run adds 0
    LL += e * gl[k];
    AA += e * ga[k][t];
  }
  // rows of several tokens: row j of KV head g is token j / tok_heads, head g tok_heads + j % tok_heads
  const size_t o = tok_heads ? size_t(j / tok_heads) * q_tok_stride + (size_t(g) * tok_heads + j % tok_heads) * kHeadDim
                             : size_t(h) * kHeadDim;
  out[o + d] = AA / LL;
}

// shapes the kernels support; the runs [s*chunk, (s+1)*chunk) must cover positions 0..n-1
bool attn_args_ok(const AttnParams& p, uint32_t splits, uint32_t chunk, uint32_t n) {
  if (!p.n_kv || p.n_heads % p.n_kv || !p.qkv || !p.k_cache || !p.v_cache || !p.partial || p.max_seq == 0)
    return false;
  const uint32_t G = p.n_heads / p.n_kv;
  return (G == 1 || G == 2 || G == 4 || G == 8) && splits > 0 && chunk > 0 && uint64_t(splits) * chunk >= n;
}

// the merge over `splits` partials per q head (splits <= kAttnMaxSplits), in slices of
// kMergeDims dims per workgroup: 8 workgroups per q head instead of 1 took a 4096-step decode
// (64 runs per KV head past 1024 positions) from 1290 to 1314 tok/s and the k = 4 verify at 2048
// positions from 1.202 to 1.188 ms; slices of 32 dims: 1310 tok/s
constexpr int kMergeDims = 16;
template <int U>
hipError_t launch_merge_u(const AttnParams& p, uint32_t splits, float* out, uint32_t tok_heads, uint32_t q_tok_stride,
                          hipStream_t s) {
  if constexpr (U < kAttnMaxSplits / 8) {
    if (splits > 8u * U) return launch_merge_u<U + 1>(p, splits, out, tok_heads, q_tok_stride, s);
  }
  constexpr int DW = kMergeDims;
  hipLaunchKernelGGL((k_attn_merge<U, DW>), dim3(p.n_heads, kHeadDim / DW), dim3(8 * DW), 0, s, p.partial, splits,
                     p.n_heads / p.n_kv, out, tok_heads, q_tok_stride);
  return hipGetLastError();
}

hipError_t launch_merge(const AttnParams& p, uint32_t splits, float* out, uint32_t tok_heads, uint32_t q_tok_stride,
                        hipStream_t s) {
  static_assert(kAttnMaxSplits % 8 == 0, "8 groups of splits per q head");
  return launch_merge_u<1>(p, splits, out, tok_heads, q_tok_stride, s);
}

template <bool DECODE>
hipError_t launch_split(const AttnParams& pin, uint32_t splits, uint32_t chunk, hipStream_t s) {
  AttnParams p = pin;
  p.splits = splits;
  const uint32_t rsplit = !DECODE && p.row_split > 1 ? p.row_split : 1u;
  const uint32_t G = pin.n_heads / pin.n_kv / rsplit;  // rows per workgroup
  // prefetch workgroups: whole rows of the grid after the attention's `splits` rows (dispatched
  // after them: ahead of them, they delay the attention more than they gain)
  const uint32_t gx = p.n_kv * rsplit;
  const dim3 grid(gx, splits + ceil_div(8 * p.pf_slots, gx));
#define QE_ATT(GG)                                                                                          \
  if (G == GG) {                                                                                            \
    if (p.kv_bf16) hipLaunchKernelGGL((k_attn_split<GG, true, DECODE>), grid, dim3(256), 0, s, p, chunk);   \
    else hipLaunchKernelGGL((k_attn_split<GG, false, DECODE>), grid, dim3(256), 0, s, p, chunk);            \
    return hipGetLastError();                                                                               \
  }
  QE_ATT(1)
  QE_ATT(2)
  QE_ATT(4)
  QE_ATT(8)
#undef QE_ATT
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_attention_split(const AttnParams& p, uint32_t splits, hipStream_t s) {
  if (!attn_args_ok(p, splits, ceil_div(p.max_seq, max(splits, 1u)), p.max_seq) ||
      splits > uint32_t(kAttnMaxWideSplits) || !p.state || !p.rope_cur || !p.q_norm || !p.k_norm || !p.err)
    return hipErrorInvalidValue;
  return launch_split<true>(p, splits, 0, s);
}

hipError_t launch_attention_merge(const AttnParams& p, uint32_t splits, float* out, hipStream_t s) {
  if (!p.n_kv || p.n_heads % p.n_kv || !p.partial || !out || splits == 0 || splits > uint32_t(kAttnMaxSplits))
    return hipErrorInvalidValue;
  return launch_merge(p, splits, out, 0u, 0u, s);
}

hipError_t launch_attention_op(const AttnParams& p, uint32_t splits, float* out, hipStream_t s) {
  if (p.n_pos_fixed == 0 || p.n_pos_fixed > p.max_seq || splits == 0 || splits > uint32_t(kAttnMaxSplits) || !out)
    return hipErrorInvalidValue;
  const uint32_t chunk = ceil_div(p.n_pos_fixed, splits);
  if (!attn_args_ok(p, splits, chunk, p.n_pos_fixed) || p.kv_bf16 || p.row_split > 1) return hipErrorInvalidValue;
  hipError_t e = launch_split<false>(p, splits, chunk, s);
  if (e != hipSuccess) return e;
  return launch_merge(p, splits, out, 0u, 0u, s);
}

hipError_t launch_attention_rows(const AttnParams& p, uint32_t splits, float* out, hipStream_t s) {
  if (p.n_pos_fixed == 0 || p.n_pos_fixed > p.max_seq || splits == 0 || splits > uint32_t(kAttnMaxSplits) ||
      !p.n_kv || !p.tok_heads || (p.n_heads / p.n_kv) % p.tok_heads || !p.q_tok_stride)
    return hipErrorInvalidValue;
  const uint32_t tokens = p.n_heads / p.n_kv / p.tok_heads;
  if (tokens > p.n_pos_fixed) return hipErrorInvalidValue;
  if (p.row_split > 1 && ((p.n_heads / p.n_kv) % p.row_split || (p.n_heads / p.n_kv / p.row_split) % p.tok_heads))
    return hipErrorInvalidValue;
  const uint32_t chunk = ceil_div(p.n_pos_fixed, splits);
  if (!attn_args_ok(p, splits, chunk, p.n_pos_fixed)) return hipErrorInvalidValue;
  hipError_t e = launch_split<false>(p, splits, chunk, s);
  if (e != hipSuccess || !out) return e;
  return launch_merge(p, splits, out, p.tok_heads, p.q_tok_stride, s);
}

}  // namespace qe
