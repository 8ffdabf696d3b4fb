// Fused decode layer for the Qwen3-0.6B shape (hidden 1024, 16 q heads over 8 KV heads of 128,
// SwiGLU 3072): two launches per layer instead of one per dependent stage.
//
// Reference: cpu_inference.rs:126-172 (one layer of Model::forward), inference.metal:113-346.
//
// The MI355X has 8 XCDs, each with its own L2. The workgroups of a launch are dealt to the XCDs
// round-robin, starting where the previous dispatch left off: workgroup i runs on XCD
// (start + i) % 8 with a start that varies from launch to launch. So a workgroup takes its XCD x
// from HW_REG_XCC_ID and its slot from i / 8, which gives each XCD the slots 0..31 whatever the
// start. The model has 8 KV heads, so XCD x serves KV head x and the slices of the other
// projections that go with it.
//
// Inside one launch the stages of an XCD hand their outputs to each other through that XCD's L2
// only, as (value bits, tag) pairs written with one 64-bit store each (the vector L1 writes
// through to L2). A consumer polls the pairs it needs with device-scope loads (sc1: they miss the
// vector L1 and read the XCD's L2) until every tag is this launch's; the producer never waits for
// its stores, so loads it has in flight (weights, K/V) hold nothing up. The tag: every launch
// reads its XCD's generation word at the start and uses tag = generation + 1; slot 0 stores tag
// as the new generation at its end, which comes after every workgroup of the XCD has published
// data with that tag (so after all of them read the word). Tags are compared for equality, so
// nothing is reset and the count can wrap.
// Every wait is bounded: past kSpinMax polls it sets kErrSync and goes on, so no wave waits for
// ever (a host check at model load runs this path only if a launch deals its workgroups
// round-robin, and the 256 workgroups of a launch, one per CU, are all resident at once). A
// placement that broke the slot assignment would leave some pairs unwritten, and the waits for
// them would end in kErrSync, so it cannot pass silently.
//
// What crosses XCDs goes through a launch boundary: o_proj and down are split over the XCDs by
// input columns (XCD x owns attention heads 2x, 2x+1 and h[384x .. 384x+383]), each XCD writes a
// partial output vector, and the next launch adds the 8 partials to the residual stream in a
// fixed order.
//
//   attention block (k_fused_attn), workgroup (x, s = slot 0..31):
//     x = res + sum partials (layer 0: the embedding row) -> RMSNorm -> 16 of XCD x's 512 q|k|v
//     rows; slots s < splits: run s of the split attention of KV head x (q/k RMSNorm, RoPE, K/V
//     append by the run that holds pos); o_proj slots (16..31 with up to 16 runs, all 32 with
//     32): merge of the runs -> 64 (or 32) rows of o_proj over columns [256x, 256x+256) -> partial x
//   MLP block (k_fused_mlp):
//     x = res + sum partials -> RMSNorm -> 24 of XCD x's 768 gate|up rows, silu * up -> 12 of
//     h[384x..] -> 32 rows of down over columns [384x, 384x+384) -> partial x
// Weights are loaded at the start of each workgroup (o_proj's once the q|k|v rows are out), and
// workgroups past the 256 of a launch can load a later launch's weights into the L2 of their XCD.
#include <cmath>

#include "attn_tile.h"
#include "device_common.h"
#include "kernels.h"
#include "l2_prefetch.h"
#include "xcd_exchange.h"

#ifndef QE_PF32
#define QE_PF32 1
#endif
// QE_FUSED_TIMED: this file compiled a second time (fused_timed.hip) with clock stamps in the
// layer kernels and the two layer launchers named *_timed
#ifdef QE_FUSED_TIMED
#define QE_FUSED_LAUNCHER(name) name##_timed
#else
#define QE_FUSED_LAUNCHER(name) name
#endif
// attention blocks with at least this many runs merge them in two rounds (below)
#ifndef QE_MERGE2_MIN_SM
#define QE_MERGE2_MIN_SM 8
#endif

namespace qe {
namespace {

constexpr uint32_t H = kFusedH, I = kFusedI, D = kHeadDim, NKV = kFusedKv, G = kFusedHeads / kFusedKv;
constexpr uint32_t QD = kFusedHeads * D, KD = NKV * D;
constexpr uint32_t NX = kFusedXcds, NS = kFusedSlots;
constexpr uint32_t kQkvRowPairs = uint32_t(kFusedQkvRowPairs);  // p.qkv pairs per token row

static_assert(NKV == NX, "one KV head per XCD");
static_assert(G == 2 && H == 1024 && I == 3072, "the launch layouts below are written for these sizes");
static_assert((G * D + 2 * D) == 16 * NS, "16 q|k|v rows per workgroup");
static_assert(2 * I / NX == 24 * NS && H == 32 * NS, "24 gate|up rows and 32 down rows per workgroup");

__device__ __forceinline__ uint32_t* gen_word(uint32_t* sync, uint32_t x) { return sync + x * kFusedLineWords; }

// One scalar load per 64-byte line of the argument block at the kernel's start, so that the
// compiler's later loads of the arguments find them in the scalar cache instead of missing there
// on the critical path. The loaded words are never read: their registers stay reserved to the end
// of the kernel (kcache_release), where every scalar load has long completed.
struct KcacheWarm {
  uint32_t d[6];
};
__device__ __forceinline__ KcacheWarm kcache_warm() {
  KcacheWarm w;
  const auto ka = __builtin_amdgcn_kernarg_segment_ptr();
  asm volatile(
      "s_load_dword %0, %6, 0x40\n\ts_load_dword %1, %6, 0x80\n\ts_load_dword %2, %6, 0xc0\n\t"
      "s_load_dword %3, %6, 0x100\n\ts_load_dword %4, %6, 0x140\n\ts_load_dword %5, %6, 0x180"
      : "=s"(w.d[0]), "=s"(w.d[1]), "=s"(w.d[2]), "=s"(w.d[3]), "=s"(w.d[4]), "=s"(w.d[5])
      : "s"(ka));
  return w;
}
__device__ __forceinline__ void kcache_release(const KcacheWarm& w) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::"s"(w.d[0]), "s"(w.d[1]), "s"(w.d[2]), "s"(w.d[3]), "s"(w.d[4]), "s"(w.d[5]));
}

// Clock stamps, in the QE_FUSED_TIMED compilation of this file only: a layer workgroup reads the
// 100 MHz real-time clock at its start (kept in registers, so nothing at the start waits for the
// argument block) and at its exit writes both to FusedLayerParams::ts[2 b], ts[2 b + 1], b = its
// workgroup index. The other compilation reads no clock and writes nothing.
__device__ __forceinline__ uint64_t clock_start() {
#ifdef QE_FUSED_TIMED
  return __builtin_amdgcn_s_memrealtime();
#else
  return 0;
#endif
}

// every exit of a layer kernel's workgroup: the scalar-cache warm loads are in; the clock stamps
__device__ __forceinline__ void finish(const KcacheWarm& w, uint64_t* ts, uint64_t t_start) {
  kcache_release(w);
#ifdef QE_FUSED_TIMED
  if (ts && threadIdx.x == 0) {
    ts[2 * blockIdx.x] = t_start;
    ts[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime();
  }
#else
  (void)ts;
  (void)t_start;
#endif
}

// x[4 tid .. 4 tid + 3] = xin + part[0] + ... + part[7] (a fixed order) into xs; workgroup 0
// also stores it to res_out. Returns the RMSNorm scale 1 / sqrt(mean(x^2) + eps) of all of x.
// R rows (a verify pass): row r from xin[r], xp[r] into xs + r H and res_out + r H, scale rs[r].
template <int R>
__device__ __forceinline__ void residual_and_scale(const float4 (&xin)[R], const float4 (&xp)[R][NX], bool add_parts,
                                                   float* xs, float* res_out, float eps, float (*red4)[4],
                                                   float (&rs)[R]) {
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int r = 0; r < R; r++) {
    float4 v = xin[r];
    if (add_parts) {
#pragma unroll
      for (uint32_t g = 0; g < NX; g++) v = add4(v, xp[r][g]);
    }
    reinterpret_cast<float4*>(xs + r * H)[tid] = v;
    if (blockIdx.x == 0) reinterpret_cast<float4*>(res_out + r * H)[tid] = v;
    const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
    if (lane == 0) red4[r][wave] = ss;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float tot = (red4[r][0] + red4[r][1]) + (red4[r][2] + red4[r][3]);
    rs[r] = 1.0f / sqrtf(tot / float(H) + eps);
  }
}

// first q|k|v row of slot s of KV head x: slots 0-15 take 16 rows each of q heads 2x, 2x+1,
// slots 16-23 of k head x, slots 24-31 of v head x (a slot's 16 rows are consecutive)
__device__ __forceinline__ uint32_t qkv_row0(uint32_t x, uint32_t s) {
  return s < 16 ? x * G * D + 16 * s : s < 24 ? QD + x * D + 16 * (s - 16) : QD + KD + x * D + 16 * (s - 24);
}

// Prefetcher k of n on this XCD loads one word of every 64-byte half line i = k + n j of the
// lines of regions T0..T1-1 on XCD x, so the lines sit in this XCD's L2 when the later launch's
// workgroups on XCD x read them; the words only feed an empty asm statement, which keeps the loads.
template <int T0 = 0, int T1 = kFusedMaxPrefetch>
__device__ __forceinline__ void fused_prefetch(const FusedLayerParams& p, uint32_t x, uint32_t k, uint32_t n) {
  constexpr uint32_t U = 8, SEG = 64;
  uint32_t per_row[kFusedMaxPrefetch], span[kFusedMaxPrefetch], tot = 0;
#pragma unroll
  for (int t = 0; t < kFusedMaxPrefetch; t++) {
    const bool on = t >= T0 && t < T1 && p.pf[t].base;
    per_row[t] = on ? ceil_div(p.pf[t].row_bytes, SEG) : 0;
    span[t] = per_row[t] * (on ? p.pf[t].rows : 0);
    tot += span[t];
  }
  if (tot == 0) return;
  uint32_t hsum = 0;
  for (uint32_t j0 = 0; (j0 * n + k) * 256 < tot; j0 += U) {
    uint32_t v[U];
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      uint32_t i = min(((j0 + u) * n + k) * 256 + threadIdx.x, tot - 1);
      uint32_t t = 0;
#pragma unroll
      for (int q = 0; q + 1 < kFusedMaxPrefetch; q++) {
        if (t == uint32_t(q) && i >= span[q]) {
          i -= span[q];
          t = q + 1;
        }
      }
      const FusedPrefetch& r = p.pf[t];
      const uint32_t row = i / per_row[t], seg = i - row * per_row[t];
      const uint8_t* a = r.base + size_t(x) * r.xcd_bytes + size_t(row) * r.stride + min(seg * SEG, r.row_bytes - 4);
      v[u] = *reinterpret_cast<const uint32_t*>(a);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t u = 0; u < U; u++) hsum ^= v[u];
  }
  asm volatile("" ::"v"(hsum));
}

// The same for one region T, with the line's row and segment advanced by constant steps from
// load to load instead of divided out for every load (fewer instructions before the last load
// issues). Lines past the region's end load the region's last line again.
template <int T>
__device__ __forceinline__ void prefetch_region(const FusedLayerParams& p, uint32_t x, uint32_t k, uint32_t n) {
  constexpr uint32_t U = 8, SEG = 64;
  const FusedPrefetch& r = p.pf[T];
  if (!r.base || !r.rows) return;
  const uint32_t per_row = ceil_div(r.row_bytes, SEG), span = per_row * r.rows, step = n * 256;
  const uint32_t dq = step / per_row, dr = step - dq * per_row;
  const uint32_t i0 = k * 256 + threadIdx.x;
  uint32_t row = i0 / per_row, seg = i0 - row * per_row;
  const uint8_t* base = r.base + size_t(x) * r.xcd_bytes;
  const uint32_t last_row = r.rows - 1, last_off = r.row_bytes - 4;
  uint32_t hsum = 0;
  for (uint32_t j0 = 0; k * 256 + j0 * step < span; j0 += U) {
    uint32_t v[U];
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      const bool in = row <= last_row;
      const uint8_t* a = base + size_t(in ? row : last_row) * r.stride + (in ? min(seg * SEG, last_off) : last_off);
      v[u] = *reinterpret_cast<const uint32_t*>(a);
      seg += dr;
      row += dq;
      if (seg >= per_row) {
        seg -= per_row;
        row++;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t u = 0; u < U; u++) hsum ^= v[u];
  }
  asm volatile("" ::"v"(hsum));
}

// ---------------------------------------------------------------------------------------------
// attention block of one layer. SM: merge slots (>= splits), KV_BF16: cache element type,
// MULTI: runs of more than one 64-position tile (only with 32 runs), NT: positions per tile and
// per single-tile run (64, or 32 for short contexts: half the K/V each run's CU takes in).
// R: token rows (1: a decode step; 2: a verify pass over positions pos and pos + 1, whose rows
// share every weight load; row r's buffers sit r row strides on, its q heads are q vectors
// r G .. r G + G - 1 of the KV head, and it attends to positions 0 .. pos + r).
// ---------------------------------------------------------------------------------------------
// The arguments the first loads need come first, as plain pointers (preloaded into scalar
// registers at wave launch, as in k_fused_mlp).
template <bool FIRST, bool KV_BF16, int SM, bool MULTI, int NT, int R>
__global__ __launch_bounds__(256) void k_fused_attn(uint32_t* sync, const StepState* state, const float* res_in,
                                                    const float* part_in, const uint16_t* w_qkv, const uint16_t* w_in,
                                                    uint32_t n_runs, uint32_t run_len, FusedLayerParams p) {
  static_assert(SM == 32 || !MULTI, "runs of several tiles come with 32 runs");
  static_assert(NT == 64 || (NT == 32 && !MULTI), "runs of several tiles use 64-position tiles");
  static_assert(R == 1 || (R == 2 && SM <= 16), "verify rows: single-tile runs, up to 16");
  constexpr uint32_t T = NT, VP = NT / 8;  // positions per tile, per thread in the P.V layout
  constexpr uint32_t QV = R * G;           // q vectors per KV head
  // o_proj: with up to 16 runs, slots 16..31 take 64 rows each (4 per 16-thread row group), so
  // the attention runs (slots 0..15) carry no o_proj weights; with 32 runs every slot takes 32
  constexpr uint32_t ORR = SM <= 16 ? 4 : 2;
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t x = fused_xcd(p.err);
  if (blockIdx.x >= NX * NS) {  // a prefetch workgroup (the whole workgroup)
    if (state->pos < p.pf_max_pos) fused_prefetch(p, x, (blockIdx.x - NX * NS) / NX, p.pf_wgs);
    return;
  }
  const uint64_t t_start = clock_start();
  const KcacheWarm kw = kcache_warm();
  const uint32_t s = blockIdx.x / NX;
  const int pg = tid >> 3, dc = tid & 7, dg = tid & 31, pp = tid >> 5;
  const uint32_t splits = max(n_runs, 1u);
  const bool attn = s < splits;  // this workgroup also runs attention run s of KV head x
  const bool oproj = SM <= 16 ? s >= 16 : true;
  const uint32_t orow0 = SM <= 16 ? 64 * (s - 16) : 32 * s;

  __shared__ __align__(16) float xs[R * H];
  __shared__ float red4[R][4];
  __shared__ __align__(16) float qs[QV][D];
  __shared__ __align__(16) float knew[R][D];
  __shared__ __align__(16) float vnew[R][D];
  __shared__ float sc[QV][T], pes[QV][T];
  __shared__ float Ms[QV], Ls[QV], Cs[QV];
  __shared__ __align__(16) float red[8][QV][D];
  __shared__ __align__(16) float att[R][G * D];
  __shared__ float mw[QV][SM], msum[QV];  // merge weights of the runs and their sums per q vector

  const uint32_t tag = *gen_word(sync, x) + 1;
  // this step's position (set before the step's first launch), read now so that no load of it
  // waits behind the attention's polls. It is read as a per-lane value (the offset comes from an
  // asm statement, which the compiler takes as varying across lanes): a uniform value would be
  // moved to a scalar register right after the load, and the wave would wait for it there
  // instead of issuing its weight loads.
  uint32_t lane_zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(lane_zero));
  const uint32_t pos_step = (&state->pos)[lane_zero];

  // ---- loads that depend on no other workgroup, issued before any use ----
  // the residual stream (from the previous launch) or the embedding row
  float4 xin[R];
  float4 xp[R][NX];
#pragma unroll
  for (int r = 0; r < R; r++) {
    if constexpr (FIRST) {
      uint32_t tok = p.tokens[state->tok_idx + r];
      if (tok >= p.vocab) {
        if (blockIdx.x == 0 && tid == 0) atomicOr(p.err, kErrToken);
        tok = 0;
      }
      const uint2 e = reinterpret_cast<const uint2*>(p.embed + size_t(tok) * H)[tid];
      xin[r] = bf16x4(e.x, e.y);
#pragma unroll
      for (uint32_t g = 0; g < NX; g++) xp[r][g] = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      xin[r] = reinterpret_cast<const float4*>(res_in + r * H)[tid];
#pragma unroll
      for (uint32_t g = 0; g < NX; g++) xp[r][g] = reinterpret_cast<const float4*>(part_in + (r * NX + g) * H)[tid];
    }
  }
  // q|k|v: row group = wave, 4 rows of 1024 columns, lane l holds chunks l and l + 64
  const uint4* Wq = reinterpret_cast<const uint4*>(w_qkv);
  const uint32_t qrow0 = __builtin_amdgcn_readfirstlane(qkv_row0(x, s) + 4 * wave);
  uint4 wq[4][2];
#pragma unroll
  for (int r = 0; r < 4; r++) {
#pragma unroll
    for (int k = 0; k < 2; k++) wq[r][k] = Wq[size_t(qrow0 + r) * (H / 8) + lane + 64 * k];
  }
  uint4 gin[2];
#pragma unroll
  for (int k = 0; k < 2; k++) gin[k] = reinterpret_cast<const uint4*>(w_in)[lane + 64 * k];
  // Attention inputs, issued behind the residual and q|k|v weight loads: loads complete in issue
  // order, so they do not hold up this workgroup's q|k|v rows (which every run waits for), and
  // they arrive while the rows are computed instead of after them. The raw norm gains, this
  // position's RoPE row, and the first K/V tile of the run (the row at pos is not read from it:
  // the run that holds pos substitutes the new row from LDS). Every workgroup issues all of
  // them, the tile through descriptors over the run's first rows (none for a workgroup without
  // a run: its loads read 0 without touching memory): behind a branch, the wait counts of the
  // two paths would merge and every workgroup's q|k|v rows would wait for the tile.
  // A 32-position tile is issued only once the residual is in (below): issued here it delays
  // the run workgroups' residual by ~0.3 us (2321 vs 2305 tok/s at positions 130..257), while a
  // 64-position tile issued there arrives too late (1740 vs 1767 tok/s over 4096 steps).
  const size_t head_base = size_t(x) * p.max_seq * D;
  KVTile<KV_BF16, NT> A;
  auto load_first_tile = [&]() __attribute__((always_inline)) {
    constexpr uint32_t EL = KV_BF16 ? 2 : 4;
    const uint32_t r0 = s * run_len;
    const uint32_t rows = attn && r0 < p.max_seq ? min(p.max_seq - r0, T) : 0u;
    auto run_rsrc = [&](const void* cache) __attribute__((always_inline)) {
      const uint8_t* b = static_cast<const uint8_t*>(cache) + (head_base + size_t(r0) * D) * EL;
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(b), short(0), int(rows * D * EL), 0x00020000);
    };
    load_tile_buf<KV_BF16, NT>(A, run_rsrc(p.k_cache), run_rsrc(p.v_cache), 0, tid);
  };
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t gq[2] = {p.q_norm[lane], p.q_norm[lane + 64]};
  const uint16_t gk[2] = {p.k_norm[lane], p.k_norm[lane + 64]};
  // RoPE row of the step's position (one row: rope_cur, no wait for pos); a verify pass's rows
  // read theirs from the table at pos + r once the attention starts (pos is in by then)
  float2 cs[R];
  if constexpr (R == 1) cs[0] = reinterpret_cast<const float2*>(p.rope_cur)[lane];
  if constexpr (NT != 32) load_first_tile();
  // o_proj rows orow0 + ORR rg + r over columns [256 x, 256 x + 256): 16 threads per row, chunks
  // t16 and t16 + 16 of the slice
  const uint32_t rg = tid >> 4, t16 = tid & 15;
  const uint4* Wo = reinterpret_cast<const uint4*>(p.w_o);
  uint4 wo[ORR][2];
  auto load_wo = [&]() {
#pragma unroll
    for (uint32_t r = 0; r < ORR; r++) {
#pragma unroll
      for (int k = 0; k < 2; k++) wo[r][k] = Wo[size_t(orow0 + ORR * rg + r) * (QD / 8) + 32 * x + t16 + 16 * k];
    }
  };
  __builtin_amdgcn_sched_barrier(0);

  // ---- input RMSNorm + this workgroup's 16 q|k|v rows (cpu_inference.rs:129-132) ----
  {
    float rs[R];
    residual_and_scale<R>(xin, xp, !FIRST, xs, p.res_out, p.eps, red4, rs);
    if constexpr (NT == 32) load_first_tile();
    float acc[R][4];
#pragma unroll
    for (int t = 0; t < R; t++) {
      const float4* xs4 = reinterpret_cast<const float4*>(xs + t * H);
#pragma unroll
      for (int r = 0; r < 4; r++) acc[t][r] = 0.f;
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const uint32_t c = lane + 64 * k;
        float4 a = xs4[2 * c], b = xs4[2 * c + 1];
        scale8(a, b, gin[k]);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = dot8(wq[r][k], a, b, acc[t][r]);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) acc[t][r] = wave_sum(acc[t][r]) * rs[t];
    }
    if (lane == 0) {
#pragma unroll
      for (int t = 0; t < R; t++) {
#pragma unroll
        for (int r = 0; r < 4; r++) p.qkv[t * kQkvRowPairs + qrow0 + r] = pair(acc[t][r], tag);
      }
    }
  }
  if (SM > 16 && attn) load_wo();

  // ---- attention run s of KV head x (cpu_inference.rs:134-162) ----
  // With 32 runs every slot runs attention and holds o_proj rows (no idle slot), and each loads
  // the 24 gate|up rows of MLP slot s on this XCD (48 KB, one word of each 64-byte half line)
  // into its L2 while its run computes. Loads complete in issue order, so the issue point is
  // after the loads the run waits for and before the merge's polls, which would otherwise wait
  // for this HBM round trip: a single-tile run issues it once its q|k|v pairs are in, a run of
  // several tiles right after its second tile's loads (after the partial, where the merge's
  // polls waited for it: 1765 -> 1786 tok/s over 4096 steps, 1556 -> 1598 over the last 512).
  // With pf region 2 set, a run also loads the down columns of MLP slot s (rows 32 s .., 768
  // bytes each; load_gdn), through a descriptor that holds no bytes otherwise: a single-tile run
  // with the gate|up rows (positions 1154..1665: 1893 -> 1975 tok/s), a run of several tiles once
  // its first tile is computed (2178..2689: 1659 -> 1688; issued with the gate|up rows, after the
  // second tile's loads, it cost 1652 -> 1607 at 3202..3713).
  uint32_t gpf[5] = {0u, 0u, 0u, 0u, 0u};
  auto load_gdn = [&]() __attribute__((always_inline)) {
    constexpr uint32_t DL = (I / NX) * 2 / 64;  // 64-byte lines of one down row's slice: 12
    const bool dn = p.pf[2].base != nullptr;
    const __amdgpu_buffer_rsrc_t rd = rsrc_of(p.w_down + size_t(32 * s) * I + (I / NX) * x,
                                              dn ? 31 * I * 2 + DL * 64 : 0u);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const uint32_t i = min(tid + 256 * k, 32 * DL - 1), row = i / DL;
      gpf[3 + k] = __builtin_amdgcn_raw_buffer_load_b32(rd, int(row * I * 2 + (i - row * DL) * 64), 0, 0);
    }
  };
  auto load_gpf = [&]() __attribute__((always_inline)) {
    const uint8_t* gb = reinterpret_cast<const uint8_t*>(p.w_gu + size_t((2 * I / NX) * x + 24 * s) * H);
#pragma unroll
    for (int k = 0; k < 3; k++) gpf[k] = *reinterpret_cast<const uint32_t*>(gb + (tid + 256 * k) * 64);
    if constexpr (!MULTI) load_gdn();
  };
  auto attention = [&]() __attribute__((always_inline)) {
    // raw rows: wave w takes row w of [q head 2x, q head 2x+1, k, v] of every token row; lane l
    // holds dims l, l + 64
    const __amdgpu_buffer_rsrc_t rq = rsrc_of(p.qkv, uint32_t(R * kQkvRowPairs * 8));
    const uint32_t off = wave < G ? (x * G + wave) * D : wave == G ? QD + x * D : QD + KD + x * D;
    if constexpr (R > 1) {
#pragma unroll
      for (int r = 0; r < R; r++)
        cs[r] = reinterpret_cast<const float2*>(p.rope_cur + size_t(min(pos_step + r, p.max_seq - 1)) * D)[lane];
    }
    uint2 qa[R], qb[R];
    for (uint32_t spins = 0;;) {
      bool ok = true;
#pragma unroll
      for (int r = 0; r < R; r++) {
        qa[r] = ld_pair(rq, r * kQkvRowPairs + off + lane);
        qb[r] = ld_pair(rq, r * kQkvRowPairs + off + lane + 64);
        ok = ok && qa[r].y == tag && qb[r].y == tag;
      }
      if (poll_done(ok, spins, p.err)) break;
    }
#if QE_PF32
    if constexpr (SM == 32 && !MULTI) load_gpf();  // (see gpf above)
#endif

    const uint32_t pos = pos_step;
    const bool bad = R == 1 ? pos >= p.max_seq : pos + R > p.max_seq;
    if (bad && x == 0 && s == 0 && tid == 0) atomicOr(p.err, kErrPos);
    uint32_t n = bad ? 0u : pos + R;  // positions 0 .. pos + R - 1
    const uint32_t run = run_len;
    if (n > splits * run) {  // the host's runs would skip positions
      if (x == 0 && s == 0 && tid == 0) atomicOr(p.err, kErrShape);
      n = 0;
    }
    const uint32_t t0 = s * run, t1 = min(n, t0 + run);
    const bool owns_new = n != 0 && pos >= t0 && pos < t0 + run;  // (row 0)
    // row r sees positions up to pos + r (cpu_inference.rs:144-162 at each row's position)
    uint32_t t1r[R];
    t1r[0] = t1;
#pragma unroll
    for (int r = 1; r < R; r++) t1r[r] = min(n == 0 ? 0u : pos + r + 1, t0 + run);
    if constexpr (R > 1) t1r[0] = min(n == 0 ? 0u : pos + 1, t0 + run);

#pragma unroll
    for (int r = 0; r < R; r++) {
      float a = __uint_as_float(qa[r].x), b = __uint_as_float(qb[r].x);
      // q/k RMSNorm (cpu_inference.rs:189-194) + rotate-half RoPE (cpu_inference.rs:203-215)
      if (wave <= G) {
        const float ss = wave_sum(a * a + b * b);
        const float scl = 1.0f / sqrtf(ss / float(D) + p.eps);
        a = a * scl * bf16f(wave < G ? gq[0] : gk[0]);
        b = b * scl * bf16f(wave < G ? gq[1] : gk[1]);
        const float ar = a * cs[r].x - b * cs[r].y, br = b * cs[r].x + a * cs[r].y;
        a = ar;
        b = br;
      }
      if (KV_BF16 && wave >= G) {  // attend with the values later steps read back
        a = bf16f(f32_to_bf16(a));
        b = bf16f(f32_to_bf16(b));
      }
      float* dst = wave < G ? qs[r * G + wave] : (wave == G ? knew[r] : vnew[r]);
      dst[lane] = a;
      dst[lane + 64] = b;
    }
    if (tid < QV) {
      Ms[tid] = -INFINITY;
      Ls[tid] = 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; r++) {
      if (r == 0 ? owns_new : n != 0 && pos + r >= t0 && pos + r < t0 + run) {  // append new K/V row r (cpu_inference.rs:140-141)
        const size_t slot = head_base + size_t(pos + r) * D + (tid & (D - 1));
        const float val = tid < D ? knew[r][tid] : vnew[r][tid - D];
        void* cache = wave < 2 ? p.k_cache : p.v_cache;  // (threads tid < D: waves 0 and 1)
        if (KV_BF16) static_cast<uint16_t*>(cache)[slot] = f32_to_bf16(val);
        else static_cast<float*>(cache)[slot] = val;
      }
    }

    float4 acc[QV];
#pragma unroll
    for (uint32_t j = 0; j < QV; j++) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);

    auto process = [&](const KVTile<KV_BF16, NT>& X, uint32_t tile) __attribute__((always_inline)) {
      // scores s_t = (q . k_t) * scale (cpu_inference.rs:144-152); the new positions' k rows are
      // knew (the cache rows this launch writes are not read back)
#pragma unroll
      for (int u = 0; u < int(NT / 32); u++) {
        const uint32_t t = tile + uint32_t(pg + 32 * u);
        float4 k4[4];
        tile_k<KV_BF16>(X, u, k4);
        const uint32_t dn = t - pos;  // new row dn when dn < R
        const bool sub = R == 1 ? owns_new && t == pos : n != 0 && dn < uint32_t(R);
        const float4* kn = reinterpret_cast<const float4*>(knew[R == 1 ? 0 : min(dn, uint32_t(R - 1))]) + 4 * dc;
#pragma unroll
        for (int i = 0; i < 4; i++) k4[i] = sel4(sub, kn[i], k4[i]);
        float sv[QV];
#pragma unroll
        for (uint32_t j = 0; j < QV; j++) {
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
          for (uint32_t j = 0; j < QV; j++) sc[j][pg + 32 * u] = t < t1r[j / G] ? sv[j] * p.scale : -INFINITY;
        }
      }
      __syncthreads();
      // softmax (cpu_inference.rs:217-223) as an online update: running max, rescaled sum
      if (wave < QV) {
        const uint32_t j = wave;
        const float xv = lane < T ? sc[j][lane] : -INFINITY;
        const float m_old = Ms[j];
        const float m_new = fmaxf(m_old, wave_max(xv));
        const float pe = xv == -INFINITY ? 0.f : expf(xv - m_new);
        const float c = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
        const float tsum = wave_sum(pe);
        if (lane < T) pes[j][lane] = pe;
        if (lane == 0) {
          Ls[j] = Ls[j] * c + tsum;
          Ms[j] = m_new;
          Cs[j] = c;
        }
      }
      __syncthreads();
      // out += p_t * v_t (cpu_inference.rs:153-160); positions past the run add 0
      float4 v4[VP];
      float4 vn[R];
#pragma unroll
      for (int r = 0; r < R; r++) vn[r] = reinterpret_cast<const float4*>(vnew[r])[dg];
#pragma unroll
      for (int i = 0; i < int(VP); i++) {
        const uint32_t t = tile + uint32_t(VP * pp + i);
        if constexpr (R == 1) {
          v4[i] = sel4(owns_new && t == pos, vn[0], tile_v<KV_BF16>(X, i));
        } else {
          const uint32_t dn = t - pos;
          v4[i] = sel4(n != 0 && dn < uint32_t(R), dn == 0 ? vn[0] : vn[1], tile_v<KV_BF16>(X, i));
        }
        v4[i] = sel4(t < t1, v4[i], make_float4(0.f, 0.f, 0.f, 0.f));
      }
#pragma unroll
      for (uint32_t j = 0; j < QV; j++) {
        const float c = Cs[j];
        float4 o = make_float4(acc[j].x * c, acc[j].y * c, acc[j].z * c, acc[j].w * c);
#pragma unroll
        for (int i = 0; i < int(VP); i++) {
          const float pe = pes[j][VP * pp + i];
          o.x += pe * v4[i].x;
          o.y += pe * v4[i].y;
          o.z += pe * v4[i].z;
          o.w += pe * v4[i].w;
        }
        acc[j] = o;
      }
    };

    if constexpr (MULTI) {
      // runs of several tiles alternate between two register sets, so the next tile's loads are
      // in flight while one is computed (sc / pes / Cs are rewritten only after the next barrier)
      KVTile<KV_BF16, NT> B;
      for (uint32_t tile = t0;; tile += 2 * T) {
        const bool more = tile + T < t1;
        if (more) load_tile<KV_BF16>(B, p.k_cache, p.v_cache, p.max_seq, head_base, tile + T, tid);
#if QE_PF32
        if (tile == t0) load_gpf();  // (see gpf above)
#endif
        __builtin_amdgcn_sched_barrier(0);
        process(A, tile);
        if (tile == t0) load_gdn();  // (see gpf above)
        if (!more) break;
        const bool more2 = tile + 2 * T < t1;
        if (more2) load_tile<KV_BF16>(A, p.k_cache, p.v_cache, p.max_seq, head_base, tile + 2 * T, tid);
        __builtin_amdgcn_sched_barrier(0);
        process(B, tile + T);
        if (!more2) break;
      }
    } else {
      process(A, t0);
    }

    // the 8 position groups meet; m and l are the softmax state; the partial goes out as pairs
#pragma unroll
    for (uint32_t j = 0; j < QV; j++) reinterpret_cast<float4*>(red[pp][j])[dg] = acc[j];
    __syncthreads();
    uint2* part = p.attn_part + (size_t(x) * kFusedMaxRuns + s) * QV * kPartStride;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t j = r * G + tid / D, d = tid % D;  // 256 threads = G x D outputs per row
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < 8; q++) v += red[q][j][d];
      part[j * kPartStride + 4 + d] = pair(v, tag);
      if (d == 0) {
        part[j * kPartStride] = pair(Ms[j], tag);
        part[j * kPartStride + 1] = pair(Ls[j], tag);
      }
    }
  };

  // ---- merge of the runs, then o_proj ----
  // out = sum_s e_s acc_s / sum_s e_s l_s, e_s = exp(m_s - max m); empty runs (m = -inf) and
  // slots past the last run weigh 0.
  auto merge_oproj = [&]() __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rp = rsrc_of(p.attn_part + size_t(x) * kFusedMaxRuns * QV * kPartStride,
                                              uint32_t(kFusedMaxRuns * QV * kPartStride * 8));
    if constexpr (SM >= QE_MERGE2_MIN_SM) {
      // In two rounds. The OW slots with o_proj rows (all 32 with 32 runs, else slots 16..31)
      // each merge VW = 256 / OW of the XCD's 256 values (head j1) of every token row over the
      // runs: thread t takes run t / VW, value t % VW, wave 0 lanes 0..SM-1 the (m, l) of the runs;
      // the merged values go out as pairs after the q|k|v pairs, and every o_proj slot then
      // gathers the 256 of each row (one per thread), instead of each polling SM pairs per thread
      // of every run.
      constexpr uint32_t OW = SM <= 16 ? 16 : 32, VW = G * D / OW;
      const uint32_t o = SM <= 16 ? s - 16 : s;
      const uint32_t q = tid / VW, e = tid % VW, j1 = (VW * o) / D;
      const uint32_t d1 = (VW * o) % D + e;
      const bool live = wave == 0 && lane < SM && lane < splits;
      const bool mine = q < SM && q < splits;
      uint4 ml[R];
      uint2 a1[R];
#pragma unroll
      for (int r = 0; r < R; r++) {
        ml[r] = make_uint4(0u, 0u, 0u, 0u);
        a1[r] = make_uint2(0u, 0u);
      }
      for (uint32_t spins = 0;;) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < R; r++) {
          const uint32_t jq = r * G + j1;
          if (wave == 0) ml[r] = ld_pair2(rp, (min(lane, splits - 1) * QV + jq) * kPartStride);
          a1[r] = ld_pair(rp, (min(q, splits - 1) * QV + jq) * kPartStride + 4 + d1);
          ok = ok && (!live || (ml[r].y == tag && ml[r].w == tag)) && (!mine || a1[r].y == tag);
        }
        if (poll_done(ok, spins, p.err)) break;
      }
      if (wave == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) {
          const float m = live ? __uint_as_float(ml[r].x) : -INFINITY;
          float M = m;
#pragma unroll
          for (int w = 1; w < int(SM); w <<= 1) M = fmaxf(M, __shfl_xor(M, w));
          const float wt = m != -INFINITY ? expf(m - M) : 0.f;
          float L = wt * (live ? __uint_as_float(ml[r].z) : 0.f);
#pragma unroll
          for (int w = 1; w < int(SM); w <<= 1) L += __shfl_xor(L, w);
          if (lane < SM) mw[r][lane] = wt;
          if (lane == 0) msum[r] = L;
        }
      }
      __syncthreads();
      // sum over the runs: the lanes of a wave with the same value index, then the 4 waves in LDS
#pragma unroll
      for (int r = 0; r < R; r++) {
        float c = mine ? mw[r][q] * __uint_as_float(a1[r].x) : 0.f;
#pragma unroll
        for (uint32_t w = VW; w < 64; w <<= 1) c += __shfl_xor(c, w);
        if (lane < VW) red[wave][r][lane] = c;
      }
      __syncthreads();
      uint2* ax = p.qkv + kFusedQkvPairs + size_t(x) * (G * D);
      if (tid < VW) {
#pragma unroll
        for (int r = 0; r < R; r++) {
          const float v = ((red[0][r][tid] + red[1][r][tid]) + (red[2][r][tid] + red[3][r][tid])) * (1.0f / msum[r]);
          ax[r * kQkvRowPairs + VW * o + tid] = pair(v, tag);
        }
      }
      const __amdgpu_buffer_rsrc_t ra = rsrc_of(ax, ((R - 1) * kQkvRowPairs + G * D) * 8);
      uint2 av1[R];
      for (uint32_t spins = 0;;) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < R; r++) {
          av1[r] = ld_pair(ra, r * kQkvRowPairs + tid);
          ok = ok && av1[r].y == tag;
        }
        if (poll_done(ok, spins, p.err)) break;
      }
#pragma unroll
      for (int r = 0; r < R; r++) att[r][tid] = __uint_as_float(av1[r].x);
      asm volatile("" ::"v"(gpf[0] ^ gpf[1] ^ gpf[2] ^ gpf[3] ^ gpf[4]));  // (in: the polls waited for every load)
      __syncthreads();
    } else {
    // Wave 0 takes the (m, l) of every run (lane u: q vector u / SM, run u % SM) and leaves the
    // weights e_s and the sums in LDS; then thread (head 2x + tid / 128, dim tid % 128) adds up its
    // acc values of every row. One poll round trip for both: wave 0's (m, l) pairs and every
    // thread's acc values.
    static_assert(QV * SM <= 64, "one (m, l) pair per lane of wave 0");
    const uint32_t j = tid >> 7, d = tid & 127;
    const uint32_t jh = min(lane / SM, QV - 1), u = lane % SM;
    const bool live = wave == 0 && lane < QV * SM && u < splits;
    const uint32_t base = (min(u, splits - 1) * QV + jh) * kPartStride;
    uint4 ml = make_uint4(0u, 0u, 0u, 0u);  // pairs m, l (wave 0)
    uint2 av[R][SM];
    for (uint32_t spins = 0;;) {
      if (wave == 0) ml = ld_pair2(rp, base);
#pragma unroll
      for (int r = 0; r < R; r++) {
#pragma unroll
        for (int q = 0; q < SM; q++)
          av[r][q] = ld_pair(rp, (min(uint32_t(q), splits - 1) * QV + r * G + j) * kPartStride + 4 + d);
      }
      bool ok = !live || (ml.y == tag && ml.w == tag);
#pragma unroll
      for (int r = 0; r < R; r++) {
#pragma unroll
        for (int q = 0; q < SM; q++) ok = ok && av[r][q].y == tag;
      }
      if (poll_done(ok, spins, p.err)) break;
    }
    if (wave == 0) {
      const float m = live ? __uint_as_float(ml.x) : -INFINITY;
      float M = m;
#pragma unroll
      for (int o = 1; o < SM; o <<= 1) M = fmaxf(M, __shfl_xor(M, o));
      const float e = m != -INFINITY ? expf(m - M) : 0.f;
      float L = e * (live ? __uint_as_float(ml.z) : 0.f);
#pragma unroll
      for (int o = 1; o < SM; o <<= 1) L += __shfl_xor(L, o);
      if (lane < QV * SM) {
        mw[jh][u] = e;
        if (u == 0) msum[jh] = L;
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t jq = r * G + j;
      float Av = 0.f;
#pragma unroll
      for (int q = 0; q < SM; q++) Av += uint32_t(q) < splits ? mw[jq][q] * __uint_as_float(av[r][q].x) : 0.f;
      att[r][tid] = Av * (1.0f / msum[jq]);
    }
    __syncthreads();
    }
    // o_proj over this XCD's 256 columns (cpu_inference.rs:163-164): the partial of rows orow0..;
    // the next launch adds the 8 partials and the residual
    float oa[R][ORR];
#pragma unroll
    for (int t = 0; t < R; t++) {
      const float4* at4 = reinterpret_cast<const float4*>(att[t]);
#pragma unroll
      for (uint32_t r = 0; r < ORR; r++) oa[t][r] = 0.f;
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const uint32_t c = t16 + 16 * k;
        const float4 a = at4[2 * c], b = at4[2 * c + 1];
#pragma unroll
        for (uint32_t r = 0; r < ORR; r++) oa[t][r] = dot8(wo[r][k], a, b, oa[t][r]);
      }
#pragma unroll
      for (uint32_t r = 0; r < ORR; r++) oa[t][r] = sum16(oa[t][r]);
    }
    if (t16 == 0) {
#pragma unroll
      for (int t = 0; t < R; t++) {
#pragma unroll
        for (uint32_t r = 0; r < ORR; r++) p.part_out[(t * NX + x) * H + orow0 + ORR * rg + r] = oa[t][r];
      }
    }
  };

  // Slot 0 stores the new generation when its part of the launch is done: every workgroup of
  // the XCD has published its q|k|v rows with this tag by then (the attention reads all of them),
  // so all of them have read the word.
  if constexpr (SM <= 16) {
    if (attn) {  // slots 0..15: the attention runs, no o_proj rows
      attention();
      if (s == 0 && tid == 0)
        __hip_atomic_store(gen_word(sync, x), tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      // done before the merge and o_proj: the run workgroups load pf region 1 (the rest of the
      // MLP block's gate|up rows) while those finish
      if (p.pf_run) prefetch_region<1>(p, x, s, splits);
      finish(kw, p.ts, t_start);
      return;
    }
    if (!oproj) {
      // slots splits..15 are done once their q|k|v rows are out: they load the pf regions (this
      // layer's gate|up rows of XCD x) into the XCD's L2 for the MLP launch (fewer than 16 runs
      // are fewer than 1024 positions, where prefetching pays at any cache element type)
      if (p.pf_idle && splits < 16) prefetch_region<0>(p, x, s - splits, 16 - splits);
      finish(kw, p.ts, t_start);
      return;
    }
    load_wo();
    // the MLP block's down columns of this XCD (pf region 2, when set) into its L2 while the
    // runs work
    prefetch_region<2>(p, x, s - 16, 16);
    merge_oproj();
    finish(kw, p.ts, t_start);
  } else {
    attention();
    merge_oproj();
    if (s == 0 && tid == 0)
      __hip_atomic_store(gen_word(sync, x), tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    finish(kw, p.ts, t_start);
  }
}

// ---------------------------------------------------------------------------------------------
// MLP block of one layer (cpu_inference.rs:166-172)
// ---------------------------------------------------------------------------------------------
// The arguments the first loads need come first, as plain pointers: those are preloaded into
// scalar registers at wave launch (the build's -amdgpu-kernarg-preload-count), so the loads do not
// wait for a scalar load of the argument block.
template <int R>
__global__ __launch_bounds__(256) void k_fused_mlp(uint32_t* sync, const float* res_in, const float* part_in,
                                                   const uint16_t* w_gu, const uint16_t* w_post, const uint16_t* w_down,
                                                   const uint16_t* qkv_next, FusedLayerParams p) {
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t x = fused_xcd(p.err);
  if (blockIdx.x >= NX * NS) {  // a prefetch workgroup (the whole workgroup)
    if (p.state->pos < p.pf_max_pos) fused_prefetch(p, x, (blockIdx.x - NX * NS) / NX, p.pf_wgs);
    return;
  }
  const uint64_t t_start = clock_start();
  const KcacheWarm kw = kcache_warm();
  const uint32_t s = blockIdx.x / NX;
  __shared__ __align__(16) float xs[R * H];
  __shared__ float red4[R][4];
  __shared__ __align__(16) float hs[R][I / NX];  // this XCD's h values of every token row

  const uint32_t tag = *gen_word(sync, x) + 1;

  // gate|up: rows 768 x + 24 s + 6 wave + r (pairs (gate_i, up_i) interleaved), lane l holds
  // chunks l and l + 64. These rows sit in the XCD's L2 (the attention block loaded them) and go
  // first: loads complete in issue order, and they arrive while the residual and the partials come
  // from beyond L2 (with the arguments preloaded, 2252 -> 2300 tok/s against residual first).
  const uint4* Wg = reinterpret_cast<const uint4*>(w_gu);
  const uint32_t row0 = __builtin_amdgcn_readfirstlane((2 * I / NX) * x + 24 * s + 6 * wave);
  uint4 wg[6][2];
#pragma unroll
  for (int r = 0; r < 6; r++) {
#pragma unroll
    for (int k = 0; k < 2; k++) wg[r][k] = Wg[size_t(row0 + r) * (H / 8) + lane + 64 * k];
  }
  __builtin_amdgcn_sched_barrier(0);
  float4 xin[R];
  float4 xp[R][NX];
#pragma unroll
  for (int r = 0; r < R; r++) {
    xin[r] = reinterpret_cast<const float4*>(res_in + r * H)[tid];
#pragma unroll
    for (uint32_t g = 0; g < NX; g++) xp[r][g] = reinterpret_cast<const float4*>(part_in + (r * NX + g) * H)[tid];
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 gp[2];
#pragma unroll
  for (int k = 0; k < 2; k++) gp[k] = reinterpret_cast<const uint4*>(w_post)[lane + 64 * k];
  // down rows 32 s + 2 rg + r over columns [384 x, 384 x + 384): 16 threads per row, chunks
  // t16, t16 + 16, t16 + 32 of the slice
  const uint32_t rg = tid >> 4, t16 = tid & 15;
  const uint4* Wd = reinterpret_cast<const uint4*>(w_down);
  uint4 wd[2][3];
#pragma unroll
  for (int r = 0; r < 2; r++) {
#pragma unroll
    for (int k = 0; k < 3; k++) wd[r][k] = Wd[size_t(32 * s + 2 * rg + r) * (I / 8) + 48 * x + t16 + 16 * k];
  }
  // the next layer's q|k|v rows that slot s of its attention block reads (16 rows of 2 KB: 512
  // 64-byte half lines) into XCD x's L2, one word of half lines tid and tid + 256, through a
  // descriptor that holds no bytes for the last layer (its loads then read 0 without touching
  // memory; a branch here would make the waits after it wait for every load)
  const __amdgpu_buffer_rsrc_t rq = rsrc_of(qkv_next ? qkv_next + size_t(qkv_row0(x, s)) * H : w_gu,
                                            qkv_next ? 16 * H * 2 : 0);
  uint32_t pfw[2];
#pragma unroll
  for (int k = 0; k < 2; k++) pfw[k] = __builtin_amdgcn_raw_buffer_load_b32(rq, int((tid + 256 * k) * 64), 0, 0);
  __builtin_amdgcn_sched_barrier(0);

  // post_attention_layernorm + gate|up + silu * up (cpu_inference.rs:167-170)
  {
    float rs[R];
    residual_and_scale<R>(xin, xp, true, xs, p.res_out, p.eps, red4, rs);
    float acc[R][6];
#pragma unroll
    for (int t = 0; t < R; t++) {
      const float4* xs4 = reinterpret_cast<const float4*>(xs + t * H);
#pragma unroll
      for (int r = 0; r < 6; r++) acc[t][r] = 0.f;
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const uint32_t c = lane + 64 * k;
        float4 a = xs4[2 * c], b = xs4[2 * c + 1];
        scale8(a, b, gp[k]);
#pragma unroll
        for (int r = 0; r < 6; r++) acc[t][r] = dot8(wg[r][k], a, b, acc[t][r]);
      }
#pragma unroll
      for (int r = 0; r < 6; r++) acc[t][r] = wave_sum(acc[t][r]) * rs[t];
    }
    if (lane == 0) {
#pragma unroll
      for (int t = 0; t < R; t++) {
#pragma unroll
        for (int i = 0; i < 3; i++) {
          const float gt = acc[t][2 * i];
          p.h[t * I + (row0 >> 1) + i] = pair(gt / (1.0f + expf(-gt)) * acc[t][2 * i + 1], tag);
        }
      }
    }
  }

  // down over this XCD's 384 columns (cpu_inference.rs:171-172): the partial of rows 32 s ..
  // Wave 0 alone polls the XCD's 384 h pairs (lane l: pairs 6 l .. 6 l + 5) and leaves the values
  // in LDS: a poll round is 3 KB of L2 reads per workgroup instead of every thread's 24 pairs.
  const __amdgpu_buffer_rsrc_t rh = rsrc_of(p.h + (I / NX) * x, ((R - 1) * I + I / NX) * 8);
  if (wave < uint32_t(R)) {  // wave t: token row t
    const uint32_t t = wave;
    uint4 hv[3];
    for (uint32_t spins = 0;;) {
#pragma unroll
      for (int k = 0; k < 3; k++) hv[k] = ld_pair2(rh, t * I + 6 * lane + 2 * k);
      bool ok = true;
#pragma unroll
      for (int k = 0; k < 3; k++) ok = ok && hv[k].y == tag && hv[k].w == tag;
      if (poll_done(ok, spins, p.err)) break;
    }
#pragma unroll
    for (int k = 0; k < 3; k++) {
      hs[t][6 * lane + 2 * k] = __uint_as_float(hv[k].x);
      hs[t][6 * lane + 2 * k + 1] = __uint_as_float(hv[k].z);
    }
  }
  __syncthreads();
  float da[R][2];
#pragma unroll
  for (int t = 0; t < R; t++) {
    const float4* hs4 = reinterpret_cast<const float4*>(hs[t]);
    da[t][0] = 0.f;
    da[t][1] = 0.f;
#pragma unroll
    for (int k = 0; k < 3; k++) {  // chunk c = t16 + 16 k: h values 8 c .. 8 c + 7
      const uint32_t c = t16 + 16 * k;
      const float4 ha = hs4[2 * c], hb = hs4[2 * c + 1];
#pragma unroll
      for (int r = 0; r < 2; r++) da[t][r] = dot8(wd[r][k], ha, hb, da[t][r]);
    }
  }
  // keeps the prefetch loads: they were issued after down's weights, which are in by now (a wait
  // for them after this wave's next store would also wait for that store)
  asm volatile("" ::"v"(pfw[0] ^ pfw[1]));
#pragma unroll
  for (int t = 0; t < R; t++) {
#pragma unroll
    for (int r = 0; r < 2; r++) da[t][r] = sum16(da[t][r]);
  }
  if (t16 == 0) {
#pragma unroll
    for (int t = 0; t < R; t++) {
#pragma unroll
      for (int r = 0; r < 2; r++) p.part_out[(t * NX + x) * H + 32 * s + 2 * rg + r] = da[t][r];
    }
  }
  // every workgroup of the XCD has published its h values with this tag (the down rows need all
  // of them), so all of them have read the generation word
  if (s == 0 && tid == 0)
    __hip_atomic_store(gen_word(sync, x), tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  finish(kw, p.ts, t_start);
}

// x = res + part[0] + ... + part[7], workgroup r for token row r. With a gain, out = the final
// RMSNorm of x instead, (x s) gain with s = 1 / sqrt(mean(x^2) + eps), the
// lm_head's prologue summed in its order (cpu_inference.rs:175-176), so that no lm_head workgroup
// repeats it.
__global__ __launch_bounds__(256) void k_fused_reduce(const float* __restrict__ res, const float* __restrict__ part,
                                                      float* __restrict__ out, const uint16_t* __restrict__ gain,
                                                      float eps) {
  const uint32_t tid = threadIdx.x, r = blockIdx.x;
  res += r * H;
  part += r * NX * H;
  out += r * H;
  float4 v = reinterpret_cast<const float4*>(res)[tid];
  float4 xp[NX];
#pragma unroll
  for (uint32_t g = 0; g < NX; g++) xp[g] = reinterpret_cast<const float4*>(part + g * H)[tid];
#pragma unroll
  for (uint32_t g = 0; g < NX; g++) v = add4(v, xp[g]);
  if (gain) {
    __shared__ float red[4];
    const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float sc = 1.0f / sqrtf(tot / float(H) + eps);
    const uint2 gw = reinterpret_cast<const uint2*>(gain)[tid];
    v.x = v.x * sc * __uint_as_float(gw.x << 16);
    v.y = v.y * sc * __uint_as_float(gw.x & 0xFFFF0000u);
    v.z = v.z * sc * __uint_as_float(gw.y << 16);
    v.w = v.w * sc * __uint_as_float(gw.y & 0xFFFF0000u);
  }
  reinterpret_cast<float4*>(out)[tid] = v;
}

// ids[i] = the XCD workgroup i runs on
__global__ __launch_bounds__(256) void k_place_check(uint32_t* ids) {
  if (threadIdx.x == 0) ids[blockIdx.x] = xcc_id();
}

template <bool FIRST, bool KV_BF16, int SM, bool MULTI, int NT, int R>
void launch_attn_v(const FusedLayerParams& p, hipStream_t s) {
  hipLaunchKernelGGL((k_fused_attn<FIRST, KV_BF16, SM, MULTI, NT, R>), dim3(NX * (NS + p.pf_wgs)), dim3(256), 0, s,
                     p.sync, p.state, p.res_in, p.part_in, p.w_qkv, p.w_in, p.splits, p.run, p);
}

template <bool FIRST, bool KV_BF16, int R>
hipError_t launch_attn_sm(const FusedLayerParams& p, hipStream_t s) {
  if (p.run == 32) {  // runs of one 32-position tile
    if (p.splits <= 4) launch_attn_v<FIRST, KV_BF16, 4, false, 32, R>(p, s);
    else if (p.splits <= 8) launch_attn_v<FIRST, KV_BF16, 8, false, 32, R>(p, s);
    else launch_attn_v<FIRST, KV_BF16, 16, false, 32, R>(p, s);
  } else if (p.splits <= 4) {
    launch_attn_v<FIRST, KV_BF16, 4, false, 64, R>(p, s);
  } else if (p.splits <= 8) {
    launch_attn_v<FIRST, KV_BF16, 8, false, 64, R>(p, s);
  } else if (p.splits <= 16) {
    launch_attn_v<FIRST, KV_BF16, 16, false, 64, R>(p, s);
  } else if constexpr (R == 1) {
    if (p.run == 64) launch_attn_v<FIRST, KV_BF16, 32, false, 64, 1>(p, s);
    else launch_attn_v<FIRST, KV_BF16, 32, true, 64, 1>(p, s);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

bool common_ok(const FusedLayerParams& p) {
  if (!p.res_out || !p.part_out || !p.sync || !p.err || !p.state || p.pf_wgs > 64) return false;
  for (const FusedPrefetch& r : p.pf)
    if (r.base && (r.row_bytes < 4 || r.rows == 0)) return false;
  return true;
}

}  // namespace

hipError_t QE_FUSED_LAUNCHER(launch_fused_attn)(const FusedLayerParams& p, bool first_layer, hipStream_t s) {
  if (!common_ok(p) || !p.w_in || !p.w_qkv || !p.q_norm || !p.k_norm || !p.w_o || !p.qkv || !p.attn_part ||
      !p.k_cache || !p.v_cache || !p.rope_cur || p.max_seq == 0 || p.splits == 0 || p.splits > kFusedMaxRuns ||
      (p.splits > 16 && p.splits != kFusedMaxRuns) || (p.splits <= 16 && p.run != 64 && p.run != 32) ||
      (p.splits > 16 && (p.run == 0 || p.run % 64)))
    return hipErrorInvalidValue;
  if (first_layer ? (!p.embed || !p.tokens || p.vocab == 0) : (!p.res_in || !p.part_in)) return hipErrorInvalidValue;
  if (p.rows == 2) {  // verify rows: single-tile runs only
    if (p.splits > 16) return hipErrorInvalidValue;
    if (first_layer) return p.kv_bf16 ? launch_attn_sm<true, true, 2>(p, s) : launch_attn_sm<true, false, 2>(p, s);
    return p.kv_bf16 ? launch_attn_sm<false, true, 2>(p, s) : launch_attn_sm<false, false, 2>(p, s);
  }
  if (p.rows != 1) return hipErrorInvalidValue;
  if (first_layer) return p.kv_bf16 ? launch_attn_sm<true, true, 1>(p, s) : launch_attn_sm<true, false, 1>(p, s);
  return p.kv_bf16 ? launch_attn_sm<false, true, 1>(p, s) : launch_attn_sm<false, false, 1>(p, s);
}

hipError_t QE_FUSED_LAUNCHER(launch_fused_mlp)(const FusedLayerParams& p, hipStream_t s) {
  if (!common_ok(p) || !p.res_in || !p.part_in || !p.w_post || !p.w_gu || !p.w_down || !p.h) return hipErrorInvalidValue;
  if (p.rows == 1)
    hipLaunchKernelGGL(k_fused_mlp<1>, dim3(NX * (NS + p.pf_wgs)), dim3(256), 0, s, p.sync, p.res_in, p.part_in, p.w_gu,
                       p.w_post, p.w_down, p.qkv_next, p);
  else if (p.rows == 2)
    hipLaunchKernelGGL(k_fused_mlp<2>, dim3(NX * (NS + p.pf_wgs)), dim3(256), 0, s, p.sync, p.res_in, p.part_in, p.w_gu,
                       p.w_post, p.w_down, p.qkv_next, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

#ifndef QE_FUSED_TIMED
hipError_t launch_fused_reduce(const float* res, const float* part, float* x, uint32_t rows, const uint16_t* gain,
                               float eps, hipStream_t s) {
  if (!res || !part || !x || rows == 0 || rows > kFusedMaxRows) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_fused_reduce, dim3(rows), dim3(256), 0, s, res, part, x, gain, eps);
  return hipGetLastError();
}

hipError_t fused_placement_check(uint32_t* dev_ids, uint32_t* host_ids, bool* ok, hipStream_t s) {
  *ok = false;
  hipLaunchKernelGGL(k_place_check, dim3(NX * NS), dim3(256), 0, s, dev_ids);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(host_ids, dev_ids, NX * NS * 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return e;
  bool good = host_ids[0] < NX;
  for (uint32_t i = 0; i < NX * NS; i++) good = good && host_ids[i] == (host_ids[0] + i) % NX;
  *ok = good;
  return e;
}
#endif

}  // namespace qe
