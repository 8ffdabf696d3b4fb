// The decode step's 28 layers in one persistent launch, for the Qwen3-0.6B shape (hidden 1024,
// 16 q heads over 8 KV heads of 128, SwiGLU 3072). The lm_head and the argmax follow as launches
// of their own.
//
// Reference: cpu_inference.rs:98-173 (Model::forward up to the final norm), inference.metal.
//
// 256 workgroups of 512 threads, one per CU, all resident at once: XCD x (HW_REG_XCC_ID) serves
// KV head x, slot s = blockIdx.x / 8 (each XCD gets the slots 0..31 whatever the round-robin
// start of the launch). The work of a layer is that of the two launches of fused.hip (attention
// block, MLP block); what those launches hand over at a launch boundary is exchanged here too:
//   - inside an XCD (q|k|v rows, attention partials, h, the gathered residual stream): (value,
//     tag) pairs with plain stores, read with device-scope (sc1) loads from the XCD's L2;
//   - across XCDs (the o_proj and down outputs, split over the XCDs' input columns): pairs with
//     device-scope stores, written through to memory. Workgroup (x, s) sums the 8 XCDs' partials
//     of columns [32s, 32s+32) onto its copy of the residual stream (every XCD keeps the whole
//     stream, the same values in each), publishes them inside its XCD, and every workgroup
//     gathers the 1024 values from its XCD's L2.
// Loads complete in issue order within a wave, so a wave that has weights in flight cannot see a
// polled value before they arrive. The waves are therefore split: waves 0-3 compute (they hold
// the weights, and issue the next stage's weight loads as soon as a stage's outputs are out),
// waves 4-7 poll, reduce and gather into LDS and load nothing else. The two groups meet at
// workgroup barriers, seven per layer plus the attention's own.
// Tags: tag = (generation + 1) * 32 + layer, one value per layer and step; every buffer is written
// once per layer, and no workgroup can reach a buffer's next layer before every reader of its
// previous one has read it (each layer ends in a reduction every workgroup takes part in).
// Workgroup 0 advances the generation word after its last reduction, which needs the down rows of
// every XCD's slot 0, which need the h values of every workgroup: all of them read the word by then.
// Every wait is bounded (kSpinMax polls, then kErrSync; once one wait has given up the others
// stop within 1024 polls), so no wave waits for ever.
#include <cmath>

#include "attn_tile.h"
#include "device_common.h"
#include "kernels.h"
#include "xcd_exchange.h"

namespace qe {
namespace {

constexpr uint32_t H = kFusedH, I = kFusedI, D = kHeadDim, NKV = kFusedKv, G = kFusedHeads / kFusedKv;
constexpr uint32_t QD = kFusedHeads * D, KD = NKV * D;
constexpr uint32_t NX = kFusedXcds, NS = kFusedSlots;

static_assert(NKV == NX && G == 2 && H == 1024 && I == 3072, "the layouts below are written for these sizes");

// sum of the 4 exchange waves' partial sums of squares -> RMSNorm scale
__device__ __forceinline__ float norm_scale(const float* ssq, float eps) {
  return 1.0f / sqrtf(((ssq[0] + ssq[1]) + (ssq[2] + ssq[3])) / float(H) + eps);
}

// first q|k|v row of slot s of KV head x (16 consecutive rows per slot, see fused.hip)
__device__ __forceinline__ uint32_t prow0(uint32_t x, uint32_t s) {
  return s < 16 ? x * G * D + 16 * s : s < 24 ? QD + x * D + 16 * (s - 16) : QD + KD + x * D + 16 * (s - 24);
}

// p, hidden from the compiler once per layer: addresses formed from it are recomputed in the
// layer loop (a few ALU instructions) instead of being hoisted out of it and held in registers
// for the whole loop
template <typename T>
__device__ __forceinline__ T* opaque(T* p) {
  asm volatile("" : "+s"(p));
  return p;
}

// Waits, reading one sentinel value per lane and sleeping SLEEP x 64 clocks between reads, until
// every lane's sentinel carries the tag (the data it stands for is then read and checked in full):
// waiting waves keep their request traffic low while the critical loads run.
template <int SLEEP, typename F>
__device__ __forceinline__ void await(F sentinel_ready, uint32_t* err) {
  for (uint32_t spins = 0;;) {
    if (poll_done(sentinel_ready(), spins, err)) break;
    __builtin_amdgcn_s_sleep(SLEEP);
  }
}

template <typename T>
__device__ __forceinline__ const T* at_layer(const T* base, uint64_t stride, uint32_t l) {
  return reinterpret_cast<const T*>(reinterpret_cast<const uint8_t*>(base) + size_t(l) * stride);
}

template <bool KV_BF16, int SM, bool MULTI>
__global__ __launch_bounds__(512) void k_decode_persist(PersistParams p) {
  static_assert(SM == 32 || !MULTI, "runs of several tiles come with 32 runs");
  constexpr uint32_t T = 64;
  constexpr uint32_t ORR = SM <= 16 ? 4 : 2;  // o_proj rows per 16-thread row group
  const uint32_t tid = threadIdx.x;
  const bool cw = tid < 256;  // compute waves 0-3 / exchange waves 4-7 (wave-uniform)
  const uint32_t ct = tid & 255, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t cwave = wave & 3;
  const uint32_t x = fused_xcd(p.err), s = blockIdx.x / NX;
  const uint32_t splits = max(p.splits, 1u);
  const bool attn = s < splits;
  const bool oproj = SM <= 16 ? s >= 16 : true;
  const uint32_t orow0 = SM <= 16 ? 64 * (s - 16) : 32 * s;
  const int pg = ct >> 3, dc = ct & 7, dg = ct & 31, pp = ct >> 5;
  const uint32_t rg = ct >> 4, t16 = ct & 15;

  __shared__ __align__(16) float xs[H];
  __shared__ float ssq[4];
  __shared__ __align__(16) float qraw[G + 2][D];
  __shared__ __align__(16) float qs[G][D];
  __shared__ __align__(16) float knew[D];
  __shared__ __align__(16) float vnew[D];
  __shared__ float sc[G][T], pes[G][T];
  __shared__ float Ms[G], Ls[G], Cs[G];
  __shared__ __align__(16) float red[8][G][D];
  __shared__ __align__(16) float att[G * D];
  __shared__ __align__(16) float hs[I / NX];

  const uint32_t tb = (__hip_atomic_load(p.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1) << 5;

  // the step's position and this slot's attention run (the same for every layer)
  const uint32_t pos = p.state->pos;
  const bool bad = pos >= p.max_seq;
  if (bad && blockIdx.x == 0 && tid == 0) atomicOr(p.err, kErrPos);
  uint32_t n = bad ? 0u : pos + 1;
  if (n > splits * p.run) {  // the host's runs would skip positions
    if (blockIdx.x == 0 && tid == 0) atomicOr(p.err, kErrShape);
    n = 0;
  }
  const uint32_t t0 = s * p.run, t1 = min(n, t0 + p.run);
  const bool owns_new = n != 0 && pos >= t0 && pos < t0 + p.run;
  const uint32_t ntiles = t1 > t0 ? ceil_div(t1 - t0, T) : 1u;  // an empty run takes one masked tile

  // Compute waves and exchange waves run separate loops (so neither holds the other's registers)
  // that pass the same workgroup barriers in the same order: per layer one after the q|k|v rows,
  // the attention's (2 + 2 per tile, attention runs only), and four after the merge, o_proj,
  // gate|up and down.
  if (cw) {
    // ================= compute waves: weights in registers =================
    const uint32_t qrow0 = __builtin_amdgcn_readfirstlane(prow0(x, s) + 4 * cwave);
    const uint32_t grow0 = __builtin_amdgcn_readfirstlane((2 * I / NX) * x + 24 * s + 6 * cwave);
    const size_t head_base = size_t(x) * p.max_seq * D;
    uint4 wq[4][2], gin[2], wo[ORR][2], wg[6][2], gp[2], wd[2][3];
    KVTile<KV_BF16> A;
    uint16_t gq[2] = {0, 0}, gk[2] = {0, 0};
    float2 cs = make_float2(0.f, 0.f);
    // Weight loads go through buffer descriptors: the layer's tensor base in scalar registers,
    // row offsets as scalar offsets and one 32-bit lane offset per layout, so that no 64-bit
    // per-lane address lives across the layer loop.
    const uint32_t lane16 = lane * 16;                                                 // q|k|v, gate|up, gains
    const uint32_t wo_off = ((orow0 + ORR * rg) * (QD / 8) + 32 * x + t16) * 16;    // o_proj
    const uint32_t wd_off = ((32 * s + 2 * rg) * (I / 8) + 48 * x + t16) * 16;      // down
    auto wbuf = [&](const uint16_t* base, uint32_t l, uint32_t bytes) __attribute__((always_inline)) {
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(at_layer(base, p.layer_stride, l)), short(0),
                                               int(bytes), 0x00020000);
    };
    auto ldw = [](__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) __attribute__((always_inline)) {
      return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), 0));
    };
    // layer l's q|k|v rows and their norm gain (loaded at the end of layer l - 1)
    auto load_qkv_w = [&](uint32_t l) __attribute__((always_inline)) {
      const __amdgpu_buffer_rsrc_t rq = wbuf(p.w_qkv, l, (QD + 2 * KD) * H * 2);
#pragma unroll
      for (int r = 0; r < 4; r++) {
#pragma unroll
        for (int k = 0; k < 2; k++) wq[r][k] = ldw(rq, lane16 + 1024 * k, (qrow0 + r) * (H * 2));
      }
      const __amdgpu_buffer_rsrc_t ri = wbuf(p.w_in, l, H * 2);
#pragma unroll
      for (int k = 0; k < 2; k++) gin[k] = ldw(ri, lane16 + 1024 * k, 0);
    };
    // an attention run's first K/V tile of layer l, its q/k norm gains and this position's RoPE
    // row (loaded once the run's q|k|v rows are out)
    // this head's K and V regions of layer l
    constexpr uint32_t EL = KV_BF16 ? 2 : 4;
    auto kv_rsrc = [&](const void* cache, uint32_t l) __attribute__((always_inline)) {
      const uint8_t* b = static_cast<const uint8_t*>(cache) + (size_t(l) * p.layer_kv + head_base) * EL;
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(b), short(0), int(p.max_seq * D * EL), 0x00020000);
    };
    auto load_attn_inputs = [&](uint32_t l) __attribute__((always_inline)) {
      load_tile_buf<KV_BF16>(A, kv_rsrc(p.k_cache, l), kv_rsrc(p.v_cache, l), t0, ct);
      const uint16_t* qn = at_layer(p.q_norm, p.layer_stride, l);
      const uint16_t* kn = at_layer(p.k_norm, p.layer_stride, l);
      gq[0] = qn[lane];
      gq[1] = qn[lane + 64];
      gk[0] = kn[lane];
      gk[1] = kn[lane + 64];
      cs = reinterpret_cast<const float2*>(p.rope_cur)[lane];
    };
    // layer l's o_proj rows (o_proj slots), gate|up rows and their norm gain (the layouts of
    // fused.hip)
    auto load_out_w = [&](uint32_t l) __attribute__((always_inline)) {
      if (oproj) {
        const __amdgpu_buffer_rsrc_t ro = wbuf(p.w_o, l, H * QD * 2);
#pragma unroll
        for (uint32_t r = 0; r < ORR; r++) {
#pragma unroll
          for (int k = 0; k < 2; k++) wo[r][k] = ldw(ro, wo_off + 256 * k, r * (QD * 2));
        }
      }
      const __amdgpu_buffer_rsrc_t rgu = wbuf(p.w_gu, l, 2 * I * H * 2);
#pragma unroll
      for (int r = 0; r < 6; r++) {
#pragma unroll
        for (int k = 0; k < 2; k++) wg[r][k] = ldw(rgu, lane16 + 1024 * k, (grow0 + r) * (H * 2));
      }
      const __amdgpu_buffer_rsrc_t rp = wbuf(p.w_post, l, H * 2);
#pragma unroll
      for (int k = 0; k < 2; k++) gp[k] = ldw(rp, lane16 + 1024 * k, 0);
    };
    // layer l's down rows (loaded once the gate|up rows are out, so that they never share
    // registers with the o_proj rows)
    auto load_down_w = [&](uint32_t l) __attribute__((always_inline)) {
      const __amdgpu_buffer_rsrc_t rd = wbuf(p.w_down, l, H * I * 2);
#pragma unroll
      for (int r = 0; r < 2; r++) {
#pragma unroll
        for (int k = 0; k < 3; k++) wd[r][k] = ldw(rd, wd_off + 256 * k, r * (I * 2));
      }
    };

    load_qkv_w(0);
    __syncthreads();  // layer 0's x (the embedding row) is in xs

    for (uint32_t l = 0; l < p.n_layers; l++) {
      const uint32_t tag = tb + l;
      const size_t kv_off = size_t(l) * p.layer_kv * (KV_BF16 ? 2 : 4);
      void* k_cache = static_cast<uint8_t*>(p.k_cache) + kv_off;
      void* v_cache = static_cast<uint8_t*>(p.v_cache) + kv_off;

      // ---- input RMSNorm + 16 q|k|v rows (cpu_inference.rs:129-132) ----
      {
        const float rs = norm_scale(ssq, p.eps);
        const float4* xs4 = reinterpret_cast<const float4*>(xs);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 2; k++) {
          const uint32_t c = lane + 64 * k;
          float4 a = xs4[2 * c], b = xs4[2 * c + 1];
          scale8(a, b, gin[k]);
#pragma unroll
          for (int q = 0; q < 4; q++) acc[q] = dot8(wq[q][k], a, b, acc[q]);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) acc[q] = wave_sum(acc[q]) * rs;
        if (lane == 0) {
#pragma unroll
          for (int q = 0; q < 4; q++) opaque(p.qkv)[qrow0 + q] = pair(acc[q], tag);
        }
      }
      // an attention run's next loads: its K/V tile
      if (attn) load_attn_inputs(l);
      __syncthreads();  // the run's raw q/k/v rows are in qraw

      // ---- attention run s of KV head x (cpu_inference.rs:134-162) ----
      if (attn) {
        {
          // q/k RMSNorm (cpu_inference.rs:189-194) + rotate-half RoPE (cpu_inference.rs:203-215)
          float a = qraw[cwave][lane], b = qraw[cwave][lane + 64];
          if (cwave <= G) {
            const float ss = wave_sum(a * a + b * b);
            const float scl = 1.0f / sqrtf(ss / float(D) + p.eps);
            a = a * scl * bf16f(cwave < G ? gq[0] : gk[0]);
            b = b * scl * bf16f(cwave < G ? gq[1] : gk[1]);
            const float ar = a * cs.x - b * cs.y, br = b * cs.x + a * cs.y;
            a = ar;
            b = br;
          }
          if (KV_BF16 && cwave >= G) {  // attend with the values later steps read back
            a = bf16f(f32_to_bf16(a));
            b = bf16f(f32_to_bf16(b));
          }
          float* dst = cwave < G ? qs[cwave] : (cwave == G ? knew : vnew);
          dst[lane] = a;
          dst[lane + 64] = b;
          if (ct < G) {
            Ms[ct] = -INFINITY;
            Ls[ct] = 0.f;
          }
        }
        __syncthreads();
        if (owns_new) {  // append the new K/V row (cpu_inference.rs:140-141)
          const size_t slot = head_base + size_t(pos) * D + (ct & (D - 1));
          const float val = ct < D ? knew[ct] : vnew[ct - D];
          void* cache = ct < D ? k_cache : v_cache;
          if (KV_BF16) static_cast<uint16_t*>(cache)[slot] = f32_to_bf16(val);
          else static_cast<float*>(cache)[slot] = val;
        }
        float4 acc[G];
#pragma unroll
        for (uint32_t j = 0; j < G; j++) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        // one 64-position tile, with its two barriers
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
            for (uint32_t j = 0; j < G; j++) {
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
              for (uint32_t j = 0; j < G; j++) sc[j][pg + 32 * u] = t < t1 ? sv[j] * p.scale : -INFINITY;
            }
          }
          __syncthreads();
          // softmax (cpu_inference.rs:217-223) as an online update: running max, rescaled sum
          if (cwave < G) {
            const uint32_t j = cwave;
            const float xv = sc[j][lane];
            const float m_old = Ms[j];
            const float m_new = fmaxf(m_old, wave_max(xv));
            const float pe = xv == -INFINITY ? 0.f : expf(xv - m_new);
            const float c = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
            const float tsum = wave_sum(pe);
            pes[j][lane] = pe;
            if (lane == 0) {
              Ls[j] = Ls[j] * c + tsum;
              Ms[j] = m_new;
              Cs[j] = c;
            }
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
          for (uint32_t j = 0; j < G; j++) {
            const float c = Cs[j];
            float4 o = make_float4(acc[j].x * c, acc[j].y * c, acc[j].z * c, acc[j].w * c);
#pragma unroll
            for (int i = 0; i < 8; i++) {
              const float pe = pes[j][8 * pp + i];
              o.x += pe * v4[i].x;
              o.y += pe * v4[i].y;
              o.z += pe * v4[i].z;
              o.w += pe * v4[i].w;
            }
            acc[j] = o;
          }
        };
        if constexpr (MULTI) {
          // runs of several tiles alternate between two register sets, so the next tile's loads
          // are in flight while one is computed
          KVTile<KV_BF16> B;
          const __amdgpu_buffer_rsrc_t rk = kv_rsrc(p.k_cache, l), rv = kv_rsrc(p.v_cache, l);
          for (uint32_t i = 0;; i += 2) {
            const bool more = i + 1 < ntiles;
            if (more) load_tile_buf<KV_BF16>(B, rk, rv, t0 + T * (i + 1), ct);
            __builtin_amdgcn_sched_barrier(0);
            process(A, t0 + T * i);
            if (!more) break;
            const bool more2 = i + 2 < ntiles;
            if (more2) load_tile_buf<KV_BF16>(A, rk, rv, t0 + T * (i + 2), ct);
            __builtin_amdgcn_sched_barrier(0);
            process(B, t0 + T * (i + 1));
            if (!more2) break;
          }
        } else {
          process(A, t0);
        }
        // the 8 position groups meet; m and l are the softmax state; the partial goes out as pairs
#pragma unroll
        for (uint32_t j = 0; j < G; j++) reinterpret_cast<float4*>(red[pp][j])[dg] = acc[j];
        __syncthreads();
        {
          uint2* part = opaque(p.attn_part) + (size_t(x) * kFusedMaxRuns + s) * G * kPartStride;
          const uint32_t j = ct / D, d = ct % D;
          float v = 0.f;
#pragma unroll
          for (int q = 0; q < 8; q++) v += red[q][j][d];
          part[j * kPartStride + 4 + d] = pair(v, tag);
          if (d == 0) {
            part[j * kPartStride] = pair(Ms[j], tag);
            part[j * kPartStride + 1] = pair(Ls[j], tag);
          }
        }
      }
      // this layer's o_proj and MLP weights (right after the q|k|v rows in slots without an
      // attention run; loaded at one point so that they never share registers with a K/V tile)
      load_out_w(l);
      __syncthreads();  // the merged attention output is in att

      // ---- o_proj rows over this XCD's 256 columns (cpu_inference.rs:163-164), to every XCD ----
      if (oproj) {
        const float4* at4 = reinterpret_cast<const float4*>(att);
        float oa[ORR];
#pragma unroll
        for (uint32_t q = 0; q < ORR; q++) oa[q] = 0.f;
#pragma unroll
        for (int k = 0; k < 2; k++) {
          const uint32_t c = t16 + 16 * k;
          const float4 a = at4[2 * c], b = at4[2 * c + 1];
#pragma unroll
          for (uint32_t q = 0; q < ORR; q++) oa[q] = dot8(wo[q][k], a, b, oa[q]);
        }
#pragma unroll
        for (uint32_t q = 0; q < ORR; q++) oa[q] = sum16(oa[q]);
        if (t16 == 0) {
#pragma unroll
          for (uint32_t q = 0; q < ORR; q++) st_pair_dev(opaque(p.part_a) + x * H + orow0 + ORR * rg + q, pair(oa[q], tag));
        }
      }
      __syncthreads();  // x' (after the attention) is in xs

      // ---- post_attention_layernorm + gate|up + silu * up (cpu_inference.rs:167-170) ----
      {
        const float rs = norm_scale(ssq, p.eps);
        const float4* xs4 = reinterpret_cast<const float4*>(xs);
        float acc[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 2; k++) {
          const uint32_t c = lane + 64 * k;
          float4 a = xs4[2 * c], b = xs4[2 * c + 1];
          scale8(a, b, gp[k]);
#pragma unroll
          for (int q = 0; q < 6; q++) acc[q] = dot8(wg[q][k], a, b, acc[q]);
        }
#pragma unroll
        for (int q = 0; q < 6; q++) acc[q] = wave_sum(acc[q]) * rs;
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < 3; i++) {
            const float gt = acc[2 * i];
            opaque(p.h)[(grow0 >> 1) + i] = pair(gt / (1.0f + expf(-gt)) * acc[2 * i + 1], tag);
          }
        }
      }
      load_down_w(l);
      __syncthreads();  // this XCD's h values are in hs

      // ---- down rows over this XCD's 384 columns (cpu_inference.rs:171-172), to every XCD; then
      // the next layer's q|k|v weights ----
      {
        const float4* h4 = reinterpret_cast<const float4*>(hs);
        float da[2] = {0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 3; k++) {
          const uint32_t c = t16 + 16 * k;
          const float4 a = h4[2 * c], b = h4[2 * c + 1];
#pragma unroll
          for (int q = 0; q < 2; q++) da[q] = dot8(wd[q][k], a, b, da[q]);
        }
#pragma unroll
        for (int q = 0; q < 2; q++) da[q] = sum16(da[q]);
        if (t16 == 0) {
#pragma unroll
          for (int q = 0; q < 2; q++) st_pair_dev(opaque(p.part_m) + x * H + 32 * s + 2 * rg + q, pair(da[q], tag));
        }
      }
      if (l + 1 < p.n_layers) load_qkv_w(l + 1);
      __syncthreads();  // the next layer's x is in xs
    }
  } else {
    // ================= exchange waves: polls, reductions, gathers =================
    // wave 4 keeps this slot's columns [32 s, 32 s + 32) of the residual stream (lanes c and
    // c + 32 both hold column c)
    float r = 0.f;
    // x += the 8 XCDs' partials of this slot's columns (sum order (P0 + P2 + P4 + P6) + (P1 + P3
    // + P5 + P7), the same in every XCD), published inside the XCD; then (gather) every exchange
    // thread collects 4 of the 1024 values into xs and the sums of squares into ssq
    auto reduce_gather = [&](const uint2* part, uint2* xbuf, uint32_t tag, bool gather) __attribute__((always_inline)) {
      if (wave == 4) {
        const uint32_t c = lane & 31, g0 = lane >> 5;
        await<4>([&] { return ld_pair_dev(opaque(part) + (g0 + 6) * H + 32 * s + c).y == tag; }, p.err);
        uint2 v[4];
        for (uint32_t spins = 0;;) {
          bool ok = true;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            v[k] = ld_pair_dev(opaque(part) + (g0 + 2 * k) * H + 32 * s + c);
            ok = ok && v[k].y == tag;
          }
          if (poll_done(ok, spins, p.err)) break;
        }
        const float mine = (__uint_as_float(v[0].x) + __uint_as_float(v[1].x)) +
                           (__uint_as_float(v[2].x) + __uint_as_float(v[3].x));
        r = r + (mine + __shfl_xor(mine, 32));
        if (lane < 32) opaque(xbuf)[x * H + 32 * s + c] = pair(r, tag);
      }
      if (gather) {
        const __amdgpu_buffer_rsrc_t rx = rsrc_of(xbuf + x * H, H * 8);
        await<2>([&] { return ld_pair(rx, ct + 768).y == tag; }, p.err);
        uint2 w[4];
        for (uint32_t spins = 0;;) {
          bool ok = true;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            w[k] = ld_pair(rx, ct + 256 * k);
            ok = ok && w[k].y == tag;
          }
          if (poll_done(ok, spins, p.err)) break;
        }
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float v = __uint_as_float(w[k].x);
          xs[ct + 256 * k] = v;
          ss += v * v;
        }
        ss = wave_sum(ss);
        if (lane == 0) ssq[wave - 4] = ss;
      }
    };

    // layer 0's input: the embedding row of the step's token
    {
      uint32_t tok = p.tokens[p.state->tok_idx];
      if (tok >= p.vocab) {
        if (blockIdx.x == 0 && ct == 0) atomicOr(p.err, kErrToken);
        tok = 0;
      }
      const uint2 e = reinterpret_cast<const uint2*>(p.embed + size_t(tok) * H)[ct];
      const float4 v = bf16x4(e.x, e.y);
      reinterpret_cast<float4*>(xs)[ct] = v;
      const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
      if (lane == 0) ssq[wave - 4] = ss;
      if (wave == 4) r = bf16f(p.embed[size_t(tok) * H + 32 * s + (lane & 31)]);
    }
    __syncthreads();

    for (uint32_t l = 0; l < p.n_layers; l++) {
      const uint32_t tag = tb + l;
      // the raw q/k/v rows of KV head x: row ct / 64 of [q head 2x, q head 2x+1, k, v], lane l
      // takes dims l and l + 64
      if (attn) {
        const __amdgpu_buffer_rsrc_t rq = rsrc_of(p.qkv, uint32_t(kFusedQkvPairs * 8));
        const uint32_t row = ct >> 6;
        const uint32_t off = row < G ? (x * G + row) * D : row == G ? QD + x * D : QD + KD + x * D;
        uint2 qa, qb;
        for (uint32_t spins = 0;;) {
          qa = ld_pair(rq, off + lane);
          qb = ld_pair(rq, off + lane + 64);
          if (poll_done(qa.y == tag && qb.y == tag, spins, p.err)) break;
          __builtin_amdgcn_s_sleep(1);
        }
        qraw[row][lane] = __uint_as_float(qa.x);
        qraw[row][lane + 64] = __uint_as_float(qb.x);
      }
      __syncthreads();
      if (attn) {  // the attention's barriers: q/k prepared, two per tile, the partials reduced
        __syncthreads();
        for (uint32_t i = 0; i < ntiles; i++) {
          __syncthreads();
          __syncthreads();
        }
        __syncthreads();
      }
      // ---- merge of the runs (head 2x + ct / 128, dim ct % 128) ----
      // out = sum_s e_s acc_s / sum_s e_s l_s, e_s = exp(m_s - max m); empty runs (m = -inf)
      // and slots past the last run weigh 0. In every exchange wave lane u takes (m, l) of head
      // u / SM, run u % SM, so the weights come from lane shuffles and a thread holds only its
      // acc values.
      if (oproj) {
        const __amdgpu_buffer_rsrc_t rp = rsrc_of(p.attn_part + size_t(x) * kFusedMaxRuns * G * kPartStride,
                                                  uint32_t(kFusedMaxRuns * G * kPartStride * 8));
        const uint32_t j = ct >> 7, d = ct & 127;  // j is wave-uniform
        const uint32_t jh = min(lane / SM, G - 1), uu = lane % SM;
        const bool live = lane < G * SM && uu < splits;
        uint4 ml;  // pairs m, l
        uint2 av[SM];
        await<4>([&] { return ld_pair(rp, ((splits - 1) * G + j) * kPartStride + 4 + d).y == tag; }, p.err);
        for (uint32_t spins = 0;;) {
          ml = ld_pair2(rp, (min(uu, splits - 1) * G + jh) * kPartStride);
          bool ok = !live || (ml.y == tag && ml.w == tag);
#pragma unroll
          for (int u = 0; u < SM; u++) {
            av[u] = ld_pair(rp, (min(uint32_t(u), splits - 1) * G + j) * kPartStride + 4 + d);
            ok = ok && av[u].y == tag;
          }
          if (poll_done(ok, spins, p.err)) break;
        }
        const float m = live ? __uint_as_float(ml.x) : -INFINITY;
        float M = m;
#pragma unroll
        for (int o = 1; o < SM; o <<= 1) M = fmaxf(M, __shfl_xor(M, o));
        const float e = m != -INFINITY ? expf(m - M) : 0.f;
        float L = e * (live ? __uint_as_float(ml.z) : 0.f);
#pragma unroll
        for (int o = 1; o < SM; o <<= 1) L += __shfl_xor(L, o);
        float Av = 0.f;
#pragma unroll
        for (int u = 0; u < SM; u++) Av += __shfl(e, int(j * SM + u)) * __uint_as_float(av[u].x);
        att[ct] = Av * (1.0f / __shfl(L, int(j * SM)));
      }
      __syncthreads();
      // x' = x + the 8 XCDs' o_proj partials, gathered into xs
      reduce_gather(p.part_a, p.xa, tag, true);
      __syncthreads();
      // this XCD's h values (waves 4-6; wave 7 has nothing to poll)
      if (ct < I / NX / 2) {
        const __amdgpu_buffer_rsrc_t rh = rsrc_of(p.h + (I / NX) * x, (I / NX) * 8);
        uint4 hv;
        for (uint32_t spins = 0;;) {
          hv = ld_pair2(rh, 2 * ct);
          if (poll_done(hv.y == tag && hv.w == tag, spins, p.err)) break;
          __builtin_amdgcn_s_sleep(1);
        }
        hs[2 * ct] = __uint_as_float(hv.x);
        hs[2 * ct + 1] = __uint_as_float(hv.z);
      }
      __syncthreads();
      // x = x' + the 8 XCDs' down partials (gathered unless this was the last layer)
      reduce_gather(p.part_m, p.xm, tag, l + 1 < p.n_layers);
      __syncthreads();
    }

    // the last layer's output (every XCD holds the same values; XCD s % 8 writes slot s's columns)
    if (wave == 4 && lane < 32 && s % NX == x) p.x_out[32 * s + lane] = r;
    // workgroup 0's last reduction needed every XCD's slot 0 down rows, which needed every
    // workgroup's h values: all of them have read the generation word
    if (blockIdx.x == 0 && wave == 4 && lane == 0)
      __hip_atomic_store(p.gen, (tb >> 5), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <bool KV_BF16>
hipError_t launch_persist_kv(const PersistParams& p, hipStream_t s) {
  const dim3 grid(NX * NS), block(512);
  if (p.splits <= 4) hipLaunchKernelGGL((k_decode_persist<KV_BF16, 4, false>), grid, block, 0, s, p);
  else if (p.splits <= 8) hipLaunchKernelGGL((k_decode_persist<KV_BF16, 8, false>), grid, block, 0, s, p);
  else if (p.splits <= 16) hipLaunchKernelGGL((k_decode_persist<KV_BF16, 16, false>), grid, block, 0, s, p);
  else if (p.run == 64) hipLaunchKernelGGL((k_decode_persist<KV_BF16, 32, false>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((k_decode_persist<KV_BF16, 32, true>), grid, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_persist(const PersistParams& p, hipStream_t s) {
  if (!p.w_in || !p.w_qkv || !p.q_norm || !p.k_norm || !p.w_o || !p.w_post || !p.w_gu || !p.w_down ||
      !p.embed || !p.tokens || !p.vocab || !p.state || !p.k_cache || !p.v_cache || !p.rope_cur || !p.x_out ||
      !p.qkv || !p.attn_part || !p.h || !p.xa || !p.xm || !p.part_a || !p.part_m || !p.gen || !p.err ||
      p.n_layers == 0 || p.n_layers > 32 || p.max_seq == 0 || p.max_seq > (1u << 22) || p.splits == 0 ||
      p.splits > kFusedMaxRuns ||
      (p.splits > 16 && p.splits != kFusedMaxRuns) || (p.splits <= 16 && p.run != 64) || p.run == 0 || p.run % 64)
    return hipErrorInvalidValue;
  return p.kv_bf16 ? launch_persist_kv<true>(p, s) : launch_persist_kv<false>(p, s);
}

}  // namespace qe
