// Device side of the L2 weight prefetch that latency-bound decode launches carry (gfx950: one
// L2 per XCD, workgroup j of a launch runs on XCD j % 8).
#pragma once

#include "device_common.h"
#include "kernels.h"

namespace qe {
namespace {

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}

// Prefetch workgroup q (slot q / 8 of the XCD it runs on; consecutive q land on consecutive
// XCDs) loads the chunks of the consumer workgroups j = x + 8 (slot + slots k) of each target,
// x = this XCD, so they sit in the L2 those workgroups will read. All of a thread's loads are
// issued before any is used; the values only feed a never-taken store.
__device__ __forceinline__ void l2_prefetch(const L2Prefetch (&pf)[kMaxPrefetch], uint32_t ns, uint32_t q,
                                            uint32_t* sink) {
  constexpr int KMAX = 16;
  const uint32_t x = xcc_id(), slot = q / 8, tid = threadIdx.x;
  uint32_t cnt[kMaxPrefetch], tot = 0;
#pragma unroll
  for (int t = 0; t < kMaxPrefetch; t++) {
    const uint32_t j0 = x + 8 * slot;
    cnt[t] = pf[t].w && j0 < pf[t].n_cwg ? ceil_div(pf[t].n_cwg - j0, 8 * ns) : 0;
    tot += cnt[t] * pf[t].cw_chunks;
  }
  if (tot == 0) return;
  uint4 v[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; k++) {
    // chunk i of this workgroup's share: target t, its consumer workgroup jj, chunk c in it
    uint32_t i = min(tid + 256u * k, tot - 1);
    const uint16_t* w = pf[0].w;
    uint32_t cw = pf[0].cw_chunks, nc = pf[0].n_chunks, span = cnt[0] * cw;
#pragma unroll
    for (int t = 1; t < kMaxPrefetch; t++) {
      if (i >= span) {
        i -= span;
        w = pf[t].w;
        cw = pf[t].cw_chunks;
        nc = pf[t].n_chunks;
        span = cnt[t] * cw;
      }
    }
    const uint32_t jj = i / cw, c = i - jj * cw;
    const uint32_t j = x + 8 * (slot + ns * jj);
    v[k] = reinterpret_cast<const uint4*>(w)[min(j * cw + c, nc - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t h = 0;
#pragma unroll
  for (int k = 0; k < KMAX; k++) h ^= v[k].x ^ v[k].w;
  if (ns == 0xFFFFFFFFu && h == 0x5A5A5A5Au) *sink = h;  // never: keeps the loads
}

// For consumers that each read more than one prefetch workgroup loads (a GEMM's column tile j,
// whose row tiles and K splits all run on XCD j % 8): the chunks of consumers j = x, x + 8,
// x + 16, ... of each target (x = this XCD) form one list, and prefetch workgroup q loads piece
// q / 8 of it, 256 x 16 chunks. A launch carries 8 x tile_prefetch_slots() such workgroups at
// consecutive linear ids, so each XCD gets every piece once.
__device__ __forceinline__ void l2_prefetch_tiles(const L2Prefetch (&pf)[kMaxPrefetch], uint32_t q,
                                                  uint32_t* sink) {
  constexpr uint32_t KMAX = 16;
  const uint32_t x = xcc_id(), tid = threadIdx.x;
  uint32_t span[kMaxPrefetch], tot = 0;
#pragma unroll
  for (int t = 0; t < kMaxPrefetch; t++) {
    span[t] = pf[t].w && x < pf[t].n_cwg ? ceil_div(pf[t].n_cwg - x, 8u) * pf[t].cw_chunks : 0;
    tot += span[t];
  }
  const uint32_t base = (q / 8) * 256 * KMAX;
  if (base >= tot) return;
  uint4 v[KMAX];
#pragma unroll
  for (uint32_t k = 0; k < KMAX; k++) {
    uint32_t i = min(base + tid + 256 * k, tot - 1);
    const uint16_t* w = pf[0].w;
    uint32_t cw = pf[0].cw_chunks, nc = pf[0].n_chunks, sp = span[0];
#pragma unroll
    for (int t = 1; t < kMaxPrefetch; t++) {
      if (i >= sp) {
        i -= sp;
        w = pf[t].w;
        cw = pf[t].cw_chunks;
        nc = pf[t].n_chunks;
        sp = span[t];
      }
    }
    const uint32_t jj = i / cw, c = i - jj * cw;
    v[k] = reinterpret_cast<const uint4*>(w)[min((x + 8 * jj) * cw + c, nc - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t h = 0;
#pragma unroll
  for (uint32_t k = 0; k < KMAX; k++) h ^= v[k].x ^ v[k].w;
  if (q == 0xFFFFFFFFu && h == 0x5A5A5A5Au) *sink = h;  // never: keeps the loads
}

}  // namespace
}  // namespace qe
