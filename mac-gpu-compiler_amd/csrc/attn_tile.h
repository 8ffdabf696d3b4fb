// K/V tile loads of the decode attention kernels (attention.hip, fused.hip, persist.hip): one tile
// of NT = 64 (or 32) positions of one KV head in the two per-thread layouts the score and P.V
// phases use.
#pragma once

#include "device_common.h"
#include "kernels.h"

namespace qe {
namespace {

template <bool KV_BF16, int NT = 64>
struct KVTile;
template <int NT>
struct KVTile<false, NT> {
  float4 k[NT / 32][4];  // scores layout: NT / 32 positions x 16 dims
  float4 v[NT / 8];      // PV layout: NT / 8 positions x 4 dims
};
template <int NT>
struct KVTile<true, NT> {
  uint4 k[NT / 32][2];
  uint2 v[NT / 8];
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

// K/V rows of positions tile.. of the head at head_base (elements) in this thread's two layouts
// (256 threads): thread (pg = tid / 8, dc = tid % 8) holds positions tile + pg and tile + pg + 32
// over dims [16 dc, 16 dc + 16) of K; thread (dg = tid % 32, pp = tid / 32) holds positions
// tile + 8 pp .. + 7 over dims [4 dg, 4 dg + 4) of V. Rows past the cache end are clamped.
template <bool KV_BF16>
__device__ __forceinline__ void load_tile(KVTile<KV_BF16>& X, const void* k_cache, const void* v_cache,
                                          uint32_t max_seq, size_t head_base, uint32_t tile, int tid) {
  constexpr int D = kHeadDim;
  const uint32_t last = max_seq - 1;
  const int pg = tid >> 3, dc = tid & 7, dg = tid & 31, pp = tid >> 5;
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const size_t row = head_base + size_t(min(tile + uint32_t(pg + 32 * u), last)) * D + 16 * dc;
    if constexpr (KV_BF16) {
      const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(k_cache) + row);
      X.k[u][0] = src[0];
      X.k[u][1] = src[1];
    } else {
      const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(k_cache) + row);
#pragma unroll
      for (int i = 0; i < 4; i++) X.k[u][i] = src[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const size_t row = head_base + size_t(min(tile + uint32_t(8 * pp + i), last)) * D + 4 * dg;
    if constexpr (KV_BF16) {
      X.v[i] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(v_cache) + row);
    } else {
      X.v[i] = *reinterpret_cast<const float4*>(static_cast<const float*>(v_cache) + row);
    }
  }
}

// load_tile through buffer descriptors over one head's K and V regions ([max_seq][D] each, so
// rows past the cache end read as 0 instead of being clamped): two lane offsets, and the rows'
// distances as scalar or immediate offsets. A tile of NT = 32 positions: thread (pg, dc) holds
// position tile + pg of K, thread (dg, pp) positions tile + 4 pp .. + 3 of V.
template <bool KV_BF16, int NT = 64>
__device__ __forceinline__ void load_tile_buf(KVTile<KV_BF16, NT>& X, __amdgpu_buffer_rsrc_t rk,
                                              __amdgpu_buffer_rsrc_t rv, uint32_t tile, int tid) {
  constexpr uint32_t D = kHeadDim, EL = KV_BF16 ? 2 : 4, VP = NT / 8;
  const int pg = tid >> 3, dc = tid & 7, dg = tid & 31, pp = tid >> 5;
  const uint32_t koff = ((tile + pg) * D + 16 * dc) * EL, voff = ((tile + VP * pp) * D + 4 * dg) * EL;
#pragma unroll
  for (int u = 0; u < NT / 32; u++) {
    if constexpr (KV_BF16) {
#pragma unroll
      for (int i = 0; i < 2; i++)
        X.k[u][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, int(koff + 16 * i), int(u * 32 * D * EL), 0));
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++)
        X.k[u][i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, int(koff + 16 * i), int(u * 32 * D * EL), 0));
    }
  }
#pragma unroll
  for (int i = 0; i < int(VP); i++) {
    if constexpr (KV_BF16) {
      X.v[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, int(voff), int(i * D * EL), 0));
    } else {
      X.v[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, int(voff), int(i * D * EL), 0));
    }
  }
}

template <bool KV_BF16, int NT>
__device__ __forceinline__ void tile_k(const KVTile<KV_BF16, NT>& X, int u, float4 (&k4)[4]) {
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

template <bool KV_BF16, int NT>
__device__ __forceinline__ float4 tile_v(const KVTile<KV_BF16, NT>& X, int i) {
  if constexpr (KV_BF16) {
    return bf16x4(X.v[i].x, X.v[i].y);
  } else {
    return X.v[i];
  }
}

}  // namespace
}  // namespace qe
