// Device helpers shared by the decode kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

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

// As dpp(), but lanes the control does not write keep -inf (the identity of max).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_ninf(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(int(0xFF800000u), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Max over the 64 lanes of a wave, returned to every lane (same lane pattern as wave_sum).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_ninf<0xB1>(v));
  v = fmaxf(v, dpp_ninf<0x4E>(v));
  v = fmaxf(v, dpp_ninf<0x141>(v));
  v = fmaxf(v, dpp_ninf<0x140>(v));
  v = fmaxf(v, dpp_ninf<0x142, 0xA>(v));
  v = fmaxf(v, dpp_ninf<0x143, 0xC>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
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

// Sum over each aligned group of 8 lanes, returned to the 8 lanes of the group
// (quad xor1, quad xor2, half-row mirror).
__device__ __forceinline__ float sum8(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v;
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

// A 16-byte load with the non-temporal hint (`nt`): on gfx950 the line is not allocated in the
// memory-side cache (MALL), which lets a stream that is read once per step run faster (a 1 GiB
// stream: 6.8 vs 6.1 TB/s) and leaves the MALL's contents alone. Only for data no later launch
// expects in a cache: an nt line does not stay in L2 either.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__host__ __device__ __forceinline__ uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

}  // namespace
}  // namespace qe
