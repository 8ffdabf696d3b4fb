// Exchange between the workgroups of a launch through the L2 of their XCD (fused.hip,
// persist.hip): (value bits, tag) pairs, device-scope (sc1) loads that miss the vector L1, and
// bounded polling.
#pragma once

#include "device_common.h"
#include "kernels.h"
#include "l2_prefetch.h"

namespace qe {
namespace {

constexpr uint32_t kSpinMax = 1u << 16;
constexpr int kSc1 = 16;  // buffer-load cache policy: device scope (sc1), misses the vector L1

// the XCD this workgroup runs on (wave-uniform); an id past the 8 XCDs is an error
__device__ __forceinline__ uint32_t fused_xcd(uint32_t* err) {
  const uint32_t x = xcc_id();
  if (x >= kFusedXcds) {
    if (threadIdx.x == 0) atomicOr(err, kErrPlace);
    return x % kFusedXcds;
  }
  return x;
}

__device__ __forceinline__ uint2 pair(float v, uint32_t tag) { return make_uint2(__float_as_uint(v), tag); }

// L1-bypassing loads of pairs another workgroup of this XCD writes during the launch
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), short(0), int(bytes), 0x00020000);
}
__device__ __forceinline__ uint2 ld_pair(__amdgpu_buffer_rsrc_t r, uint32_t pair_idx) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, int(pair_idx * 8), 0, kSc1));
}
__device__ __forceinline__ uint4 ld_pair2(__amdgpu_buffer_rsrc_t r, uint32_t pair_idx) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, int(pair_idx * 8), 0, kSc1));
}

// Spin bookkeeping of a wave's poll loop: true once every lane's pairs carry the tag, or once the
// wait has run out of spins (kErrSync) or another wait of the step has (checked every 1024
// polls), so a failing step ends within milliseconds.
__device__ __forceinline__ bool poll_done(bool ok, uint32_t& spins, uint32_t* err) {
  if (__all(ok)) return true;
  ++spins;
  if ((spins & 1023) == 0 && (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSync))
    return true;
  if (spins >= kSpinMax) {
    if ((threadIdx.x & 63) == 0) atomicOr(err, kErrSync);
    return true;
  }
  return false;
}

// sum over each aligned group of 16 lanes, returned to all 16
__device__ __forceinline__ float sum16(float v) {
  v = sum8(v);
  v += dpp<0x140>(v);  // row mirror
  return v;
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// a, b (8 columns) times their bf16 gains
__device__ __forceinline__ void scale8(float4& a, float4& b, uint4 g) {
  a.x *= __uint_as_float(g.x << 16);
  a.y *= __uint_as_float(g.x & 0xFFFF0000u);
  a.z *= __uint_as_float(g.y << 16);
  a.w *= __uint_as_float(g.y & 0xFFFF0000u);
  b.x *= __uint_as_float(g.z << 16);
  b.y *= __uint_as_float(g.z & 0xFFFF0000u);
  b.z *= __uint_as_float(g.w << 16);
  b.w *= __uint_as_float(g.w & 0xFFFF0000u);
}

// device-scope 64-bit store: written through to memory, so the L2 of another XCD can see it
__device__ __forceinline__ void st_pair_dev(uint2* p, uint2 v) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), (unsigned long long)v.x | ((unsigned long long)v.y << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// device-scope 64-bit load (sc1)
__device__ __forceinline__ uint2 ld_pair_dev(const uint2* p) {
  const unsigned long long v =
      __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint2(uint32_t(v), uint32_t(v >> 32));
}

}  // namespace
}  // namespace qe
