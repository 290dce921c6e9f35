// Shared device helpers for the gfx950 attention kernels.
//
// bf16 is carried as raw uint16_t bits so that every rounding step is explicit
// and matches torch's c10::BFloat16 (round-to-nearest-even, NaN -> 0x7FC0).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SOLORT_HD 128          // head_dim of every Qwen3 shape this library serves
#define SOLORT_LANES_PER_ROW 16  // 16 lanes x 8 bf16 (16 bytes) cover one 128-dim row

namespace solort {

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// float -> bf16 bits, round to nearest even; NaN becomes the canonical 0x7FC0.
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// bf16 round trip of an fp32 value (the per-op rounding torch applies to bf16 tensors).
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// Unpack 8 bf16 (one 16-byte vector) into fp32.
__device__ __forceinline__ void unpack8(const uint4& v, float* x) {
  x[0] = __uint_as_float(v.x << 16); x[1] = __uint_as_float(v.x & 0xffff0000u);
  x[2] = __uint_as_float(v.y << 16); x[3] = __uint_as_float(v.y & 0xffff0000u);
  x[4] = __uint_as_float(v.z << 16); x[5] = __uint_as_float(v.z & 0xffff0000u);
  x[6] = __uint_as_float(v.w << 16); x[7] = __uint_as_float(v.w & 0xffff0000u);
}

__device__ __forceinline__ uint4 pack8(const float* x) {
  uint4 v;
  v.x = f2bf(x[0]) | (f2bf(x[1]) << 16);
  v.y = f2bf(x[2]) | (f2bf(x[3]) << 16);
  v.z = f2bf(x[4]) | (f2bf(x[5]) << 16);
  v.w = f2bf(x[6]) | (f2bf(x[7]) << 16);
  return v;
}

// Lane exchange within a wavefront (64 lanes); xor masks < 64.
__device__ __forceinline__ float xshfl(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Device-scope (agent) fences used by the last-workgroup-combines pattern.
__device__ __forceinline__ void fence_release_agent() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
__device__ __forceinline__ void fence_acquire_agent() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace solort
