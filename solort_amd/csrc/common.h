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

// DPP lane moves inside a 16-lane row (VALU, no LDS round trip).
//   0xB1 quad_perm [1,0,3,2]: lane i reads lane i^1
//   0x4E quad_perm [2,3,0,1]: lane i reads lane i^2
//   0x141 row_half_mirror:    lane i reads lane 7-i (within 8)
//   0x140 row_mirror:         lane i reads lane 15-i
//   0x128 row_ror:8:          lane i reads lane (i+8)%16 = i^8
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a row, the same value in every lane: pairwise
// over lane distance 1, then 2, then 4 (half mirror), then 8 (mirror), i.e.
// an xor butterfly with offsets 1, 2, 4, 8.
__device__ __forceinline__ float row16_sum(float v) {
  v = v + dpp<0xB1>(v);
  v = v + dpp<0x4E>(v);
  v = v + dpp<0x141>(v);
  v = v + dpp<0x140>(v);
  return v;
}

// The value held by lane i^8 of the same 16-lane row.
__device__ __forceinline__ float row16_swap8(float v) { return dpp<0x128>(v); }

// Maximum / sum over all 64 lanes of a wavefront, the same value in every lane.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, xshfl(v, 16));
  return fmaxf(v, xshfl(v, 32));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v = v + xshfl(v, 16);
  return v + xshfl(v, 32);
}

// RoPE angle, cos and sin of the reference's _cos_sin
// (src/solort/model/cuda_graph_executor.py:95-98): the fp32 product
// float(pos) * inv_freq, then the device library's fp32 cosf/sinf rounded to
// bf16.  Every kernel that applies RoPE evaluates them through these helpers,
// and the table kernel (rope.hip) does too; a test checks that table against
// torch's for every position served.
__device__ __forceinline__ float rope_angle(int64_t pos, float inv_f) { return (float)pos * inv_f; }
__device__ __forceinline__ float rope_cos(float ang) { return rbf(cosf(ang)); }
__device__ __forceinline__ float rope_sin(float ang) { return rbf(sinf(ang)); }

// cos/sin of position `pos` for 8 consecutive frequencies inv_freq8[0..7].
__device__ __forceinline__ void rope_cs8(int64_t pos, const float* inv_freq8, float* c, float* s) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float ang = rope_angle(pos, inv_freq8[i]);
    c[i] = rope_cos(ang);
    s[i] = rope_sin(ang);
  }
}

// Device-scope (agent) fences used by the last-workgroup-combines pattern.
__device__ __forceinline__ void fence_release_agent() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
__device__ __forceinline__ void fence_acquire_agent() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace solort
