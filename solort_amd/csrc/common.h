// Shared device helpers for the gfx950 attention kernels.
//
// bf16 is carried as raw uint16_t bits so that every rounding step is explicit
// and matches torch's c10::BFloat16 (round-to-nearest-even).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SOLORT_HD 128          // head_dim of every Qwen3 shape this library serves
#define SOLORT_LANES_PER_ROW 16  // 16 lanes x 8 bf16 (16 bytes) cover one 128-dim row

namespace solort {

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// float -> bf16 bits, round to nearest even, by gfx950's v_cvt_pk_bf16_f32.
// For every non-NaN input this is bit-identical to torch's c10::BFloat16
// rounding (checked over all 2^32 fp32 patterns, denormals and infinities
// included); a NaN stays a NaN.
__device__ __forceinline__ uint32_t f2bf(float f) { return __builtin_bit_cast(unsigned short, (__bf16)f); }

// Two values, one instruction: bits of bf16(lo) | bf16(hi) << 16.
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
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
  v.x = pack2(x[0], x[1]);
  v.y = pack2(x[2], x[3]);
  v.z = pack2(x[4], x[5]);
  v.w = pack2(x[6], x[7]);
  return v;
}

// fp32 dot product of two bf16 pairs plus an accumulator (v_dot2c_f32_bf16);
// the bf16 products are exact in fp32.
__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
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

// Reduce-scatter over a 16-lane row: each of v[0..7] is summed over the row's
// 16 lanes, and lane j returns the total of value j >> 1 (lanes j and j ^ 1
// hold the same one).  Each step pairs lanes that differ in one more bit
// (bit 3 via row_ror:8, bit 2 via half mirror, bit 1, then bit 0); the lane
// with that bit set keeps the upper half of its list, its partner the lower
// half, and each adds the half the other hands over.  22 VALU operations
// instead of 32 for eight separate row sums, and the eight totals end in
// different lanes.
__device__ __forceinline__ float row16_reduce8(const float (&v)[8], int j) {
  const bool h3 = j & 8, h2 = j & 4, h1 = j & 2;
  float a[4], b[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = h3 ? v[i + 4] : v[i], give = h3 ? v[i] : v[i + 4];
    a[i] = keep + dpp<0x128>(give);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = h2 ? a[i + 2] : a[i], give = h2 ? a[i] : a[i + 2];
    b[i] = keep + dpp<0x141>(give);
  }
  const float keep = h1 ? b[1] : b[0], give = h1 ? b[0] : b[1];
  const float c = keep + dpp<0x4E>(give);
  return c + dpp<0xB1>(c);
}

// The value of lane i ^ 16 (i ^ 32) combined with this lane's by OP, using
// gfx950's row-swap instructions: after swapping rows, each lane holds its own
// value in one result and its partner's in the other.  (The elements are read
// with __uint_as_float: __builtin_bit_cast of a vector element reads element 0.)
template <typename OP>
__device__ __forceinline__ float xor16_combine(float v, OP op) {
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return op(__uint_as_float(r0), __uint_as_float(r1));
}
template <typename OP>
__device__ __forceinline__ float xor32_combine(float v, OP op) {
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return op(__uint_as_float(r0), __uint_as_float(r1));
}

// Maximum / sum over all 64 lanes of a wavefront, the same value in every lane.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = xor16_combine(v, [](float x, float y) { return fmaxf(x, y); });
  return xor32_combine(v, [](float x, float y) { return fmaxf(x, y); });
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v = xor16_combine(v, [](float x, float y) { return x + y; });
  return xor32_combine(v, [](float x, float y) { return x + y; });
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

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also waits
// for every global load the wave has in flight, which would stall a kernel
// that issues its HBM loads early and synchronises on LDS before using them.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Phase stamps (tracing build only).  A library built with SOLORT_PHASE_STAMPS
// (python -m solort_amd.build --stamps, a separate .so) records, per workgroup
// of the most recent launch of each instrumented kernel, the device clock
// (s_memrealtime, 100 MHz) at fixed points of its work, in a per-source
// array read back by solort_phase_stamps_* (declared in
// include/solort_trace.h).  In the normal build SOLORT_STAMP is empty and the
// kernels are unchanged.  SOLORT_STAMP_TU() defines the array once per source
// file; slot i < 16 of linear workgroup b is written by the calling thread.
constexpr int kStampBlocks = 4096;  // workgroups with stamps (later ones are skipped)
constexpr int kStampSlots = 16;
#ifdef SOLORT_PHASE_STAMPS
#define SOLORT_STAMP_TU() __device__ unsigned long long g_phase_stamps[kStampBlocks * kStampSlots]
#define SOLORT_STAMP(cond, b, i)                                                        \
  do {                                                                                 \
    if ((cond) && (b) < kStampBlocks)                                                  \
      g_phase_stamps[(b) * kStampSlots + (i)] = __builtin_amdgcn_s_memrealtime();       \
  } while (0)
#else
#define SOLORT_STAMP_TU() static_assert(true, "")
#define SOLORT_STAMP(cond, b, i) ((void)0)
#endif

// Two fp32 values as tagged 8-byte pairs (value, tag, value, tag): a naturally
// aligned 8-byte store is single-copy atomic, so a reader that finds the tag
// it expects in a pair also holds that pair's value.  Workgroups of one launch
// hand partial results to each other this way without fences or atomics.
__device__ __forceinline__ uint4 tagged2(float x, float y, unsigned tag) {
  return make_uint4(__float_as_uint(x), tag, __float_as_uint(y), tag);
}

// A load of data streamed once (weights, K/V rows) with the non-temporal
// hint (`nt`): measured on MI355X, it speeds up the decode K/V streams and the
// large weight streams (the hint keeps them from displacing cached data).
__device__ __forceinline__ uint4 ld_stream(const void* p) {
  typedef unsigned u32x4s __attribute__((ext_vector_type(4)));
  const u32x4s v = __builtin_nontemporal_load(reinterpret_cast<const u32x4s*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Stores with the non-temporal hint: the split partials of the two-launch
// combine, read once by the next launch (5-token verify 10.44 -> 10.36 us per
// call in one same-box A/B).
__device__ __forceinline__ void st_stream(float4* p, float4 v) {
  typedef float f32x4s __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(f32x4s{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4s*>(p));
}
__device__ __forceinline__ void st_stream(float2* p, float2 v) {
  typedef float f32x2s __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store(f32x2s{v.x, v.y}, reinterpret_cast<f32x2s*>(p));
}

// Device-scope 16-byte load (cache policy sc1): misses the CU's L1, reads the XCD's L2.
__device__ __forceinline__ uint4 ld_l2(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
}

// Small uniform values read with vector (buffer) loads: they complete in
// order with the vector loads issued before them (vmcnt), so an LDS wait
// (lgkmcnt), which a scalar load would share, never waits for them.
__device__ __forceinline__ uint2 ld_vec8(const void* p) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 8, 0x00020000);
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, 0, 0, 0));
}
__device__ __forceinline__ unsigned ld_vec4(const void* p) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 4, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 0);
}

// Greedy-argmax key of (value, index): high word = an order-preserving image
// of the fp32 value (-0 and +0 equal, NaN above every number), low word =
// 0xffffffff - index, so the integer maximum is torch.argmax's answer (the
// lowest index among equal maxima, the first NaN if there is one).
__device__ __forceinline__ uint64_t argmax_key(float f, int64_t idx) {
  uint32_t u = __float_as_uint(f);
  uint32_t k;
  if ((u & 0x7fffffffu) > 0x7f800000u) k = 0xffffffffu;        // NaN
  else if ((u & 0x7fffffffu) == 0u) k = 0x80000000u;           // +-0
  else k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)k << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Folds a workgroup's best key into the row's slot and lets the last
// workgroup of the grid (atomic ticket) decode the index and clear the slot
// and ticket for the next launch.  Called by one thread per workgroup.
//
// Only atomics carry data between workgroups, so no release/acquire fence is
// needed (on gfx950 an agent-scope fence is an L2 writeback plus invalidate,
// which per workgroup of a 10,000-workgroup grid cost 4x the whole kernel).
// The ticket must not be counted before the max has been performed: it is
// issued with an operand computed from the max's returned value, so it waits
// for that return.  The last workgroup reads the slot with an atomic
// read-modify-write, after its ticket returned.
__device__ __forceinline__ void argmax_fold(uint64_t best, uint64_t* slot, unsigned* ticket, unsigned nblocks,
                                            int64_t* out) {
  const uint64_t prev = __hip_atomic_fetch_max(slot, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned zero;
  asm volatile("v_and_b32 %0, 0, %1" : "=v"(zero) : "v"((uint32_t)prev));
  if (__hip_atomic_fetch_add(ticket, 1u + zero, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nblocks - 1) {
    const uint64_t k = __hip_atomic_fetch_max(slot, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *out = (int64_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
    __hip_atomic_store(slot, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace solort
