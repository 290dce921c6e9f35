// Pieces of the decode-step matrix-vector product that the GEMV kernels and
// the fused qkv + attention kernel share, so both give the same bits: the
// staging of x in LDS (optionally RMS-normalised) and the wavefront sum.
#pragma once

#include "common.h"

namespace solort {

__device__ __forceinline__ float wave_sum64(float v) {
  v += xshfl(v, 1);
  v += xshfl(v, 2);
  v += xshfl(v, 4);
  v += xshfl(v, 8);
  v += xshfl(v, 16);
  return xor32_combine(v, [](float x, float y) { return x + y; });
}

// x [K] bf16 into sx as K / 8 chunks of 16 bytes, every thread of a 256-thread
// workgroup taking part; NORM: bf16(fp32(x) * rsqrt(mean(fp32(x)^2) + eps) *
// fp32(norm_w)), the sum of squares in fp32 with one block reduction (s_red: 4
// floats).  In two parts, so that a caller can issue the loads early:
// gemv_x_load reads this thread's first kXReg chunks of x and norm_w (K <= 4096
// in one round; larger K re-reads the rest in gemv_x_finish), gemv_x_finish
// normalises and stores them and ends with a workgroup barrier.  Two chunks
// per thread cover K <= 4096 (every hidden size served here); four held 16
// more VGPRs while the weight rows are in flight (gate_up, 4 rows x 5 chunks
// per lane: 153 VGPRs then, 120 now with uniform row pointers, four
// wavefronts per SIMD instead of three; its time did not change).
constexpr int kXReg = 2;
struct XChunks {
  uint4 x[kXReg], g[kXReg];
};

template <bool NORM>
__device__ __forceinline__ void gemv_x_load(const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w, int K,
                                            XChunks& c) {
  const int tid = threadIdx.x, nch = K >> 3;
  if constexpr (NORM) {
#pragma unroll
    for (int q = 0; q < kXReg; ++q) {
      const int i = tid + 256 * q;
      if (i < nch) {
        c.x[q] = *reinterpret_cast<const uint4*>(x + 8 * i);
        c.g[q] = *reinterpret_cast<const uint4*>(norm_w + 8 * i);
      }
    }
  }
}

template <bool NORM>
__device__ __forceinline__ void gemv_x_finish(const XChunks& c, const uint16_t* __restrict__ x,
                                              const uint16_t* __restrict__ norm_w, float eps, int K, uint4* sx,
                                              float* s_red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = K >> 3;
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < kXReg; ++q) {
      if (tid + 256 * q < nch) {
        float v[8];
        unpack8(c.x[q], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
      }
    }
    for (int i = tid + 256 * kXReg; i < nch; i += 256) {
      float v[8];
      unpack8(*reinterpret_cast<const uint4*>(x + 8 * i), v);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
    }
    ss = wave_sum64(ss);
    if (lane == 0) s_red[wave] = ss;
    __syncthreads();
    const float mean = (s_red[0] + s_red[1] + s_red[2] + s_red[3]) / (float)K;
    const float r = 1.0f / __builtin_sqrtf(mean + eps);
#pragma unroll
    for (int q = 0; q < kXReg; ++q) {
      const int i = tid + 256 * q;
      if (i < nch) {
        float v[8], g[8];
        unpack8(c.x[q], v);
        unpack8(c.g[q], g);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (v[e] * r) * g[e];
        sx[i] = pack8(v);
      }
    }
    for (int i = tid + 256 * kXReg; i < nch; i += 256) {
      float v[8], g[8];
      unpack8(*reinterpret_cast<const uint4*>(x + 8 * i), v);
      unpack8(*reinterpret_cast<const uint4*>(norm_w + 8 * i), g);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (v[e] * r) * g[e];
      sx[i] = pack8(v);
    }
  } else {
    for (int i = tid; i < nch; i += 256) sx[i] = *reinterpret_cast<const uint4*>(x + 8 * i);
  }
  __syncthreads();
}

template <bool NORM>
__device__ __forceinline__ void gemv_stage_x(const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w,
                                             float eps, int K, uint4* sx, float* s_red) {
  XChunks c;
  gemv_x_load<NORM>(x, norm_w, K, c);
  gemv_x_finish<NORM>(c, x, norm_w, eps, K, sx, s_red);
}

}  // namespace solort
