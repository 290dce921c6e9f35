// Per-row QK-RMSNorm + RoPE on one 16-lane group, shared by the standalone
// prologue kernel and the fused decode kernel so both write identical bits.
//
// Follows src/solort/model/cuda_graph_executor.py:
//   _rmsnorm :25-28   y = bf16( (fp32(x) * rsqrt(mean(x^2) + eps)) * fp32(w) )
//   _rope    :100-102 out = bf16( bf16(y * cos) + bf16(rotate_half(y) * sin) )
// Lane j of the group holds dims [8j, 8j+8).  The 128-term sum of squares
// (an order torch leaves unspecified) is fixed: each lane adds its 8 squares
// left to right, then the 16 lane sums meet in an xor butterfly over lane
// distances 1, 2, 4, 8 (row16_sum).  Squares of bf16 values are exact in fp32, so fused
// multiply-adds cannot change the sum.  1/sqrt uses the correctly rounded
// fp32 sqrt and divide.  All 16 lanes of the group must be active.
#pragma once
#include "common.h"

namespace solort {

// raw: this lane's 8 bf16 of the row; w8: this lane's 8 weights (bf16 bits);
// c/s: this lane's 8 cos/sin values (bf16 values as fp32) for frequencies
// 8(j%8)..+7, from rope_cs8.
__device__ __forceinline__ uint4 qknorm_rope_row(const uint4 raw, const uint4 w8, const float* c,
                                                 const float* s, float eps, int j) {
#pragma clang fp contract(off)
  float x[8];
  unpack8(raw, x);
  float ss = x[0] * x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) ss = ss + x[i] * x[i];
  ss = row16_sum(ss);
  const float mean = ss * (1.0f / 128.0f);  // exact: power-of-two scale
  const float r = 1.0f / __builtin_sqrtf(mean + eps);
  float wf[8], y[8], yp[8], o[8];
  unpack8(w8, wf);
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = rbf((x[i] * r) * wf[i]);
  // rotate_half partner: dim d pairs with d +- 64, held by lane j ^ 8.
#pragma unroll
  for (int i = 0; i < 8; ++i) yp[i] = row16_swap8(y[i]);
  const bool lo = j < 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = rbf(y[i] * c[i]);
    const float rot = lo ? -yp[i] : yp[i];
    const float b = rbf(rot * s[i]);
    o[i] = a + b;  // rounded to bf16 by pack8
  }
  return pack8(o);
}

}  // namespace solort
