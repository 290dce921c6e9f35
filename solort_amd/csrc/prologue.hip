// Per-head QK-RMSNorm + RoPE prologue with the in-place KV-cache write.
//
// Follows src/solort/model/cuda_graph_executor.py:
//   _rmsnorm :25-28   y = bf16( (fp32(x) * rsqrt(mean(x^2) + eps)) * fp32(w) )
//   _rope    :100-102 out = bf16( bf16(y * cos) + bf16(rotate_half(y) * sin) )
//   KV write :122-123 (prefill), :178-179 (decode), :259-260 (verify)
//
// Mapping: one 16-lane group per (token, head) row of the fused qkv output;
// lane j of the group holds dims [8j, 8j+8) as one 16-byte vector.  Rows are
// the nh q heads, then nkv k heads (normed + roped, written to k_cache), then
// nkv v heads (copied raw to v_cache).
//
// Bit-exactness: every rounding the reference performs is reproduced in the
// same order.  The one step the reference leaves unspecified, the order of
// the 128-term sum of squares, is fixed here: each lane adds its 8 squares
// left to right, then the 16 lane sums are combined with an xor butterfly
// over lane distances 8, 4, 2, 1.  (Squares of bf16 values are exact in fp32,
// so fused multiply-adds cannot change the result.)  1/sqrt is computed with
// the correctly rounded fp32 sqrt and divide.
#include "common.h"
#include "capi_internal.h"

namespace solort {

#pragma clang fp contract(off)

__global__ __launch_bounds__(256) void qknorm_rope_kvwrite_kernel(
    const uint16_t* __restrict__ qkv, int64_t qkv_stride, int T, int nh, int nkv,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w, float eps,
    const uint16_t* __restrict__ cos_tab, const uint16_t* __restrict__ sin_tab, int64_t pos_limit,
    const int64_t* __restrict__ pos0_dev, uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int64_t tok_stride, int64_t head_stride) {
  const int j = threadIdx.x & 15;
  const int heads = nh + 2 * nkv;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (row >= (int64_t)T * heads) return;  // whole 16-lane groups retire together
  const int t = (int)(row / heads);
  const int hs = (int)(row % heads);
  const int64_t pos = (pos0_dev ? pos0_dev[0] : 0) + t;
  const bool pos_ok = pos >= 0 && pos < pos_limit;

  const uint4 raw = *reinterpret_cast<const uint4*>(qkv + (int64_t)t * qkv_stride + hs * SOLORT_HD + j * 8);
  if (hs >= nh + nkv) {  // V rows: raw copy (V is neither normed nor roped)
    if (pos_ok)
      *reinterpret_cast<uint4*>(vc + pos * tok_stride + (int64_t)(hs - nh - nkv) * head_stride + j * 8) = raw;
    return;
  }

  float x[8];
  unpack8(raw, x);
  float ss = x[0] * x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) ss = ss + x[i] * x[i];
  ss = ss + xshfl(ss, 8);
  ss = ss + xshfl(ss, 4);
  ss = ss + xshfl(ss, 2);
  ss = ss + xshfl(ss, 1);
  const float mean = ss * (1.0f / 128.0f);  // exact: power-of-two scale
  const float r = 1.0f / __builtin_sqrtf(mean + eps);

  const uint16_t* w = (hs < nh) ? qn_w : kn_w;
  float wf[8];
  unpack8(*reinterpret_cast<const uint4*>(w + j * 8), wf);
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = rbf((x[i] * r) * wf[i]);

  // rotate_half partner: dim d pairs with d +- 64, held by lane j ^ 8.
  float yp[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) yp[i] = xshfl(y[i], 8);

  const int64_t prow = pos_ok ? pos : 0;  // nothing reaches the cache when !pos_ok
  float c[8], s[8];
  unpack8(*reinterpret_cast<const uint4*>(cos_tab + prow * 64 + (j & 7) * 8), c);
  unpack8(*reinterpret_cast<const uint4*>(sin_tab + prow * 64 + (j & 7) * 8), s);
  const bool lo = j < 8;
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = rbf(y[i] * c[i]);
    const float rot = lo ? -yp[i] : yp[i];
    const float b = rbf(rot * s[i]);
    o[i] = a + b;  // rounded to bf16 by pack8
  }
  const uint4 ov = pack8(o);
  if (hs < nh) {
    *reinterpret_cast<uint4*>(q_out + ((int64_t)t * nh + hs) * SOLORT_HD + j * 8) = ov;
  } else if (pos_ok) {
    *reinterpret_cast<uint4*>(kc + pos * tok_stride + (int64_t)(hs - nh) * head_stride + j * 8) = ov;
  }
}

}  // namespace solort

using namespace solort;

extern "C" int solort_qknorm_rope_kvwrite(const void* qkv, int64_t qkv_row_stride, int T, int nh,
                                          int nkv, int hd, const void* qn_w, const void* kn_w,
                                          float eps, const void* cos_tab, const void* sin_tab,
                                          int64_t tab_rows, const int64_t* pos0_dev, void* q_out,
                                          void* k_cache, void* v_cache, int64_t kv_tok_stride,
                                          int64_t kv_head_stride, int64_t max_len,
                                          solort_stream_t stream) {
  if (hd != SOLORT_HD) return set_error(SOLORT_EINVAL, "qknorm_rope_kvwrite: head_dim %d != 128", hd);
  if (T < 0 || nh <= 0 || nkv <= 0 || nh % nkv != 0)
    return set_error(SOLORT_EINVAL, "qknorm_rope_kvwrite: bad shape T=%d nh=%d nkv=%d", T, nh, nkv);
  if (!qkv || !qn_w || !kn_w || !cos_tab || !sin_tab || !q_out || !k_cache || !v_cache)
    return set_error(SOLORT_EINVAL, "qknorm_rope_kvwrite: null pointer");
  if (!aligned16(qkv) || !aligned16(qn_w) || !aligned16(kn_w) || !aligned16(cos_tab) ||
      !aligned16(sin_tab) || !aligned16(q_out) || !aligned16(k_cache) || !aligned16(v_cache))
    return set_error(SOLORT_EINVAL, "qknorm_rope_kvwrite: pointers must be 16-byte aligned");
  if (qkv_row_stride < (int64_t)(nh + 2 * nkv) * hd || qkv_row_stride % 8 != 0)
    return set_error(SOLORT_EINVAL, "qknorm_rope_kvwrite: qkv_row_stride %lld", (long long)qkv_row_stride);
  if (kv_tok_stride % 8 != 0 || kv_head_stride % 8 != 0 || kv_tok_stride <= 0 || kv_head_stride <= 0)
    return set_error(SOLORT_EINVAL, "qknorm_rope_kvwrite: KV strides must be positive multiples of 8");
  if (max_len <= 0 || tab_rows <= 0)
    return set_error(SOLORT_EINVAL, "qknorm_rope_kvwrite: max_len and tab_rows must be positive");
  if (T == 0) return 0;
  const int64_t rows = (int64_t)T * (nh + 2 * nkv);
  const int64_t blocks = (rows + 15) / 16;
  if (blocks > 0x7fffffff) return set_error(SOLORT_EINVAL, "qknorm_rope_kvwrite: too many rows");
  const int64_t pos_limit = max_len < tab_rows ? max_len : tab_rows;
  hipLaunchKernelGGL(qknorm_rope_kvwrite_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)qkv, qkv_row_stride, T, nh, nkv,
                     (const uint16_t*)qn_w, (const uint16_t*)kn_w, eps, (const uint16_t*)cos_tab,
                     (const uint16_t*)sin_tab, pos_limit, pos0_dev, (uint16_t*)q_out,
                     (uint16_t*)k_cache, (uint16_t*)v_cache, kv_tok_stride, kv_head_stride);
  return check_launch("qknorm_rope_kvwrite");
}
