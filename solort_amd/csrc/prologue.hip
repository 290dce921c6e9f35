// Per-head QK-RMSNorm + RoPE prologue with the in-place KV-cache write, for
// T tokens at positions pos0..pos0+T-1 (decode T=1, verify T=K+1, prefill T).
//
// Follows src/solort/model/cuda_graph_executor.py: _rmsnorm :25-28, _rope
// :100-102, KV write :122-123 (prefill), :178-179 (decode), :259-260 (verify).
// The row arithmetic (and its fixed summation order) lives in qknorm_rope.h,
// shared with the fused decode kernel.
//
// Mapping: one block per token; one 16-lane group per (token, head) row of
// the fused qkv output, lane j holding dims [8j, 8j+8) as one 16-byte vector.
// Rows are the nh q heads, then nkv k heads (normed + roped, written to
// k_cache), then nkv v heads (copied raw to v_cache).  The token's cos/sin
// come either from a table of the step's rows (rope_rows_kernel, the values
// the reference computes once per forward, :111, :164, :248) or are
// evaluated once per block into LDS from inv_freq.
#include "common.h"
#include "capi_internal.h"
#include "qknorm_rope.h"

namespace solort {

// rope_src: TABLE, the step's cos/sin rows rope_cs [2][T][64] bf16; else
// inv_freq [64] fp32.  The arguments the first loads need lead (qkv ..
// rope_src: 14 dwords), so they arrive preloaded in SGPRs.
template <bool TABLE>
__global__ __launch_bounds__(256) void qknorm_rope_kvwrite_kernel(
    const uint16_t* __restrict__ qkv, int64_t qkv_stride, int T, int nh, int nkv, int row0,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w, const void* __restrict__ rope_src,
    float eps, int64_t pos_limit, const int64_t* __restrict__ pos0_dev, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t tok_stride, int64_t head_stride) {
  // Block = one token; the 16 slots of 16 lanes take its head rows row0 ..
  // (row0 = nh: the K and V rows only, q_out unused).
  const int tid = threadIdx.x, j = tid & 15, slot = tid >> 4;
  const int t = blockIdx.x;
  const int heads = nh + 2 * nkv;
  // This slot's rows hs = slot + 16 p, all loaded before any is computed (a
  // load issued after the previous row's math would add a memory latency per
  // row); past the last row the loads re-read it and are not used.  These
  // loads (and, TABLE, the cos/sin rows) need only preloaded arguments and go
  // out before the position, which the writes need, is read.
  constexpr int kMaxPass = 6;  // heads <= 96
  uint4 cs_raw{}, sn_raw{};
  if constexpr (TABLE) {  // rope_cs [2][T][64]: this lane's 8 cos then sin values of row t
    const uint16_t* rope_cs = reinterpret_cast<const uint16_t*>(rope_src);
    cs_raw = *reinterpret_cast<const uint4*>(rope_cs + (int64_t)t * 64 + (j & 7) * 8);
    sn_raw = *reinterpret_cast<const uint4*>(rope_cs + ((int64_t)T + t) * 64 + (j & 7) * 8);
  }
  const uint4 wq = *reinterpret_cast<const uint4*>(qn_w + j * 8), wk = *reinterpret_cast<const uint4*>(kn_w + j * 8);
  uint4 raws[kMaxPass];
#pragma unroll
  for (int p = 0; p < kMaxPass; ++p)
    raws[p] = *reinterpret_cast<const uint4*>(qkv + (int64_t)t * qkv_stride +
                                              min(row0 + slot + 16 * p, heads - 1) * SOLORT_HD + j * 8);
  __builtin_amdgcn_sched_barrier(0);

  const int64_t pos = (pos0_dev ? pos0_dev[0] : 0) + t;
  const bool pos_ok = pos >= 0 && pos < pos_limit;
  float c[8], s[8];
  if constexpr (TABLE) {
    unpack8(cs_raw, c);
    unpack8(sn_raw, s);
  } else {  // the token's 128 cos/sin values, one per thread, through LDS
    __shared__ float s_cs[64], s_sn[64];
    if (tid < 128) {
      const float ang = rope_angle(pos, reinterpret_cast<const float*>(rope_src)[tid >> 1]);
      if (tid & 1) s_sn[tid >> 1] = rope_sin(ang);
      else s_cs[tid >> 1] = rope_cos(ang);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      c[i] = s_cs[(j & 7) * 8 + i];
      s[i] = s_sn[(j & 7) * 8 + i];
    }
  }
#pragma unroll
  for (int p = 0; p < kMaxPass; ++p) {  // whole 16-lane groups take a row
    const int hs = row0 + slot + 16 * p;
    if (hs >= heads) break;
    const uint4 raw = raws[p];
    if (hs >= nh + nkv) {  // V rows: raw copy (V is neither normed nor roped)
      if (pos_ok)
        *reinterpret_cast<uint4*>(vc + pos * tok_stride + (int64_t)(hs - nh - nkv) * head_stride + j * 8) = raw;
      continue;
    }
    const uint4 ov = qknorm_rope_row(raw, hs < nh ? wq : wk, c, s, eps, j);
    if (hs < nh) {
      *reinterpret_cast<uint4*>(q_out + ((int64_t)t * nh + hs) * SOLORT_HD + j * 8) = ov;
    } else if (pos_ok) {
      *reinterpret_cast<uint4*>(kc + pos * tok_stride + (int64_t)(hs - nh) * head_stride + j * 8) = ov;
    }
  }
}

}  // namespace solort

using namespace solort;

// Checks shared by the prologue entry points and solort_prefill_layer.
int solort::check_prologue(const char* name, const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv, int hd,
                          const void* qn_w, const void* kn_w, const void* rope_src, const void* q_out,
                          const void* k_cache, const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                          int64_t max_len) {
  if (hd != SOLORT_HD) return set_error(SOLORT_EINVAL, "%s: head_dim %d != 128", name, hd);
  if (T < 0 || nh <= 0 || nkv <= 0 || nh % nkv != 0)
    return set_error(SOLORT_EINVAL, "%s: bad shape T=%d nh=%d nkv=%d", name, T, nh, nkv);
  if (!qkv || !qn_w || !kn_w || !rope_src || !q_out || !k_cache || !v_cache)
    return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(qkv) || !aligned16(qn_w) || !aligned16(kn_w) || !aligned16(rope_src) || !aligned16(q_out) ||
      !aligned16(k_cache) || !aligned16(v_cache))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (qkv_row_stride < (int64_t)(nh + 2 * nkv) * hd || qkv_row_stride % 8 != 0)
    return set_error(SOLORT_EINVAL, "%s: qkv_row_stride %lld", name, (long long)qkv_row_stride);
  if (kv_tok_stride % 8 != 0 || kv_head_stride % 8 != 0 || kv_tok_stride <= 0 || kv_head_stride <= 0)
    return set_error(SOLORT_EINVAL, "%s: KV strides must be positive multiples of 8", name);
  if (max_len <= 0) return set_error(SOLORT_EINVAL, "%s: max_len must be positive", name);
  if (nh + 2 * nkv > 96) return set_error(SOLORT_EINVAL, "%s: %d head rows exceed 96", name, nh + 2 * nkv);
  return 0;
}

extern "C" int solort_qknorm_rope_kvwrite(const void* qkv, int64_t qkv_row_stride, int T, int nh,
                                          int nkv, int hd, const void* qn_w, const void* kn_w,
                                          float eps, const float* inv_freq, const int64_t* pos0_dev,
                                          void* q_out, void* k_cache, void* v_cache, int64_t kv_tok_stride,
                                          int64_t kv_head_stride, int64_t max_len, solort_stream_t stream) {
  int rc = check_prologue("qknorm_rope_kvwrite", qkv, qkv_row_stride, T, nh, nkv, hd, qn_w, kn_w, inv_freq, q_out,
                          k_cache, v_cache, kv_tok_stride, kv_head_stride, max_len);
  if (rc || T == 0) return rc;
  hipLaunchKernelGGL(qknorm_rope_kvwrite_kernel<false>, dim3((unsigned)T), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, qkv_row_stride, T, nh, nkv, 0, (const uint16_t*)qn_w,
                     (const uint16_t*)kn_w, (const void*)inv_freq, eps, max_len, pos0_dev, (uint16_t*)q_out,
                     (uint16_t*)k_cache, (uint16_t*)v_cache, kv_tok_stride, kv_head_stride);
  return check_launch("qknorm_rope_kvwrite");
}

extern "C" int solort_qknorm_rope_kvwrite_cs(const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv,
                                             int hd, const void* qn_w, const void* kn_w, float eps,
                                             const void* rope_cs, const int64_t* pos0_dev, void* q_out,
                                             void* k_cache, void* v_cache, int64_t kv_tok_stride,
                                             int64_t kv_head_stride, int64_t max_len, solort_stream_t stream) {
  int rc = check_prologue("qknorm_rope_kvwrite_cs", qkv, qkv_row_stride, T, nh, nkv, hd, qn_w, kn_w, rope_cs,
                          q_out, k_cache, v_cache, kv_tok_stride, kv_head_stride, max_len);
  if (rc || T == 0) return rc;
  hipLaunchKernelGGL(qknorm_rope_kvwrite_kernel<true>, dim3((unsigned)T), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, qkv_row_stride, T, nh, nkv, 0, (const uint16_t*)qn_w,
                     (const uint16_t*)kn_w, rope_cs, eps, max_len, pos0_dev, (uint16_t*)q_out, (uint16_t*)k_cache,
                     (uint16_t*)v_cache, kv_tok_stride, kv_head_stride);
  return check_launch("qknorm_rope_kvwrite_cs");
}

// The K and V rows of T tokens at positions 0..T-1 (the prefill layer's
// prologue; its q rows are normalised inside the attention kernel).  The
// caller has validated the arguments as for solort_qknorm_rope_kvwrite_cs.
int solort::launch_kv_rows_cs(const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv, const void* kn_w,
                              float eps, const void* rope_cs, void* k_cache, void* v_cache, int64_t kv_tok_stride,
                              int64_t kv_head_stride, int64_t max_len, hipStream_t stream) {
  hipLaunchKernelGGL(qknorm_rope_kvwrite_kernel<true>, dim3((unsigned)T), dim3(256), 0, stream, (const uint16_t*)qkv,
                     qkv_row_stride, T, nh, nkv, nh, (const uint16_t*)kn_w, (const uint16_t*)kn_w, rope_cs, eps,
                     max_len, (const int64_t*)nullptr, (uint16_t*)nullptr, (uint16_t*)k_cache, (uint16_t*)v_cache,
                     kv_tok_stride, kv_head_stride);
  return check_launch("prefill_layer (K/V rows)");
}
