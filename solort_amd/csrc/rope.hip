// RoPE cos/sin on the device: row p holds bf16(cos(float(p) * inv_freq[i]))
// and bf16(sin(...)) for i < half_dim, i.e. the first half of the reference's
// _cos_sin(p) row (src/solort/model/cuda_graph_executor.py:95-98; the second
// half of that row repeats the first).  inv_freq is the caller's fp32 vector
// (the reference computes it at :64-66).
//   rope_table_kernel: rows 0..rows-1 (a whole table).
//   rope_rows_kernel:  the rows of positions pos0..pos0+n-1, pos0 read on the
//                      device; a decode or verify step computes them once and
//                      every layer's fused kernel loads them, as the reference
//                      computes cos, sin once per step (:164, :248).
// Both evaluate rope_angle/rope_cos/rope_sin (common.h), the functions the
// prefill prologue evaluates in-kernel, so comparing the table with torch's
// checks all RoPE inputs.
#include "common.h"
#include "capi_internal.h"

namespace solort {

__global__ __launch_bounds__(256) void rope_table_kernel(const float* __restrict__ inv_freq, int half_dim,
                                                         int64_t rows, uint16_t* __restrict__ cos_out,
                                                         uint16_t* __restrict__ sin_out) {
  // One thread per group of 8 frequencies of one row (half_dim % 8 == 0).
  const int groups = half_dim / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * groups) return;
  const int64_t p = idx / groups;
  const int f0 = (int)(idx % groups) * 8;
  float fr[8], c[8], s[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) fr[i] = inv_freq[f0 + i];
  rope_cs8(p, fr, c, s);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    cos_out[p * half_dim + f0 + i] = (uint16_t)f2bf(c[i]);
    sin_out[p * half_dim + f0 + i] = (uint16_t)f2bf(s[i]);
  }
}

// One thread per (row, cos|sin, frequency); cs_out = cos [n][half_dim] then sin [n][half_dim].
__global__ __launch_bounds__(256) void rope_rows_kernel(const float* __restrict__ inv_freq, int half_dim,
                                                        const int64_t* __restrict__ pos0_dev, int n,
                                                        uint16_t* __restrict__ cs_out) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= 2 * n * half_dim) return;
  const int f = idx % half_dim, t = (idx / half_dim) % n, sn = idx / (half_dim * n);
  const float ang = rope_angle(pos0_dev[0] + t, inv_freq[f]);
  cs_out[idx] = (uint16_t)f2bf(sn ? rope_sin(ang) : rope_cos(ang));
}

}  // namespace solort

using namespace solort;

extern "C" int solort_rope_rows(const float* inv_freq, int half_dim, const int64_t* pos0_dev, int n, void* cs_out,
                                solort_stream_t stream) {
  if (!inv_freq || !pos0_dev || !cs_out) return set_error(SOLORT_EINVAL, "rope_rows: null pointer");
  if (half_dim < 1 || half_dim > 1024 || n < 1 || n > (1 << 20))
    return set_error(SOLORT_EINVAL, "rope_rows: bad shape half_dim=%d n=%d", half_dim, n);
  const int total = 2 * n * half_dim;
  hipLaunchKernelGGL(rope_rows_kernel, dim3((total + 255) / 256), dim3(256), 0, (hipStream_t)stream, inv_freq,
                     half_dim, pos0_dev, n, (uint16_t*)cs_out);
  return check_launch("rope_rows");
}

extern "C" int solort_rope_table(const float* inv_freq, int half_dim, int64_t rows, void* cos_out,
                                 void* sin_out, solort_stream_t stream) {
  if (!inv_freq || !cos_out || !sin_out) return set_error(SOLORT_EINVAL, "rope_table: null pointer");
  if (half_dim < 8 || half_dim > 1024 || half_dim % 8 || rows < 0 || rows > (1LL << 26))
    return set_error(SOLORT_EINVAL, "rope_table: bad shape half_dim=%d rows=%lld", half_dim, (long long)rows);
  if (rows == 0) return 0;
  const int64_t n = rows * (half_dim / 8);
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     inv_freq, half_dim, rows, (uint16_t*)cos_out, (uint16_t*)sin_out);
  return check_launch("rope_table");
}
