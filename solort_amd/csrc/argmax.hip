// Greedy argmax over rows of logits, ties to the lowest index, NaN ranked
// above every number (first NaN wins), matching torch.argmax as used by
// src/solort/model/cuda_graph_executor.py:201/:206 (in-graph), :234 (draft),
// :475 (verify).
//
// Every element maps to one 64-bit key: high word = an order-preserving
// image of its fp32 value (-0 and +0 equal, NaN largest), low word =
// 0xffffffff - index.  The row's answer is the maximum key, so blocks reduce
// with a plain integer max (wave shuffles, then LDS), fold their result into
// the row's slot with one 64-bit atomic max, and the last block of the row
// (atomic ticket) decodes the index and clears the slot and ticket for the
// next launch.
#include "common.h"
#include "capi_internal.h"

namespace solort {

template <int F32>
__global__ __launch_bounds__(256) void argmax_rows_kernel(const void* __restrict__ logits, int64_t vocab,
                                                          int64_t row_stride, int64_t per_block,
                                                          int vec_ok, uint64_t* __restrict__ ws_best,
                                                          unsigned* __restrict__ ws_cnt,
                                                          int64_t* __restrict__ out) {
  constexpr int VEC = F32 ? 4 : 8;  // elements per 16-byte load
  __shared__ uint64_t s_best[4];
  const int tid = threadIdx.x;
  const int row = blockIdx.y;
  const int64_t beg = (int64_t)blockIdx.x * per_block;
  const int64_t end = min(beg + per_block, vocab);
  const char* base = reinterpret_cast<const char*>(logits) + (int64_t)row * row_stride * (F32 ? 4 : 2);

  uint64_t best = 0;  // below every real key
  for (int64_t i = beg + (int64_t)tid * VEC; i < end; i += 256 * VEC) {
    float x[8];
    int n = (int)min((int64_t)VEC, end - i);
    if (vec_ok && n == VEC) {
      const uint4 v = *reinterpret_cast<const uint4*>(base + i * (F32 ? 4 : 2));
      if (F32) {
        x[0] = __uint_as_float(v.x); x[1] = __uint_as_float(v.y);
        x[2] = __uint_as_float(v.z); x[3] = __uint_as_float(v.w);
      } else {
        unpack8(v, x);
      }
    } else {
      for (int e = 0; e < n; ++e)
        x[e] = F32 ? reinterpret_cast<const float*>(base)[i + e]
                   : bf2f(reinterpret_cast<const uint16_t*>(base)[i + e]);
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      if (e < n) best = umax64(best, argmax_key(x[e], i + e));
  }
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) best = umax64(best, __shfl_xor(best, mask, 64));
  if ((tid & 63) == 0) s_best[tid >> 6] = best;
  __syncthreads();
  if (tid == 0)
    argmax_fold(umax64(umax64(s_best[0], s_best[1]), umax64(s_best[2], s_best[3])), ws_best + row, ws_cnt + row,
                gridDim.x, out + row);
}

}  // namespace solort

using namespace solort;

extern "C" size_t solort_argmax_workspace_bytes(int rows) {
  if (rows < 1) return 0;
  const size_t best = ((size_t)rows * 8 + 255) & ~(size_t)255;
  const size_t cnt = ((size_t)rows * 4 + 255) & ~(size_t)255;
  return best + cnt;
}

extern "C" int solort_argmax_rows(const void* logits, int dtype, int rows, int64_t vocab,
                                  int64_t row_stride, int64_t* out_idx, void* ws,
                                  solort_stream_t stream) {
  if (dtype != SOLORT_DTYPE_BF16 && dtype != SOLORT_DTYPE_F32)
    return set_error(SOLORT_EINVAL, "argmax_rows: dtype %d", dtype);
  if (rows < 1 || rows > 65535 || vocab < 1 || vocab > 0xffffffffLL || row_stride < vocab)
    return set_error(SOLORT_EINVAL, "argmax_rows: bad shape rows=%d vocab=%lld stride=%lld", rows,
                     (long long)vocab, (long long)row_stride);
  if (!logits || !out_idx || !ws) return set_error(SOLORT_EINVAL, "argmax_rows: null pointer");
  if (((uintptr_t)ws & 7u) || ((uintptr_t)out_idx & 7u))
    return set_error(SOLORT_EINVAL, "argmax_rows: ws and out_idx must be 8-byte aligned");
  const int esz = dtype == SOLORT_DTYPE_F32 ? 4 : 2;
  const int vec = 16 / esz;
  const int vec_ok = aligned16(logits) && ((row_stride * esz) % 16 == 0);
  // About 256 blocks in total, each a multiple of 256 threads x one vector.
  const int64_t unit = 256LL * vec;
  int64_t target = (256 + rows - 1) / rows;
  int64_t per_block = (vocab + target - 1) / target;
  per_block = ((per_block + unit - 1) / unit) * unit;
  const int64_t nblk = (vocab + per_block - 1) / per_block;
  const size_t best_bytes = ((size_t)rows * 8 + 255) & ~(size_t)255;
  uint64_t* ws_best = (uint64_t*)ws;
  unsigned* ws_cnt = (unsigned*)((char*)ws + best_bytes);
  dim3 grid((unsigned)nblk, (unsigned)rows);
  if (dtype == SOLORT_DTYPE_F32)
    hipLaunchKernelGGL(argmax_rows_kernel<1>, grid, dim3(256), 0, (hipStream_t)stream, logits, vocab,
                       row_stride, per_block, vec_ok, ws_best, ws_cnt, out_idx);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<0>, grid, dim3(256), 0, (hipStream_t)stream, logits, vocab,
                       row_stride, per_block, vec_ok, ws_best, ws_cnt, out_idx);
  return check_launch("argmax_rows");
}
