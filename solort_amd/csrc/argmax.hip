// Greedy argmax over rows of logits, ties to the lowest index, NaN ranked
// above every number (first NaN wins), matching torch.argmax as used by
// src/solort/model/cuda_graph_executor.py:201/:206 (in-graph), :234 (draft),
// :475 (verify).
//
// Every element maps to one 64-bit key: high word = an order-preserving
// image of its fp32 value (-0 and +0 equal, NaN largest), low word =
// 0xffffffff - index.  The row's answer is the maximum key.  Each row is cut
// into chunks, one block each; a block reduces its chunk's keys (wave
// shuffles, then LDS) and stores its best key in its slot of the row, tagged
// with this launch's epoch.  Two ways to reduce the slots:
//   - one launch (where the placement below has been checked): the row's
//     last block polls the slots until every one carries the epoch, reduces
//     them, writes the index and advances the row's epoch.  No atomic and no
//     store acknowledgement lies on the row's path, and no slot needs
//     clearing: a slot of an earlier launch carries an earlier epoch.
//   - two launches (placement unverified, or solort_argmax_mode(0)): every
//     block stores its slot and a one-wavefront launch per row reduces the
//     slots after the launch boundary and advances the epoch.
// Both give the same index.
//
// Workspace per row (zero-filled once): kMaxChunks slots of 16 bytes, two
// 8-byte pairs (key low, epoch) and (key high, epoch), then a 16-byte item
// holding the row's 32-bit epoch and, in the next word, the number of calls
// whose reduction failed (a slot never carried its tag), so that calls with
// any number of rows find a row's slots and epoch at the same place.  A
// naturally aligned 8-byte store is single-copy atomic, so a pair that
// carries the epoch carries its half of the key.  A launch reads the row's
// epoch e and tags its slots e + 1 (never 0, the zero-filled value, before
// 2^32 launches).  A failed reduction still writes an index inside the row
// (the best key among the slots it found, its own chunk's included) and
// counts the failure, which the host reads at its next synchronisation: no
// index outside [0, vocab) is ever written.
//
// Placement (one launch): block (x, y) = (row slot, chunk) has linear index
// x + rows8 y with rows8 a multiple of 8, so all chunks of a row run on the
// XCD of row % 8 (workgroup b runs on the XCD of b % 8, checked by
// solort_init), where their slots meet in the L2; the reading block is the
// row's last chunk, dispatched after the others.
#include "common.h"
#include "capi_internal.h"

namespace solort {

constexpr int kMaxChunks = 64;     // chunks (blocks) per row
constexpr int kRowItems = kMaxChunks + 1;  // 16-byte items per row: the slots, then the epoch
constexpr int kArgmaxSpin = 1 << 20;  // polling rounds before the reader gives up (counts a failure)

__device__ __forceinline__ int64_t key_to_index(uint64_t k) {
  return (int64_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
}

// ONE: the one-launch reduction (the row's last block polls); otherwise every
// block stores its slot and argmax_finish_kernel reduces them.
// spin: the reader's polling limit (kArgmaxSpin; 0 in the test mode of solort_argmax_mode(2)).
template <int F32, bool ONE>
__global__ __launch_bounds__(256) void argmax_rows_kernel(const void* __restrict__ logits, int64_t vocab,
                                                          int64_t row_stride, int64_t per_block, int rows,
                                                          int vec_ok, uint4* __restrict__ slots,
                                                          int64_t* __restrict__ out, int spin) {
  constexpr int VEC = F32 ? 4 : 8;  // elements per 16-byte load
  __shared__ uint64_t s_best[4];
  const int tid = threadIdx.x;
  const int row = blockIdx.x, chunk = blockIdx.y, nchunk = gridDim.y;
  if (row >= rows) return;  // padding of the row dimension to a multiple of 8
  const int64_t beg = (int64_t)chunk * per_block;
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
  uint4* rs = slots + (int64_t)row * kRowItems;
  unsigned* epoch = reinterpret_cast<unsigned*>(rs + kMaxChunks);
  const unsigned ep = *epoch + 1u;  // this launch's tag
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) best = umax64(best, __shfl_xor(best, mask, 64));
  if ((tid & 63) == 0) s_best[tid >> 6] = best;
  __syncthreads();
  best = umax64(umax64(s_best[0], s_best[1]), umax64(s_best[2], s_best[3]));
  if (!ONE || chunk != nchunk - 1) {
    if (tid == 0) rs[chunk] = make_uint4((uint32_t)best, ep, (uint32_t)(best >> 32), ep);
    return;
  }
  // The row's last block: lane j polls slot j with device-scope loads (they
  // miss the L1 and read the XCD's L2).  The empty asm keeps the compiler
  // from hoisting the load out of the loop.
  if (tid >= 64) return;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(rs, (short)0, kMaxChunks * 16, 0x00020000);
  uint64_t k = tid == chunk ? best : 0;
  bool pend = tid < nchunk && tid != chunk;
  for (int it = 0; __builtin_amdgcn_ballot_w64(pend) != 0 && it < spin; ++it) {
    asm volatile("" ::: "memory");
    const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, tid * 16, 0, 16));
    if (pend && v.y == ep && v.w == ep) {
      k = ((uint64_t)v.z << 32) | v.x;
      pend = false;
    }
  }
  const bool timed_out = __builtin_amdgcn_ballot_w64(pend) != 0;
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) k = umax64(k, __shfl_xor(k, mask, 64));
  if (tid == 0) {
    // k holds at least this block's own key (its chunk is not empty), so the index is in the row.
    out[row] = key_to_index(k);
    if (timed_out) epoch[1] += 1u;
    *epoch = ep;
  }
}

// Two-launch reduction: one wavefront per row; lane j reads slot j (the
// launch boundary orders these reads after the slot stores), checks its tag,
// reduces, writes the index and advances the row's epoch.  A slot without
// the tag (never expected) is left out and counted as a failure; with no
// valid slot at all the index written is 0.
__global__ __launch_bounds__(64) void argmax_finish_kernel(int nchunk, uint4* __restrict__ slots,
                                                           int64_t* __restrict__ out) {
  const int row = blockIdx.x, lane = threadIdx.x;
  uint4* rs = slots + (int64_t)row * kRowItems;
  unsigned* epoch = reinterpret_cast<unsigned*>(rs + kMaxChunks);
  const unsigned ep = *epoch + 1u;
  uint64_t k = 0;
  bool bad = false;
  if (lane < nchunk) {
    const uint4 v = rs[lane];
    if (v.y == ep && v.w == ep)
      k = ((uint64_t)v.z << 32) | v.x;
    else
      bad = true;
  }
  const bool failed = __builtin_amdgcn_ballot_w64(bad) != 0;
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) k = umax64(k, __shfl_xor(k, mask, 64));
  if (lane == 0) {
    out[row] = k ? key_to_index(k) : 0;
    if (failed) epoch[1] += 1u;
    *epoch = ep;
  }
}

namespace {
constexpr int kMaxDev = 64;
// Per device, the mode solort_argmax_mode set, stored as mode + 1 so that the zero-filled start
// means mode 1: 1 the one-launch reduction where the placement check passed, 0 always two
// launches, 2 the one-launch reduction whose reducing block gives up at once (test mode).
int g_argmax_mode[kMaxDev];
}  // namespace

// The mode in effect on the current device: the one-launch forms need the
// round-robin placement checked by solort_init.
static int argmax_mode_now() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
  const int m = g_argmax_mode[dev] == 0 ? 1 : g_argmax_mode[dev] - 1;  // stored as mode + 1
  return m != 0 && xcd_round_robin(dev) ? m : 0;
}

}  // namespace solort

using namespace solort;

extern "C" int solort_argmax_mode(int mode) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev)
    return set_error(SOLORT_EINVAL, "argmax_mode: no current device");
  if (mode < -1 || mode > 2) return set_error(SOLORT_EINVAL, "argmax_mode: mode %d", mode);
  if (mode >= 0) g_argmax_mode[dev] = mode + 1;
  return argmax_mode_now();
}

extern "C" size_t solort_argmax_workspace_bytes(int rows) {
  if (rows < 1) return 0;
  return ((size_t)rows * kRowItems * 16 + 255) & ~(size_t)255;
}

extern "C" int solort_argmax_rows(const void* logits, int dtype, int rows, int64_t vocab,
                                  int64_t row_stride, int64_t* out_idx, void* ws,
                                  solort_stream_t stream) {
  if (dtype != SOLORT_DTYPE_BF16 && dtype != SOLORT_DTYPE_F32)
    return set_error(SOLORT_EINVAL, "argmax_rows: dtype %d", dtype);
  if (rows < 1 || rows > 65528 || vocab < 1 || vocab > 0xffffffffLL || row_stride < vocab)
    return set_error(SOLORT_EINVAL, "argmax_rows: bad shape rows=%d vocab=%lld stride=%lld", rows,
                     (long long)vocab, (long long)row_stride);
  if (!logits || !out_idx || !ws) return set_error(SOLORT_EINVAL, "argmax_rows: null pointer");
  if (!aligned16(ws) || ((uintptr_t)out_idx & 7u))
    return set_error(SOLORT_EINVAL, "argmax_rows: ws must be 16-byte and out_idx 8-byte aligned");
  const int esz = dtype == SOLORT_DTYPE_F32 ? 4 : 2;
  const int vec = 16 / esz;
  const int vec_ok = aligned16(logits) && ((row_stride * esz) % 16 == 0);
  // About 256 blocks in total (measured best for [5, 151936]: 5.0 us at 38 or
  // more blocks per row, 6.4 at 24, 7.2 at 16), at most kMaxChunks per row,
  // each a multiple of 256 threads x one vector.
  const int64_t unit = 256LL * vec;
  int64_t target = (256 + rows - 1) / rows;
  target = target < 1 ? 1 : (target > kMaxChunks ? kMaxChunks : target);
  int64_t per_block = (vocab + target - 1) / target;
  per_block = ((per_block + unit - 1) / unit) * unit;
  const int64_t nblk = (vocab + per_block - 1) / per_block;  // <= target
  uint4* slots = (uint4*)ws;
  hipStream_t s = (hipStream_t)stream;
  const int mode = argmax_mode_now();
  if (mode != 0) {
    const int rows8 = (rows + 7) & ~7;
    const dim3 grid((unsigned)rows8, (unsigned)nblk);
    const int spin = mode == 2 ? 0 : kArgmaxSpin;
    if (dtype == SOLORT_DTYPE_F32)
      hipLaunchKernelGGL((argmax_rows_kernel<1, true>), grid, dim3(256), 0, s, logits, vocab, row_stride, per_block,
                         rows, vec_ok, slots, out_idx, spin);
    else
      hipLaunchKernelGGL((argmax_rows_kernel<0, true>), grid, dim3(256), 0, s, logits, vocab, row_stride, per_block,
                         rows, vec_ok, slots, out_idx, spin);
    return check_launch("argmax_rows");
  }
  const dim3 grid((unsigned)rows, (unsigned)nblk);
  if (dtype == SOLORT_DTYPE_F32)
    hipLaunchKernelGGL((argmax_rows_kernel<1, false>), grid, dim3(256), 0, s, logits, vocab, row_stride, per_block,
                       rows, vec_ok, slots, out_idx, 0);
  else
    hipLaunchKernelGGL((argmax_rows_kernel<0, false>), grid, dim3(256), 0, s, logits, vocab, row_stride, per_block,
                       rows, vec_ok, slots, out_idx, 0);
  const int rc = check_launch("argmax_rows");
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_finish_kernel, dim3((unsigned)rows), dim3(64), 0, s, (int)nblk, slots, out_idx);
  return check_launch("argmax_rows");
}
