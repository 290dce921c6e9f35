// Split-KV (flash-decoding) grouped-query attention for 1..8 new tokens over
// the static KV cache, optionally fused with the QK-RMSNorm + RoPE prologue
// and KV write; the splits are merged in the same launch or by a small
// second kernel.
//
// Reference semantics (src/solort/model/cuda_graph_executor.py):
//   decode :168, :173-184  q/k norm + rope, KV write at pos, then
//                          softmax(qg K^T * scale, keys > pos masked) V over
//                          the bucket                             (nq = 1)
//   verify :247-263        the same for query t at position pos0+t, which
//                          attends keys 0..pos0+t                 (nq = K+1)
// Scores, softmax and the weighted sum are computed in fp32 (the reference
// rounds scores and probabilities to bf16 between its torch ops); the output
// is rounded once, to bf16, or left in fp32 on request.
//
// Grid: nkv * n_split workgroups of 256 threads; block (kvh, split) serves
// KV head kvh and a static key chunk of [0, bound) (with 8 KV heads on 8
// XCDs, all splits of a head share one XCD's L2).  Every block issues its
// first K/V loads at launch, before the device-side position has arrived;
// keys past the live length are masked.  Fused variant: while those loads
// are in flight, 16-lane slots compute the q rows and the new tokens' K/V
// rows from the fused qkv projection and the step's cos/sin rows
// (qknorm_rope.h, bit identical to the standalone prologue).  Split 0 of
// each KV head writes the new rows to the cache; every block substitutes the
// fresh rows for the cache rows pos0..pos0+nq-1 it loaded, so no block waits
// for that write.  Two split kernels share this structure:
//   - decode_lanes_kernel, for short chunks of one new token (latency-bound):
//     16 row slots of 16 lanes take U key rows per step (lane j: dims
//     8j..8j+7); the query group sits in registers as bf16 pairs, a score is
//     four bf16 pair dot products reduced over the slot with DPP, and scores
//     and V rows go through LDS so that each wavefront accumulates its own
//     query row (two output dims per lane).  For the fused layer on a
//     contiguous cache whose strides fit 16 bits (in 16-byte units), the same
//     body runs as decode_lanes_packed_kernel, whose packed arguments keep
//     every pointer the first loads need among the preloaded dwords.
//   - decode_mfma_kernel, for long chunks and several new tokens: each
//     wavefront takes 32-key tiles (kbeg + 32w + 128i), stages K and V
//     through its LDS tile with whole-row loads, and computes S^T = K q^T and
//     O^T += V^T P^T on v_mfma_f32_32x32x16_bf16 with the query rows (at most
//     32) as the N dimension; V^T comes from transposing LDS reads and P
//     enters as bf16 high and low parts (~16 bits), with a lazily moved
//     softmax maximum.  The wavefronts merge in LDS at the end.  Fused, on a
//     contiguous cache with packed qkv rows, the same body runs as
//     decode_mfma_packed_kernel (packed arguments, as above).
// Output: with one split the block writes the answer; otherwise its partial
// (running max in log2 units, sum, unnormalised output), tagged.  The
// partials of each KV head are merged (log-sum-exp) by the head's last
// splits, which poll for the tags of this launch (in-launch merge), or by
// the combine kernel, whose launch boundary orders its reads after the split
// kernel's writes.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "capi_internal.h"
#include "qknorm_rope.h"
#include "gemv_common.h"

namespace solort {

SOLORT_STAMP_TU();  // phase stamps of the tracing build (common.h)

// The kernel's leading arguments are the ones its first loads need; the
// compiler preloads the leading kernel arguments into SGPRs (14 dwords, see
// -amdgpu-kernarg-preload-count in the build), so those loads issue without
// waiting for the kernel-argument fetch.  The rest travel in DecodeTail.
struct DecodeTail {
  const uint16_t* kn_w;
  const uint16_t* rope_cs;  // [2][nq][64] bf16: cos rows, then sin rows, of this step
  const int64_t* pos0_dev;
  // Partials of the splits.  In-launch merge: tagged, ws_o [nkv][n_split][R][64] items (O[2i],
  // tag, O[2i+1], tag) and ws_ml [nkv][n_split][R] items (running max in log2 units, tag, sum,
  // tag).  Otherwise untagged, in the same regions: fp32 [nkv][n_split][R][128] and
  // [nkv][n_split][R][2].
  uint4* ws_o;
  uint4* ws_ml;
  void* out;     // [nq][nh][128]
  float qscale;  // softmax scale * log2(e)
  float eps;
  int pos_limit;  // positions >= pos_limit are not written
  int out_f32;
  // Paged cache (PAGED kernels): position t lives in page page_table[t >> page_shift], row
  // t & (2^page_shift - 1); a page is page_stride elements from the next.
  const int32_t* page_table;
  int64_t page_stride;
  int page_shift;
  int num_pages;
  // Per KV head a 32-bit launch counter of the in-launch merge, 128 bytes apart (the
  // workspace's start).
  unsigned* epochs;
  int n_split;  // splits per KV head
  int merge;    // 1: the in-launch merge; 0: the combine kernel's second launch
};

// The qkv product computed inside the decode launch (decode_qkv_lanes_kernel):
// x, in_w, wqkv and hidden travel among the preloaded arguments; these in the
// tail.
struct QkvIn {
  const uint16_t* qn_w;
  uint2* items;  // [nkv][(G + 2) * 64] tagged pairs (two bf16 outputs, tag)
  float eps;     // the input RMSNorm's
};

// Element offset of the cache row at position t (head 0, dim 0).  Paged: a
// table entry outside [0, num_pages) is clamped into the pool, so a bad
// entry reads a wrong row but never leaves the allocation.
template <bool PAGED>
__device__ __forceinline__ int64_t row_off(int64_t t, int tok_stride, const DecodeTail& a) {
  if constexpr (PAGED) {
    const int p = min(max(a.page_table[t >> a.page_shift], 0), a.num_pages - 1);
    return (int64_t)p * a.page_stride + (t & ((1 << a.page_shift) - 1)) * tok_stride;
  } else {
    return t * tok_stride;
  }
}

__device__ __forceinline__ float4 f4fma(float w, const float4 v, float4 acc) {
  acc.x = fmaf(w, v.x, acc.x);
  acc.y = fmaf(w, v.y, acc.y);
  acc.z = fmaf(w, v.z, acc.z);
  acc.w = fmaf(w, v.w, acc.w);
  return acc;
}

// Writes float4 column col of KV head kvh's [R][128] output block.
__device__ __forceinline__ void store_out(void* out, int out_f32, int nh, int kvh, int G, int col, float4 O) {
  const int r = col >> 5, d = (col & 31) * 4;
  const int t = r / G, g = r % G;
  const int64_t oi = ((int64_t)t * nh + kvh * G + g) * SOLORT_HD + d;
  if (out_f32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + oi) = O;
  } else {
    uint2 v;
    v.x = f2bf(O.x) | (f2bf(O.y) << 16);
    v.y = f2bf(O.z) | (f2bf(O.w) << 16);
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + oi) = v;
  }
}

// Writes dims d, d+1 of output row r (query t = r / G, head kvh*G + r % G).
__device__ __forceinline__ void store_out2(void* out, int out_f32, int nh, int kvh, int G, int r, int d, float o0,
                                           float o1) {
  const int t = r / G, g = r % G;
  const int64_t oi = ((int64_t)t * nh + kvh * G + g) * SOLORT_HD + d;
  if (out_f32)
    *reinterpret_cast<float2*>(reinterpret_cast<float*>(out) + oi) = make_float2(o0, o1);
  else
    *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(out) + oi) = f2bf(o0) | (f2bf(o1) << 16);
}

// ---------------------------------------------------------------- split combine
// The log-sum-exp combine of the n_split partials of one KV head: thread =
// (float4 column c of the head's [R][128] output, split group sg of 8) merges
// splits sg, sg + 8, ... on its own (up to kCombB loads in flight per batch),
// then the 8 split groups meet once in LDS.  The combine kernel and the
// in-launch merge both run one row (32 columns) per workgroup with these
// functions, so both give the same bits.

constexpr int kCombB = 8;  // splits per thread per batch (combine kernel)

struct CombAcc {
  float m, l;  // max (log2 units) and sum of the merged splits
  float4 o;    // their unnormalised output column
};

__device__ __forceinline__ CombAcc comb_init() { return CombAcc{-INFINITY, 0.f, make_float4(0.f, 0.f, 0.f, 0.f)}; }

// Folds a batch of B partials (max -inf: an empty or absent split) into acc.
// Branch-free, so that the compiler keeps every load of the batch ahead of
// it: with no split seen yet (mb = -inf) all weights are 0 and acc stays
// (m = -inf, l = 0, o = 0).
template <int B>
__device__ __forceinline__ void comb_merge(CombAcc& acc, const float2 (&ml)[B], const float4 (&ov)[B]) {
  float mb = acc.m;
#pragma unroll
  for (int k = 0; k < B; ++k) mb = fmaxf(mb, ml[k].x);
  const float mr = mb == -INFINITY ? 0.f : mb;  // reference for the weights
  const float sc = fast_exp2(acc.m - mr);       // acc.m = -inf gives 0
  acc.l *= sc;
  acc.o.x *= sc; acc.o.y *= sc; acc.o.z *= sc; acc.o.w *= sc;
#pragma unroll
  for (int k = 0; k < B; ++k) {
    const float w = (ml[k].x == -INFINITY) ? 0.f : fast_exp2(ml[k].x - mr);
    acc.l = fmaf(w, ml[k].y, acc.l);
    acc.o = f4fma(w, ov[k], acc.o);
  }
  acc.m = mb;
}

// The 8 split groups of one column, [8][n_cols] in LDS (s_m, s_l, s_o), folded
// in group order; returns the normalised column.
__device__ __forceinline__ float4 comb_final(const float* s_m, const float* s_l, const float4* s_o, int n_cols,
                                             int c) {
  float Mx = -INFINITY;
#pragma unroll
  for (int g = 0; g < 8; ++g) Mx = fmaxf(Mx, s_m[g * n_cols + c]);
  float Ls = 0.f;
  float4 Os = make_float4(0.f, 0.f, 0.f, 0.f);
  if (Mx != -INFINITY) {
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const float mg = s_m[g * n_cols + c];
      const float w = (mg == -INFINITY) ? 0.f : fast_exp2(mg - Mx);
      Ls = fmaf(w, s_l[g * n_cols + c], Ls);
      Os = f4fma(w, s_o[g * n_cols + c], Os);
    }
  }
  const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
  Os.x *= inv; Os.y *= inv; Os.z *= inv; Os.w *= inv;
  return Os;
}

// ---------------------------------------------------------------- in-launch merge
// In-launch mode (DecodeTail::merge), with more than one split: each split
// stores its partial as tagged 8-byte pairs (value, tag): per row of the
// head, 64 items of 16 bytes (O[2i], tag, O[2i+1], tag), then one item (max,
// tag, sum, tag).  A naturally aligned 8-byte store is single-copy atomic, so
// a reader that sees the tag of this launch in a pair also sees that pair's
// value.  The tag is this launch's value of the KV head's counter, and the
// last K = min(n_split, R) splits of the head each merge rows j, j + K, ...
// (j = split - (n_split - K)) once every split's items for them carry the
// tag: they poll the items with loads that miss the CU's L1 (cache policy
// sc1) and read the XCD's L2, where every split of the head stores (blocks
// (kvh, split) have linear index kvh + nkv * split, nkv is a multiple of 8,
// and workgroup b runs on the XCD of workgroup b % 8, checked by
// solort_init).  No store waits for an acknowledgement, no atomic is issued
// and nothing is cleared: items of earlier launches carry earlier tags.  The
// merge functions are the combine kernel's, so both modes give the same bits.
// (Two-launch mode: untagged partials, half the bytes, which the combine
// kernel reads after the launch boundary.)
//
// Tags: the head's counter (32 bits, 128 bytes apart per head at the start of
// the workspace, zero-filled once) holds c; this launch uses n = c + 1
// (skipping multiples of 2^25) and tag (n mod 2^25) << 7 | kvh, and the block
// merging the head's first row stores n once its poll is done (by then every
// split of the head has read c: its tagged items depend on it).  A tag is
// never another head's, and it repeats only after 2^25 - 1 launches on the
// head.
constexpr int kMergeMaxSplit = 64;   // in-launch merge: splits per head (8 per split group)
constexpr int kMergeHeads = 128;     // ... KV heads (counters at the start of the workspace)
constexpr int kMergeSpin = 1 << 18;  // polling rounds before a merging block gives up (writes NaN)

__device__ __forceinline__ unsigned merge_next(unsigned c) {
  unsigned n = c + 1u;
  if ((n & 0x1ffffffu) == 0u) ++n;
  return n;
}
__device__ __forceinline__ unsigned merge_tag(unsigned n, int kvh) { return ((n & 0x1ffffffu) << 7) | (unsigned)kvh; }


// Merges the head's rows j, j + K, ... (see above) and writes them.  Called
// by every thread of a merging block, after its own partial is stored; lds:
// 6 KiB no other wave still uses.  Thread (column c of the row, split group
// sg) polls splits sg + 8k.
template <int R>
__device__ __forceinline__ void split_merge(const DecodeTail& a, int kvh, int split, int NS, int nh, int G,
                                            unsigned tag, unsigned next, uint8_t* lds) {
  const int K = min(NS, R);
  const int j = split - (NS - K);
  if (j < 0) return;  // block-uniform
  __shared__ int s_bad;
  const int tid = threadIdx.x, c = tid & 31, sg = tid >> 5;
  const int nk = (NS - sg + 7) >> 3;  // splits sg + 8k (k < nk) exist
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_o + (size_t)kvh * NS * R * 64, (short)0, NS * R * 64 * 16, 0x00020000);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_ml + (size_t)kvh * NS * R, (short)0, NS * R * 16, 0x00020000);
  float* s_m = reinterpret_cast<float*>(lds);
  float* s_l = s_m + 8 * 32;
  float4* s_o = reinterpret_cast<float4*>(s_l + 8 * 32);
  for (int r = j; r < R; r += K) {
    if (tid == 0) s_bad = 0;
    __syncthreads();  // the LDS region is free; s_bad is set
    float2 ml[kCombB];
    float4 ov[kCombB];
#pragma unroll
    for (int k = 0; k < kCombB; ++k) {
      ml[k] = make_float2(-INFINITY, 0.f);  // an absent split
      ov[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    bool pend = true;
    SOLORT_STAMP(tid == 0 && r == j, blockIdx.x + gridDim.x * blockIdx.y, 6);
    for (int it = 0; it < kMergeSpin; ++it) {
      pend = false;
      // Splits in batches of four per thread (the second only past 32 splits): fewer registers.
#pragma unroll
      for (int k0 = 0; k0 < kCombB; k0 += 4) {
        if (k0 < nk) {
          asm volatile("" ::: "memory");  // a fresh load every round
          uint4 mv[4], xv[4], yv[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if (k0 + k < nk) {
              const int pr = (sg + 8 * (k0 + k)) * R + r;
              mv[k] = ld_l2(rm, pr * 16);
              xv[k] = ld_l2(ro, (pr * 64 + 2 * c) * 16);
              yv[k] = ld_l2(ro, (pr * 64 + 2 * c + 1) * 16);
            }
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if (k0 + k < nk) {
              ml[k0 + k] = make_float2(__uint_as_float(mv[k].x), __uint_as_float(mv[k].z));
              ov[k0 + k] = make_float4(__uint_as_float(xv[k].x), __uint_as_float(xv[k].z),
                                       __uint_as_float(yv[k].x), __uint_as_float(yv[k].z));
              pend |= (mv[k].y != tag) | (mv[k].w != tag) | (xv[k].y != tag) | (xv[k].w != tag) |
                      (yv[k].y != tag) | (yv[k].w != tag);
            }
          }
        }
      }
      if (__builtin_amdgcn_ballot_w64(pend) == 0) break;
    }
    if (pend) s_bad = 1;
    SOLORT_STAMP(tid == 0 && r == j, blockIdx.x + gridDim.x * blockIdx.y, 7);
    CombAcc acc = comb_init();
    comb_merge<kCombB>(acc, ml, ov);
    s_m[sg * 32 + c] = acc.m;
    s_l[sg * 32 + c] = acc.l;
    s_o[sg * 32 + c] = acc.o;
    __syncthreads();
    // Every wave has seen every split's items: each split has read the counter.
    if (r == 0 && tid == 0) a.epochs[kvh * 32] = next;
    if (tid < 32) {
      float4 v = comb_final(s_m, s_l, s_o, 32, c);
      if (s_bad) v = make_float4(NAN, NAN, NAN, NAN);
      store_out(a.out, a.out_f32, nh, kvh, G, 32 * r + c, v);
    }
    __syncthreads();  // LDS and s_bad are reused by the next row
  }
}

// The qkv product inside a decode launch (one new token), shared by both
// split kernels.  qkv_issue: this wave's RW weight rows of the KV head's
// (G + 2) * 128 outputs (outputs i0 .. i0 + RW - 1: the rows of q heads
// kvh*G .. kvh*G + G - 1, then its K and V rows), lane l taking 16-byte chunks
// l + 64u as the GEMV kernel does.
template <int G, int RW, int CPL>
__device__ __forceinline__ void qkv_issue(uint4 (&wv)[RW][CPL], const uint16_t* wqkv, int hidden, int i0, int kvh,
                                          int nh, int nkv, int lane) {
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int i = i0 + r, c = i >> 7;
    const int hs = c < G ? kvh * G + c : (c == G ? nh + kvh : nh + nkv + kvh);
    const uint16_t* wrow = wqkv + (int64_t)(hs * SOLORT_HD + (i & 127)) * hidden;
#pragma unroll
    for (int u = 0; u < CPL; ++u) wv[r][u] = ld_stream(wrow + 8 * (lane + 64 * u));
  }
}

// x normalised into s_x (LDS free until the caller's next use of it), the
// wave's RW dot products in the GEMV kernel's order and rounding, stored as
// tagged pairs (two bf16 outputs, the launch's tag); then the calling lane's 8
// values of row prow (of the head's G + 2 rows), polled from the XCD's L2 where
// the head's splits store them.  A lane that gives up after kMergeSpin rounds
// returns NaN.  Every thread of the 256-thread block calls it.
template <int G, int RW, int CPL>
__device__ __forceinline__ uint4 qkv_handover(const uint4 (&wv)[RW][CPL], const XChunks& xin, const uint16_t* x,
                                              const uint16_t* in_w, float eps, int hidden, uint4* s_x, float* s_red,
                                              uint2* items, unsigned tag, int i0, int prow, int j, int lane,
                                              int stamp_block) {
  gemv_x_finish<true>(xin, x, in_w, eps, hidden, s_x, s_red);
  float acc[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) acc[r] = 0.f;
#pragma unroll
  for (int u = 0; u < CPL; ++u) {
    const uint4 xv = s_x[lane + 64 * u];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      float d = dot2bf(wv[r][u].x, xv.x, acc[r]);
      d = dot2bf(wv[r][u].y, xv.y, d);
      d = dot2bf(wv[r][u].z, xv.z, d);
      acc[r] = dot2bf(wv[r][u].w, xv.w, d);
    }
  }
  uint32_t mine = 0;
#pragma unroll
  for (int r = 0; r < RW; r += 2) {
    const uint32_t pr = f2bf(wave_sum64(acc[r])) | f2bf(wave_sum64(acc[r + 1])) << 16;
    if (lane == r / 2) mine = pr;
  }
  if (lane < RW / 2) items[i0 / 2 + lane] = make_uint2(mine, tag);
  SOLORT_STAMP(threadIdx.x == 0, stamp_block, 8);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(items, (short)0, (G + 2) * 64 * 8, 0x00020000);
  const int off = (prow * 64 + 4 * j) * 8;
  uint4 a01 = make_uint4(0u, 0u, 0u, 0u), a23 = a01;
  bool pend = true;
  for (int it = 0; it < kMergeSpin && pend; ++it) {
    asm volatile("" ::: "memory");  // a fresh load every round
    a01 = ld_l2(rq, off);
    a23 = ld_l2(rq, off + 16);
    const bool bad = (a01.y != tag) | (a01.w != tag) | (a23.y != tag) | (a23.w != tag);
    pend = __builtin_amdgcn_ballot_w64(bad) != 0;
  }
  SOLORT_STAMP(threadIdx.x == 0, stamp_block, 9);
  return pend ? make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u)  // NaN: gave up
              : make_uint4(a01.x, a01.z, a23.x, a23.z);
}

__device__ __forceinline__ int64_t pos_from(uint2 v) {
  return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)v.y) << 32) |
                   (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)v.x));
}

// Lane-parallel split kernel, for short key chunks (latency-bound: one to a
// few key rows per slot).  Grid (nkv, n_split): block (kvh, split).  qsrc:
// fused, the qkv rows (row stride qsrc_stride); unfused, the q rows
// [nq][nh][128] (qsrc_stride = nh*128).
template <int NQ, int G, int U, bool FUSED, bool PAGED, int RW = 0, int CPL = 0>
__device__ __forceinline__ void decode_lanes_body(uint16_t* kc, uint16_t* vc, int tok_stride, int head_stride,
                                                  int chunk, int bound, const uint16_t* qsrc, int qsrc_stride,
                                                  int nh, const uint16_t* qn_w, const uint16_t* kn_w,
                                                  const uint16_t* rope_cs, const DecodeTail& a,
                                                  const uint16_t* x = nullptr, const uint16_t* wqkv = nullptr,
                                                  const uint16_t* in_w = nullptr, int hidden = 0,
                                                  const QkvIn* qi = nullptr) {
  constexpr bool QKV = RW > 0;  // the qkv rows computed in this launch from x and wqkv
  constexpr int R = NQ * G;            // query rows sharing one KV head
  constexpr int KPI = 16 * U;          // keys per iteration (16 slots x U)
  constexpr int RPW = (R + 3) / 4;     // output rows per wavefront
  __shared__ __align__(16) uint4 s_q[R * 16];         // q rows, bf16 bits [row][16 x 16 B]
  __shared__ uint4 s_new[FUSED ? 2 * NQ * 16 : 1];   // fresh K rows then V rows (bf16 bits)
  // the iteration's V rows [key][16 x 16 B]; at least 6 KiB (the in-launch merge's LDS)
  __shared__ __align__(16) uint4 s_v[KPI * 16 > 384 ? KPI * 16 : 384];
  __shared__ __align__(16) float s_s[R * KPI];       // its masked scores [row][key] (log2 units), then p

  const int tid = threadIdx.x, j = tid & 15, slot = tid >> 4, wave = tid >> 6, lane = tid & 63;
  const int kvh = blockIdx.x, split = blockIdx.y;
  const int nkv = nh / G;  // = gridDim.x, without the hidden-argument load
  const int kbeg = min(split * chunk, bound);
  const int kstat = min(kbeg + chunk, bound);
  SOLORT_STAMP(tid == 0, kvh + nkv * split, 0);

  // 1. Loads for this slot's first prologue row (fused: with its norm
  //    weights and its token's cos/sin), issued before the K/V loads: vector
  //    loads complete in issue order, so the prologue then waits for its own
  //    rows only.  Every load of phases 1 and 2 is unconditional (idle lanes
  //    load a valid row they ignore): a load skipped on some path would make
  //    the compiler wait for all of them before the first use.
  constexpr int NROWS = FUSED ? NQ * (G + 2) : R;
  uint4 raw0 = make_uint4(0u, 0u, 0u, 0u), wq0 = raw0, wk0 = raw0, c0 = raw0, s0 = raw0;
  XChunks xin;  // QKV: this thread's chunks of x and the input norm weight, loaded first
  if constexpr (QKV) gemv_x_load<true>(x, in_w, hidden, xin);
  if constexpr (!QKV) {
    const int row = min(slot, NROWS - 1);
    if constexpr (FUSED) {
      const int t = row / (G + 2), c = row % (G + 2);
      const int hs = c < G ? kvh * G + c : (c == G ? nh + kvh : nh + nkv + kvh);
      raw0 = *reinterpret_cast<const uint4*>(qsrc + (int64_t)t * qsrc_stride + hs * SOLORT_HD + j * 8);
      wq0 = *reinterpret_cast<const uint4*>(qn_w + j * 8);
      wk0 = *reinterpret_cast<const uint4*>(kn_w + j * 8);
      c0 = *reinterpret_cast<const uint4*>(rope_cs + t * 64 + (j & 7) * 8);
      s0 = *reinterpret_cast<const uint4*>(rope_cs + (NQ + t) * 64 + (j & 7) * 8);
    } else {
      const int t = row / G, g = row % G;
      raw0 = *reinterpret_cast<const uint4*>(qsrc + (int64_t)t * qsrc_stride + (kvh * G + g) * SOLORT_HD + j * 8);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the K/V loads

  // 2. First K/V loads: static addresses, independent of the position.  Rows
  //    past this split's chunk re-read its last row (an empty chunk: row 0)
  //    and are masked below.
  const uint16_t* kp = kc + (int64_t)kvh * head_stride + j * 8;
  const uint16_t* vp = vc + (int64_t)kvh * head_stride + j * 8;
  const int kclamp = kstat > kbeg ? kstat - 1 : 0;
  uint4 kr[U], vr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int kid = min(kbeg + u * 16 + slot, kclamp);
    const int64_t off = row_off<PAGED>(kid, tok_stride, a);
    kr[u] = ld_stream(kp + off);
    vr[u] = ld_stream(vp + off);
  }
  __builtin_amdgcn_sched_barrier(0);  // every K/V load issues before the position is read

  // The qkv product in the launch: this wave's RW weight rows of the head's (G + 2) * 128 outputs
  // (outputs i0 .. i0 + RW - 1 of q heads kvh*G .. kvh*G + G - 1, then the K and V rows), lane l
  // taking 16-byte chunks l + 64u as the GEMV kernel does; then the prologue's own inputs.
  constexpr int QRW = QKV ? RW : 1, QCPL = QKV ? CPL : 1;
  uint4 wv[QRW][QCPL];
  const int i0 = (split * 4 + wave) * RW;
  if constexpr (QKV) {
    qkv_issue<G, RW, CPL>(wv, wqkv, hidden, i0, kvh, nh, nkv, lane);
    const int row = min(slot, NROWS - 1);
    wq0 = *reinterpret_cast<const uint4*>(qn_w + j * 8);
    wk0 = *reinterpret_cast<const uint4*>(kn_w + j * 8);
    c0 = *reinterpret_cast<const uint4*>(rope_cs + (row / (G + 2)) * 64 + (j & 7) * 8);
    s0 = *reinterpret_cast<const uint4*>(rope_cs + (NQ + row / (G + 2)) * 64 + (j & 7) * 8);
  }

  int64_t pos0;
  unsigned next;
  uint2 posv = make_uint2(0u, 0u);
  unsigned epv = 0u;
  if constexpr (QKV) {
    // Read by vector loads behind the weight loads: first used after the product, and a scalar
    // load's wait would be shared by the LDS barriers ahead of that.  (The merge counter is read
    // before any partial or qkv item of the block is stored, as below.)
    posv = ld_vec8(a.pos0_dev);
    epv = ld_vec4(a.epochs + kvh * 32);
    pos0 = 0;
    next = 0u;
  } else {
    pos0 = a.pos0_dev[0];
    // The KV head's merge counter, read by every wave ahead of the staging barrier below: each wave
    // of the block has read it before any partial of the block is stored, hence before the head's
    // row-0 merger (which waits for every split's partial) can advance it; and its round trip
    // overlaps the prologue instead of preceding the partial stores.
    next = a.merge ? merge_next(a.epochs[kvh * 32]) : 0u;
  }
  SOLORT_STAMP(tid == 0, kvh + nkv * split, 1);

  if constexpr (QKV) {
    // x normalised into LDS (s_v, free until the key loop), the wave's RW dot products in the GEMV
    // kernel's order and rounding, stored as tagged pairs; then each slot polls its row of the
    // head's qkv outputs, stored by the head's splits (all on this XCD) with this launch's tag.
    __shared__ float s_red[4];
    next = merge_next((unsigned)__builtin_amdgcn_readfirstlane((int)epv));
    raw0 = qkv_handover<G, RW, CPL>(wv, xin, x, in_w, qi->eps, hidden, reinterpret_cast<uint4*>(s_v), s_red,
                                    qi->items + (int64_t)kvh * (G + 2) * 64, merge_tag(next, kvh), i0,
                                    min(slot, NROWS - 1), j, lane, kvh + nkv * split);
    pos0 = pos_from(posv);
  }

  // 3. q rows (and, fused, the new tokens' K/V rows) into LDS.
  for (int row = slot; row < NROWS; row += 16) {
    uint4 raw = raw0, w8, c8 = c0, s8 = s0;
    if constexpr (FUSED) {
      const int t = row / (G + 2), c = row % (G + 2);
      w8 = c < G ? wq0 : wk0;
      const int64_t pos = pos0 + t;
      const bool pos_ok = pos >= 0 && pos < a.pos_limit;
      if (row != slot) {  // rows past the first (verify): loaded here
        const int hs = c < G ? kvh * G + c : (c == G ? nh + kvh : nh + nkv + kvh);
        raw = *reinterpret_cast<const uint4*>(qsrc + (int64_t)t * qsrc_stride + hs * SOLORT_HD + j * 8);
        c8 = *reinterpret_cast<const uint4*>(rope_cs + t * 64 + (j & 7) * 8);
        s8 = *reinterpret_cast<const uint4*>(rope_cs + (NQ + t) * 64 + (j & 7) * 8);
      }
      if (c == G + 1) {  // V row: raw
        s_new[(NQ + t) * 16 + j] = raw;
        if (split == 0 && pos_ok)
          *reinterpret_cast<uint4*>(vc + row_off<PAGED>(pos, tok_stride, a) + (int64_t)kvh * head_stride + j * 8) = raw;
        continue;
      }
      float cs[8], sn[8];
      unpack8(c8, cs);
      unpack8(s8, sn);
      const uint4 ov = qknorm_rope_row(raw, w8, cs, sn, a.eps, j);
      if (c < G) {
        s_q[(t * G + c) * 16 + j] = ov;
      } else {
        s_new[t * 16 + j] = ov;
        if (split == 0 && pos_ok)
          *reinterpret_cast<uint4*>(kc + row_off<PAGED>(pos, tok_stride, a) + (int64_t)kvh * head_stride + j * 8) = ov;
      }
    } else {
      const int t = row / G, g = row % G;
      if (row != slot)
        raw = *reinterpret_cast<const uint4*>(qsrc + (int64_t)t * qsrc_stride + (kvh * G + g) * SOLORT_HD + j * 8);
      s_q[row * 16 + j] = raw;
    }
  }
  lds_barrier();
  uint4 qb[R];  // this lane's 8 dims of every q row, bf16 pairs
#pragma unroll
  for (int r = 0; r < R; ++r) qb[r] = s_q[r * 16 + j];

  SOLORT_STAMP(tid == 0, kvh + nkv * split, 2);
  // 4. Per iteration: the 16 slots score U keys each (bf16 pair dot products
  //    over the slot's 16 lanes, reduced with DPP) and stage the scores and V
  //    rows in LDS.  Then each wavefront takes the rows it owns (wave + 4i):
  //    lane k evaluates p for key k, the wavefront's p go through its own LDS
  //    row, and each lane accumulates dims 2*lane, 2*lane+1 of the output, so
  //    no per-slot state is merged.
  int64_t live64 = pos0 + NQ;
  live64 = live64 < 0 ? 0 : (live64 > bound ? bound : live64);
  const int kend = min(kstat, (int)live64);
  float M[RPW], Lk[RPW], O[RPW][2];  // Lk: this lane's share of the sum (its keys)
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    M[i] = -INFINITY;
    Lk[i] = 0.f;
    O[i][0] = O[i][1] = 0.f;
  }
  const uint32_t* s_v32 = reinterpret_cast<const uint32_t*>(s_v);
  for (int k0 = kbeg; k0 < kend; k0 += KPI) {
    const int k1 = k0 + KPI;
    uint4 kn[U], vn[U];
    if (k1 < kend) {  // prefetch the next iteration of a long split (block-uniform)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kid = min(k1 + u * 16 + slot, kend - 1);
        const int64_t off = row_off<PAGED>(kid, tok_stride, a);
        kn[u] = ld_stream(kp + off);
        vn[u] = ld_stream(vp + off);
      }
    }
    float part[U * R];  // this lane's share of each score, index u * R + r
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kid = k0 + u * 16 + slot;
      if constexpr (FUSED) {
        const int64_t off = (int64_t)kid - pos0;
        if (off >= 0 && off < NQ) {  // the new tokens' rows: fresh values, not the cache
          kr[u] = s_new[off * 16 + j];
          vr[u] = s_new[(NQ + off) * 16 + j];
        }
      }
      if (kid >= kend) vr[u] = make_uint4(0u, 0u, 0u, 0u);  // p = 0 must not meet a non-finite value
      s_v[(u * 16 + slot) * 16 + j] = vr[u];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = dot2bf(kr[u].x, qb[r].x, 0.f);
        d = dot2bf(kr[u].y, qb[r].y, d);
        d = dot2bf(kr[u].z, qb[r].z, d);
        part[u * R + r] = dot2bf(kr[u].w, qb[r].w, d);
      }
    }
    // Sum the shares over the slot's 16 lanes, eight scores at a time: lane j
    // ends with score c * 8 + j / 2 and the even lanes write them.
#pragma unroll
    for (int c = 0; c < (U * R + 7) / 8; ++c) {
      float v8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v8[i] = c * 8 + i < U * R ? part[c * 8 + i] : 0.f;
      const float sum = row16_reduce8(v8, j);
      const int idx = c * 8 + (j >> 1);
      if ((j & 1) == 0 && idx < U * R) {
        const int u = idx / R, r = idx % R, t = r / G;
        const int kid = k0 + u * 16 + slot;
        s_s[r * KPI + u * 16 + slot] = kid < kend && (int64_t)kid <= pos0 + t ? sum * a.qscale : -INFINITY;
      }
    }
    lds_barrier();
    // Dims 2*lane, 2*lane+1 of every key of the iteration, held in registers
    // when the wave owns one row (re-read from LDS per row otherwise).
    constexpr bool kHoistV = RPW == 1;
    uint32_t v2[kHoistV ? KPI : 1];
    if constexpr (kHoistV) {
#pragma unroll
      for (int k = 0; k < KPI; ++k) v2[k] = s_v32[k * 64 + lane];
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = wave + 4 * i;
      if (r < R) {  // wave-uniform
        float* srow = s_s + r * KPI;
        float sk = -INFINITY;
#pragma unroll
        for (int h = 0; h < KPI; h += 64)
          if (h + lane < KPI) sk = srow[h + lane];  // KPI <= 64: one key per lane
        const float mx = fmaxf(M[i], wave_max(sk));
        if (mx != -INFINITY) {  // wave-uniform
          const float alpha = fast_exp2(M[i] - mx);  // M = -inf gives 0
          const float pk = fast_exp2(sk - mx);       // masked or idle lane: 0
          Lk[i] = Lk[i] * alpha + pk;
          if (lane < KPI) srow[lane] = pk;
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
          const float4* p4 = reinterpret_cast<const float4*>(srow);
          float oa[4] = {O[i][0] * alpha, 0.f, 0.f, 0.f}, ob[4] = {O[i][1] * alpha, 0.f, 0.f, 0.f};
#pragma unroll
          for (int k4 = 0; k4 < KPI / 4; ++k4) {  // four independent accumulator chains per dim
            const float4 p = p4[k4];
            const float pp[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int k = 4 * k4 + e;
              const uint32_t vk = kHoistV ? v2[kHoistV ? k : 0] : s_v32[k * 64 + lane];
              oa[e] = fmaf(pp[e], __uint_as_float(vk << 16), oa[e]);
              ob[e] = fmaf(pp[e], __uint_as_float(vk & 0xffff0000u), ob[e]);
            }
          }
          O[i][0] = (oa[0] + oa[1]) + (oa[2] + oa[3]);
          O[i][1] = (ob[0] + ob[1]) + (ob[2] + ob[3]);
          M[i] = mx;
        }
      }
    }
    lds_barrier();  // s_s and s_v are rewritten by the next iteration
    if (k1 < kend) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        kr[u] = kn[u];
        vr[u] = vn[u];
      }
    }
  }

  SOLORT_STAMP(tid == 0, kvh + nkv * split, 3);
  // 5. One split: the answer; otherwise this split's tagged partial (max,
  //    sum, unnormalised output), merged in this launch or by the combine
  //    kernel.
  const int NS = a.n_split;
  const bool inl = a.merge;
  const unsigned tag = merge_tag(next, kvh);
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = wave + 4 * i;
    if (r >= R) continue;
    const float Ls = wave_sum(Lk[i]);
    const int64_t pr = (int64_t)(kvh * NS + split) * R + r;
    if (NS == 1) {
      const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
      store_out2(a.out, a.out_f32, nh, kvh, G, r, 2 * lane, O[i][0] * inv, O[i][1] * inv);
    } else if (inl) {
      a.ws_o[pr * 64 + lane] = tagged2(O[i][0], O[i][1], tag);
      if (lane == 0) a.ws_ml[pr] = tagged2(M[i], Ls, tag);
    } else {
      st_stream(reinterpret_cast<float2*>(a.ws_o) + pr * 64 + lane, make_float2(O[i][0], O[i][1]));
      if (lane == 0) st_stream(reinterpret_cast<float2*>(a.ws_ml) + pr, make_float2(M[i], Ls));
    }
  }
  SOLORT_STAMP(tid == 0, kvh + nkv * split, 4);
  // s_v (>= 6 KiB) is free: every wave passed the loop's last barrier.
  if (NS > 1 && inl) split_merge<R>(a, kvh, split, NS, nh, G, tag, next, reinterpret_cast<uint8_t*>(s_v));
  SOLORT_STAMP(tid == 0, kvh + nkv * split, 5);
}

// Arguments as the entry points pass them: the leading 14 dwords arrive
// preloaded in SGPRs; kn_w and rope_cs travel in the tail.
template <int NQ, int G, int U, bool FUSED, bool PAGED>
__global__ __launch_bounds__(256) void decode_lanes_kernel(uint16_t* kc, uint16_t* vc, int tok_stride, int head_stride,
                                                     int chunk, int bound, const uint16_t* qsrc, int qsrc_stride,
                                                     int nh, const uint16_t* qn_w, const DecodeTail a) {
  decode_lanes_body<NQ, G, U, FUSED, PAGED>(kc, vc, tok_stride, head_stride, chunk, bound, qsrc, qsrc_stride, nh,
                                            qn_w, a.kn_w, a.rope_cs, a);
}

// One new token, fused, contiguous cache: every pointer the first loads need
// fits the 14 preloaded dwords, so no load waits for the kernel-argument
// fetch.  strides8 = tok_stride / 8 | (head_stride / 8) << 16; geom =
// (chunk / 16 - 1) | nh << 2 | bound << 13 (chunk <= 64, nh < 2048, bound <
// 2^19).  The qkv row stride is not needed for one token.
template <int G, int U>
__global__ __launch_bounds__(256) void decode_lanes_packed_kernel(uint16_t* kc, uint16_t* vc, unsigned strides8,
                                                            unsigned geom, const uint16_t* qkv,
                                                            const uint16_t* qn_w, const uint16_t* kn_w,
                                                            const uint16_t* rope_cs, const DecodeTail a) {
  const int tok_stride = (int)(strides8 & 0xffffu) * 8, head_stride = (int)(strides8 >> 16) * 8;
  const int chunk = ((int)(geom & 3u) + 1) * 16, nh = (int)((geom >> 2) & 2047u), bound = (int)(geom >> 13);
  decode_lanes_body<1, G, U, true, false>(kc, vc, tok_stride, head_stride, chunk, bound, qkv, 0, nh, qn_w, kn_w,
                                          rope_cs, a);
}

// One new token, fused with the qkv product: x [hidden] (the layer input),
// in_w (the input RMSNorm weight) and wqkv [(nh + 2 nkv) * 128][hidden] lead
// the arguments, so the K/V and weight loads issue without waiting for the
// argument fetch; 32 splits per KV head, each computing RW = G + 2 outputs per
// wavefront (hidden = 512 CPL).  strides8 and geom as for the packed kernel.
template <int G, int U, int RW, int CPL>
__global__ __launch_bounds__(256) void decode_qkv_lanes_kernel(uint16_t* kc, uint16_t* vc, unsigned strides8,
                                                         unsigned geom, const uint16_t* x, const uint16_t* wqkv,
                                                         const uint16_t* in_w, const DecodeTail a, const QkvIn q) {
  const int tok_stride = (int)(strides8 & 0xffffu) * 8, head_stride = (int)(strides8 >> 16) * 8;
  const int chunk = ((int)(geom & 3u) + 1) * 16, nh = (int)((geom >> 2) & 2047u), bound = (int)(geom >> 13);
  decode_lanes_body<1, G, U, true, false, RW, CPL>(kc, vc, tok_stride, head_stride, chunk, bound, nullptr, 0, nh,
                                                   q.qn_w, a.kn_w, a.rope_cs, a, x, wqkv, in_w, CPL * 512, &q);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kTile = 32;           // keys per wave per step (one MFMA tile)
constexpr int kQStride = 128 + 8;   // q rows in LDS (bf16): 272 B, conflict-free 16-byte reads
constexpr int kVStride = 128 + 16;  // V tile rows in LDS (bf16): 288 B, conflict-free transposing reads
constexpr int kMergeFloats = 66 * 64;  // one wave's (O, m, l) handed over at the end

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives in slot k
// element i % 4 of the 8 bytes addressed by lane 4k + i / 4 of the group.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)(__attribute__((address_space(3))) uint16_t*)(p));
  return __builtin_bit_cast(uint2, v);
}

// One key tile in flight: lane l holds 16-byte column l%16 of K and V rows
// k0 + l/16 + 4i, i < 8.
struct KVTile {
  uint4 k0, k1, k2, k3, k4, k5, k6, k7, v0, v1, v2, v3, v4, v5, v6, v7;
};

// Loads of the tile at key k0 (k0 past the split: its first rows again, which
// are cached).  Rows are clamped to kclamp, a row the split may read.  NT: the
// non-temporal hint, for one new token (the long decode streams); the several
// tokens of a verify step keep plain loads (measured: 10.45 against 10.6 us
// per layer call with the hint).
template <bool PAGED, bool NT>
__device__ __forceinline__ KVTile fetch_tile(const uint16_t* kp, const uint16_t* vp, int tok_stride, int k0, int kbeg,
                                             int kstat, int kclamp, int lrow, const DecodeTail& a) {
  const int base = k0 < kstat ? k0 : kbeg;
  const bool whole = base + kTile - 1 <= kclamp;  // wave-uniform: no row needs clamping
  const int64_t off0 = (int64_t)(base + lrow) * tok_stride, step = (int64_t)4 * tok_stride;
  KVTile t;
  auto ld = [&](int i, uint4& kd, uint4& vd) {
    int64_t off;
    if constexpr (PAGED)
      off = row_off<true>(min(base + lrow + 4 * i, kclamp), tok_stride, a);
    else
      off = whole ? off0 + i * step : (int64_t)min(base + lrow + 4 * i, kclamp) * tok_stride;
    kd = NT ? ld_stream(kp + off) : *reinterpret_cast<const uint4*>(kp + off);
    vd = NT ? ld_stream(vp + off) : *reinterpret_cast<const uint4*>(vp + off);
  };
  ld(0, t.k0, t.v0); ld(1, t.k1, t.v1); ld(2, t.k2, t.v2); ld(3, t.k3, t.v3);
  ld(4, t.k4, t.v4); ld(5, t.k5, t.v5); ld(6, t.k6, t.v6); ld(7, t.k7, t.v7);
  return t;
}

// Grid (nkv, n_split): block (kvh, split), 4 wavefronts.  qsrc: fused, the
// qkv rows (row stride qsrc_stride); unfused, the q rows [nq][nh][128]
// (qsrc_stride = nh*128).
template <int NQ, int G, bool FUSED, bool PAGED, int RW = 0, int CPL = 0>
__device__ __forceinline__ void decode_mfma_body(uint16_t* kc, uint16_t* vc, int tok_stride, int head_stride,
                                                 int chunk, int bound, const uint16_t* qsrc, int qsrc_stride,
                                                 int nh, const uint16_t* qn_w, const uint16_t* kn_w,
                                                 const uint16_t* rope_cs, const DecodeTail& a,
                                                 const uint16_t* x = nullptr, const uint16_t* wqkv = nullptr,
                                                 const uint16_t* in_w = nullptr, int hidden = 0,
                                                 const QkvIn* qi = nullptr) {
  constexpr bool QKV = RW > 0;  // the qkv rows computed in this launch from x and wqkv (one new token)
  constexpr int R = NQ * G;  // query rows sharing one KV head (<= 32)
  constexpr int NROWS = FUSED ? NQ * (G + 2) : R;
  static_assert(R <= 32, "at most 32 query rows per KV head");
  __shared__ __align__(16) uint16_t s_new[FUSED ? 2 * NQ * 128 : 8];  // fresh K rows, then V rows
  // One region, three uses in turn: the q tile (rows zero past R) until every
  // wave holds its q operand; then each wave's K and V tiles; at the end the
  // waves' (O, m, l) handed over for the merge.
  constexpr int kTileBytes = kTile * (kQStride + kVStride) * 2;  // one wave's K + V tiles
  constexpr int kXBytes = 4 * kMergeFloats * 4 > 4 * kTileBytes ? 4 * kMergeFloats * 4 : 4 * kTileBytes;
  __shared__ __align__(16) uint8_t s_x[kXBytes];
  uint16_t* s_q = reinterpret_cast<uint16_t*>(s_x);

  const int tid = threadIdx.x, j = tid & 15, slot = tid >> 4, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hi = lane >> 5;
  const int kvh = blockIdx.x, split = blockIdx.y;
  const int nkv = nh / G;  // = gridDim.x, without the hidden-argument load
  const int kbeg = min(split * chunk, bound);
  const int kstat = min(kbeg + chunk, bound);
  const int kclamp = kstat > kbeg ? kstat - 1 : (kbeg > 0 ? kbeg - 1 : 0);  // a row this split may read
  SOLORT_STAMP(tid == 0, kvh + nkv * split, 0);

  // 1. Loads for this slot's prologue rows slot, slot + 16, ... (fused: with
  //    the norm weights and each row's token's cos/sin), issued before the K/V
  //    loads: vector loads complete in issue order, so the prologue then waits
  //    for its own rows only.  Every load of phases 1 and 2 is unconditional
  //    (idle lanes load a valid row they ignore): a load skipped on some path
  //    would make the compiler wait for all of them before the first use.
  constexpr int NPASS = (NROWS + 15) / 16;
  static_assert(!QKV || (NQ == 1 && FUSED && !PAGED), "the qkv product in the launch serves one new token");
  uint4 raw[NPASS], cr[NPASS], sr[NPASS];
  uint4 wq0 = make_uint4(0u, 0u, 0u, 0u), wk0 = wq0;
  XChunks xin;  // QKV: this thread's chunks of x and the input norm weight, loaded first
  if constexpr (QKV) gemv_x_load<true>(x, in_w, hidden, xin);
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    const int row = min(slot + 16 * ps, NROWS - 1);
    cr[ps] = sr[ps] = raw[ps] = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (QKV) {
      // loaded behind the weight rows below
    } else if constexpr (FUSED) {
      const int t = row / (G + 2), c = row % (G + 2);
      const int hs = c < G ? kvh * G + c : (c == G ? nh + kvh : nh + nkv + kvh);
      raw[ps] = *reinterpret_cast<const uint4*>(qsrc + (int64_t)t * qsrc_stride + hs * SOLORT_HD + j * 8);
      cr[ps] = *reinterpret_cast<const uint4*>(rope_cs + t * 64 + (j & 7) * 8);
      sr[ps] = *reinterpret_cast<const uint4*>(rope_cs + (NQ + t) * 64 + (j & 7) * 8);
    } else {
      const int t = row / G, g = row % G;
      raw[ps] = *reinterpret_cast<const uint4*>(qsrc + (int64_t)t * qsrc_stride + (kvh * G + g) * SOLORT_HD + j * 8);
    }
  }
  if constexpr (FUSED && !QKV) {
    wq0 = *reinterpret_cast<const uint4*>(qn_w + j * 8);
    wk0 = *reinterpret_cast<const uint4*>(kn_w + j * 8);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the K/V loads

  // 2. This wave's first key tile, at static addresses (before the device-side
  //    position arrives): lane l loads 16-byte column l%16 of key rows
  //    k0 + l/16 + 4i (i < 8) of K and of V, so each load instruction reads
  //    four whole 256-byte rows.  Rows past the split re-read a row of it; a
  //    wave without a tile re-reads the split's first rows (wave 0's, so no
  //    extra traffic reaches HBM).
  const uint16_t* kp = kc + (int64_t)kvh * head_stride + 8 * j;
  const uint16_t* vp = vc + (int64_t)kvh * head_stride + 8 * j;
  const int lrow = lane >> 4;  // this lane's first row of the tile; rows lrow + 4i
  KVTile kv = fetch_tile<PAGED, NQ == 1>(kp, vp, tok_stride, kbeg + kTile * wave, kbeg, kstat, kclamp, lrow, a);

  // QKV: this wave's weight rows, then the prologue's own inputs (as in the lane kernel).
  constexpr int QRW = QKV ? RW : 1, QCPL = QKV ? CPL : 1;
  uint4 wv[QRW][QCPL];
  const int i0 = (split * 4 + wave) * RW;
  if constexpr (QKV) {
    qkv_issue<G, RW, CPL>(wv, wqkv, hidden, i0, kvh, nh, nkv, lane);
    cr[0] = *reinterpret_cast<const uint4*>(rope_cs + (j & 7) * 8);
    sr[0] = *reinterpret_cast<const uint4*>(rope_cs + 64 + (j & 7) * 8);
    wq0 = *reinterpret_cast<const uint4*>(qn_w + j * 8);
    wk0 = *reinterpret_cast<const uint4*>(kn_w + j * 8);
  }
  int64_t pos0;
  unsigned next;
  uint2 posv = make_uint2(0u, 0u);
  unsigned epv = 0u;
  if constexpr (QKV) {  // vector loads, first used after the product (see the lane kernel)
    posv = ld_vec8(a.pos0_dev);
    epv = ld_vec4(a.epochs + kvh * 32);
    pos0 = 0;
    next = 0u;
  } else {
    pos0 = a.pos0_dev[0];
    // The KV head's merge counter, read ahead of the staging barrier (as in the lane kernel: before
    // any partial of the block is stored, and off the path to the partial stores).
    next = a.merge ? merge_next(a.epochs[kvh * 32]) : 0u;
  }
  SOLORT_STAMP(tid == 0, kvh + nkv * split, 1);
  if constexpr (QKV) {
    // x staged past the q tile (the K/V tiles use this region only after the q barriers)
    __shared__ float s_red[4];
    next = merge_next((unsigned)__builtin_amdgcn_readfirstlane((int)epv));
    raw[0] = qkv_handover<G, RW, CPL>(wv, xin, x, in_w, qi->eps, hidden, reinterpret_cast<uint4*>(s_x + 16384), s_red,
                                      qi->items + (int64_t)kvh * (G + 2) * 64, merge_tag(next, kvh), i0,
                                      min(slot, NROWS - 1), j, lane, kStampBlocks);
    pos0 = pos_from(posv);
  }

  // 3. q rows (and, fused, the new tokens' K/V rows) into LDS; rows R..31 of
  //    the q tile are zero.  Fused: every pass's row is normalised first,
  //    without branches (V rows and idle slots too, unused), so the passes'
  //    reduction chains overlap; then the rows are stored.
  if constexpr (FUSED) {
    uint4 ov[NPASS];
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int c = min(slot + 16 * ps, NROWS - 1) % (G + 2);
      float cs[8], sn[8];
      unpack8(cr[ps], cs);
      unpack8(sr[ps], sn);
      ov[ps] = qknorm_rope_row(raw[ps], c < G ? wq0 : wk0, cs, sn, a.eps, j);
    }
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int row = slot + 16 * ps;
      if (row >= NROWS) break;
      const int t = row / (G + 2), c = row % (G + 2);
      const int64_t pos = pos0 + t;
      const bool pos_ok = pos >= 0 && pos < a.pos_limit;
      if (c == G + 1) {  // V row: raw
        *reinterpret_cast<uint4*>(&s_new[(NQ + t) * 128 + j * 8]) = raw[ps];
        if (split == 0 && pos_ok)
          *reinterpret_cast<uint4*>(vc + row_off<PAGED>(pos, tok_stride, a) + (int64_t)kvh * head_stride + j * 8) =
              raw[ps];
      } else if (c < G) {
        *reinterpret_cast<uint4*>(&s_q[(t * G + c) * kQStride + j * 8]) = ov[ps];
      } else {
        *reinterpret_cast<uint4*>(&s_new[t * 128 + j * 8]) = ov[ps];
        if (split == 0 && pos_ok)
          *reinterpret_cast<uint4*>(kc + row_off<PAGED>(pos, tok_stride, a) + (int64_t)kvh * head_stride + j * 8) =
              ov[ps];
      }
    }
  } else {
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int row = slot + 16 * ps;
      if (row >= NROWS) break;
      *reinterpret_cast<uint4*>(&s_q[row * kQStride + j * 8]) = raw[ps];
    }
  }
  for (int i = tid; i < (32 - R) * 16; i += 256)
    *reinterpret_cast<uint4*>(&s_q[(R + (i >> 4)) * kQStride + (i & 15) * 8]) = make_uint4(0u, 0u, 0u, 0u);
  lds_barrier();

  // q^T operand of the eight 16-dim steps: lane l holds row l%32, dims 16kk + 8(l/32) .. +7.
  bf16x8 qb[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    qb[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(&s_q[l32 * kQStride + 16 * kk + 8 * hi]));
  lds_barrier();  // the q tile's space becomes the waves' K/V tiles

  SOLORT_STAMP(tid == 0, kvh + nkv * split, 2);
  // 4. Key tiles k0 = kbeg + 32 wave + 128 i.  Per tile: V into this wave's
  //    LDS tile, S^T = K q^T (8 MFMAs), the next tile's loads, softmax with a
  //    lazy maximum, then O^T += V^T P^T with P split into bf16 high and low
  //    parts (16 MFMAs), which keeps P to ~16 bits.
  int64_t live64 = pos0 + NQ;
  live64 = live64 < 0 ? 0 : (live64 > bound ? bound : live64);
  const int kend = min(kstat, (int)live64);
  const int64_t rowpos = pos0 + (l32 < R ? l32 / G : NQ - 1);  // this lane's query position
  const float qs = a.qscale;
  uint16_t* sk = reinterpret_cast<uint16_t*>(s_x + wave * kTileBytes);  // [32][kQStride] K tile
  uint16_t* sv = sk + kTile * kQStride;                                  // [32][kVStride] V tile
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  float m = -INFINITY, lsum = 0.f;  // reference max (raw score units); this lane's share of the row sum
  for (int k0 = kbeg + kTile * wave; k0 < kend; k0 += 4 * kTile) {
    // Wave-uniform: does the tile hold the new tokens' rows, or rows past the
    // live length, or keys past some query's position?
    const bool has_new = FUSED && (int64_t)k0 <= pos0 + NQ - 1 && (int64_t)(k0 + kTile) > pos0;
    const bool tail = k0 + kTile > kend;
    const bool edge = tail || (int64_t)(k0 + kTile - 1) > pos0;
    auto stage_row = [&](int i, uint4 kd, uint4 vd) {
      const int key = k0 + lrow + 4 * i;
      if (has_new) {  // the new tokens' rows: fresh values, not the cache
        const int64_t off = (int64_t)key - pos0;
        if (off >= 0 && off < NQ) {
          kd = *reinterpret_cast<const uint4*>(&s_new[off * 128 + 8 * j]);
          vd = *reinterpret_cast<const uint4*>(&s_new[(NQ + off) * 128 + 8 * j]);
        }
      }
      if (tail && key >= kend) vd = make_uint4(0u, 0u, 0u, 0u);  // p = 0 must not meet a non-finite value
      *reinterpret_cast<uint4*>(&sk[(lrow + 4 * i) * kQStride + 8 * j]) = kd;
      *reinterpret_cast<uint4*>(&sv[(lrow + 4 * i) * kVStride + 8 * j]) = vd;
    };
    stage_row(0, kv.k0, kv.v0); stage_row(1, kv.k1, kv.v1); stage_row(2, kv.k2, kv.v2); stage_row(3, kv.k3, kv.v3);
    stage_row(4, kv.k4, kv.v4); stage_row(5, kv.k5, kv.v5); stage_row(6, kv.k6, kv.v6); stage_row(7, kv.k7, kv.v7);
    // The next tile, only if the loop takes it (wave-uniform): a load left in flight past the
    // last tile would hold the wave merge below, whose registers it writes.
    if (k0 + 4 * kTile < kend)
      kv = fetch_tile<PAGED, NQ == 1>(kp, vp, tok_stride, k0 + 4 * kTile, kbeg, kstat, kclamp, lrow, a);
    SOLORT_STAMP(lane == 0 && k0 + 4 * kTile < kend && k0 + 8 * kTile >= kend, kvh + nkv * split, 12 + wave);
    f32x16 s = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const uint4 ka = *reinterpret_cast<const uint4*>(&sk[l32 * kQStride + 16 * kk + 8 * hi]);
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ka), qb[kk], s, 0, 0, 0);
    }

    // s[i] is the score of key k0 + 8(i/4) + 4hi + i%4 for query row l%32.
    if (edge) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = k0 + 8 * (i >> 2) + 4 * hi + (i & 3);
        if (key >= kend || (int64_t)key > rowpos) s[i] = -INFINITY;
      }
    }
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
    mx = xor32_combine(mx, [](float x, float y) { return fmaxf(x, y); });
    // Lazy maximum: the reference max moves only when a tile's max exceeds it
    // by more than 8 (log2 units), so p <= 2^8; before a row's first visible
    // key m = -inf and O = 0, l = 0, so it takes the tile's max without a rescale.
    const bool bump = mx * qs > m * qs + 8.f;
    const float mn = bump ? mx : m;
    const float mq = mn == -INFINITY ? 0.f : mn * qs;
    const float alpha = (bump && m != -INFINITY) ? fast_exp2(m * qs - mq) : 1.f;
    float ps = 0.f;
    uint32_t ph[8], pl[8];  // p as bf16 pairs: high parts and the low remainders
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float e0 = fast_exp2(fmaf(s[i], qs, -mq)), e1 = fast_exp2(fmaf(s[i + 1], qs, -mq));
      ps += e0 + e1;
      const uint32_t h2 = pack2(e0, e1);
      ph[i >> 1] = h2;
      pl[i >> 1] = pack2(e0 - __uint_as_float(h2 << 16), e1 - __uint_as_float(h2 & 0xffff0000u));
    }
    lsum = fmaf(lsum, alpha, ps);
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // some row's reference max moved
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
    }
    m = mn;
    // O^T += V^T P^T; key step h covers keys k0 + 16h + {4hi + 0..3, 8 + 4hi + 0..3}.  The V^T
    // operand comes from the row-major tile by transposing reads: lane 16G + jj addresses key
    // row 4(G/2) + jj/4 (+8 for the upper four keys) at dims 16(G%2) + 4(jj%4), so lane l
    // receives dim l%32 of the four keys its P^T slots hold.
    const uint16_t* vb = sv + (4 * hi + ((lane & 15) >> 2)) * kVStride + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bf16x8 pbh = as_bf16x8(make_uint4(ph[4 * h], ph[4 * h + 1], ph[4 * h + 2], ph[4 * h + 3]));
      const bf16x8 pbl = as_bf16x8(make_uint4(pl[4 * h], pl[4 * h + 1], pl[4 * h + 2], pl[4 * h + 3]));
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint16_t* vr8 = vb + 16 * h * kVStride + 32 * dt;
        const uint2 lo = lds_read_tr16(vr8);
        const uint2 up = lds_read_tr16(vr8 + 8 * kVStride);
        const bf16x8 va = as_bf16x8(make_uint4(lo.x, lo.y, up.x, up.y));
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pbh, o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pbl, o[dt], 0, 0, 0);
      }
    }
  }

  SOLORT_STAMP(tid == 0, kvh + nkv * split, 3);
  SOLORT_STAMP(lane == 0, kvh + nkv * split, 8 + wave);
  // 5. Merge the wavefronts that saw keys (log-sum-exp) and write this
  //    split's partial (max in log2 units, sum, unnormalised output) or, with
  //    one split, the answer.  O^T: lane l, register i of o[dt] holds dim
  //    32dt + 8(i/4) + 4(l/32) + i%4 of row l%32.  With one active wave it
  //    writes directly; otherwise every wave hands (O, m, l) over through LDS
  //    and wave w merges and writes dims 32w .. 32w + 31.
  lsum = xor32_combine(lsum, [](float x, float y) { return x + y; });  // both halves of the row
  const int nact = kend > kbeg ? min(4, (kend - kbeg + kTile - 1) / kTile) : 1;  // block-uniform
  f32x16 om;  // the output dims this wave writes: o[wave] (merged) or, alone, all four in turn
  if (nact > 1) {
    __syncthreads();  // every wave is done with its V tile
    float* xf = reinterpret_cast<float*>(s_x);
    float* xw = xf + wave * kMergeFloats;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<float4*>(&xw[(dt * 4 + q4) * 256 + 4 * lane]) =
            make_float4(o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]);
    xw[64 * 64 + lane] = m;
    xw[65 * 64 + lane] = lsum;
    __syncthreads();
    float mw[4], lw[4], mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = w < nact ? xf[w * kMergeFloats + 64 * 64 + lane] : -INFINITY;
      lw[w] = w < nact ? xf[w * kMergeFloats + 65 * 64 + lane] : 0.f;
      mt = fmaxf(mt, mw[w]);
    }
    om = f32x16{};
    lsum = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (w >= nact) break;  // block-uniform
      const float aw = mt == -INFINITY ? 0.f : fast_exp2((mw[w] - mt) * qs);  // -inf gives 0
      lsum = fmaf(lw[w], aw, lsum);
      const float* src = xf + w * kMergeFloats + (wave * 4) * 256 + 4 * lane;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 v = *reinterpret_cast<const float4*>(src + q4 * 256);
        om[4 * q4] = fmaf(v.x, aw, om[4 * q4]);
        om[4 * q4 + 1] = fmaf(v.y, aw, om[4 * q4 + 1]);
        om[4 * q4 + 2] = fmaf(v.z, aw, om[4 * q4 + 2]);
        om[4 * q4 + 3] = fmaf(v.w, aw, om[4 * q4 + 3]);
      }
    }
    m = mt;
  }
  // With one active wave only wave 0 writes; rows past R are padding.
  const bool writer = (nact > 1 || wave == 0) && l32 < R;
  const int NS = a.n_split;
  const bool inl = a.merge;
  const unsigned tag = merge_tag(next, kvh);
  const int r = l32;
  // Writes dims 32dt .. 32dt + 31 of row r (this lane's 16 of them) from od.
  auto write_dims = [&](const f32x16& od, int dt) {
    if (NS == 1) {
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      const int t = r / G, g = r % G;
      const int64_t ob = ((int64_t)t * nh + kvh * G + g) * SOLORT_HD + 4 * hi + 32 * dt;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 v = make_float4(od[4 * q4] * inv, od[4 * q4 + 1] * inv, od[4 * q4 + 2] * inv,
                                     od[4 * q4 + 3] * inv);
        if (a.out_f32) {
          *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + ob + 8 * q4) = v;
        } else {
          uint2 pk;
          pk.x = pack2(v.x, v.y);
          pk.y = pack2(v.z, v.w);
          *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + ob + 8 * q4) = pk;
        }
      }
    } else {
      // dims 32dt + 8q4 + 4hi .. +3: tagged items 16dt + 4q4 + 2hi, +1, or one float4
      uint4* dst = a.ws_o + ((int64_t)(kvh * NS + split) * R + r) * 64 + 16 * dt + 2 * hi;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        if (inl) {
          dst[4 * q4] = tagged2(od[4 * q4], od[4 * q4 + 1], tag);
          dst[4 * q4 + 1] = tagged2(od[4 * q4 + 2], od[4 * q4 + 3], tag);
        } else {
          st_stream(reinterpret_cast<float4*>(a.ws_o) + ((int64_t)(kvh * NS + split) * R + r) * 32 + 8 * dt + 2 * q4 + hi,
                    make_float4(od[4 * q4], od[4 * q4 + 1], od[4 * q4 + 2], od[4 * q4 + 3]));
        }
      }
    }
  };
  if (writer) {
    if (nact > 1) {
      write_dims(om, wave);
    } else {
      write_dims(o[0], 0);
      write_dims(o[1], 1);
      write_dims(o[2], 2);
      write_dims(o[3], 3);
    }
    if (NS > 1 && hi == 0 && (nact == 1 || wave == 0)) {
      const int64_t pr = (int64_t)(kvh * NS + split) * R + r;
      const float mq = m == -INFINITY ? m : m * qs;
      if (inl)
        a.ws_ml[pr] = tagged2(mq, lsum, tag);
      else
        st_stream(reinterpret_cast<float2*>(a.ws_ml) + pr, make_float2(mq, lsum));
    }
  }
  SOLORT_STAMP(tid == 0, kvh + nkv * split, 4);
  // s_x is free: the merge above read it before its last barrier, and the
  // in-launch merge's first barrier comes before any of its LDS writes.
  if (NS > 1 && inl) split_merge<R>(a, kvh, split, NS, nh, G, tag, next, s_x);
  SOLORT_STAMP(tid == 0, kvh + nkv * split, 5);
}

// Arguments as the entry points pass them: the leading 14 dwords arrive
// preloaded in SGPRs; kn_w and rope_cs travel in the tail.
template <int NQ, int G, bool FUSED, bool PAGED>
__global__ __launch_bounds__(256, 2) void decode_mfma_kernel(uint16_t* kc, uint16_t* vc, int tok_stride, int head_stride,
                                                        int chunk, int bound, const uint16_t* qsrc, int qsrc_stride,
                                                        int nh, const uint16_t* qn_w, const DecodeTail a) {
  decode_mfma_body<NQ, G, FUSED, PAGED>(kc, vc, tok_stride, head_stride, chunk, bound, qsrc, qsrc_stride, nh, qn_w,
                                        a.kn_w, a.rope_cs, a);
}

// Fused, contiguous cache, packed qkv rows: every pointer the first loads
// need fits the 14 preloaded dwords.  strides8 = tok_stride / 8 |
// (head_stride / 8) << 16; geom = (chunk / 32 - 1) | nh << 5 | bound << 16
// (chunk <= 1024, nh < 2048, bound < 2^16); the qkv row stride is
// (nh + 2 nkv) * 128.
template <int NQ, int G>
__global__ __launch_bounds__(256, 2) void decode_mfma_packed_kernel(uint16_t* kc, uint16_t* vc, unsigned strides8,
                                                               unsigned geom, const uint16_t* qkv,
                                                               const uint16_t* qn_w, const uint16_t* kn_w,
                                                               const uint16_t* rope_cs, const DecodeTail a) {
  const int tok_stride = (int)(strides8 & 0xffffu) * 8, head_stride = (int)(strides8 >> 16) * 8;
  const int chunk = ((int)(geom & 31u) + 1) * 32, nh = (int)((geom >> 5) & 2047u), bound = (int)(geom >> 16);
  decode_mfma_body<NQ, G, true, false>(kc, vc, tok_stride, head_stride, chunk, bound, qkv,
                                       (nh + 2 * (nh / G)) * SOLORT_HD, nh, qn_w, kn_w, rope_cs, a);
}

// One new token, fused with the qkv product (see decode_qkv_lanes_kernel); the
// geometry holds key chunks of 128 to 1024 keys, launch_qkv routes 128-key
// chunks here; strides8 and geom as for the packed MFMA kernel.  One block per
// CU: the weight rows in flight need the registers.
template <int G, int RW, int CPL>
__global__ __launch_bounds__(256, 1) void decode_qkv_mfma_kernel(uint16_t* kc, uint16_t* vc, unsigned strides8,
                                                                 unsigned geom, const uint16_t* x,
                                                                 const uint16_t* wqkv, const uint16_t* in_w,
                                                                 const DecodeTail a, const QkvIn q) {
  const int tok_stride = (int)(strides8 & 0xffffu) * 8, head_stride = (int)(strides8 >> 16) * 8;
  const int chunk = ((int)(geom & 31u) + 1) * 32, nh = (int)((geom >> 5) & 2047u), bound = (int)(geom >> 16);
  decode_mfma_body<1, G, true, false, RW, CPL>(kc, vc, tok_stride, head_stride, chunk, bound, nullptr, 0, nh, q.qn_w,
                                               a.kn_w, a.rope_cs, a, x, wqkv, in_w, CPL * 512, &q);
}

// The combine kernel (two-launch mode): the log-sum-exp combine of the
// n_split untagged partials of each KV head.  Grid (nkv, column blocks): block = (KV
// head, 32 float4 columns of its [R][128] output); thread = (column, split
// group sg of 8): it merges splits sg, sg+8, ... on its own, kCombB at a time
// (all loads of a batch issued together), then the 8 split groups meet once
// in LDS.  Every argument is preloaded.
template <int NQ, int G>
__global__ __launch_bounds__(256) void combine_kernel(const uint4* ws_o, const uint4* ws_ml, void* out, int nh,
                                                      int n_split, int out_f32) {
  constexpr int R = NQ * G;
  constexpr int C = R * 32;  // float4 columns
  __shared__ float s_m[8 * 32], s_l[8 * 32];
  __shared__ float4 s_o[8 * 32];
  const int tid = threadIdx.x, c = tid & 31, sg = tid >> 5;
  const int kvh = blockIdx.x, cb = blockIdx.y;
  const int col = cb * 32 + c;
  const bool act = col < C;
  const int r = col >> 5;
  const int NS = n_split;
  const float2* wml = reinterpret_cast<const float2*>(ws_ml) + (int64_t)kvh * NS * R;
  const float4* wo = reinterpret_cast<const float4*>(ws_o) + (int64_t)kvh * NS * C;
  CombAcc acc = comb_init();
  for (int s0 = sg; s0 < NS; s0 += 8 * kCombB) {
    float2 ml[kCombB];
    float4 ov[kCombB];
#pragma unroll
    for (int k = 0; k < kCombB; ++k) {
      const int s = s0 + 8 * k;
      if (act && s < NS) {
        ml[k] = wml[(int64_t)s * R + r];
        ov[k] = wo[(int64_t)s * C + col];
      } else {
        ml[k] = make_float2(-INFINITY, 0.f);
        ov[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    comb_merge<kCombB>(acc, ml, ov);
  }
  s_m[sg * 32 + c] = acc.m;
  s_l[sg * 32 + c] = acc.l;
  s_o[sg * 32 + c] = acc.o;
  __syncthreads();
  if (tid < 32 && act) store_out(out, out_f32, nh, kvh, G, col, comb_final(s_m, s_l, s_o, 32, c));
}

// ---------------------------------------------------------------- host side

constexpr int kMaxRows = 32;       // nq * group limit: one MFMA tile of query rows
constexpr int kLanesMaxGroup = 8;  // the lane-parallel kernel serves one token of up to 8 query heads
constexpr int kLanesMaxChunk = 64;  // ... and key chunks of at most 64 rows (4 per slot)
constexpr int kMaxSplit = 1024;

// Everything a launch needs, gathered by prepare() and the entry points.
struct DecodeArgs {
  uint16_t* kc;
  uint16_t* vc;
  int tok_stride, head_stride, chunk, bound;
  const uint16_t* qsrc;
  int qsrc_stride, nh, nkv, n_split;
  const uint16_t* qn_w;
  bool lanes;  // the lane-parallel kernel (short chunks, one new token), else the MFMA kernel
  bool paged;  // K/V rows through the page table in tail
  int U;       // key rows per slot per step of the lane-parallel kernel
  DecodeTail tail;

  dim3 grid() const { return dim3(nkv, n_split); }
};

// Workspace: the per-KV-head launch counters of the in-launch merge (128
// bytes per head, for up to kMergeHeads heads, at a fixed offset so that
// calls of any shape sharing a workspace agree on them), then the splits'
// tagged (max, sum) items and output items.
constexpr size_t kCounterBytes = (size_t)kMergeHeads * 128;

struct WsLayout {
  size_t ml_off, o_off, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static WsLayout ws_layout(int nq, int nh, int nkv, int n_split) {
  const size_t R = (size_t)nq * (nh / nkv);
  WsLayout w;
  w.ml_off = kCounterBytes;
  w.o_off = align256(w.ml_off + (size_t)nkv * n_split * R * 16);
  w.total = align256(w.o_off + (size_t)nkv * n_split * R * 64 * 16);
  return w;
}

// In-launch merge, per device: on once solort_init has checked the workgroup
// placement (probe.hip), unless switched off by solort_combine_mode.
namespace {
constexpr int kMaxDev = 64;
int g_combine_off[kMaxDev];
}  // namespace

// The in-launch merge needs every split of a head on one XCD (nkv a multiple
// of 8, round-robin placement) and at most kMergeMaxSplit splits (one batch
// of loads per polling round).  A merging block waits for blocks dispatched
// before it and for the head's other merging blocks; at most 256 merging
// blocks in all (one per CU) keeps the blocks they wait for from being held
// back by blocks that wait.  It is used for at most kMergeMaxRows query rows
// per KV head: its partials carry a tag per value (twice the bytes), which
// the merge saving pays for only while they are few.  Measured on MI355X,
// one call, graph of 288 calls on distinct caches: Qwen3-4B decode at KV
// 1024 (4 rows, 32 splits) 5.68 us in-launch against 5.91 us two-launch;
// Qwen3-8B at KV 32768 (4 rows, 32 splits of 1024 keys) 32.7 against 32.9;
// a 5-token verify at 4096 (20 rows, 32 splits) 10.90 against 10.55.
constexpr int kMergeMaxRows = 8;

static bool merge_ok(int rows, int n_split, int nkv) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return false;
  return !g_combine_off[dev] && xcd_round_robin(dev) && n_split > 1 && n_split <= kMergeMaxSplit && nkv % 8 == 0 &&
         nkv <= kMergeHeads && rows <= kMergeMaxRows && nkv * (n_split < rows ? n_split : rows) <= 256;
}

template <int NQ, int G, bool FUSED, bool PAGED>
static bool launch_split_p(const DecodeArgs& a, hipStream_t s) {
  if constexpr (NQ * G <= kMaxRows) {
    const dim3 grid = a.grid();
    if constexpr (NQ == 1 && G <= kLanesMaxGroup) {
      if constexpr (FUSED && !PAGED) {
        // The packed-argument kernel when the layout fits its fields.
        if (a.lanes && a.tok_stride < (1 << 19) && a.head_stride < (1 << 19) && a.nh < 2048 && a.bound < (1 << 19)) {
          const unsigned strides8 = (unsigned)(a.tok_stride / 8) | (unsigned)(a.head_stride / 8) << 16;
          const unsigned geom = (unsigned)(a.chunk / 16 - 1) | (unsigned)a.nh << 2 | (unsigned)a.bound << 13;
          if (a.U == 4)
            hipLaunchKernelGGL((decode_lanes_packed_kernel<G, 4>), grid, dim3(256), 0, s, a.kc, a.vc, strides8, geom,
                               a.qsrc, a.qn_w, a.tail.kn_w, a.tail.rope_cs, a.tail);
          else if (a.U == 2)
            hipLaunchKernelGGL((decode_lanes_packed_kernel<G, 2>), grid, dim3(256), 0, s, a.kc, a.vc, strides8, geom,
                               a.qsrc, a.qn_w, a.tail.kn_w, a.tail.rope_cs, a.tail);
          else
            hipLaunchKernelGGL((decode_lanes_packed_kernel<G, 1>), grid, dim3(256), 0, s, a.kc, a.vc, strides8, geom,
                               a.qsrc, a.qn_w, a.tail.kn_w, a.tail.rope_cs, a.tail);
          return true;
        }
      }
      if (a.lanes) {
        if (a.U == 4)
          hipLaunchKernelGGL((decode_lanes_kernel<NQ, G, 4, FUSED, PAGED>), grid, dim3(256), 0, s, a.kc, a.vc,
                             a.tok_stride, a.head_stride, a.chunk, a.bound, a.qsrc, a.qsrc_stride, a.nh, a.qn_w,
                             a.tail);
        else if (a.U == 2)
          hipLaunchKernelGGL((decode_lanes_kernel<NQ, G, 2, FUSED, PAGED>), grid, dim3(256), 0, s, a.kc, a.vc,
                             a.tok_stride, a.head_stride, a.chunk, a.bound, a.qsrc, a.qsrc_stride, a.nh, a.qn_w,
                             a.tail);
        else
          hipLaunchKernelGGL((decode_lanes_kernel<NQ, G, 1, FUSED, PAGED>), grid, dim3(256), 0, s, a.kc, a.vc,
                             a.tok_stride, a.head_stride, a.chunk, a.bound, a.qsrc, a.qsrc_stride, a.nh, a.qn_w,
                             a.tail);
        return true;
      }
    }
    if constexpr (FUSED && !PAGED) {
      // The packed-argument kernel when the layout fits its fields.
      if (a.tok_stride < (1 << 19) && a.head_stride < (1 << 19) && a.nh < 2048 && a.bound < (1 << 16) &&
          a.chunk <= 1024 && a.qsrc_stride == (a.nh + 2 * a.nkv) * SOLORT_HD) {
        const unsigned strides8 = (unsigned)(a.tok_stride / 8) | (unsigned)(a.head_stride / 8) << 16;
        const unsigned geom = (unsigned)(a.chunk / 32 - 1) | (unsigned)a.nh << 5 | (unsigned)a.bound << 16;
        hipLaunchKernelGGL((decode_mfma_packed_kernel<NQ, G>), grid, dim3(256), 0, s, a.kc, a.vc, strides8, geom,
                           a.qsrc, a.qn_w, a.tail.kn_w, a.tail.rope_cs, a.tail);
        return true;
      }
    }
    hipLaunchKernelGGL((decode_mfma_kernel<NQ, G, FUSED, PAGED>), grid, dim3(256), 0, s, a.kc, a.vc, a.tok_stride,
                       a.head_stride, a.chunk, a.bound, a.qsrc, a.qsrc_stride, a.nh, a.qn_w, a.tail);
    return true;
  } else {
    return false;
  }
}

// The paged cache is served by the fused layer entry point only.
template <int NQ, int G, bool FUSED>
static bool launch_split(const DecodeArgs& a, hipStream_t s) {
  if constexpr (FUSED) {
    if (a.paged) return launch_split_p<NQ, G, true, true>(a, s);
  }
  return launch_split_p<NQ, G, FUSED, false>(a, s);
}

template <int NQ, int G>
static bool launch_combine(const DecodeArgs& a, hipStream_t s) {
  if constexpr (NQ * G <= kMaxRows) {
    constexpr int C = NQ * G * 32;  // float4 columns per KV head
    hipLaunchKernelGGL((combine_kernel<NQ, G>), dim3(a.nkv, (C + 31) / 32), dim3(256), 0, s, a.tail.ws_o,
                       a.tail.ws_ml, a.tail.out, a.nh, a.n_split, a.tail.out_f32);
    return true;
  } else {
    return false;
  }
}

// Dispatches on nq to FN<NQ, G>(args...).
#define SOLORT_DISPATCH_NQ(G, FN, ...)    \
  switch (nq) {                           \
    case 1: return FN<1, G>(__VA_ARGS__); \
    case 2: return FN<2, G>(__VA_ARGS__); \
    case 3: return FN<3, G>(__VA_ARGS__); \
    case 4: return FN<4, G>(__VA_ARGS__); \
    case 5: return FN<5, G>(__VA_ARGS__); \
    case 6: return FN<6, G>(__VA_ARGS__); \
    case 7: return FN<7, G>(__VA_ARGS__); \
    case 8: return FN<8, G>(__VA_ARGS__); \
  }                                       \
  return false;

template <int NQ, int G>
static bool launch_attn(bool fused, const DecodeArgs& a, hipStream_t s) {
  return fused ? launch_split<NQ, G, true>(a, s) : launch_split<NQ, G, false>(a, s);
}

template <int G>
static bool attn_nq(int nq, bool fused, const DecodeArgs& a, hipStream_t s) {
  SOLORT_DISPATCH_NQ(G, launch_attn, fused, a, s)
}

template <int G>
static bool combine_nq(int nq, const DecodeArgs& a, hipStream_t s) {
  SOLORT_DISPATCH_NQ(G, launch_combine, a, s)
}

static bool dispatch_attn(int G, int nq, bool fused, const DecodeArgs& a, hipStream_t s) {
  switch (G) {
    case 1: return attn_nq<1>(nq, fused, a, s);
    case 2: return attn_nq<2>(nq, fused, a, s);
    case 4: return attn_nq<4>(nq, fused, a, s);
    case 8: return attn_nq<8>(nq, fused, a, s);
  }
  return false;
}

static bool dispatch_combine(int G, int nq, const DecodeArgs& a, hipStream_t s) {
  switch (G) {
    case 1: return combine_nq<1>(nq, a, s);
    case 2: return combine_nq<2>(nq, a, s);
    case 4: return combine_nq<4>(nq, a, s);
    case 8: return combine_nq<8>(nq, a, s);
  }
  return false;
}

constexpr int64_t kMaxI32 = 0x7fffffff;

// Checks shared by every attention entry point; fills the attention part of `a`.
static int prepare(const char* name, int nq, int nh, int nkv, int hd, void* k_cache, void* v_cache,
                   int64_t kv_tok_stride, int64_t kv_head_stride, int64_t max_len,
                   const int64_t* pos0_dev, int bound, float scale, void* ws, int n_split, void* out,
                   int out_dtype, DecodeArgs& a) {
  if (hd != SOLORT_HD) return set_error(SOLORT_EINVAL, "%s: head_dim %d != 128", name, hd);
  if (nh <= 0 || nkv <= 0 || nh % nkv != 0)
    return set_error(SOLORT_EINVAL, "%s: nh=%d must be a positive multiple of nkv=%d", name, nh, nkv);
  const int G = nh / nkv;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return set_error(SOLORT_EINVAL, "%s: query group %d not in {1,2,4,8}", name, G);
  if (nq < 1 || nq > 8 || nq * G > kMaxRows)
    return set_error(SOLORT_EINVAL, "%s: nq=%d with group %d exceeds %d query rows", name, nq, G, kMaxRows);
  if (!k_cache || !v_cache || !pos0_dev || !ws || !out)
    return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(ws) || !aligned16(out))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (kv_tok_stride <= 0 || kv_head_stride <= 0 || kv_tok_stride % 8 || kv_head_stride % 8 ||
      kv_tok_stride > kMaxI32 || kv_head_stride > kMaxI32)
    return set_error(SOLORT_EINVAL, "%s: KV strides must be positive multiples of 8 below 2^31", name);
  if (max_len < 1 || max_len > kMaxI32)
    return set_error(SOLORT_EINVAL, "%s: max_len %lld outside [1, 2^31)", name, (long long)max_len);
  if (bound < 1 || bound > max_len || bound > (1 << 30))
    return set_error(SOLORT_EINVAL, "%s: bound %d outside [1, max_len=%lld]", name, bound, (long long)max_len);
  if (n_split < 1 || n_split > kMaxSplit)
    return set_error(SOLORT_EINVAL, "%s: n_split %d outside [1, %d]", name, n_split, kMaxSplit);
  if (out_dtype != SOLORT_DTYPE_BF16 && out_dtype != SOLORT_DTYPE_F32)
    return set_error(SOLORT_EINVAL, "%s: out_dtype %d", name, out_dtype);
  const WsLayout w = ws_layout(nq, nh, nkv, n_split);
  a.kc = (uint16_t*)k_cache;
  a.vc = (uint16_t*)v_cache;
  a.tok_stride = (int)kv_tok_stride;
  a.head_stride = (int)kv_head_stride;
  // Short chunks of one new token are latency-bound: the lane-parallel kernel
  // (chunk a multiple of 16 keys).  Longer chunks and several new tokens: the
  // MFMA kernel (chunk a multiple of its 32-key tile).
  const int raw_chunk = (bound + n_split - 1) / n_split;
  a.lanes = nq == 1 && G <= kLanesMaxGroup && raw_chunk <= kLanesMaxChunk;
  const int gran = a.lanes ? 16 : kTile;
  a.chunk = ((raw_chunk + gran - 1) / gran) * gran;  // static key chunk per split
  a.U = a.chunk >= 64 ? 4 : (a.chunk >= 32 ? 2 : 1);
  a.bound = bound;
  a.nh = nh;
  a.nkv = nkv;
  // Trailing splits without keys are dropped: they add nothing to the combine.
  a.n_split = (bound + a.chunk - 1) / a.chunk;
  a.tail.pos0_dev = pos0_dev;
  a.tail.ws_o = (uint4*)((char*)ws + w.o_off);
  a.tail.ws_ml = (uint4*)((char*)ws + w.ml_off);
  a.tail.epochs = (unsigned*)ws;
  a.tail.n_split = a.n_split;
  a.tail.merge = merge_ok(nq * G, a.n_split, nkv) ? 1 : 0;
  a.tail.out = out;
  a.tail.qscale = scale * 1.4426950408889634f;
  a.tail.pos_limit = (int)max_len;
  a.tail.out_f32 = out_dtype == SOLORT_DTYPE_F32;
  return 0;
}

// Launches the split kernel, then (more than one split) the combine kernel.
static int launch_all(const char* name, bool fused, int nq, const DecodeArgs& a, hipStream_t s) {
  const int G = a.nh / a.nkv;
  if (!dispatch_attn(G, nq, fused, a, s))
    return set_error(SOLORT_EINVAL, "%s: no kernel for nq=%d group=%d", name, nq, G);
  int rc = check_launch(name);
  if (rc || a.n_split == 1 || a.tail.merge) return rc;
  if (!dispatch_combine(G, nq, a, s))
    return set_error(SOLORT_EINVAL, "%s: no combine kernel for nq=%d group=%d", name, nq, G);
  return check_launch(name);
}

static int attn_impl(const char* name, const void* q, int nq, int nh, int nkv, int hd,
                     const void* k_cache, const void* v_cache, int64_t kv_tok_stride,
                     int64_t kv_head_stride, int64_t max_len, const int64_t* pos0_dev, int bound,
                     float scale, void* ws, int n_split, void* out, int out_dtype,
                     solort_stream_t stream) {
  DecodeArgs a = {};
  int rc = prepare(name, nq, nh, nkv, hd, (void*)k_cache, (void*)v_cache, kv_tok_stride, kv_head_stride,
                   max_len, pos0_dev, bound, scale, ws, n_split, out, out_dtype, a);
  if (rc) return rc;
  if (!q || !aligned16(q)) return set_error(SOLORT_EINVAL, "%s: q must be a 16-byte aligned pointer", name);
  a.qsrc = (const uint16_t*)q;
  a.qsrc_stride = nh * SOLORT_HD;
  return launch_all(name, false, nq, a, (hipStream_t)stream);
}

// The fused qkv + attention launch: one new token, packed layout, the
// lane-parallel kernel at 32 splits per KV head with the in-launch merge, and
// a (group, hidden) pair the kernel is built for.  Returns false when any
// condition fails (the caller then runs the product as its own launch).
constexpr int kQkvSplits = 32;

static size_t qkv_items_bytes(int nh, int nkv) { return align256((size_t)nkv * (nh / nkv + 2) * 64 * 8); }

template <int G, int RW, int CPL>
static void launch_qkv_u(const DecodeArgs& a, unsigned strides8, unsigned geom, const void* x, const void* wqkv,
                         const void* in_w, const QkvIn& q, hipStream_t s) {
  const dim3 grid = a.grid();
  if (a.U == 4)
    hipLaunchKernelGGL((decode_qkv_lanes_kernel<G, 4, RW, CPL>), grid, dim3(256), 0, s, a.kc, a.vc, strides8, geom,
                       (const uint16_t*)x, (const uint16_t*)wqkv, (const uint16_t*)in_w, a.tail, q);
  else if (a.U == 2)
    hipLaunchKernelGGL((decode_qkv_lanes_kernel<G, 2, RW, CPL>), grid, dim3(256), 0, s, a.kc, a.vc, strides8, geom,
                       (const uint16_t*)x, (const uint16_t*)wqkv, (const uint16_t*)in_w, a.tail, q);
  else
    hipLaunchKernelGGL((decode_qkv_lanes_kernel<G, 1, RW, CPL>), grid, dim3(256), 0, s, a.kc, a.vc, strides8, geom,
                       (const uint16_t*)x, (const uint16_t*)wqkv, (const uint16_t*)in_w, a.tail, q);
}

template <int G, int RW, int CPL>
static void launch_qkv_mfma(const DecodeArgs& a, unsigned strides8, const void* x, const void* wqkv, const void* in_w,
                            const QkvIn& q, hipStream_t s) {
  const unsigned geom = (unsigned)(a.chunk / 32 - 1) | (unsigned)a.nh << 5 | (unsigned)a.bound << 16;
  hipLaunchKernelGGL((decode_qkv_mfma_kernel<G, RW, CPL>), a.grid(), dim3(256), 0, s, a.kc, a.vc, strides8, geom,
                     (const uint16_t*)x, (const uint16_t*)wqkv, (const uint16_t*)in_w, a.tail, q);
}

static bool launch_qkv(const DecodeArgs& a, int hidden, const void* x, const void* wqkv, const void* in_w,
                       const QkvIn& q, hipStream_t s) {
  const int G = a.nh / a.nkv;
  if (a.n_split != kQkvSplits || !a.tail.merge || a.tok_stride >= (1 << 19) || a.head_stride >= (1 << 19) ||
      a.nh >= 2048 || a.bound >= (1 << 19))
    return false;
  const unsigned strides8 = (unsigned)(a.tok_stride / 8) | (unsigned)(a.head_stride / 8) << 16;
  if (!a.lanes) {
    // MFMA split kernel, 128-key chunks.  Its geometry holds chunks up to 1024 keys, but from 256 on
    // the two launches were as fast or faster (Qwen3-4B, us per layer: KV 4096 17.19 against 17.30,
    // KV 8192 20.62 against 20.25): a wavefront holds one key tile before the product, and the
    // chunk's later tiles are loaded after the handover.
    if (a.chunk > 128 || a.bound >= (1 << 16)) return false;
    if (G == 2 && hidden == 1024) {
      launch_qkv_mfma<2, 4, 2>(a, strides8, x, wqkv, in_w, q, s);
    } else if (G == 4 && hidden == 2560) {
      launch_qkv_mfma<4, 6, 5>(a, strides8, x, wqkv, in_w, q, s);
    } else if (G == 4 && hidden == 4096) {
      launch_qkv_mfma<4, 6, 8>(a, strides8, x, wqkv, in_w, q, s);
    } else {
      return false;
    }
    return true;
  }
  const unsigned geom = (unsigned)(a.chunk / 16 - 1) | (unsigned)a.nh << 2 | (unsigned)a.bound << 13;
  if (G == 2 && hidden == 1024) {
    launch_qkv_u<2, 4, 2>(a, strides8, geom, x, wqkv, in_w, q, s);
  } else if (G == 4 && hidden == 2560) {
    launch_qkv_u<4, 6, 5>(a, strides8, geom, x, wqkv, in_w, q, s);
  } else if (G == 4 && hidden == 4096) {
    launch_qkv_u<4, 6, 8>(a, strides8, geom, x, wqkv, in_w, q, s);
  } else {
    return false;
  }
  return true;
}

}  // namespace solort

using namespace solort;

extern "C" int solort_combine_mode(int mode) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev)
    return set_error(SOLORT_EINVAL, "combine_mode: no current device");
  if (mode != -1 && mode != 0 && mode != 1) return set_error(SOLORT_EINVAL, "combine_mode: mode %d", mode);
  if (mode >= 0) g_combine_off[dev] = mode == 0;
  return !g_combine_off[dev] && xcd_round_robin(dev) ? 1 : 0;
}

extern "C" size_t solort_attn_workspace_bytes(int nq, int nh, int nkv, int hd, int n_split) {
  if (nq < 1 || nh <= 0 || nkv <= 0 || nh % nkv || hd != SOLORT_HD || n_split < 1) return 0;
  return ws_layout(nq, nh, nkv, n_split).total;
}

extern "C" int solort_decode_attn(const void* q, int nq, int nh, int nkv, int hd, const void* k_cache,
                                  const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                                  int64_t max_len, const int64_t* pos0_dev, int bound, float scale,
                                  void* ws, int n_split, void* out, int out_dtype,
                                  solort_stream_t stream) {
  return attn_impl("decode_attn", q, nq, nh, nkv, hd, k_cache, v_cache, kv_tok_stride, kv_head_stride,
                   max_len, pos0_dev, bound, scale, ws, n_split, out, out_dtype, stream);
}

extern "C" int solort_verify_attn(const void* q, int nq, int nh, int nkv, int hd, const void* k_cache,
                                  const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                                  int64_t max_len, const int64_t* pos0_dev, int bound, float scale,
                                  void* ws, int n_split, void* out, int out_dtype,
                                  solort_stream_t stream) {
  return attn_impl("verify_attn", q, nq, nh, nkv, hd, k_cache, v_cache, kv_tok_stride, kv_head_stride,
                   max_len, pos0_dev, bound, scale, ws, n_split, out, out_dtype, stream);
}

extern "C" int solort_decode_layer(const void* qkv, int64_t qkv_row_stride, int nq, int nh, int nkv, int hd,
                                   const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                                   const int64_t* pos0_dev, void* k_cache, void* v_cache, int64_t kv_tok_stride,
                                   int64_t kv_head_stride, int64_t max_len, int bound, float scale, void* ws,
                                   int n_split, void* out, int out_dtype, solort_stream_t stream) {
  const char* name = "decode_layer";
  DecodeArgs a = {};
  int rc = prepare(name, nq, nh, nkv, hd, k_cache, v_cache, kv_tok_stride, kv_head_stride, max_len, pos0_dev,
                   bound, scale, ws, n_split, out, out_dtype, a);
  if (rc) return rc;
  if (!qkv || !qn_w || !kn_w || !rope_cs) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(qkv) || !aligned16(qn_w) || !aligned16(kn_w) || !aligned16(rope_cs))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (qkv_row_stride < (int64_t)(nh + 2 * nkv) * hd || qkv_row_stride % 8 != 0 || qkv_row_stride > kMaxI32)
    return set_error(SOLORT_EINVAL, "%s: qkv_row_stride %lld", name, (long long)qkv_row_stride);
  a.qsrc = (const uint16_t*)qkv;
  a.qsrc_stride = (int)qkv_row_stride;
  a.qn_w = (const uint16_t*)qn_w;
  a.tail.kn_w = (const uint16_t*)kn_w;
  a.tail.rope_cs = (const uint16_t*)rope_cs;
  a.tail.eps = eps;
  return launch_all(name, true, nq, a, (hipStream_t)stream);
}

extern "C" size_t solort_decode_qkv_workspace_bytes(int nh, int nkv, int n_split) {
  if (nh <= 0 || nkv <= 0 || nh % nkv || n_split < 1) return 0;
  return ws_layout(1, nh, nkv, n_split).total + qkv_items_bytes(nh, nkv);
}

extern "C" int solort_decode_qkv_layer(const void* x, int hidden, const void* in_w, float in_eps, const void* wqkv,
                                       int64_t wqkv_row_stride, int nh, int nkv, int hd, const void* qn_w,
                                       const void* kn_w, float eps, const void* rope_cs, const int64_t* pos0_dev,
                                       void* k_cache, void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                                       int64_t max_len, int bound, float scale, void* ws, int n_split, void* qkv_out,
                                       void* out, int out_dtype, solort_stream_t stream) {
  const char* name = "decode_qkv_layer";
  DecodeArgs a = {};
  int rc = prepare(name, 1, nh, nkv, hd, k_cache, v_cache, kv_tok_stride, kv_head_stride, max_len, pos0_dev, bound,
                   scale, ws, n_split, out, out_dtype, a);
  if (rc) return rc;
  if (!x || !in_w || !wqkv || !qn_w || !kn_w || !rope_cs || !qkv_out)
    return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(x) || !aligned16(in_w) || !aligned16(wqkv) || !aligned16(qn_w) || !aligned16(kn_w) ||
      !aligned16(rope_cs) || !aligned16(qkv_out))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (hidden < 8 || hidden % 8 || hidden > 65536 || wqkv_row_stride < hidden || wqkv_row_stride % 8 ||
      wqkv_row_stride > kMaxI32)
    return set_error(SOLORT_EINVAL, "%s: hidden %d, wqkv_row_stride %lld", name, hidden, (long long)wqkv_row_stride);
  a.qn_w = (const uint16_t*)qn_w;
  a.tail.kn_w = (const uint16_t*)kn_w;
  a.tail.rope_cs = (const uint16_t*)rope_cs;
  a.tail.eps = eps;
  QkvIn q;
  q.qn_w = (const uint16_t*)qn_w;
  q.items = (uint2*)((char*)ws + ws_layout(1, nh, nkv, n_split).total);
  q.eps = in_eps;
  if (wqkv_row_stride == hidden && launch_qkv(a, hidden, x, wqkv, in_w, q, (hipStream_t)stream))
    return check_launch(name);
  // Otherwise the product as its own launch, then the attention block on its output.
  const int width = (nh + 2 * nkv) * hd;
  rc = solort_gemv(wqkv, wqkv_row_stride, width, hidden, x, in_w, in_eps, nullptr, SOLORT_GEMV_PLAIN, 0, qkv_out,
                   stream);
  if (rc) return rc;
  a.qsrc = (const uint16_t*)qkv_out;
  a.qsrc_stride = width;
  return launch_all(name, true, 1, a, (hipStream_t)stream);
}

extern "C" int solort_paged_decode_layer(const void* qkv, int64_t qkv_row_stride, int nq, int nh, int nkv, int hd,
                                         const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                                         const int64_t* pos0_dev, void* k_pages, void* v_pages, int64_t page_stride,
                                         int64_t kv_tok_stride, int64_t kv_head_stride, int page_size,
                                         int num_pages, const int32_t* page_table, int table_len, int bound,
                                         float scale, void* ws, int n_split, void* out, int out_dtype,
                                         solort_stream_t stream) {
  const char* name = "paged_decode_layer";
  if (page_size < 1 || page_size > (1 << 20) || (page_size & (page_size - 1)))
    return set_error(SOLORT_EINVAL, "%s: page_size %d must be a power of two up to 2^20", name, page_size);
  if (num_pages < 1 || table_len < 1 || (int64_t)table_len * page_size > kMaxI32)
    return set_error(SOLORT_EINVAL, "%s: num_pages=%d table_len=%d page_size=%d", name, num_pages, table_len,
                     page_size);
  if (!page_table || ((uintptr_t)page_table & 3u))
    return set_error(SOLORT_EINVAL, "%s: page_table must be a 4-byte aligned pointer", name);
  if (page_stride < (int64_t)page_size * kv_tok_stride || page_stride % 8 != 0 ||
      (int64_t)(num_pages - 1) * page_stride > ((int64_t)1 << 40))
    return set_error(SOLORT_EINVAL, "%s: page_stride %lld must hold page_size rows and be a multiple of 8", name,
                     (long long)page_stride);
  if (kv_tok_stride < (int64_t)nkv * kv_head_stride && kv_head_stride < (int64_t)page_size * kv_tok_stride)
    return set_error(SOLORT_EINVAL, "%s: token and head strides overlap", name);
  DecodeArgs a = {};
  // The logical capacity, table_len pages, plays the part of max_len.
  int rc = prepare(name, nq, nh, nkv, hd, k_pages, v_pages, kv_tok_stride, kv_head_stride,
                   (int64_t)table_len * page_size, pos0_dev, bound, scale, ws, n_split, out, out_dtype, a);
  if (rc) return rc;
  if (!qkv || !qn_w || !kn_w || !rope_cs) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(qkv) || !aligned16(qn_w) || !aligned16(kn_w) || !aligned16(rope_cs))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (qkv_row_stride < (int64_t)(nh + 2 * nkv) * hd || qkv_row_stride % 8 != 0 || qkv_row_stride > kMaxI32)
    return set_error(SOLORT_EINVAL, "%s: qkv_row_stride %lld", name, (long long)qkv_row_stride);
  a.qsrc = (const uint16_t*)qkv;
  a.qsrc_stride = (int)qkv_row_stride;
  a.qn_w = (const uint16_t*)qn_w;
  a.tail.kn_w = (const uint16_t*)kn_w;
  a.tail.rope_cs = (const uint16_t*)rope_cs;
  a.tail.eps = eps;
  a.paged = true;
  a.tail.page_table = page_table;
  a.tail.page_stride = page_stride;
  a.tail.page_shift = __builtin_ctz((unsigned)page_size);
  a.tail.num_pages = num_pages;
  return launch_all(name, true, nq, a, (hipStream_t)stream);
}

#ifdef SOLORT_PHASE_STAMPS
// Tracing build: copies the phase stamps of the split kernels' most recent
// launch (n_blocks workgroups, linear index kvh + nkv * split) to host.
extern "C" int solort_phase_stamps_decode(void* host, int n_blocks) {
  if (!host || n_blocks < 1 || n_blocks > kStampBlocks) return set_error(SOLORT_EINVAL, "phase_stamps_decode: bad arguments");
  const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(g_phase_stamps), (size_t)n_blocks * kStampSlots * 8, 0,
                                           hipMemcpyDeviceToHost);
  return e == hipSuccess ? 0 : set_error((int)e, "phase_stamps_decode: %s", hipGetErrorString(e));
}
#endif
