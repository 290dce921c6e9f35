// Split-KV (flash-decoding) grouped-query attention for 1..8 new tokens over
// the static KV cache, with the log-sum-exp combine fused into the launch,
// optionally fused with the QK-RMSNorm + RoPE prologue and KV write.
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
// Grid: nkv * n_split workgroups of 256 threads.  Block b serves KV head
// b % nkv and key split b / nkv.  The key range [0, bound) is cut into
// n_split static chunks, so every block issues its first K/V loads at launch,
// before the device-side position has arrived; keys past the live length are
// masked (and later iterations of long splits stop at the live length).
// Inside a block, 16 row slots of 16 lanes each take one key row per step;
// lane j of a slot loads dims [8j, 8j+8) of K and V as 16-byte vectors and
// holds the q rows of the whole query group (nq * g rows) in registers, so a
// KV head is read once for all of its query heads (no repeat_interleave).
//
// Fused variant: while the K/V loads are in flight, slots compute the q rows
// and the new tokens' K/V rows from the fused qkv projection (qknorm_rope.h,
// bit-identical to the standalone prologue).  Split 0 of each KV head writes
// the new rows to the cache; every block substitutes the fresh rows for the
// cache rows pos0..pos0+nq-1 it loaded, so no block depends on that write.
//
// Combine: each block merges its slots and waves, stores its partial
// (running max in log2 units, sum, unnormalised output) to the workspace,
// and takes a ticket (one agent-scope release per block).  The last block of
// a KV head acquires, loads every split's partial with all loads issued
// together, merges them and writes the output, then resets the ticket so the
// workspace is ready for the next launch.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "capi_internal.h"
#include "qknorm_rope.h"

namespace solort {

struct DecodeArgs {
  // fused prologue inputs
  const uint16_t* qkv;
  int64_t qkv_stride;
  const uint16_t* qn_w;
  const uint16_t* kn_w;
  const float* inv_freq;  // [64] RoPE frequencies
  int64_t pos_limit;      // positions >= pos_limit are not written
  float eps;
  // unfused: q rows [nq][nh][128]
  const uint16_t* q;
  // cache and attention
  uint16_t* kc;
  uint16_t* vc;
  int64_t tok_stride;
  int64_t head_stride;
  const int64_t* pos0_dev;
  float* ws_o;       // [nkv][n_split][R][128]
  float* ws_ml;      // [nkv][n_split][R][2]
  unsigned* ws_cnt;  // [nkv] tickets, zero between launches
  void* out;         // [nq][nh][128]
  float qscale;      // softmax scale * log2(e)
  int nh, nkv, bound, n_split, out_f32;
};

__device__ __forceinline__ float4 f4fma(float w, const float4 v, float4 acc) {
  acc.x = fmaf(w, v.x, acc.x);
  acc.y = fmaf(w, v.y, acc.y);
  acc.z = fmaf(w, v.z, acc.z);
  acc.w = fmaf(w, v.w, acc.w);
  return acc;
}

template <int R, int G>
__device__ __forceinline__ void combine_head(const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
                                             int NS, int nh, int kvh, int c0, int c1, void* out, int out_f32,
                                             float* smem);

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

template <int NQ, int G, int U, bool FUSED, bool COMBINE>
__global__ __launch_bounds__(256) void decode_kernel(const DecodeArgs a) {
  constexpr int R = NQ * G;  // query rows sharing one KV head
  constexpr int C = R * 32;  // float4 columns of an [R][128] block
  extern __shared__ __align__(16) float smem[];
  __shared__ __align__(16) float s_q[R * 128];
  __shared__ uint4 s_new[FUSED ? 2 * NQ * 16 : 1];  // fresh K rows then V rows (bf16 bits)
  __shared__ float s_rope[FUSED ? 2 * NQ * 64 : 1];  // cos [t][64] then sin [t][64]
  __shared__ unsigned s_ticket;

  const int tid = threadIdx.x, j = tid & 15, slot = tid >> 4, wave = tid >> 6;
  const int kvh = blockIdx.x % a.nkv;
  const int split = blockIdx.x / a.nkv;
  const int NS = a.n_split;
  int chunk = (a.bound + NS - 1) / NS;
  chunk = (chunk + 15) & ~15;
  const int kbeg = min(split * chunk, a.bound);
  const int kstat = min(kbeg + chunk, a.bound);

  // 1. Loads for this slot's first prologue row (and this thread's RoPE
  //    frequency), issued before the K/V loads: vector loads complete in
  //    issue order, so the prologue then waits for its own rows only.
  constexpr int NROWS = FUSED ? NQ * (G + 2) : R;
  constexpr int NROPE = FUSED ? 2 * NQ * 64 : 0;  // (token, frequency, cos|sin) values
  uint4 raw0 = make_uint4(0u, 0u, 0u, 0u), w0 = raw0;
  float fr0 = 0.f;
  if (slot < NROWS) {
    if constexpr (FUSED) {
      const int t = slot / (G + 2), c = slot % (G + 2);
      const int hs = c < G ? kvh * G + c : (c == G ? a.nh + kvh : a.nh + a.nkv + kvh);
      raw0 = *reinterpret_cast<const uint4*>(a.qkv + (int64_t)t * a.qkv_stride + hs * SOLORT_HD + j * 8);
      if (c <= G) w0 = *reinterpret_cast<const uint4*>((c < G ? a.qn_w : a.kn_w) + j * 8);
    } else {
      const int t = slot / G, g = slot % G;
      raw0 = *reinterpret_cast<const uint4*>(a.q + ((int64_t)t * a.nh + kvh * G + g) * SOLORT_HD + j * 8);
    }
  }
  if (FUSED && tid < NROPE) fr0 = a.inv_freq[(tid >> 1) & 63];

  // 2. First K/V loads: static addresses, independent of the position.
  const uint16_t* kp = a.kc + (int64_t)kvh * a.head_stride + j * 8;
  const uint16_t* vp = a.vc + (int64_t)kvh * a.head_stride + j * 8;
  uint4 kr[U], vr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int kid = kbeg + u * 16 + slot;
    if (kid < kstat) {
      kr[u] = *reinterpret_cast<const uint4*>(kp + (int64_t)kid * a.tok_stride);
      vr[u] = *reinterpret_cast<const uint4*>(vp + (int64_t)kid * a.tok_stride);
    } else {
      kr[u] = make_uint4(0u, 0u, 0u, 0u);
      vr[u] = make_uint4(0u, 0u, 0u, 0u);
    }
  }

  const int64_t pos0 = a.pos0_dev[0];

  // 3. q rows (and, fused, the new tokens' K/V rows) into LDS.  Fused: every
  //    thread first evaluates one (or a few) of the RoPE cos/sin values.
  if constexpr (FUSED) {
    for (int e = tid; e < NROPE; e += 256) {
      const int t = e >> 7, f = (e >> 1) & 63;
      const float ang = rope_angle(pos0 + t, e == tid ? fr0 : a.inv_freq[f]);
      s_rope[(e & 1) * NQ * 64 + t * 64 + f] = (e & 1) ? rope_sin(ang) : rope_cos(ang);
    }
    __syncthreads();
  }
  for (int row = slot; row < NROWS; row += 16) {
    uint4 raw = raw0, w8 = w0;
    if constexpr (FUSED) {
      const int t = row / (G + 2), c = row % (G + 2);
      const int64_t pos = pos0 + t;
      const bool pos_ok = pos >= 0 && pos < a.pos_limit;
      if (row != slot) {  // rows past the first (verify): loaded here
        const int hs = c < G ? kvh * G + c : (c == G ? a.nh + kvh : a.nh + a.nkv + kvh);
        raw = *reinterpret_cast<const uint4*>(a.qkv + (int64_t)t * a.qkv_stride + hs * SOLORT_HD + j * 8);
        if (c <= G) w8 = *reinterpret_cast<const uint4*>((c < G ? a.qn_w : a.kn_w) + j * 8);
      }
      if (c == G + 1) {  // V row: raw
        s_new[(NQ + t) * 16 + j] = raw;
        if (split == 0 && pos_ok)
          *reinterpret_cast<uint4*>(a.vc + pos * a.tok_stride + (int64_t)kvh * a.head_stride + j * 8) = raw;
        continue;
      }
      float cs[8], sn[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        cs[i] = s_rope[t * 64 + (j & 7) * 8 + i];
        sn[i] = s_rope[NQ * 64 + t * 64 + (j & 7) * 8 + i];
      }
      const uint4 ov = qknorm_rope_row(raw, w8, cs, sn, a.eps, j);
      if (c < G) {
        float y[8];
        unpack8(ov, y);
#pragma unroll
        for (int i = 0; i < 8; ++i) s_q[(t * G + c) * 128 + j * 8 + i] = y[i] * a.qscale;
      } else {
        s_new[t * 16 + j] = ov;
        if (split == 0 && pos_ok)
          *reinterpret_cast<uint4*>(a.kc + pos * a.tok_stride + (int64_t)kvh * a.head_stride + j * 8) = ov;
      }
    } else {
      const int t = row / G, g = row % G;
      if (row != slot)
        raw = *reinterpret_cast<const uint4*>(a.q + ((int64_t)t * a.nh + kvh * G + g) * SOLORT_HD + j * 8);
      float x[8];
      unpack8(raw, x);
#pragma unroll
      for (int i = 0; i < 8; ++i) s_q[row * 128 + j * 8 + i] = x[i] * a.qscale;
    }
  }
  __syncthreads();
  float qf[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[r][i] = s_q[r * 128 + j * 8 + i];

  // 4. Online softmax over this split's live keys.
  int64_t live64 = pos0 + NQ;
  live64 = live64 < 0 ? 0 : (live64 > a.bound ? a.bound : live64);
  const int kend = min(kstat, (int)live64);
  float m[R], l[R], acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[r][i] = 0.f;
  }
  for (int k0 = kbeg; k0 < kend; k0 += 16 * U) {
    uint4 kn[U], vn[U];
    const int k1 = k0 + 16 * U;
#pragma unroll
    for (int u = 0; u < U; ++u) {  // prefetch the next step of a long split
      const int kid = k1 + u * 16 + slot;
      if (kid < kend) {
        kn[u] = *reinterpret_cast<const uint4*>(kp + (int64_t)kid * a.tok_stride);
        vn[u] = *reinterpret_cast<const uint4*>(vp + (int64_t)kid * a.tok_stride);
      } else {
        kn[u] = make_uint4(0u, 0u, 0u, 0u);
        vn[u] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    int kid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kid[u] = k0 + u * 16 + slot;
      if constexpr (FUSED) {
        const int64_t off = (int64_t)kid[u] - pos0;
        if (off >= 0 && off < NQ) {
          kr[u] = s_new[off * 16 + j];
          vr[u] = s_new[(NQ + off) * 16 + j];
        }
      }
    }
    float s[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kf[8];
      unpack8(kr[u], kf);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = qf[r][0] * kf[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) d = fmaf(qf[r][i], kf[i], d);
        s[u][r] = d;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r) s[u][r] = row16_sum(s[u][r]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = kid[u] < kend;
#pragma unroll
      for (int t = 0; t < NQ; ++t)
#pragma unroll
        for (int g = 0; g < G; ++g)
          if (!in || (int64_t)kid[u] > pos0 + t) s[u][t * G + g] = -INFINITY;
    }
    float vf[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) unpack8(vr[u], vf[u]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float mx = m[r];
#pragma unroll
      for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u][r]);
      if (mx != -INFINITY) {
        const float alpha = fast_exp2(m[r] - mx);  // m = -inf gives 0
        float ls = l[r] * alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r][i] *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float p = fast_exp2(s[u][r] - mx);
          ls += p;
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[r][i] = fmaf(p, vf[u][i], acc[r][i]);
        }
        l[r] = ls;
        m[r] = mx;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kr[u] = kn[u];
      vr[u] = vn[u];
    }
  }

  // 5. Merge the 16 row slots into this split's partial (running max in
  //    log2 units, sum, unnormalised output), as float4 columns col of the
  //    [R][128] block: thread col < C handles dims 4*(col%32).. of row col/32.
  float4 part_o[(C + 255) / 256];
  float part_m[(C + 255) / 256], part_l[(C + 255) / 256];
  if constexpr (R <= 4) {
    // Every slot's state goes to LDS, then each column merges 16 slots.
    float* s_acc = smem;               // [16][R][128]
    float* s_m = smem + 16 * R * 128;  // [16][R]
    float* s_l = s_m + 16 * R;         // [16][R]
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float4* dst = reinterpret_cast<float4*>(s_acc + (slot * R + r) * 128 + j * 8);
      dst[0] = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
      dst[1] = make_float4(acc[r][4], acc[r][5], acc[r][6], acc[r][7]);
      if (j == 0) {
        s_m[slot * R + r] = m[r];
        s_l[slot * R + r] = l[r];
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < (C + 255) / 256; ++k) {
      const int col = tid + 256 * k;
      if (col < C) {
        const int r = col >> 5, d = (col & 31) * 4;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 16; ++w) M = fmaxf(M, s_m[w * R + r]);
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
          const float mw = s_m[w * R + r];
          const float sc = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
          O = f4fma(sc, *reinterpret_cast<const float4*>(s_acc + (w * R + r) * 128 + d), O);
          L = fmaf(s_l[w * R + r], sc, L);
        }
        part_o[k] = O;
        part_m[k] = M;
        part_l[k] = L;
      }
    }
  } else {
    // Larger query groups: merge the 4 slots of each wavefront with lane
    // exchanges first, then the 4 wavefronts through LDS.
#pragma unroll
    for (int mask = 16; mask <= 32; mask <<= 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float mo = xshfl(m[r], mask), lo = xshfl(l[r], mask);
        const float mn = fmaxf(m[r], mo);
        const float sa = (m[r] == -INFINITY) ? 0.f : fast_exp2(m[r] - mn);
        const float sb = (mo == -INFINITY) ? 0.f : fast_exp2(mo - mn);
        l[r] = l[r] * sa + lo * sb;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float ao = xshfl(acc[r][i], mask);
          acc[r][i] = acc[r][i] * sa + ao * sb;
        }
        m[r] = mn;
      }
    }
    float* s_acc = smem;              // [4][R][128]
    float* s_m = smem + 4 * R * 128;  // [4][R]
    float* s_l = s_m + 4 * R;         // [4][R]
    if ((tid & 63) < 16) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float4* dst = reinterpret_cast<float4*>(s_acc + (wave * R + r) * 128 + j * 8);
        dst[0] = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
        dst[1] = make_float4(acc[r][4], acc[r][5], acc[r][6], acc[r][7]);
        if (j == 0) {
          s_m[wave * R + r] = m[r];
          s_l[wave * R + r] = l[r];
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < (C + 255) / 256; ++k) {
      const int col = tid + 256 * k;
      if (col < C) {
        const int r = col >> 5, d = (col & 31) * 4;
        float M = s_m[r];
#pragma unroll
        for (int w = 1; w < 4; ++w) M = fmaxf(M, s_m[w * R + r]);
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float mw = s_m[w * R + r];
          const float sc = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
          O = f4fma(sc, *reinterpret_cast<const float4*>(s_acc + (w * R + r) * 128 + d), O);
          L = fmaf(s_l[w * R + r], sc, L);
        }
        part_o[k] = O;
        part_m[k] = M;
        part_l[k] = L;
      }
    }
  }

  // 6. One split: the partial is the answer.
  if (NS == 1) {
#pragma unroll
    for (int k = 0; k < (C + 255) / 256; ++k) {
      const int col = tid + 256 * k;
      if (col < C) {
        const float inv = part_l[k] > 0.f ? 1.f / part_l[k] : 0.f;
        float4 O = part_o[k];
        O.x *= inv; O.y *= inv; O.z *= inv; O.w *= inv;
        store_out(a.out, a.out_f32, a.nh, kvh, G, col, O);
      }
    }
    return;
  }

  // 7. Store the partial.
  {
    float4* wo = reinterpret_cast<float4*>(a.ws_o + (int64_t)(kvh * NS + split) * R * 128);
    float* wml = a.ws_ml + (int64_t)(kvh * NS + split) * R * 2;
#pragma unroll
    for (int k = 0; k < (C + 255) / 256; ++k) {
      const int col = tid + 256 * k;
      if (col < C) {
        wo[col] = part_o[k];
        if ((col & 31) == 0) *reinterpret_cast<float2*>(wml + (col >> 5) * 2) = make_float2(part_m[k], part_l[k]);
      }
    }
  }
  if constexpr (!COMBINE) {
    return;  // solort_attn_combine merges the partials in the next launch
  } else {
    // 8. Ticket: the last block of this KV head merges every split's partial.
    __syncthreads();
    if (tid == 0) {
      fence_release_agent();
      s_ticket = __hip_atomic_fetch_add(a.ws_cnt + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_ticket != (unsigned)(NS - 1)) return;
    fence_acquire_agent();
    combine_head<R, G>(a.ws_o, a.ws_ml, NS, a.nh, kvh, 0, C, a.out, a.out_f32, smem);
    if (tid == 0) a.ws_cnt[kvh] = 0u;
  }
}

// Merges the n_split partials of KV head kvh for float4 columns [c0, c1) of
// its [R][128] output block and writes them (the log-sum-exp combine).  A
// thread's first batch of partial loads is issued before anything waits; the
// per-row maximum and sum are wavefront reductions.
template <int R, int G>
__device__ __forceinline__ void combine_head(const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
                                             int NS, int nh, int kvh, int c0, int c1, void* out, int out_f32,
                                             float* smem) {
  constexpr int C = R * 32;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ncol = c1 - c0;
  const int SG = ncol >= 256 ? 1 : 256 / ncol;  // split groups sharing one column
  constexpr int B = 16;                          // loads issued together per thread
  const int NSR4 = (NS * R + 3) & ~3;
  float* s_m = smem;                             // [NS][R] maxima
  float* s_l = smem + NSR4;                      // [NS][R] sums
  float* s_w = smem + 2 * NSR4;                  // [NS][R] combine weights
  float4* s_red = reinterpret_cast<float4*>(smem + 3 * NSR4);  // [SG][ncol]
  const float* wml_all = ws_ml + (int64_t)kvh * NS * R * 2;
  const float4* wo4 = reinterpret_cast<const float4*>(ws_o + (int64_t)kvh * NS * R * 128);

  const int col0 = c0 + tid % ncol, sg0 = tid / ncol;
  const bool act0 = tid < ncol * SG;
  float4 v[B];
#pragma unroll
  for (int k = 0; k < B; ++k) {
    const int s = sg0 + k * SG;
    v[k] = (act0 && s < NS) ? wo4[(int64_t)s * C + col0] : make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // Combine weights exp2(m_s - M) / L for the rows this block writes.
  const int r0 = c0 >> 5, r1 = (c1 - 1) >> 5;
  for (int r = r0 + wave; r <= r1; r += 4) {
    float mx = -INFINITY;
    for (int s = lane; s < NS; s += 64) {
      const float2 ml = *reinterpret_cast<const float2*>(wml_all + (s * R + r) * 2);
      s_m[s * R + r] = ml.x;
      s_l[s * R + r] = ml.y;
      mx = fmaxf(mx, ml.x);
    }
    mx = wave_max(mx);
    float sum = 0.f;
    for (int s = lane; s < NS; s += 64) {
      const float ms = s_m[s * R + r];
      if (ms != -INFINITY) sum = fmaf(s_l[s * R + r], fast_exp2(ms - mx), sum);
    }
    sum = wave_sum(sum);
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
    for (int s = lane; s < NS; s += 64) {
      const float ms = s_m[s * R + r];
      s_w[s * R + r] = (ms == -INFINITY) ? 0.f : fast_exp2(ms - mx) * inv;
    }
  }
  __syncthreads();
  for (int base = tid; base < ncol * SG; base += 256) {
    const int col = c0 + base % ncol, sg = base / ncol, r = col >> 5;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = sg; s0 < NS; s0 += SG * B) {
      if (!(base == tid && s0 == sg)) {
#pragma unroll
        for (int k = 0; k < B; ++k) {
          const int s = s0 + k * SG;
          v[k] = s < NS ? wo4[(int64_t)s * C + col] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int k = 0; k < B; ++k) {
        const int s = s0 + k * SG;
        if (s < NS) O = f4fma(s_w[s * R + r], v[k], O);
      }
    }
    s_red[(SG == 1 ? 0 : sg) * ncol + (col - c0)] = O;
  }
  __syncthreads();
  for (int cc = tid; cc < ncol; cc += 256) {
    float4 O = s_red[cc];
    for (int sg = 1; sg < SG; ++sg) {
      const float4 o2 = s_red[sg * ncol + cc];
      O.x += o2.x; O.y += o2.y; O.z += o2.z; O.w += o2.w;
    }
    store_out(out, out_f32, nh, kvh, G, c0 + cc, O);
  }
}

struct CombineArgs {
  const float* ws_o;
  const float* ws_ml;
  void* out;
  int nh, nkv, n_split, out_f32, cols_per_block;
};

// Grid: nkv * ceil(C / cols_per_block) blocks; block b merges KV head b % nkv,
// float4 columns [cb * cols_per_block, ...) with cb = b / nkv.
template <int NQ, int G>
__global__ __launch_bounds__(256) void combine_kernel(const CombineArgs a) {
  constexpr int R = NQ * G;
  constexpr int C = R * 32;
  extern __shared__ __align__(16) float smem[];
  const int kvh = blockIdx.x % a.nkv, cb = blockIdx.x / a.nkv;
  const int c0 = cb * a.cols_per_block;
  const int c1 = min(c0 + a.cols_per_block, C);
  combine_head<R, G>(a.ws_o, a.ws_ml, a.n_split, a.nh, kvh, c0, c1, a.out, a.out_f32, smem);
}

// ---------------------------------------------------------------- host side

constexpr int kMaxRows = 20;  // nq * group limit (registers and LDS)
constexpr int kMaxSplit = 1024;
constexpr int kCombineCols = 32;  // float4 columns per block of the combine kernel

struct WsLayout {
  size_t o_off, ml_off, cnt_off, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The tickets sit at offset 0 whatever the split count, so one workspace sized
// for the largest split count can serve launches with any smaller one: every
// launch leaves its tickets at zero, and the partials it leaves behind never
// overlap another launch's tickets.
static WsLayout ws_layout(int nq, int nh, int nkv, int n_split) {
  const size_t R = (size_t)nq * (nh / nkv);
  WsLayout w;
  w.cnt_off = 0;
  w.ml_off = align256((size_t)nkv * sizeof(unsigned));
  w.o_off = align256(w.ml_off + (size_t)nkv * n_split * R * 2 * sizeof(float));
  w.total = align256(w.o_off + (size_t)nkv * n_split * R * 128 * sizeof(float));
  return w;
}

static size_t combine_floats(int R, int n_split, int ncol) {
  const int SG = ncol >= 256 ? 1 : 256 / ncol;
  return 3 * (((size_t)n_split * R + 3) & ~(size_t)3) + (size_t)SG * ncol * 4;
}

static size_t decode_smem_bytes(int R, int n_split, bool combine_in_kernel) {
  const size_t main_f = R <= 4 ? (size_t)16 * R * 128 + 32 * R : (size_t)4 * R * 128 + 8 * R;
  const size_t comb_f = combine_in_kernel ? combine_floats(R, n_split, R * 32) : 0;
  return (main_f > comb_f ? main_f : comb_f) * sizeof(float);
}

// How the split partials are merged: 0 = a separate combine launch (the
// kernel boundary orders the partials; the default), 1 = the last block of
// each KV head merges them inside the same launch (agent-scope release and
// acquire around an atomic ticket).  SOLORT_DECODE_COMBINE=ticket selects 1.
static int combine_mode() {
  static int mode = -1;
  if (mode < 0) {
    const char* e = getenv("SOLORT_DECODE_COMBINE");
    mode = (e && strcmp(e, "ticket") == 0) ? 1 : 0;
  }
  return mode;
}

template <int NQ, int G, bool FUSED, bool COMBINE>
static bool launch_u(int U, const DecodeArgs& a, int blocks, size_t smem, hipStream_t s) {
  if constexpr (NQ * G <= kMaxRows) {
    if constexpr (NQ == 1) {
      if (U == 4) {
        hipLaunchKernelGGL((decode_kernel<NQ, G, 4, FUSED, COMBINE>), dim3(blocks), dim3(256), smem, s, a);
        return true;
      }
    }
    hipLaunchKernelGGL((decode_kernel<NQ, G, 2, FUSED, COMBINE>), dim3(blocks), dim3(256), smem, s, a);
    return true;
  } else {
    return false;
  }
}

template <int NQ, int G>
static bool launch_combine(const CombineArgs& c, int blocks, size_t smem, hipStream_t s) {
  if constexpr (NQ * G <= kMaxRows) {
    hipLaunchKernelGGL((combine_kernel<NQ, G>), dim3(blocks), dim3(256), smem, s, c);
    return true;
  } else {
    return false;
  }
}

// Dispatches on (nq, G) to fn<NQ, G>(args...).
#define SOLORT_DISPATCH_NQ(G, FN, ...)                       \
  switch (nq) {                                              \
    case 1: return FN<1, G>(__VA_ARGS__);                    \
    case 2: return FN<2, G>(__VA_ARGS__);                    \
    case 3: return FN<3, G>(__VA_ARGS__);                    \
    case 4: return FN<4, G>(__VA_ARGS__);                    \
    case 5: return FN<5, G>(__VA_ARGS__);                    \
    case 6: return FN<6, G>(__VA_ARGS__);                    \
    case 7: return FN<7, G>(__VA_ARGS__);                    \
    case 8: return FN<8, G>(__VA_ARGS__);                    \
  }                                                          \
  return false;

template <int NQ, int G>
static bool launch_attn(bool fused, bool combine, int U, const DecodeArgs& a, int blocks, size_t smem,
                        hipStream_t s) {
  if (fused)
    return combine ? launch_u<NQ, G, true, true>(U, a, blocks, smem, s)
                   : launch_u<NQ, G, true, false>(U, a, blocks, smem, s);
  return combine ? launch_u<NQ, G, false, true>(U, a, blocks, smem, s)
                 : launch_u<NQ, G, false, false>(U, a, blocks, smem, s);
}

template <int G>
static bool attn_nq(int nq, bool fused, bool combine, int U, const DecodeArgs& a, int blocks, size_t smem,
                    hipStream_t s) {
  SOLORT_DISPATCH_NQ(G, launch_attn, fused, combine, U, a, blocks, smem, s)
}

template <int G>
static bool combine_nq(int nq, const CombineArgs& c, int blocks, size_t smem, hipStream_t s) {
  SOLORT_DISPATCH_NQ(G, launch_combine, c, blocks, smem, s)
}

static bool dispatch_attn(int G, int nq, bool fused, bool combine, int U, const DecodeArgs& a, int blocks,
                          size_t smem, hipStream_t s) {
  switch (G) {
    case 1: return attn_nq<1>(nq, fused, combine, U, a, blocks, smem, s);
    case 2: return attn_nq<2>(nq, fused, combine, U, a, blocks, smem, s);
    case 4: return attn_nq<4>(nq, fused, combine, U, a, blocks, smem, s);
    case 8: return attn_nq<8>(nq, fused, combine, U, a, blocks, smem, s);
  }
  return false;
}

static bool dispatch_combine(int G, int nq, const CombineArgs& c, int blocks, size_t smem, hipStream_t s) {
  switch (G) {
    case 1: return combine_nq<1>(nq, c, blocks, smem, s);
    case 2: return combine_nq<2>(nq, c, blocks, smem, s);
    case 4: return combine_nq<4>(nq, c, blocks, smem, s);
    case 8: return combine_nq<8>(nq, c, blocks, smem, s);
  }
  return false;
}

// Checks shared by every attention entry point; fills the attention part of `a`.
static int prepare(const char* name, int nq, int nh, int nkv, int hd, void* k_cache, void* v_cache,
                   int64_t kv_tok_stride, int64_t kv_head_stride, int64_t max_len,
                   const int64_t* pos0_dev, int bound, float scale, void* ws, int n_split, void* out,
                   int out_dtype, DecodeArgs& a, int& U) {
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
  if (kv_tok_stride <= 0 || kv_head_stride <= 0 || kv_tok_stride % 8 || kv_head_stride % 8)
    return set_error(SOLORT_EINVAL, "%s: KV strides must be positive multiples of 8", name);
  if (bound < 1 || bound > max_len || bound > (1 << 30))
    return set_error(SOLORT_EINVAL, "%s: bound %d outside [1, max_len=%lld]", name, bound, (long long)max_len);
  if (n_split < 1 || n_split > kMaxSplit)
    return set_error(SOLORT_EINVAL, "%s: n_split %d outside [1, %d]", name, n_split, kMaxSplit);
  if (out_dtype != SOLORT_DTYPE_BF16 && out_dtype != SOLORT_DTYPE_F32)
    return set_error(SOLORT_EINVAL, "%s: out_dtype %d", name, out_dtype);
  const int R = nq * G;
  const size_t static_lds = (size_t)R * 128 * 4 + (size_t)2 * nq * 16 * 16 + (size_t)2 * nq * 64 * 4 + 16;
  const size_t smem_max = decode_smem_bytes(R, n_split, true);
  const size_t comb_max = combine_floats(R, n_split, kCombineCols < R * 32 ? kCombineCols : R * 32) * 4;
  if (smem_max + static_lds > 64 * 1024 || comb_max > 64 * 1024)
    return set_error(SOLORT_EINVAL, "%s: n_split %d too large for %d query rows", name, n_split, R);
  const WsLayout w = ws_layout(nq, nh, nkv, n_split);
  a.kc = (uint16_t*)k_cache;
  a.vc = (uint16_t*)v_cache;
  a.tok_stride = kv_tok_stride;
  a.head_stride = kv_head_stride;
  a.pos0_dev = pos0_dev;
  a.ws_o = (float*)((char*)ws + w.o_off);
  a.ws_ml = (float*)((char*)ws + w.ml_off);
  a.ws_cnt = (unsigned*)((char*)ws + w.cnt_off);
  a.out = out;
  a.qscale = scale * 1.4426950408889634f;
  a.nh = nh;
  a.nkv = nkv;
  a.bound = bound;
  a.n_split = n_split;
  a.out_f32 = out_dtype == SOLORT_DTYPE_F32;
  const int per_split = (((bound + n_split - 1) / n_split) + 15) & ~15;
  U = per_split >= 64 ? 4 : 2;
  return 0;
}

// Launches the split kernel and, in the default mode, the combine kernel.
static int launch_all(const char* name, bool fused, int nq, const DecodeArgs& a, int U, hipStream_t s) {
  const int G = a.nh / a.nkv, R = nq * G, C = R * 32;
  const bool in_kernel = a.n_split > 1 && combine_mode() == 1;
  const size_t smem = decode_smem_bytes(R, a.n_split, in_kernel);
  if (!dispatch_attn(G, nq, fused, in_kernel, U, a, a.n_split * a.nkv, smem, s))
    return set_error(SOLORT_EINVAL, "%s: no kernel for nq=%d group=%d", name, nq, G);
  int rc = check_launch(name);
  if (rc || a.n_split == 1 || in_kernel) return rc;
  CombineArgs c;
  c.ws_o = a.ws_o;
  c.ws_ml = a.ws_ml;
  c.out = a.out;
  c.nh = a.nh;
  c.nkv = a.nkv;
  c.n_split = a.n_split;
  c.out_f32 = a.out_f32;
  c.cols_per_block = kCombineCols < C ? kCombineCols : C;
  const int cb = (C + c.cols_per_block - 1) / c.cols_per_block;
  const size_t csmem = combine_floats(R, a.n_split, c.cols_per_block) * sizeof(float);
  if (!dispatch_combine(G, nq, c, cb * a.nkv, csmem, s))
    return set_error(SOLORT_EINVAL, "%s: no combine kernel for nq=%d group=%d", name, nq, G);
  return check_launch(name);
}

static int attn_impl(const char* name, const void* q, int nq, int nh, int nkv, int hd,
                     const void* k_cache, const void* v_cache, int64_t kv_tok_stride,
                     int64_t kv_head_stride, int64_t max_len, const int64_t* pos0_dev, int bound,
                     float scale, void* ws, int n_split, void* out, int out_dtype,
                     solort_stream_t stream) {
  DecodeArgs a = {};
  int U = 2;
  int rc = prepare(name, nq, nh, nkv, hd, (void*)k_cache, (void*)v_cache, kv_tok_stride, kv_head_stride,
                   max_len, pos0_dev, bound, scale, ws, n_split, out, out_dtype, a, U);
  if (rc) return rc;
  if (!q || !aligned16(q)) return set_error(SOLORT_EINVAL, "%s: q must be a 16-byte aligned pointer", name);
  a.q = (const uint16_t*)q;
  return launch_all(name, false, nq, a, U, (hipStream_t)stream);
}

}  // namespace solort

using namespace solort;

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
                                   const void* qn_w, const void* kn_w, float eps, const float* inv_freq,
                                   const int64_t* pos0_dev, void* k_cache, void* v_cache, int64_t kv_tok_stride,
                                   int64_t kv_head_stride, int64_t max_len, int bound, float scale, void* ws,
                                   int n_split, void* out, int out_dtype, solort_stream_t stream) {
  const char* name = "decode_layer";
  DecodeArgs a = {};
  int U = 2;
  int rc = prepare(name, nq, nh, nkv, hd, k_cache, v_cache, kv_tok_stride, kv_head_stride, max_len, pos0_dev,
                   bound, scale, ws, n_split, out, out_dtype, a, U);
  if (rc) return rc;
  if (!qkv || !qn_w || !kn_w || !inv_freq) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(qkv) || !aligned16(qn_w) || !aligned16(kn_w) || !aligned16(inv_freq))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (qkv_row_stride < (int64_t)(nh + 2 * nkv) * hd || qkv_row_stride % 8 != 0)
    return set_error(SOLORT_EINVAL, "%s: qkv_row_stride %lld", name, (long long)qkv_row_stride);
  a.qkv = (const uint16_t*)qkv;
  a.qkv_stride = qkv_row_stride;
  a.qn_w = (const uint16_t*)qn_w;
  a.kn_w = (const uint16_t*)kn_w;
  a.inv_freq = inv_freq;
  a.pos_limit = max_len;
  a.eps = eps;
  return launch_all(name, true, nq, a, U, (hipStream_t)stream);
}
