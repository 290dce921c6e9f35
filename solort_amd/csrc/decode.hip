// Split-KV (flash-decoding) grouped-query attention for 1..8 new tokens over
// the static KV cache, optionally fused with the QK-RMSNorm + RoPE prologue
// and KV write, followed by a small kernel that combines the splits.
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
// Split kernel.  Grid: nkv * n_split workgroups of 256 threads; block b
// serves KV head b % nkv and key split b / nkv (with 8 KV heads on 8 XCDs, all
// splits of a head share one XCD's L2).  The key range [0, bound) is cut into
// n_split static chunks, so every block issues its first K/V loads at launch,
// before the device-side position has arrived; keys past the live length are
// masked, and later iterations of a long split stop at the live length.
//   - 16 row slots of 16 lanes each take U key rows per iteration; lane j of a
//     slot loads dims [8j, 8j+8) of K and V as 16-byte vectors.  The query
//     group (nq * g rows) sits in registers as bf16 pairs, so each KV head is
//     read once for all of its query heads (no repeat_interleave); a score is
//     four bf16 pair dot products per lane, reduced over the slot with DPP.
//   - Scores and V rows of the iteration go to LDS.  Each wavefront then takes
//     the rows it owns: lane k evaluates p for key k, the p values go through
//     the wavefront's own LDS row, and every lane accumulates two output dims,
//     so no per-slot state is merged.
//   - Fused variant: while the K/V loads are in flight, slots compute the q
//     rows and the new tokens' K/V rows from the fused qkv projection and the
//     step's cos/sin rows (qknorm_rope.h, bit identical to the standalone
//     prologue).  Split 0 of each KV head writes the new rows to the cache;
//     every block substitutes the fresh rows for the cache rows
//     pos0..pos0+nq-1 it loaded, so no block waits for that write.
//   - Barriers order LDS only (lds_barrier): the K/V loads stay in flight
//     across them.
//   - Output: with one split the block writes the answer; otherwise its
//     partial (running max in log2 units, sum, unnormalised output).
// Combine kernel: merges the partials of each KV head (log-sum-exp); the
// kernel boundary orders its reads after the split kernel's writes.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "capi_internal.h"
#include "qknorm_rope.h"

namespace solort {

// The kernel's leading arguments are the ones its first loads need; the
// compiler preloads the leading kernel arguments into SGPRs (14 dwords, see
// -amdgpu-kernarg-preload-count in the build), so those loads issue without
// waiting for the kernel-argument fetch.  The rest travel in DecodeTail.
struct DecodeTail {
  const uint16_t* kn_w;
  const uint16_t* rope_cs;  // [2][nq][64] bf16: cos rows, then sin rows, of this step
  const int64_t* pos0_dev;
  float* ws_o;   // [nkv][n_split][R][128]
  float* ws_ml;  // [nkv][n_split][R][2]: running max (log2 units), sum
  void* out;     // [nq][nh][128]
  float qscale;  // softmax scale * log2(e)
  float eps;
  int pos_limit;  // positions >= pos_limit are not written
  int out_f32;
};

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

// Grid (nkv, n_split): block (kvh, split).  qsrc: fused, the qkv rows (row
// stride qsrc_stride); unfused, the q rows [nq][nh][128] (qsrc_stride = nh*128).
template <int NQ, int G, int U, bool FUSED>
__global__ __launch_bounds__(256) void decode_kernel(uint16_t* kc, uint16_t* vc, int tok_stride, int head_stride,
                                                     int chunk, int bound, const uint16_t* qsrc, int qsrc_stride,
                                                     int nh, const uint16_t* qn_w, const DecodeTail a) {
  constexpr int R = NQ * G;            // query rows sharing one KV head
  constexpr int KPI = 16 * U;          // keys per iteration (16 slots x U)
  constexpr int RPW = (R + 3) / 4;     // output rows per wavefront
  __shared__ __align__(16) uint4 s_q[R * 16];         // q rows, bf16 bits [row][16 x 16 B]
  __shared__ uint4 s_new[FUSED ? 2 * NQ * 16 : 1];   // fresh K rows then V rows (bf16 bits)
  __shared__ __align__(16) uint4 s_v[KPI * 16];      // the iteration's V rows [key][16 x 16 B]
  __shared__ __align__(16) float s_s[R * KPI];       // its masked scores [row][key] (log2 units), then p

  const int tid = threadIdx.x, j = tid & 15, slot = tid >> 4, wave = tid >> 6, lane = tid & 63;
  const int kvh = blockIdx.x, split = blockIdx.y, nkv = gridDim.x, NS = gridDim.y;
  const int kbeg = min(split * chunk, bound);
  const int kstat = min(kbeg + chunk, bound);

  // 1. Loads for this slot's first prologue row (fused: with its norm
  //    weights and its token's cos/sin), issued before the K/V loads: vector
  //    loads complete in issue order, so the prologue then waits for its own
  //    rows only.  Every load of phases 1 and 2 is unconditional (idle lanes
  //    load a valid row they ignore): a load skipped on some path would make
  //    the compiler wait for all of them before the first use.
  constexpr int NROWS = FUSED ? NQ * (G + 2) : R;
  uint4 raw0, wq0 = make_uint4(0u, 0u, 0u, 0u), wk0 = wq0, c0 = wq0, s0 = wq0;
  {
    const int row = min(slot, NROWS - 1);
    if constexpr (FUSED) {
      const int t = row / (G + 2), c = row % (G + 2);
      const int hs = c < G ? kvh * G + c : (c == G ? nh + kvh : nh + nkv + kvh);
      raw0 = *reinterpret_cast<const uint4*>(qsrc + (int64_t)t * qsrc_stride + hs * SOLORT_HD + j * 8);
      wq0 = *reinterpret_cast<const uint4*>(qn_w + j * 8);
      wk0 = *reinterpret_cast<const uint4*>(a.kn_w + j * 8);
      c0 = *reinterpret_cast<const uint4*>(a.rope_cs + t * 64 + (j & 7) * 8);
      s0 = *reinterpret_cast<const uint4*>(a.rope_cs + (NQ + t) * 64 + (j & 7) * 8);
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
    kr[u] = *reinterpret_cast<const uint4*>(kp + (int64_t)kid * tok_stride);
    vr[u] = *reinterpret_cast<const uint4*>(vp + (int64_t)kid * tok_stride);
  }

  const int64_t pos0 = a.pos0_dev[0];

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
        c8 = *reinterpret_cast<const uint4*>(a.rope_cs + t * 64 + (j & 7) * 8);
        s8 = *reinterpret_cast<const uint4*>(a.rope_cs + (NQ + t) * 64 + (j & 7) * 8);
      }
      if (c == G + 1) {  // V row: raw
        s_new[(NQ + t) * 16 + j] = raw;
        if (split == 0 && pos_ok)
          *reinterpret_cast<uint4*>(vc + pos * tok_stride + (int64_t)kvh * head_stride + j * 8) = raw;
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
          *reinterpret_cast<uint4*>(kc + pos * tok_stride + (int64_t)kvh * head_stride + j * 8) = ov;
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
        kn[u] = *reinterpret_cast<const uint4*>(kp + (int64_t)kid * tok_stride);
        vn[u] = *reinterpret_cast<const uint4*>(vp + (int64_t)kid * tok_stride);
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

  // 5. One split: the answer; otherwise this split's partial (max, sum,
  //    unnormalised output) for the combine kernel.
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = wave + 4 * i;
    if (r >= R) continue;
    const float Ls = wave_sum(Lk[i]);
    if (NS == 1) {
      const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
      store_out2(a.out, a.out_f32, nh, kvh, G, r, 2 * lane, O[i][0] * inv, O[i][1] * inv);
    } else {
      const int64_t pr = (int64_t)(kvh * NS + split) * R + r;
      *reinterpret_cast<float2*>(a.ws_o + pr * 128 + 2 * lane) = make_float2(O[i][0], O[i][1]);
      if (lane == 0) *reinterpret_cast<float2*>(a.ws_ml + pr * 2) = make_float2(M[i], Ls);
    }
  }
}

// The log-sum-exp combine of the n_split partials of each KV head.  Grid
// (nkv, column blocks): block = (KV head, 32 float4 columns of its [R][128]
// output); thread = (column, split group sg of 8): it merges splits sg,
// sg+8, ... on its own (all loads issued together), then the 8 split groups
// meet once in LDS.  Every argument is preloaded.
template <int NQ, int G>
__global__ __launch_bounds__(256) void combine_kernel(const float* ws_o, const float* ws_ml, void* out, int nh,
                                                      int n_split, int out_f32) {
  constexpr int R = NQ * G;
  constexpr int C = R * 32;  // float4 columns
  constexpr int B = 8;       // splits per thread per batch
  __shared__ float s_m[8][32], s_l[8][32];
  __shared__ float4 s_o[8][32];
  const int tid = threadIdx.x, c = tid & 31, sg = tid >> 5;
  const int kvh = blockIdx.x, cb = blockIdx.y;
  const int col = cb * 32 + c;
  const bool act = col < C;
  const int r = col >> 5;
  const int NS = n_split;
  const float2* wml = reinterpret_cast<const float2*>(ws_ml) + (int64_t)kvh * NS * R;
  const float4* wo = reinterpret_cast<const float4*>(ws_o) + (int64_t)kvh * NS * C;
  float mloc = -INFINITY, lloc = 0.f;
  float4 oloc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = sg; s0 < NS; s0 += 8 * B) {
    float2 ml[B];
    float4 ov[B];
#pragma unroll
    for (int k = 0; k < B; ++k) {
      const int s = s0 + 8 * k;
      if (act && s < NS) {
        ml[k] = wml[(int64_t)s * R + r];
        ov[k] = wo[(int64_t)s * C + col];
      } else {
        ml[k] = make_float2(-INFINITY, 0.f);
        ov[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    float mb = mloc;
#pragma unroll
    for (int k = 0; k < B; ++k) mb = fmaxf(mb, ml[k].x);
    if (mb != -INFINITY) {
      const float sc = fast_exp2(mloc - mb);  // mloc = -inf gives 0
      lloc *= sc;
      oloc.x *= sc; oloc.y *= sc; oloc.z *= sc; oloc.w *= sc;
#pragma unroll
      for (int k = 0; k < B; ++k) {
        const float w = (ml[k].x == -INFINITY) ? 0.f : fast_exp2(ml[k].x - mb);
        lloc = fmaf(w, ml[k].y, lloc);
        oloc = f4fma(w, ov[k], oloc);
      }
      mloc = mb;
    }
  }
  s_m[sg][c] = mloc;
  s_l[sg][c] = lloc;
  s_o[sg][c] = oloc;
  __syncthreads();
  if (tid < 32 && act) {
    float Mx = -INFINITY;
#pragma unroll
    for (int g = 0; g < 8; ++g) Mx = fmaxf(Mx, s_m[g][c]);
    float Ls = 0.f;
    float4 Os = make_float4(0.f, 0.f, 0.f, 0.f);
    if (Mx != -INFINITY) {
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const float w = (s_m[g][c] == -INFINITY) ? 0.f : fast_exp2(s_m[g][c] - Mx);
        Ls = fmaf(w, s_l[g][c], Ls);
        Os = f4fma(w, s_o[g][c], Os);
      }
    }
    const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
    Os.x *= inv; Os.y *= inv; Os.z *= inv; Os.w *= inv;
    store_out(out, out_f32, nh, kvh, G, col, Os);
  }
}

// ---------------------------------------------------------------- host side

constexpr int kMaxRows = 20;  // nq * group limit (registers and LDS)
constexpr int kMaxSplit = 1024;

// Everything a launch needs, gathered by prepare() and the entry points.
struct DecodeArgs {
  uint16_t* kc;
  uint16_t* vc;
  int tok_stride, head_stride, chunk, bound;
  const uint16_t* qsrc;
  int qsrc_stride, nh, nkv, n_split;
  const uint16_t* qn_w;
  DecodeTail tail;
};

struct WsLayout {
  size_t ml_off, o_off, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static WsLayout ws_layout(int nq, int nh, int nkv, int n_split) {
  const size_t R = (size_t)nq * (nh / nkv);
  WsLayout w;
  w.ml_off = 0;
  w.o_off = align256((size_t)nkv * n_split * R * 2 * sizeof(float));
  w.total = align256(w.o_off + (size_t)nkv * n_split * R * 128 * sizeof(float));
  return w;
}

template <int NQ, int G, int U, bool FUSED>
static void launch_split(const DecodeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((decode_kernel<NQ, G, U, FUSED>), dim3(a.nkv, a.n_split), dim3(256), 0, s, a.kc, a.vc,
                     a.tok_stride, a.head_stride, a.chunk, a.bound, a.qsrc, a.qsrc_stride, a.nh, a.qn_w, a.tail);
}

template <int NQ, int G, bool FUSED>
static bool launch_u(int U, const DecodeArgs& a, hipStream_t s) {
  if constexpr (NQ * G <= kMaxRows) {
    if constexpr (NQ == 1) {
      if (U == 4) {
        launch_split<NQ, G, 4, FUSED>(a, s);
        return true;
      }
    }
    launch_split<NQ, G, 2, FUSED>(a, s);
    return true;
  } else {
    return false;
  }
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
static bool launch_attn(bool fused, int U, const DecodeArgs& a, hipStream_t s) {
  return fused ? launch_u<NQ, G, true>(U, a, s) : launch_u<NQ, G, false>(U, a, s);
}

template <int G>
static bool attn_nq(int nq, bool fused, int U, const DecodeArgs& a, hipStream_t s) {
  SOLORT_DISPATCH_NQ(G, launch_attn, fused, U, a, s)
}

template <int G>
static bool combine_nq(int nq, const DecodeArgs& a, hipStream_t s) {
  SOLORT_DISPATCH_NQ(G, launch_combine, a, s)
}

static bool dispatch_attn(int G, int nq, bool fused, int U, const DecodeArgs& a, hipStream_t s) {
  switch (G) {
    case 1: return attn_nq<1>(nq, fused, U, a, s);
    case 2: return attn_nq<2>(nq, fused, U, a, s);
    case 4: return attn_nq<4>(nq, fused, U, a, s);
    case 8: return attn_nq<8>(nq, fused, U, a, s);
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
  a.chunk = ((((bound + n_split - 1) / n_split) + 15) / 16) * 16;  // static key chunk per split
  a.bound = bound;
  a.nh = nh;
  a.nkv = nkv;
  a.n_split = n_split;
  a.tail.pos0_dev = pos0_dev;
  a.tail.ws_o = (float*)((char*)ws + w.o_off);
  a.tail.ws_ml = (float*)((char*)ws + w.ml_off);
  a.tail.out = out;
  a.tail.qscale = scale * 1.4426950408889634f;
  a.tail.pos_limit = (int)max_len;
  a.tail.out_f32 = out_dtype == SOLORT_DTYPE_F32;
  U = a.chunk >= 64 ? 4 : 2;
  return 0;
}

// Launches the split kernel, then (more than one split) the combine kernel.
static int launch_all(const char* name, bool fused, int nq, const DecodeArgs& a, int U, hipStream_t s) {
  const int G = a.nh / a.nkv;
  if (!dispatch_attn(G, nq, fused, U, a, s))
    return set_error(SOLORT_EINVAL, "%s: no kernel for nq=%d group=%d", name, nq, G);
  int rc = check_launch(name);
  if (rc || a.n_split == 1) return rc;
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
  int U = 2;
  int rc = prepare(name, nq, nh, nkv, hd, (void*)k_cache, (void*)v_cache, kv_tok_stride, kv_head_stride,
                   max_len, pos0_dev, bound, scale, ws, n_split, out, out_dtype, a, U);
  if (rc) return rc;
  if (!q || !aligned16(q)) return set_error(SOLORT_EINVAL, "%s: q must be a 16-byte aligned pointer", name);
  a.qsrc = (const uint16_t*)q;
  a.qsrc_stride = nh * SOLORT_HD;
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
                                   const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                                   const int64_t* pos0_dev, void* k_cache, void* v_cache, int64_t kv_tok_stride,
                                   int64_t kv_head_stride, int64_t max_len, int bound, float scale, void* ws,
                                   int n_split, void* out, int out_dtype, solort_stream_t stream) {
  const char* name = "decode_layer";
  DecodeArgs a = {};
  int U = 2;
  int rc = prepare(name, nq, nh, nkv, hd, k_cache, v_cache, kv_tok_stride, kv_head_stride, max_len, pos0_dev,
                   bound, scale, ws, n_split, out, out_dtype, a, U);
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
  return launch_all(name, true, nq, a, U, (hipStream_t)stream);
}
