// Causal grouped-query prefill attention on bf16 MFMA (gfx950).
//
// Reference: src/solort/model/cuda_graph_executor.py:124-130, i.e.
//   SDPA(q, repeat_interleave(k, g), repeat_interleave(v, g), is_causal=True,
//        scale=hd**-0.5) over the T prompt rows, written as ctx [T, nh*128].
// K and V are read from the cache rows 0..T-1 the prologue just wrote (the
// reference attends the same k/v values it writes at :122-123).  No repeat:
// the query heads of a KV head share every K/V tile staged in LDS.
//
// Block = 4 wavefronts = one KV head x 64 query rows: 16 positions x 4 query
// heads at g = 4 (8 x 8 at g = 8, 32 x 2 at g = 2, 64 positions at g = 1); block row R is
// query head kvh*g + R / PB at position p0 + R % PB (PB = 64 / g positions).
// Wave w = (row group rg = w % 2, key half kh = w / 2) owns rows 32 rg ..
// 32 rg + 31.  Each iteration stages 64 keys of K and V, both row-major, in
// LDS (double buffered, 71.7 KB: two blocks share a CU, and their waves
// interleave on each SIMD without shared barriers; the next stage's loads fly
// during this one's math and barriers order only LDS); half kh takes the
// stage's 32 keys kh, and the two halves of every row merge through LDS at the
// end.  Per 32-key half:
//   S^T = K Q^T   v_mfma_f32_32x32x16_bf16, A = K (LDS, one 16-byte read per
//                 operand), B = Q^T (registers), 8 dim steps
//   online softmax in fp32 with a lazy maximum: a row's reference max moves
//                 only when a stage's max exceeds it by more than 8 (log2
//                 units), so p = 2^(s*c - m*c) <= 2^8 (c = scale*log2(e))
//                 and O is rarely rescaled; bf16 output: P is rounded to bf16
//                 and the row sum adds the rounded P (v_dot2_f32_bf16); fp32
//                 output: P enters as bf16 high + low parts (two MFMAs) and
//                 the row sum adds P in fp32
//   O^T += V^T P^T  A = V^T from the row-major V tile by ds_read_b64_tr_b16,
//                 B = P^T straight from the S^T registers, 4 dim tiles x 2
//                 key steps
// MFMA operand layouts (checked on gfx950): A[m][k] lane l holds
// A[l%32][8(l/32)+s]; B[k][n] lane l holds B[8(l/32)+s][l%32]; D[m][n] lane
// l, register i holds D[8(i/4)+4(l/32)+i%4][l%32].  With S^T and O^T a lane
// keeps one query row (l%32), so softmax statistics move between lanes only
// for the row max (one exchange with lane l^32).  The key order inside each
// 16-key MFMA step is a permutation shared by P^T (the registers of S^T) and
// the V^T reads, so P needs no data movement.
// Causal: a block reads stages up to its last position; waves skip keys past
// their own rows and mask only the keys that cross their diagonal.  All tiles
// of a KV head run on one XCD (block index mod 8).  The first round of blocks
// (one per CU: `round` per KV head) takes the tiles heaviest first, the second
// round lightest first, so the CU that holds the heaviest tile holds the
// lightest beside it.
#include <math.h>

#include <type_traits>

#include "common.h"
#include "capi_internal.h"
#include "qknorm_rope.h"

namespace solort {

SOLORT_STAMP_TU();  // phase stamps of the tracing build (common.h)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;      // 4 wavefronts
constexpr int kKeys = 32;          // keys per wave per stage
constexpr int kStage = 2 * kKeys;  // keys staged per stage
constexpr int kKStride = 128 + 8;   // K tile row stride (bf16): 272 B, conflict-free 16-byte reads
constexpr int kVStride = 128 + 16;  // V tile row stride (bf16): 288 B, conflict-free transposing reads
constexpr int kKAhead = 6;          // K operand reads in flight ahead of the score MFMAs
constexpr int kVAhead = 6;          // V operand reads in flight ahead of the P V MFMAs

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// One stage of 64 keys in flight in registers: per thread 4 K and 4 V chunks
// of 16 bytes, key rows r0 + 16 i, dims 8 ch .. 8 ch + 7.
struct Staged {
  uint4 k0, k1, k2, k3, v0, v1, v2, v3;
};

// Buffer resource over one KV head's rows 0..T-1 (byte offsets
// [0, ((T-1) * tok_stride + 128) * 2)); loads past it return zeros, which is
// what the rows at or past T must contribute (the causal mask gives them
// weight 0 in every row < T).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kv_rsrc(const uint16_t* base, int T, int64_t ts) {
  const int nbytes = (int)(((int64_t)(T - 1) * ts + SOLORT_HD) * 2);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, nbytes, 0x00020000);
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Global loads of the stage whose first key sits at byte offset soff: voff[i]
// is this thread's byte offset of key row r0 + 16 i, dims 8ch...
__device__ __forceinline__ Staged prefill_fetch(__amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                                const int (&voff)[4], int soff) {
  Staged st;
  st.k0 = bload16(kr, voff[0], soff);
  st.k1 = bload16(kr, voff[1], soff);
  st.k2 = bload16(kr, voff[2], soff);
  st.k3 = bload16(kr, voff[3], soff);
  st.v0 = bload16(vr, voff[0], soff);
  st.v1 = bload16(vr, voff[1], soff);
  st.v2 = bload16(vr, voff[2], soff);
  st.v3 = bload16(vr, voff[3], soff);
  return st;
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives in slot k
// element i % 4 of the 8 bytes addressed by lane 4k + i / 4 of the group.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)(__attribute__((address_space(3))) uint16_t*)(p));
  return __builtin_bit_cast(uint2, v);
}

// Scalar arguments: the first ten (15 SGPRs: every address and index the
// first loads need) arrive preloaded (-amdgpu-kernarg-preload-count); qscale,
// eps and out load meanwhile.  q: row pos, head h at q + pos * q_stride + 128 h
// (the [T][nh][128] buffer, or with FUSED the raw q rows of the qkv projection,
// which the kernel normalises with qn_w, eps and the cos/sin rows rope_cs
// [2][T][64] as solort_qknorm_rope_kvwrite_cs would, bit for bit); t_nkv = T |
// nkv << 24; round = blocks per KV head in one block per CU; out [T][nh * 128]
// in fp32 (F32) or bf16; qscale = softmax scale * log2(e).
template <int G, bool F32, bool FUSED>
__global__ __launch_bounds__(kThreads, 2) void prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ rope_cs, int t_nkv, int tok_stride,
    int head_stride, int q_stride, int round, float qscale, float eps, void* __restrict__ out_ptr) {
  const int T = t_nkv & 0xffffff, nkv = (int)((unsigned)t_nkv >> 24);
  constexpr int PB = 64 / G;  // positions per block
  const int nh = nkv * G, n_qtiles = (T + PB - 1) / PB;
  __shared__ __align__(16) uint16_t sK[2][kStage * kKStride];
  __shared__ __align__(16) uint16_t sV[2][kStage * kVStride];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kh = wave >> 1, rg = wave & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  const int kvh = blockIdx.x % nkv;
  const int ib = (int)(blockIdx.x / nkv);
  const int rank = ib < round ? ib : n_qtiles - 1 - (ib - round);
  const int tile = n_qtiles - 1 - rank;  // first round heaviest first; second round lightest first
  SOLORT_STAMP(tid == 0, (int)blockIdx.x, 0);
  const int p0 = tile * PB;
  const int qrow = p0 + (32 * rg + l32) % PB;                // the query row of this lane's scores
  const int pw = p0 + (G == 1 ? 32 * rg : 0);                // this wave's first position
  const int kend_w = min(T, pw + (PB < 32 ? PB : 32));       // keys this wave attends (wave-uniform)

  // The block's 64 Q rows, loaded coalesced: thread t takes rows t / 16 + 16 i, bytes
  // 16 (t % 16) .. +15 (positions past T repeat row T-1).  They pass through the second K buffer.
  uint4 qv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int R = (tid >> 4) + 16 * i;
    const int pos = min(p0 + R % PB, T - 1);
    qv[i] = *reinterpret_cast<const uint4*>(q + (int64_t)pos * q_stride + (kvh * G + R / PB) * SOLORT_HD +
                                           8 * (tid & 15));
  }
  // FUSED: this lane's weights and cos/sin values of the q rows it stages (row i at position
  // offset (t / 16 + 16 i) % PB: 4 / G distinct positions, group i % NP; one from G = 4 on).
  constexpr int NP = FUSED && G < 4 ? 4 / G : 1;
  uint4 wq{}, cs4[NP], sn4[NP];
  if constexpr (FUSED) {
    wq = *reinterpret_cast<const uint4*>(qn_w + 8 * (tid & 15));
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      const int pos = min(p0 + ((tid >> 4) + 16 * pp) % PB, T - 1);
      cs4[pp] = *reinterpret_cast<const uint4*>(rope_cs + (int64_t)pos * 64 + (tid & 7) * 8);
      sn4[pp] = *reinterpret_cast<const uint4*>(rope_cs + ((int64_t)T + pos) * 64 + (tid & 7) * 8);
    }
  }

  const uint16_t* kbase = kc + kvh * head_stride;
  const uint16_t* vbase = vc + kvh * head_stride;
  const int kend = min(T, p0 + PB);  // keys the block reads
  const int nit = (kend + kStage - 1) / kStage;
  const int r0 = tid >> 4, ch = tid & 15;  // staging: key rows r0 + 16i, dims 8ch..8ch+7
  const __amdgpu_buffer_rsrc_t krs = kv_rsrc(kbase, T, tok_stride), vrs = kv_rsrc(vbase, T, tok_stride);
  const int ts2 = tok_stride * 2;  // bytes per key row
  int voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) voff[i] = (r0 + 16 * i) * ts2 + ch * 16;
  const auto stage = [&](const Staged& st, uint16_t* sk, uint16_t* sv) {
    uint16_t* kd = sk + r0 * kKStride + ch * 8;
    *reinterpret_cast<uint4*>(kd) = st.k0;
    *reinterpret_cast<uint4*>(kd + 16 * kKStride) = st.k1;
    *reinterpret_cast<uint4*>(kd + 32 * kKStride) = st.k2;
    *reinterpret_cast<uint4*>(kd + 48 * kKStride) = st.k3;
    uint16_t* vd = sv + r0 * kVStride + ch * 8;
    *reinterpret_cast<uint4*>(vd) = st.v0;
    *reinterpret_cast<uint4*>(vd + 16 * kVStride) = st.v1;
    *reinterpret_cast<uint4*>(vd + 32 * kVStride) = st.v2;
    *reinterpret_cast<uint4*>(vd + 48 * kVStride) = st.v3;
  };

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  float m = -INFINITY, lsum = 0.f;  // running max of raw scores; this lane's share of the row sum
  const float qs = qscale;

  Staged st = prefill_fetch(krs, vrs, voff, 0);
  if constexpr (FUSED) {
    __builtin_amdgcn_sched_barrier(0);  // block 0's loads issue first and fly meanwhile
    float c[NP][8], sn[NP][8];
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      unpack8(cs4[pp], c[pp]);
      unpack8(sn4[pp], sn[pp]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = qknorm_rope_row(qv[i], wq, c[i % NP], sn[i % NP], eps, tid & 15);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<uint4*>(&sK[1][((tid >> 4) + 16 * i) * kKStride + 8 * (tid & 15)]) = qv[i];
  stage(st, sK[0], sV[0]);
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  if (nit > 1) st = prefill_fetch(krs, vrs, voff, kStage * ts2);
  bf16x8 qb[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    qb[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(&sK[1][(32 * rg + l32) * kKStride + 16 * kk + 8 * hi]));
  lds_barrier();  // every wave holds its Q before the first iteration restages this buffer

  for (int j = 0; j < nit; ++j) {
    const int buf = j & 1;
    const int k0 = j * kStage + kh * kKeys;  // this half's 32 keys
    if (k0 < kend_w) {                         // wave-uniform
      // S^T for the 32 keys: s[i] = score of key k0 + 8(i/4) + 4hi + i%4.
      f32x16 s = f32x16{};
      const uint16_t* kr = &sK[buf][(kh * kKeys + l32) * kKStride + 8 * hi];
      bf16x8 ka[8];
#pragma unroll
      for (int g = 0; g < kKAhead; ++g) ka[g] = as_bf16x8(*reinterpret_cast<const uint4*>(kr + 16 * g));
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        if (g + kKAhead < 8) ka[g + kKAhead] = as_bf16x8(*reinterpret_cast<const uint4*>(kr + 16 * (g + kKAhead)));
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[g], qb[g], s, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      const uint16_t* vb = &sV[buf][(kh * kKeys + 4 * hi + ((lane & 15) >> 2)) * kVStride +
                                    16 * ((lane >> 4) & 1) + 4 * (lane & 3)];
      uint2 vlo[8], vup[8];
#pragma unroll
      for (int qq = 0; qq < kVAhead; ++qq) {
        const uint16_t* vr = vb + (16 * (qq >> 2)) * kVStride + 32 * (qq & 3);
        vlo[qq] = lds_read_tr16(vr);
        vup[qq] = lds_read_tr16(vr + 8 * kVStride);
      }
      if (k0 + kKeys - 1 > pw) {  // the keys cross this wave's diagonal: mask keys past each row
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = k0 + 8 * (i >> 2) + 4 * hi + (i & 3);
          if (key > qrow) s[i] = -INFINITY;
        }
      }
      float mx = s[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
      mx = xor32_combine(mx, [](float x, float y) { return fmaxf(x, y); });
      // Lazy maximum: a row keeps the reference max m it last rescaled to
      // until a stage's max exceeds it by more than 8 (log2 units), so p <= 2^8
      // and O is rescaled only on those rare steps.  Before its first visible
      // key a row has m = -inf and O = 0, l = 0, so it takes the stage's max
      // without rescaling.  Keys all masked for a row (mx = -inf) change nothing.
      const bool bump = mx * qs > m * qs + 8.f;
      const float mn = bump ? mx : m;
      const float mq = mn == -INFINITY ? 0.f : mn * qs;
      const float alpha = (bump && m != -INFINITY) ? fast_exp2(m * qs - mq) : 1.f;
      // p in bf16 pairs.  bf16 output: p enters P V rounded to bf16 and the row
      // sum adds the rounded p.  fp32 output: p enters as a bf16 high part plus
      // the bf16 remainder (two MFMAs, ~16 bits of p) and the row sum adds p in
      // fp32, which keeps the output within 1e-4 of exact attention.
      float ps = 0.f;
      uint32_t pk[8];            // bf16 pairs of p (high parts)
      uint32_t pl[F32 ? 8 : 1];  // fp32 output: the remainders p - high
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float e0 = fast_exp2(fmaf(s[i], qs, -mq)), e1 = fast_exp2(fmaf(s[i + 1], qs, -mq));
        const uint32_t pr = pack2(e0, e1);
        pk[i >> 1] = pr;
        if constexpr (F32) {
          pl[i >> 1] = pack2(e0 - __uint_as_float(pr << 16), e1 - __uint_as_float(pr & 0xffff0000u));
          ps += e0 + e1;
        } else {
          ps = dot2bf(pr, 0x3f803f80u, ps);  // + p_lo + p_hi
        }
      }
      lsum = fmaf(lsum, alpha, ps);
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // some row's reference max moved
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
      }
      m = mn;
      // O^T += V^T P^T: step qq = (h, dt) = (qq / 4, qq % 4) covers keys k0 + 16h + {4hi + 0..3,
      // 8 + 4hi + 0..3}; the V operand of step qq + kVAhead is read before MFMA qq issues.
#pragma unroll
      for (int qq = 0; qq < 8; ++qq) {
        if (qq + kVAhead < 8) {
          const uint16_t* vr = vb + (16 * ((qq + kVAhead) >> 2)) * kVStride + 32 * ((qq + kVAhead) & 3);
          vlo[qq + kVAhead] = lds_read_tr16(vr);
          vup[qq + kVAhead] = lds_read_tr16(vr + 8 * kVStride);
        }
        const int h = qq >> 2;
        const bf16x8 pb = as_bf16x8(make_uint4(pk[4 * h], pk[4 * h + 1], pk[4 * h + 2], pk[4 * h + 3]));
        const bf16x8 va = as_bf16x8(make_uint4(vlo[qq].x, vlo[qq].y, vup[qq].x, vup[qq].y));
        o[qq & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, o[qq & 3], 0, 0, 0);
        if constexpr (F32) {
          const bf16x8 pbl = as_bf16x8(make_uint4(pl[4 * h], pl[4 * h + 1], pl[4 * h + 2], pl[4 * h + 3]));
          o[qq & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pbl, o[qq & 3], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // The last stage stages and fetches nothing (a load left in flight would hold the epilogue);
    // its barrier stays: the merge below reuses the staging buffers.
    if (j + 1 < nit) stage(st, sK[(j + 1) & 1], sV[(j + 1) & 1]);  // block-uniform
    lds_barrier();  // orders the LDS tiles only: the loads below stay in flight
    if (j + 2 < nit) st = prefill_fetch(krs, vrs, voff, (j + 2) * kStage * ts2);
  }

  SOLORT_STAMP(tid == 0, (int)blockIdx.x, 3);
  // Merge the two key halves of every row, each half finishing 64 of the 128
  // dims: half 0 dims 0..63 (o[0], o[1]), half 1 dims 64..127 (o[2], o[3]).
  // Each wave hands the other half's dims and its (m, l) over through LDS (the
  // staging buffers are free after the last barrier): region 2 rg + kh of
  // kXWords floats, [8][64] float4 items (o[2 (1 - kh) + d][4 q .. 4 q + 3] at
  // item 4 d + q) and [64] float2 (m, l).  Both halves then merge with half
  // 0's values first (the same expressions in either wave), stage their 64 dims
  // of the 32 rows row-major in `theirs` (read before, in program order; the
  // other half never touches it again), and each store instruction writes whole
  // 128-byte (bf16) or 256-byte (fp32) half rows.
  constexpr int kXWords = 34 * 64;
  float* const xs = reinterpret_cast<float*>(&sK[0][0]);
  float* const mine = xs + (2 * rg + kh) * kXWords;
  float* const theirs = xs + (2 * rg + 1 - kh) * kXWords;
  static_assert(4 * kXWords * 4 <= 2 * kStage * kKStride * 2, "the exchange regions fit the K staging buffers");
  const auto hand_over = [&](auto khc) {
    constexpr int OTHER = 2 - 2 * decltype(khc)::value;
    float4* const m4 = reinterpret_cast<float4*>(mine);
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        m4[(4 * d + q4) * 64 + lane] = make_float4(o[OTHER + d][4 * q4], o[OTHER + d][4 * q4 + 1],
                                                   o[OTHER + d][4 * q4 + 2], o[OTHER + d][4 * q4 + 3]);
    reinterpret_cast<float2*>(mine + 32 * 64)[lane] = make_float2(m, lsum);
  };
  // Block row of wave row r: position p0 + (32 rg + r) % PB, head kvh * G + (32 rg + r) / PB.
  const int64_t orow = (int64_t)nh * SOLORT_HD;
  const auto out_off = [&](int r) -> int64_t {
    const int R = 32 * rg + r;
    return (int64_t)(p0 + R % PB) * orow + (int64_t)(kvh * G + R / PB) * SOLORT_HD;
  };
  const auto finish = [&](auto khc) {
    constexpr int KH = decltype(khc)::value;
    constexpr int OWN = 2 * KH;
    const float2 ml = reinterpret_cast<const float2*>(theirs + 32 * 64)[lane];
    const float m0 = KH == 0 ? m : ml.x, l0 = KH == 0 ? lsum : ml.y;
    const float m1 = KH == 0 ? ml.x : m, l1 = KH == 0 ? ml.y : lsum;
    const float mt = fmaxf(m0, m1);  // finite: half 0 saw key 0
    const float a0 = fast_exp2((m0 - mt) * qs), a1 = fast_exp2((m1 - mt) * qs);  // m1 = -inf gives 0
    const float lt = xor32_combine(fmaf(l0, a0, l1 * a1), [](float x, float y) { return x + y; });
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const float4* const t4 = reinterpret_cast<const float4*>(theirs);
    float r[2][16];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 v = t4[(4 * d + q4) * 64 + lane];
        const float vo[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float own = o[OWN + d][4 * q4 + e];
          const float h0 = KH == 0 ? own : vo[e], h1 = KH == 0 ? vo[e] : own;
          r[d][4 * q4 + e] = fmaf(h0, a0, h1 * a1) * inv;
        }
      }
    if constexpr (F32) {
      constexpr int kOS = 64 + 4;
      static_assert(32 * kOS <= kXWords, "fp32 staging fits the region");
#pragma unroll
      for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4*>(theirs + l32 * kOS + 32 * d + 8 * g + 4 * hi) =
              make_float4(r[d][4 * g], r[d][4 * g + 1], r[d][4 * g + 2], r[d][4 * g + 3]);
      float* out = reinterpret_cast<float*>(out_ptr) + 64 * KH;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int row = 4 * it + (lane >> 4), c = 4 * (lane & 15);
        const float4 v = *reinterpret_cast<const float4*>(theirs + row * kOS + c);
        typedef float f32x4n __attribute__((ext_vector_type(4)));
        if (p0 + (32 * rg + row) % PB < T)
          __builtin_nontemporal_store(f32x4n{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4n*>(out + out_off(row) + c));
      }
    } else {
      constexpr int kOS = 64 + 8;
      uint16_t* xo = reinterpret_cast<uint16_t*>(theirs);
#pragma unroll
      for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint2 pkd;
          pkd.x = pack2(r[d][4 * g], r[d][4 * g + 1]);
          pkd.y = pack2(r[d][4 * g + 2], r[d][4 * g + 3]);
          *reinterpret_cast<uint2*>(xo + l32 * kOS + 32 * d + 8 * g + 4 * hi) = pkd;
        }
      uint16_t* out = reinterpret_cast<uint16_t*>(out_ptr) + 64 * KH;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int row = 8 * it + (lane >> 3), c = 8 * (lane & 7);
        const uint4 v = *reinterpret_cast<const uint4*>(xo + row * kOS + c);
        typedef unsigned u32x4n __attribute__((ext_vector_type(4)));
        if (p0 + (32 * rg + row) % PB < T)
          __builtin_nontemporal_store(u32x4n{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4n*>(out + out_off(row) + c));
      }
    }
  };
  if (kh == 0)
    hand_over(std::integral_constant<int, 0>{});
  else
    hand_over(std::integral_constant<int, 1>{});
  __syncthreads();
  if (kh == 0)
    finish(std::integral_constant<int, 0>{});
  else
    finish(std::integral_constant<int, 1>{});
  SOLORT_STAMP(tid == 0, (int)blockIdx.x, 5);
}

}  // namespace solort

using namespace solort;

// Checks shared by the prefill entry points; 0 or the error code.
static int check_prefill(const char* name, int T, int nh, int nkv, int hd, const void* k_cache, const void* v_cache,
                         int64_t kv_tok_stride, int64_t kv_head_stride, int64_t max_len, void* out, int out_dtype) {
  if (hd != SOLORT_HD) return set_error(SOLORT_EINVAL, "%s: head_dim %d != 128", name, hd);
  if (nh <= 0 || nkv <= 0 || nh % nkv != 0)
    return set_error(SOLORT_EINVAL, "%s: nh=%d must be a positive multiple of nkv=%d", name, nh, nkv);
  const int G = nh / nkv;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return set_error(SOLORT_EINVAL, "%s: query group %d not in {1,2,4,8}", name, G);
  if (nkv > 255) return set_error(SOLORT_EINVAL, "%s: nkv=%d above 255", name, nkv);
  if (T < 0 || T > max_len || T >= (1 << 24))
    return set_error(SOLORT_EINVAL, "%s: T=%d outside [0, max_len=%lld]", name, T, (long long)max_len);
  if (!k_cache || !v_cache || !out) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (kv_tok_stride <= 0 || kv_head_stride <= 0 || kv_tok_stride % 8 || kv_head_stride % 8)
    return set_error(SOLORT_EINVAL, "%s: KV strides must be positive multiples of 8", name);
  if (out_dtype != SOLORT_DTYPE_BF16 && out_dtype != SOLORT_DTYPE_F32)
    return set_error(SOLORT_EINVAL, "%s: out_dtype %d", name, out_dtype);
  // K/V rows are addressed with 32-bit byte offsets from the head's row 0, up
  // to one stage past T; the kernel takes 32-bit strides, the heads'
  // offsets within 2^31 elements of the cache base.
  if (((int64_t)T + 4 * kStage) * kv_tok_stride * 2 >= ((int64_t)1 << 31))
    return set_error(SOLORT_EINVAL, "%s: T=%d rows of stride %lld exceed 32-bit byte offsets", name, T,
                     (long long)kv_tok_stride);
  if ((int64_t)nkv * kv_head_stride >= ((int64_t)1 << 31))
    return set_error(SOLORT_EINVAL, "%s: KV head stride %lld exceeds 32-bit offsets", name,
                     (long long)kv_head_stride);
  return 0;
}

// The attention launch; q rows at q + pos * q_stride (elements), fused: raw
// q rows normalised in the kernel.
static int launch_prefill(const char* name, const void* q, int64_t q_stride, bool fused, const void* qn_w,
                          const void* rope_cs, float eps, int T, int nh, int nkv, const void* k_cache,
                          const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride, float scale, void* out,
                          int out_dtype, hipStream_t s) {
  if (q_stride > 0x7fffffff) return set_error(SOLORT_EINVAL, "%s: q row stride %lld too large", name, (long long)q_stride);
  const int G = nh / nkv;
  const int pb = 64 / G;  // positions per block
  const int n_qtiles = (T + pb - 1) / pb;
  const int64_t blocks = (int64_t)n_qtiles * nkv;
  if (blocks > 0x7fffffff) return set_error(SOLORT_EINVAL, "%s: too many tiles", name);
  const float qscale = scale * 1.4426950408889634f;
  const bool f32 = out_dtype == SOLORT_DTYPE_F32;
  const int t_nkv = T | nkv << 24;
  const int round = cu_count() / nkv > 0 ? cu_count() / nkv : 1;  // blocks per KV head, one per CU
#define SOLORT_PREFILL_LAUNCH(GG, FF, QQ)                                                                          \
  hipLaunchKernelGGL((prefill_kernel<GG, FF, QQ>), dim3((unsigned)blocks), dim3(kThreads), 0, s, (const uint16_t*)q, \
                     (const uint16_t*)k_cache, (const uint16_t*)v_cache, (const uint16_t*)qn_w,                      \
                     (const uint16_t*)rope_cs, t_nkv, (int)kv_tok_stride, (int)kv_head_stride, (int)q_stride, round, \
                     qscale, eps, out)
  switch (G * 4 + (f32 ? 2 : 0) + (fused ? 1 : 0)) {
    case 4: SOLORT_PREFILL_LAUNCH(1, false, false); break;
    case 5: SOLORT_PREFILL_LAUNCH(1, false, true); break;
    case 6: SOLORT_PREFILL_LAUNCH(1, true, false); break;
    case 7: SOLORT_PREFILL_LAUNCH(1, true, true); break;
    case 8: SOLORT_PREFILL_LAUNCH(2, false, false); break;
    case 9: SOLORT_PREFILL_LAUNCH(2, false, true); break;
    case 10: SOLORT_PREFILL_LAUNCH(2, true, false); break;
    case 11: SOLORT_PREFILL_LAUNCH(2, true, true); break;
    case 16: SOLORT_PREFILL_LAUNCH(4, false, false); break;
    case 17: SOLORT_PREFILL_LAUNCH(4, false, true); break;
    case 18: SOLORT_PREFILL_LAUNCH(4, true, false); break;
    case 19: SOLORT_PREFILL_LAUNCH(4, true, true); break;
    case 32: SOLORT_PREFILL_LAUNCH(8, false, false); break;
    case 33: SOLORT_PREFILL_LAUNCH(8, false, true); break;
    case 34: SOLORT_PREFILL_LAUNCH(8, true, false); break;
    case 35: SOLORT_PREFILL_LAUNCH(8, true, true); break;
  }
#undef SOLORT_PREFILL_LAUNCH
  return check_launch(name);
}

extern "C" int solort_prefill_attn(const void* q, int T, int nh, int nkv, int hd, const void* k_cache,
                                   const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                                   int64_t max_len, float scale, void* out, int out_dtype,
                                   solort_stream_t stream) {
  const char* name = "prefill_attn";
  int rc = check_prefill(name, T, nh, nkv, hd, k_cache, v_cache, kv_tok_stride, kv_head_stride, max_len, out,
                         out_dtype);
  if (rc) return rc;
  if (!q) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(q)) return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (T == 0) return 0;
  return launch_prefill(name, q, (int64_t)nh * SOLORT_HD, false, nullptr, nullptr, 0.f, T, nh, nkv, k_cache, v_cache,
                        kv_tok_stride, kv_head_stride, scale, out, out_dtype, (hipStream_t)stream);
}

extern "C" int solort_prefill_layer(const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv, int hd,
                                    const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                                    void* k_cache, void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                                    int64_t max_len, float scale, void* out, int out_dtype, solort_stream_t stream) {
  const char* name = "prefill_layer";
  // q_out is not materialised: out stands in for it in the null/alignment checks.
  int rc = check_prologue(name, qkv, qkv_row_stride, T, nh, nkv, hd, qn_w, kn_w, rope_cs, out, k_cache, v_cache,
                          kv_tok_stride, kv_head_stride, max_len);
  if (rc) return rc;
  rc = check_prefill(name, T, nh, nkv, hd, k_cache, v_cache, kv_tok_stride, kv_head_stride, max_len, out, out_dtype);
  if (rc || T == 0) return rc;
  hipStream_t s = (hipStream_t)stream;
  rc = launch_kv_rows_cs(qkv, qkv_row_stride, T, nh, nkv, kn_w, eps, rope_cs, k_cache, v_cache, kv_tok_stride,
                         kv_head_stride, max_len, s);
  if (rc) return rc;
  return launch_prefill(name, qkv, qkv_row_stride, true, qn_w, rope_cs, eps, T, nh, nkv, k_cache, v_cache,
                        kv_tok_stride, kv_head_stride, scale, out, out_dtype, s);
}

#ifdef SOLORT_PHASE_STAMPS
// Tracing build: copies the phase stamps of prefill_kernel's most recent
// launch (n_blocks workgroups) to host.
extern "C" int solort_phase_stamps_prefill(void* host, int n_blocks) {
  if (!host || n_blocks < 1 || n_blocks > kStampBlocks) return set_error(SOLORT_EINVAL, "phase_stamps_prefill: bad arguments");
  const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(g_phase_stamps), (size_t)n_blocks * kStampSlots * 8, 0,
                                           hipMemcpyDeviceToHost);
  return e == hipSuccess ? 0 : set_error((int)e, "phase_stamps_prefill: %s", hipGetErrorString(e));
}
#endif
