// Causal grouped-query prefill attention on bf16 MFMA (gfx950).
//
// Reference: src/solort/model/cuda_graph_executor.py:124-130, i.e.
//   SDPA(q, repeat_interleave(k, g), repeat_interleave(v, g), is_causal=True,
//        scale=hd**-0.5) over the T prompt rows, written as ctx [T, nh*128].
// K and V are read from the cache rows 0..T-1 the prologue just wrote (the
// reference attends the same k/v values it writes at :122-123).  No repeat:
// the g query heads of a KV head share every K/V tile staged in LDS.
//
// Block = 4 wavefronts = (KV head, tile of 16*(4/g) query rows); wave w owns
// query head kvh*g + w%g and 16 query rows.  Per 64-key block:
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16, A = K tile (LDS, row-major),
//                 B = Q^T (registers), 4 key tiles x 4 dim steps
//   online softmax in fp32 (log2 domain), P rounded to bf16
//   O^T += V^T P^T  A = V^T (LDS, stored transposed), B = P^T (registers),
//                 8 dim tiles x 2 key steps
// Operand layouts (checked on gfx950): A[m][k] lane l holds
// A[l%16][8(l/16)+s]; B[k][n] lane l holds B[8(l/16)+s][l%16]; D[m][n] lane l
// holds D[4(l/16)+i][l%16].  With S^T and O^T every lane keeps one query row
// (l%16), so softmax statistics never move between lanes except for the row
// max (two lane exchanges).  The MFMA's key index is a permutation of the
// block's keys shared by A and B, which lets P^T be fed straight from the
// registers that hold S^T.
// Causal: a tile reads only key blocks up to its last row and masks keys past
// each row; tiles are dispatched heaviest first.
#include <math.h>

#include "common.h"
#include "capi_internal.h"

namespace solort {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const uint16_t* q;  // [T][nh][128]
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t tok_stride, head_stride;
  void* out;     // [T][nh * 128]
  float qscale;  // softmax scale * log2(e)
  int T, nh, nkv, n_qtiles, out_f32;
};

constexpr int kKeys = 64;        // keys per staged block
constexpr int kKStride = 128 + 8;  // K tile row stride (bf16), 272 bytes
constexpr int kVStride = 64 + 4;   // V^T tile row stride (bf16), 136 bytes

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4 v) { return __builtin_bit_cast(bf16x8, v); }

template <int G>
__global__ __launch_bounds__(256) void prefill_kernel(const PrefillArgs a) {
  constexpr int RW = 16 * (4 / G);  // query rows per block
  __shared__ __align__(16) uint16_t sK[kKeys * kKStride];
  __shared__ __align__(16) uint16_t sVt[128 * kVStride];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;  // MFMA row / lane group
  const int kvh = blockIdx.x % a.nkv;
  const int tile = a.n_qtiles - 1 - (int)(blockIdx.x / a.nkv);  // heaviest first
  const int q0 = tile * RW;
  const int head = kvh * G + (wave % G);
  const int qrow = q0 + (wave / G) * 16 + lr;  // query row of this lane's scores

  bf16x8 qb[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (qrow < a.T)
      v = *reinterpret_cast<const uint4*>(a.q + ((int64_t)qrow * a.nh + head) * SOLORT_HD + 32 * ks + 8 * lg);
    qb[ks] = as_bf16x8(v);
  }
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;

  const uint16_t* kbase = a.kc + (int64_t)kvh * a.head_stride;
  const uint16_t* vbase = a.vc + (int64_t)kvh * a.head_stride;
  const int kend = min(a.T, q0 + RW);
  const int kg = tid >> 4, dg = tid & 15;  // V^T staging: 4 keys x 8 dims per thread

  // Global loads of a block's K rows (4 chunks of 16 B per thread) and V rows
  // (4 keys x 8 dims per thread); rows at or past T read as zero.
  uint4 kv[4], vv[4];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, r = c >> 4, ch = c & 15;
      kv[i] = (kb + r < a.T) ? *reinterpret_cast<const uint4*>(kbase + (int64_t)(kb + r) * a.tok_stride + ch * 8)
                             : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * kg + i;
      vv[i] = (kb + r < a.T) ? *reinterpret_cast<const uint4*>(vbase + (int64_t)(kb + r) * a.tok_stride + dg * 8)
                             : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  fetch(0);

  for (int k0 = 0; k0 < kend; k0 += kKeys) {
    // Stage the fetched block: K [64][128] row-major, V^T [128][64].
    __syncthreads();  // the previous block's tiles are no longer read
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, r = c >> 4, ch = c & 15;
      *reinterpret_cast<uint4*>(sK + r * kKStride + ch * 8) = kv[i];
    }
    {
      const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&vv[0]);
      const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&vv[1]);
      const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&vv[2]);
      const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&vv[3]);
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const int sh = (d & 1) * 16, wi = d >> 1;
        uint2 pk;
        pk.x = ((w0[wi] >> sh) & 0xffffu) | (((w1[wi] >> sh) & 0xffffu) << 16);
        pk.y = ((w2[wi] >> sh) & 0xffffu) | (((w3[wi] >> sh) & 0xffffu) << 16);
        *reinterpret_cast<uint2*>(sVt + (dg * 8 + d) * kVStride + 4 * kg) = pk;
      }
    }
    __syncthreads();
    // The next block's global loads fly while this block is computed.
    if (k0 + kKeys < kend) fetch(k0 + kKeys);

    // S^T = K Q^T for the block's 64 keys.
    f32x4 s[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 ka = as_bf16x8(*reinterpret_cast<const uint4*>(sK + (kt * 16 + lr) * kKStride + 32 * ks + 8 * lg));
        s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[ks], s[kt], 0, 0, 0);
      }
    }
    // Scale, causal mask, online softmax for row qrow.
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = k0 + kt * 16 + 4 * lg + i;
        float v = s[kt][i] * a.qscale;
        if (key > qrow || key >= a.T) v = -INFINITY;
        s[kt][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, xshfl(mx, 16));
    mx = fmaxf(mx, xshfl(mx, 32));
    const float mn = fmaxf(m, mx);
    const bool live = mn != -INFINITY;
    const float alpha = live ? fast_exp2(m - mn) : 1.f;
    float ps = 0.f;
    uint32_t pw[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = live ? fast_exp2(s[kt][i] - mn) : 0.f;
        ps += p[i];
      }
      pw[kt][0] = f2bf(p[0]) | (f2bf(p[1]) << 16);
      pw[kt][1] = f2bf(p[2]) | (f2bf(p[3]) << 16);
    }
    lsum = lsum * alpha + ps;
    m = mn;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;

    // O^T += V^T P^T over the block's two 32-key halves.
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const bf16x8 pb = as_bf16x8(make_uint4(pw[2 * c][0], pw[2 * c][1], pw[2 * c + 1][0], pw[2 * c + 1][1]));
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint16_t* vrow = sVt + (dt * 16 + lr) * kVStride + 32 * c + 4 * lg;
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16);
        const bf16x8 va = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, o[dt], 0, 0, 0);
      }
    }
  }

  float lt = lsum + xshfl(lsum, 16);
  lt += xshfl(lt, 32);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (qrow < a.T) {
    const int64_t base = ((int64_t)qrow * a.nh + head) * SOLORT_HD + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const float4 v = make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
      if (a.out_f32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + base + dt * 16) = v;
      } else {
        uint2 pk;
        pk.x = f2bf(v.x) | (f2bf(v.y) << 16);
        pk.y = f2bf(v.z) | (f2bf(v.w) << 16);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + base + dt * 16) = pk;
      }
    }
  }
}

}  // namespace solort

using namespace solort;

extern "C" int solort_prefill_attn(const void* q, int T, int nh, int nkv, int hd, const void* k_cache,
                                   const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                                   int64_t max_len, float scale, void* out, int out_dtype,
                                   solort_stream_t stream) {
  const char* name = "prefill_attn";
  if (hd != SOLORT_HD) return set_error(SOLORT_EINVAL, "%s: head_dim %d != 128", name, hd);
  if (nh <= 0 || nkv <= 0 || nh % nkv != 0)
    return set_error(SOLORT_EINVAL, "%s: nh=%d must be a positive multiple of nkv=%d", name, nh, nkv);
  const int G = nh / nkv;
  if (G != 1 && G != 2 && G != 4) return set_error(SOLORT_EINVAL, "%s: query group %d not in {1,2,4}", name, G);
  if (T < 0 || T > max_len || T > (1 << 24))
    return set_error(SOLORT_EINVAL, "%s: T=%d outside [0, max_len=%lld]", name, T, (long long)max_len);
  if (!q || !k_cache || !v_cache || !out) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (kv_tok_stride <= 0 || kv_head_stride <= 0 || kv_tok_stride % 8 || kv_head_stride % 8)
    return set_error(SOLORT_EINVAL, "%s: KV strides must be positive multiples of 8", name);
  if (out_dtype != SOLORT_DTYPE_BF16 && out_dtype != SOLORT_DTYPE_F32)
    return set_error(SOLORT_EINVAL, "%s: out_dtype %d", name, out_dtype);
  if (T == 0) return 0;
  PrefillArgs a;
  a.q = (const uint16_t*)q;
  a.kc = (const uint16_t*)k_cache;
  a.vc = (const uint16_t*)v_cache;
  a.tok_stride = kv_tok_stride;
  a.head_stride = kv_head_stride;
  a.out = out;
  a.qscale = scale * 1.4426950408889634f;
  a.T = T;
  a.nh = nh;
  a.nkv = nkv;
  a.out_f32 = out_dtype == SOLORT_DTYPE_F32;
  const int rw = 16 * (4 / G);
  a.n_qtiles = (T + rw - 1) / rw;
  const int64_t blocks = (int64_t)a.n_qtiles * nkv;
  if (blocks > 0x7fffffff) return set_error(SOLORT_EINVAL, "%s: too many tiles", name);
  hipStream_t s = (hipStream_t)stream;
  switch (G) {
    case 1: hipLaunchKernelGGL(prefill_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(prefill_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(prefill_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
  }
  return check_launch(name);
}
