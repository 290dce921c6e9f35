// Split-KV (flash-decoding) grouped-query attention for 1..8 new tokens over
// the static KV cache, with the log-sum-exp combine fused into the launch.
//
// Reference semantics (src/solort/model/cuda_graph_executor.py):
//   decode :168, :180-184  qg = q.reshape(nkv, g, hd); softmax(qg K^T * scale,
//                          keys > pos masked) V over the bucket  (nq = 1)
//   verify :247-250, :261-263  query t at position pos0+t attends keys
//                          0..pos0+t of the cache                (nq = K+1)
// Scores, softmax and the weighted sum are computed in fp32 (the reference
// rounds scores and probabilities to bf16 between its torch ops); the output
// is rounded once, to bf16, or left in fp32 on request.
//
// Grid: nkv * n_split workgroups of 256 threads.  Block b serves KV head
// b % nkv and key split b / nkv, so consecutive blocks walk the KV heads and
// (with 8 KV heads on 8 XCDs, blocks dealt round-robin) all splits of one head
// share one XCD and its L2, where the combine reads their partials.
// Inside a block, 16 row slots of 16 lanes each take one key row per step;
// lane j of a slot loads dims [8j, 8j+8) of K and V as 16-byte vectors and
// keeps the q rows of the whole query group (nq * g rows) in registers, so
// the KV head is read once for all of its query heads (no repeat_interleave).
// The last block of a KV head to finish (atomic ticket) merges the splits'
// (max, sum, unnormalised output) partials and writes the result, then resets
// its ticket so the workspace is ready for the next launch.
#include <math.h>

#include "common.h"
#include "capi_internal.h"

namespace solort {

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t tok_stride;
  int64_t head_stride;
  const int64_t* pos0_dev;
  float* ws_o;       // [nkv][n_split][R][128]
  float* ws_ml;      // [nkv][n_split][R][2]  (running max in log2 units, sum)
  unsigned* ws_cnt;  // [nkv] tickets, zero between launches
  void* out;         // [nq][nh][128]
  float qscale;      // softmax scale * log2(e)
  int nh, nkv, bound, n_split, out_f32;
};

template <int NQ, int G, int U>
__global__ __launch_bounds__(256) void splitkv_attn_kernel(const AttnArgs a) {
  constexpr int R = NQ * G;  // query rows sharing one KV head
  extern __shared__ float smem[];
  __shared__ unsigned s_ticket;

  const int tid = threadIdx.x, j = tid & 15, slot = tid >> 4, wave = tid >> 6;
  const int kvh = blockIdx.x % a.nkv;
  const int split = blockIdx.x / a.nkv;

  const int64_t pos0 = a.pos0_dev[0];
  int64_t live64 = pos0 + NQ;  // keys [0, live) exist for the last query
  live64 = live64 < 0 ? 0 : (live64 > a.bound ? a.bound : live64);
  const int live = (int)live64;
  int chunk = (live + a.n_split - 1) / a.n_split;
  chunk = (chunk + 15) & ~15;
  const int kbeg = min(split * chunk, live);
  const int kend = min(kbeg + chunk, live);

  float qf[R][8];
#pragma unroll
  for (int t = 0; t < NQ; ++t)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x[8];
      unpack8(*reinterpret_cast<const uint4*>(a.q + ((int64_t)t * a.nh + kvh * G + g) * SOLORT_HD + j * 8), x);
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[t * G + g][i] = x[i] * a.qscale;
    }

  float m[R], l[R], acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[r][i] = 0.f;
  }

  const uint16_t* kp = a.kc + (int64_t)kvh * a.head_stride + j * 8;
  const uint16_t* vp = a.vc + (int64_t)kvh * a.head_stride + j * 8;
  for (int k0 = kbeg; k0 < kend; k0 += 16 * U) {
    uint4 kr[U], vr[U];
    int kid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kid[u] = k0 + u * 16 + slot;
      if (kid[u] < kend) {
        kr[u] = *reinterpret_cast<const uint4*>(kp + (int64_t)kid[u] * a.tok_stride);
        vr[u] = *reinterpret_cast<const uint4*>(vp + (int64_t)kid[u] * a.tok_stride);
      } else {
        kr[u] = make_uint4(0u, 0u, 0u, 0u);
        vr[u] = make_uint4(0u, 0u, 0u, 0u);
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
      for (int r = 0; r < R; ++r) {
        float d = s[u][r];
        d += xshfl(d, 8);
        d += xshfl(d, 4);
        d += xshfl(d, 2);
        d += xshfl(d, 1);
        s[u][r] = d;
      }
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
  }

  // Merge the 4 row slots of each wavefront (lane distance 16 and 32).
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

  // Merge the 4 wavefronts through LDS into this split's partial.
  float* s_acc = smem;              // [4][R][128]
  float* s_m = smem + 4 * R * 128;  // [4][R]
  float* s_l = s_m + 4 * R;         // [4][R]
  if ((tid & 63) < 16) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int i = 0; i < 8; ++i) s_acc[(wave * R + r) * 128 + j * 8 + i] = acc[r][i];
      if (j == 0) {
        s_m[wave * R + r] = m[r];
        s_l[wave * R + r] = l[r];
      }
    }
  }
  __syncthreads();
  {
    float* wo = a.ws_o + (int64_t)(kvh * a.n_split + split) * R * 128;
    float* wml = a.ws_ml + (int64_t)(kvh * a.n_split + split) * R * 2;
    for (int e = tid; e < R * 128; e += 256) {
      const int r = e >> 7, d = e & 127;
      float M = s_m[r];
#pragma unroll
      for (int w = 1; w < 4; ++w) M = fmaxf(M, s_m[w * R + r]);
      float O = 0.f, L = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float mw = s_m[w * R + r];
        const float sc = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
        O += s_acc[(w * R + r) * 128 + d] * sc;
        L += s_l[w * R + r] * sc;
      }
      wo[r * 128 + d] = O;
      if (d == 0) {
        wml[r * 2] = M;
        wml[r * 2 + 1] = L;
      }
    }
  }

  // Publish the partial; the last block of this KV head combines.
  fence_release_agent();
  __syncthreads();
  if (tid == 0)
    s_ticket = __hip_atomic_fetch_add(a.ws_cnt + kvh, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_ticket != (unsigned)(a.n_split - 1)) return;
  fence_acquire_agent();

  const int NS = a.n_split;
  float* s_w = smem;             // [NS][R]: max, then combine weight
  float* s_ll = smem + NS * R;   // [NS][R]: sum
  float* s_M = s_ll + NS * R;    // [R]
  float* s_L = s_M + R;          // [R]
  const float* wml_all = a.ws_ml + (int64_t)kvh * NS * R * 2;
  for (int e = tid; e < NS * R; e += 256) {
    s_w[e] = wml_all[2 * e];
    s_ll[e] = wml_all[2 * e + 1];
  }
  __syncthreads();
  if (tid < R) {
    float M = -INFINITY;
    for (int s = 0; s < NS; ++s) M = fmaxf(M, s_w[s * R + tid]);
    float L = 0.f;
    for (int s = 0; s < NS; ++s) {
      const float ms = s_w[s * R + tid];
      if (ms != -INFINITY) L += s_ll[s * R + tid] * fast_exp2(ms - M);
    }
    s_M[tid] = M;
    s_L[tid] = L > 0.f ? 1.f / L : 0.f;
  }
  __syncthreads();
  for (int e = tid; e < NS * R; e += 256) {
    const int r = e % R;
    const float ms = s_w[e];
    s_w[e] = (ms == -INFINITY) ? 0.f : fast_exp2(ms - s_M[r]) * s_L[r];
  }
  __syncthreads();
  const float* wo_all = a.ws_o + (int64_t)kvh * NS * R * 128;
  for (int e = tid; e < R * 128; e += 256) {
    const int r = e >> 7, d = e & 127;
    float O = 0.f;
    for (int s = 0; s < NS; ++s) O = fmaf(s_w[s * R + r], wo_all[((int64_t)s * R + r) * 128 + d], O);
    const int t = r / G, g = r % G;
    const int64_t oi = ((int64_t)t * a.nh + kvh * G + g) * SOLORT_HD + d;
    if (a.out_f32)
      reinterpret_cast<float*>(a.out)[oi] = O;
    else
      reinterpret_cast<uint16_t*>(a.out)[oi] = (uint16_t)f2bf(O);
  }
  if (tid == 0) a.ws_cnt[kvh] = 0u;
}

// ---------------------------------------------------------------- host side

constexpr int kMaxRows = 24;      // nq * group limit (register budget)
constexpr int kMaxSplit = 1024;

struct WsLayout {
  size_t o_off, ml_off, cnt_off, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static WsLayout ws_layout(int nq, int nh, int nkv, int n_split) {
  const size_t R = (size_t)nq * (nh / nkv);
  WsLayout w;
  w.o_off = 0;
  w.ml_off = align256(w.o_off + (size_t)nkv * n_split * R * 128 * sizeof(float));
  w.cnt_off = align256(w.ml_off + (size_t)nkv * n_split * R * 2 * sizeof(float));
  w.total = align256(w.cnt_off + (size_t)nkv * sizeof(unsigned));
  return w;
}

template <int NQ, int G, int U>
static void launch_one(const AttnArgs& a, int blocks, size_t smem, hipStream_t s) {
  hipLaunchKernelGGL((splitkv_attn_kernel<NQ, G, U>), dim3(blocks), dim3(256), smem, s, a);
}

template <int NQ, int G>
static bool launch_u(int U, const AttnArgs& a, int blocks, size_t smem, hipStream_t s) {
  if constexpr (NQ * G <= kMaxRows) {
    if (U == 4 && NQ == 1) launch_one<NQ, G, 4>(a, blocks, smem, s);
    else launch_one<NQ, G, 2>(a, blocks, smem, s);
    return true;
  } else {
    return false;
  }
}

template <int G>
static bool launch_nq(int nq, int U, const AttnArgs& a, int blocks, size_t smem, hipStream_t s) {
  switch (nq) {
    case 1: return launch_u<1, G>(U, a, blocks, smem, s);
    case 2: return launch_u<2, G>(U, a, blocks, smem, s);
    case 3: return launch_u<3, G>(U, a, blocks, smem, s);
    case 4: return launch_u<4, G>(U, a, blocks, smem, s);
    case 5: return launch_u<5, G>(U, a, blocks, smem, s);
    case 6: return launch_u<6, G>(U, a, blocks, smem, s);
    case 7: return launch_u<7, G>(U, a, blocks, smem, s);
    case 8: return launch_u<8, G>(U, a, blocks, smem, s);
  }
  return false;
}

static int attn_impl(const char* name, const void* q, int nq, int nh, int nkv, int hd,
                     const void* k_cache, const void* v_cache, int64_t kv_tok_stride,
                     int64_t kv_head_stride, int64_t max_len, const int64_t* pos0_dev, int bound,
                     float scale, void* ws, int n_split, void* out, int out_dtype,
                     solort_stream_t stream) {
  if (hd != SOLORT_HD) return set_error(SOLORT_EINVAL, "%s: head_dim %d != 128", name, hd);
  if (nh <= 0 || nkv <= 0 || nh % nkv != 0)
    return set_error(SOLORT_EINVAL, "%s: nh=%d must be a positive multiple of nkv=%d", name, nh, nkv);
  const int G = nh / nkv;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return set_error(SOLORT_EINVAL, "%s: query group %d not in {1,2,4,8}", name, G);
  if (nq < 1 || nq > 8 || nq * G > kMaxRows)
    return set_error(SOLORT_EINVAL, "%s: nq=%d with group %d exceeds %d query rows", name, nq, G, kMaxRows);
  if (!q || !k_cache || !v_cache || !pos0_dev || !ws || !out)
    return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(ws) || !aligned16(out))
    return set_error(SOLORT_EINVAL, "%s: pointers must be 16-byte aligned", name);
  if (kv_tok_stride <= 0 || kv_head_stride <= 0 || kv_tok_stride % 8 || kv_head_stride % 8)
    return set_error(SOLORT_EINVAL, "%s: KV strides must be positive multiples of 8", name);
  if (bound < 1 || bound > max_len || bound > (1 << 30))
    return set_error(SOLORT_EINVAL, "%s: bound %d outside [1, max_len=%lld]", name, bound, (long long)max_len);
  if (n_split < 1 || n_split > kMaxSplit || (int64_t)n_split * nkv > 0x7fffffff)
    return set_error(SOLORT_EINVAL, "%s: n_split %d outside [1, %d]", name, n_split, kMaxSplit);
  if (out_dtype != SOLORT_DTYPE_BF16 && out_dtype != SOLORT_DTYPE_F32)
    return set_error(SOLORT_EINVAL, "%s: out_dtype %d", name, out_dtype);
  const int R = nq * G;
  const size_t smem_main = (size_t)(4 * R * 128 + 8 * R) * sizeof(float);
  const size_t smem_comb = (size_t)(2 * n_split * R + 2 * R) * sizeof(float);
  const size_t smem = smem_main > smem_comb ? smem_main : smem_comb;
  if (smem > 64 * 1024)
    return set_error(SOLORT_EINVAL, "%s: n_split %d too large for %d query rows", name, n_split, R);

  const WsLayout w = ws_layout(nq, nh, nkv, n_split);
  AttnArgs a;
  a.q = (const uint16_t*)q;
  a.kc = (const uint16_t*)k_cache;
  a.vc = (const uint16_t*)v_cache;
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
  const int U = per_split >= 64 ? 4 : 2;
  const int blocks = n_split * nkv;
  hipStream_t s = (hipStream_t)stream;
  bool ok = false;
  switch (G) {
    case 1: ok = launch_nq<1>(nq, U, a, blocks, smem, s); break;
    case 2: ok = launch_nq<2>(nq, U, a, blocks, smem, s); break;
    case 4: ok = launch_nq<4>(nq, U, a, blocks, smem, s); break;
    case 8: ok = launch_nq<8>(nq, U, a, blocks, smem, s); break;
  }
  if (!ok) return set_error(SOLORT_EINVAL, "%s: no kernel for nq=%d group=%d", name, nq, G);
  return check_launch(name);
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
