// Decode-step matrix-vector products around the attention block, HBM-bound
// weight streams: y = W x for one token, W [N][K] bf16 row-major (the torch
// Linear weight layout), fp32 accumulation, bf16 results.
//
// Follows src/solort/model/cuda_graph_executor.py:165-190 (decode) with the
// fused weights of :54-63:
//   h  = _rmsnorm(x, in_ln);   qkv = h @ wqkv.T            (NORM, PLAIN)
//   x  = x + ctx @ wo.T                                    (RESID)
//   h2 = _rmsnorm(x, post_ln); gate, up = (h2 @ wgu.T).split
//   x  = x + (silu(gate) * up) @ wd.T                      (NORM + SWIGLU, RESID)
//   _rmsnorm(x, final_norm) @ lm_head.T                    (NORM, PLAIN)
//   argmax(logits) (:190, :206) folded into the lm_head      (NORM, ARGMAX)
// Each op rounds to bf16 as the reference's bf16 tensors do: the RMSNorm
// output (_rmsnorm :25-28: fp32 x * rsqrt(mean(x^2) + eps), * fp32 w, to
// bf16), the product, silu(gate), silu(gate) * up and the residual sum.
//
// Mapping: a workgroup (4 wavefronts) first stages x into LDS, normalised
// when NORM (every workgroup recomputes the 1-row norm: K <= 16384, a few KB
// from L2), then each wavefront streams R weight rows: lane l takes the
// 16-byte chunks l, l + 64, ... of each row (1 KB per row per instruction,
// coalesced, with the non-temporal hint: measured in the Qwen3-4B decode
// step, 538 tokens/s with it on every weight stream against 525 with it on
// gate_up and lm_head only and 511 without), dotting them with x by
// v_dot2_f32_bf16, and the 64 lanes' sums meet by DPP/permute reductions.
// SWIGLU wavefronts take R / 2 outputs: gate rows o and up rows o + inter.
// R is chosen so the grid holds at least two workgroups per CU.  ARGMAX
// workgroups reduce their outputs' argmax keys
// (the bf16 logit, as torch.argmax sees the reference's bf16 product cast to
// fp32) and store the best one in their own workspace slot; a one-workgroup
// launch after the grid reduces the slots and decodes the index.
#include "common.h"
#include "capi_internal.h"
#include "gemv_common.h"

namespace solort {

enum { kGemvPlain = 0, kGemvResid = 1, kGemvSwiglu = 2, kGemvArgmax = 3 };

// silu(g) = g * sigmoid(g) = g / (1 + exp(-g)) in fp32 (torch's formula),
// rounded to bf16 as F.silu on a bf16 tensor.
__device__ __forceinline__ float silu_bf16(float g) { return rbf(g / (1.0f + __expf(-g))); }

// The arguments the first loads need lead (w .. norm_w: 13 dwords), so they
// arrive preloaded in SGPRs and the weight stream starts without waiting for
// the kernel-argument fetch.
template <int R, int U, int EPI, bool NORM>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ w, int64_t w_stride, int n_out,
                                                   int K, int64_t inter, const uint16_t* __restrict__ x,
                                                   const uint16_t* __restrict__ norm_w, float eps,
                                                   const uint16_t* res, uint16_t* out, uint64_t* arg_ws,
                                                   int64_t* arg_idx) {
  extern __shared__ uint4 sx[];  // x as K / 8 chunks of 16 bytes
  __shared__ float s_red[4];
  __shared__ uint64_t s_key[4];
  // wave is uniform: the row pointers below live in scalar registers.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nch = K >> 3;

  // This wavefront's R weight rows; lane l streams their 16-byte chunks
  // l + 64 i, U chunks per row in flight.
  constexpr int NO = EPI == kGemvSwiglu ? R / 2 : R;  // outputs per wavefront
  const int o0 = (blockIdx.x * 4 + wave) * NO;
  const uint16_t* rows[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int o = min(o0 + (EPI == kGemvSwiglu ? r % NO : r), n_out - 1);  // past the end: repeat the last
    const int64_t row = EPI == kGemvSwiglu && r >= NO ? o + inter : o;
    rows[r] = w + row * w_stride;
  }
  uint4 wv[U][R];
#define SOLORT_GEMV_LOADS(C0)                                                                    \
  _Pragma("unroll") for (int u = 0; u < U; ++u) {                                                \
    const int c = (C0) + 64 * u;                                                                 \
    if (c < nch) {                                                                               \
      _Pragma("unroll") for (int r = 0; r < R; ++r) wv[u][r] = ld_stream(rows[r] + 8 * c);         \
    }                                                                                            \
  }
  // The first weight loads go out before x is staged: they do not depend on
  // it, and its load and norm then overlap their latency.  (Measured: x and the
  // norm weight loaded ahead of the weight rows made the o_proj, gate_up and
  // down products slower, the Qwen3-4B decode step 3 % slower.)
  SOLORT_GEMV_LOADS(lane)

  // x into LDS (normalised: sum of squares in fp32, one block reduction).
  gemv_stage_x<NORM>(x, norm_w, eps, K, sx, s_red);

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int c0 = lane;;) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + 64 * u < nch) {
        const uint4 xv = sx[c0 + 64 * u];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d = dot2bf(wv[u][r].x, xv.x, acc[r]);
          d = dot2bf(wv[u][r].y, xv.y, d);
          d = dot2bf(wv[u][r].z, xv.z, d);
          acc[r] = dot2bf(wv[u][r].w, xv.w, d);
        }
      }
    }
    c0 += 64 * U;
    if (c0 >= nch) break;
    SOLORT_GEMV_LOADS(c0)
  }
#undef SOLORT_GEMV_LOADS
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum64(acc[r]);

  if constexpr (EPI == kGemvArgmax) {
    // Lane i < NO holds output o0 + i; out (the bf16 logits) is optional.
    // The workgroup's best key goes to its own slot with a plain store (same-
    // address atomics from ~10^4 workgroups serialise on one L2 channel and
    // stall the weight stream behind it); a later launch reduces the slots.
    uint64_t key = 0;  // below every real key
    if (lane < NO) {
      float a = acc[0];
#pragma unroll
      for (int i = 1; i < NO; ++i)
        if (lane == i) a = acc[i];
      const int o = o0 + lane;
      if (o < n_out) {
        const float y = rbf(a);
        if (out) out[o] = f2bf(y);
        key = argmax_key(y, o);
      }
    }
    static_assert(NO <= 4, "the key reduction covers lanes 0..3");
    key = umax64(key, __shfl_xor(key, 1, 64));
    key = umax64(key, __shfl_xor(key, 2, 64));
    if (lane == 0) s_key[wave] = key;
    __syncthreads();
    if (tid == 0) arg_ws[blockIdx.x] = umax64(umax64(s_key[0], s_key[1]), umax64(s_key[2], s_key[3]));
    return;
  }
  // Epilogue: lane i < NO stores output o0 + i.
  if (lane < NO) {
    float a = acc[0], b = 0.f;
#pragma unroll
    for (int i = 1; i < NO; ++i)
      if (lane == i) a = acc[i];
    if constexpr (EPI == kGemvSwiglu) {
#pragma unroll
      for (int i = 0; i < NO; ++i)
        if (lane == i) b = acc[NO + i];
    }
    const int o = o0 + lane;
    if (o < n_out) {
      float y;
      if constexpr (EPI == kGemvPlain) {
        y = a;
      } else if constexpr (EPI == kGemvResid) {
        y = bf2f(res[o]) + rbf(a);
      } else {
        y = silu_bf16(rbf(a)) * rbf(b);
      }
      out[o] = f2bf(y);
    }
  }
}

// The maximum of the n keys an ARGMAX grid stored, in every thread of a
// 1024-thread workgroup.  Sixteen independent loads per thread are in flight
// (n <= 16384 in one round: a 151,936-token lm_head stores 9,496 keys).
__device__ __forceinline__ uint64_t reduce_keys_1024(const uint64_t* __restrict__ keys, int n) {
  __shared__ uint64_t s_best[16];
  uint64_t best = 0;
  for (int base = 0; base < n; base += 16 * 1024) {
    uint64_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = base + j * 1024 + (int)threadIdx.x;
      v[j] = i < n ? keys[i] : 0;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) best = umax64(best, v[j]);
  }
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) best = umax64(best, __shfl_xor(best, mask, 64));
  if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) best = umax64(best, s_best[i]);
  return best;
}

__device__ __forceinline__ int64_t key_index(uint64_t k) { return (int64_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu)); }

__global__ __launch_bounds__(1024) void argmax_keys_finish_kernel(const uint64_t* __restrict__ keys, int n,
                                                                  int64_t* __restrict__ out) {
  const uint64_t best = reduce_keys_1024(keys, n);
  if (threadIdx.x == 0) *out = key_index(best);
}

// The greedy step's tail: the token the keys name becomes the next input
// (tok), is recorded at tokens[step], step and pos advance by one, and its
// embedding row is copied into x for the next step.  Keys that name no row
// of the vocabulary (a workspace no solort_gemv_argmax call filled) are
// recorded as token -1, which the host reads as an error, while row 0 is
// embedded: no row outside the table is ever read.
__global__ __launch_bounds__(1024) void greedy_advance_kernel(const uint64_t* __restrict__ keys, int n, int vocab,
                                                              const uint16_t* __restrict__ embed,
                                                              int64_t row_stride, int hidden,
                                                              uint16_t* __restrict__ x, int64_t* __restrict__ tok,
                                                              int64_t* __restrict__ tokens, int max_tokens,
                                                              int64_t* __restrict__ step, int64_t* __restrict__ pos) {
  const int64_t t = key_index(reduce_keys_1024(keys, n));
  const bool ok = t >= 0 && t < vocab;
  const int64_t te = ok ? t : 0;
  const uint4* src = reinterpret_cast<const uint4*>(embed + te * row_stride);
  for (int i = threadIdx.x; i < hidden / 8; i += 1024) reinterpret_cast<uint4*>(x)[i] = src[i];
  if (threadIdx.x == 0) {
    const int64_t s = *step;
    *tok = te;
    if (s >= 0 && s < max_tokens) tokens[s] = ok ? t : -1;
    *step = s + 1;
    *pos += 1;
  }
}

}  // namespace solort

using namespace solort;

namespace {

// Rows per wavefront (R) and workgroups: enough workgroups (4 wavefronts
// each) for two per CU.
int64_t gemv_blocks(int n_out, int mode, int* R_out) {
  int R = 4;
  const int per = mode == kGemvSwiglu ? 2 : 1;  // weight rows per output
  if ((int64_t)n_out * per / (4 * 4) < 512) R = 2;
  if ((int64_t)n_out * per / (4 * 2) < 512) R = mode == kGemvSwiglu ? 2 : 1;
  const int no = mode == kGemvSwiglu ? R / 2 : R;
  *R_out = R;
  return ((int64_t)n_out + 4 * no - 1) / (4 * no);
}

// Chooses rows per wavefront and chunks in flight, then launches.  mode is
// checked by the callers; arg_ws / arg_idx are used by kGemvArgmax only.
int launch_gemv(const char* name, const void* w, int64_t w_row_stride, int n_out, int k, const void* x,
                const void* norm_w, float eps, const void* res, int mode, int64_t inter, void* out, uint64_t* arg_ws,
                int64_t* arg_idx, hipStream_t s, int* nblocks_out = nullptr) {
  if (n_out < 1 || k < 8 || k % 8 != 0 || k > 65536)
    return set_error(SOLORT_EINVAL, "%s: bad shape n_out=%d k=%d (k a multiple of 8, <= 65536)", name, n_out, k);
  if (w_row_stride < k || w_row_stride % 8 != 0)
    return set_error(SOLORT_EINVAL, "%s: w_row_stride %lld", name, (long long)w_row_stride);
  if (!aligned16(w) || !aligned16(x) || (norm_w && !aligned16(norm_w)) || ((uintptr_t)out & 1u) ||
      (res && ((uintptr_t)res & 1u)))
    return set_error(SOLORT_EINVAL, "%s: w, x and norm_w must be 16-byte aligned", name);
  int R = 0;
  const int64_t blocks = gemv_blocks(n_out, mode, &R);
  if (blocks > 0x7fffffff) return set_error(SOLORT_EINVAL, "%s: too many rows", name);

  if (nblocks_out) *nblocks_out = (int)blocks;
  const size_t lds = (size_t)k * 2;
  const bool norm = norm_w != nullptr;
  // Chunks per row in flight: 5 when a lane's share is a multiple of 5 (k = 2560: one batch) or for
  // four-row wavefronts (registers); single-row wavefronts take up to 20 (k = 9728: one batch); else 8.
  const int cpl = (k / 8 + 63) / 64;
  const int U = (R == 4 || cpl % 5 == 0 || cpl < 5) ? 5 : (R == 1 && cpl > 8 && cpl <= 20 ? 20 : 8);
#define SOLORT_GEMV_U(RR, UU, EE, NN)                                                                         \
  hipLaunchKernelGGL((gemv_kernel<RR, UU, EE, NN>), dim3((unsigned)blocks), dim3(256), lds, s,               \
                     (const uint16_t*)w, w_row_stride, n_out, k, inter, (const uint16_t*)x,                    \
                     (const uint16_t*)norm_w, eps, (const uint16_t*)res, (uint16_t*)out, arg_ws, arg_idx)
#define SOLORT_GEMV(RR, EE, NN)                              \
  do {                                                       \
    if (U == 5) SOLORT_GEMV_U(RR, 5, EE, NN);                \
    else if (U == 8) SOLORT_GEMV_U(RR, 8, EE, NN);           \
    else SOLORT_GEMV_U(1, 20, EE, NN); /* U = 20 only with R = 1 */ \
  } while (0)
#define SOLORT_GEMV_R(EE, NN)        \
  switch (R) {                       \
    case 1: SOLORT_GEMV(1, EE, NN); break; \
    case 2: SOLORT_GEMV(2, EE, NN); break; \
    default: SOLORT_GEMV(4, EE, NN); break; \
  }
  if (mode == kGemvPlain) {
    if (norm) { SOLORT_GEMV_R(kGemvPlain, true) } else { SOLORT_GEMV_R(kGemvPlain, false) }
  } else if (mode == kGemvResid) {
    if (norm) { SOLORT_GEMV_R(kGemvResid, true) } else { SOLORT_GEMV_R(kGemvResid, false) }
  } else if (mode == kGemvArgmax) {
    if (norm) { SOLORT_GEMV_R(kGemvArgmax, true) } else { SOLORT_GEMV_R(kGemvArgmax, false) }
  } else {  // R is 2 or 4 here
    if (norm) {
      if (R == 2) SOLORT_GEMV(2, kGemvSwiglu, true); else SOLORT_GEMV(4, kGemvSwiglu, true);
    } else {
      if (R == 2) SOLORT_GEMV(2, kGemvSwiglu, false); else SOLORT_GEMV(4, kGemvSwiglu, false);
    }
  }
#undef SOLORT_GEMV_R
#undef SOLORT_GEMV
#undef SOLORT_GEMV_U
  return check_launch(name);
}

}  // namespace

extern "C" int solort_gemv(const void* w, int64_t w_row_stride, int n_out, int k, const void* x, const void* norm_w,
                           float eps, const void* res, int mode, int64_t inter, void* out, solort_stream_t stream) {
  const char* name = "gemv";
  if (mode != kGemvPlain && mode != kGemvResid && mode != kGemvSwiglu)
    return set_error(SOLORT_EINVAL, "%s: mode %d", name, mode);
  if (!w || !x || !out || (mode == kGemvResid && !res)) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (mode == kGemvSwiglu && inter < n_out)
    return set_error(SOLORT_EINVAL, "%s: swiglu needs inter >= n_out (up rows follow the gate rows)", name);
  return launch_gemv(name, w, w_row_stride, n_out, k, x, norm_w, eps, res, mode, inter, out, nullptr, nullptr,
                     (hipStream_t)stream);
}

extern "C" size_t solort_gemv_argmax_workspace_bytes(int n_out) {
  if (n_out < 1 || n_out > (1 << 30)) return 0;
  // One key per workgroup; a workgroup covers at least 4 outputs.
  return (((size_t)n_out + 3) / 4 * 8 + 255) & ~(size_t)255;
}

extern "C" int solort_gemv_argmax(const void* w, int64_t w_row_stride, int n_out, int k, const void* x,
                                  const void* norm_w, float eps, void* logits, int64_t* out_idx, void* ws,
                                  solort_stream_t stream) {
  const char* name = "gemv_argmax";
  if (!w || !x || !ws) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (((uintptr_t)ws & 7u) || ((uintptr_t)out_idx & 7u))
    return set_error(SOLORT_EINVAL, "%s: ws and out_idx must be 8-byte aligned", name);
  if (n_out < 1 || n_out > (1 << 30)) return set_error(SOLORT_EINVAL, "%s: bad shape n_out=%d", name, n_out);
  int nblocks = 0;
  const int rc = launch_gemv(name, w, w_row_stride, n_out, k, x, norm_w, eps, nullptr, kGemvArgmax, 0, logits,
                             (uint64_t*)ws, out_idx, (hipStream_t)stream, &nblocks);
  if (rc || !out_idx) return rc;
  hipLaunchKernelGGL(argmax_keys_finish_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, (const uint64_t*)ws,
                     nblocks, out_idx);
  return check_launch(name);
}

extern "C" int solort_greedy_advance(const void* ws, int vocab, const void* embed, int64_t embed_row_stride, int hidden,
                                     void* x, int64_t* tok, int64_t* tokens, int max_tokens, int64_t* step,
                                     int64_t* pos, solort_stream_t stream) {
  const char* name = "greedy_advance";
  if (!ws || !embed || !x || !tok || !step || !pos || (max_tokens > 0 && !tokens))
    return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (vocab < 1 || vocab > (1 << 30) || hidden < 8 || hidden % 8 != 0 || embed_row_stride < hidden ||
      embed_row_stride % 8 != 0 || max_tokens < 0)
    return set_error(SOLORT_EINVAL, "%s: bad shape vocab=%d hidden=%d stride=%lld max_tokens=%d", name, vocab, hidden,
                     (long long)embed_row_stride, max_tokens);
  if (!aligned16(embed) || !aligned16(x) || ((uintptr_t)ws & 7u) || ((uintptr_t)tok & 7u) ||
      ((uintptr_t)tokens & 7u) || ((uintptr_t)step & 7u) || ((uintptr_t)pos & 7u))
    return set_error(SOLORT_EINVAL, "%s: embed and x must be 16-byte, ws and the int64 buffers 8-byte aligned", name);
  int R = 0;
  const int nkeys = (int)gemv_blocks(vocab, kGemvArgmax, &R);
  hipLaunchKernelGGL(greedy_advance_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, (const uint64_t*)ws, nkeys,
                     vocab, (const uint16_t*)embed, embed_row_stride, hidden, (uint16_t*)x, tok, tokens, max_tokens, step,
                     pos);
  return check_launch(name);
}
