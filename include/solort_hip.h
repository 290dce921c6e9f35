/*
 * solort_hip.h - C ABI of the gfx950 (MI355X) attention hot path of a
 * Qwen3 static-KV decode/prefill/verify step.
 *
 * The reference (SoloRT) runs this path as inline torch code inside
 * _GraphQwen3Runner (src/solort/model/cuda_graph_executor.py); it has no FFI.
 * Each entry point below replaces one block of that inline code and is cited
 * to it.  Plain pointers and sizes only: every buffer is owned by the caller,
 * and apart from the one-time solort_init nothing here allocates, frees,
 * synchronises or reads device memory back, so every call can be recorded
 * into a hipGraph.  The position of the token(s)
 * is read on the device from `pos0_dev`, exactly like the reference's
 * `pos_buf` (cuda_graph_executor.py:71), so one captured graph serves every
 * position inside its bucket.
 *
 * Element types: bf16 buffers are passed as raw 16-bit words (uint16_t bits
 * of a bfloat16).  head_dim must be 128.  KV caches are addressed with
 * explicit token and head strides (in elements), so both the reference's
 * token-major layout [max_len, nkv, hd] (cuda_graph_executor.py:67-69) and a
 * head-major [nkv, max_len, hd] layout are accepted.  Every pointer passed
 * to these functions must be 16-byte aligned and every stride a multiple of 8
 * elements.
 *
 * Return value: 0 on success; SOLORT_EINVAL (negative) when an argument is
 * rejected before launch; otherwise the hipError_t reported by the launch.
 * solort_last_error() returns the message of the last failure on the calling
 * thread.
 */
#ifndef SOLORT_HIP_H
#define SOLORT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SOLORT_EINVAL (-22)

#define SOLORT_DTYPE_BF16 0
#define SOLORT_DTYPE_F32 1

#define SOLORT_GEMV_PLAIN 0
#define SOLORT_GEMV_RESID 1
#define SOLORT_GEMV_SWIGLU 2

/* hipStream_t, passed opaquely (torch.cuda.current_stream().cuda_stream). */
typedef void* solort_stream_t;

/* Version of this ABI; bumped when a signature changes. */
int solort_abi_version(void);

/* 64-bit hash of the sources the library was built from (its HIP sources and
 * headers), so a loader can refuse a library built from other sources. */
uint64_t solort_source_id(void);

/* Message of the last failed call on this thread ("" if none). */
const char* solort_last_error(void);

/*
 * Per-device set-up (no counterpart in the reference, whose attention is
 * inline torch code): call once per device, with that device current and
 * outside graph capture (it launches a probe, synchronises and allocates a
 * few KB that it frees).  It checks that workgroup b of a launch always runs
 * on the XCD (L2 domain) of workgroup b % 8, the round-robin placement of
 * MI355X, which the in-launch split merge relies on (see
 * solort_decode_attn).  Without it, or if the check fails, every split call
 * combines in a second launch.  It also looks up the device address of
 * solort_decode_layer_noalloc's scratch array.
 */
int solort_init(void);

/*
 * Split-combine mode of the current device: mode 1 = one launch where
 * eligible (needs solort_init), 0 = always a second launch, -1 = query only.
 * Returns the mode in effect (1 only when solort_init's check passed).  Both
 * modes give the same bits.
 */
int solort_combine_mode(int mode);

/*
 * Per-head QK-RMSNorm + RoPE prologue with the in-place KV-cache write.
 * Replaces, per layer, cuda_graph_executor.py:117-123 (prefill),
 * :173-179 (decode) and :254-260 (verify):
 *   q = rope(rmsnorm(q, qn_w, eps), cos, sin); k = rope(rmsnorm(k, kn_w, eps), cos, sin)
 *   k_cache[pos] = k; v_cache[pos] = v            (rmsnorm :25-28, rope :100-102)
 * qkv      [T, (nh + 2*nkv) * 128] bf16, row stride `qkv_row_stride` elements
 *          (the fused QKV projection output, q | k | v column blocks).
 * qn_w, kn_w [128] bf16 (q_norm / k_norm weights).
 * inv_freq [64] fp32 RoPE frequencies as the reference computes them (:64-66);
 *          cos/sin of pos * inv_freq are evaluated on the device, with the
 *          same values solort_rope_table produces.
 * pos0_dev int64 on the device: token t sits at position *pos0_dev + t
 *          (NULL means position 0, the prefill case, :111).
 * q_out    [T, nh, 128] bf16.
 * k_cache, v_cache: this layer's cache; row `pos`, head h starts at
 *          pos * kv_tok_stride + h * kv_head_stride.
 * Positions outside [0, max_len) are not written.
 * The K/V rows written are bit-exact with the reference's op sequence given
 * the same cos/sin values; the sum of squares uses a fixed reduction order.
 */
int solort_qknorm_rope_kvwrite(const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv,
                               int hd, const void* qn_w, const void* kn_w, float eps,
                               const float* inv_freq, const int64_t* pos0_dev, void* q_out,
                               void* k_cache, void* v_cache, int64_t kv_tok_stride,
                               int64_t kv_head_stride, int64_t max_len, solort_stream_t stream);

/*
 * The same prologue with the cos/sin rows given: rope_cs [2, T, 64] bf16 is
 * solort_rope_rows(inv_freq, 64, pos0_dev, T) of this step (cos rows of
 * positions pos0..pos0+T-1, then the sin rows), as the reference computes
 * cos, sin once per forward (cuda_graph_executor.py:111, :164, :248) and every
 * layer's prologue (:120-121, :176-177, :257-258) applies them.  Results are
 * bit-identical to solort_qknorm_rope_kvwrite on the same inputs.
 */
int solort_qknorm_rope_kvwrite_cs(const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv, int hd,
                                  const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                                  const int64_t* pos0_dev, void* q_out, void* k_cache, void* v_cache,
                                  int64_t kv_tok_stride, int64_t kv_head_stride, int64_t max_len,
                                  solort_stream_t stream);

/*
 * RoPE table on the device: cos_out/sin_out [rows, half_dim] bf16 with row p
 * = bf16(cos/sin(float(p) * inv_freq[i])), the first half of the reference's
 * _cos_sin(p) row (cuda_graph_executor.py:95-98); inv_freq [half_dim] fp32 as
 * the reference computes it (:64-66).
 */
int solort_rope_table(const float* inv_freq, int half_dim, int64_t rows, void* cos_out, void* sin_out,
                      solort_stream_t stream);

/*
 * cos/sin rows of the positions of one step (decode, verify or prefill),
 * computed once per step and read by every layer's solort_decode_layer or
 * solort_qknorm_rope_kvwrite_cs, as the reference computes cos, sin =
 * _cos_sin(positions) once per step (cuda_graph_executor.py:111, :164, :248)
 * and every layer applies them.  n <= 2^20.
 * cs_out [2, n, half_dim] bf16: cos rows of positions *pos0_dev + t
 *        (t < n), then the sin rows; values as in solort_rope_table.
 */
int solort_rope_rows(const float* inv_freq, int half_dim, const int64_t* pos0_dev, int n, void* cs_out,
                     solort_stream_t stream);

/* Workspace bytes needed by solort_decode_attn / solort_verify_attn /
 * solort_decode_layer for `nq` query tokens and `n_split` key splits: 16 KB
 * of per-KV-head launch counters of the in-launch merge, then the splits'
 * partial results (per KV head, split and query row: running max and sum,
 * and the unnormalised 128-dim output, fp32, each value paired with a 32-bit
 * tag: 1040 bytes).  The caller allocates it once, zero-fills it once and
 * reuses it (each call advances the counters of its KV heads).  A workspace
 * sized for (nq, n_split) serves any call with the same nh/nkv and no larger
 * nq or n_split, and calls of different shapes may share one.  Calls that
 * overlap in time must not share a workspace. */
size_t solort_attn_workspace_bytes(int nq, int nh, int nkv, int hd, int n_split);

/*
 * Grouped-query attention of `nq` new tokens over the static KV cache, split
 * across `n_split` workgroups per KV head (flash-decoding), and the
 * log-sum-exp combine of the splits (none when n_split is 1).  The combine
 * runs inside the same launch -- each split tags its partial with the KV
 * head's launch counter and the head's last min(n_split, nq * nh / nkv)
 * splits each merge rows of the output once every split's partial carries
 * the tag, in the L2 of the XCD all of the head's splits run on -- when
 * solort_init's placement check passed, nkv is a multiple of 8 up to 128,
 * n_split <= 64 and nq * nh / nkv <= 8; otherwise as a second launch on the
 * same stream.
 * Replaces the decode block cuda_graph_executor.py:168, :180-184 (nq = 1:
 * softmax(q K^T * scale, keys > pos masked) V over the bucket) and the verify
 * block :247-250, :261-263 (nq = K+1, query t at position pos0+t sees keys
 * 0..pos0+t).  No KV repeat: query head h reads KV head h / (nh / nkv).
 * q        [nq, nh, 128] bf16 (prologue output).
 * pos0_dev int64 on the device (position of query 0).
 * bound    static bucket: keys at or beyond `bound` are never read
 *          (requires pos0 + nq <= bound <= max_len).
 * scale    softmax scale (head_dim ** -0.5 in the reference, :44).
 * ws       solort_attn_workspace_bytes(nq, nh, nkv, hd, n_split) bytes.
 * out      [nq, nh * 128], bf16 (out_dtype 0) or fp32 (out_dtype 1).
 */
int solort_decode_attn(const void* q, int nq, int nh, int nkv, int hd, const void* k_cache,
                       const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                       int64_t max_len, const int64_t* pos0_dev, int bound, float scale, void* ws,
                       int n_split, void* out, int out_dtype, solort_stream_t stream);

/* Speculative-verify attention (cuda_graph_executor.py:245-263): the same
 * kernel as solort_decode_attn with nq = K+1 query tokens at positions
 * pos0..pos0+K, each causal over the cache (the reference scans all max_len
 * keys under a mask; here `bound` may be any bucket >= pos0+K+1).
 *
 * For both entry points the key range [0, bound) is cut into n_split static
 * chunks whose first step is loaded before the position is known, so keys
 * between the live length and `bound` may be fetched and discarded: pass the
 * tightest bucket. */
int solort_verify_attn(const void* q, int nq, int nh, int nkv, int hd, const void* k_cache,
                       const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                       int64_t max_len, const int64_t* pos0_dev, int bound, float scale, void* ws,
                       int n_split, void* out, int out_dtype, solort_stream_t stream);

/*
 * The whole per-layer attention block: QK-RMSNorm + RoPE of the new tokens'
 * q/k rows, the KV-cache write of their K/V rows, and the split-KV attention
 * in one launch, then the combine of the splits as in solort_decode_attn.  Replaces, per layer,
 * cuda_graph_executor.py:173-184 (decode, nq = 1) and :254-263 (verify,
 * nq = K+1); results equal solort_qknorm_rope_kvwrite followed by
 * solort_decode_attn on the same inputs (the KV rows bit for bit).
 * rope_cs  [2, nq, 64] bf16 from solort_rope_rows(inv_freq, 64, pos0_dev, nq)
 *          of this step (16-byte aligned).
 * Other arguments as in those two functions; the workspace is sized by
 * solort_attn_workspace_bytes(nq, nh, nkv, hd, n_split).  q is not
 * materialised.
 */
int solort_decode_layer(const void* qkv, int64_t qkv_row_stride, int nq, int nh, int nkv, int hd,
                        const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                        const int64_t* pos0_dev, void* k_cache, void* v_cache, int64_t kv_tok_stride,
                        int64_t kv_head_stride, int64_t max_len, int bound, float scale, void* ws,
                        int n_split, void* out, int out_dtype, solort_stream_t stream);

/*
 * The decode step's qkv product and attention block for one new token:
 * qkv = _rmsnorm(x, in_w, in_eps) @ wqkv^T (cuda_graph_executor.py:170-171),
 * then solort_decode_layer on it (:173-184).  Results equal solort_gemv
 * (SOLORT_GEMV_PLAIN, norm_w = in_w) followed by solort_decode_layer, bit for
 * bit.  x [hidden] bf16 (the layer input); wqkv [(nh + 2 nkv) * hd][row
 * stride] bf16.  Where the shapes allow (32 key splits per KV head of 16 to
 * 128 keys, the in-launch merge, the packed cache layout, (group, hidden) in
 * {(2, 1024), (4, 2560), (4, 4096)}, wqkv rows contiguous) it is one launch:
 * the splits of each KV head compute that head's q, k and v rows, hand them
 * over through the XCD's L2 as tagged pairs, and continue with the attention,
 * whose first K/V loads were issued at launch; qkv_out is then not written.
 * Otherwise it runs the two calls, the product into qkv_out [(nh + 2 nkv) *
 * hd] bf16.  The workspace is sized by solort_decode_qkv_workspace_bytes(nh,
 * nkv, n_split).  Other arguments as in solort_decode_layer with nq = 1.
 */
size_t solort_decode_qkv_workspace_bytes(int nh, int nkv, int n_split);
int solort_decode_qkv_layer(const void* x, int hidden, const void* in_w, float in_eps, const void* wqkv,
                            int64_t wqkv_row_stride, int nh, int nkv, int hd, const void* qn_w, const void* kn_w,
                            float eps, const void* rope_cs, const int64_t* pos0_dev, void* k_cache, void* v_cache,
                            int64_t kv_tok_stride, int64_t kv_head_stride, int64_t max_len, int bound, float scale,
                            void* ws, int n_split, void* qkv_out, void* out, int out_dtype, solort_stream_t stream);

/*
 * solort_decode_layer without a workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under graph capture that must not call hipMalloc, tight serving loops,
 * harnesses that forbid allocation).  The partials live in a fixed
 * per-device array of SOLORT_NOALLOC_SCRATCH_BYTES (8 MiB) inside the
 * library, held until the process ends; a call whose
 * solort_attn_workspace_bytes(nq, nh, nkv, hd, n_split) exceeds it returns
 * SOLORT_EINVAL.  It allocates nothing: the array's device address is looked
 * up once per device (by solort_init, else by the first call on the device).
 * All calls on one GPU share the array, so calls that overlap in time on one
 * GPU race.  Results equal solort_decode_layer's with any workspace, bit for
 * bit.  Other arguments as in solort_decode_layer.
 */
#define SOLORT_NOALLOC_SCRATCH_BYTES (8u << 20)
int solort_decode_layer_noalloc(const void* qkv, int64_t qkv_row_stride, int nq, int nh, int nkv, int hd,
                                const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                                const int64_t* pos0_dev, void* k_cache, void* v_cache, int64_t kv_tok_stride,
                                int64_t kv_head_stride, int64_t max_len, int bound, float scale, int n_split,
                                void* out, int out_dtype, solort_stream_t stream);

/*
 * solort_decode_layer over a paged KV cache: the layout of the reference's
 * tensor-backed PagedKVCache (src/solort/cache/kv_cache.py:71-100: per layer
 * [num_pages, 2, page_size, nkv, hd], K then V within a page, "NHD"), read
 * and written through a page table as FlashInfer-style paged decode would
 * (page_indices, :113-129).  Position t of the sequence is row
 * t % page_size of page page_table[t / page_size], i.e. physical slot
 * page_table[t / page_size] * page_size + t % page_size, the reference's
 * slot_mapping (:131-145); the new tokens' K/V rows go to the slots of
 * pos0..pos0+nq-1 (its store_layer_tokens, :191-230).
 * k_pages, v_pages  page 0 of K and of V (for the reference layout, v_pages =
 *                   k_pages + page_size * nkv * hd); page_stride elements
 *                   from one page to the next (2 * page_size * nkv * hd).
 * kv_tok_stride, kv_head_stride  strides of a row and of a head within a page.
 * page_size         a power of two; num_pages pages in the pool.
 * page_table        int32 [table_len]; entries 0..ceil(bound/page_size)-1 are
 *                   read (entries past the live pages are read and their rows
 *                   masked); an entry outside [0, num_pages) is clamped into
 *                   the pool (a wrong row, never an out-of-bounds access).
 * Positions >= table_len * page_size are not written.  Results equal
 * solort_decode_layer over the same rows in a contiguous cache, bit for bit,
 * for the same bound and n_split.  Other arguments as in solort_decode_layer.
 */
int solort_paged_decode_layer(const void* qkv, int64_t qkv_row_stride, int nq, int nh, int nkv, int hd,
                              const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                              const int64_t* pos0_dev, void* k_pages, void* v_pages, int64_t page_stride,
                              int64_t kv_tok_stride, int64_t kv_head_stride, int page_size, int num_pages,
                              const int32_t* page_table, int table_len, int bound, float scale, void* ws,
                              int n_split, void* out, int out_dtype, solort_stream_t stream);

/*
 * Slot-mapped row copies for the paged arena (layout as in
 * solort_paged_decode_layer).  store: K/V row t of the contiguous rows
 * (k_rows/v_rows, token stride row_tok_stride, head stride row_head_stride)
 * -> physical slot slot_mapping[t] (page slot / page_size, row
 * slot % page_size), the reference's store_layer_tokens
 * (src/solort/cache/kv_cache.py:191-230; slots from its slot_mapping,
 * :131-145).  gather: slot slot_mapping[t] -> row t, its gather_layer_tokens
 * (:232-256).  slot_mapping int64 [T]; a slot outside [0, num_pages *
 * page_size) is skipped by store and reads as zeros in gather.  A prompt
 * reaches the pages by solort_prefill_layer into T contiguous rows, then
 * store.
 */
int solort_paged_kv_store(const void* k_rows, const void* v_rows, int64_t row_tok_stride, int64_t row_head_stride,
                          int T, int nkv, int hd, const int64_t* slot_mapping, void* k_pages, void* v_pages,
                          int64_t page_stride, int64_t kv_tok_stride, int64_t kv_head_stride, int page_size,
                          int num_pages, solort_stream_t stream);
int solort_paged_kv_gather(const void* k_pages, const void* v_pages, int64_t page_stride, int64_t kv_tok_stride,
                           int64_t kv_head_stride, int page_size, int num_pages, const int64_t* slot_mapping, int T,
                           int nkv, int hd, void* k_rows, void* v_rows, int64_t row_tok_stride,
                           int64_t row_head_stride, solort_stream_t stream);

/*
 * Causal grouped-query prefill attention on bf16 MFMA.
 * Replaces cuda_graph_executor.py:124-130: SDPA(q, repeat_interleave(k, g),
 * repeat_interleave(v, g), is_causal=True, scale) over T prompt rows at
 * positions 0..T-1, with K/V read from cache rows 0..T-1 (written first by
 * solort_qknorm_rope_kvwrite, as the reference writes them at :122-123).
 * q   [T, nh, 128] bf16; out [T, nh * 128] bf16 or fp32.  T <= max_len.
 * Query groups g = nh / nkv of 1, 2, 4 or 8.  Accumulation and softmax are
 * fp32; with a bf16 output the probabilities enter the second matrix product
 * rounded to bf16, with an fp32 output as bf16 high + low parts (~16 bits),
 * which keeps it within 1e-4 of exact attention over the same bf16 q/K/V.
 */
int solort_prefill_attn(const void* q, int T, int nh, int nkv, int hd, const void* k_cache,
                        const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                        int64_t max_len, float scale, void* out, int out_dtype, solort_stream_t stream);

/*
 * One layer's prefill attention block: QK-RMSNorm + RoPE of the T prompt
 * rows' q and k heads, the cache write of their K and V rows at positions
 * 0..T-1, and the causal attention into out.  Replaces, per layer,
 * cuda_graph_executor.py:117-130 (the norms and rope :120-121, the cache
 * writes :122-123, the SDPA :124-130).  Results equal
 * solort_qknorm_rope_kvwrite_cs followed by solort_prefill_attn on the same
 * inputs, bit for bit (the cache rows and out); q is not materialised: the
 * attention kernel normalises the q rows it stages.  Two launches on
 * `stream` (the K/V rows, then the attention).  It saves the q round trip
 * through HBM but puts the q normalisation ahead of each attention
 * workgroup's first MFMA: on MI355X it wins from about 400 rows on (Qwen3-4B
 * shape, 1024 rows: 27.0 against 30.1 us per layer) and loses below.
 * qkv [T, qkv_row_stride] bf16 (q, k, v heads of each row); rope_cs [2, T, 64]
 * bf16 from solort_rope_rows(inv_freq, 64, pos0 = 0, T).  Other arguments as
 * in solort_qknorm_rope_kvwrite_cs and solort_prefill_attn.
 */
int solort_prefill_layer(const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv, int hd, const void* qn_w,
                         const void* kn_w, float eps, const void* rope_cs, void* k_cache, void* v_cache,
                         int64_t kv_tok_stride, int64_t kv_head_stride, int64_t max_len, float scale, void* out,
                         int out_dtype, solort_stream_t stream);

/*
 * Greedy speculative acceptance, on the device.  Replaces
 * cuda_graph_executor.py:476, a = int((tg[:k] == draft).cumprod(0).sum()),
 * and picks the token the round appends after the accepted drafts, tg[a]
 * (:478, :481).  target [k + 1] int64: the argmax of the K+1 verify rows
 * (solort_argmax_rows); draft [k] int64; out [2] int64 receives a and
 * target[a].  One tiny launch, no host synchronisation.  1 <= k <= 2^20.
 */
int solort_accept_prefix(const int64_t* target, const int64_t* draft, int k, int64_t* out, solort_stream_t stream);

/*
 * Decode-step matrix-vector product around the attention block, one token:
 * W [rows][w_row_stride] bf16 row-major (torch Linear weight), x [k] bf16,
 * fp32 accumulation, bf16 out [n_out].  Replaces the T = 1 GEMMs of
 * cuda_graph_executor.py:165-190 with their neighbours fused:
 *   norm_w non-NULL: x is first _rmsnorm(x, norm_w, eps) (:25-28; :170, :186, :190)
 *   mode SOLORT_GEMV_PLAIN   out = W x                          (qkv :171, logits :190)
 *   mode SOLORT_GEMV_RESID   out = res + W x (out may be res)   (:185, :188)
 *   mode SOLORT_GEMV_SWIGLU  out[i] = silu(g_i) * u_i, g = rows 0..n_out-1,
 *                            u = rows inter..inter+n_out-1 of W (wgu, :187-188)
 * with the reference's bf16 rounding of each intermediate tensor.  x must not
 * alias out.  k a multiple of 8 up to 65536; w, x, norm_w 16-byte aligned.
 */
int solort_gemv(const void* w, int64_t w_row_stride, int n_out, int k, const void* x, const void* norm_w, float eps,
                const void* res, int mode, int64_t inter, void* out, solort_stream_t stream);

/* Workspace bytes for solort_gemv_argmax with n_out outputs (one 8-byte key
 * per workgroup; no zero-fill needed). */
size_t solort_gemv_argmax_workspace_bytes(int n_out);

/*
 * The lm_head product fused with the greedy argmax, one token: logits =
 * _rmsnorm(x, norm_w) @ W.T (norm_w may be NULL), then out_idx[0] =
 * argmax(logits.float()) with the lowest index winning ties and NaN ranked
 * highest, as cuda_graph_executor.py:189-190 followed by :206 computes it.
 * The index is bit-identical to solort_argmax_rows over solort_gemv's bf16
 * logits (the key is taken from the same bf16-rounded value).  Each
 * workgroup of the product stores the best (value, index) key of its outputs
 * in ws; a one-workgroup launch reduces those keys into out_idx.  With
 * out_idx NULL that launch is skipped and the keys stay in ws for
 * solort_greedy_advance.  logits [n_out] bf16 is written when non-NULL.  ws:
 * solort_gemv_argmax_workspace_bytes(n_out) bytes, 8-byte aligned; calls
 * that overlap in time must not share it.
 */
int solort_gemv_argmax(const void* w, int64_t w_row_stride, int n_out, int k, const void* x, const void* norm_w,
                       float eps, void* logits, int64_t* out_idx, void* ws, solort_stream_t stream);

/*
 * The tail of a greedy decode step and the head of the next, in one launch
 * after solort_gemv_argmax(..., out_idx = NULL, ws): the argmax token t of the
 * keys in ws (vocab = that call's n_out) becomes the next input, *tok = t
 * (tok_buf, cuda_graph_executor.py:206 and :241), is recorded at
 * tokens[*step] when *step < max_tokens (the chunk's token list, :372-374),
 * *step and *pos advance by one (pos_buf, :242), and x [hidden] bf16 receives
 * embed row t (x = self.embed[self.tok_buf], :165).  embed [vocab,
 * embed_row_stride] bf16 16-byte aligned, hidden a multiple of 8.  Keys that
 * name no row of the vocabulary (ws not filled by solort_gemv_argmax) are
 * recorded as token -1 in tokens, an error for the caller to report, and row
 * 0 is embedded: no row outside embed is read.
 */
int solort_greedy_advance(const void* ws, int vocab, const void* embed, int64_t embed_row_stride, int hidden,
                          void* x, int64_t* tok, int64_t* tokens, int max_tokens, int64_t* step, int64_t* pos,
                          solort_stream_t stream);

/* Workspace bytes for solort_argmax_rows with `rows` rows: per row 64 slots
 * of 16 bytes, then a 16-byte item whose first 32-bit word is the row's
 * epoch (the launch count of the row, which tags the slots each launch
 * writes) and whose second word counts the calls whose reduction failed
 * (see solort_argmax_rows).  Allocate once, zero-fill once, reuse (16-byte
 * aligned) for any call with no more rows; overlapping calls must not share
 * it. */
size_t solort_argmax_workspace_bytes(int rows);

/*
 * Greedy argmax over each row of logits [rows, vocab] (row stride
 * `row_stride` elements), bf16 (dtype 0) or fp32 (dtype 1), into int64
 * out_idx[rows].  Ties go to the lowest index and NaN counts as the maximum
 * (first NaN wins), as torch.argmax does.  Up to 64 blocks per row each
 * store their best key; the row's last block reduces them in the same
 * launch where solort_init's placement check passed (and solort_argmax_mode
 * allows it), else a one-wavefront-per-row launch does after it.  Every
 * index written lies in [0, vocab): a reduction that fails (a block's key
 * never seen within the polling limit) writes the best key it found and
 * adds 1 to the row's failure count in ws, which callers read at their next
 * synchronisation.  Replaces cuda_graph_executor.py:201/:206 (in-graph),
 * :234 (draft) and :475 (verify) `argmax(-1)`.  rows <= 65528.
 */
int solort_argmax_rows(const void* logits, int dtype, int rows, int64_t vocab, int64_t row_stride,
                       int64_t* out_idx, void* ws, solort_stream_t stream);

/*
 * Reduction mode of solort_argmax_rows on the current device (no
 * counterpart in the reference): 1 = one launch where the placement check
 * passed (the default), 0 = always the second launch, 2 = one launch whose
 * reducing block gives up at once (a test of the failure path: every index
 * stays in the row, built from the keys it saw, and each row counts a
 * failure), -1 = query only.  Returns the mode in effect (0 when the
 * placement is unverified).  Modes 0 and 1 give the same indices.
 */
int solort_argmax_mode(int mode);

/*
 * Device probes (no counterpart in the reference): the launch and streaming
 * floor a latency-bound call on this device is compared with.
 * probe_placement: out[2b] = XCD index, out[2b + 1] = HW_ID register of
 *   workgroup b of an n_wg-workgroup launch (out: 2 * n_wg words).
 * probe_empty: an empty kernel of n_wg workgroups of 64 threads.
 * probe_read: streams nbytes (a multiple of 16) from src with n_wg
 *   workgroups of 256 threads, in_flight (1, 2 or 4) 16-byte loads in flight
 *   per thread, plus 16 for loads with the non-temporal hint (the hint the
 *   decode K/V and weight streams use); workgroup b writes one word to
 *   sink[b] (sink: n_wg words).
 * probe_read_heads: the split decode kernel's K/V reads without arithmetic,
 *   over caches k, v of rows x nkv x 128 bf16 (token-major, heads interleaved):
 *   workgroup h + nkv * s reads head h's rows of keys [s * c, (s + 1) * c),
 *   c = rows / n_split (a multiple of 128), in the decode's 32-row tiles per
 *   wavefront with the non-temporal hint, tiles_in_flight (1, as the decode
 *   keeps, or 2) tiles in flight per wavefront; workgroup b writes one word
 *   to sink[b] (sink: nkv * n_split words).
 */
int solort_probe_placement(uint32_t* out, int n_wg, solort_stream_t stream);
int solort_probe_empty(int n_wg, solort_stream_t stream);
int solort_probe_read(const void* src, int64_t nbytes, int n_wg, int in_flight, uint32_t* sink,
                      solort_stream_t stream);
int solort_probe_read_heads(const void* k, const void* v, int64_t rows, int nkv, int n_split, int tiles_in_flight,
                            uint32_t* sink, solort_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SOLORT_HIP_H */
