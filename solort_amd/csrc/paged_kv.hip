// Slot-mapped K/V row copies between a contiguous row buffer and the paged
// arena of the reference's tensor-backed PagedKVCache
// (src/solort/cache/kv_cache.py:71-100: per layer [num_pages, 2, page_size,
// nkv, hd], K then V within a page):
//   store  (store_layer_tokens, :191-230): row t of src -> physical slot
//          slot_mapping[t] (page slot / page_size, row slot % page_size)
//   gather (gather_layer_tokens, :232-256): slot slot_mapping[t] -> row t
// One 16-lane group per (token, head) row of 128 bf16 (256 bytes, one 16-byte
// chunk per lane); K and V move in the same launch.  A slot outside
// [0, num_pages * page_size) is skipped (store) or yields zeros (gather), so
// no access leaves the arena.
#include "common.h"
#include "capi_internal.h"

namespace solort {

template <bool STORE>
__global__ __launch_bounds__(256) void paged_kv_copy_kernel(uint16_t* __restrict__ rk, uint16_t* __restrict__ rv,
                                                            int64_t r_tok, int64_t r_head, int T, int nkv,
                                                            const int64_t* __restrict__ slots,
                                                            uint16_t* __restrict__ pk, uint16_t* __restrict__ pv,
                                                            int64_t page_stride, int64_t p_tok, int64_t p_head,
                                                            int page_size, int64_t n_slots) {
  const int64_t g = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // (token, head) row
  const int j = threadIdx.x & 15;
  if (g >= (int64_t)T * nkv) return;
  const int t = (int)(g / nkv), h = (int)(g % nkv);
  const int64_t slot = slots[t];
  const bool ok = slot >= 0 && slot < n_slots;
  const int64_t poff = ok ? (slot / page_size) * page_stride + (slot % page_size) * p_tok + h * p_head + 8 * j : 0;
  const int64_t roff = (int64_t)t * r_tok + h * r_head + 8 * j;
  if constexpr (STORE) {
    if (!ok) return;
    *reinterpret_cast<uint4*>(pk + poff) = *reinterpret_cast<const uint4*>(rk + roff);
    *reinterpret_cast<uint4*>(pv + poff) = *reinterpret_cast<const uint4*>(rv + roff);
  } else {
    const uint4 z = make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(rk + roff) = ok ? *reinterpret_cast<const uint4*>(pk + poff) : z;
    *reinterpret_cast<uint4*>(rv + roff) = ok ? *reinterpret_cast<const uint4*>(pv + poff) : z;
  }
}

}  // namespace solort

using namespace solort;

static int paged_copy(const char* name, bool store, void* rk, void* rv, int64_t r_tok, int64_t r_head, int T,
                      int nkv, int hd, const int64_t* slots, void* pk, void* pv, int64_t page_stride, int64_t p_tok,
                      int64_t p_head, int page_size, int num_pages, solort_stream_t stream) {
  if (hd != SOLORT_HD) return set_error(SOLORT_EINVAL, "%s: head_dim %d != 128", name, hd);
  if (T < 0 || nkv < 1 || (int64_t)T * nkv > ((int64_t)1 << 34))
    return set_error(SOLORT_EINVAL, "%s: bad shape T=%d nkv=%d", name, T, nkv);
  if (page_size < 1 || num_pages < 1) return set_error(SOLORT_EINVAL, "%s: page_size %d, num_pages %d", name,
                                                       page_size, num_pages);
  if (T == 0) return 0;
  if (!rk || !rv || !slots || !pk || !pv) return set_error(SOLORT_EINVAL, "%s: null pointer", name);
  if (!aligned16(rk) || !aligned16(rv) || !aligned16(pk) || !aligned16(pv) || ((uintptr_t)slots & 7u))
    return set_error(SOLORT_EINVAL, "%s: rows must be 16-byte and slot_mapping 8-byte aligned", name);
  if (r_tok % 8 || r_head % 8 || p_tok % 8 || p_head % 8 || page_stride % 8 || r_tok < 1 || r_head < 1 ||
      p_tok < 1 || p_head < 1 || page_stride < (int64_t)page_size * p_tok)
    return set_error(SOLORT_EINVAL, "%s: strides must be positive multiples of 8 and a page must hold its rows",
                     name);
  const int64_t rows = (int64_t)T * nkv;
  const dim3 grid((unsigned)((rows + 15) / 16));
  const int64_t n_slots = (int64_t)num_pages * page_size;
  if (store)
    hipLaunchKernelGGL(paged_kv_copy_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, (uint16_t*)rk,
                       (uint16_t*)rv, r_tok, r_head, T, nkv, slots, (uint16_t*)pk, (uint16_t*)pv, page_stride, p_tok,
                       p_head, page_size, n_slots);
  else
    hipLaunchKernelGGL(paged_kv_copy_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, (uint16_t*)rk,
                       (uint16_t*)rv, r_tok, r_head, T, nkv, slots, (uint16_t*)pk, (uint16_t*)pv, page_stride, p_tok,
                       p_head, page_size, n_slots);
  return check_launch(name);
}

extern "C" int solort_paged_kv_store(const void* k_rows, const void* v_rows, int64_t row_tok_stride,
                                     int64_t row_head_stride, int T, int nkv, int hd, const int64_t* slot_mapping,
                                     void* k_pages, void* v_pages, int64_t page_stride, int64_t kv_tok_stride,
                                     int64_t kv_head_stride, int page_size, int num_pages, solort_stream_t stream) {
  return paged_copy("paged_kv_store", true, (void*)k_rows, (void*)v_rows, row_tok_stride, row_head_stride, T, nkv, hd,
                    slot_mapping, k_pages, v_pages, page_stride, kv_tok_stride, kv_head_stride, page_size, num_pages,
                    stream);
}

extern "C" int solort_paged_kv_gather(const void* k_pages, const void* v_pages, int64_t page_stride,
                                      int64_t kv_tok_stride, int64_t kv_head_stride, int page_size, int num_pages,
                                      const int64_t* slot_mapping, int T, int nkv, int hd, void* k_rows, void* v_rows,
                                      int64_t row_tok_stride, int64_t row_head_stride, solort_stream_t stream) {
  return paged_copy("paged_kv_gather", false, k_rows, v_rows, row_tok_stride, row_head_stride, T, nkv, hd,
                    slot_mapping, (void*)k_pages, (void*)v_pages, page_stride, kv_tok_stride, kv_head_stride,
                    page_size, num_pages, stream);
}
