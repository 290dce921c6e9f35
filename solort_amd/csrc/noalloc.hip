// solort_decode_layer without a caller-supplied workspace, for callers that
// cannot allocate device memory.  The splits' partials and the in-launch
// merge's per-KV-head counters live in `scratch`, one fixed array per GPU
// (SOLORT_NOALLOC_SCRATCH_BYTES), loaded with the library and held until the
// process ends.
//
// The array starts zeroed (the counters' first value) and keeps the last
// call's counters and partials: each call advances the counters of its KV
// heads and tags its partials with them, so no partial of an earlier call is
// taken for one of this call.  All calls on one GPU share it, so calls that
// overlap in time on one GPU race.
//
// In host code `scratch` names a host-side stand-in, not the device array:
// its device address comes from hipGetSymbolAddress, once per device with
// that device current (solort_init, or the entry point's first call on the
// device), and only that address is ever passed to a kernel.
#include <mutex>

#include "common.h"
#include "capi_internal.h"

namespace solort {

constexpr size_t kScratchBytes = SOLORT_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device
}  // namespace

int noalloc_scratch_setup(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return set_error(SOLORT_EINVAL, "noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_scratch[dev]) return 0;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr)
    return set_error(e != hipSuccess ? (int)e : SOLORT_EINVAL, "noalloc: hipGetSymbolAddress(scratch): %s",
                     hipGetErrorString(e));
  g_scratch[dev] = ptr;
  return 0;
}

}  // namespace solort

using namespace solort;

extern "C" int solort_decode_layer_noalloc(const void* qkv, int64_t qkv_row_stride, int nq, int nh, int nkv, int hd,
                                           const void* qn_w, const void* kn_w, float eps, const void* rope_cs,
                                           const int64_t* pos0_dev, void* k_cache, void* v_cache,
                                           int64_t kv_tok_stride, int64_t kv_head_stride, int64_t max_len, int bound,
                                           float scale, int n_split, void* out, int out_dtype,
                                           solort_stream_t stream) {
  const size_t need = solort_attn_workspace_bytes(nq, nh, nkv, hd, n_split);
  if (need == 0)
    return set_error(SOLORT_EINVAL, "decode_layer_noalloc: bad shape nq=%d nh=%d nkv=%d hd=%d n_split=%d", nq, nh,
                     nkv, hd, n_split);
  if (need > kScratchBytes)
    return set_error(SOLORT_EINVAL,
                     "decode_layer_noalloc: nq=%d nh=%d nkv=%d n_split=%d needs %zu bytes of scratch, above the "
                     "fixed %zu",
                     nq, nh, nkv, n_split, need, kScratchBytes);
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error((int)e, "decode_layer_noalloc: no device: %s", hipGetErrorString(e));
  const int rc = noalloc_scratch_setup(dev);
  if (rc) return rc;
  void* ws;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    ws = g_scratch[dev];
  }
  return solort_decode_layer(qkv, qkv_row_stride, nq, nh, nkv, hd, qn_w, kn_w, eps, rope_cs, pos0_dev, k_cache,
                             v_cache, kv_tok_stride, kv_head_stride, max_len, bound, scale, ws, n_split, out, out_dtype,
                             stream);
}
