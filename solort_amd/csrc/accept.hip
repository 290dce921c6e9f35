// Greedy speculative acceptance on the device: the length of the prefix of
// draft tokens the target model agrees with, and the token that follows it.
//
// Follows src/solort/model/cuda_graph_executor.py:476,
//   a = int((tg[:k] == draft_vec).cumprod(0).sum().item())
// with tg = argmax of the K+1 verify rows (:475), and the token the round
// appends after the accepted drafts, tg[a] (:478, :481).  The reference reads
// `a` back to the host; here it stays on the device, so the verify graph
// (argmax, then this) needs no synchronisation.
//
// One wavefront scans the k pairs 64 at a time; a ballot of the mismatches
// gives the first one (count trailing zeros).
#include "common.h"
#include "capi_internal.h"

namespace solort {

__global__ __launch_bounds__(64) void accept_prefix_kernel(const int64_t* __restrict__ target,
                                                           const int64_t* __restrict__ draft, int k,
                                                           int64_t* __restrict__ out) {
  const int lane = threadIdx.x;
  int a = k;
  for (int i0 = 0; i0 < k; i0 += 64) {
    const int i = i0 + lane;
    const bool miss = i < k && target[i] != draft[i];
    const uint64_t m = __builtin_amdgcn_ballot_w64(miss);
    if (m) {
      a = i0 + (int)__builtin_ctzll(m);
      break;
    }
  }
  if (lane == 0) {
    out[0] = a;
    out[1] = target[a];
  }
}

}  // namespace solort

using namespace solort;

extern "C" int solort_accept_prefix(const int64_t* target, const int64_t* draft, int k, int64_t* out,
                                    solort_stream_t stream) {
  if (k < 1 || k > (1 << 20)) return set_error(SOLORT_EINVAL, "accept_prefix: k=%d outside [1, 2^20]", k);
  if (!target || !draft || !out) return set_error(SOLORT_EINVAL, "accept_prefix: null pointer");
  if (((uintptr_t)target | (uintptr_t)draft | (uintptr_t)out) & 7u)
    return set_error(SOLORT_EINVAL, "accept_prefix: pointers must be 8-byte aligned");
  hipLaunchKernelGGL(accept_prefix_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, target, draft, k, out);
  return check_launch("accept_prefix");
}
