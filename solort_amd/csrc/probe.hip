// Device probes: where workgroups run, and the launch / streaming floor that
// bounds a latency-bound call on this device.
//
// None of these has a counterpart in the reference; bench.py uses them to
// measure the floor a decode-attention call is compared with, and the
// library uses the placement probe once per device (solort_init) before it
// relies on the workgroup -> XCD placement for the single-launch split
// combine (decode.hip).
#include <mutex>

#include "common.h"
#include "capi_internal.h"

namespace solort {

// hwreg(HW_REG_XCC_ID, 0, 16): the index of the accelerator complex die
// (XCD) the wave runs on; hwreg(HW_REG_HW_ID): CU, SIMD and wave slot.
__device__ __forceinline__ uint32_t xcc_id() { return __builtin_amdgcn_s_getreg(20 | (0 << 6) | ((16 - 1) << 11)); }
__device__ __forceinline__ uint32_t hw_id() { return __builtin_amdgcn_s_getreg(4 | (0 << 6) | ((32 - 1) << 11)); }

__global__ __launch_bounds__(64) void placement_kernel(uint32_t* __restrict__ out) {
  if (threadIdx.x == 0) {
    out[2 * blockIdx.x] = xcc_id();
    out[2 * blockIdx.x + 1] = hw_id();
  }
}

__global__ __launch_bounds__(64) void empty_kernel() {}

constexpr int kProbeReadNT = 16;  // solort_probe_read's in_flight flag: non-temporal loads

// Streaming read of n16 16-byte chunks, grid-stride, U loads in flight per
// thread (NT: with the non-temporal hint); each workgroup stores one word of
// the xor of what it read (so the loads cannot be dropped).
template <int U, bool NT>
__global__ __launch_bounds__(256) void read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                   uint32_t* __restrict__ sink) {
  __shared__ uint32_t s_x[4];
  const int64_t stride = (int64_t)gridDim.x * 256;
  uint32_t x = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      v[u] = i + u * stride < n16 ? (NT ? ld_stream(src + i + u * stride) : src[i + u * stride])
                                  : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int u = 0; u < U; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (int m = 32; m >= 1; m >>= 1) x ^= __shfl_xor(x, m, 64);
  if ((threadIdx.x & 63) == 0) s_x[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = s_x[0] ^ s_x[1] ^ s_x[2] ^ s_x[3];
}

// The long-context decode's K/V reads with no arithmetic: block (h, s) of an
// (nkv, n_split) grid (linear index h + nkv * s, as the decode's) reads KV head
// h's 256-byte rows of keys [s * chunk, (s + 1) * chunk) of k and of v, from
// caches laid out [rows][nkv][128] bf16.  Wavefront w takes the 32-row tiles at
// s * chunk + 32 w + 128 i, lane l the 16-byte column l % 16 of rows l / 16 + 4 q
// (q < 8), with the non-temporal hint.  D = 1: a tile's loads issue once the
// previous tile has arrived (one tile in flight per wavefront, as the decode
// keeps); D = 2: the next tile's loads issue before the current tile is used
// (two in flight).  Each workgroup stores one word of the xor of what it read.
template <int D>
__global__ __launch_bounds__(256) void read_heads_kernel(const uint16_t* __restrict__ k,
                                                         const uint16_t* __restrict__ v, int nkv, int chunk,
                                                         uint32_t* __restrict__ sink) {
  __shared__ uint32_t s_x[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 15, lrow = lane >> 4;
  const int h = blockIdx.x % nkv, s = blockIdx.x / nkv;
  const int64_t tok = (int64_t)nkv * 128;
  const uint16_t* kp = k + h * 128 + 8 * j;
  const uint16_t* vp = v + h * 128 + 8 * j;
  uint32_t x = 0;
  uint4 kt[D][8], vt[D][8];
  auto fetch = [&](int b, int k0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t off = (int64_t)(k0 + lrow + 4 * q) * tok;
      kt[b][q] = ld_stream(kp + off);
      vt[b][q] = ld_stream(vp + off);
    }
  };
  auto use = [&](int b) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
      x ^= kt[b][q].x ^ kt[b][q].y ^ kt[b][q].z ^ kt[b][q].w ^ vt[b][q].x ^ vt[b][q].y ^ vt[b][q].z ^ vt[b][q].w;
  };
  const int kend = (s + 1) * chunk;
  int k0 = s * chunk + 32 * wave;  // the tile in buffer 0
  fetch(0, k0);
  if constexpr (D == 1) {
    for (;;) {
      use(0);
      k0 += 128;
      if (k0 >= kend) break;
      fetch(0, k0);
    }
  } else {
    // Buffers alternate; the tile at k0 sits in buffer 0 at the top of each round.
    for (;;) {
      const bool more = k0 + 128 < kend;
      if (more) fetch(1, k0 + 128);
      use(0);
      if (!more) break;
      const bool more2 = k0 + 256 < kend;
      if (more2) fetch(0, k0 + 256);
      use(1);
      if (!more2) break;
      k0 += 256;
    }
  }
  for (int m = 32; m >= 1; m >>= 1) x ^= __shfl_xor(x, m, 64);
  if (lane == 0) s_x[wave] = x;
  __syncthreads();
  if (tid == 0) sink[blockIdx.x] = s_x[0] ^ s_x[1] ^ s_x[2] ^ s_x[3];
}

namespace {
constexpr int kMaxDevices = 64;
constexpr int kProbeBlocks = 2048;
std::mutex g_mu;
int g_xcd_state[kMaxDevices];  // 0 unknown, 1 verified round robin over 8, -1 not
int g_cus[kMaxDevices];        // compute units, 0 until first asked
}  // namespace

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

// Runs the placement probe on the current device and records whether
// workgroup b always runs on the XCD of workgroup b % 8.  Synchronous: call
// outside graph capture.
int verify_xcd_placement(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return set_error(SOLORT_EINVAL, "init: device %d out of range", dev);
  uint32_t* d = nullptr;
  const size_t bytes = (size_t)kProbeBlocks * 2 * sizeof(uint32_t);
  hipError_t e = hipMalloc((void**)&d, bytes);
  if (e != hipSuccess) return set_error((int)e, "init: hipMalloc: %s", hipGetErrorString(e));
  uint32_t h[kProbeBlocks * 2];
  hipLaunchKernelGGL(placement_kernel, dim3(kProbeBlocks), dim3(64), 0, (hipStream_t)0, d);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpy(h, d, bytes, hipMemcpyDeviceToHost);
  hipFree(d);
  if (e != hipSuccess) return set_error((int)e, "init: placement probe: %s", hipGetErrorString(e));
  bool ok = true;
  for (int b = 8; b < kProbeBlocks && ok; ++b) ok = h[2 * b] == h[2 * (b % 8)];
  std::lock_guard<std::mutex> lk(g_mu);
  g_xcd_state[dev] = ok ? 1 : -1;
  return 0;
}

bool xcd_round_robin(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lk(g_mu);
  return g_xcd_state[dev] == 1;
}

}  // namespace solort

using namespace solort;

extern "C" int solort_probe_placement(uint32_t* out, int n_wg, solort_stream_t stream) {
  if (!out || ((uintptr_t)out & 3u)) return set_error(SOLORT_EINVAL, "probe_placement: out must be 4-byte aligned");
  if (n_wg < 1 || n_wg > (1 << 20)) return set_error(SOLORT_EINVAL, "probe_placement: n_wg %d", n_wg);
  hipLaunchKernelGGL(placement_kernel, dim3(n_wg), dim3(64), 0, (hipStream_t)stream, out);
  return check_launch("probe_placement");
}

extern "C" int solort_probe_empty(int n_wg, solort_stream_t stream) {
  if (n_wg < 1 || n_wg > (1 << 20)) return set_error(SOLORT_EINVAL, "probe_empty: n_wg %d", n_wg);
  hipLaunchKernelGGL(empty_kernel, dim3(n_wg), dim3(64), 0, (hipStream_t)stream);
  return check_launch("probe_empty");
}

extern "C" int solort_probe_read(const void* src, int64_t nbytes, int n_wg, int in_flight, uint32_t* sink,
                                 solort_stream_t stream) {
  if (!src || !sink || !aligned16(src) || ((uintptr_t)sink & 3u))
    return set_error(SOLORT_EINVAL, "probe_read: src must be 16-byte and sink 4-byte aligned");
  if (nbytes < 16 || nbytes % 16) return set_error(SOLORT_EINVAL, "probe_read: nbytes %lld", (long long)nbytes);
  if (n_wg < 1 || n_wg > (1 << 20)) return set_error(SOLORT_EINVAL, "probe_read: n_wg %d", n_wg);
  const int64_t n16 = nbytes / 16;
  hipStream_t s = (hipStream_t)stream;
#define SOLORT_READ(UU, NN) \
  hipLaunchKernelGGL((read_kernel<UU, NN>), dim3(n_wg), dim3(256), 0, s, (const uint4*)src, n16, sink)
  switch (in_flight) {
    case 1: SOLORT_READ(1, false); break;
    case 2: SOLORT_READ(2, false); break;
    case 4: SOLORT_READ(4, false); break;
    case 1 | kProbeReadNT: SOLORT_READ(1, true); break;
    case 2 | kProbeReadNT: SOLORT_READ(2, true); break;
    case 4 | kProbeReadNT: SOLORT_READ(4, true); break;
    default: return set_error(SOLORT_EINVAL, "probe_read: in_flight %d not in {1, 2, 4} (+16: non-temporal)", in_flight);
  }
#undef SOLORT_READ
  return check_launch("probe_read");
}

extern "C" int solort_probe_read_heads(const void* k, const void* v, int64_t rows, int nkv, int n_split,
                                       int tiles_in_flight, uint32_t* sink, solort_stream_t stream) {
  if (!k || !v || !sink || !aligned16(k) || !aligned16(v) || ((uintptr_t)sink & 3u))
    return set_error(SOLORT_EINVAL, "probe_read_heads: k and v must be 16-byte and sink 4-byte aligned");
  if (nkv < 1 || nkv > 1024 || n_split < 1 || n_split > 65536 || rows < 128 || rows > (1LL << 30) ||
      rows % n_split != 0 || (rows / n_split) % 128 != 0 || (int64_t)nkv * n_split > (1 << 20))
    return set_error(SOLORT_EINVAL, "probe_read_heads: rows %lld must split into n_split %d chunks of a multiple "
                     "of 128 rows (nkv %d)", (long long)rows, n_split, nkv);
  if (tiles_in_flight != 1 && tiles_in_flight != 2)
    return set_error(SOLORT_EINVAL, "probe_read_heads: tiles_in_flight %d not 1 or 2", tiles_in_flight);
  if (tiles_in_flight == 1)
    hipLaunchKernelGGL(read_heads_kernel<1>, dim3((unsigned)(nkv * n_split)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)k, (const uint16_t*)v, nkv, (int)(rows / n_split), sink);
  else
    hipLaunchKernelGGL(read_heads_kernel<2>, dim3((unsigned)(nkv * n_split)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)k, (const uint16_t*)v, nkv, (int)(rows / n_split), sink);
  return check_launch("probe_read_heads");
}
