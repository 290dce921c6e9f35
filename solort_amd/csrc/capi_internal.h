// Error reporting shared by the C-ABI entry points (include/solort_hip.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/solort_hip.h"

namespace solort {

// Records a printf-style message for solort_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Returns 0 if the last launch on this thread succeeded, else records and
// returns the hipError_t.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// prologue.hip: argument checks of the QK-RMSNorm + RoPE + KV-write entry
// points (rope_src: inv_freq or the cos/sin table); 0 or the error code.
int check_prologue(const char* name, const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv, int hd,
                   const void* qn_w, const void* kn_w, const void* rope_src, const void* q_out, const void* k_cache,
                   const void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride, int64_t max_len);

// probe.hip: runs the workgroup-placement probe on device `dev` (current)
// and records whether workgroup b always runs on the XCD of workgroup b % 8;
// synchronous.  0 or the error code.
int verify_xcd_placement(int dev);
// probe.hip: whether that check passed on device `dev`.
bool xcd_round_robin(int dev);
// probe.hip: compute units of the current device (queried once per device; 0
// if the query fails).
int cu_count();

// noalloc.hip: looks up the device address of the allocation-free entry
// point's scratch array on device `dev` (current), once.  0 or the error code.
int noalloc_scratch_setup(int dev);

// prologue.hip: QK-RMSNorm + RoPE of the K rows and the cache write of the K
// and V rows of T tokens at positions 0..T-1 (no q rows), cos/sin from a
// solort_rope_rows table; arguments already validated.
int launch_kv_rows_cs(const void* qkv, int64_t qkv_row_stride, int T, int nh, int nkv, const void* kn_w, float eps,
                      const void* rope_cs, void* k_cache, void* v_cache, int64_t kv_tok_stride, int64_t kv_head_stride,
                      int64_t max_len, hipStream_t stream);

}  // namespace solort
