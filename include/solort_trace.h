/*
 * solort_trace.h - phase stamps of the tracing build of libsolort_hip.
 *
 * No counterpart in the reference (whose tracing is host-side timing of whole
 * steps).  A library built with SOLORT_PHASE_STAMPS (python -m
 * solort_amd.build --stamps, written as libsolort_hip_stamps.so beside the
 * normal library) records in its decode and prefill kernels, per workgroup of
 * the most recent launch, the device clock (s_memrealtime, 100 MHz ticks) at
 * fixed points of the workgroup's work; the functions below copy them to host
 * (synchronous; call after the launch completed, outside graph capture).  The
 * normal library has neither the stamps nor these functions.
 *
 * Layout: 16 uint64 slots per workgroup, workgroup b at [16 b, 16 b + 16);
 * slots not reached by a workgroup keep their previous contents (clear them
 * by comparing against a launch's first stamp).
 *   decode split kernels (linear workgroup kvh + nkv * split):
 *     0 start, 1 position read, 2 q rows normalised and in LDS, 3 key loop
 *     done (wave 0), 4 partial stored, 5 end, 6 merge poll started and
 *     7 merge poll done (merging workgroups of the in-launch merge only);
 *     MFMA split kernel only: 8 + w key loop done by wavefront w, 12 + w
 *     wavefront w issued the loads of its last key tile
 *   prefill_kernel (workgroup blockIdx.x):
 *     0 start, 3 key loop done (wave 0), 5 end (outputs stored)
 */
#ifndef SOLORT_TRACE_H
#define SOLORT_TRACE_H

#ifdef __cplusplus
extern "C" {
#endif

/* 0 on success.  n_blocks <= 4096. */
int solort_phase_stamps_decode(void* host, int n_blocks);
int solort_phase_stamps_prefill(void* host, int n_blocks);

#ifdef __cplusplus
}
#endif

#endif /* SOLORT_TRACE_H */
