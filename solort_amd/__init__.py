"""MI355X-native (gfx950) attention hot path of a Qwen3 static-KV decode step.

Hand-written HIP kernels behind a C ABI (include/solort_hip.h), driven from
PyTorch-ROCm:

  ops       one torch-tensor function per C-ABI entry point
  runner    attention layer loop over the static KV cache with per-bucket
            hipGraph capture (the attention block of SoloRT's
            _GraphQwen3Runner)
  workloads seeded synthetic inputs for the parity tests and the benchmark
  build     hipcc recipe for libsolort_hip.so
"""
__all__ = ["ops", "runner", "workloads"]
