"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only to check the HIP results against (or, for the CPU
baseline, as the thing timed on the host).  The product path (solort_amd) never imports it and has
no CPU fallback.

Contents (every function cites the reference file:line it restates; paths are
relative to the SoloRT source tree, src/solort/...):
  ref.py      line-faithful torch-on-CPU restatement of the reference runner's
              math, in the reference's own op order and dtype (bf16 or fp32).
  exact.py    numpy restatements used to pin ref.py and the kernels: fp64
              brute-force attention, the fixed-order fp32/bf16 prologue the
              kernels reproduce bit for bit, argmax, and the split-KV
              log-sum-exp combine.

Parity pins (each checked in tests/test_oracle.py):
  rmsnorm       fp64 closed form; constant rows; scale invariance.
  cos/sin/rope  position 0 is the identity; pair norms preserved; q.k after
                rotation depends only on the position difference.
  KV write      the fixed-order prologue equals the torch restatement up to
                rare one-ulp differences from the unspecified torch sum order.
  decode        fp64 brute force; L=1 gives V[0]; equal keys give mean(V);
                a dominant key selects its V row; key permutation invariance;
                grouped-query map equals repeat_interleave; split + combine
                equals unsplit.
  prefill       row 0 is V[0]; last row equals decode at the last position;
                equals an explicit masked softmax.
  verify        equals K+1 sequential decode steps; bottom-right causal
                alignment pinned on the reference's own fallback test inputs
                (tests/test_transformers_flashinfer.py:20-48).
  argmax        numpy.argmax / torch.argmax first-maximum rule, planted ties,
                NaN.
No function of the oracle is left unpinned.
"""
