"""Attention block of the reference's CUDA-graph Qwen3 runner, on the gfx950 kernels.

Mirrors the attention part of ``_GraphQwen3Runner``
(src/solort/model/cuda_graph_executor.py:31-289): a runner-owned static KV
cache ``kc``/``vc`` [layers, max_len, nkv, 128] (:67-69), a device-side
position buffer ``pos_buf`` (:71), length-bucketed decode graphs captured
lazily and routed by position (:75-77, :192-214), bucketed prefill graphs
(:83-85, :137-161), a fixed K+1-token verify graph (:270-289) and the in-graph
greedy argmax (:206).  Everything outside attention (embedding, QKV/o_proj
GEMMs, MLP, lm_head) is not part of this library: each layer's fused QKV
projection output is a static input buffer the caller fills (the role the
QKV GEMM plays at :115, :171, :253), and each layer's attention output
``ctx`` [T, nh*128] is left in a static output buffer (what o_proj consumes
at :131, :185, :264).  Logits for the argmax are likewise a caller-filled
buffer.

Decode and verify run one launch per layer (solort_decode_layer: prologue,
KV write, split-KV attention and combine); prefill runs the prologue launch
then the MFMA causal attention launch.  No launch synchronises the host, so
one graph replay runs a whole step.  Unlike the reference, which captures one
verify graph over all max_len keys, verify graphs are bucketed like decode
so that only the bucket holding the K+1 positions is scanned.
"""
from __future__ import annotations

import torch

from . import ops

HD = 128
DECODE_BUCKETS = (128, 256, 512, 1024, 2048, 4096)
PREFILL_BUCKETS = (16, 32, 64, 128, 256, 512, 1024)


# Prefill buckets from this length on use solort_prefill_layer (q normalised inside the attention
# kernel); shorter ones the two-launch prologue + attention.  The fused layer saves the q round
# trip through HBM and adds the normalisation work ahead of each attention workgroup's first MFMA.
# Measured on MI355X, Qwen3-4B shape, graphed 36-layer step per layer (two-launch against fused):
# 128 rows 9.28 against 9.40 us, 256 rows 11.64 against 11.43, 512 rows 17.83 against 16.28, 1024
# rows 30.1 against 26.6.
FUSED_PREFILL_MIN = 256


def decode_splits(bound: int, nkv: int) -> int:
    """Key splits per KV head for a decode bucket.  Up to 256 keys: 16 keys per split; 512 keys: 32
    (short chunks, latency-bound).  From 1024 keys on: 256 // nkv splits, i.e. one workgroup per CU
    of the 256-CU MI355X with 8 KV heads, the chunk growing with the bucket (32 keys at 1024, 64 at
    2048, ..., 1024 at 32768), and at least bound // 1024 splits (the MFMA kernel's chunks stay at
    most 1024 keys).  Measured on MI355X, Qwen3-4B decode call (32 q / 8 kv heads, graphs of 8 or
    288 calls): KV 128 4.33 us at 8 splits against 4.67 at 4 and 6.30 at 1; KV 256 4.54 at 16
    against 4.67 at 8; KV 512 4.90 at 16 against 4.94 at 32 and 5.49 at 8; KV 1024 5.35 at 32
    against 5.73 at 16 and 6.60 at 64; KV 2048 7.19 at 32 against 8.05 at 64 and 8.74 at 16; KV
    4096 9.72 at 32 against 9.78 at 64 and 11.1 at 128; KV 8192 12.98 at 32 against 13.39 at 64
    and 21.87 at 8; KV 16384 19.1 at 32 against 20.3 at 64 and 23.7 at 16; KV 32768 28.7 at 32
    against 29.7 at 64."""
    if bound <= 256:
        return max(1, bound // 16)
    if bound <= 512:
        return max(1, bound // 32)
    return max(1, min(256 // max(1, nkv), bound // 16), bound // 1024)


def decode_qkv_splits(bound: int, nkv: int) -> int:
    """Key splits per KV head for solort_decode_qkv_layer, which runs the QKV product inside the
    attention launch at 256 // nkv splits (one workgroup per CU for 8 KV heads) with chunks of 16 to
    128 keys: that count from 512 keys on (at 512 keys, 32 splits of 16 keys against the attention's
    own 16 of 32: 4.94 against 4.90 us per attention call, while the fused launch saves ~1.3 us of
    the product's own; from 1024 keys on decode_splits routes 32 as well), decode_splits elsewhere
    (up to 32768 keys also 32 splits, which the entry point runs as two launches)."""
    n = max(1, 256 // max(1, nkv))
    return n if 512 <= bound and 16 <= bound // n <= 128 else decode_splits(bound, nkv)


def verify_bound(last_pos: int, buckets) -> int:
    """Keys a K+1-token verify step scans, its last position last_pos: the decode bucket holding it
    (the first above it, as for decode), cut at the next multiple of max(128, bucket // 8) past it,
    so at most an eighth of the scanned keys lie past the live length (a verify graph per bound, at
    most eight per bucket).  The reference's verify scans all max_len keys under a mask
    (cuda_graph_executor.py:245-263).  Measured on MI355X, Qwen3-4B shape, 5 tokens at 2048..2052,
    128-key splits (us per call, the same outputs): bound 4096 (the bucket, 32 splits, 15 without
    a live key) 10.24, 3072 (24 splits) 10.00, 2560 (20) 9.84, 2176 (17) 9.78."""
    for b in buckets:
        if b > last_pos:
            g = max(128, b // 8)
            return min(b, (last_pos // g + 1) * g)
    raise RuntimeError(f"verify position {last_pos} exceeds the last bucket {max(buckets)}")


def verify_splits(bound: int, nkv: int = 8) -> int:
    """Key splits per KV head for a K+1-token verify bucket.  Up to 4096 keys: 128 keys per split
    (one key tile per wavefront), at most 64 splits; longer buckets: 256 // nkv splits (one
    workgroup per CU for 8 KV heads), chunks of at most 1024 keys.  Measured on MI355X, Qwen3-4B
    shape, 5 tokens at the bucket's end (us per call): KV 4096 12.06 at 32 against 13.4 at 64 and
    13.5 at 16; KV 8192 15.3 at 32 against 16.3 at 64; KV 16384 20.4 at 32 against 23.2 at 64;
    KV 32768 35.3 at 32 against 37.2 at 64."""
    if bound <= 4096:
        return max(1, min(64, bound // 128))
    return max(1, min(256 // max(1, nkv), bound // 128), bound // 1024)


class GraphQwen3Attention:
    """Static-shape attention runner over a runner-owned bf16 KV cache, with hipGraph capture."""

    def __init__(self, nh: int, nkv: int, layers: int, max_len: int, qn_w: torch.Tensor,
                 kn_w: torch.Tensor, eps: float = 1e-6, theta: float = 1e6,
                 device: torch.device | str = "cuda", verify_tokens: int = 5,
                 vocab: int = 151936) -> None:
        if nh % nkv:
            raise RuntimeError(f"nh={nh} must be a multiple of nkv={nkv}")
        self.dev = torch.device(device)
        self.nh, self.nkv, self.L, self.max_len = nh, nkv, layers, int(max_len)
        self.groups = nh // nkv
        self.eps = float(eps)
        self.scale = HD ** -0.5
        self.width = (nh + 2 * nkv) * HD
        self.qn_w = qn_w.to(self.dev, torch.bfloat16).contiguous()
        self.kn_w = kn_w.to(self.dev, torch.bfloat16).contiguous()
        if self.qn_w.shape != (layers, HD) or self.kn_w.shape != (layers, HD):
            raise RuntimeError(f"norm weights must be [{layers}, {HD}]")
        kv_shape = (layers, self.max_len, nkv, HD)
        self.kc = torch.zeros(kv_shape, dtype=torch.bfloat16, device=self.dev)
        self.vc = torch.zeros(kv_shape, dtype=torch.bfloat16, device=self.dev)
        self.inv_freq = ops.inv_freq(HD, theta, self.dev)
        self.pos_buf = torch.zeros(1, dtype=torch.long, device=self.dev)
        self.buckets = sorted({b for b in DECODE_BUCKETS if b < self.max_len} | {self.max_len})
        self.pre_buckets = sorted({b for b in PREFILL_BUCKETS if b <= self.max_len})
        self.vocab = int(vocab)
        # decode: static inputs/outputs of the captured graphs
        self.qkv_dec = torch.zeros(layers, 1, self.width, dtype=torch.bfloat16, device=self.dev)
        self.ctx_dec = torch.zeros(layers, 1, nh * HD, dtype=torch.bfloat16, device=self.dev)
        self.logits_dec = torch.zeros(1, self.vocab, dtype=torch.float32, device=self.dev)
        self.tok_dec = torch.zeros(1, dtype=torch.long, device=self.dev)
        self.cs_dec = torch.zeros(2, 1, HD // 2, dtype=torch.bfloat16, device=self.dev)  # this step's cos/sin
        self.ws_dec = ops.attn_workspace(1, nh, nkv, max(decode_splits(b, nkv) for b in self.buckets), self.dev)
        self.ws_arg = ops.argmax_workspace(max(1, verify_tokens), self.dev)
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        # verify (K+1 tokens)
        self.k1 = int(verify_tokens)
        self.qkv_ver = torch.zeros(layers, self.k1, self.width, dtype=torch.bfloat16, device=self.dev)
        self.ctx_ver = torch.zeros(layers, self.k1, nh * HD, dtype=torch.bfloat16, device=self.dev)
        self.logits_ver = torch.zeros(self.k1, self.vocab, dtype=torch.float32, device=self.dev)
        self.tok_ver = torch.zeros(self.k1, dtype=torch.long, device=self.dev)
        self.draft_ver = torch.zeros(max(1, self.k1 - 1), dtype=torch.long, device=self.dev)  # the K drafts
        self.acc_ver = torch.zeros(2, dtype=torch.long, device=self.dev)  # accepted count, next token
        self.vpos0 = torch.zeros(1, dtype=torch.long, device=self.dev)
        self.cs_ver = torch.zeros(2, self.k1, HD // 2, dtype=torch.bfloat16, device=self.dev)
        self.ws_ver = ops.attn_workspace(self.k1, nh, nkv, max(verify_splits(b, nkv) for b in self.buckets), self.dev)
        self._ver_graphs: dict[int, torch.cuda.CUDAGraph] = {}
        # prefill: padded prompt rows per layer, bucketed graphs
        pmax = self.pre_buckets[-1]
        self.qkv_pre = torch.zeros(layers, pmax, self.width, dtype=torch.bfloat16, device=self.dev)
        self.zero_pos = torch.zeros(1, dtype=torch.long, device=self.dev)  # prefill positions start at 0
        self.cs_pre = torch.zeros(2 * pmax * (HD // 2), dtype=torch.bfloat16, device=self.dev)  # step cos/sin
        self.ctx_pre = torch.zeros(layers, pmax, nh * HD, dtype=torch.bfloat16, device=self.dev)
        # q of the short buckets (the fused layer does not materialise it)
        self.q_pre = torch.zeros(min(pmax, FUSED_PREFILL_MIN), nh, HD, dtype=torch.bfloat16, device=self.dev)
        self._pre_graphs: dict[int, torch.cuda.CUDAGraph] = {}

    # ------------------------------------------------------------ decode

    def _decode_forward(self, bound: int) -> None:
        ns = decode_splits(bound, self.nkv)
        ops.rope_rows(self.inv_freq, self.pos_buf, 1, self.cs_dec)  # once per step (:164)
        for li in range(self.L):
            ops.decode_layer(self.qkv_dec[li], self.qn_w[li], self.kn_w[li], self.eps, self.cs_dec, self.pos_buf,
                             self.kc[li], self.vc[li], bound, self.scale, self.ws_dec, ns,
                             self.ctx_dec[li], self.nh, self.nkv)
        ops.argmax_rows(self.logits_dec, self.tok_dec, self.ws_arg)

    def _bucket_for(self, pos: int) -> int:
        """cuda_graph_executor.py:192-193: the first bucket strictly above the position."""
        for b in self.buckets:
            if b > pos:
                return b
        raise RuntimeError(f"decode position {pos} exceeds max_len {self.max_len}")

    def _capture(self, bound: int) -> None:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._decode_forward(bound)
        self._graphs[bound] = graph

    def _replay(self, pos: int) -> int:
        bound = self._bucket_for(pos)
        if bound not in self._graphs:
            self._capture(bound)
        self._graphs[bound].replay()
        return bound

    def decode(self, qkv: torch.Tensor, pos: int) -> torch.Tensor:
        """One decode step at `pos`: qkv [layers, 1, (nh+2nkv)*128] -> ctx [layers, 1, nh*128] (static buffer)."""
        if not 0 <= pos < self.max_len:
            raise RuntimeError(f"decode position {pos} outside [0, {self.max_len})")
        self.qkv_dec.copy_(qkv)
        self.pos_buf.fill_(int(pos))
        self._replay(pos)
        return self.ctx_dec

    def decode_argmax(self, qkv: torch.Tensor, pos: int, logits: torch.Tensor) -> torch.Tensor:
        """decode() plus the in-graph greedy argmax of `logits` [1, vocab]; returns the [1] token buffer."""
        self.logits_dec.copy_(logits)
        self.decode(qkv, pos)
        return self.tok_dec

    # ------------------------------------------------------------ prefill

    def _prefill_forward(self, bound: int) -> None:
        """cuda_graph_executor.py:109-130 (attention part): rows 0..bound-1 at positions 0..bound-1."""
        cs = self.cs_pre[: 2 * bound * (HD // 2)].view(2, bound, HD // 2)
        ops.rope_rows(self.inv_freq, self.zero_pos, bound, cs)  # cos/sin once per step (:111)
        for li in range(self.L):
            if bound >= FUSED_PREFILL_MIN:  # prologue of the K/V rows, then attention normalising q itself
                ops.prefill_layer(self.qkv_pre[li, :bound], self.qn_w[li], self.kn_w[li], self.eps, cs, self.kc[li],
                                  self.vc[li], self.scale, self.ctx_pre[li, :bound], self.nh, self.nkv)
            else:  # short prompts: the whole prologue, then attention on the materialised q
                ops.qknorm_rope_kvwrite_cs(self.qkv_pre[li, :bound], self.qn_w[li], self.kn_w[li], self.eps, cs,
                                           None, self.q_pre[:bound], self.kc[li], self.vc[li], self.nh, self.nkv)
                ops.prefill_attn(self.q_pre[:bound], self.kc[li], self.vc[li], self.scale,
                                 self.ctx_pre[li, :bound])

    def prefill(self, qkv: torch.Tensor) -> torch.Tensor:
        """Graphed bucketed prefill (cuda_graph_executor.py:149-161): qkv [layers, plen, width] for
        prompt positions 0..plen-1, padded with zero rows to the first bucket >= plen.  Writes cache
        rows 0..bucket-1 (padding rows included, as in the reference; decode never reads them) and
        returns ctx [layers, plen, nh*128] (a view of the static buffer)."""
        plen = int(qkv.shape[1])
        bound = next((b for b in self.pre_buckets if b >= plen), None)
        if bound is None or plen < 1:
            raise RuntimeError(f"prompt length {plen} outside the prefill buckets {self.pre_buckets}")
        self.qkv_pre[:, :plen].copy_(qkv)
        self.qkv_pre[:, plen:bound].zero_()
        if bound not in self._pre_graphs:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._prefill_forward(bound)
            self._pre_graphs[bound] = graph
        self._pre_graphs[bound].replay()
        return self.ctx_pre[:, :plen]

    # ------------------------------------------------------------ verify

    def _verify_forward(self, bound: int) -> None:
        ns = verify_splits(bound, self.nkv)
        ops.rope_rows(self.inv_freq, self.vpos0, self.k1, self.cs_ver)  # once per step (:248)
        for li in range(self.L):
            ops.decode_layer(self.qkv_ver[li], self.qn_w[li], self.kn_w[li], self.eps, self.cs_ver, self.vpos0,
                             self.kc[li], self.vc[li], bound, self.scale, self.ws_ver, ns,
                             self.ctx_ver[li], self.nh, self.nkv)
        ops.argmax_rows(self.logits_ver, self.tok_ver, self.ws_arg)
        if self.k1 > 1:  # greedy acceptance on the device (:476, :478, :481)
            ops.accept_prefix(self.tok_ver, self.draft_ver, self.acc_ver)

    def verify(self, qkv: torch.Tensor, pos_start: int, logits: torch.Tensor | None = None,
               draft: torch.Tensor | None = None) -> torch.Tensor:
        """Score K+1 tokens at pos_start..pos_start+K (cuda_graph_executor.py:270-289).

        qkv [layers, K+1, width]; returns ctx [layers, K+1, nh*128].  If logits [K+1, vocab] are
        given, tok_ver holds their argmax after the replay; with the K draft tokens (int64), acc_ver
        then holds the accepted-prefix length and the token that follows it.
        """
        if not 0 <= pos_start <= self.max_len - self.k1:
            raise RuntimeError(f"verify positions {pos_start}..{pos_start + self.k1 - 1} exceed max_len")
        bound = verify_bound(pos_start + self.k1 - 1, self.buckets)
        if bound not in self._ver_graphs:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._verify_forward(bound)
            self._ver_graphs[bound] = graph
        self.qkv_ver.copy_(qkv)
        if logits is not None:
            self.logits_ver.copy_(logits)
        if draft is not None:
            self.draft_ver.copy_(draft)
        self.vpos0.fill_(int(pos_start))
        self._ver_graphs[bound].replay()
        return self.ctx_ver
