"""Benchmark of the gfx950 attention hot path on one MI355X.

Step = one graph replay of a Qwen3-4B decode step's attention block at KV
length 1024: for each of 36 layers, the QK-RMSNorm + RoPE prologue with the
KV write, then split-KV GQA decode attention (32 q / 8 kv heads, head_dim
128, bf16), then the greedy argmax over a 151,936-entry logits row.  The
reported value is microseconds per layer.  Eight independent KV caches
(1.2 GB) are rotated so that every step reads its KV from HBM, not from the
256 MB infinity cache.

Alongside: the time of one decode-attention call (the split-KV kernel and its
combine kernel; HIP events around graph replays of 36 x 8 calls over distinct
KV slices) against the HBM roofline, prefill attention TFLOP/s when the
prefill kernel is built, and the CPU baseline: the oracle's fp32 torch
restatement of the reference path timed on the host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
# The split kernel of one Qwen3-4B decode-attention call at KV 1024 (32 q / 8 kv heads, 32 splits).
DECODE_KERNEL = "decode_lanes_packed_kernel<4, 2>"
# The 64 MiB device copy bench.py issues outside its timed regions: the reference that scales the
# FETCH_SIZE / WRITE_SIZE counters into bytes.
CALIB_BYTES = 64 << 20


def decode_bytes(live: int, nh: int = 32, nkv: int = 8, hd: int = 128) -> int:
    """Algorithmic HBM bytes of one decode-attention launch: K and V rows 0..live-1 of every KV head,
    plus q in and the output out (bf16)."""
    return 2 * nkv * live * hd * 2 + 2 * nh * hd * 2


def prefill_flops(T: int, nh: int = 32, hd: int = 128) -> int:
    """Causal attention flops: 2 matmuls x 2 flop x nh x hd over the T(T+1)/2 visible pairs."""
    return 4 * nh * hd * T * (T + 1) // 2


def prefill_bytes(T: int, nh: int = 32, nkv: int = 8, hd: int = 128) -> int:
    """Algorithmic HBM bytes of one layer's prefill attention block: the qkv rows read, the K/V
    cache rows and the output rows written (bf16)."""
    return T * hd * 2 * ((nh + 2 * nkv) + 2 * nkv + nh)


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--live", type=int, default=1024, help="KV live length of the decode workload")
    p.add_argument("--kv-sets", type=int, default=8, help="independent KV caches rotated per step")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-sweep", action="store_true", help="skip the per-bucket decode extras")
    p.add_argument("--no-traffic", action="store_true",
                   help="skip the in-run HBM traffic measurement (two short rocprofv3 --pmc passes)")
    p.add_argument("--only", choices=("all", "decode", "prefill", "long", "verify", "gemv", "model", "paged",
                                      "torchref", "floor", "cpu", "stamps"),
                   default="all",
                   help="decode: the decode step and its kernel only; prefill: the prefill kernels only; "
                        "long: the Qwen3-8B KV 32768 decode only; verify: the speculative verify and argmax "
                        "only; gemv: the decode-step GEMVs only; model: whole-model greedy decode only; paged: the "
                        "paged-KV decode only; torchref: the reference's torch decode ops on this GPU only; "
                        "floor: the launch and streaming floor probes only; cpu: the CPU baselines only; stamps: "
                        "in-kernel phase timelines of the decode (KV 1024, KV 32768) and prefill (T 1024) kernels "
                        "from the tracing build (python -m solort_amd.build --stamps) (for per-workload profiles)")
    return p.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): there is no multi-GPU path; "
              "each GPU would run its own KV heads or key splits.", file=sys.stderr)
        return 2
    if args.only == "cpu":
        print(json.dumps({"cpu_baseline": cpu_baseline(args.cpu_seconds, args.live)}), flush=True)
        return 0

    import torch

    from solort_amd import _lib
    if args.only == "stamps":
        _lib.use_stamp_build()
    from solort_amd import ops
    from solort_amd import workloads as wl
    from solort_amd.runner import GraphQwen3Attention, decode_splits

    dev = torch.device("cuda:0")
    sh = wl.QWEN3_4B
    live = int(args.live)
    pos = live - 1
    bound = next(b for b in (128, 256, 512, 1024) if b > pos) if live <= 1024 else live
    max_len = max(1024, bound)
    gen = torch.Generator(device=dev).manual_seed(1001)

    def rnd(*shape, std=1.0, mean=0.0):
        return (torch.randn(*shape, generator=gen, device=dev) * std + mean).to(torch.bfloat16)

    qn_w = rnd(sh.layers, 128, std=0.1, mean=1.0)
    kn_w = rnd(sh.layers, 128, std=0.1, mean=1.0)
    runners = []
    for _ in range(args.kv_sets):
        r = GraphQwen3Attention(sh.nh, sh.nkv, sh.layers, max_len, qn_w, kn_w, device=dev)
        r.kc[:, :pos].copy_(rnd(sh.layers, pos, sh.nkv, 128))
        r.vc[:, :pos].copy_(rnd(sh.layers, pos, sh.nkv, 128))
        r.qkv_dec.copy_(rnd(sh.layers, 1, sh.qkv_width))
        r.logits_dec.copy_(torch.randn(1, wl.VOCAB, generator=gen, device=dev) * 3)
        r.pos_buf.fill_(pos)
        r._capture(bound)
        runners.append(r)
    torch.cuda.synchronize()

    if args.only == "prefill":
        print(json.dumps({"prefill": prefill_extras(torch, ops, runners, dev, sh)}), flush=True)
        return 0
    if args.only == "long":
        print(json.dumps({"decode_8b_kv32768": long_decode_extras(torch, ops, wl, dev),
                          "decode_mid_kv": mid_decode_extras(torch, ops, wl, dev)}), flush=True)
        return 0
    if args.only == "verify":
        print(json.dumps(verify_extras(torch, ops, wl, runners, dev, sh)), flush=True)
        return 0
    if args.only == "gemv":
        print(json.dumps({"decode_gemv": gemv_extras(torch, ops, dev),
                          "decode_qkv_layer": qkv_layer_extras(torch, ops, wl, dev)}), flush=True)
        return 0
    if args.only == "torchref":
        print(json.dumps({"torch_reference_decode": torch_reference_extras(torch, runners, dev, sh, bound)}),
              flush=True)
        return 0
    if args.only == "paged":
        print(json.dumps({"paged_decode_kv1024": paged_extras(torch, ops, runners, dev, sh)}), flush=True)
        return 0
    if args.only == "floor":
        print(json.dumps({"floor": floor_extras(torch, ops, runners, dev, sh)}), flush=True)
        return 0
    if args.only == "stamps":
        print(json.dumps({"stamps": stamp_extras(torch, ops, wl, runners, dev, sh, bound)}), flush=True)
        return 0
    if args.only == "model":
        del runners
        torch.cuda.empty_cache()
        print(json.dumps({"decode_model": model_extras(torch, dev)}), flush=True)
        return 0

    # ---------------------------------------------------------------- timed graph replays
    for i in range(args.warmup):
        runners[i % len(runners)]._graphs[bound].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        runners[i % len(runners)]._graphs[bound].replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    us_per_layer = ms_per_step * 1e3 / sh.layers

    # ---------------------------------------------------------------- decode kernel alone (roofline)
    ns = decode_splits(bound, sh.nkv)
    lib = _lib.load()
    single = lib.solort_combine_mode(-1) == 1
    kern_us = time_decode_kernel(torch, ops, runners, bound, ns, sh, dev, reps=4)
    kbytes = decode_bytes(live, sh.nh, sh.nkv)
    achieved = kbytes / (kern_us * 1e-6) / 1e9
    # A plain 64 MiB device copy, outside every timed region: the reference point that scales the
    # FETCH_SIZE / WRITE_SIZE hardware counters of a profiling run into bytes.
    calib_src = torch.empty(CALIB_BYTES, dtype=torch.uint8, device=dev)
    torch.empty_like(calib_src).copy_(calib_src)
    torch.cuda.synchronize()

    result = {
        "metric": "decode-attn us/layer + HBM GB/s (Qwen3-4B, KV 1024); prefill attn TFLOP/s",
        "value": round(us_per_layer, 4),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) KV/qkv, norm weights N(1,0.1), logits N(0,3))",
        "config": {"workload": f"Qwen3-4B decode attention, batch 1, 32q/8kv heads, head_dim 128, "
                               f"KV live {live} (bucket {bound}), 36 layers per step, {args.kv_sets} rotated "
                               f"KV sets", "live": live, "bucket": bound, "layers": sh.layers,
                   "n_split": ns},
        "decode_gbps": round(kbytes / (us_per_layer * 1e-6) / 1e9, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "kernel": (f"solort_decode_layer = {DECODE_KERNEL} (split-KV attention, splits "
                                "merged in the same launch)" if single else
                                f"solort_decode_layer = {DECODE_KERNEL} + combine_kernel<1, 4>"),
                     "kernel_us": round(kern_us, 3),
                     "algorithmic_bytes": kbytes,
                     "in_launch_merge": single},
    }

    if args.only == "decode":
        # A graph of 288 empty kernels, timed like the decode calls: under a kernel tracer its
        # dispatches give the tracer's per-dispatch duration beside the decode kernel's.
        def empty():
            _lib.check(lib.solort_probe_empty(1, torch.cuda.current_stream(dev).cuda_stream), "probe_empty")
        result["empty_node_us"] = round(_graph_us(torch, dev, [empty] * 288, reps=4), 3)

    if not args.no_sweep and args.only == "all":
        result["extras"] = extras(torch, ops, wl, runners, dev, sh)
        result["extras"]["floor"] = floor_extras(torch, ops, runners, dev, sh)
        result["extras"].update(verify_extras(torch, ops, wl, runners, dev, sh))
        result["extras"]["decode_8b_kv32768"] = long_decode_extras(torch, ops, wl, dev)
        result["extras"]["decode_mid_kv"] = mid_decode_extras(torch, ops, wl, dev)
        result["extras"]["decode_gemv"] = gemv_extras(torch, ops, dev)
        result["extras"]["decode_qkv_layer"] = qkv_layer_extras(torch, ops, wl, dev)
        result["extras"]["paged_decode_kv1024"] = paged_extras(torch, ops, runners, dev, sh)
        result["extras"]["torch_reference_decode"] = torch_reference_extras(torch, runners, dev, sh, bound)
        result["extras"]["decode_model"] = model_extras(torch, dev)
    if args.only == "all":
        by_t = prefill_extras(torch, ops, runners, dev, sh)
        result["prefill"] = {"T": 1024, **by_t["1024"], "by_T": by_t}
        result["prefill_tflops"] = by_t["1024"]["tflops"]

    if not args.no_traffic and args.only == "all" and live == 1024:
        tr = measure_traffic(DECODE_KERNEL)
        result["roofline"]["traffic"] = tr.get("bytes")
        result["roofline"]["traffic_detail"] = tr

    if not args.no_cpu and args.only in ("all", "cpu"):
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds, live)

    print(json.dumps(result), flush=True)
    return 0


def time_decode_kernel(torch, ops, runners, bound, ns, sh, dev, reps=3, pos=None) -> float:
    """Mean time (us) of one solort_decode_layer call (its split-KV kernel plus its combine kernel),
    from HIP events around replays of a graph holding one call per layer of every KV set, so each
    call reads a distinct KV slice from HBM.  Each call rewrites the new token's K/V row with the same
    bits."""
    stream = torch.cuda.current_stream(dev)
    ws = ops.attn_workspace(1, sh.nh, sh.nkv, ns, dev)
    out = torch.empty(1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
    order = [(r, li) for r in runners for li in range(sh.layers)]
    cs = {id(r): ops.rope_rows(r.inv_freq, r.pos_buf if pos is None else pos, 1) for r in runners}

    def run_all():
        for r, li in order:
            ops.decode_layer(r.qkv_dec[li], r.qn_w[li], r.kn_w[li], r.eps, cs[id(r)],
                             r.pos_buf if pos is None else pos, r.kc[li], r.vc[li], bound, sh.scale, ws, ns, out,
                             sh.nh, sh.nkv)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_all()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(order))


def extras(torch, ops, wl, runners, dev, sh) -> dict:
    """Decode attention call times per bucket (same rotation), with the split combine in the same
    launch (the default where the placement check passed) and as a second launch; and a split-count
    sweep at KV 1024."""
    from solort_amd import _lib
    from solort_amd.runner import decode_splits

    lib = _lib.load()
    default_mode = lib.solort_combine_mode(-1)
    out: dict = {"decode_call_us": {}, "n_split_sweep_kv1024": {}, "in_launch_merge": default_mode == 1}
    for live in (128, 256, 512, 1024):
        ns = decode_splits(live, sh.nkv)
        pos = torch.tensor([live - 1], dtype=torch.long, device=dev)
        us = time_decode_kernel(torch, ops, runners, live, ns, sh, dev, reps=3, pos=pos)
        lib.solort_combine_mode(0)
        us2 = time_decode_kernel(torch, ops, runners, live, ns, sh, dev, reps=3, pos=pos)
        lib.solort_combine_mode(1)
        gbs = decode_bytes(live) / (us * 1e-6) / 1e9
        out["decode_call_us"][str(live)] = {"us": round(us, 3), "gbps": round(gbs, 1),
                                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "n_split": ns,
                                            "two_launch_us": round(us2, 3)}
    pos = torch.tensor([1023], dtype=torch.long, device=dev)
    for ns in (8, 16, 32, 64, 128):
        us = time_decode_kernel(torch, ops, runners, 1024, ns, sh, dev, reps=3, pos=pos)
        out["n_split_sweep_kv1024"][str(ns)] = round(us, 3)
    lib.solort_combine_mode(default_mode)
    return out


def floor_extras(torch, ops, runners, dev, sh) -> dict:
    """The launch and streaming floor a decode-attention call at KV 1024 is compared with, measured
    the way the call is (HIP events around replays of one graph holding 288 launches):
      empty_node_us      an empty kernel (1 workgroup) per graph node
      read_4mib_us       one launch streaming 4 MiB (the call's K and V bytes) with the call's 256
                         workgroups, one 16-byte load in flight per thread; and with 512 workgroups
                         x 2 loads in flight (the best shape found); *_nt_us: both with
                         the non-temporal hint
      read_4mib_then_32wg_us  the same read followed by a dependent 32-workgroup launch reading
                         512 KiB (the two-launch combine's shape)
      read_4mib_by_workgroups  the 4 MiB read by 8..256 workgroups: the streaming rate per
                         workgroup (one workgroup per KV head would be 8)
      empty_after_predecessor_us  an empty kernel's cost after a ~3 us and after a ~12 us read
    Sources rotate over 144 distinct 4 MiB slices of the rotated KV caches (576 MiB, beyond the 256
    MB Infinity Cache), as the decode calls do."""
    from solort_amd import _lib

    lib = _lib.load()
    slices = []
    for r in runners:
        flat = r.kc.view(-1)
        n4 = flat.numel() * 2 // (4 << 20)
        slices += [flat[i * (2 << 20):(i + 1) * (2 << 20)] for i in range(n4)]
    slices = slices[:288]
    sink = torch.zeros(1024, dtype=torch.int32, device=dev)
    small = torch.zeros(512 << 10, dtype=torch.uint8, device=dev)

    def empty(n_wg=1):  # on the current stream: the capture stream inside a graph capture
        _lib.check(lib.solort_probe_empty(n_wg, torch.cuda.current_stream(dev).cuda_stream), "probe_empty")

    def read(src_ptr, nbytes, n_wg, inflight):
        _lib.check(lib.solort_probe_read(src_ptr, nbytes, n_wg, inflight, sink.data_ptr(),
                                         torch.cuda.current_stream(dev).cuda_stream), "probe_read")

    res = {"empty_node_us": round(_graph_us(torch, dev, [empty] * 288, reps=4), 3)}
    res["read_4mib_us"] = round(_graph_us(
        torch, dev, [lambda x=x: read(x.data_ptr(), 4 << 20, 256, 1) for x in slices], reps=4), 3)
    res["read_4mib_512wg_x2_us"] = round(_graph_us(
        torch, dev, [lambda x=x: read(x.data_ptr(), 4 << 20, 512, 2) for x in slices], reps=4), 3)
    # the same two shapes with the non-temporal hint the decode K/V loads carry
    res["read_4mib_nt_us"] = round(_graph_us(
        torch, dev, [lambda x=x: read(x.data_ptr(), 4 << 20, 256, 1 | 16) for x in slices], reps=4), 3)
    res["read_4mib_512wg_x2_nt_us"] = round(_graph_us(
        torch, dev, [lambda x=x: read(x.data_ptr(), 4 << 20, 512, 2 | 16) for x in slices], reps=4), 3)
    res["read_4mib_then_32wg_us"] = round(_graph_us(
        torch, dev, [lambda x=x: (read(x.data_ptr(), 4 << 20, 256, 1), read(small.data_ptr(), 512 << 10, 32, 4))
                     for x in slices], reps=4), 3)
    res["slices"] = len(slices)
    # Streaming rate of few workgroups: 4 MiB read by n_wg workgroups (4 non-temporal loads in
    # flight per thread), GB/s in all and per workgroup; one workgroup per KV head would be 8.
    per_wg = {}
    for n_wg in (8, 32, 64, 128, 256):
        us = _graph_us(torch, dev, [lambda x=x, n=n_wg: read(x.data_ptr(), 4 << 20, n, 4 | 16) for x in slices[:72]],
                       reps=2)
        per_wg[str(n_wg)] = {"us": round(us, 3), "gbps": round((4 << 20) / (us * 1e-6) / 1e9, 1),
                             "gbps_per_wg": round((4 << 20) / (us * 1e-6) / 1e9 / n_wg, 2)}
    res["read_4mib_by_workgroups"] = per_wg
    # The cost of a one-workgroup empty kernel after a short (4 MiB read, ~3 us) and after a long
    # (64 MiB read, ~12 us) predecessor: each pair's time minus the predecessor's time alone.
    big = [r.kc.view(-1)[:32 << 20] for r in runners]
    t_short = _graph_us(torch, dev, [lambda x=x: read(x.data_ptr(), 4 << 20, 512, 4 | 16) for x in slices[:64]],
                        reps=4)
    t_short_e = _graph_us(torch, dev, [lambda x=x: (read(x.data_ptr(), 4 << 20, 512, 4 | 16), empty())
                                       for x in slices[:64]], reps=4)
    t_long = _graph_us(torch, dev, [lambda x=x: read(x.data_ptr(), 64 << 20, 512, 4 | 16) for x in big * 4], reps=4)
    t_long_e = _graph_us(torch, dev, [lambda x=x: (read(x.data_ptr(), 64 << 20, 512, 4 | 16), empty())
                                      for x in big * 4], reps=4)
    res["empty_after_predecessor_us"] = {
        "short_read_us": round(t_short, 3), "after_short": round(t_short_e - t_short, 3),
        "long_read_us": round(t_long, 3), "after_long": round(t_long_e - t_long, 3),
        "penalty": round((t_long_e - t_long) - (t_short_e - t_short), 3)}
    return res


STAMP_PHASES_DECODE = {0: "start", 1: "position read", 2: "q ready", 3: "key loop done", 4: "partial stored",
                       5: "end", 6: "merge poll started", 7: "merge poll done"}
STAMP_PHASES_PREFILL = {0: "start", 3: "key loop done", 5: "end"}
STAMP_PHASES_QKV = {0: "start", 8: "qkv outputs stored", 9: "qkv rows polled", 2: "q ready", 3: "key loop done",
                    4: "partial stored", 6: "merge poll started", 7: "merge poll done", 5: "end"}


def _stamp_summary(np, st, phases, groups=None) -> dict:
    """Per phase: min / median / p90 / max in microseconds after the launch's first workgroup start
    (100 MHz ticks), over the workgroups that reached it; optional per-group medians of one phase."""
    st = st.astype(np.int64)
    t0 = st[:, 0].min()
    out = {}
    for i, name in phases.items():
        v = st[:, i]
        v = (v[(v >= t0) & (v < t0 + 10_000_000)] - t0) / 100.0  # this launch's stamps only
        if v.size:
            out[name] = {"min": round(float(v.min()), 2), "median": round(float(np.median(v)), 2),
                         "p90": round(float(np.percentile(v, 90)), 2), "max": round(float(v.max()), 2),
                         "workgroups": int(v.size)}
    if groups is not None:
        name, idx, col = groups
        out[name] = [round(float(np.median((st[g, col] - t0) / 100.0)), 2) for g in idx]
    return out


def _wave_stamps(np, st, heads) -> dict:
    """Per-wavefront phases of the MFMA split kernel (slots 8 + w: key loop done by wavefront w,
    12 + w: the loads of its last key tile issued), microseconds after the launch's first start:
    percentiles over every wavefront, the spread of loop ends inside each workgroup, and per KV head
    the last wavefront's loop end and the last workgroup's end."""
    st = st.astype(np.int64)
    t0 = st[:, 0].min()
    us = (st - t0) / 100.0
    ok = (st >= t0) & (st < t0 + 10_000_000)

    def pct(v):
        v = v[np.isfinite(v)]
        return {"min": round(float(v.min()), 2), "median": round(float(np.median(v)), 2),
                "p90": round(float(np.percentile(v, 90)), 2), "max": round(float(v.max()), 2)} if v.size else {}

    done = np.where(ok[:, 8:12], us[:, 8:12], np.nan)
    issued = np.where(ok[:, 12:16], us[:, 12:16], np.nan)
    end = np.where(ok[:, 5], us[:, 5], np.nan)
    return {"wave key loop done": pct(done.ravel()),
            "wave last tile issued": pct(issued.ravel()),
            "wave loop-end spread in a workgroup": pct(np.nanmax(done, 1) - np.nanmin(done, 1)),
            "last wave loop done per KV head": [round(float(np.nanmax(done[h])), 2) for h in heads],
            "last end per KV head": [round(float(np.nanmax(end[h])), 2) for h in heads]}


def stamp_extras(torch, ops, wl, runners, dev, sh, bound) -> dict:
    """In-kernel phase timelines from the tracing build (include/solort_trace.h): the last
    solort_decode_layer launch of a replayed Qwen3-4B decode step at KV 1024, the last call of a
    graph of 8 Qwen3-8B calls at KV 32768 (32 splits), the last of 4 verify calls (5 tokens at 2048,
    the 17 of its 20 splits that hold keys), the last prefill_kernel launch of a graph at T = 1024
    and the last decode_qkv_lanes_kernel launch (qkv product in the decode launch) of a 36-layer graph
    at KV 1024."""
    import numpy as np

    from solort_amd import _lib
    from solort_amd.runner import DECODE_BUCKETS, decode_splits, verify_bound, verify_splits

    lib = _lib.load()
    res = {"clock": "s_memrealtime, 100 MHz; microseconds after the launch's first workgroup started"}

    def read(fn, nb):
        h = np.zeros(nb * 16, dtype=np.uint64)
        _lib.check(getattr(lib, fn)(h.ctypes.data, nb), fn)
        return h.reshape(nb, 16)

    # Qwen3-4B decode at KV 1024: the step graph's last layer call
    for i in range(4):
        runners[i % len(runners)]._graphs[bound].replay()
    torch.cuda.synchronize()
    ns = decode_splits(bound, sh.nkv)
    st = read("solort_phase_stamps_decode", sh.nkv * ns)
    res["decode_qwen3_4b_kv1024"] = _stamp_summary(np, st, STAMP_PHASES_DECODE)
    # Qwen3-8B at KV 32768, 32 splits: per-KV-head (one XCD each) median key-loop end
    s8 = wl.QWEN3_8B
    L, pos, nc = 32768, 32767, 8
    gen = torch.Generator(device=dev).manual_seed(1003)
    kcs = [torch.randn(L, s8.nkv, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(nc)]
    vcs = [torch.randn(L, s8.nkv, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(nc)]
    qkv = torch.randn(nc, 1, s8.qkv_width, generator=gen, device=dev).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(2, 128, generator=gen, device=dev)).to(torch.bfloat16)
    posb = torch.tensor([pos], dtype=torch.long, device=dev)
    cs = ops.rope_rows(ops.inv_freq(128, wl.THETA, dev), posb, 1)
    out = torch.empty(1, s8.nh * 128, dtype=torch.bfloat16, device=dev)
    ws = ops.attn_workspace(1, s8.nh, s8.nkv, 32, dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(nc):
            ops.decode_layer(qkv[i], w[0], w[1], wl.EPS, cs, posb, kcs[i], vcs[i], L, s8.scale, ws, 32, out, s8.nh,
                             s8.nkv)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    st = read("solort_phase_stamps_decode", s8.nkv * 32)
    heads = [[kvh + s8.nkv * sp for sp in range(32)] for kvh in range(s8.nkv)]
    res["decode_qwen3_8b_kv32768"] = _stamp_summary(np, st, STAMP_PHASES_DECODE,
                                                    ("key loop done, median per KV head", heads, 3))
    res["decode_qwen3_8b_kv32768"].update(_wave_stamps(np, st, heads))
    del kcs, vcs
    torch.cuda.empty_cache()
    # speculative verify, 5 tokens at 2048 over a max-4096 cache (the runner's verify bound 2560, 20
    # splits, the combine in a second launch): the split kernel's phases
    pos0, K1, vb = 2048, 5, 4096
    kc = torch.randn(vb, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(vb, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16)
    qv = torch.randn(K1, sh.qkv_width, generator=gen, device=dev).to(torch.bfloat16)
    pv = torch.tensor([pos0], dtype=torch.long, device=dev)
    csv = ops.rope_rows(runners[0].inv_freq, pv, K1)
    vbound = verify_bound(pos0 + K1 - 1, sorted({b for b in DECODE_BUCKETS if b < vb} | {vb}))  # 2560
    nsv = verify_splits(vbound, sh.nkv)  # 20 splits of 128 keys
    wsv = ops.attn_workspace(K1, sh.nh, sh.nkv, nsv, dev)
    ov = torch.empty(K1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for li in range(4):
            ops.decode_layer(qv, runners[0].qn_w[li], runners[0].kn_w[li], runners[0].eps, csv, pv, kc, vc, vbound,
                             sh.scale, wsv, nsv, ov, sh.nh, sh.nkv)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    st = read("solort_phase_stamps_decode", sh.nkv * nsv)
    live = [kvh + sh.nkv * sp for sp in range(17) for kvh in range(sh.nkv)]  # splits holding keys 0..2052
    res["verify_qwen3_4b_5_tokens"] = _stamp_summary(np, st[live], STAMP_PHASES_DECODE)
    del kc, vc
    # prefill attention at T = 1024 over the first runner's cache
    T = 1024
    r = runners[0]
    q = torch.randn(T, sh.nh, 128, generator=gen, device=dev).to(torch.bfloat16)
    o = torch.empty(T, sh.nh * 128, dtype=torch.bfloat16, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for li in range(4):
            ops.prefill_attn(q, r.kc[li], r.vc[li], sh.scale, o)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    n_tiles = T // 16  # 16 positions x 4 query heads per block
    nb = n_tiles * sh.nkv
    st_pre = read("solort_phase_stamps_prefill", nb)
    # block index of a tile by rank (0 = heaviest): the first round of blocks (one per CU) takes
    # ranks in order, the second round from the lightest up
    rnd = max(1, torch.cuda.get_device_properties(dev).multi_processor_count // sh.nkv)
    ib = [rk if rk < rnd else rnd + (n_tiles - 1 - rk) for rk in range(n_tiles)]
    tiles = [[kvh + sh.nkv * ib[rk] for kvh in range(sh.nkv)] for rk in range(n_tiles)]  # heaviest tile first
    # the qkv product inside the decode launch: the last of 36 layers (distinct weights) at KV 1024
    nl, hidden, width = 36, 2560, sh.qkv_width
    wq = [(torch.randn(width, hidden, generator=gen, device=dev) * hidden ** -0.5).to(torch.bfloat16)
          for _ in range(nl)]
    in_w = (1.0 + 0.1 * torch.randn(hidden, generator=gen, device=dev)).to(torch.bfloat16)
    xs = torch.randn(nl, hidden, generator=gen, device=dev).to(torch.bfloat16)
    pq = torch.tensor([1000], dtype=torch.long, device=dev)
    csq = ops.rope_rows(r.inv_freq, pq, 1)
    wsq = ops.decode_qkv_workspace(sh.nh, sh.nkv, 32, dev)
    oq = torch.empty(nl, 1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
    qkv = torch.empty(width, dtype=torch.bfloat16, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for li in range(nl):
            ops.decode_qkv_layer(xs[li], in_w, wl.EPS, wq[li], r.qn_w[li], r.kn_w[li], r.eps, csq, pq, r.kc[li],
                                 r.vc[li], 1024, sh.scale, wsq, 32, qkv, oq[li], sh.nh, sh.nkv)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    st = read("solort_phase_stamps_decode", sh.nkv * 32)
    res["decode_qkv_layer_qwen3_4b_kv1024"] = _stamp_summary(np, st, STAMP_PHASES_QKV)
    del wq
    torch.cuda.empty_cache()
    res["prefill_qwen3_4b_t1024"] = _stamp_summary(np, st_pre, STAMP_PHASES_PREFILL,
                                                   ("end, median per query tile (heaviest first)", tiles, 5))
    return res


def measure_traffic(kernel: str, timeout_s: int = 120) -> dict:
    """HBM bytes per launch of `kernel`, measured in this run: two rocprofv3 --pmc passes (FETCH_SIZE,
    then WRITE_SIZE) over `bench.py --only decode`, each counter scaled by what it reads for the
    64 MiB device copy that run issues (CALIB_BYTES read and written).  Returns the bytes and the
    raw figures, or the reason they are missing."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return {"bytes": None, "reason": "rocprofv3 not found"}
    here = os.path.dirname(os.path.abspath(__file__))
    env = {**os.environ, "TMPDIR": "/tmp"}
    out = {"kernel": kernel, "calibration": "64 MiB device copy"}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix=f"solort_pmc_{counter.lower()}_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "p", "--",
               sys.executable, os.path.join(here, "bench.py"), "--only", "decode", "--steps", "10", "--warmup", "2",
               "--no-cpu", "--no-traffic"]
        try:
            subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                           timeout=timeout_s)
        except subprocess.TimeoutExpired:
            return {"bytes": None, "reason": f"rocprofv3 --pmc {counter} timed out"}
        files = [os.path.join(r, f) for r, _, fs in os.walk(d) for f in fs if f.endswith("counter_collection.csv")]
        if not files:
            return {"bytes": None, "reason": f"no counter output for {counter}"}
        vals, calib = [], []
        with open(files[0], newline="") as f:
            rows = sorted((r for r in csv.DictReader(f) if r["Counter_Name"] == counter),
                          key=lambda r: int(r["Dispatch_Id"]))
        for row in rows:
            name, v = row["Kernel_Name"], float(row["Counter_Value"])
            if kernel in name:
                vals.append(v)
            elif "copyBuffer" in name:
                calib.append(v)
        shutil.rmtree(d, ignore_errors=True)
        if not vals or not calib:
            return {"bytes": None, "reason": f"{counter}: kernel or calibration copy not found in the profile"}
        kib = statistics.mean(vals)
        factor = (CALIB_BYTES / 1024) / calib[-1]  # the run's last device copy is the calibration copy
        out[counter] = {"kib_raw": round(kib, 1), "dispatches": len(vals), "calib_kib_raw": calib[-1],
                        "factor": round(factor, 4), "bytes": int(kib * factor * 1024)}
    out["bytes"] = out["FETCH_SIZE"]["bytes"] + out["WRITE_SIZE"]["bytes"]
    return out


def _graph_us(torch, dev, calls, reps=3) -> float:
    """Mean time (us) per call of `calls` (a list of closures, each one launch sequence), from HIP
    events around replays of one graph that holds them all."""
    stream = torch.cuda.current_stream(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in calls:
            c()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(calls))


def gemv_extras(torch, ops, dev, copies: int = 4) -> dict:
    """Qwen3-4B decode-step GEMVs (one token) with their fused neighbours (RMSNorm before qkv, gate_up
    and lm_head; residual add after o_proj and down; SwiGLU after gate_up), next to torch's F.linear
    (hipBLASLt) on the same weights without the neighbours.  Each is timed in a graph over `copies`
    weight sets (2 for the 778 MB lm_head; 808 MB in all for the layer GEMVs, more than the 256 MB
    Infinity Cache), four calls per set, HIP events around replays.  Bytes = the weight matrix."""
    import functools
    F = torch.nn.functional
    gen = torch.Generator(device=dev).manual_seed(1005)
    K, I = 2560, 9728
    shapes = {"qkv": (6144, K, "norm"), "o_proj": (K, 4096, "resid"), "gate_up": (2 * I, K, "swiglu"),
              "down": (K, I, "resid"), "lm_head": (151936, K, "norm")}
    out = {}
    for name, (rows, k, kind) in shapes.items():
        nset = 2 if name == "lm_head" else copies
        ws = [(torch.randn(rows, k, generator=gen, device=dev) * 0.02).to(torch.bfloat16) for _ in range(nset)]
        x = torch.randn(k, generator=gen, device=dev).to(torch.bfloat16)
        nw = (torch.randn(k, generator=gen, device=dev) * 0.1 + 1).to(torch.bfloat16)
        n = I if kind == "swiglu" else rows
        y = torch.zeros(n, dtype=torch.bfloat16, device=dev)

        def call(w, kind=kind, x=x, nw=nw, y=y):
            if kind == "norm":
                ops.gemv(w, x, y, nw, 1e-6)
            elif kind == "resid":
                ops.gemv(w, x, y, res=y, mode=ops.GEMV_RESID)
            else:
                ops.gemv(w, x, y, nw, 1e-6, mode=ops.GEMV_SWIGLU, inter=I)

        xm = x.view(1, k)
        F.linear(xm, ws[0])  # the BLAS initialises outside the capture
        torch.cuda.synchronize()
        us = _graph_us(torch, dev, [functools.partial(call, w) for w in ws] * 4)
        tus = _graph_us(torch, dev, [functools.partial(F.linear, xm, w) for w in ws] * 4)
        nbytes = rows * k * 2
        out[name] = {"us": round(us, 3), "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "torch_linear_us": round(tus, 3), "bytes": nbytes, "fused": kind}
        if name == "lm_head":  # the lm_head fused with the greedy argmax against the two launches
            aws = ops.argmax_workspace(1, dev)
            gws = ops.gemv_argmax_workspace(rows, dev)
            idx = torch.zeros(1, dtype=torch.long, device=dev)
            fused = _graph_us(torch, dev, [functools.partial(ops.gemv_argmax, w, x, idx, gws, nw, 1e-6, y)
                                           for w in ws] * 4)
            apart = _graph_us(torch, dev, [c for w in ws for c in (functools.partial(call, w),
                                           functools.partial(ops.argmax_rows, y.view(1, -1), idx, aws))] * 4) * 2
            out["lm_head_argmax"] = {"us": round(fused, 3), "two_launch_us": round(apart, 3),
                                     "gbps": round(nbytes / (fused * 1e-6) / 1e9, 1),
                                     "frac_hbm": round(nbytes / (fused * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del ws
        torch.cuda.empty_cache()
    layer = sum(out[n]["us"] for n in ("qkv", "o_proj", "gate_up", "down"))
    out["layer_gemv_us"] = round(layer, 3)
    out["layer_torch_linear_us"] = round(sum(out[n]["torch_linear_us"] for n in ("qkv", "o_proj", "gate_up", "down")), 3)
    return out


def paged_extras(torch, ops, runners, dev, sh, page_size: int = 16, bound: int = 1024) -> dict:
    """Paged-KV decode at KV 1024: each runner layer's cache rows copied into a paged arena
    [pages, 2, page_size, 8, 128] (the reference PagedKVCache layout) at a random block table (64 live
    pages + 8 spare per layer, 1.36 GB in all), one solort_paged_decode_layer call per layer of every
    set in one graph, HIP events around replays; next to the contiguous call of the same graph shape."""
    from solort_amd.runner import decode_splits
    ns = decode_splits(bound, sh.nkv)
    n_log = bound // page_size
    gen = torch.Generator().manual_seed(1013)
    arenas = []
    for r in runners:
        per = []
        for li in range(sh.layers):
            table = torch.randperm(n_log + 8, generator=gen)[:n_log].to(torch.int32)
            slots = torch.arange(bound)
            pg = table.long()[slots // page_size]
            kv = torch.empty(n_log + 8, 2, page_size, sh.nkv, 128, dtype=torch.bfloat16, device=dev)
            kv[pg.to(dev), 0, (slots % page_size).to(dev)] = r.kc[li, :bound]
            kv[pg.to(dev), 1, (slots % page_size).to(dev)] = r.vc[li, :bound]
            per.append((kv, table.to(dev)))
        arenas.append(per)
    ws = ops.attn_workspace(1, sh.nh, sh.nkv, ns, dev)
    out = torch.empty(1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
    calls = []
    for r, per in zip(runners, arenas):
        cs = ops.rope_rows(r.inv_freq, r.pos_buf, 1)
        for li, (kv, table) in enumerate(per):
            calls.append(lambda r=r, li=li, kv=kv, table=table, cs=cs: ops.paged_decode_layer(
                r.qkv_dec[li], r.qn_w[li], r.kn_w[li], r.eps, cs, r.pos_buf, kv, table, bound, sh.scale, ws, ns, out,
                sh.nh, sh.nkv))
    us = _graph_us(torch, dev, calls, reps=4)
    contiguous = time_decode_kernel(torch, ops, runners, bound, ns, sh, dev, reps=4)
    del arenas
    torch.cuda.empty_cache()
    nbytes = decode_bytes(bound)
    return {"page_size": page_size, "bound": bound, "n_split": ns, "us": round(us, 3),
            "gbps": round(nbytes / (us * 1e-6) / 1e9, 1), "contiguous_us": round(contiguous, 3)}


def model_extras(torch, dev, live: int = 960, n: int = 48) -> dict:
    """Whole-model greedy decode of a random-weight Qwen3-4B (36 layers, tied 151,936 x 2560
    embedding, 8.05 GB of bf16 weights): one graph replay per token, tokens `live`..`live`+n-1 in the
    KV 1024 bucket over a seeded N(0,1) context, HIP events around n back-to-back replays, for the
    model's step (each layer's qkv product inside the attention launch, the argmax in the lm_head
    launch, one advance launch), the same step with the qkv product as its own launch
    (`qkv_own_launch`) and the separate-ops tail.  Bytes per token = every weight matrix once (the
    layer GEMVs and the lm_head) plus the K/V rows read."""
    from solort_amd.model import QWEN3_4B, GraphQwen3Decode, RandomQwen3
    s = QWEN3_4B
    w = RandomQwen3(s, dev, seed=1011)
    gen = torch.Generator(device=dev).manual_seed(1012)
    ctx_k = torch.randn(s.layers, live, s.nkv, 128, generator=gen, device=dev).to(torch.bfloat16)
    ctx_v = torch.randn(s.layers, live, s.nkv, 128, generator=gen, device=dev).to(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)
    wbytes = 2 * (s.layers * s.hidden * (s.qkv_width + s.nh * 128 + 3 * s.inter) + s.vocab * s.hidden)
    kvbytes = s.layers * 2 * (live + n // 2) * s.nkv * 128 * 2
    out = {"model": s.name, "live_start": live, "tokens": n, "bytes_per_token": wbytes + kvbytes}
    # the model's path; the same with the qkv product as its own launch; the reference's separate tail ops
    for fused, fused_qkv in ((True, True), (True, False), (False, False)):
        m = GraphQwen3Decode(w, 1024, fused_tail=fused, fused_qkv=fused_qkv)
        m.kc[:, :live].copy_(ctx_k)
        m.vc[:, :live].copy_(ctx_v)
        m.generate(11, live, n)  # captures the bucket's graph and warms every kernel
        g = m.graph(1024)
        ms = []
        for _ in range(3):
            m.start(11, live)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(n):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1) / n)
        ms = min(ms)
        r = {"tokens_per_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4),
             "gbps": round((wbytes + kvbytes) / (ms * 1e-3) / 1e9, 1),
             "frac_hbm": round((wbytes + kvbytes) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
             "first_tokens": m.tokens[:8].tolist()}
        if fused and not fused_qkv:
            out["qkv_own_launch"] = r
        elif fused:
            # the attention's cost inside the step: the same step captured without the attention
            # call of each layer (its tokens are not the model's), timed the same way
            m.attention_in_step = False
            g0 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g0):
                m._step(1024)
            ms0 = []
            for _ in range(3):
                m.start(11, live)
                torch.cuda.synchronize()
                e0.record(stream)
                for _ in range(n):
                    g0.replay()
                e1.record(stream)
                torch.cuda.synchronize()
                ms0.append(e0.elapsed_time(e1) / n)
            m.attention_in_step = True
            del g0
            r["attention_in_step_us_per_layer"] = round((ms - min(ms0)) * 1e3 / s.layers, 3)
            r["step_without_attention_ms"] = round(min(ms0), 4)
            # time to first token: a prompt's prefill graph plus the last row's lm_head and argmax
            ttft = {}
            for plen in (128, 1024):
                ids = torch.randint(0, s.vocab, (plen,), generator=torch.Generator().manual_seed(plen)).tolist()
                m.prefill(ids)  # captures the bucket's graph
                reps = []
                for _ in range(3):
                    torch.cuda.synchronize()
                    e0.record(stream)
                    m.prefill(ids)
                    e1.record(stream)
                    torch.cuda.synchronize()
                    reps.append(e0.elapsed_time(e1))
                ttft[str(plen)] = {"ms": round(min(reps), 3), "tokens_per_s": round(plen / min(reps) * 1e3, 1)}
            r["prefill_ttft"] = ttft
            out.update(r)
        else:
            out["separate_tail"] = r
        del m, g
        torch.cuda.empty_cache()
    kc = torch.zeros(s.layers, 1024, s.nkv, 128, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    kc[:, :live].copy_(ctx_k)
    vc[:, :live].copy_(ctx_v)
    ref_ms = torch_reference_model_ms(torch, w, kc, vc, live, n)
    out["torch_reference"] = {"ms_per_token": round(ref_ms, 4), "tokens_per_s": round(1e3 / ref_ms, 1),
                              "note": "the reference's decode step as torch ops on this GPU, graphed; K^T and V "
                                      "made contiguous for the batched attention products"}
    return out


def long_decode_extras(torch, ops, wl, dev, n_caches: int = 8) -> dict:
    """Qwen3-8B-shape decode at KV 32768 (32 q / 8 kv heads, bucket 32768): one solort_decode_layer
    call per distinct 134 MB layer cache, n_caches caches (1.07 GB) rotated, for several split
    counts.  Algorithmic bytes: K and V rows 0..32767 plus q and the output."""
    sh = wl.QWEN3_8B
    L, pos = 32768, 32767
    gen = torch.Generator(device=dev).manual_seed(1003)
    kcs = [torch.randn(L, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(n_caches)]
    vcs = [torch.randn(L, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(n_caches)]
    qkv = torch.randn(n_caches, 1, sh.qkv_width, generator=gen, device=dev).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(2, 128, generator=gen, device=dev)).to(torch.bfloat16)
    posb = torch.tensor([pos], dtype=torch.long, device=dev)
    inv = ops.inv_freq(128, wl.THETA, dev)
    cs = ops.rope_rows(inv, posb, 1)
    out = torch.empty(1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
    kbytes = decode_bytes(L, sh.nh, sh.nkv)
    res = {"workload": "Qwen3-8B decode attention, batch 1, 32q/8kv heads, KV live 32768 (bucket 32768), "
                       f"{n_caches} rotated layer caches", "algorithmic_bytes": kbytes, "by_n_split": {}}
    best = None
    for ns in (32, 64, 128, 256):
        ws = ops.attn_workspace(1, sh.nh, sh.nkv, ns, dev)
        calls = [(lambda i=i, ws=ws, ns=ns: ops.decode_layer(qkv[i], w[0], w[1], wl.EPS, cs, posb, kcs[i], vcs[i],
                                                             L, sh.scale, ws, ns, out, sh.nh, sh.nkv))
                 for i in range(n_caches)]
        us = _graph_us(torch, dev, calls, reps=4)
        gbs = kbytes / (us * 1e-6) / 1e9
        res["by_n_split"][str(ns)] = {"us": round(us, 3), "gbps": round(gbs, 1),
                                      "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        if best is None or us < best[1]:
            best = (ns, us, gbs)
    res.update({"n_split": best[0], "us": round(best[1], 3), "gbps": round(best[2], 1),
                "frac_hbm": round(best[2] / HBM_PEAK_GBS, 4)})
    # Streaming ceiling for the same traffic: a plain 16-byte streaming-read kernel (grid-stride,
    # 2 or 4 loads in flight per thread, with and without the non-temporal hint the decode K/V
    # loads carry) over the same 16 rotating 67 MB K and V buffers, one launch per buffer, in one
    # graph; the best shape's GB/s, launches included.
    from solort_amd import _lib
    lib = _lib.load()
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    bufs = [t for pair in zip(kcs, vcs) for t in pair]
    nbytes = bufs[0].numel() * 2
    ceil = {}
    for n_wg in (512, 1024, 2048):
        for inflight in (2, 4):
            for nt in (0, 16):
                def rd(x, n_wg=n_wg, inflight=inflight | nt):
                    _lib.check(lib.solort_probe_read(x.data_ptr(), nbytes, n_wg, inflight, sink.data_ptr(),
                                                     torch.cuda.current_stream(dev).cuda_stream), "probe_read")
                us = _graph_us(torch, dev, [lambda x=x: rd(x) for x in bufs], reps=4)
                ceil[f"{n_wg}x{inflight}{'nt' if nt else ''}"] = round(nbytes / (us * 1e-6) / 1e9, 1)
    top = max(ceil, key=ceil.get)
    res["stream_ceiling"] = {"gbps": ceil[top], "frac_hbm": round(ceil[top] / HBM_PEAK_GBS, 4), "shape": top,
                             "by_shape_gbps": ceil, "bytes_per_launch": nbytes,
                             "note": "streaming read of the same rotated K/V buffers (nt: non-temporal loads)"}
    res["frac_of_stream_ceiling"] = round(best[2] / ceil[top], 4)
    # The decode's own K/V reads without arithmetic (solort_probe_read_heads: the same grid of 8 x 32
    # workgroups, 32-row tiles per wavefront, one tile in flight as the decode keeps, or two;
    # non-temporal loads) over the same caches, one launch per cache in one graph: what the call's
    # streaming alone costs.
    heads = torch.zeros(sh.nkv * 32, dtype=torch.int32, device=dev)
    pat = {}
    for d in (1, 2):
        def rh(i, d=d):
            _lib.check(lib.solort_probe_read_heads(kcs[i].data_ptr(), vcs[i].data_ptr(), L, sh.nkv, 32, d,
                                                   heads.data_ptr(), torch.cuda.current_stream(dev).cuda_stream),
                       "probe_read_heads")
        pat[d] = _graph_us(torch, dev, [lambda i=i: rh(i) for i in range(n_caches)], reps=4)
    pgbs = 2 * nbytes / (pat[1] * 1e-6) / 1e9
    res["pattern_ceiling"] = {"us": round(pat[1], 3), "gbps": round(pgbs, 1), "frac_hbm": round(pgbs / HBM_PEAK_GBS, 4),
                              "n_split": 32, "bytes_per_launch": 2 * nbytes,
                              "us_two_tiles_in_flight": round(pat[2], 3),
                              "note": "the decode kernel's K/V loads alone (same grid and tiles, one tile in flight "
                                      "per wavefront; us_two_tiles_in_flight: two)"}
    res["frac_of_pattern_ceiling"] = round(pat[1] / best[1], 4)
    del kcs, vcs
    torch.cuda.empty_cache()
    return res


def qkv_layer_extras(torch, ops, wl, dev, L: int = 36) -> dict:
    """Qwen3-4B decode layer's qkv product and attention block: solort_decode_qkv_layer (the product
    inside the attention launch) against solort_gemv + solort_decode_layer, each as a graph of L
    layers with distinct weights (1.1 GB) and caches, at KV 1024, 2048 and 4096 (32 splits; at 4096
    the MFMA split kernel; longer chunks run as the two launches inside the entry point); us per
    layer.
    The bytes per layer are the wqkv matrix plus the attention's K/V rows."""
    sh = wl.QWEN3_4B
    hidden, width = 2560, sh.qkv_width
    res = {"workload": f"Qwen3-4B decode, {L} layers of distinct weights and caches, one token", "by_kv": {}}
    for bound, pos in ((1024, 1000), (2048, 2000), (4096, 4000)):
        gen = torch.Generator(device=dev).manual_seed(77)
        wq = [(torch.randn(width, hidden, generator=gen, device=dev) * hidden ** -0.5).to(torch.bfloat16)
              for _ in range(L)]
        in_w = (1.0 + 0.1 * torch.randn(hidden, generator=gen, device=dev)).to(torch.bfloat16)
        nw = (1.0 + 0.1 * torch.randn(128, generator=gen, device=dev)).to(torch.bfloat16)
        kc = torch.randn(L, bound, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        vc = torch.randn(L, bound, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        posb = torch.tensor([pos], dtype=torch.long, device=dev)
        cs = ops.rope_rows(ops.inv_freq(128, wl.THETA, dev), posb, 1)
        ws = ops.decode_qkv_workspace(sh.nh, sh.nkv, 32, dev)
        xs = torch.randn(L, hidden, generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty(L, 1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
        qkv = torch.empty(1, width, dtype=torch.bfloat16, device=dev)

        def two_launches():
            for li in range(L):
                ops.gemv(wq[li], xs[li], qkv.view(-1), in_w, wl.EPS)
                ops.decode_layer(qkv, nw, nw, wl.EPS, cs, posb, kc[li], vc[li], bound, sh.scale, ws, 32, out[li],
                                 sh.nh, sh.nkv)

        def one_launch():
            for li in range(L):
                ops.decode_qkv_layer(xs[li], in_w, wl.EPS, wq[li], nw, nw, wl.EPS, cs, posb, kc[li], vc[li], bound,
                                     sh.scale, ws, 32, qkv.view(-1), out[li], sh.nh, sh.nkv)
        us1 = _graph_us(torch, dev, [one_launch], reps=5) / L
        us2 = _graph_us(torch, dev, [two_launches], reps=5) / L
        nbytes = width * hidden * 2 + decode_bytes(pos + 1)
        res["by_kv"][str(bound)] = {"one_launch_us": round(us1, 3), "two_launches_us": round(us2, 3),
                                    "gbps": round(nbytes / (us1 * 1e-6) / 1e9, 1), "bytes": nbytes}
        del wq, kc, vc
        torch.cuda.empty_cache()
    return res


def mid_decode_extras(torch, ops, wl, dev, n_caches: int = 8) -> dict:
    """Qwen3-4B decode call at KV 2048 / 4096 / 8192 / 16384 (bucket = live length), one
    solort_decode_layer call per distinct layer cache, n_caches caches rotated in one graph, for the
    split count the runner routes (decode_splits) and its neighbours (chunks of 32 to 1024 keys)."""
    from solort_amd.runner import decode_splits

    sh = wl.QWEN3_4B
    res = {"workload": "Qwen3-4B decode attention, batch 1, 32q/8kv heads, KV live = bucket, "
                       f"{n_caches} rotated layer caches; us per call by n_split x chunk", "by_kv": {}}
    for L in (2048, 4096, 8192, 16384):
        gen = torch.Generator(device=dev).manual_seed(1004)
        kcs = [torch.randn(L, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(n_caches)]
        vcs = [torch.randn(L, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(n_caches)]
        qkv = torch.randn(n_caches, 1, sh.qkv_width, generator=gen, device=dev).to(torch.bfloat16)
        w = (1.0 + 0.1 * torch.randn(2, 128, generator=gen, device=dev)).to(torch.bfloat16)
        posb = torch.tensor([L - 1], dtype=torch.long, device=dev)
        cs = ops.rope_rows(ops.inv_freq(128, wl.THETA, dev), posb, 1)
        out = torch.empty(1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
        routed = decode_splits(L, sh.nkv)
        # neighbours of the routed count, and the count of the earlier rule (32-key chunks up to 4096
        # keys, 1024-key chunks beyond)
        r = {"routed_n_split": routed, "by_split": {}}
        for ns in sorted({routed, routed // 2, routed * 2, min(256, L // 32) if L <= 4096 else L // 1024} - {0}):
            ws = ops.attn_workspace(1, sh.nh, sh.nkv, ns, dev)
            calls = [(lambda i=i, ws=ws, ns=ns: ops.decode_layer(qkv[i], w[0], w[1], wl.EPS, cs, posb, kcs[i], vcs[i],
                                                                 L, sh.scale, ws, ns, out, sh.nh, sh.nkv))
                     for i in range(n_caches)]
            us = _graph_us(torch, dev, calls, reps=4)
            r["by_split"][f"{ns}x{L // ns}"] = round(us, 3)
        us = r["by_split"][f"{routed}x{L // routed}"]
        gbs = decode_bytes(L) / (us * 1e-6) / 1e9
        r.update({"us": us, "gbps": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
        res["by_kv"][str(L)] = r
        del kcs, vcs
        torch.cuda.empty_cache()
    # speculative verify (5 tokens at the bucket's end) over the same lengths from 8192 on: the routed
    # split count against the earlier rule (64 splits of 128-key multiples)
    from solort_amd.runner import verify_splits
    K1 = 5
    res["verify_by_kv"] = {}
    for L in (8192, 16384, 32768):
        gen = torch.Generator(device=dev).manual_seed(1005)
        nc = 4
        kcs = [torch.randn(L, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(nc)]
        vcs = [torch.randn(L, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(nc)]
        qkv = torch.randn(nc, K1, sh.qkv_width, generator=gen, device=dev).to(torch.bfloat16)
        w = (1.0 + 0.1 * torch.randn(2, 128, generator=gen, device=dev)).to(torch.bfloat16)
        posb = torch.tensor([L - K1], dtype=torch.long, device=dev)
        cs = ops.rope_rows(ops.inv_freq(128, wl.THETA, dev), posb, K1)
        out = torch.empty(K1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
        routed = verify_splits(L, sh.nkv)
        r = {"routed_n_split": routed, "by_split": {}}
        for ns in sorted({routed, 64}):
            ws = ops.attn_workspace(K1, sh.nh, sh.nkv, ns, dev)
            calls = [(lambda i=i, ws=ws, ns=ns: ops.decode_layer(qkv[i], w[0], w[1], wl.EPS, cs, posb, kcs[i], vcs[i],
                                                                 L, sh.scale, ws, ns, out, sh.nh, sh.nkv))
                     for i in range(nc)]
            r["by_split"][f"{ns}x{L // ns}"] = round(_graph_us(torch, dev, calls, reps=4), 3)
        r["us"] = r["by_split"][f"{routed}x{L // routed}"]
        res["verify_by_kv"][str(L)] = r
        del kcs, vcs
        torch.cuda.empty_cache()
    return res


def verify_extras(torch, ops, wl, runners, dev, sh) -> dict:
    """Speculative verify, Qwen3-4B shape: 5 queries at 2048..2052 over the cache (the runner's
    routing: bucket 4096, its verify bound 2560 and split count; also the whole bucket at 32
    splits), one solort_decode_layer call per layer of every KV set; then the greedy argmax of
    [5, 151936] bf16 logits.  Uses fresh max-4096 caches (8 sets x 36 layers rotated)."""
    from solort_amd.runner import DECODE_BUCKETS, verify_bound, verify_splits

    pos0, K1, max_len = 2048, 5, 4096
    buckets = sorted({b for b in DECODE_BUCKETS if b < max_len} | {max_len})
    bucket = next(b for b in buckets if b > pos0 + K1 - 1)
    bound = verify_bound(pos0 + K1 - 1, buckets)
    gen = torch.Generator(device=dev).manual_seed(1004)
    sets = []
    for _ in range(len(runners)):
        kc = torch.randn(sh.layers, max_len, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        vc = torch.randn(sh.layers, max_len, sh.nkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        sets.append((kc, vc))
    qkv = torch.randn(sh.layers, K1, sh.qkv_width, generator=gen, device=dev).to(torch.bfloat16)
    posb = torch.tensor([pos0], dtype=torch.long, device=dev)
    r0 = runners[0]
    cs = ops.rope_rows(r0.inv_freq, posb, K1)
    ns = verify_splits(bound, sh.nkv)
    out = torch.empty(K1, sh.nh * 128, dtype=torch.bfloat16, device=dev)
    vbytes = 2 * sh.nkv * (pos0 + K1) * 128 * 2 + K1 * 2 * sh.nh * 128 * 2

    def time_splits(n, bnd=bound):
        ws = ops.attn_workspace(K1, sh.nh, sh.nkv, n, dev)
        calls = [(lambda kc=kc, vc=vc, li=li: ops.decode_layer(qkv[li], r0.qn_w[li], r0.kn_w[li], r0.eps, cs, posb,
                                                               kc[li], vc[li], bnd, sh.scale, ws, n, out, sh.nh,
                                                               sh.nkv))
                 for kc, vc in sets for li in range(sh.layers)]
        return _graph_us(torch, dev, calls, reps=3)

    us = time_splits(ns)
    sweep = {str(n): round(time_splits(n), 3) for n in (10, 16, 20, 32, 40)}
    bucket_us = time_splits(verify_splits(bucket, sh.nkv), bucket)
    gbs = vbytes / (us * 1e-6) / 1e9
    del sets
    torch.cuda.empty_cache()
    res = {"verify": {"us_per_layer_call": round(us, 3), "gbps": round(gbs, 1),
                      "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "n_split": ns, "bucket": bucket, "bound": bound,
                      "algorithmic_bytes": vbytes, "n_split_sweep": sweep,
                      "whole_bucket": {"us": round(bucket_us, 3), "n_split": verify_splits(bucket, sh.nkv)}}}
    g2 = torch.Generator().manual_seed(1004)
    logits = [wl.planted_logits(g2, K1, wl.VOCAB).to(dev) for _ in range(2)]
    logits += [torch.randn(K1, wl.VOCAB, generator=gen, device=dev).to(torch.bfloat16) for _ in range(6)]
    idx = torch.empty(K1, dtype=torch.long, device=dev)
    aws = ops.argmax_workspace(K1, dev)
    calls = [(lambda x=x: ops.argmax_rows(x, idx, aws)) for x in logits]
    aus = _graph_us(torch, dev, calls, reps=20)
    abytes = K1 * wl.VOCAB * 2
    res["argmax_5x151936_bf16"] = {"us": round(aus, 3), "gbps": round(abytes / (aus * 1e-6) / 1e9, 1),
                                   "algorithmic_bytes": abytes}
    return res


def prefill_extras(torch, ops, runners, dev, sh) -> dict:
    """Prefill attention at T in {128, 512, 1024}: the MFMA kernel alone (solort_prefill_attn on a
    materialised q; graph of one launch per layer of every KV set, HIP events around replays) and
    the graphed prefill step (cos/sin rows, then per layer the K/V prologue and the attention
    normalising q itself, 36 layers) per layer.  Overwrites cache rows 0..T-1 of every set."""
    out = {}
    stream = torch.cuda.current_stream(dev)
    gen = torch.Generator(device=dev).manual_seed(1002)
    for T in (128, 512, 1024):
        for r in runners:
            r.prefill((torch.randn(sh.layers, T, sh.qkv_width, generator=gen, device=dev)).to(torch.bfloat16))
        torch.cuda.synchronize()
        outs = [torch.empty(T, sh.nh * 128, dtype=torch.bfloat16, device=dev) for _ in range(2)]
        # the attention kernel alone reads a materialised q: layer 0's, from the prompt just
        # prefilled (the prologue rewrites the same cache rows with the same values)
        qs = []
        for r in runners:
            q = torch.empty(T, sh.nh, 128, dtype=torch.bfloat16, device=dev)
            cs = ops.rope_rows(r.inv_freq, r.zero_pos, T)
            ops.qknorm_rope_kvwrite_cs(r.qkv_pre[0, :T], r.qn_w[0], r.kn_w[0], r.eps, cs, None, q, r.kc[0], r.vc[0],
                                       sh.nh, sh.nkv)
            qs.append(q)

        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 3

        def kernel_us():
            def run_all():
                for i, r in enumerate(runners):
                    for li in range(sh.layers):
                        ops.prefill_attn(qs[i], r.kc[li], r.vc[li], sh.scale, outs[(i + li) % 2])

            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                run_all()
            graph.replay()
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / (reps * len(runners) * sh.layers)

        kern_us = kernel_us()
        # whole graphed prefill step (prologue + attention per layer)
        e0.record(stream)
        for i in range(reps):
            runners[i % len(runners)]._pre_graphs[T].replay()
        e1.record(stream)
        torch.cuda.synchronize()
        step_us = e0.elapsed_time(e1) * 1e3 / (reps * sh.layers)
        fl = prefill_flops(T, sh.nh)
        tf = fl / (kern_us * 1e-6) / 1e12
        # roofline at this T: min(MFMA peak, arithmetic intensity x HBM peak), with the
        # algorithmic bytes of the attention block (qkv rows in, K/V rows and output out)
        nbytes = prefill_bytes(T, sh.nh, sh.nkv)
        roof = min(BF16_PEAK_TFLOPS, fl / nbytes * HBM_PEAK_GBS / 1e3)
        out[str(T)] = {"kernel_us": round(kern_us, 3), "tflops": round(tf, 2),
                       "frac_mfma_peak": round(tf / BF16_PEAK_TFLOPS, 4),
                       "roofline_tflops": round(roof, 1), "frac_roofline": round(tf / roof, 4),
                       "step_us_per_layer": round(step_us, 3), "flop": fl, "bytes": nbytes}
    # The two prefill forms per prompt length (runner.FUSED_PREFILL_MIN picks between them): the
    # whole K/V + q prologue then attention on the materialised q, against the K/V prologue and
    # attention normalising q itself; graphed 36-layer steps over the first runner's cache, per layer.
    r = runners[0]
    zp = torch.zeros(1, dtype=torch.long, device=dev)
    forms = {}
    for T in (128, 256, 512):
        qkv = torch.randn(sh.layers, T, sh.qkv_width, generator=gen, device=dev).to(torch.bfloat16)
        cs = torch.empty(2, T, 64, dtype=torch.bfloat16, device=dev)
        q = torch.empty(T, sh.nh, 128, dtype=torch.bfloat16, device=dev)
        ctx = torch.empty(sh.layers, T, sh.nh * 128, dtype=torch.bfloat16, device=dev)

        def two_launch(T=T, qkv=qkv, cs=cs, q=q, ctx=ctx):
            ops.rope_rows(r.inv_freq, zp, T, cs)
            for li in range(sh.layers):
                ops.qknorm_rope_kvwrite_cs(qkv[li], r.qn_w[li], r.kn_w[li], r.eps, cs, None, q, r.kc[li], r.vc[li],
                                           sh.nh, sh.nkv)
                ops.prefill_attn(q, r.kc[li], r.vc[li], sh.scale, ctx[li])

        def fused(T=T, qkv=qkv, cs=cs, ctx=ctx):
            ops.rope_rows(r.inv_freq, zp, T, cs)
            for li in range(sh.layers):
                ops.prefill_layer(qkv[li], r.qn_w[li], r.kn_w[li], r.eps, cs, r.kc[li], r.vc[li], sh.scale, ctx[li],
                                  sh.nh, sh.nkv)
        forms[str(T)] = {"two_launch_us_per_layer": round(_graph_us(torch, dev, [two_launch], reps=3) / sh.layers, 3),
                         "fused_us_per_layer": round(_graph_us(torch, dev, [fused], reps=3) / sh.layers, 3)}
    out["forms_by_T"] = forms
    return out


def _ref_rmsnorm(x, w, eps: float = 1e-6):
    """cuda_graph_executor.py:25-28 (torch ops)."""
    xf = x.float()
    return ((xf * xf.square().mean(-1, keepdim=True).add(eps).rsqrt()) * w.float()).to(x.dtype)


def _ref_rope(x, cos, sin):
    """cuda_graph_executor.py:100-102 (torch ops)."""
    import torch
    d = x.shape[-1] // 2
    return x * cos + torch.cat([-x[..., d:], x[..., :d]], -1) * sin


def torch_reference_model_ms(torch, w, kc, vc, live: int, n: int, bound: int = 1024) -> float:
    """The reference's whole greedy decode step (cuda_graph_executor.py:163-206: embedding, per layer
    input norm, QKV product, q/k norm + RoPE, KV write, grouped attention, o_proj, post norm,
    gate/up, SiLU, down; final norm, lm_head, argmax into the token buffer) as torch ops on this GPU,
    graphed as the reference's _capture does, over the given weights and caches.  The batched
    attention products get contiguous K^T and V (batched bf16 products on transposed views are
    unsafe on this device).  Returns ms per token over n replays from position `live`."""
    F = torch.nn.functional
    s = w.shape
    nh, nkv, hd, g = s.nh, s.nkv, 128, s.nh // s.nkv
    dev = kc.device
    tok_buf = torch.tensor([11], dtype=torch.long, device=dev)
    pos_buf = torch.tensor([live], dtype=torch.long, device=dev)
    inv = 1.0 / (1e6 ** (torch.arange(0, hd, 2, device=dev).float() / hd))
    arange = torch.arange(bound, device=dev)

    def step():
        freqs = pos_buf.float().view(-1, 1) * inv.view(1, -1)
        emb = torch.cat([freqs, freqs], -1)
        cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
        x = w.embed[tok_buf]
        nkeep = (arange > pos_buf).view(1, 1, bound)
        for li in range(s.layers):
            qkv = _ref_rmsnorm(x, w.in_ln[li]) @ w.wqkv[li].T
            q, k, v = qkv.split([nh * hd, nkv * hd, nkv * hd], dim=-1)
            q = _ref_rope(_ref_rmsnorm(q.view(1, nh, hd).transpose(0, 1), w.qn[li]), cos, sin)
            k = _ref_rope(_ref_rmsnorm(k.view(1, nkv, hd).transpose(0, 1), w.kn[li]), cos, sin)
            kc[li].index_copy_(0, pos_buf, k.transpose(0, 1))
            vc[li].index_copy_(0, pos_buf, v.view(1, nkv, hd))
            kt = kc[li, :bound].permute(1, 2, 0).contiguous()
            vb = vc[li, :bound].permute(1, 0, 2).contiguous()
            sc = (torch.matmul(q.reshape(nkv, g, hd), kt) * hd ** -0.5).masked_fill(nkeep, float("-inf"))
            ctx = torch.matmul(torch.softmax(sc, -1).to(torch.bfloat16), vb).reshape(1, nh * hd)
            x = x + ctx @ w.wo[li].T
            gate, up = (_ref_rmsnorm(x, w.post_ln[li]) @ w.wgu[li].T).split([s.inter, s.inter], dim=-1)
            x = x + (F.silu(gate) * up) @ w.wd[li].T
        lg = (_ref_rmsnorm(x, w.final_norm) @ w.lm_head.T).float()
        tok_buf.copy_(lg.argmax(-1))
        pos_buf.add_(1)

    for _ in range(2):
        step()  # eager first: the BLAS initialises outside the capture
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    pos_buf.fill_(live)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(n):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def torch_reference_extras(torch, runners, dev, sh, bound: int) -> dict:
    """The reference's own decode-attention ops (cuda_graph_executor.py:164, :168, :173-184) as torch
    kernels on this GPU, for context: per layer the q/k split, two per-head RMSNorms (:25-28), two
    RoPEs (:100-102), the two KV index_copy_ writes, the grouped score matmul, scale, mask, softmax
    and the P V matmul, in bf16.  The transposed K^T and the permuted V views are made contiguous
    before their batched products (batched bf16 products on transposed views are unsafe on this
    device); that adds two copies per layer.  One graph per KV set replays the 36 layers, rotated
    over the sets, HIP events around the replays."""
    nh, nkv, hd, g = sh.nh, sh.nkv, 128, sh.nh // sh.nkv
    scale = 128 ** -0.5
    rmsnorm, rope = _ref_rmsnorm, _ref_rope

    arange = torch.arange(bound, device=dev)
    graphs = []
    for r in runners:
        pos_buf = r.pos_buf
        inv = r.inv_freq

        def step(r=r, pos_buf=pos_buf, inv=inv):
            freqs = pos_buf.float().view(-1, 1) * inv.view(1, -1)                     # :95-98
            emb = torch.cat([freqs, freqs], -1)
            cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
            nkeep = (arange > pos_buf).view(1, 1, bound)                              # :168
            for li in range(sh.layers):
                q, k, v = r.qkv_dec[li].split([nh * hd, nkv * hd, nkv * hd], dim=-1)  # :173-175
                q = q.view(1, nh, hd).transpose(0, 1)
                k = k.view(1, nkv, hd).transpose(0, 1)
                v = v.view(1, nkv, hd).transpose(0, 1)
                q = rope(rmsnorm(q, r.qn_w[li]), cos, sin)                             # :176-177
                k = rope(rmsnorm(k, r.kn_w[li]), cos, sin)
                r.kc[li].index_copy_(0, pos_buf, k.transpose(0, 1))                   # :178-179
                r.vc[li].index_copy_(0, pos_buf, v.transpose(0, 1))
                qg = q.reshape(nkv, g, hd)                                            # :180-184
                kt = r.kc[li, :bound].permute(1, 2, 0).contiguous()
                vb = r.vc[li, :bound].permute(1, 0, 2).contiguous()
                sc = (torch.matmul(qg, kt) * scale).masked_fill(nkeep, float("-inf"))
                torch.matmul(torch.softmax(sc, -1).to(torch.bfloat16), vb).reshape(1, nh * hd)

        for _ in range(2):
            step()  # eager first: the BLAS initialises outside the capture
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        graphs.append(graph)
    stream = torch.cuda.current_stream(dev)
    for gr in graphs:
        gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 3
    e0.record(stream)
    for _ in range(reps):
        for gr in graphs:
            gr.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * len(graphs) * sh.layers)
    return {"us_per_layer": round(us, 3), "bound": bound,
            "note": "reference decode-attention torch ops on this GPU, graphed; K^T and V made contiguous"}


def _median_us(fn, budget_s: float, warm: int = 5, min_runs: int = 20, max_runs: int = 200) -> tuple[float, int]:
    """Median wall time (us) of fn() over at least min_runs timed runs after `warm` untimed ones,
    continuing up to max_runs while the budget lasts (perf_counter_ns around each run)."""
    for _ in range(warm):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) / 1e3)
    return statistics.median(times), len(times)


def cpu_baseline(budget_s: float, live: int) -> dict:
    """The oracle's fp32 torch restatement of the reference path (cuda_graph_executor.py; the
    reference's own method is synchronize + perf_counter over N replays, scripts/microbench_decode.py:
    30-35) on the host cores, per benchmark config, on the same seeded inputs as the GPU workloads:
      config 1  Qwen3-0.6B decode, all 28 layers, 513 keys (bucket 1024), in full
      config 2  Qwen3-4B decode, 36 layers, KV 128 / 256 / 512 / 1024 (`value`: KV `live`)
      config 3  Qwen3-4B prefill T = 512: prologue + KV write + causal attention, 6 of the 36 layers
      config 4  Qwen3-8B decode at KV 32768, 2 of the 36 layers (4.3 GB of fp32 cache per 16 layers)
      config 5  Qwen3-4B verify: 5 tokens at 2048.. over the max-4096 cache, 6 of the 36 layers; and
                the greedy argmax of the [5, 151936] logits
    Each figure is the median of at least 20 runs after 5 warm-ups, per layer where the config has
    layers."""
    import torch

    from oracle import ref
    from solort_amd import workloads as wl

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    per = budget_s / 8
    f32 = torch.float32
    inv = ref.inv_freq(128, wl.THETA)

    def decode_fn(case):
        sh = case.shape
        cos, sin = ref.cos_sin(torch.tensor([case.pos]), inv, f32)
        return lambda: ref.decode_layers(case.qkv, case.qn_w, case.kn_w, wl.EPS, cos, sin, case.kc, case.vc,
                                         case.pos, case.bound, sh.nh, sh.nkv, sh.scale)

    configs: dict = {}
    c1 = wl.decode_case(0, dtype=f32)
    us, n = _median_us(decode_fn(c1), per)
    configs["1"] = {"us_per_layer": round(us / c1.shape.layers, 2), "us_per_step": round(us, 1), "runs": n,
                    "workload": "Qwen3-0.6B decode, 28 layers, 513 keys (bucket 1024), fp32"}
    c2 = {}
    for L in wl.DECODE_LIVE:
        case = wl.decode_case(1, live=L, dtype=f32)
        us, n = _median_us(decode_fn(case), per / 2)
        c2[str(L)] = {"us_per_layer": round(us / case.shape.layers, 2), "runs": n}
        del case
    configs["2"] = {"by_live": c2, "workload": "Qwen3-4B decode, 36 layers, fp32"}

    nl = 6  # layers timed for configs 3 and 5 (each layer is the same work)
    pc = wl.prefill_case(512, layers=nl, dtype=f32)
    sh = pc.shape
    cos, sin = ref.cos_sin(torch.arange(pc.T), inv, f32)
    kc = torch.zeros(nl, pc.max_len, sh.nkv, 128)
    vc = torch.zeros_like(kc)

    def prefill():
        for li in range(nl):
            q, k, v = ref.prologue(pc.qkv[li], pc.qn_w[li], pc.kn_w[li], wl.EPS, cos, sin, sh.nh, sh.nkv)
            ref.write_kv(kc[li], vc[li], k, v, 0)
            ref.prefill_attn(q, k, v, sh.scale)

    us, n = _median_us(prefill, per)
    configs["3"] = {"us_per_layer": round(us / nl, 2), "runs": n,
                    "workload": f"Qwen3-4B prefill T=512: prologue + KV write + causal attention, {nl} layers, fp32"}
    del pc, kc, vc

    c4 = wl.decode_case(3, layers=2, dtype=f32)
    us, n = _median_us(decode_fn(c4), per)
    configs["4"] = {"us_per_layer": round(us / 2, 2), "runs": n,
                    "workload": "Qwen3-8B decode at KV 32768, 2 layers, fp32"}
    del c4

    c5 = wl.decode_case(4, layers=nl, dtype=f32)
    sh = c5.shape
    cos, sin = ref.cos_sin(c5.pos + torch.arange(c5.nq), inv, f32)

    def verify():
        for li in range(nl):
            q, k, v = ref.prologue(c5.qkv[li], c5.qn_w[li], c5.kn_w[li], wl.EPS, cos, sin, sh.nh, sh.nkv)
            ref.write_kv(c5.kc[li], c5.vc[li], k, v, c5.pos)
            ref.verify_attn(q, c5.kc[li], c5.vc[li], c5.pos, sh.scale)

    us, n = _median_us(verify, per)
    logits = c5.logits.float()
    aus, an = _median_us(lambda: ref.argmax(logits), per / 4)
    configs["5"] = {"us_per_layer": round(us / nl, 2), "runs": n, "argmax_us": round(aus, 2),
                    "argmax_runs": an,
                    "workload": f"Qwen3-4B verify, 5 tokens at 2048 over the max-4096 cache, {nl} layers, fp32; "
                                "argmax of [5, 151936] fp32 logits"}
    del c5

    head = c2.get(str(live), c2["1024"])
    return {"value": head["us_per_layer"], "unit": "us/layer", "cores": cores, "kind": "port",
            "sample": f"config 2 (Qwen3-4B decode, 36 layers, KV {live}) in fp32 torch on {cores} threads of "
                      f"'{model}': median of {head['runs']} steps after 5 warm-ups, per layer; the other "
                      "configs under `configs`",
            "cpu_model": model, "configs": configs}


if __name__ == "__main__":
    sys.exit(main())
