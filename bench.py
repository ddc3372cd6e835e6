"""Benchmark of the MLA decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 100] [--warmup 10]

A step is one mla_decode over the measured workload: batch 32, 128 heads,
8192 cached tokens per sequence, bf16, page size 64, shuffled block tables,
inputs ~ N(0, 1) drawn on the CPU with seed 0 and resident in HBM before
timing. Every launch is preceded by a 512 MiB read that evicts the 256 MiB
Infinity Cache (a read, so no dirty lines are left for the timed kernels to
write back); HIP events on the launch stream bracket each launch.

The timed region runs the K steps four ways, interleaved step by step so
that no form is always the one measured first after the warm-up:
  * the two-kernel form (tmla_mla_decode: partial + combine kernels),
  * the single launch (tmla_mla_decode_fused: the merge inside the partial
    kernel),
  * the partial kernel alone (the dominant kernel of the roofline),
  * the public ``triton_mla.mla_decode(...)`` call, timed the way the
    reference's bench times it (output and workspace allocation and the
    host-side argument checks included; its host time per call is reported
    as ``public_call_host_us``).
``value`` is the form mla_decode() runs by default; the others are reported
beside it with min / median / p90.

Then the other measured shapes (``shapes`` in the JSON line; ``--no-shapes``
skips them and the layer): B=1 and B=8 at 1K tokens (128 heads), the ragged
B=64 workload (1K..32K tokens, seed 0) with 128 and with 16 heads, and B=8
with 64 heads at 16K tokens, each with its two-kernel step, partial kernel,
HBM roofline and 70%-of-roofline target; and ``layer_step``: one decode step
of the MLA layer at DeepSeek-V3 dims (B=16, 16K tokens), eager and replayed
from a HIP graph, against the roofline of its weights plus cache.

Then the fp8-cache legs (``fp8_cache`` and ``fp8_cache_h128`` in the JSON
line; ``--no-fp8`` skips them): the 16-head ragged workload (B=64, 1K..32K
tokens, page 64) and the measured 128-head workload above, each with its
cache quantised to E4M3 with one float32 scale per page, timed interleaved
with the bf16 decode of the unquantised cache (two-kernel steps and partial
kernels alone), with the fp8 partial kernel's roofline over the fp8 bytes.

``--copy-mib N`` adds, after the timed steps, three device-to-device copies
of N MiB: kernels of known traffic against which the HBM counters of a
profiler run (FETCH_SIZE, WRITE_SIZE) are scaled.

Prints one JSON line: throughput in TFLOP/s (flops = 2 * H * (576 + 512) per
cached token), microseconds per step, the HBM roofline of the partial kernel
and the reference's CPU path (float32 torch ``mla_decode_ref``, per
sequence, and the eager batched ``mla_decode_torch``) timed on this host's
cores; the float64 C oracle is the correctness gate.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "triton-mla_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
METRIC = "mla_decode µs/step + TFLOPS (% roofline), B=32 H=128 ctx 8K bf16, 1 GPU"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_b32_h128_ctx8k.json")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--splits", default="balanced",
                   help="'balanced' (device-side tile balancing) or an integer split count")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on each CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-fp8", action="store_true", help="skip the fp8-cache leg (16-head ragged workload)")
    p.add_argument("--no-shapes", action="store_true",
                   help="skip the other decode shapes and the layer step")
    p.add_argument("--no-flush", action="store_true", help="do not evict caches between steps")
    p.add_argument("--copy-mib", type=int, default=0,
                   help="after timing, run 3 copies of this many MiB (counter calibration)")
    return p.parse_args()


def spread(times):
    t = sorted(times)
    return {"min": round(t[0], 2), "median": round(statistics.median(t), 2),
            "p90": round(t[min(len(t) - 1, int(0.9 * len(t)))], 2), "mean": round(statistics.fmean(t), 2)}


def cpu_baseline(inp, target_s):
    """The reference's CPU path on this host's cores: the float32 per-sequence
    mla_decode_ref (src/triton_mla/reference.py:16-31) on the whole workload
    (median of 3 after a warm-up run, each bounded by target_s), and the
    eager batched mla_decode_torch (reference.py:34-44) on the sequences that
    fit target_s."""
    import torch

    from triton_mla.reference import mla_decode_ref, mla_decode_torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    args = (inp.q, inp.kv_cache, inp.seqlens, inp.block_table, 512, inp.softmax_scale)

    def timed(fn, n):
        t0 = time.perf_counter()
        fn(inp.q[:n], inp.kv_cache, inp.seqlens[:n], inp.block_table[:n], 512, inp.softmax_scale)
        return time.perf_counter() - t0

    # fp32 reference: whole workload if a first sequence says it fits
    t1 = timed(mla_decode_ref, 1)
    n_ref = int(max(1, min(inp.batch, target_s / max(t1, 1e-4))))
    runs = [timed(mla_decode_ref, n_ref) for _ in range(3)]
    t_ref = statistics.median(runs)
    out_ref, _ = mla_decode_ref(*args) if n_ref == inp.batch else (None, None)
    # eager batched torch path (bf16 matmuls on the CPU)
    t1 = timed(mla_decode_torch, 1)
    n_torch = int(max(1, min(inp.batch, target_s / max(t1, 1e-4))))
    t_torch = timed(mla_decode_torch, n_torch)
    return {"cores": cores, "n_ref": n_ref, "t_ref": t_ref, "n_torch": n_torch, "t_torch": t_torch,
            "out_ref": out_ref}


def shape_legs(args, dev, flush, stream, hosts):
    """The decode on the other measured shapes: the two-kernel step of
    mla_decode's default partition and its partial kernel alone, interleaved
    rep by rep, each against the HBM roofline of its algorithmic bytes and
    the 70% of it that the step is meant to reach (shapes whose roofline is
    under 10 us are launch-bound: their targets are not given)."""
    import torch

    from triton_mla.kernel import DecodeLaunch

    out = {}
    for host in hosts:
        g = host.to(dev)
        call = DecodeLaunch(g.q, g.kv_cache, g.seqlens, g.block_table, 512, host.softmax_scale, None)
        forms = {"step": call.run, "partial": call.partial}
        for _ in range(max(args.warmup // 2, 2)):
            for fn in forms.values():
                if flush:
                    flush()
                fn()
        steps = max(args.steps // 2, 10)
        ev = {k: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
              for k in forms}
        torch.cuda.synchronize(dev)
        for i in range(steps):
            for k, fn in forms.items():
                if flush:
                    flush()
                ev[k][i][0].record(stream)
                fn()
                ev[k][i][1].record(stream)
        torch.cuda.synchronize(dev)
        us = {k: [a.elapsed_time(b) * 1e3 for a, b in v] for k, v in ev.items()}
        nbytes = host.algorithmic_bytes()
        roof = nbytes / (HBM_PEAK_GBS * 1e9) * 1e6
        step = statistics.median(us["step"])
        out[host.name] = {
            "batch": host.batch, "heads": host.heads, "tokens": int(host.seqlens.sum()),
            "algorithmic_bytes": nbytes, "roofline_us": round(roof, 2),
            "target_us_70pct": round(roof / 0.7, 1) if roof >= 10 else None,
            "step_us": spread(us["step"]), "partial_us": spread(us["partial"]),
            "step_frac": round(roof / step, 4),
            "tflops": round(host.flops() / (step * 1e-6) / 1e12, 2),
        }
        del call, g
        torch.cuda.empty_cache()
    return out


def layer_leg(args, dev, flush, stream):
    """One decode step of the MLA layer at DeepSeek-V3 dims (hidden 7168,
    q_lora 1536, latent 512 + rope 64, 128 heads), batch 16, 16384 cached
    tokens, random weights ~ N(0, 0.02): eager (HIP glue) and replayed from
    a HIP graph, against the HBM roofline of its weights plus cache."""
    import torch

    from triton_mla.bench import capture_layer_step
    from triton_mla.model import MLA, MLAConfig

    cfg = MLAConfig()
    gen = torch.Generator().manual_seed(0)
    model = MLA(cfg)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if "norm" not in name:
                prm.copy_(torch.randn(prm.shape, generator=gen) * 0.02)
    model = model.to(dev, torch.bfloat16)
    batch, ctx, page = 16, 16384, 64
    pages = -(-(ctx + 1) // page)
    cache = torch.randn(batch * pages, page, cfg.kv_cache_dim, generator=gen).to(dev, torch.bfloat16)
    bt = torch.randperm(batch * pages, generator=gen).view(batch, pages).int().to(dev)
    seqlens = torch.full((batch,), ctx, dtype=torch.int32, device=dev)
    x = torch.randn(batch, cfg.hidden_size, generator=gen).to(dev, torch.bfloat16)
    with torch.no_grad():
        eager = lambda: model(x, cache, seqlens, bt)  # noqa: E731
        out_e, _ = eager()
        graph, out_g = capture_layer_step(model, x, cache, seqlens, bt, dev)
        graph.replay()
        torch.cuda.synchronize(dev)
        same = torch.equal(out_g, out_e)
        forms = {"eager": eager, "graph": graph.replay}
        for _ in range(3):
            for fn in forms.values():
                if flush:
                    flush()
                fn()
        steps = max(args.steps // 4, 10)
        ev = {k: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
              for k in forms}
        torch.cuda.synchronize(dev)
        for i in range(steps):
            for k, fn in forms.items():
                if flush:
                    flush()
                ev[k][i][0].record(stream)
                fn()
                ev[k][i][1].record(stream)
        torch.cuda.synchronize(dev)
    us = {k: [a.elapsed_time(b) * 1e3 for a, b in v] for k, v in ev.items()}
    weight_bytes = sum(prm.numel() * prm.element_size() for prm in model.parameters())
    kv_bytes = batch * (ctx + 1) * cfg.kv_cache_dim * 2
    roof = (weight_bytes + kv_bytes) / (HBM_PEAK_GBS * 1e9) * 1e6
    del graph, model, cache
    torch.cuda.empty_cache()
    return {"workload": "mla_layer_v3_b16_ctx16k", "weight_bytes": weight_bytes, "kv_bytes": kv_bytes,
            "roofline_us": round(roof, 2), "step_us": spread(us["eager"]), "graph_step_us": spread(us["graph"]),
            "graph_frac": round(roof / statistics.median(us["graph"]), 4), "graph_matches_eager": same}


def fp8_leg(args, dev, flush, stream, host, kernel):
    """The fp8 (E4M3, one scale per page) cache on one workload: the
    two-kernel step and the partial kernel alone, interleaved with the bf16
    decode of the same cache before quantisation."""
    import torch

    from triton_mla import quantize_kv_fp8
    from triton_mla.kernel import DecodeLaunch

    g = host.to(dev)
    codes, scale = quantize_kv_fp8(g.kv_cache, "page")
    c8 = DecodeLaunch(g.q, codes, g.seqlens, g.block_table, 512, host.softmax_scale, None, kv_scale=scale)
    c16 = DecodeLaunch(g.q, g.kv_cache, g.seqlens, g.block_table, 512, host.softmax_scale, None)
    forms = {"fp8_step": c8.run, "fp8_partial": c8.partial, "bf16_step": c16.run, "bf16_partial": c16.partial}
    for _ in range(max(args.warmup // 2, 2)):
        for fn in forms.values():
            if flush:
                flush()
            fn()
    steps = max(args.steps // 2, 10)
    ev = {k: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
          for k in forms}
    torch.cuda.synchronize(dev)
    for i in range(steps):
        for k, fn in forms.items():
            if flush:
                flush()
            ev[k][i][0].record(stream)
            fn()
            ev[k][i][1].record(stream)
    torch.cuda.synchronize(dev)
    us = {k: [a.elapsed_time(b) * 1e3 for a, b in v] for k, v in ev.items()}
    c8.run()
    torch.cuda.synchronize(dev)
    tokens = int(host.seqlens.sum())
    q_out = host.q.numel() * 2 + host.batch * host.heads * 512 * 2
    bytes8 = tokens * 576 + scale.numel() * 4 + q_out
    bytes16 = host.algorithmic_bytes()
    med = {k: statistics.median(v) for k, v in us.items()}
    p8 = statistics.fmean(us["fp8_partial"])
    summary = {
        "workload": host.name, "batch": host.batch, "heads": host.heads, "tokens": tokens, "page_size": 64,
        "format": "e4m3 codes + float32 scale per page", "algorithmic_bytes": bytes8,
        "step_us": {k: spread(v) for k, v in us.items()},
        "roofline": {"bound": "hbm", "kernel": kernel, "partial_us_mean": round(p8, 2),
                     "achieved": round(bytes8 / (p8 * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(bytes8 / (p8 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "step_frac": round(bytes8 / (med["fp8_step"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        "bf16_same_workload": {"algorithmic_bytes": bytes16,
                               "step_frac": round(bytes16 / (med["bf16_step"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        "speedup_vs_bf16_step": round(med["bf16_step"] / med["fp8_step"], 3),
    }
    gate = {"q": host.q, "codes": codes.view(torch.uint8).cpu().numpy(), "scale": scale.cpu().numpy(),
            "seqlens": host.seqlens.numpy(), "bt": host.block_table.numpy(), "softmax_scale": host.softmax_scale,
            "out": c8.out.cpu()}
    del c8, c16, g, codes, scale
    torch.cuda.empty_cache()
    return {"summary": summary, "gate": gate}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the decode path runs and is measured on a single MI355X; see DESIGN.md for how "
              "it would shard)", file=sys.stderr)
        sys.exit(2)

    import torch

    import triton_mla
    from triton_mla import workloads
    from triton_mla.kernel import DecodeLaunch, DEFAULT_SINGLE_LAUNCH
    from triton_mla.timing import Flusher

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = workloads.b32_h128_8k().to(dev)
    splits = None if args.splits == "balanced" else int(args.splits)
    call = DecodeLaunch(inp.q, inp.kv_cache, inp.seqlens, inp.block_table, 512, inp.softmax_scale, splits)
    flush = None if args.no_flush else Flusher(dev)
    stream = torch.cuda.current_stream(dev)
    default_single = DEFAULT_SINGLE_LAUNCH and call.fused

    # the public call, as the reference's bench times it (bench.py:68-69, 78):
    # fresh outputs and workspace, host-side checks and launches per call;
    # timed in the same loop as the reused launch, step by step
    pub_fn = lambda: triton_mla.mla_decode(inp.q, inp.kv_cache, inp.seqlens, inp.block_table,  # noqa: E731
                                           softmax_scale=inp.softmax_scale, num_splits=splits)
    forms = {
        "two_kernel": lambda: call.run(single_launch=False),
        "single_launch": lambda: call.run(single_launch=True),
        "partial_only": call.partial,
        "public_call": pub_fn,
    }
    if not call.fused:
        del forms["single_launch"]
    for _ in range(args.warmup):
        for fn in forms.values():
            if flush:
                flush()
            fn()
    torch.cuda.synchronize(dev)

    # timed region: K steps of each form, interleaved step by step
    ev = {k: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)] for k in forms}
    torch.cuda.synchronize(dev)
    host_us = []  # host time of each public call
    wall0 = time.perf_counter()
    for i in range(args.steps):
        for k, fn in forms.items():
            if flush:
                flush()
            ev[k][i][0].record(stream)
            t0 = time.perf_counter()
            fn()
            if k == "public_call":
                host_us.append((time.perf_counter() - t0) * 1e6)
            ev[k][i][1].record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    us = {k: [a.elapsed_time(b) * 1e3 for a, b in v] for k, v in ev.items()}
    public_us = us.pop("public_call")

    headline = "single_launch" if default_single else "two_kernel"
    # outputs of both forms on the same inputs: the same merge code on the same partials
    call.run(single_launch=False)
    torch.cuda.synchronize(dev)
    eager_out = call.out.clone()
    single_same = None
    if call.fused:
        call.out.fill_(1.0)
        call.run(single_launch=True)
        torch.cuda.synchronize(dev)
        single_same = torch.equal(call.out, eager_out)

    pub_out = pub_fn()
    torch.cuda.synchronize(dev)
    public_same = torch.equal(pub_out, eager_out)

    # the same step captured once in a HIP graph and replayed (how a serving
    # loop launches it): every replay must reproduce the eager result exactly
    graph_ok = None
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            forms[headline]()
        graph_ok = True
        for _ in range(3):
            call.out.zero_()
            graph.replay()
            torch.cuda.synchronize(dev)
            graph_ok = graph_ok and torch.equal(call.out, eager_out)
            torch.randn(1024, device=dev).sum().item()  # eager work between replays
        del graph
    except RuntimeError as exc:  # capture unsupported in this environment
        print(f"graph capture failed: {exc}", file=sys.stderr)

    shapes, layer = {}, None
    ragged16 = None
    if not args.no_shapes:
        ragged16 = workloads.ragged_b64_h16()
        shapes = shape_legs(args, dev, flush, stream, [workloads.b1_h128_1k(), workloads.b8_h128_1k(),
                                                        workloads.ragged_b64_h128(), ragged16,
                                                        workloads.b8_h64_16k()])
        layer = layer_leg(args, dev, flush, stream)

    fp8 = {}
    if not args.no_fp8:
        # 16 heads: the 16-head-group kernel; 128 heads: the 16-bit kernel
        # with the cache widened once per workgroup into its ring
        fp8["fp8_cache"] = fp8_leg(args, dev, flush, stream, ragged16 or workloads.ragged_b64_h16(),
                                   "mla_partial_fp8_kernel")
        fp8["fp8_cache_h128"] = fp8_leg(args, dev, flush, stream, workloads.b32_h128_8k(),
                                        "mla_partial_kernel (fp8 cache widened into the ring)")

    if args.copy_mib > 0:
        src = torch.ones(args.copy_mib << 18, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            if flush:
                flush()
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        del src, dst

    step = us[headline]
    t_med = statistics.median(step)
    p_us = statistics.fmean(us["partial_only"])
    nbytes = inp.algorithmic_bytes()
    flops = inp.flops()
    tflops = flops / (t_med * 1e-6) / 1e12
    achieved_gbs = nbytes / (p_us * 1e-6) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        traffic = json.load(open(TRAFFIC_FILE)).get("hbm_bytes_per_launch")

    result = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_med / 1e3, 5),
        "us_per_step": round(t_med, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (randn q/cache, randperm block tables, seed 0)",
        "config": {"workload": inp.name, "batch": inp.batch, "heads": inp.heads, "seq_len": 8192,
                   "page_size": 64, "num_splits": args.splits, "cache_flush_mib": 0 if args.no_flush else 512,
                   "form": headline},
        "roofline": {"bound": "hbm", "kernel": "mla_partial_own_kernel", "achieved": round(achieved_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes": nbytes,
                     "partial_us_mean": round(p_us, 2),
                     "step_frac": round(nbytes / (t_med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)},
        "step_us": {k: spread(v) for k, v in us.items()},
        "single_launch_matches": single_same,
        "public_call_us": spread(public_us),
        "public_call_host_us": spread(host_us),
        "public_call_matches": public_same,
        "wall_s_timed_region": round(wall, 4),
        "timed_launches": {k: args.steps for k in ev},
        "graph_replay_matches_eager": graph_ok,
    }
    if shapes:
        result["shapes"] = shapes
    if layer:
        result["layer_step"] = layer
    for key, leg in fp8.items():
        result[key] = leg["summary"]

    if not args.no_cpu_baseline:
        import numpy as np

        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle

        host = workloads.b32_h128_8k()
        # correctness gate: the float64 C oracle on the first two sequences
        n = 2

        def u16(t):
            return t.contiguous().view(torch.int16).numpy().view(np.uint16)

        ref_out, _ = oracle.mla_decode_ref(u16(host.q[:n]), u16(host.kv_cache), host.seqlens[:n].numpy(),
                                           host.block_table[:n].numpy(), 512, host.softmax_scale)
        err = (eager_out[:n].float().cpu() - torch.from_numpy(ref_out)).abs().max().item()
        if not err <= 1e-2:
            print(f"correctness gate failed: max |gpu - oracle| = {err}", file=sys.stderr)
            sys.exit(1)
        cb = cpu_baseline(host, args.cpu_seconds)
        per_seq_flops = flops / inp.batch
        cpu_tflops = cb["n_ref"] * per_seq_flops / cb["t_ref"] / 1e12
        result["cpu_baseline"] = {
            "value": round(cpu_tflops, 5), "unit": "TFLOP/s", "cores": cb["cores"], "kind": "port",
            "sample": f"float32 torch mla_decode_ref (reference.py:16-31, per sequence) on {cb['n_ref']} of "
                      f"{inp.batch} sequences (8192 tokens, 128 heads), median of 3: {cb['t_ref']:.3f} s",
            "us_per_step_equiv": round(cb["t_ref"] / cb["n_ref"] * inp.batch * 1e6, 1),
            "eager_torch": {"value": round(cb["n_torch"] * per_seq_flops / cb["t_torch"] / 1e12, 5),
                            "unit": "TFLOP/s", "sample": f"mla_decode_torch (reference.py:34-44) on "
                            f"{cb['n_torch']} sequences: {cb['t_torch']:.3f} s"},
            "gpu_vs_oracle_max_abs_err": err,
        }
        if cb["out_ref"] is not None:
            result["cpu_baseline"]["gpu_vs_cpu_ref_max_abs_err"] = \
                (eager_out.float().cpu() - cb["out_ref"].float()).abs().max().item()
        for key, leg in fp8.items():
            # the fp8 legs' gates: the float64 fp8 oracle on their first two sequences
            f = leg["gate"]
            ref8, _ = oracle.mla_decode_fp8_ref(u16(f["q"][:n]), f["codes"], f["scale"], f["seqlens"][:n],
                                                f["bt"][:n], 512, f["softmax_scale"])
            err8 = (f["out"][:n].float() - torch.from_numpy(ref8)).abs().max().item()
            if not err8 <= 1e-2:
                print(f"{key} correctness gate failed: max |gpu - oracle| = {err8}", file=sys.stderr)
                sys.exit(1)
            result[key]["gpu_vs_oracle_max_abs_err"] = err8
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
