"""triton-mla-bench: time mla_decode against PyTorch eager and torch.compile.

    triton-mla-bench --batch 1 32 128 --seqlen 1024 4096 16384
    python -m triton_mla.bench --workload b32_h128_ctx8k ragged_b64_h16_ctx1k-32k

Same command line and CSV columns as the reference's benchmark
(src/triton_mla/bench.py:16-108): --batch/--seqlen grid, --heads,
--page-size, --dtype, --compile-mode, --no-eager, --csv. The ``triton_us``
column keeps its name for drop-in CSV consumers and holds the HIP kernels'
time; ``config`` names the launch shape that ran. Additions: --workload runs
the named seeded workloads of triton_mla.workloads (uniform and ragged
lengths), --splits picks the split scheme, --no-compile skips torch.compile,
--head-dim-v / --rope-dim set the head dims (make_inputs' d_latent / d_rope:
other dims run the generic decode), --dtype fp32 decodes float32 inputs,
--kv-fp8 decodes an E4M3 copy of the cache, --layer times one decode step of the whole MLA layer at DeepSeek-V3 dims
(random N(0, 0.02) bf16 weights, --batch sequences of --seqlen cached tokens)
with the HIP glue (MLA.forward) and with the reference's torch glue
(MLA.forward_torch_glue) around the same mla_decode.

Timing: median of --reps runs, each preceded by a 512 MiB read that evicts
the Infinity Cache, bracketed by HIP events on the current stream (the
reference uses triton.testing.do_bench with a 256 MiB flush). Bytes and FLOPs
follow the reference's formulas (src/triton_mla/bench.py:80-81) with the sum
of sequence lengths for ragged batches.
"""

from __future__ import annotations

import argparse
import csv
import os

import torch

from . import _native, workloads
from . import kernel as kernel_mod
from .fp8 import dequantize_kv_fp8, quantize_kv_fp8
from .kernel import DecodeLaunch, _num_sms, balanced_pieces, mla_decode
from .reference import mla_decode_torch
from .timing import Flusher, time_us

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
CSV_FIELDS = ["gpu", "batch", "seqlen", "heads", "num_splits", "config", "bytes", "triton_us", "eager_us", "compile_us"]
WORKLOADS = {
    "b1_h128_ctx1k": workloads.b1_h128_1k,
    "b8_h128_ctx1k": workloads.b8_h128_1k,
    "b32_h128_ctx8k": workloads.b32_h128_8k,
    "ragged_b64_h128_ctx1k-32k": workloads.ragged_b64_h128,
    "ragged_b64_h16_ctx1k-32k": workloads.ragged_b64_h16,
    "b8_h64_ctx16k": workloads.b8_h64_16k,
}


def make_inputs(batch, seqlen, num_heads, page_size, dtype, device, d_latent=512, d_rope=64, seed=0):
    """Uniform-length inputs (the reference's make_inputs recipe and
    arguments, bench.py:20-27, seeded)."""
    inp = workloads.uniform(batch, num_heads, seqlen, dtype=dtype, seed=seed, page=page_size, d_latent=d_latent,
                            d_rope=d_rope)
    return inp.to(device)


def _splits_arg(text):
    return None if text == "balanced" else int(text)


def bench_one(inp, args, device, flush, compiled, writer, gpu):
    splits = _splits_arg(args.splits)
    torch_cache = inp.kv_cache
    generic = inp.head_dim_v != 512 or inp.q.shape[-1] != 576 or inp.q.dtype == torch.float32
    if generic:
        if args.kv_fp8 != "none":
            raise SystemExit("--kv-fp8 runs at --head-dim-v 512 --rope-dim 64 only")
        if splits is None:
            splits = kernel_mod._generic_splits(inp.batch, inp.heads, inp.kv_cache.shape[1] * inp.block_table.shape[1],
                                                _num_sms(device),
                                                max(_native.load().tmla_generic_heads_per_workgroup(
                                                    inp.head_dim_v, inp.q.shape[-1] - inp.head_dim_v,
                                                    _native.DTYPE_CODE[inp.q.dtype]), 1))
        call = _GenericCall(inp, splits)
    elif args.kv_fp8 != "none":
        # the HIP decode reads the E4M3 cache; the PyTorch baselines decode the
        # same values dequantised to the input dtype
        codes, scale = quantize_kv_fp8(inp.kv_cache, args.kv_fp8)
        torch_cache = dequantize_kv_fp8(codes, scale).to(inp.q.dtype)
        call = DecodeLaunch(inp.q, codes, inp.seqlens, inp.block_table, 512, inp.softmax_scale, splits,
                            kv_scale=scale)
    else:
        call = DecodeLaunch(inp.q, inp.kv_cache, inp.seqlens, inp.block_table, 512, inp.softmax_scale, splits)
    call.run()
    torch.cuda.synchronize(device)
    out = call.out

    def run_torch(fn):
        return fn(inp.q, torch_cache, inp.seqlens, inp.block_table, head_dim_v=inp.head_dim_v,
                  softmax_scale=inp.softmax_scale)

    t_compile = None
    if compiled is not None:
        print(f"# compiling the torch.compile leg for batch {inp.batch}, heads {inp.heads}, "
              f"max length {int(inp.seqlens.max())}", flush=True)
        ref = run_torch(compiled)
        torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=2e-2)
        t_compile = time_us(lambda: run_torch(compiled), reps=args.reps, flush=flush, device=device)["median"]
    elif not args.no_eager:
        ref = run_torch(mla_decode_torch)
        torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=2e-2)

    t_hip = time_us(call.run, reps=args.reps, flush=flush, device=device)["median"]
    t_eager = None
    if not args.no_eager:
        t_eager = time_us(lambda: run_torch(mla_decode_torch), reps=max(args.reps // 4, 5), flush=flush,
                          device=device)["median"]

    nbytes = inp.algorithmic_bytes()
    if args.kv_fp8 != "none":  # one byte per cache element (+ the scales)
        tokens = int(inp.seqlens.sum())
        nbytes -= tokens * inp.kv_cache.shape[-1]
        nbytes += (scale.numel() * 4)
    flops = inp.flops()
    workers = call.workers or call.splits * inp.batch
    # (the heads per workgroup are chosen inside the library from the call's
    # shape, so the label names the partition only)
    config = "hip/" + (f"balanced{workers}" if splits is None else f"splits{splits}")
    if generic:
        config += f"/generic-{inp.head_dim_v}+{inp.q.shape[-1] - inp.head_dim_v}"
    if args.kv_fp8 != "none":
        config += f"/fp8-{args.kv_fp8}"
    seqlen = int(inp.seqlens.max())
    # the CSV's num_splits is an integer, as the reference writes it
    # (bench.py:98): the uniform count, or for the balanced partition the
    # largest number of workers one sequence is cut into
    num_splits = splits if splits is not None else balanced_pieces(inp.seqlens.tolist(), workers)
    row = [inp.batch, seqlen, num_splits, config, f"{t_hip:.1f}", f"{nbytes / t_hip / 1e6:.2f}",
           f"{flops / t_hip / 1e6:.0f}"]
    if not args.no_eager:
        row.append(f"{t_eager:.1f}")
    if t_compile is not None:
        row += [f"{t_compile:.1f}", f"{t_compile / t_hip:.2f}x"]
    print("| " + " | ".join(str(c) for c in row) + " |", flush=True)
    if writer:
        writer.writerow({"gpu": gpu, "batch": inp.batch, "seqlen": seqlen, "heads": inp.heads,
                         "num_splits": num_splits, "config": config, "bytes": nbytes, "triton_us": t_hip,
                         "eager_us": t_eager, "compile_us": t_compile})


class _GenericCall:
    """A decode at other head dims or fp32 (the generic kernels through the
    public mla_decode), with DecodeLaunch's run/out/workers/splits."""

    def __init__(self, inp, splits):
        self.inp, self.splits, self.workers = inp, splits, 0
        self.out = None

    def run(self):
        i = self.inp
        self.out = mla_decode(i.q, i.kv_cache, i.seqlens, i.block_table, head_dim_v=i.head_dim_v,
                              softmax_scale=i.softmax_scale, num_splits=self.splits)
        return self.out


def capture_layer_step(model, x, cache, seqlens, bt, device):
    """One MLA.forward step captured in a CUDA (HIP) graph on a side stream
    of default priority, after two eager steps there that allocate the
    step's cached buffers (the projections' workspace of that stream, which
    the graph then shares); returns the graph and its output tensor."""
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for _ in range(2):
            model(x, cache, seqlens, bt)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        out, _ = model(x, cache, seqlens, bt)
    return graph, out


def bench_layer(args, device, flush):
    """One MLA decode step at DeepSeek-V3 dims: HIP glue vs torch glue."""
    from .model import MLA, MLAConfig

    cfg = MLAConfig()
    gen = torch.Generator().manual_seed(0)
    model = MLA(cfg)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" not in name:
                p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    model = model.to(device, DTYPES[args.dtype])
    weight_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    print(f"# MLA layer step, DeepSeek-V3 dims, weights {weight_bytes / 1e6:.1f} MB, {args.dtype}")
    print("| batch | context | hip glue us | hip glue, graph us | torch glue us | mla_decode us | glue saved us "
          "| layer roofline us |")
    print("|---|---|---|---|---|---|---|---|")
    for batch in args.batch:
        for ctx in args.seqlen:
            page = args.page_size
            pages = -(-(ctx + 1) // page)
            cache = torch.randn(batch * pages, page, cfg.kv_cache_dim, generator=gen).to(device, model.wq_a.weight.dtype)
            bt = torch.randperm(batch * pages, generator=gen).view(batch, pages).int().to(device)
            seqlens = torch.full((batch,), ctx, dtype=torch.int32, device=device)
            x = torch.randn(batch, cfg.hidden_size, generator=gen).to(device, cache.dtype)
            with torch.no_grad():
                out_h, _ = model(x, cache, seqlens, bt)
                out_t, _ = model.forward_torch_glue(x, cache, seqlens, bt)
                torch.testing.assert_close(out_h.float(), out_t.float(), atol=3e-2, rtol=3e-2)
                t_h = time_us(lambda: model(x, cache, seqlens, bt), reps=args.reps, flush=flush, device=device)
                t_t = time_us(lambda: model.forward_torch_glue(x, cache, seqlens, bt), reps=args.reps, flush=flush,
                              device=device)
                # the HIP-glue step captured in one graph (no host work between its kernels)
                graph, out_g = capture_layer_step(model, x, cache, seqlens, bt, device)
                graph.replay()
                torch.cuda.synchronize(device)
                assert torch.equal(out_g, out_h), "graph replay differs from the eager step"
                t_g = time_us(graph.replay, reps=args.reps, flush=flush, device=device)
                del graph, out_g
                q = torch.randn(batch, cfg.num_heads, cfg.kv_cache_dim, generator=gen).to(device, cache.dtype)
                call = DecodeLaunch(q, cache, seqlens + 1, bt, cfg.kv_lora_rank, cfg.qk_head_dim ** -0.5, None)
                t_d = time_us(call.run, reps=args.reps, flush=flush, device=device)
            kv_bytes = batch * (ctx + 1) * cfg.kv_cache_dim * cache.element_size()
            roof = (weight_bytes + kv_bytes) / 8.0e12 * 1e6
            print(f"| {batch} | {ctx} | {t_h['median']:.1f} | {t_g['median']:.1f} | {t_t['median']:.1f} | "
                  f"{t_d['median']:.1f} | "
                  f"{t_t['median'] - t_h['median']:.1f} | {roof:.1f} |", flush=True)
            del cache, bt, x, q, call
            torch.cuda.empty_cache()


def bench_projections(args, device, flush):
    """The MLA layer's dense projections at DeepSeek-V3 dims for --batch rows:
    tmla_mla_project against the library GEMM (torch.nn.functional.linear)."""
    import torch.nn.functional as F

    from . import layer_ops

    cfg_shapes = {"wq_a": (1536, 7168), "wq_b": (128 * 192, 1536), "wkv_a": (576, 7168), "wo": (7168, 128 * 128)}
    gen = torch.Generator(device=device).manual_seed(0)
    dtype = DTYPES[args.dtype]
    print(f"# MLA layer projections, DeepSeek-V3 dims, {args.dtype}")
    print("| rows | projection | N x K | weight MB | library us | tmla_mla_project us | project TB/s |")
    print("|---|---|---|---|---|---|---|")
    for m in args.batch:
        for name, (n, k) in cfg_shapes.items():
            x = torch.randn(m, k, device=device, generator=gen).to(dtype)
            w = (0.02 * torch.randn(n, k, device=device, generator=gen)).to(dtype)
            if not layer_ops.project_fits(x, w):
                continue
            lib_t = time_us(lambda: F.linear(x, w), reps=args.reps, flush=flush, device=device)["median"]
            hip_t = time_us(lambda: layer_ops.project(x, w), reps=args.reps, flush=flush, device=device)["median"]
            mb = n * k * w.element_size() / 1e6
            print(f"| {m} | {name} | {n} x {k} | {mb:.1f} | {lib_t:.2f} | {hip_t:.2f} | {mb / hip_t:.2f} |",
                  flush=True)
            del x, w


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--batch", type=int, nargs="+", default=[1, 8, 32, 64, 128])
    parser.add_argument("--seqlen", type=int, nargs="+", default=[1024, 4096, 8192, 16384, 32768])
    parser.add_argument("--heads", type=int, default=128, help="128 for one GPU, 16 per GPU under TP8")
    parser.add_argument("--page-size", type=int, default=64)
    parser.add_argument("--dtype", choices=DTYPES, default="bf16")
    parser.add_argument("--head-dim-v", type=int, default=512,
                        help="latent dims (make_inputs' d_latent); not 512 runs the generic decode")
    parser.add_argument("--rope-dim", type=int, default=64, help="RoPE dims (make_inputs' d_rope)")
    parser.add_argument("--compile-mode", default="max-autotune-no-cudagraphs")
    parser.add_argument("--no-eager", action="store_true")
    parser.add_argument("--no-compile", action="store_true", help="skip the torch.compile baseline")
    parser.add_argument("--csv", help="also write results to this CSV file")
    parser.add_argument("--workload", nargs="+", choices=sorted(WORKLOADS),
                        help="run these named workloads instead of the --batch x --seqlen grid")
    parser.add_argument("--splits", default="balanced", help="'balanced' or a per-sequence split count")
    parser.add_argument("--reps", type=int, default=100)
    parser.add_argument("--kv-fp8", choices=["none", "page", "token", "tensor"], default="none",
                        help="decode an E4M3 copy of the cache (scales per page, token or tensor); the "
                             "PyTorch baselines decode the dequantised values")
    parser.add_argument("--layer", action="store_true",
                        help="time the MLA layer step at DeepSeek-V3 dims (HIP glue vs torch glue)")
    parser.add_argument("--projections", action="store_true",
                        help="time the layer's dense projections for --batch rows (HIP kernel vs library GEMM)")
    args = parser.parse_args(argv)

    device = torch.device("cuda")
    dtype = DTYPES[args.dtype]
    flush = Flusher(device)
    if args.projections:
        bench_projections(args, device, flush)
        return
    if args.layer:
        bench_layer(args, device, flush)
        return
    compiled = None
    if not args.no_compile:
        compiled = torch.compile(mla_decode_torch, mode=args.compile_mode, dynamic=False)

    gpu = torch.cuda.get_device_name()
    writer = None
    if args.csv:
        os.makedirs(os.path.dirname(os.path.abspath(args.csv)), exist_ok=True)
        csv_file = open(args.csv, "w", newline="")
        writer = csv.DictWriter(csv_file, fieldnames=CSV_FIELDS)
        writer.writeheader()

    print(f"# {gpu}  CUs={_num_sms(device)}  heads={args.heads}  page={args.page_size}  {args.dtype}  "
          f"dims {args.head_dim_v}+{args.rope_dim}")
    cols = ["batch", "seqlen", "splits", "config", "hip us", "TB/s", "TFLOPS"]
    if not args.no_eager:
        cols.append("eager us")
    if compiled is not None:
        cols += ["compile us", "speedup"]
    print("| " + " | ".join(cols) + " |")
    print("|" + "---|" * len(cols))

    if args.workload:
        cases = [lambda name=name: WORKLOADS[name](dtype).to(device) for name in args.workload]
    else:
        cases = [lambda b=b, s=s: make_inputs(b, s, args.heads, args.page_size, dtype, device, args.head_dim_v,
                                              args.rope_dim)
                 for b in args.batch for s in args.seqlen]
    for make in cases:
        inp = make()
        bench_one(inp, args, device, flush, compiled, writer, gpu)
        del inp
        torch.cuda.empty_cache()
    if writer:
        csv_file.close()


if __name__ == "__main__":
    main()
