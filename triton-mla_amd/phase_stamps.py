"""Phase split of the partial kernel from the profiling build's stamps.

    python triton-mla_amd/build.py --stamps        # once, on a build host
    python triton-mla_amd/phase_stamps.py [--reps 25] [--workload b32_h128_ctx8k]

Runs the partial kernel of the workload --reps times (each after a 512 MiB
cache-evicting read) with the library built with TMLA_STAMPS=1 and prints,
per phase, the median over workgroups of its duration (microseconds, wall
clock) and the median over runs: partition (entry to work range), start-up
(page ids, Q, first copies), loop, finalize (normalisation and stores), the
shader clock, clocks per 32-token sub-tile, and the parts of one loop
iteration (128-head workgroups: the S^T MFMAs of the next sub-tile beside
the exponentials of this one, then the value MFMAs, then the copy wait and
the barrier; 32/64-head workgroups: S beside half of PV, the rest of PV
beside the softmax, the probabilities' publication and the barrier). Stamp
slots are defined at phase_stamp in csrc/mla_decode.hip; --spread adds the
per-workgroup percentiles and per-XCD medians of each launch.
"""

from __future__ import annotations

import argparse
import ctypes
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
os.environ.setdefault("TRITON_MLA_LIB", os.path.join(HERE, "triton_mla", "libtriton_mla_hip_stamps.so"))
sys.path.insert(0, HERE)

import numpy as np  # noqa: E402
import torch  # noqa: E402

from triton_mla import _native  # noqa: E402
from triton_mla.bench import WORKLOADS  # noqa: E402
from triton_mla.kernel import DecodeLaunch  # noqa: E402
from triton_mla.timing import Flusher  # noqa: E402

WORKERS, SLOTS = 4096, 9


def print_spread(run, wg, rt, ck, t0):
    """Percentiles over the workgroups of one launch, then per-XCD medians."""
    cols = dict(
        entry_us=(rt[:, 0] - t0) / 100,
        loop_start_us=(rt[:, 2] - t0) / 100,
        loop_end_us=(rt[:, 3] - t0) / 100,
        end_us=(rt[:, 4] - t0) / 100,
        loop_us=(rt[:, 3] - rt[:, 2]) / 100,
        ghz=(ck[:, 3] - ck[:, 2]) / np.maximum(1, (rt[:, 3] - rt[:, 2]) * 10.0),
    )
    print(f"run {run}: {len(wg)} workgroups", flush=True)
    for k, v in cols.items():
        q = np.percentile(v, [0, 10, 50, 90, 100])
        print(f"  {k:14s} min {q[0]:8.2f}  p10 {q[1]:8.2f}  p50 {q[2]:8.2f}  p90 {q[3]:8.2f}  max {q[4]:8.2f}")
    xcd = wg % 8
    line = "  per XCD (median loop_us / end_us / ghz):"
    for x in range(8):
        m = xcd == x
        if m.any():
            line += (f" {x}: {np.median(cols['loop_us'][m]):.1f}/{np.median(cols['end_us'][m]):.1f}"
                     f"/{np.median(cols['ghz'][m]):.2f}")
    print(line, flush=True)
    late = np.argsort(cols["end_us"])[-4:]
    print("  latest workgroups (id: entry, loop start, loop end, end us):",
          "; ".join(f"{wg[i]}: {cols['entry_us'][i]:.1f}, {cols['loop_start_us'][i]:.1f}, "
                    f"{cols['loop_end_us'][i]:.1f}, {cols['end_us'][i]:.1f}" for i in late), flush=True)


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--reps", type=int, default=25)
    p.add_argument("--workload", default="b32_h128_ctx8k", choices=sorted(WORKLOADS))
    p.add_argument("--spread", action="store_true",
                   help="also print, per run, percentiles over workgroups of entry, loop end and end "
                        "(from the first entry), loop time and clocks per sub-tile, and the medians of "
                        "the workgroups of each XCD (workgroup x runs on XCD x mod 8)")
    args = p.parse_args()
    dev = torch.device("cuda:0")
    inp = WORKLOADS[args.workload]().to(dev)
    call = DecodeLaunch(inp.q, inp.kv_cache, inp.seqlens, inp.block_table, 512, inp.softmax_scale, None)
    nwg = call.workers
    flush = Flusher(dev)
    buf = np.zeros(WORKERS * SLOTS * 2, dtype=np.uint64)
    rows = []
    for it in range(args.reps):
        buf[:] = 0
        flush()
        call.partial()
        torch.cuda.synchronize(dev)
        _native.check(call.lib.tmla_debug_stamps(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes),
                      "tmla_debug_stamps")
        if it < 3:
            continue
        s = buf[: nwg * SLOTS * 2].reshape(nwg, SLOTS, 2).astype(np.int64)
        rt, ck = s[:, :, 0], s[:, :, 1]
        ok = (rt[:, 4] > rt[:, 0]) & (rt[:, 0] > 0)  # workgroups with a segment
        wg = np.nonzero(ok)[0]
        if wg.size == 0:
            raise SystemExit(f"workload {args.workload}: no workgroup recorded stamps (the stamps are placed in "
                             "the 32/64/128-head partial kernels, not in the 16-head or fp8 kernels)")
        rt, ck = rt[ok], ck[ok]
        t0 = rt[:, 0].min()
        if args.spread and it < 6:
            print_spread(it, wg, rt, ck, t0)
        nsub = float(np.median((ck[:, 3] - ck[:, 2]))) / max(1.0, float(np.median(ck[:, 8] - ck[:, 5])))
        it_ok = (rt[:, 8] > rt[:, 5])
        r = dict(
            partition_us=np.median(rt[:, 1] - rt[:, 0]) / 100,
            startup_us=np.median(rt[:, 2] - rt[:, 1]) / 100,
            loop_us=np.median(rt[:, 3] - rt[:, 2]) / 100,
            finalize_us=np.median(rt[:, 4] - rt[:, 3]) / 100,
            ghz=np.median((ck[:, 3] - ck[:, 2]) / ((rt[:, 3] - rt[:, 2]) * 10.0)),
            loop_end_median_us=np.median(rt[:, 3] - t0) / 100,
            end_max_us=(rt[:, 4] - t0).max() / 100,
            iter_clk=np.median(ck[it_ok, 8] - ck[it_ok, 5]),
            iter_pass1_clk=np.median(ck[it_ok, 6] - ck[it_ok, 5]),
            iter_pass2_clk=np.median(ck[it_ok, 7] - ck[it_ok, 6]),
            iter_publish_barrier_clk=np.median(ck[it_ok, 8] - ck[it_ok, 7]),
            loop_iterations=nsub,
        )
        rows.append(r)
    print(f"workload {args.workload}: {len(rows)} runs, {nwg} workers")
    for k in rows[0]:
        v = [r[k] for r in rows]
        print(f"{k:26s} median {statistics.median(v):9.2f}   min {min(v):9.2f}   max {max(v):9.2f}", flush=True)


if __name__ == "__main__":
    main()
