"""Phase split of the partial kernel from the profiling build's stamps.

    python triton-mla_amd/build.py --stamps        # once, on a build host
    python triton-mla_amd/phase_stamps.py [--reps 25] [--workload b32_h128_ctx8k]

Runs the partial kernel of the workload --reps times (each after a 512 MiB
cache-evicting read) with the library built with TMLA_STAMPS=1 and prints,
per phase, the median over workgroups of its duration (microseconds, wall
clock) and the median over runs: partition (entry to work range), start-up
(page ids, Q, first copies), loop, finalize (normalisation and stores), the
shader clock, clocks per 32-token sub-tile, and the parts of one loop
iteration (first pass: S of the next sub-tile beside half of PV; second
pass: the rest of PV beside the softmax; then the probabilities' publication
and the barrier). Stamp slots are defined at phase_stamp in
csrc/mla_decode.hip.
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


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--reps", type=int, default=25)
    p.add_argument("--workload", default="b32_h128_ctx8k", choices=sorted(WORKLOADS))
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
        rt, ck = rt[ok], ck[ok]
        t0 = rt[:, 0].min()
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
