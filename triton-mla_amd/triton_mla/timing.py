"""GPU timing helpers: hipEvent-timed repetitions with a cache flush between them.

MI355X has a 256 MiB Infinity Cache in front of HBM, so every timed
repetition is preceded by a *read* of ``flush_bytes`` (default 512 MiB) that
evicts the previous repetition's working set. A read is used rather than a
write: a write flush leaves up to 256 MiB of dirty lines whose write-back
would then be charged to the timed kernel (measured: +40-50 us on a
300 MB streaming kernel).
"""

from __future__ import annotations

import statistics

import torch


class Flusher:
    """A row-sum over ``flush_bytes`` of int64: one reduction kernel that reads
    the whole buffer and writes 8 KiB (same dtype in and out, so no converted
    copy of the buffer is materialised)."""

    def __init__(self, device, flush_bytes: int = 512 << 20):
        rows = 1024
        self.buf = torch.ones(rows, max(flush_bytes // 8 // rows, 1), dtype=torch.int64, device=device)
        self.sink = torch.empty(rows, dtype=torch.int64, device=device)

    def __call__(self):
        torch.sum(self.buf, dim=1, out=self.sink)


def time_us(fn, reps: int = 100, warmup: int = 5, flush: Flusher | None = None,
            device=None) -> dict:
    """Median / mean / min microseconds of ``fn()`` over ``reps`` timed runs.

    Each run is bracketed by events recorded on the current stream of
    ``device``; the flush (if any) runs before the start event.
    """
    device = torch.device(device) if device is not None else torch.device("cuda")
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize(device)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    stream = torch.cuda.current_stream(device)
    for i in range(reps):
        if flush is not None:
            flush()
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize(device)
    times = [s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends)]
    return {"median": statistics.median(times), "mean": statistics.fmean(times), "min": min(times),
            "reps": reps}
