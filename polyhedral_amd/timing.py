"""Timing harness: the call surface of gpu/bench.py (time_ms, paired_time, report).

Medians of HIP-event timings after warm-up, with a cache flush between
repetitions.  The flush buffer defaults to 512 MB rather than the reference's
64 MB (gpu/bench.py:12): MI355X keeps a 256 MB Infinity Cache (MALL) in front of
HBM, and a flush smaller than that would leave inputs resident between reps.
"""
import statistics

import torch

FLUSH_BYTES = 512 * 1024 * 1024


def _flush_buffer(flush_l2, nbytes=FLUSH_BYTES):
    return torch.empty(nbytes // 4, dtype=torch.int32, device="cuda") if flush_l2 else None


def time_ms(fn, warmup=25, reps=100, flush_l2=True):
    """(median ms, stdev ms) of fn() between two events on the current stream."""
    cache = _flush_buffer(flush_l2)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        if cache is not None:
            cache.zero_()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e))
    return statistics.median(out), statistics.stdev(out) if len(out) > 1 else 0.0


def report(rows, cols, title=None, note=None):
    if title:
        print(f"\n{title}")
        print("-" * max(len(title), sum(w for _, w in cols)))
    print("".join(f"{h:>{w}}" for h, w in cols))
    for r in rows:
        print("".join(
            (f"{v:>{w}.{3 if isinstance(v, float) else 0}f}" if isinstance(v, (int, float))
             else f"{str(v):>{w}}")
            for v, (_, w) in zip(r, cols)))
    if note:
        print(f"\n{note}")


def paired_time(fn_a, fn_b, warmup=25, reps=200, flush_l2=True):
    """Interleaved timing of two callables (gpu/bench.py:42-74).

    Returns (median_a, median_b, median of per-pair b/a ratios, stdev of ratios)."""
    cache = _flush_buffer(flush_l2)
    for _ in range(warmup):
        fn_a()
        fn_b()
    torch.cuda.synchronize()
    a_s, b_s, ratios = [], [], []
    for _ in range(reps):
        pair = []
        for fn in (fn_a, fn_b):
            if cache is not None:
                cache.zero_()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            torch.cuda.synchronize()
            pair.append(s.elapsed_time(e))
        a_s.append(pair[0])
        b_s.append(pair[1])
        if pair[0] > 0:
            ratios.append(pair[1] / pair[0])
    return (statistics.median(a_s), statistics.median(b_s), statistics.median(ratios),
            statistics.stdev(ratios) if len(ratios) > 1 else 0.0)
