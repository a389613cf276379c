"""Kernel timer (reference behaviour: ezops/ops/utils/bench.py:24-150).

Protocol: warm up, capture the call into a HIP graph (eager fallback), then
``n_trials`` trials of ``n_repeat`` timed calls, each preceded by a cache
flush; the result is the median trial mean in milliseconds.  How the calls
are timed differs from the reference (``bench_kernel``'s ``method``): the
default times the flush+call graph against the flush-only graph, because an
event pair per call costs ~13 µs on MI355X.

MI355X difference: the reference sizes its flush buffer to
``L2_cache_size``.  Here L2 is 4 MB per XCD but the 256 MB Infinity Cache
(MALL) sits behind it, so a weight of a few hundred MB would stay resident
and the measured GB/s would be inflated.  The flush covers 1 GiB, four times
the MALL.  The flush *reads* the buffer (a sum kernel): a write flush would
leave the MALL full of dirty lines whose write-back then competes with the
kernel being timed.
"""

from __future__ import annotations

from typing import Any, Callable, Optional

import torch

FLUSH_BYTES = 1 << 30

_flush_buf: Optional[torch.Tensor] = None


def flush_cache() -> None:
    """Read 1 GiB on the current stream, evicting L2 and MALL with clean lines."""
    global _flush_buf
    from ... import _hip

    if _flush_buf is None:
        _flush_buf = torch.zeros(FLUSH_BYTES // 4 + 4, dtype=torch.float32, device="cuda")
    n = FLUSH_BYTES // 4
    # kind 0 = read probe; the 4 extra floats receive its (never taken) store
    _hip.call("ezops_hbm_probe", 0, _flush_buf[n:].data_ptr(), _flush_buf.data_ptr(), None, n, 0.0,
              _hip.stream())


def _capture(body):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        body()
    torch.cuda.synchronize()
    return g


def bench_kernel(
    fn: Callable,
    args: tuple[Any, ...] = (),
    n_warmup: int = 10,
    n_repeat: int = 50,
    n_trials: int = 3,
    flush: bool = True,
    use_graph: bool = True,
    method: str = "diff",
) -> float:
    """Median-of-trials mean latency of ``fn(*args)`` in ms, caches cold.

    ``method="diff"`` (default): one graph holds the flush and the call, a
    second the flush alone; a trial alternates ``n_repeat`` replays of each,
    every replay between its own event pair, and returns the median of the
    pairwise differences.
    On MI355X an event pair around nothing reads ~5 µs and a graph replay
    timed alone ~7 µs more (ROCm 7, measured), so the reference's
    per-call event pairs put a ~13 µs floor under every op; in the
    difference both costs appear on each side and cancel, leaving the
    call's own GPU time plus its one dispatch gap.  A cold kernel's own time
    varies from launch to launch (the config-G GEMV: 6.9-10.3 µs per
    dispatch in a kernel trace), so repeated calls of this timer spread by
    about +-1 µs for kernels under ~10 µs; a profiler's kernel trace is the
    precise figure there.
    ``method="events"``: the reference protocol as written (an event pair
    around each replay, flush outside it), floor included.
    Graph capture falls back to eager calls, with a warning."""
    for _ in range(n_warmup):
        if flush:
            flush_cache()
        fn(*args)
    torch.cuda.synchronize()
    if not flush:
        method = "events"

    call = lambda: fn(*args)  # noqa: E731
    both = lambda: (flush_cache(), fn(*args))  # noqa: E731
    run1, run0, run = both, flush_cache, call
    if use_graph:
        try:
            g = _capture(call)
            run = g.replay
            if method == "diff":
                g1, g0 = _capture(both), _capture(flush_cache)
                run1, run0 = g1.replay, g0.replay
        except Exception as e:  # not capturable: time eagerly, say so
            run, run1, run0 = call, both, flush_cache
            print(f"warning: graph capture failed for {getattr(fn, '__name__', fn)!r} "
                  f"({type(e).__name__}: {e}); timing eager launches")
    for _ in range(n_warmup):
        if flush:
            flush_cache()
        run()
        if method == "diff":
            run1()
            run0()
    torch.cuda.synchronize()

    means = []
    for t in range(n_trials):
        if method == "diff":
            # (flush + call) and flush-alone replays alternate, each between
            # its own event pair; a trial is the median of the pairwise
            # differences, so clock drift between the two kinds cancels too
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(2 * n_repeat)]
            for i in range(n_repeat):
                for k, r in ((0, run1), (1, run0)) if (i + t) % 2 == 0 else ((1, run0), (0, run1)):
                    a, b = ev[2 * i + k]
                    a.record()
                    r()
                    b.record()
            torch.cuda.synchronize()
            d = sorted(ev[2 * i][0].elapsed_time(ev[2 * i][1]) - ev[2 * i + 1][0].elapsed_time(ev[2 * i + 1][1])
                       for i in range(n_repeat))
            means.append(d[len(d) // 2])
            continue
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_repeat)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_repeat)]
        for i in range(n_repeat):
            if flush:
                flush_cache()
            starts[i].record()
            run()
            ends[i].record()
        torch.cuda.synchronize()
        ts = [s.elapsed_time(e) for s, e in zip(starts, ends, strict=True)]
        means.append(sum(ts) / len(ts))
    means.sort()
    return means[len(means) // 2]
