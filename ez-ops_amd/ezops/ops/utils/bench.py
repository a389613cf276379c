"""Kernel timer (reference behaviour: ezops/ops/utils/bench.py:24-150).

Protocol: warm up, capture the call into a HIP graph (eager fallback), then
``n_trials`` trials of ``n_repeat`` event-timed replays, each preceded by a
cache flush outside the timed region; the result is the median trial mean in
milliseconds.

MI355X difference: the reference sizes its flush buffer to
``L2_cache_size``.  Here L2 is 4 MB per XCD but the 256 MB Infinity Cache
(MALL) sits behind it, so a weight of a few hundred MB would stay resident
and the measured GB/s would be inflated.  The flush writes 1 GiB, four times
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


def bench_kernel(
    fn: Callable,
    args: tuple[Any, ...] = (),
    n_warmup: int = 10,
    n_repeat: int = 50,
    n_trials: int = 3,
    flush: bool = True,
    use_graph: bool = True,
) -> float:
    """Median-of-trials mean latency of ``fn(*args)`` in ms."""
    for _ in range(n_warmup):
        if flush:
            flush_cache()
        fn(*args)
    torch.cuda.synchronize()

    graph = None
    if use_graph:
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn(*args)
            torch.cuda.synchronize()
            graph = g
        except Exception as e:  # not capturable: time eagerly, say so
            graph = None
            print(f"warning: graph capture failed for {getattr(fn, '__name__', fn)!r} "
                  f"({type(e).__name__}: {e}); timing eager launches")
    run = graph.replay if graph is not None else (lambda: fn(*args))
    if graph is not None:
        for _ in range(n_warmup):
            if flush:
                flush_cache()
            run()
        torch.cuda.synchronize()

    means = []
    for _ in range(n_trials):
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
