"""Judge-style accuracy helpers (reference: ezops/ops/utils/accuracy.py:19-78).

``sqnr_db`` (pass mark 28 dB), byte-exact ``check_determinism`` over two
calls, and ``check_input_readonly``.
"""

from __future__ import annotations

import math
from collections.abc import Callable, Iterable

import torch

SQNR_THRESHOLD_DB = 28.0


def sqnr_db(ref: torch.Tensor, out: torch.Tensor) -> float:
    """10*log10(||ref||^2 / ||ref-out||^2); inf when bitwise equal."""
    r = ref.detach().double()
    noise = (r - out.detach().double()).pow(2).sum().item()
    if noise == 0.0:
        return math.inf
    return 10.0 * math.log10(r.pow(2).sum().item() / noise)


def _bytes(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().reshape(-1).view(torch.uint8)


def bitwise_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Byte-for-byte equality (tells -0.0 from +0.0 and NaN payloads apart)."""
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    return bool(torch.equal(_bytes(a), _bytes(b)))


def _tup(x) -> tuple:
    return (x,) if isinstance(x, torch.Tensor) else tuple(x)


def check_determinism(fn: Callable, inputs: Iterable[torch.Tensor], outputs) -> bool:
    ins, outs = _tup(inputs), _tup(outputs)
    fn(*ins, *outs)
    first = [o.clone() for o in outs]
    fn(*ins, *outs)
    return all(bitwise_equal(o, f) for o, f in zip(outs, first, strict=True))


def check_input_readonly(fn: Callable, inputs: Iterable[torch.Tensor], outputs) -> bool:
    ins, outs = _tup(inputs), _tup(outputs)
    before = [i.clone() for i in ins]
    fn(*ins, *outs)
    return all(bitwise_equal(i, b) for i, b in zip(ins, before, strict=True))
