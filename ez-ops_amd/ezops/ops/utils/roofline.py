"""Algorithmic flop/byte counting (reference: ezops/ops/utils/roofline.py:1-88).

Flops come from ``torch.utils.flop_counter.FlopCounterMode`` with extra rules
that count one flop per output element for elementwise aten ops and ``2*N*K``
for ``aten.mv``.  Bytes are every tensor argument plus every returned tensor,
i.e. the fused (read-once, write-once) traffic.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch.utils.flop_counter import FlopCounterMode


def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= d
    return n


def _elemwise_flop(*input_shapes, out_shape=None, **kwargs) -> int:
    return _numel(out_shape) if out_shape is not None else 0


def _mv_flop(*input_shapes, out_shape=None, **kwargs) -> int:
    if len(input_shapes) >= 2 and len(input_shapes[0]) == 2:
        rows, cols = input_shapes[0]
        return 2 * rows * cols
    return 0


_aten = torch.ops.aten
_ELEMENTWISE = (
    _aten.add, _aten.sub, _aten.mul, _aten.div, _aten.neg, _aten.abs, _aten.exp,
    _aten.log, _aten.sqrt, _aten.rsqrt, _aten.relu, _aten.sigmoid, _aten.tanh,
    _aten.silu, _aten.gelu, _aten.pow, _aten.copy, _aten.clone, _aten.where,
    _aten.maximum, _aten.minimum,
)

_FLOP_RULES = {op: _elemwise_flop for op in _ELEMENTWISE}
_FLOP_RULES[_aten.mv] = _mv_flop


@dataclass(frozen=True)
class RooflineResult:
    flops: int
    bytes: int
    fused_bytes: int
    arithmetic_intensity: float = 0.0

    def __post_init__(self):
        ai = self.flops / self.bytes if self.bytes > 0 else float("inf")
        object.__setattr__(self, "arithmetic_intensity", ai)


def _returned_bytes(result) -> int:
    if isinstance(result, torch.Tensor):
        return result.nbytes
    if isinstance(result, (tuple, list)):
        return sum(t.nbytes for t in result if isinstance(t, torch.Tensor))
    return 0


def measure_roofline(fn, args: tuple, kwargs: dict) -> RooflineResult:
    with FlopCounterMode(display=False, custom_mapping=_FLOP_RULES) as counter:
        result = fn(*args, **kwargs)
    nbytes = sum(a.nbytes for a in args if isinstance(a, torch.Tensor))
    nbytes += sum(v.nbytes for v in kwargs.values() if isinstance(v, torch.Tensor))
    nbytes += _returned_bytes(result)
    return RooflineResult(flops=counter.get_total_flops(), bytes=nbytes, fused_bytes=nbytes)
