"""Op base class (reference: ezops/ops/base_op.py:8-33).

An op is a shape-specialised spec: ``forward`` dispatches to the registered
backend kernel (or to ``_ref_forward`` when ``backend == "ref"``),
``gen_data`` makes a seeded workload, ``check`` is the tolerance test and
``get_roofline`` counts algorithmic flops/bytes of ``_ref_forward``.
"""

from abc import ABC, abstractmethod

import torch

from .utils.roofline import RooflineResult, measure_roofline


class Op(ABC):
    _backend: str
    _atol: float = 1e-6
    _rtol: float = 1e-5
    _params_desc: dict[str, str] = {}

    @abstractmethod
    def forward(self, *args, **kwargs): ...

    @abstractmethod
    def _ref_forward(self, *args, **kwargs): ...

    @abstractmethod
    def gen_data(self, device=None): ...

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def get_roofline(self) -> RooflineResult:
        # Shapes alone fix the counts, so the count runs on meta tensors
        # (no allocation, works without a GPU).
        data = self.gen_data(device="meta")
        if not isinstance(data, tuple):
            data = (data,)
        return measure_roofline(self._ref_forward, data, {})

    def check(self, actual, expected) -> bool:
        return torch.allclose(actual, expected, atol=self._atol, rtol=self._rtol)


def default_device(device):
    """Device that ``gen_data`` places tensors on (the reference hard-codes cuda)."""
    return torch.device("cuda") if device is None else torch.device(device)


def randn(*shape, dtype, device, scale=None, mean=None):
    """Seeded normal sample drawn on the CPU generator, then moved to ``device``.

    Drawing on the CPU keeps the values identical for a GPU run and for the
    CPU oracle that checks it, under ``torch.manual_seed``.
    """
    if torch.device(device).type == "meta":
        return torch.empty(*shape, dtype=dtype, device="meta")
    t = torch.randn(*shape, dtype=torch.float32)
    if scale is not None:
        t.mul_(scale)
    if mean is not None:
        t.add_(mean)
    return t.to(dtype).to(device)
