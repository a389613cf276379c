"""Full fp32 sum spec (reference: ezops/ops/reduce.py:7-31).

``Out[0] = sum(A)``; the absolute tolerance scales as ``1e-7 * n`` because
summation order differs between backends (reduce.py:13-15).
"""

import torch

from ..registry import get_kernel
from .base_op import Op, default_device, randn


class ReduceOp(Op):
    _params_desc = {"n": "Number of input elements"}

    def __init__(self, n: int, backend: str = "ref"):
        self.n = n
        self._backend = backend
        self._atol = 1e-7 * n
        if backend != "ref":
            self._kernel = get_kernel("reduce", backend)(n=n)
        else:
            self._kernel = self._ref_forward

    def forward(self, A: torch.Tensor, Out: torch.Tensor) -> None:
        self._kernel(A, Out)

    def gen_data(self, device=None):
        dev = default_device(device)
        A = randn(self.n, dtype=torch.float32, device=dev)
        Out = torch.empty(1, dtype=torch.float32, device=dev)
        return A, Out

    def _ref_forward(self, A: torch.Tensor, Out: torch.Tensor) -> None:
        Out.copy_(A.sum())
