"""HIP deterministic fp32 full sum (replaces ezops/kernels/reduce/reduce_cu.py)."""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel


@register_kernel("reduce", "hip")
class ReduceHipKernel(BaseKernel):
    def __init__(self, n: int):
        if n < 1:
            raise ValueError(f"n ({n}) must be >= 1")
        self.n = n
        self._ws = _hip.Workspace()

    def __call__(self, A: torch.Tensor, Out: torch.Tensor) -> None:
        dev = _hip.require_gpu(A, Out)
        _hip.check(A, "A", (self.n,), torch.float32)
        _hip.check(Out, "Out", (1,), torch.float32)
        nbytes = _hip.size("ezops_reduce_sum_workspace_size", self.n)
        ws = self._ws.get(nbytes, dev)
        _hip.call("ezops_reduce_sum_f32", A.data_ptr(), Out.data_ptr(), self.n, ws.data_ptr(), ws.numel(),
                  _hip.stream(dev))
