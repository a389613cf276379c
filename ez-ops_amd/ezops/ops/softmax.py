"""Row softmax spec (reference: ezops/ops/softmax.py:7-34): fp32 ``softmax(X, -1)``."""

import torch

from ..registry import get_kernel
from .base_op import Op, default_device, randn


class SoftmaxOp(Op):
    _params_desc = {
        "batch_size": "Number of rows",
        "dim": "Feature dimension per row (softmax over dim)",
    }
    _atol = 1e-6
    _rtol = 1e-5

    def __init__(self, batch_size: int, dim: int, backend: str = "ref"):
        self.batch_size = batch_size
        self.dim = dim
        self._backend = backend
        if backend != "ref":
            self._kernel = get_kernel("softmax", backend)(batch_size=batch_size, dim=dim)
        else:
            self._kernel = self._ref_forward

    def forward(self, X: torch.Tensor, Out: torch.Tensor) -> None:
        self._kernel(X, Out)

    def gen_data(self, device=None):
        dev = default_device(device)
        X = randn(self.batch_size, self.dim, dtype=torch.float32, device=dev)
        Out = torch.empty(self.batch_size, self.dim, dtype=torch.float32, device=dev)
        return X, Out

    def _ref_forward(self, X: torch.Tensor, Out: torch.Tensor) -> None:
        Out.copy_(torch.softmax(X, dim=-1))
