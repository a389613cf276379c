"""HIP fp32 row softmax (replaces ezops/kernels/softmax/softmax_cu.py)."""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel


@register_kernel("softmax", "hip")
class SoftmaxHipKernel(BaseKernel):
    def __init__(self, batch_size: int, dim: int):
        if batch_size < 1 or dim < 1:
            raise ValueError(f"batch_size ({batch_size}) and dim ({dim}) must be >= 1")
        self.batch_size, self.dim = batch_size, dim

    def __call__(self, X: torch.Tensor, Out: torch.Tensor) -> None:
        _hip.require_gpu(X, Out)
        shape = (self.batch_size, self.dim)
        _hip.check(X, "X", shape, torch.float32)
        _hip.check(Out, "Out", shape, torch.float32)
        _hip.call("ezops_softmax_f32", X.data_ptr(), Out.data_ptr(), self.batch_size, self.dim,
                  _hip.stream(X.device))
