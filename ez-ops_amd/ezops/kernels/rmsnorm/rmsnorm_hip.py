"""HIP RMSNorm (replaces ezops/kernels/rmsnorm/rmsnorm_cu.py)."""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel


@register_kernel("rmsnorm", "hip")
class RmsNormHipKernel(BaseKernel):
    """fp32 ``(X, Out)`` (reference form) or bf16 weighted ``(X, W, Out)``."""

    def __init__(self, batch_size: int, dim: int, eps: float = 1e-6,
                 dtype: torch.dtype = torch.float32, weighted: bool = False):
        if batch_size < 1 or dim < 1:
            raise ValueError(f"batch_size ({batch_size}) and dim ({dim}) must be >= 1")
        if dtype == torch.float32 and weighted:
            raise ValueError("the fp32 RMSNorm kernel has no weight (reference RmsNormOp form)")
        self.batch_size, self.dim, self.eps = batch_size, dim, eps
        self.dtype, self.weighted = dtype, weighted

    def __call__(self, *args) -> None:
        shape = (self.batch_size, self.dim)
        if self.dtype == torch.float32:
            X, Out = args
            _hip.require_gpu(X, Out)
            _hip.check(X, "X", shape, torch.float32)
            _hip.check(Out, "Out", shape, torch.float32)
            _hip.call("ezops_rmsnorm_f32", X.data_ptr(), Out.data_ptr(), self.batch_size, self.dim,
                      self.eps, _hip.stream(X.device))
            return
        if self.weighted:
            X, W, Out = args
        else:
            (X, Out), W = args, None
        _hip.require_gpu(X, W, Out)
        _hip.check(X, "X", shape, torch.bfloat16)
        _hip.check(Out, "Out", shape, torch.bfloat16)
        if W is not None:
            _hip.check(W, "W", (self.dim,), torch.bfloat16)
        _hip.call("ezops_rmsnorm_bf16", X.data_ptr(), _hip.ptr(W), Out.data_ptr(), self.batch_size,
                  self.dim, self.eps, _hip.stream(X.device))
