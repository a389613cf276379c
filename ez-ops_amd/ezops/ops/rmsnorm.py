"""RMSNorm spec (reference: ezops/ops/rmsnorm.py:7-36).

Reference form (default): fp32 ``X [rows, dim]``, no weight,
``Out = X * rsqrt(mean(X^2) + eps)``.

Weighted bf16 form (``dtype=torch.bfloat16, weighted=True``): the Qwen3
RMSNorm of ezops/ops/fused_o_proj_ffn.py:107-110, i.e. fp32 statistics and
``(x * rsqrt(var + eps) * w).to(bf16)``.  In that form the call is
``forward(X, W, Out)``.
"""

import torch

from ..registry import get_kernel
from .base_op import Op, default_device, randn


class RmsNormOp(Op):
    _params_desc = {
        "batch_size": "Number of rows",
        "dim": "Feature dimension per row (normalized over dim)",
    }
    _atol = 1e-5
    _rtol = 1e-5

    def __init__(self, batch_size: int, dim: int, backend: str = "ref", eps: float = 1e-6,
                 *, dtype: torch.dtype = torch.float32, weighted: bool = False):
        if dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"dtype must be float32 or bfloat16, got {dtype}")
        self.batch_size = batch_size
        self.dim = dim
        self.eps = eps
        self.dtype = dtype
        self.weighted = weighted
        if dtype == torch.bfloat16:
            # one bf16 rounding of an O(1) value: a bf16 ulp is up to 2^-7 relative
            self._atol, self._rtol = 2e-2, 1e-2
        self._backend = backend
        if backend != "ref":
            cls = get_kernel("rmsnorm", backend)
            self._kernel = cls(batch_size=batch_size, dim=dim, eps=eps, dtype=dtype, weighted=weighted)
        else:
            self._kernel = self._ref_forward

    def forward(self, *args) -> None:
        self._kernel(*args)

    def gen_data(self, device=None):
        dev = default_device(device)
        X = randn(self.batch_size, self.dim, dtype=self.dtype, device=dev)
        Out = torch.empty(self.batch_size, self.dim, dtype=self.dtype, device=dev)
        if self.weighted:
            W = randn(self.dim, dtype=self.dtype, device=dev, scale=0.1, mean=1.0)
            return X, W, Out
        return X, Out

    def _ref_forward(self, *args) -> None:
        if self.weighted:
            X, W, Out = args
            var = X.to(torch.float32).pow(2).mean(dim=-1, keepdim=True)
            Out.copy_((X * torch.rsqrt(var + self.eps) * W).to(Out.dtype))
        else:
            X, Out = args
            ms = X.pow(2).mean(dim=-1, keepdim=True)
            Out.copy_(X * torch.rsqrt(ms + self.eps))
