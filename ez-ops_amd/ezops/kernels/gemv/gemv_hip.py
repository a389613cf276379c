"""HIP bf16 GEMV (replaces ezops/kernels/gemv/gemv_cu.py:14-25)."""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel


@register_kernel("gemv", "hip")
class GemvHipKernel(BaseKernel):
    """``C[n] = sum_k A[k] * B[n, k]``; A [K], B [N, K], C [N], all bf16."""

    def __init__(self, N: int, K: int):
        if N < 1 or K < 1:
            raise ValueError(f"N ({N}) and K ({K}) must be >= 1")
        self.N, self.K = N, K

    def __call__(self, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor) -> None:
        _hip.require_gpu(A, B, C)
        bf = torch.bfloat16
        _hip.check(A, "A", (self.K,), bf)
        _hip.check(B, "B", (self.N, self.K), bf)
        _hip.check(C, "C", (self.N,), bf)
        _hip.call("ezops_gemv_bf16", A.data_ptr(), B.data_ptr(), C.data_ptr(), self.N, self.K,
                  _hip.stream(A.device))


def linear(X: torch.Tensor, W: torch.Tensor, Y: torch.Tensor | None = None) -> torch.Tensor:
    """``Y = X @ W.T`` for bf16 X [M, K], W [N, K] through ezops_linear_bf16."""
    _hip.require_gpu(X, W)
    M, K = X.shape
    N = W.shape[0]
    _hip.check(W, "W", (N, K), torch.bfloat16)
    if X.dtype != torch.bfloat16 or X.stride(1) != 1:
        raise ValueError("X must be bf16 with unit column stride")
    if Y is None:
        Y = torch.empty(M, N, dtype=torch.bfloat16, device=X.device)
    _hip.call("ezops_linear_bf16", X.data_ptr(), X.stride(0), W.data_ptr(), Y.data_ptr(), Y.stride(0),
              M, N, K, _hip.stream(X.device))
    return Y
