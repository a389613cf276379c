"""bf16 GEMV spec (reference: ezops/ops/gemv.py:7-38).

``C[n] = sum_k A[k] * B[n, k]`` with fp32 accumulation and one bf16 rounding.
As in the reference, the ``ref`` backend receives B as ``[K, N]`` (so
``_ref_forward`` is ``A @ B``) while kernel backends receive B as ``[N, K]``
(row-major weight, one row per output).
"""

import torch

from ..registry import get_kernel
from .base_op import Op, default_device, randn


class GemvOp(Op):
    _params_desc = {
        "N": "Number of columns of C",
        "K": "Reduction dimension (A cols, B rows)",
    }
    _atol = 1e-2
    _rtol = 1e-2

    def __init__(self, N: int, K: int, backend: str = "ref"):
        self.N = N
        self.K = K
        self._backend = backend
        if backend != "ref":
            self._kernel = get_kernel("gemv", backend)(N=N, K=K)
        else:
            self._kernel = self._ref_forward

    def forward(self, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor) -> None:
        self._kernel(A, B, C)

    def gen_data(self, device=None):
        dev = default_device(device)
        A = randn(self.K, dtype=torch.bfloat16, device=dev)
        shape = (self.K, self.N) if self._backend == "ref" else (self.N, self.K)
        B = randn(*shape, dtype=torch.bfloat16, device=dev)
        C = torch.empty(self.N, dtype=torch.bfloat16, device=dev)
        return A, B, C

    def _ref_forward(self, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor) -> None:
        C.copy_(A @ B)
