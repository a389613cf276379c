"""Post-attention tail of a Qwen3 dense decoder layer (batch x 1 token).

Reference: ezops/ops/fused_o_proj_ffn.py:8-125.

    x2  = residual + attn @ Wo.T
    xn  = rmsnorm(x2) * post_norm_w            # fp32 stats, eps 1e-6, bf16 out
    out = x2 + (silu(xn @ Wg.T) * (xn @ Wu.T)) @ Wd.T

The reference stages every intermediate in bf16 (:112-125); ``check`` is a
relative Frobenius error below 1e-2 (:51-56).
"""

import torch
import torch.nn.functional as F

from ..registry import get_kernel
from .base_op import Op, default_device, randn


def qwen3_rmsnorm_bf16(x, w, eps):
    """Qwen3RMSNorm: fp32 statistics, ``(x * rsqrt(var+eps) * w).to(x.dtype)``.

    Reference: ezops/ops/fused_o_proj_ffn.py:107-110 (and the unit-weight form
    at ezops/ops/qwen3_dense_decode.py:137-140 when ``w`` is None).
    """
    var = x.to(torch.float32).pow(2).mean(-1, keepdim=True)
    y = x * torch.rsqrt(var + eps)
    if w is not None:
        y = y * w
    return y.to(x.dtype)


def frobenius_ok(actual, expected, rtol) -> bool:
    if actual.shape != expected.shape:
        return False
    diff = (actual.float() - expected.float()).norm().item()
    base = max(expected.float().norm().item(), 1.0)
    return diff / base < rtol


class FusedOProjFfnOp(Op):
    _params_desc = {
        "batch": "Batch size (tokens per decode step)",
        "hidden_size": "Hidden dimension",
        "intermediate_size": "MLP intermediate dimension",
        "num_heads": "Number of query heads (o_proj input width = num_heads * head_dim)",
        "head_dim": "Dimension per head",
    }
    _atol = 1e-2
    _rtol = 1e-2
    rms_eps = 1e-6

    def check(self, actual, expected) -> bool:
        return frobenius_ok(actual, expected, self._rtol)

    def __init__(self, batch: int, hidden_size: int, intermediate_size: int, num_heads: int,
                 head_dim: int, backend: str = "ref"):
        self.batch = batch
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.q_rows = num_heads * head_dim
        self._backend = backend
        if backend != "ref":
            cls = get_kernel("fused_o_proj_ffn", backend)
            self._kernel = cls(batch, hidden_size, intermediate_size, num_heads, head_dim)
        else:
            self._kernel = self._ref_forward

    def forward(self, attn, residual, Wo, post_norm_w, Wg, Wu, Wd):
        return self._kernel(attn, residual, Wo, post_norm_w, Wg, Wu, Wd)

    def gen_data(self, device=None):
        dev = default_device(device)
        bf = dict(dtype=torch.bfloat16, device=dev)
        attn = randn(self.batch, self.q_rows, **bf)
        residual = randn(self.batch, self.hidden_size, **bf)
        Wo = randn(self.hidden_size, self.q_rows, **bf, scale=self.q_rows ** -0.5)
        post_norm_w = randn(self.hidden_size, **bf)
        Wg = randn(self.intermediate_size, self.hidden_size, **bf, scale=self.hidden_size ** -0.5)
        Wu = randn(self.intermediate_size, self.hidden_size, **bf, scale=self.hidden_size ** -0.5)
        Wd = randn(self.hidden_size, self.intermediate_size, **bf, scale=self.intermediate_size ** -0.5)
        return attn, residual, Wo, post_norm_w, Wg, Wu, Wd

    def _ref_forward(self, attn, residual, Wo, post_norm_w, Wg, Wu, Wd):
        x2 = residual + attn @ Wo.T
        xn = qwen3_rmsnorm_bf16(x2, post_norm_w, self.rms_eps)
        gate, up = xn @ Wg.T, xn @ Wu.T
        return x2 + (F.silu(gate) * up) @ Wd.T
