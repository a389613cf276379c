"""HIP fused o_proj + post-norm + SwiGLU FFN (replaces ezops/kernels/fused_o_proj_ffn/*)."""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel

RMS_EPS = 1e-6
TILE = 64  # row/column tiling of the linear kernels


def check_tiles(**dims):
    for name, val in dims.items():
        if val % TILE:
            raise ValueError(f"{name} ({val}) must be divisible by {TILE} for the HIP kernels")


@register_kernel("fused_o_proj_ffn", "hip")
class FusedOProjFfnHipKernel(BaseKernel):
    def __init__(self, batch: int, hidden_size: int, intermediate_size: int, num_heads: int, head_dim: int):
        check_tiles(hidden_size=hidden_size, intermediate_size=intermediate_size,
                    attention_width=num_heads * head_dim)
        self.B, self.HS, self.IS, self.QR = batch, hidden_size, intermediate_size, num_heads * head_dim
        self._ws = _hip.Workspace()

    def __call__(self, attn, residual, Wo, post_norm_w, Wg, Wu, Wd):
        dev = _hip.require_gpu(attn, residual, Wo, post_norm_w, Wg, Wu, Wd)
        bf = torch.bfloat16
        B, HS, IS, QR = self.B, self.HS, self.IS, self.QR
        _hip.check(attn, "attn", (B, QR), bf)
        _hip.check(residual, "residual", (B, HS), bf)
        _hip.check(Wo, "Wo", (HS, QR), bf)
        _hip.check(post_norm_w, "post_norm_w", (HS,), bf)
        _hip.check(Wg, "Wg", (IS, HS), bf)
        _hip.check(Wu, "Wu", (IS, HS), bf)
        _hip.check(Wd, "Wd", (HS, IS), bf)
        out = torch.empty(B, HS, dtype=bf, device=dev)
        ws = self._ws.get(_hip.size("ezops_o_proj_ffn_workspace_size", B, HS, IS, QR), dev)
        _hip.call("ezops_o_proj_ffn_bf16", attn.data_ptr(), residual.data_ptr(), Wo.data_ptr(),
                  post_norm_w.data_ptr(), Wg.data_ptr(), Wu.data_ptr(), Wd.data_ptr(), out.data_ptr(),
                  B, HS, IS, QR, RMS_EPS, ws.data_ptr(), ws.numel(), _hip.stream(dev))
        return out
