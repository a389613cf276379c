"""HIP split-KV GQA decode attention over a paged KV cache.

The attention kernel of attn_decode_hip with its K/V tile addressing routed
through a block table; it extends the reference's AttnDecodeOp
(ezops/ops/attn_decode.py:9-67), which has no paged cache.
"""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel


@register_kernel("paged_attn_decode", "hip")
class PagedAttnDecodeHipKernel(BaseKernel):
    def __init__(self, batch: int, num_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                 max_pages: int, num_pages: int):
        if num_heads % num_kv_heads or num_heads // num_kv_heads not in (1, 2, 4, 8, 16):
            raise ValueError(f"GQA group size {num_heads}/{num_kv_heads} not supported (1, 2, 4, 8 or 16)")
        if head_dim not in (64, 128):
            raise ValueError(f"head_dim ({head_dim}) must be 64 or 128")
        if page_size < 32 or page_size & (page_size - 1):
            raise ValueError(f"page_size ({page_size}) must be a power of two >= 32")
        if batch < 1 or max_pages < 1 or num_pages < 1:
            raise ValueError("batch, max_pages and num_pages must be >= 1")
        self.B, self.H, self.Hkv, self.D = batch, num_heads, num_kv_heads, head_dim
        self.P, self.M, self.NP = page_size, max_pages, num_pages
        self._ws = _hip.Workspace()

    def __call__(self, Q: torch.Tensor, K_pages: torch.Tensor, V_pages: torch.Tensor, block_table: torch.Tensor,
                 kv_lens: torch.Tensor, max_kv_len: int = 0):
        if max_kv_len < 0:
            raise ValueError(f"max_kv_len ({max_kv_len}) must be >= 0")
        dev = _hip.require_gpu(Q, K_pages, V_pages, block_table, kv_lens)
        bf = torch.bfloat16
        _hip.check(Q, "Q", (self.B, self.H, 1, self.D), bf)
        _hip.check(K_pages, "K_pages", (self.NP, self.Hkv, self.P, self.D), bf)
        _hip.check(V_pages, "V_pages", (self.NP, self.Hkv, self.P, self.D), bf)
        _hip.check(block_table, "block_table", (self.B, self.M), torch.int32)
        _hip.check(kv_lens, "kv_lens", (self.B,), torch.int32)
        Out = torch.empty(self.B, self.H, 1, self.D, dtype=bf, device=dev)
        S = self.M * self.P
        ws = self._ws.get(_hip.size("ezops_attn_decode_workspace_size", self.B, self.H, self.Hkv, S, self.D), dev)
        _hip.call("ezops_paged_attn_decode_bf16", Q.data_ptr(), K_pages.data_ptr(), V_pages.data_ptr(),
                  Out.data_ptr(), block_table.data_ptr(), kv_lens.data_ptr(), self.B, self.H, self.Hkv, self.D,
                  self.NP, self.P, self.M, int(max_kv_len), 0.0, ws.data_ptr(), ws.numel(), _hip.stream(dev))
        return Out
