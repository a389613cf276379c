"""Single-token GQA decode attention over a paged KV cache.

Extension of AttnDecodeOp (reference: ezops/ops/attn_decode.py:9-67, whose
cache is one contiguous ``[B, Hkv, S, D]`` tensor, :60-61).  Here K and V
live in page pools ``[num_pages, Hkv, page_size, D]`` shared by all
sequences; ``block_table [B, max_pages]`` (int32) maps logical page ``j`` of
sequence ``b`` (cache rows ``[j*page_size, (j+1)*page_size)``) to a pool
page, and ``kv_lens [B]`` (int32) bounds each sequence.  The result equals
AttnDecodeOp on the gathered contiguous cache.
"""

import torch

from ..registry import get_kernel
from .attn_decode import gqa_decode_reference
from .base_op import Op, default_device, randn


def paged_to_contiguous(pages, block_table):
    """[num_pages, Hkv, P, D] pool + [B, M] table -> [B, Hkv, M*P, D]."""
    g = pages[block_table.long()]  # [B, M, Hkv, P, D]
    B, M, Hkv, P, D = g.shape
    return g.permute(0, 2, 1, 3, 4).reshape(B, Hkv, M * P, D)


class PagedAttnDecodeOp(Op):
    _params_desc = {
        "batch": "Batch size",
        "num_heads": "Number of attention heads",
        "num_kv_heads": "Number of KV heads",
        "head_dim": "Dimension per head",
        "page_size": "Cache rows per page (power of two >= 32)",
        "max_pages": "Block-table width (pages per sequence)",
        "num_pages": "Pages in the shared pool (default batch * max_pages)",
    }
    _atol = 1e-2
    _rtol = 1e-2

    def __init__(self, batch: int, num_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                 max_pages: int, num_pages: int | None = None, backend: str = "ref"):
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads ({num_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
        if page_size < 32 or page_size & (page_size - 1):
            raise ValueError(f"page_size ({page_size}) must be a power of two >= 32")
        if max_pages < 1:
            raise ValueError("max_pages must be >= 1")
        self.batch, self.num_heads, self.num_kv_heads, self.head_dim = batch, num_heads, num_kv_heads, head_dim
        self.page_size, self.max_pages = page_size, max_pages
        self.num_pages = batch * max_pages if num_pages is None else num_pages
        self._backend = backend
        if backend != "ref":
            self._kernel = get_kernel("paged_attn_decode", backend)(
                batch, num_heads, num_kv_heads, head_dim, page_size, max_pages, self.num_pages)
        else:
            self._kernel = self._ref_forward

    def forward(self, Q, K_pages, V_pages, block_table, kv_lens, max_kv_len: int = 0):
        return self._kernel(Q, K_pages, V_pages, block_table, kv_lens, max_kv_len)

    def gen_data(self, device=None):
        """Random pools, a random page permutation as the block table and
        lengths in [1, max_pages * page_size]."""
        dev = default_device(device)
        shape = (self.num_pages, self.num_kv_heads, self.page_size, self.head_dim)
        Q = randn(self.batch, self.num_heads, 1, self.head_dim, dtype=torch.bfloat16, device=dev)
        Kp = randn(*shape, dtype=torch.bfloat16, device=dev)
        Vp = randn(*shape, dtype=torch.bfloat16, device=dev)
        bt = torch.randperm(self.num_pages, device="cpu")[: self.batch * self.max_pages]
        if bt.numel() < self.batch * self.max_pages:
            bt = torch.randint(0, self.num_pages, (self.batch * self.max_pages,))
        bt = bt.reshape(self.batch, self.max_pages).to(torch.int32).to(dev)
        lens = torch.randint(1, self.max_pages * self.page_size + 1, (self.batch,), dtype=torch.int32).to(dev)
        return Q, Kp, Vp, bt, lens

    def _ref_forward(self, Q, K_pages, V_pages, block_table, kv_lens, max_kv_len=0):
        K = paged_to_contiguous(K_pages, block_table)
        V = paged_to_contiguous(V_pages, block_table)
        lens = kv_lens if max_kv_len <= 0 else kv_lens.clamp(max=max_kv_len)
        return gqa_decode_reference(Q, K, V, lens)
