"""HIP causal GQA prefill attention (MFMA flash attention over the KV cache);
no reference counterpart (the reference is decode-only,
ezops/ops/attn_decode.py:9-67)."""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel


@register_kernel("prefill_attn", "hip")
class PrefillAttnHipKernel(BaseKernel):
    def __init__(self, batch: int, num_heads: int, num_kv_heads: int, head_dim: int, seq_len: int, q_lens,
                 past_lens, page_size: int | None = None, num_pages: int | None = None):
        if head_dim != 128:
            raise ValueError(f"head_dim ({head_dim}) must be 128")
        if num_heads % num_kv_heads or num_heads // num_kv_heads not in (1, 2, 4, 8):
            raise ValueError(f"GQA group size {num_heads}/{num_kv_heads} not supported (1, 2, 4 or 8)")
        self.B, self.H, self.Hkv, self.D, self.S = batch, num_heads, num_kv_heads, head_dim, seq_len
        self.q_lens, self.past_lens = list(q_lens), list(past_lens)
        self.T = sum(self.q_lens)
        self.page_size, self.num_pages = page_size, num_pages
        cu = [0]
        for n in self.q_lens:
            cu.append(cu[-1] + n)
        self._host = (cu, self.past_lens)
        self._dev: dict = {}

    def meta(self, dev):
        """Device copies of cu_seqlens [B+1] and past_lens [B] (int32)."""
        t = self._dev.get(dev)
        if t is None:
            t = tuple(torch.tensor(x, dtype=torch.int32, device=dev) for x in self._host)
            self._dev[dev] = t
        return t

    def __call__(self, Q, K_cache, V_cache, block_table=None):
        paged = self.page_size is not None
        if paged != (block_table is not None):
            raise ValueError("block_table is required with a paged cache and only then")
        dev = _hip.require_gpu(Q, K_cache, V_cache, block_table)
        bf = torch.bfloat16
        _hip.check(Q, "Q", (self.T, self.H, self.D), bf)
        kv_shape = (self.num_pages, self.Hkv, self.page_size, self.D) if paged else (self.B, self.Hkv, self.S, self.D)
        _hip.check(K_cache, "K_cache", kv_shape, bf)
        _hip.check(V_cache, "V_cache", kv_shape, bf)
        if paged:
            _hip.check(block_table, "block_table", (self.B, self.S // self.page_size), torch.int32)
        cu, past = self.meta(dev)
        Out = torch.empty(self.T, self.H, self.D, dtype=bf, device=dev)
        _hip.call("ezops_prefill_attn_bf16", Q.data_ptr(), K_cache.data_ptr(), V_cache.data_ptr(), Out.data_ptr(),
                  cu.data_ptr(), past.data_ptr(), self.B, self.T, self.H, self.Hkv, self.S, self.D,
                  max(self.q_lens, default=0), _hip.ptr(block_table), self.num_pages or 0, self.page_size or 0, 0.0,
                  _hip.stream(dev))
        return Out
