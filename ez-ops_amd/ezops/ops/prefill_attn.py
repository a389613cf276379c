"""Causal GQA prefill attention over the KV cache (the step before decode).

No reference counterpart (the reference is decode-only,
ezops/ops/attn_decode.py:9-67); this op produces the cache state that decode
then reads.  Sequence ``b`` contributes ``q_lens[b]`` new tokens, stored back
to back as rows of ``Q [T, H, D]`` (``T = sum(q_lens)``); they already sit at
cache rows ``past_lens[b] + i`` and token ``i`` attends rows
``[0, past_lens[b] + i]``.  Per token this is AttnDecodeOp's formula with
``kv_len = past + i + 1``.  The cache is ``[B, Hkv, S, D]``, or, with
``page_size``, page pools ``[num_pages, Hkv, page_size, D]`` addressed by a
block table ``[B, S / page_size]`` passed as the last input.
"""

import torch

from ..registry import get_kernel
from .base_op import Op, default_device, randn
from .paged_attn_decode import paged_to_contiguous


def prefill_attn_reference(Q, K, V, q_lens, past_lens):
    """fp32 causal attention, per sequence; Q [T,H,D], K/V [B,Hkv,S,D] -> [T,H,D] bf16."""
    T, H, D = Q.shape
    Hkv = K.shape[1]
    G = H // Hkv
    out = torch.empty(T, H, D, dtype=Q.dtype, device=Q.device)
    t0 = 0
    for b, (n, p) in enumerate(zip(q_lens, past_lens)):
        L = p + n
        q = Q[t0:t0 + n].float().reshape(n, Hkv, G, D).permute(1, 2, 0, 3)
        k = K[b, :, :L].float()[:, None]
        v = V[b, :, :L].float()[:, None]
        s = (q @ k.transpose(-1, -2)) * D ** -0.5
        mask = torch.arange(L, device=Q.device)[None, :] > (p + torch.arange(n, device=Q.device))[:, None]
        s = s.masked_fill(mask, float("-inf"))
        o = torch.softmax(s, dim=-1) @ v
        out[t0:t0 + n] = o.permute(2, 0, 1, 3).reshape(n, H, D).to(Q.dtype)
        t0 += n
    return out


class PrefillAttnOp(Op):
    _params_desc = {
        "batch": "Sequences in the chunk",
        "num_heads": "Query heads",
        "num_kv_heads": "KV heads",
        "head_dim": "Dimension per head",
        "seq_len": "KV cache capacity per sequence",
        "q_lens": "New tokens per sequence",
        "past_lens": "Cache rows before the chunk, per sequence (default 0)",
    }
    _atol = 1e-2
    _rtol = 1e-2

    def __init__(self, batch: int, num_heads: int, num_kv_heads: int, head_dim: int, seq_len: int, q_lens,
                 past_lens=None, backend: str = "ref", *, page_size: int | None = None,
                 num_pages: int | None = None):
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads ({num_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
        q_lens = [int(x) for x in q_lens]
        past_lens = [0] * batch if past_lens is None else [int(x) for x in past_lens]
        if len(q_lens) != batch or len(past_lens) != batch:
            raise ValueError("q_lens and past_lens need one entry per sequence")
        for n, p in zip(q_lens, past_lens):
            if n < 0 or p < 0 or n + p > seq_len:
                raise ValueError(f"q_len {n} + past_len {p} must fit the cache capacity {seq_len}")
        if page_size is not None:
            if page_size < 32 or page_size & (page_size - 1) or seq_len % page_size:
                raise ValueError(f"page_size ({page_size}) must be a power of two >= 32 dividing seq_len ({seq_len})")
            num_pages = batch * (seq_len // page_size) if num_pages is None else num_pages
        self.batch, self.num_heads, self.num_kv_heads, self.head_dim = batch, num_heads, num_kv_heads, head_dim
        self.seq_len, self.q_lens, self.past_lens = seq_len, q_lens, past_lens
        self.page_size, self.num_pages = page_size, num_pages
        self._backend = backend
        if backend != "ref":
            self._kernel = get_kernel("prefill_attn", backend)(
                batch, num_heads, num_kv_heads, head_dim, seq_len, q_lens, past_lens, page_size=page_size,
                num_pages=num_pages)
        else:
            self._kernel = self._ref_forward

    def forward(self, Q, K_cache, V_cache, block_table=None):
        return self._kernel(Q, K_cache, V_cache, block_table)

    def gen_data(self, device=None):
        dev = default_device(device)
        bf = dict(dtype=torch.bfloat16, device=dev)
        T = sum(self.q_lens)
        Q = randn(T, self.num_heads, self.head_dim, **bf)
        if self.page_size is None:
            shape = (self.batch, self.num_kv_heads, self.seq_len, self.head_dim)
        else:
            shape = (self.num_pages, self.num_kv_heads, self.page_size, self.head_dim)
        data = [Q, randn(*shape, **bf), randn(*shape, **bf)]
        if self.page_size is not None:
            M = self.seq_len // self.page_size
            n = self.batch * M
            ids = torch.randperm(self.num_pages)[:n] if self.num_pages >= n else torch.randint(0, self.num_pages, (n,))
            data.append(ids.reshape(self.batch, M).to(torch.int32).to(dev))
        return tuple(data)

    def _ref_forward(self, Q, K_cache, V_cache, block_table=None):
        if self.page_size is not None:
            K_cache, V_cache = paged_to_contiguous(K_cache, block_table), paged_to_contiguous(V_cache, block_table)
        return prefill_attn_reference(Q, K_cache, V_cache, self.q_lens, self.past_lens)
