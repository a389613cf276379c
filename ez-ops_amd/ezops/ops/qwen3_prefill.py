"""Prefill of one Qwen3 dense decoder layer: the step before decode.

No reference counterpart (the reference is decode only,
ezops/ops/qwen3_dense_decode.py:9-176); this op fills the KV cache that
Qwen3DenseDecodeOp then reads, with the same stages applied to every new
token:

    x        = rmsnorm(hidden) * in_norm_w              # hidden [T, HS]
    q, k, v  = x @ Wqkv.T
    q, k     = RoPE(rmsnorm(q) * q_norm_w), RoPE(rmsnorm(k) * k_norm_w)  at pos
    cache[b, :, pos] = k, v                             # pos = past_lens[b] + i
    attn     = causal GQA attention of q over cache rows [0, pos]
    h        = hidden + attn @ Wo.T
    out      = h + (silu(rmsnorm(h) @ Wg.T) * (rmsnorm(h) @ Wu.T)) @ Wd.T

``hidden [T, HS]`` holds the sequences' new tokens back to back
(``q_lens[b]`` each).  Options as in Qwen3DenseDecodeOp (``norm_weights``,
``rope_theta``, ``page_size`` / ``num_pages`` with the block table as the
last input).
"""

import torch
import torch.nn.functional as F

from ..registry import get_kernel
from .base_op import Op, default_device, randn
from .fused_o_proj_ffn import frobenius_ok, qwen3_rmsnorm_bf16
from .fused_qk_norm_rope import head_rmsnorm_f32, rope_half_f32, rope_tables
from .paged_attn_decode import paged_to_contiguous
from .prefill_attn import prefill_attn_reference


class Qwen3PrefillOp(Op):
    _params_desc = {
        "batch": "Sequences in the chunk",
        "seq_len": "KV cache capacity per sequence",
        "hidden_size": "Hidden dimension",
        "intermediate_size": "MLP intermediate dimension",
        "num_heads": "Query heads",
        "head_dim": "Dimension per head",
        "q_lens": "New tokens per sequence",
        "past_lens": "Cache rows before the chunk, per sequence (default 0)",
        "num_kv_heads": "KV heads (default: num_heads)",
    }
    _atol = 1e-2
    _rtol = 1e-2
    rms_eps = 1e-6

    def check(self, actual, expected) -> bool:
        return frobenius_ok(actual, expected, self._rtol)

    def __init__(self, batch: int, seq_len: int, hidden_size: int, intermediate_size: int, num_heads: int,
                 head_dim: int, q_lens, past_lens=None, backend: str = "ref", num_kv_heads: int | None = None, *,
                 norm_weights: bool = False, rope_theta: float | None = None, page_size: int | None = None,
                 num_pages: int | None = None):
        num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads ({num_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
        q_lens = [int(x) for x in q_lens]
        past_lens = [0] * batch if past_lens is None else [int(x) for x in past_lens]
        if len(q_lens) != batch or len(past_lens) != batch:
            raise ValueError("q_lens and past_lens need one entry per sequence")
        if sum(q_lens) < 1:
            raise ValueError("the chunk needs at least one token")
        for n, p in zip(q_lens, past_lens):
            if n < 0 or p < 0 or n + p > seq_len:
                raise ValueError(f"q_len {n} + past_len {p} must fit the cache capacity {seq_len}")
        if page_size is not None:
            if page_size < 32 or page_size & (page_size - 1) or seq_len % page_size:
                raise ValueError(f"page_size ({page_size}) must be a power of two >= 32 dividing seq_len ({seq_len})")
            num_pages = batch * (seq_len // page_size) if num_pages is None else num_pages
        self.batch, self.seq_len, self.hidden_size, self.intermediate_size = batch, seq_len, hidden_size, intermediate_size
        self.num_heads, self.head_dim, self.num_kv_heads = num_heads, head_dim, num_kv_heads
        self.q_lens, self.past_lens = q_lens, past_lens
        self.norm_weights, self.rope_theta = norm_weights, rope_theta
        self.page_size, self.num_pages = page_size, num_pages
        self.q_rows, self.kv_rows = num_heads * head_dim, num_kv_heads * head_dim
        self._backend = backend
        if backend != "ref":
            self._kernel = get_kernel("qwen3_dense_prefill", backend)(
                batch, seq_len, hidden_size, intermediate_size, num_heads, head_dim, q_lens, past_lens,
                num_kv_heads=num_kv_heads, norm_weights=norm_weights, rope_theta=rope_theta, page_size=page_size,
                num_pages=num_pages)
        else:
            self._kernel = self._ref_forward

    def forward(self, hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra):
        return self._kernel(hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra)

    def gen_data(self, device=None):
        dev = default_device(device)
        bf = dict(dtype=torch.bfloat16, device=dev)
        HS, IS, T = self.hidden_size, self.intermediate_size, sum(self.q_lens)
        if self.page_size is None:
            kv_shape = (self.batch, self.num_kv_heads, self.seq_len, self.head_dim)
        else:
            kv_shape = (self.num_pages, self.num_kv_heads, self.page_size, self.head_dim)
        data = [randn(T, HS, **bf), randn(*kv_shape, **bf), randn(*kv_shape, **bf),
                randn(self.q_rows + 2 * self.kv_rows, HS, **bf, scale=HS ** -0.5),
                randn(HS, self.q_rows, **bf, scale=self.q_rows ** -0.5), randn(2 * IS, HS, **bf, scale=HS ** -0.5),
                randn(HS, IS, **bf, scale=IS ** -0.5)]
        if self.norm_weights:
            for n in (HS, self.head_dim, self.head_dim, HS):
                data.append(randn(n, **bf, scale=0.1, mean=1.0))
        if self.rope_theta is not None:
            data += list(rope_tables(self.seq_len, self.head_dim, self.rope_theta, dev))
        if self.page_size is not None:
            M = self.seq_len // self.page_size
            n = self.batch * M
            ids = torch.randperm(self.num_pages)[:n] if self.num_pages >= n else torch.randint(0, self.num_pages, (n,))
            data.append(ids.reshape(self.batch, M).to(torch.int32).to(dev))
        return tuple(data)

    def _ref_forward(self, hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra):
        extra = list(extra)
        bt = extra.pop() if self.page_size is not None else None
        rope = extra[-2:] if self.rope_theta is not None else None
        nw = extra[:4] if self.norm_weights else [None] * 4
        in_w, q_w, k_w, post_w = nw
        T, D, dev, eps = hidden.shape[0], self.head_dim, hidden.device, self.rms_eps
        seq = torch.repeat_interleave(torch.arange(self.batch, device=dev),
                                      torch.tensor(self.q_lens, device=dev))
        pos = torch.cat([p + torch.arange(n, device=dev) for n, p in zip(self.q_lens, self.past_lens)])
        x = qwen3_rmsnorm_bf16(hidden, in_w, eps)
        qkv = x @ Wqkv.T
        q = qkv[:, : self.q_rows].view(T, self.num_heads, D)
        k = qkv[:, self.q_rows: self.q_rows + self.kv_rows].view(T, self.num_kv_heads, D)
        v = qkv[:, self.q_rows + self.kv_rows:].view(T, self.num_kv_heads, D)
        ones = torch.ones(D, dtype=hidden.dtype, device=dev)
        qn = head_rmsnorm_f32(q, ones if q_w is None else q_w, eps)
        kn = head_rmsnorm_f32(k, ones if k_w is None else k_w, eps)
        if rope is not None:
            cp, sp = rope[0][pos].float()[:, None, :], rope[1][pos].float()[:, None, :]
            q, k = rope_half_f32(qn, cp, sp), rope_half_f32(kn, cp, sp)
        else:
            q, k = qn.to(hidden.dtype), kn.to(hidden.dtype)
        if bt is None:
            K_cache[seq, :, pos] = k
            V_cache[seq, :, pos] = v
            Kc, Vc = K_cache, V_cache
        else:
            page = bt.long()[seq, pos // self.page_size]
            K_cache[page, :, pos % self.page_size] = k
            V_cache[page, :, pos % self.page_size] = v
            Kc, Vc = paged_to_contiguous(K_cache, bt), paged_to_contiguous(V_cache, bt)
        attn = prefill_attn_reference(q, Kc, Vc, self.q_lens, self.past_lens)
        h = hidden + attn.reshape(T, self.q_rows) @ Wo.T
        xn = qwen3_rmsnorm_bf16(h, post_w, eps)
        gu = xn @ Wgu.T
        gate, up = gu[:, : self.intermediate_size], gu[:, self.intermediate_size:]
        return h + (F.silu(gate) * up) @ Wd.T
