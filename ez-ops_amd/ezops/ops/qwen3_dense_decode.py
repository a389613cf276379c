"""One decode step of a Qwen3 dense decoder layer (batch x 1 token).

Reference: ezops/ops/qwen3_dense_decode.py:9-176 (reference mode, default):

    x        = rmsnorm(hidden)                         # unit weight, eps 1e-6
    q, k, v  = x @ Wqkv.T                              # fused rows [q | k | v]
    q, k     = rmsnorm(q), rmsnorm(k) over head_dim
    K_cache[:, :, S-1] = k ; V_cache[:, :, S-1] = v
    attn     = GQA softmax(q K^T / sqrt(D)) V over all S slots
    h        = hidden + attn @ Wo.T
    out      = h + (silu(rmsnorm(h) @ Wg.T) * (rmsnorm(h) @ Wu.T)) @ Wd.T

with every intermediate staged in bf16 and a Frobenius check (:64-69).

Qwen3 mode (keyword-only ctor options, for the Qwen3-8B benchmark config):
  * ``kv_lens``: one length per sequence (1 <= len <= seq_len).  The new
    token sits at slot/position ``kv_lens[b] - 1`` and attention covers
    ``[0, kv_lens[b])``.  Default: ``seq_len`` for every sequence (reference).
  * ``norm_weights=True``: input/q/k/post RMSNorm weights are inputs
    (``forward(..., in_norm_w, q_norm_w, k_norm_w, post_norm_w)``).
  * ``rope_theta``: apply half-split RoPE to q and k at the token position
    using HF bf16 cos/sin tables passed after the norm weights
    (``forward(..., cos, sin)``); q/k norm + RoPE then follow the fused
    QK-norm+RoPE stage exactly (fp32 pipeline, one bf16 rounding,
    ezops/ops/fused_qk_norm_rope.py:138-169).
  * ``page_size`` (extension, no reference counterpart): the cache is paged.
    ``K_cache`` / ``V_cache`` are page pools ``[num_pages, Hkv, page_size, D]``
    (``num_pages`` default ``batch * seq_len / page_size``) and ``forward``
    takes the int32 block table ``[batch, seq_len / page_size]`` as its last
    input; logical page ``j`` of sequence ``b`` is pool page
    ``block_table[b, j]``.  Requires ``kv_lens``.
"""

from collections.abc import Sequence

import torch
import torch.nn.functional as F

from ..registry import get_kernel
from .attn_decode import gqa_decode_reference
from .base_op import Op, default_device, randn
from .fused_o_proj_ffn import frobenius_ok, qwen3_rmsnorm_bf16
from .fused_qk_norm_rope import head_rmsnorm_f32, rope_half_f32, rope_tables


class Qwen3DenseDecodeOp(Op):
    _params_desc = {
        "batch": "Batch size (tokens per decode step)",
        "seq_len": "KV cache length; the last slot holds the token being decoded",
        "hidden_size": "Hidden dimension",
        "intermediate_size": "MLP intermediate dimension",
        "num_heads": "Number of query heads",
        "head_dim": "Dimension per head",
        "num_kv_heads": "Number of KV heads for GQA (default: num_heads)",
    }
    _atol = 1e-2
    _rtol = 1e-2
    rms_eps = 1e-6

    def check(self, actual, expected) -> bool:
        return frobenius_ok(actual, expected, self._rtol)

    def __init__(self, batch: int, seq_len: int, hidden_size: int, intermediate_size: int,
                 num_heads: int, head_dim: int, backend: str = "ref",
                 num_kv_heads: int | None = None, *, kv_lens=None,
                 norm_weights: bool = False, rope_theta: float | None = None,
                 page_size: int | None = None, num_pages: int | None = None):
        if seq_len < 1:
            raise ValueError(f"seq_len ({seq_len}) must be >= 1")
        self.batch = batch
        self.seq_len = seq_len
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if num_heads % self.num_kv_heads != 0:
            raise ValueError(
                f"num_heads ({num_heads}) must be divisible by num_kv_heads ({self.num_kv_heads})"
            )
        if rope_theta is not None and head_dim % 2:
            raise ValueError(f"head_dim ({head_dim}) must be even for RoPE")
        if kv_lens is not None:
            kv_lens = [int(x) for x in (kv_lens.tolist() if isinstance(kv_lens, torch.Tensor) else kv_lens)]
            if len(kv_lens) != batch:
                raise ValueError(f"kv_lens has {len(kv_lens)} entries, expected batch={batch}")
            for n in kv_lens:
                if not 1 <= n <= seq_len:
                    raise ValueError(f"kv_lens entry {n} must be in [1, {seq_len}]")
        self.kv_lens = kv_lens
        if page_size is not None:
            if page_size < 32 or page_size & (page_size - 1) or seq_len % page_size:
                raise ValueError(f"page_size ({page_size}) must be a power of two >= 32 dividing seq_len ({seq_len})")
            if kv_lens is None:
                raise ValueError("a paged cache requires kv_lens")
            num_pages = batch * (seq_len // page_size) if num_pages is None else num_pages
            if num_pages < 1:
                raise ValueError("num_pages must be >= 1")
        self.page_size, self.num_pages = page_size, num_pages
        self.norm_weights = norm_weights
        self.rope_theta = rope_theta
        self.q_rows = num_heads * head_dim
        self.kv_rows = self.num_kv_heads * head_dim
        self._backend = backend
        if backend != "ref":
            cls = get_kernel("qwen3_dense_decode", backend)
            self._kernel = cls(batch, seq_len, hidden_size, intermediate_size, num_heads, head_dim,
                               num_kv_heads=self.num_kv_heads, kv_lens=kv_lens,
                               norm_weights=norm_weights, rope_theta=rope_theta,
                               **({} if page_size is None else {"page_size": page_size, "num_pages": num_pages}))
        else:
            self._kernel = self._ref_forward

    def forward(self, hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra):
        return self._kernel(hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra)

    def lens(self) -> list[int]:
        return self.kv_lens if self.kv_lens is not None else [self.seq_len] * self.batch

    def gen_data(self, device=None):
        dev = default_device(device)
        bf = dict(dtype=torch.bfloat16, device=dev)
        H, I = self.hidden_size, self.intermediate_size
        hidden = randn(self.batch, H, **bf)
        if self.page_size is None:
            kv_shape = (self.batch, self.num_kv_heads, self.seq_len, self.head_dim)
        else:
            kv_shape = (self.num_pages, self.num_kv_heads, self.page_size, self.head_dim)
        K_cache = randn(*kv_shape, **bf)
        V_cache = randn(*kv_shape, **bf)
        Wqkv = randn(self.q_rows + 2 * self.kv_rows, H, **bf, scale=H ** -0.5)
        Wo = randn(H, self.q_rows, **bf, scale=self.q_rows ** -0.5)
        Wgu = randn(2 * I, H, **bf, scale=H ** -0.5)
        Wd = randn(H, I, **bf, scale=I ** -0.5)
        data = [hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd]
        if self.norm_weights:
            for n in (H, self.head_dim, self.head_dim, H):
                data.append(randn(n, **bf, scale=0.1, mean=1.0))
        if self.rope_theta is not None:
            if dev.type == "meta":
                data += [torch.empty(self.seq_len, self.head_dim, **bf)] * 2
            else:
                data += list(rope_tables(self.seq_len, self.head_dim, self.rope_theta, dev))
        if self.page_size is not None:
            M = self.seq_len // self.page_size
            n = self.batch * M
            ids = torch.randperm(self.num_pages)[:n] if self.num_pages >= n else torch.randint(0, self.num_pages, (n,))
            data.append(ids.reshape(self.batch, M).to(torch.int32).to(dev))
        return tuple(data)

    def _split_extra(self, extra):
        extra = list(extra)
        want = (4 if self.norm_weights else 0) + (2 if self.rope_theta is not None else 0)
        if len(extra) != want:
            raise ValueError(f"expected {want} extra inputs (norm weights / rope tables), got {len(extra)}")
        nw = extra[:4] if self.norm_weights else [None] * 4
        rope = extra[-2:] if self.rope_theta is not None else None
        return nw, rope

    def _ref_forward(self, hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra):
        if self.page_size is not None:
            # gather the sequences' pages, run the contiguous step, and write
            # the decoded token's rows back to their pool pages
            from .paged_attn_decode import paged_to_contiguous

            *extra, bt = extra
            Kc, Vc = paged_to_contiguous(K_cache, bt).clone(), paged_to_contiguous(V_cache, bt).clone()
            out = self._ref_contiguous(hidden, Kc, Vc, Wqkv, Wo, Wgu, Wd, *extra)
            pos = torch.tensor(self.lens(), dtype=torch.long, device=hidden.device) - 1
            b = torch.arange(hidden.shape[0], device=hidden.device)
            page = bt.long()[b, pos // self.page_size]
            K_cache[page, :, pos % self.page_size] = Kc[b, :, pos]
            V_cache[page, :, pos % self.page_size] = Vc[b, :, pos]
            return out
        return self._ref_contiguous(hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra)

    def _ref_contiguous(self, hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra):
        (in_w, q_w, k_w, post_w), rope = self._split_extra(extra)
        B, D = hidden.shape[0], self.head_dim
        dev = hidden.device
        eps = self.rms_eps
        qkv_rows = self.q_rows + 2 * self.kv_rows

        x = qwen3_rmsnorm_bf16(hidden, in_w, eps)
        qkv = x @ Wqkv.T
        q = qkv[:, : self.q_rows].view(B, self.num_heads, D)
        k = qkv[:, self.q_rows: qkv_rows - self.kv_rows].view(B, self.num_kv_heads, D)
        v = qkv[:, qkv_rows - self.kv_rows:].view(B, self.num_kv_heads, D)
        ones = torch.ones(D, dtype=hidden.dtype, device=dev)
        qn = head_rmsnorm_f32(q, ones if q_w is None else q_w, eps)
        kn = head_rmsnorm_f32(k, ones if k_w is None else k_w, eps)
        lens = torch.tensor(self.lens(), dtype=torch.long, device=dev)
        pos = lens - 1
        if rope is not None:
            cos, sin = rope
            cp = cos[pos].to(torch.float32)[:, None, :]
            sp = sin[pos].to(torch.float32)[:, None, :]
            q, k = rope_half_f32(qn, cp, sp), rope_half_f32(kn, cp, sp)
        else:
            q, k = qn.to(hidden.dtype), kn.to(hidden.dtype)

        b = torch.arange(B, device=dev)
        K_cache[b, :, pos, :] = k
        V_cache[b, :, pos, :] = v
        attn = gqa_decode_reference(q.unsqueeze(2), K_cache, V_cache,
                                    None if self.kv_lens is None else lens).squeeze(2)
        h = hidden + attn.reshape(B, self.q_rows) @ Wo.T
        xn = qwen3_rmsnorm_bf16(h, post_w, eps)
        gu = xn @ Wgu.T
        gate, up = gu[:, : self.intermediate_size], gu[:, self.intermediate_size:]
        return h + (F.silu(gate) * up) @ Wd.T
