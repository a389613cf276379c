"""Qwen3 per-head QK RMSNorm + RoPE + KV-cache write for one decode step.

Reference: ezops/ops/fused_qk_norm_rope.py:7-169.  For every query head and
every kv head of the decoded token:

    q_head = rope(rmsnorm(q_head, q_norm_w), cos[pos], sin[pos])
    k_head = rope(rmsnorm(k_head, k_norm_w), cos[pos], sin[pos])
    K_cache[b, :, pos, :] = k_head ; V_cache[b, :, pos, :] = v_head

RMSNorm statistics are fp32 over head_dim (eps 1e-6); RoPE is the half-split
(rotate_half) form against full-width HF ``[max_seq_len, head_dim]`` tables;
the whole pipeline is fp32 with a single bf16 rounding (reference :138-147).
Returns ``(q_out, k_out)``.

Extension: ``position`` may be a sequence of ``batch`` ints (one decode
position per sequence); the reference takes a single scalar (:66, :161).
"""

from collections.abc import Sequence

import torch

from ..registry import get_kernel
from .base_op import Op, default_device, randn


def rope_tables(max_seq_len: int, head_dim: int, theta: float, device=None):
    """HF-layout bf16 cos/sin tables (reference :119-125): fp32 angles, halves repeated."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ang = torch.arange(max_seq_len, dtype=torch.float32)[:, None] * inv_freq[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], dim=-1).to(torch.bfloat16)
    sin = torch.cat([ang.sin(), ang.sin()], dim=-1).to(torch.bfloat16)
    dev = default_device(device)
    return cos.to(dev), sin.to(dev)


def head_rmsnorm_f32(x, w, eps):
    """fp32 Qwen3 RMSNorm over the last dim with weight (reference :138-141)."""
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True)
    return xf * torch.rsqrt(var + eps) * w.to(torch.float32)


def rope_half_f32(x, cos_pos, sin_pos):
    """Half-split RoPE of fp32 heads, rounded once to bf16 (reference :143-147)."""
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return (x * cos_pos + rot * sin_pos).to(torch.bfloat16)


class FusedQkNormRopeOp(Op):
    _params_desc = {
        "batch": "Batch size (tokens per decode step)",
        "num_heads": "Number of query heads",
        "head_dim": "Dimension per head (must be a power of two)",
        "max_seq_len": "KV cache capacity; also the cos/sin table length",
        "position": "Decode position (int, or one int per sequence): RoPE row and cache slot",
        "num_kv_heads": "Number of KV heads for GQA (default: num_heads)",
    }
    _atol = 1e-2
    _rtol = 1e-2

    rms_eps = 1e-6
    rope_theta = 1e6

    def __init__(self, batch: int, num_heads: int, head_dim: int, max_seq_len: int,
                 position, backend: str = "ref", num_kv_heads: int | None = None):
        if head_dim <= 0 or head_dim & (head_dim - 1):
            raise ValueError(f"head_dim ({head_dim}) must be a power of two")
        if isinstance(position, Sequence) or isinstance(position, torch.Tensor):
            positions = [int(p) for p in position]
            if len(positions) != batch:
                raise ValueError(f"position list has {len(positions)} entries, expected batch={batch}")
        else:
            positions = None
        for p in positions if positions is not None else [int(position)]:
            if not 0 <= p < max_seq_len:
                raise ValueError(f"position ({p}) must be in [0, {max_seq_len})")
        self.batch = batch
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.position = position if positions is None else positions
        self.positions = positions
        self.num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if num_heads % self.num_kv_heads != 0:
            raise ValueError(
                f"num_heads ({num_heads}) must be divisible by num_kv_heads ({self.num_kv_heads})"
            )
        self._backend = backend
        if backend != "ref":
            cls = get_kernel("fused_qk_norm_rope", backend)
            self._kernel = cls(batch, num_heads, head_dim, max_seq_len, self.position,
                               num_kv_heads=self.num_kv_heads)
        else:
            self._kernel = self._ref_forward

    def forward(self, q, k, v, q_norm_w, k_norm_w, cos, sin, K_cache, V_cache):
        return self._kernel(q, k, v, q_norm_w, k_norm_w, cos, sin, K_cache, V_cache)

    def gen_data(self, device=None):
        dev = default_device(device)
        bf = dict(dtype=torch.bfloat16, device=dev)
        q = randn(self.batch, self.num_heads, self.head_dim, **bf)
        k = randn(self.batch, self.num_kv_heads, self.head_dim, **bf)
        v = randn(self.batch, self.num_kv_heads, self.head_dim, **bf)
        q_norm_w = randn(self.head_dim, **bf)
        k_norm_w = randn(self.head_dim, **bf)
        if dev.type == "meta":
            cos = torch.empty(self.max_seq_len, self.head_dim, **bf)
            sin = torch.empty(self.max_seq_len, self.head_dim, **bf)
        else:
            cos, sin = rope_tables(self.max_seq_len, self.head_dim, self.rope_theta, dev)
        K_cache = randn(self.batch, self.num_kv_heads, self.max_seq_len, self.head_dim, **bf)
        V_cache = randn(self.batch, self.num_kv_heads, self.max_seq_len, self.head_dim, **bf)
        return q, k, v, q_norm_w, k_norm_w, cos, sin, K_cache, V_cache

    def check(self, actual, expected) -> bool:
        for a, e in zip(actual, expected, strict=True):
            if a.shape != e.shape or not torch.allclose(a, e, atol=self._atol, rtol=self._rtol):
                return False
        return True

    def _positions_tensor(self, device):
        if self.positions is None:
            return torch.full((self.batch,), int(self.position), dtype=torch.long, device=device)
        return torch.tensor(self.positions, dtype=torch.long, device=device)

    def _ref_forward(self, q, k, v, q_norm_w, k_norm_w, cos, sin, K_cache, V_cache):
        pos = self._positions_tensor(q.device)
        cos_p = cos[pos].to(torch.float32)[:, None, :]  # [B,1,D]
        sin_p = sin[pos].to(torch.float32)[:, None, :]
        q_out = rope_half_f32(head_rmsnorm_f32(q, q_norm_w, self.rms_eps), cos_p, sin_p)
        k_out = rope_half_f32(head_rmsnorm_f32(k, k_norm_w, self.rms_eps), cos_p, sin_p)
        b = torch.arange(self.batch, device=q.device)
        K_cache[b, :, pos, :] = k_out
        V_cache[b, :, pos, :] = v
        return q_out, k_out
