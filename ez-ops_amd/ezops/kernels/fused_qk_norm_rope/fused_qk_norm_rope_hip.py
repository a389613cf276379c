"""HIP fused QK-norm + RoPE + KV write (replaces ezops/kernels/fused_qk_norm_rope/*)."""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel

RMS_EPS = 1e-6


@register_kernel("fused_qk_norm_rope", "hip")
class FusedQkNormRopeHipKernel(BaseKernel):
    def __init__(self, batch: int, num_heads: int, head_dim: int, max_seq_len: int, position,
                 num_kv_heads: int | None = None):
        num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if head_dim <= 0 or head_dim & (head_dim - 1) or head_dim > 512:
            raise ValueError(f"head_dim ({head_dim}) must be a power of two <= 512")
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads ({num_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
        self.B, self.H, self.D, self.S, self.Hkv = batch, num_heads, head_dim, max_seq_len, num_kv_heads
        if isinstance(position, int):
            self.positions = None
            self.position = position
        else:
            self.positions = [int(p) for p in position]
            self.position = 0
        for p in self.positions or [self.position]:
            if not 0 <= p < max_seq_len:
                raise ValueError(f"position ({p}) must be in [0, {max_seq_len})")
        self._pos_dev: dict = {}

    def _positions(self, dev):
        if self.positions is None:
            return None
        t = self._pos_dev.get(dev)
        if t is None:
            t = torch.tensor(self.positions, dtype=torch.int32, device=dev)
            self._pos_dev[dev] = t
        return t

    def __call__(self, q, k, v, q_norm_w, k_norm_w, cos, sin, K_cache, V_cache):
        dev = _hip.require_gpu(q, k, v, q_norm_w, k_norm_w, cos, sin, K_cache, V_cache)
        bf = torch.bfloat16
        B, H, Hkv, D, S = self.B, self.H, self.Hkv, self.D, self.S
        _hip.check(q, "q", (B, H, D), bf)
        _hip.check(k, "k", (B, Hkv, D), bf)
        _hip.check(v, "v", (B, Hkv, D), bf)
        _hip.check(q_norm_w, "q_norm_w", (D,), bf)
        _hip.check(k_norm_w, "k_norm_w", (D,), bf)
        _hip.check(cos, "cos", (S, D), bf)
        _hip.check(sin, "sin", (S, D), bf)
        _hip.check(K_cache, "K_cache", (B, Hkv, S, D), bf)
        _hip.check(V_cache, "V_cache", (B, Hkv, S, D), bf)
        q_out = torch.empty(B, H, D, dtype=bf, device=dev)
        k_out = torch.empty(B, Hkv, D, dtype=bf, device=dev)
        pos = self._positions(dev)
        _hip.call("ezops_qk_norm_rope_bf16", q.data_ptr(), H * D, k.data_ptr(), Hkv * D, v.data_ptr(), Hkv * D,
                  q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                  K_cache.data_ptr(), V_cache.data_ptr(), q_out.data_ptr(), k_out.data_ptr(),
                  B, H, Hkv, D, S, self.position, _hip.ptr(pos), 0, RMS_EPS, _hip.stream(dev))
        return q_out, k_out
