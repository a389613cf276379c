"""HIP split-KV GQA decode attention.

Replaces the reference's attention backends (ezops/kernels/attn_decode/
attn_decode_cu.py:14-29, attn_decode_tl.py:617-657) behind AttnDecodeOp.
"""

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel


@register_kernel("attn_decode", "hip")
class AttnDecodeHipKernel(BaseKernel):
    supports_gqa = True

    def __init__(self, batch: int, num_heads: int, seq_len: int, head_dim: int, num_kv_heads: int | None = None):
        num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads ({num_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
        if num_heads // num_kv_heads not in (1, 2, 4, 8, 16):
            raise ValueError(f"GQA group size {num_heads // num_kv_heads} not supported (1, 2, 4, 8 or 16)")
        if head_dim not in (64, 128):
            raise ValueError(f"head_dim ({head_dim}) must be 64 or 128")
        if batch < 1 or seq_len < 1:
            raise ValueError("batch and seq_len must be >= 1")
        self.B, self.H, self.S, self.D, self.Hkv = batch, num_heads, seq_len, head_dim, num_kv_heads
        self._ws = _hip.Workspace()

    def __call__(self, Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, kv_lens: torch.Tensor | None = None,
                 max_kv_len: int = 0):
        """``max_kv_len`` (extension, keyword): the caller's bound on the
        ``kv_lens`` entries, 0 = seq_len.  It plans the split-KV grid and lets
        the first K/V tiles be requested before the lengths are read; entries
        above it are treated as ``max_kv_len``."""
        if max_kv_len < 0:
            raise ValueError(f"max_kv_len ({max_kv_len}) must be >= 0")
        dev = _hip.require_gpu(Q, K, V, kv_lens)
        bf = torch.bfloat16
        _hip.check(Q, "Q", (self.B, self.H, 1, self.D), bf)
        _hip.check(K, "K", (self.B, self.Hkv, self.S, self.D), bf)
        _hip.check(V, "V", (self.B, self.Hkv, self.S, self.D), bf)
        if kv_lens is not None:
            _hip.check(kv_lens, "kv_lens", (self.B,), torch.int32)
        Out = torch.empty(self.B, self.H, 1, self.D, dtype=bf, device=dev)
        nbytes = _hip.size("ezops_attn_decode_workspace_size", self.B, self.H, self.Hkv, self.S, self.D)
        ws = self._ws.get(nbytes, dev)
        _hip.call("ezops_attn_decode_bf16", Q.data_ptr(), K.data_ptr(), V.data_ptr(), Out.data_ptr(),
                  self.B, self.H, self.Hkv, self.S, self.D, _hip.ptr(kv_lens), int(max_kv_len), 0.0, ws.data_ptr(), ws.numel(),
                  _hip.stream(dev))
        return Out
