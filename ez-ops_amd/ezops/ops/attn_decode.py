"""Single-token GQA decode attention spec (reference: ezops/ops/attn_decode.py:9-67).

``Out[b, h] = softmax(Q[b, h] . K[b, h // G]^T / sqrt(D)) . V[b, h // G]`` for
``Q [B, H, 1, D]`` and ``K, V [B, Hkv, S, D]`` (``G = H / Hkv``), bf16 in and
out.  The reference evaluates it with cuDNN SDPA (attn_decode.py:64-67),
which does not exist on ROCm; ``_ref_forward`` here is the same formula
written out in fp32.

Extension (ragged batches): ``forward(Q, K, V, kv_lens)`` with an int32
``kv_lens [B]`` attends sequence ``b`` to slots ``[0, kv_lens[b])`` only.
"""

import torch

from ..registry import get_kernel
from .base_op import Op, default_device, randn


def gqa_decode_reference(Q, K, V, kv_lens=None, scale=None):
    """fp32 GQA decode attention; Q [B,H,1,D], K/V [B,Hkv,S,D] -> [B,H,1,D] bf16."""
    B, H, _, D = Q.shape
    Hkv, S = K.shape[1], K.shape[2]
    G = H // Hkv
    scale = D ** -0.5 if scale is None else scale
    q = Q.reshape(B, Hkv, G, D).float()
    s = torch.einsum("bkgd,bksd->bkgs", q, K.float()) * scale
    if kv_lens is not None:
        pos = torch.arange(S, device=Q.device)
        mask = pos[None, :] >= kv_lens.to(Q.device).long()[:, None]  # [B,S]
        s = s.masked_fill(mask[:, None, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1)
    o = torch.einsum("bkgs,bksd->bkgd", p, V.float())
    return o.reshape(B, H, 1, D).to(Q.dtype)


class AttnDecodeOp(Op):
    _params_desc = {
        "batch": "Batch size",
        "num_heads": "Number of attention heads",
        "seq_len": "KV cache sequence length",
        "head_dim": "Dimension per head",
        "num_kv_heads": "Number of KV heads for GQA (default: num_heads)",
    }
    _atol = 1e-2
    _rtol = 1e-2

    def __init__(self, batch: int, num_heads: int, seq_len: int, head_dim: int,
                 backend: str = "ref", num_kv_heads: int | None = None):
        self.batch = batch
        self.num_heads = num_heads
        self.seq_len = seq_len
        self.head_dim = head_dim
        self.num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if num_heads % self.num_kv_heads != 0:
            raise ValueError(
                f"num_heads ({num_heads}) must be divisible by num_kv_heads ({self.num_kv_heads})"
            )
        self._backend = backend
        if backend != "ref":
            cls = get_kernel("attn_decode", backend)
            if not getattr(cls, "supports_gqa", False):
                if self.num_kv_heads != num_heads:
                    raise ValueError(
                        f"backend {backend!r} does not support GQA "
                        f"(num_kv_heads={self.num_kv_heads} != num_heads={num_heads}); "
                        "expand K/V to num_heads before calling it"
                    )
                self._kernel = cls(batch, num_heads, seq_len, head_dim)
            else:
                self._kernel = cls(batch, num_heads, seq_len, head_dim, num_kv_heads=self.num_kv_heads)
        else:
            self._kernel = self._ref_forward

    def forward(self, Q, K, V, kv_lens=None):
        if kv_lens is None:
            return self._kernel(Q, K, V)
        return self._kernel(Q, K, V, kv_lens)

    def gen_data(self, device=None):
        dev = default_device(device)
        Q = randn(self.batch, self.num_heads, 1, self.head_dim, dtype=torch.bfloat16, device=dev)
        K = randn(self.batch, self.num_kv_heads, self.seq_len, self.head_dim, dtype=torch.bfloat16, device=dev)
        V = randn(self.batch, self.num_kv_heads, self.seq_len, self.head_dim, dtype=torch.bfloat16, device=dev)
        return Q, K, V

    def _ref_forward(self, Q, K, V, kv_lens=None):
        return gqa_decode_reference(Q, K, V, kv_lens)
