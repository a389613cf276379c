"""A multi-layer Qwen3 dense decode step: the caller of the single layer.

The reference stops at one decoder layer (ezops/ops/qwen3_dense_decode.py:9-176);
a model's decode step runs ``num_layers`` of them back to back, the hidden
state of each feeding the next, then the final RMSNorm and the LM head:

    h = hidden
    for layer in layers:  h = Qwen3DenseDecodeOp(layer)(h)     # each with its own cache
    logits = (rmsnorm(h) * final_norm_w) @ lm_head.T           # if vocab_size > 0

``forward(hidden, layers, cos=None, sin=None, final_norm_w=None,
lm_head=None, block_table=None)`` returns ``(h, logits)`` (``logits`` None
without an LM head).  ``layers`` holds one tuple per layer:
``(K_cache, V_cache, Wqkv, Wo, Wgu, Wd)`` plus, with ``norm_weights``,
``(in_norm_w, q_norm_w, k_norm_w, post_norm_w)``.  The ctor options
(``kv_lens``, ``norm_weights``, ``rope_theta``, ``page_size``,
``num_pages``) mean what they mean for Qwen3DenseDecodeOp and apply to
every layer; a paged cache shares one block table across layers.
"""

import torch

from ..registry import get_kernel
from .base_op import Op, default_device, randn
from .fused_o_proj_ffn import frobenius_ok, qwen3_rmsnorm_bf16
from .qwen3_dense_decode import Qwen3DenseDecodeOp


class Qwen3DecodeStepOp(Op):
    _params_desc = {
        "batch": "Batch size (tokens per decode step)",
        "seq_len": "KV cache capacity per sequence",
        "hidden_size": "Hidden dimension",
        "intermediate_size": "MLP intermediate dimension",
        "num_heads": "Number of query heads",
        "head_dim": "Dimension per head",
        "num_layers": "Decoder layers in the step",
        "num_kv_heads": "Number of KV heads for GQA (default: num_heads)",
        "vocab_size": "LM head rows (0 = no LM head)",
    }
    _atol = 1e-2
    _rtol = 1e-2
    rms_eps = 1e-6

    def check(self, actual, expected) -> bool:
        return frobenius_ok(actual, expected, self._rtol)

    def __init__(self, batch: int, seq_len: int, hidden_size: int, intermediate_size: int, num_heads: int,
                 head_dim: int, num_layers: int, backend: str = "ref", num_kv_heads: int | None = None, *,
                 vocab_size: int = 0, kv_lens=None, norm_weights: bool = False, rope_theta: float | None = None,
                 page_size: int | None = None, num_pages: int | None = None):
        if num_layers < 1:
            raise ValueError(f"num_layers ({num_layers}) must be >= 1")
        if vocab_size < 0:
            raise ValueError(f"vocab_size ({vocab_size}) must be >= 0")
        self.layer = Qwen3DenseDecodeOp(batch, seq_len, hidden_size, intermediate_size, num_heads, head_dim,
                                        num_kv_heads=num_kv_heads, kv_lens=kv_lens, norm_weights=norm_weights,
                                        rope_theta=rope_theta, page_size=page_size, num_pages=num_pages)
        self.batch, self.seq_len, self.hidden_size = batch, seq_len, hidden_size
        self.num_layers, self.vocab_size = num_layers, vocab_size
        self.norm_weights, self.rope_theta, self.page_size = norm_weights, rope_theta, page_size
        self._backend = backend
        if backend != "ref":
            l = self.layer
            self._kernel = get_kernel("qwen3_decode_step", backend)(
                batch, seq_len, hidden_size, intermediate_size, num_heads, head_dim, num_layers,
                num_kv_heads=l.num_kv_heads, vocab_size=vocab_size, kv_lens=l.kv_lens, norm_weights=norm_weights,
                rope_theta=rope_theta, page_size=page_size, num_pages=l.num_pages)
        else:
            self._kernel = self._ref_forward

    def forward(self, hidden, layers, cos=None, sin=None, final_norm_w=None, lm_head=None, block_table=None):
        return self._kernel(hidden, layers, cos, sin, final_norm_w, lm_head, block_table)

    def gen_data(self, device=None):
        dev = default_device(device)
        bf = dict(dtype=torch.bfloat16, device=dev)
        layers, cos, sin, bt = [], None, None, None
        hidden = None
        for i in range(self.num_layers):
            d = list(self.layer.gen_data(dev))
            if self.page_size is not None:
                b = d.pop()
                bt = b if bt is None else bt
            if self.rope_theta is not None:
                s_, c_ = d.pop(), d.pop()
                cos, sin = (c_, s_) if cos is None else (cos, sin)
            hidden = d[0] if hidden is None else hidden
            layers.append(tuple(d[1:]))
        final_norm_w = randn(self.hidden_size, **bf, scale=0.1, mean=1.0) if self.norm_weights else None
        lm_head = (randn(self.vocab_size, self.hidden_size, **bf, scale=self.hidden_size ** -0.5)
                   if self.vocab_size else None)
        return hidden, layers, cos, sin, final_norm_w, lm_head, bt

    def _ref_forward(self, hidden, layers, cos=None, sin=None, final_norm_w=None, lm_head=None,
                     block_table=None):
        rope = [cos, sin] if self.rope_theta is not None else []
        paged = [block_table] if self.page_size is not None else []
        h = hidden
        for layer in layers:
            h = self.layer._ref_forward(h, *layer, *rope, *paged)
        logits = None
        if self.vocab_size:
            logits = qwen3_rmsnorm_bf16(h, final_norm_w, self.rms_eps) @ lm_head.T
        return h, logits
