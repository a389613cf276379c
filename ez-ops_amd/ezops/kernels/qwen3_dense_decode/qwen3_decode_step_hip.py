"""HIP multi-layer Qwen3 decode step (the caller of the single layer,
ezops/ops/qwen3_dense_decode.py:9-176, which the reference stops at)."""

import ctypes

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel
from .qwen3_dense_decode_hip import RMS_EPS, Qwen3DenseDecodeHipKernel


@register_kernel("qwen3_decode_step", "hip")
class Qwen3DecodeStepHipKernel(BaseKernel):
    def __init__(self, batch: int, seq_len: int, hidden_size: int, intermediate_size: int, num_heads: int,
                 head_dim: int, num_layers: int, num_kv_heads: int | None = None, vocab_size: int = 0, kv_lens=None,
                 norm_weights: bool = False, rope_theta: float | None = None, page_size: int | None = None,
                 num_pages: int | None = None):
        # the single-layer kernel validates the shapes and holds the lengths
        self.layer = Qwen3DenseDecodeHipKernel(batch, seq_len, hidden_size, intermediate_size, num_heads, head_dim,
                                               num_kv_heads=num_kv_heads, kv_lens=kv_lens,
                                               norm_weights=norm_weights, rope_theta=rope_theta,
                                               page_size=page_size, num_pages=num_pages)
        if num_layers < 1 or vocab_size < 0:
            raise ValueError("num_layers must be >= 1 and vocab_size >= 0")
        self.L, self.V = num_layers, vocab_size
        self._ws = _hip.Workspace()

    def __call__(self, hidden, layers, cos=None, sin=None, final_norm_w=None, lm_head=None, block_table=None):
        k = self.layer
        B, S, HS, IS, H, D, Hkv = k.B, k.S, k.HS, k.IS, k.H, k.D, k.Hkv
        if len(layers) != self.L:
            raise ValueError(f"expected {self.L} layers, got {len(layers)}")
        paged = k.page_size is not None
        if paged != (block_table is not None):
            raise ValueError("block_table is required with a paged cache and only then")
        bf = torch.bfloat16
        dev = _hip.require_gpu(hidden, cos, sin, final_norm_w, lm_head, block_table)
        _hip.check(hidden, "hidden", (B, HS), bf)
        if k.rope:
            _hip.check(cos, "cos", (S, D), bf)
            _hip.check(sin, "sin", (S, D), bf)
        elif cos is not None or sin is not None:
            raise ValueError("cos/sin given without rope_theta")
        if paged:
            _hip.check(block_table, "block_table", (B, S // k.page_size), torch.int32)
            kv_shape = (k.num_pages, Hkv, k.page_size, D)
        else:
            kv_shape = (B, Hkv, S, D)
        if self.V:
            _hip.check(lm_head, "lm_head", (self.V, HS), bf)
            if final_norm_w is not None:
                _hip.check(final_norm_w, "final_norm_w", (HS,), bf)
        nw_n = 4 if k.norm_weights else 0
        out = torch.empty(B, HS, dtype=bf, device=dev)
        logits = torch.empty(B, self.V, dtype=bf, device=dev) if self.V else None
        lens = k._lens(dev)
        params = (_hip.Qwen3LayerParams * self.L)()
        for i, layer in enumerate(layers):
            if len(layer) != 6 + nw_n:
                raise ValueError(f"layer {i}: expected {6 + nw_n} tensors, got {len(layer)}")
            Kc, Vc, Wqkv, Wo, Wgu, Wd = layer[:6]
            nw = list(layer[6:]) if nw_n else [None] * 4
            _hip.require_gpu(*layer)
            _hip.check(Kc, f"layer {i} K_cache", kv_shape, bf)
            _hip.check(Vc, f"layer {i} V_cache", kv_shape, bf)
            _hip.check(Wqkv, f"layer {i} Wqkv", ((H + 2 * Hkv) * D, HS), bf)
            _hip.check(Wo, f"layer {i} Wo", (HS, H * D), bf)
            _hip.check(Wgu, f"layer {i} Wgu", (2 * IS, HS), bf)
            _hip.check(Wd, f"layer {i} Wd", (HS, IS), bf)
            for t, n, name in zip(nw, (HS, D, D, HS), ("in_norm_w", "q_norm_w", "k_norm_w", "post_norm_w")):
                if t is not None:
                    _hip.check(t, f"layer {i} {name}", (n,), bf)
            p = params[i]
            p.B, p.S, p.HS, p.IS, p.H, p.Hkv, p.D, p.eps = B, S, HS, IS, H, Hkv, D, RMS_EPS
            p.hidden = hidden.data_ptr() if i == 0 else None
            p.K_cache, p.V_cache = Kc.data_ptr(), Vc.data_ptr()
            p.Wqkv, p.Wo, p.Wgu, p.Wd = Wqkv.data_ptr(), Wo.data_ptr(), Wgu.data_ptr(), Wd.data_ptr()
            p.in_norm_w, p.q_norm_w, p.k_norm_w, p.post_norm_w = (_hip.ptr(t) for t in nw)
            p.cos, p.sin = _hip.ptr(cos), _hip.ptr(sin)
            p.kv_lens = _hip.ptr(lens)
            p.max_kv_len = max(k.kv_lens) if k.kv_lens else 0
            p.out = out.data_ptr() if i == self.L - 1 else None
        ws = self._ws.get(_hip.size("ezops_qwen3_decode_step_workspace_size", params, self.L, self.V), dev)
        _hip.call("ezops_qwen3_decode_step_bf16", params, self.L, _hip.ptr(block_table),
                  k.num_pages if paged else 0, k.page_size if paged else 0, _hip.ptr(final_norm_w),
                  _hip.ptr(lm_head), self.V, _hip.ptr(logits), ws.data_ptr(), ws.numel(), _hip.stream(dev))
        return out, logits
