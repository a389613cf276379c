"""HIP prefill of one Qwen3 dense layer (no reference counterpart: the
reference is decode only, ezops/ops/qwen3_dense_decode.py:9-176)."""

import ctypes

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel
from .qwen3_dense_decode_hip import RMS_EPS


@register_kernel("qwen3_dense_prefill", "hip")
class Qwen3PrefillHipKernel(BaseKernel):
    def __init__(self, batch: int, seq_len: int, hidden_size: int, intermediate_size: int, num_heads: int,
                 head_dim: int, q_lens, past_lens, num_kv_heads: int | None = None, norm_weights: bool = False,
                 rope_theta: float | None = None, page_size: int | None = None, num_pages: int | None = None):
        num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if head_dim != 128:
            raise ValueError(f"head_dim ({head_dim}) must be 128")
        if num_heads % num_kv_heads or num_heads // num_kv_heads not in (1, 2, 4, 8):
            raise ValueError(f"GQA group size {num_heads}/{num_kv_heads} not supported (1, 2, 4 or 8)")
        if intermediate_size % 8:
            raise ValueError(f"intermediate_size ({intermediate_size}) must be a multiple of 8")
        self.B, self.S, self.HS, self.IS = batch, seq_len, hidden_size, intermediate_size
        self.H, self.D, self.Hkv = num_heads, head_dim, num_kv_heads
        self.q_lens, self.past_lens = list(q_lens), list(past_lens)
        self.T = sum(self.q_lens)
        self.norm_weights, self.rope = norm_weights, rope_theta is not None
        self.page_size, self.num_pages = page_size, num_pages
        cu = [0]
        for n in self.q_lens:
            cu.append(cu[-1] + n)
        self._host = (cu, self.past_lens)
        self._dev: dict = {}
        self._ws = _hip.Workspace()

    def _meta(self, dev):
        t = self._dev.get(dev)
        if t is None:
            t = tuple(torch.tensor(x, dtype=torch.int32, device=dev) for x in self._host)
            self._dev[dev] = t
        return t

    def __call__(self, hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra):
        extra = list(extra)
        paged = self.page_size is not None
        bt = extra.pop() if paged and extra else None
        if paged and bt is None:
            raise ValueError("paged cache: the block table is the last input")
        want = (4 if self.norm_weights else 0) + (2 if self.rope else 0)
        if len(extra) != want:
            raise ValueError(f"expected {want} extra inputs (norm weights / rope tables), got {len(extra)}")
        nw = extra[:4] if self.norm_weights else [None] * 4
        cos, sin = extra[-2:] if self.rope else (None, None)
        dev = _hip.require_gpu(hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra, *([bt] if paged else []))
        bf = torch.bfloat16
        T, S, HS, IS, H, D, Hkv = self.T, self.S, self.HS, self.IS, self.H, self.D, self.Hkv
        _hip.check(hidden, "hidden", (T, HS), bf)
        kv_shape = (self.num_pages, Hkv, self.page_size, D) if paged else (self.B, Hkv, S, D)
        _hip.check(K_cache, "K_cache", kv_shape, bf)
        _hip.check(V_cache, "V_cache", kv_shape, bf)
        if paged:
            _hip.check(bt, "block_table", (self.B, S // self.page_size), torch.int32)
        _hip.check(Wqkv, "Wqkv", ((H + 2 * Hkv) * D, HS), bf)
        _hip.check(Wo, "Wo", (HS, H * D), bf)
        _hip.check(Wgu, "Wgu", (2 * IS, HS), bf)
        _hip.check(Wd, "Wd", (HS, IS), bf)
        for t, n, name in zip(nw, (HS, D, D, HS), ("in_norm_w", "q_norm_w", "k_norm_w", "post_norm_w")):
            if t is not None:
                _hip.check(t, name, (n,), bf)
        if self.rope:
            _hip.check(cos, "cos", (S, D), bf)
            _hip.check(sin, "sin", (S, D), bf)
        out = torch.empty(T, HS, dtype=bf, device=dev)
        cu, past = self._meta(dev)
        p = _hip.Qwen3LayerParams(
            B=self.B, S=S, HS=HS, IS=IS, H=H, Hkv=Hkv, D=D, eps=RMS_EPS,
            hidden=hidden.data_ptr(), K_cache=K_cache.data_ptr(), V_cache=V_cache.data_ptr(),
            Wqkv=Wqkv.data_ptr(), Wo=Wo.data_ptr(), Wgu=Wgu.data_ptr(), Wd=Wd.data_ptr(),
            in_norm_w=_hip.ptr(nw[0]), q_norm_w=_hip.ptr(nw[1]), k_norm_w=_hip.ptr(nw[2]),
            post_norm_w=_hip.ptr(nw[3]), cos=_hip.ptr(cos), sin=_hip.ptr(sin), kv_lens=past.data_ptr(),
            max_kv_len=0, out=out.data_ptr(),
        )
        pp = ctypes.byref(p)
        ws = self._ws.get(_hip.size("ezops_qwen3_prefill_workspace_size", pp, T), dev)
        _hip.call("ezops_qwen3_prefill_bf16", pp, T, cu.data_ptr(), max(self.q_lens), _hip.ptr(bt),
                  self.num_pages or 0, self.page_size or 0, ws.data_ptr(), ws.numel(), _hip.stream(dev))
        return out
