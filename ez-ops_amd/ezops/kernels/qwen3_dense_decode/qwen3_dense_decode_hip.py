"""HIP Qwen3 dense decode layer (replaces ezops/kernels/qwen3_dense_decode/*)."""

import ctypes

import torch

from ... import _hip
from ...registry import register_kernel
from ..base_kernel import BaseKernel
from ..fused_o_proj_ffn.fused_o_proj_ffn_hip import check_tiles

RMS_EPS = 1e-6


@register_kernel("qwen3_dense_decode", "hip")
class Qwen3DenseDecodeHipKernel(BaseKernel):
    def __init__(self, batch: int, seq_len: int, hidden_size: int, intermediate_size: int, num_heads: int,
                 head_dim: int, num_kv_heads: int | None = None, kv_lens=None, norm_weights: bool = False,
                 rope_theta: float | None = None, page_size: int | None = None, num_pages: int | None = None):
        num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads ({num_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
        if num_heads // num_kv_heads not in (1, 2, 4, 8, 16):
            raise ValueError(f"GQA group size {num_heads // num_kv_heads} not supported (1, 2, 4, 8 or 16)")
        if head_dim not in (64, 128):
            raise ValueError(f"head_dim ({head_dim}) must be 64 or 128")
        check_tiles(hidden_size=hidden_size, intermediate_size=intermediate_size)
        self.B, self.S, self.HS, self.IS = batch, seq_len, hidden_size, intermediate_size
        self.H, self.D, self.Hkv = num_heads, head_dim, num_kv_heads
        self.kv_lens = None if kv_lens is None else [int(x) for x in kv_lens]
        self.norm_weights = norm_weights
        self.rope = rope_theta is not None
        if page_size is not None:
            if page_size < 32 or page_size & (page_size - 1) or seq_len % page_size:
                raise ValueError(f"page_size ({page_size}) must be a power of two >= 32 dividing seq_len ({seq_len})")
            if self.kv_lens is None:
                raise ValueError("a paged cache requires kv_lens")
            num_pages = batch * (seq_len // page_size) if num_pages is None else num_pages
        self.page_size, self.num_pages = page_size, num_pages
        self._ws = _hip.Workspace()
        self._lens_dev: dict = {}

    def _lens(self, dev):
        if self.kv_lens is None:
            return None
        t = self._lens_dev.get(dev)
        if t is None:
            t = torch.tensor(self.kv_lens, dtype=torch.int32, device=dev)
            self._lens_dev[dev] = t
        return t

    def __call__(self, hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra):
        """Paged cache: K_cache / V_cache are page pools and the block table
        is the last input."""
        bt = None
        if self.page_size is not None:
            if not extra:
                raise ValueError("paged cache: the block table is the last input")
            *extra, bt = extra
        want = (4 if self.norm_weights else 0) + (2 if self.rope else 0)
        if len(extra) != want:
            raise ValueError(f"expected {want} extra inputs (norm weights / rope tables), got {len(extra)}")
        nw = list(extra[:4]) if self.norm_weights else [None] * 4
        cos, sin = extra[-2:] if self.rope else (None, None)
        dev = _hip.require_gpu(hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, *extra, *([] if bt is None else [bt]))
        bf = torch.bfloat16
        B, S, HS, IS, H, D, Hkv = self.B, self.S, self.HS, self.IS, self.H, self.D, self.Hkv
        _hip.check(hidden, "hidden", (B, HS), bf)
        if bt is None:
            kv_shape = (B, Hkv, S, D)
        else:
            kv_shape = (self.num_pages, Hkv, self.page_size, D)
            _hip.check(bt, "block_table", (B, S // self.page_size), torch.int32)
        _hip.check(K_cache, "K_cache", kv_shape, bf)
        _hip.check(V_cache, "V_cache", kv_shape, bf)
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
        out = torch.empty(B, HS, dtype=bf, device=dev)
        lens = self._lens(dev)
        p = _hip.Qwen3LayerParams(
            B=B, S=S, HS=HS, IS=IS, H=H, Hkv=Hkv, D=D, eps=RMS_EPS,
            hidden=hidden.data_ptr(), K_cache=K_cache.data_ptr(), V_cache=V_cache.data_ptr(),
            Wqkv=Wqkv.data_ptr(), Wo=Wo.data_ptr(), Wgu=Wgu.data_ptr(), Wd=Wd.data_ptr(),
            in_norm_w=_hip.ptr(nw[0]), q_norm_w=_hip.ptr(nw[1]), k_norm_w=_hip.ptr(nw[2]),
            post_norm_w=_hip.ptr(nw[3]), cos=_hip.ptr(cos), sin=_hip.ptr(sin), kv_lens=_hip.ptr(lens),
            max_kv_len=max(self.kv_lens) if self.kv_lens else 0,
            out=out.data_ptr(),
        )
        pp = ctypes.byref(p)
        ws = self._ws.get(_hip.size("ezops_qwen3_layer_workspace_size", pp), dev)
        if bt is None:
            _hip.call("ezops_qwen3_dense_decode_bf16", pp, ws.data_ptr(), ws.numel(), _hip.stream(dev))
        else:
            _hip.call("ezops_qwen3_dense_decode_paged_bf16", pp, bt.data_ptr(), self.num_pages, self.page_size,
                      ws.data_ptr(), ws.numel(), _hip.stream(dev))
        return out
