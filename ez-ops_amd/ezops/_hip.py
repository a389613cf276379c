"""ctypes binding of libezops_hip.so (C ABI declared in include/ezops_hip.h).

The library is loaded once per process from ``ezops/_lib/libezops_hip.so``
(override with ``EZOPS_HIP_LIB``).  There is no fallback: if the library is
missing, every HIP kernel call raises RuntimeError.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("EZOPS_HIP_LIB", Path(__file__).resolve().parent / "_lib" / "libezops_hip.so"))

EINVAL = -22
ABI_VERSION = 2

_p, _i64, _f32, _sz, _i32 = C.c_void_p, C.c_int64, C.c_float, C.c_size_t, C.c_int


class Qwen3LayerParams(C.Structure):
    """Mirror of ``ezops_qwen3_layer`` in include/ezops_hip.h (field order matters)."""

    _fields_ = [
        ("B", _i64), ("S", _i64), ("HS", _i64), ("IS", _i64), ("H", _i64), ("Hkv", _i64), ("D", _i64),
        ("eps", _f32),
        ("hidden", _p), ("K_cache", _p), ("V_cache", _p), ("Wqkv", _p), ("Wo", _p), ("Wgu", _p), ("Wd", _p),
        ("in_norm_w", _p), ("q_norm_w", _p), ("k_norm_w", _p), ("post_norm_w", _p),
        ("cos", _p), ("sin", _p), ("kv_lens", _p), ("max_kv_len", _i64),
        ("out", _p),
    ]


# name -> (restype, argtypes); exactly the entry points of include/ezops_hip.h
SIGNATURES: dict[str, tuple] = {
    "ezops_hip_abi_version": (_i32, []),
    "ezops_hip_last_error": (C.c_char_p, []),
    "ezops_gemv_bf16": (_i32, [_p, _p, _p, _i64, _i64, _p]),
    "ezops_linear_bf16": (_i32, [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "ezops_linear_stage_workspace_size": (_sz, [_i64, _i64, _i32]),
    "ezops_linear_stage_bf16": (_i32, [_p, _i64, _p, _p, _p, _i64, _p, _i64, _p, _i32, _f32, _i32, _i64, _i64,
                                       _i64, _p, _sz, _p]),
    "ezops_rmsnorm_f32": (_i32, [_p, _p, _i64, _i64, _f32, _p]),
    "ezops_rmsnorm_bf16": (_i32, [_p, _p, _p, _i64, _i64, _f32, _p]),
    "ezops_softmax_f32": (_i32, [_p, _p, _i64, _i64, _p]),
    "ezops_reduce_sum_workspace_size": (_sz, [_i64]),
    "ezops_reduce_sum_f32": (_i32, [_p, _p, _i64, _p, _sz, _p]),
    "ezops_attn_decode_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "ezops_attn_decode_bf16": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _f32, _p, _sz, _p]),
    "ezops_attn_decode_noalloc_max_scratch": (_sz, []),
    "ezops_attn_decode_noalloc_bf16": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _f32, _p]),
    "ezops_prefill_attn_bf16": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64,
                                       _i64, _f32, _p]),
    "ezops_qwen3_prefill_workspace_size": (_sz, [C.POINTER(Qwen3LayerParams), _i64]),
    "ezops_qwen3_prefill_bf16": (_i32, [C.POINTER(Qwen3LayerParams), _i64, _p, _i64, _p, _i64, _i64, _p, _sz, _p]),
    "ezops_gemm_workspace_size": (_sz, []),
    "ezops_gemm_bf16": (_i32, [_p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _p, _sz, _p]),
    "ezops_gemm_swiglu_bf16": (_i32, [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "ezops_paged_attn_decode_bf16": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                            _f32, _p, _sz, _p]),
    "ezops_qk_norm_rope_bf16": (_i32, [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p,
                                       _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _f32, _p]),
    "ezops_o_proj_ffn_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "ezops_o_proj_ffn_bf16": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p, _sz, _p]),
    "ezops_qwen3_layer_workspace_size": (_sz, [C.POINTER(Qwen3LayerParams)]),
    "ezops_qwen3_dense_decode_bf16": (_i32, [C.POINTER(Qwen3LayerParams), _p, _sz, _p]),
    "ezops_qwen3_dense_decode_paged_bf16": (_i32, [C.POINTER(Qwen3LayerParams), _p, _i64, _i64, _p, _sz, _p]),
    "ezops_qwen3_decode_step_workspace_size": (_sz, [C.POINTER(Qwen3LayerParams), _i64, _i64]),
    "ezops_qwen3_decode_step_bf16": (_i32, [C.POINTER(Qwen3LayerParams), _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p,
                                            _sz, _p]),
    "ezops_hbm_probe": (_i32, [_i32, _p, _p, _p, _i64, _f32, _p]),
    "ezops_profile_read": (_i64, [_p, _i64]),
    "ezops_profile_reset": (_i32, []),
    "ezops_mfma_probe": (_i32, [_i32, _p, _i64, _i64, _p]),
}

_lib = None


def load(path: Path) -> C.CDLL:
    """Load a build of the library at ``path`` and bind every entry point."""
    if not Path(path).exists():
        raise RuntimeError(
            f"{Path(path).name} not found at {path}; build it with "
            "`python ez-ops_amd/build.py --all` (hipcc, gfx950)"
        )
    l = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args
    if l.ezops_hip_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {l.ezops_hip_abi_version()} != {ABI_VERSION}")
    return l


def lib() -> C.CDLL:
    """Load (once) and return the HIP library; raise if it is absent."""
    global _lib
    if _lib is None:
        _lib = load(LIB_PATH)
    return _lib


def call(name: str, *args) -> None:
    """Invoke an int-returning entry point; non-zero status raises RuntimeError."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().ezops_hip_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def size(name: str, *args) -> int:
    return int(getattr(lib(), name)(*args))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one GPU; the HIP backend has no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"HIP backend needs GPU tensors, got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def check(t: torch.Tensor, name: str, shape: tuple, dtype: torch.dtype) -> None:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.dtype != dtype:
        raise ValueError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


class Workspace:
    """Per-device zero-initialised scratch buffer, grown on demand.

    The kernels return their arrival counters to zero at the end of every
    call, so the buffer is zero-filled only when (re)allocated.
    """

    def __init__(self):
        self._bufs: dict[torch.device, torch.Tensor] = {}

    def get(self, nbytes: int, device: torch.device) -> torch.Tensor:
        buf = self._bufs.get(device)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
            self._bufs[device] = buf
        return buf
