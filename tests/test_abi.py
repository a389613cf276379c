"""The C-ABI library loads and exports every entry point of include/ezops_hip.h (CPU only).

Only argument-validation paths are exercised here: they return before any
HIP call, so no GPU is needed.
"""

import ctypes
import re
from pathlib import Path

import pytest

from ezops import _hip

HEADER = Path(__file__).resolve().parent.parent / "include" / "ezops_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ezops_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _hip.lib()
    names = declared_functions()
    assert len(names) >= 17
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_hip.SIGNATURES), "ctypes table and header disagree"
    assert lib.ezops_hip_abi_version() == _hip.ABI_VERSION


def test_struct_layout_matches_header():
    # int64 x7, float (+pad), then 16 eight-byte fields (15 pointers, max_kv_len)
    assert ctypes.sizeof(_hip.Qwen3LayerParams) == 7 * 8 + 8 + 16 * 8


def test_invalid_arguments_return_einval():
    lib = _hip.lib()
    assert lib.ezops_gemv_bf16(None, None, None, 16, 16, None) == _hip.EINVAL
    assert b"null" in lib.ezops_hip_last_error()
    assert lib.ezops_softmax_f32(None, None, 4, 4, None) == _hip.EINVAL
    assert lib.ezops_hbm_probe(9, None, None, None, 16, 1.0, None) == _hip.EINVAL
    with pytest.raises(RuntimeError, match="null"):
        _hip.call("ezops_rmsnorm_f32", None, None, 1, 1, 1e-6, None)


def test_workspace_sizes():
    lib = _hip.lib()
    assert lib.ezops_reduce_sum_workspace_size(1 << 28) >= 4 * 1024
    assert lib.ezops_attn_decode_workspace_size(32, 32, 8, 8192, 128) > 0
    assert lib.ezops_attn_decode_workspace_size(0, 32, 8, 8192, 128) == 0
    p = _hip.Qwen3LayerParams(B=1, S=16384, HS=4096, IS=12288, H=32, Hkv=8, D=128)
    assert lib.ezops_qwen3_layer_workspace_size(ctypes.byref(p)) > 12288 * 2


def test_new_entry_points_reject_bad_arguments():
    """Validation of the paged / prefill / step / GEMM entries happens before
    any device call, so it runs without a GPU.  Non-null dummy pointers are
    never dereferenced on these paths."""
    lib = _hip.lib()
    d = 64  # a non-null address that is never touched
    # paged attention: page size must be a power of two >= 32
    rc = lib.ezops_paged_attn_decode_bf16(d, d, d, d, d, d, 2, 32, 8, 128, 16, 48, 4, 0, 0.0, d, 1 << 20, None)
    assert rc == _hip.EINVAL and b"page_size" in lib.ezops_hip_last_error()
    # prefill attention: head_dim 128 only
    rc = lib.ezops_prefill_attn_bf16(d, d, d, d, d, None, 1, 16, 8, 8, 64, 64, 16, None, 0, 0, 0.0, None)
    assert rc == _hip.EINVAL and b"head_dim" in lib.ezops_hip_last_error()
    # prefill attention: cache offsets are 32-bit, so S < 2^23 rows
    rc = lib.ezops_prefill_attn_bf16(d, d, d, d, d, None, 1, 16, 8, 8, 1 << 23, 128, 16, None, 0, 0, 0.0, None)
    assert rc == _hip.EINVAL and b"2^23" in lib.ezops_hip_last_error()
    # prefill GEMM: empty shapes, null operands, leading dimensions below the row length
    assert lib.ezops_gemm_bf16(d, 16, d, d, 16, None, 0, 16, 16, None, 0, None) == _hip.EINVAL
    assert lib.ezops_gemm_bf16(None, 16, d, d, 16, None, 4, 16, 16, None, 0, None) == _hip.EINVAL
    assert lib.ezops_gemm_bf16(d, 8, d, d, 16, None, 4, 16, 16, None, 0, None) == _hip.EINVAL
    assert lib.ezops_gemm_workspace_size() == 0
    # fused gate/up + SwiGLU GEMM: null X / W / Y, ldx < K, IS < 1 (addresses 16-byte aligned)
    a = 4096
    for args in [(None, 64, a, a, 128, 16, 128, 64), (a, 64, None, a, 128, 16, 128, 64),
                 (a, 64, a, None, 128, 16, 128, 64), (a, 32, a, a, 128, 16, 128, 64),
                 (a, 64, a, a, 128, 16, 0, 64), (a, 64, a, a, 128, 16, 128, 0)]:
        assert lib.ezops_gemm_swiglu_bf16(*args, None) == _hip.EINVAL, args
    # layer prefill: cu_seqlens is required
    p = _hip.Qwen3LayerParams(B=1, S=128, HS=256, IS=512, H=4, Hkv=2, D=128, hidden=d, K_cache=d, V_cache=d,
                              Wqkv=d, Wo=d, Wgu=d, Wd=d, out=d)
    assert lib.ezops_qwen3_prefill_bf16(ctypes.byref(p), 16, None, 16, None, 0, 0, d, 1 << 20, None) == _hip.EINVAL
    # decode step: layers must share one shape, and there must be at least one
    layers = (_hip.Qwen3LayerParams * 2)()
    for i, hs in enumerate((256, 512)):
        layers[i] = _hip.Qwen3LayerParams(B=1, S=128, HS=hs, IS=512, H=4, Hkv=2, D=128, hidden=d, out=d)
    rc = lib.ezops_qwen3_decode_step_bf16(layers, 2, None, 0, 0, None, None, 0, None, d, 1 << 20, None)
    assert rc == _hip.EINVAL and b"shape" in lib.ezops_hip_last_error()
    assert lib.ezops_qwen3_decode_step_bf16(layers, 0, None, 0, 0, None, None, 0, None, d, 1 << 20, None) == _hip.EINVAL
    # QK-norm + RoPE: zero kv heads is rejected before the head-group division
    rc = lib.ezops_qk_norm_rope_bf16(d, 128, d, 128, d, 128, None, None, None, None, d, d, d, d, 1, 4, 0, 128, 16, 0,
                                     None, 0, 1e-6, None)
    assert rc == _hip.EINVAL and b"num_kv_heads" in lib.ezops_hip_last_error()
    # a paged decode step needs page_size a power of two dividing S
    same = (_hip.Qwen3LayerParams * 1)()
    same[0] = _hip.Qwen3LayerParams(B=1, S=128, HS=256, IS=512, H=4, Hkv=2, D=128, hidden=d, out=d)
    assert lib.ezops_qwen3_decode_step_bf16(same, 1, d, 4, 48, None, None, 0, None, d, 1 << 30, None) == _hip.EINVAL


def test_layer_entries_reject_before_any_launch():
    """Every stage's limits are checked before the first launch, so these
    return EINVAL on a machine without a GPU (a launch would fail with a
    device error instead) and, on a GPU, leave the cache and stream untouched."""
    lib = _hip.lib()
    d = 4096  # a 16-byte aligned non-null address that is never touched
    ptrs = dict(hidden=d, K_cache=d, V_cache=d, Wqkv=d, Wo=d, Wgu=d, Wd=d, out=d)

    def layer(**kw):
        shape = dict(B=1, S=128, HS=256, IS=512, H=4, Hkv=2, D=128)
        shape.update(kw)
        return _hip.Qwen3LayerParams(**shape, **ptrs)

    # decode layer: the attention stage's head_dim, group size and length bound
    for kw, text in [(dict(D=96), b"head_dim"), (dict(H=64, Hkv=2), b"group size"),
                     (dict(max_kv_len=-1), b"max_kv_len")]:
        rc = lib.ezops_qwen3_dense_decode_bf16(ctypes.byref(layer(**kw)), d, 1 << 30, None)
        assert rc == _hip.EINVAL and text in lib.ezops_hip_last_error(), (kw, lib.ezops_hip_last_error())
    # decode step over a paged cache: a later layer without kv_lens
    layers = (_hip.Qwen3LayerParams * 2)(layer(kv_lens=d), layer())
    rc = lib.ezops_qwen3_decode_step_bf16(layers, 2, d, 8, 64, None, None, 0, None, d, 1 << 30, None)
    assert rc == _hip.EINVAL and b"kv_lens" in lib.ezops_hip_last_error()
    # prefill: the attention stage's head_dim, group size, cache bound and alignment
    cu = d
    for kw, text in [(dict(D=64), b"head_dim"), (dict(H=32, Hkv=2), b"group size"),
                     (dict(S=1 << 23), b"2^23")]:
        rc = lib.ezops_qwen3_prefill_bf16(ctypes.byref(layer(**kw)), 16, cu, 16, None, 0, 0, d, 1 << 40, None)
        assert rc == _hip.EINVAL and text in lib.ezops_hip_last_error(), (kw, lib.ezops_hip_last_error())
    p = layer()
    p.K_cache = d + 2
    rc = lib.ezops_qwen3_prefill_bf16(ctypes.byref(p), 16, cu, 16, None, 0, 0, d, 1 << 40, None)
    assert rc == _hip.EINVAL and b"16-byte" in lib.ezops_hip_last_error()


def test_linear_stage_rejects_unaligned_staging_workspace():
    lib = _hip.lib()
    d = 4096
    need = lib.ezops_linear_stage_workspace_size(8, 256, 1)
    rc = lib.ezops_linear_stage_bf16(d, 256, d, None, d, 64, None, 0, None, 1, 1e-6, 0, 8, 64, 256, d + 2, need, None)
    assert rc == _hip.EINVAL and b"16-byte aligned workspace" in lib.ezops_hip_last_error()


def test_workspaces_must_be_16_byte_aligned():
    lib = _hip.lib()
    d, odd = 4096, 4096 + 4
    assert lib.ezops_reduce_sum_f32(d, d, 1 << 20, odd, 1 << 30, None) == _hip.EINVAL
    assert b"aligned" in lib.ezops_hip_last_error()
    assert lib.ezops_attn_decode_bf16(d, d, d, d, 8, 32, 8, 8192, 128, None, 0, 0.0, odd, 1 << 30, None) == _hip.EINVAL
    assert b"aligned" in lib.ezops_hip_last_error()
    assert lib.ezops_o_proj_ffn_bf16(d, d, d, None, d, d, d, d, 1, 4096, 12288, 4096, 1e-6, odd, 1 << 30,
                                     None) == _hip.EINVAL
    assert b"aligned" in lib.ezops_hip_last_error()
    p = _hip.Qwen3LayerParams(B=1, S=128, HS=256, IS=512, H=4, Hkv=2, D=128, hidden=d, K_cache=d, V_cache=d,
                              Wqkv=d, Wo=d, Wgu=d, Wd=d, out=d)
    assert lib.ezops_qwen3_dense_decode_bf16(ctypes.byref(p), odd, 1 << 30, None) == _hip.EINVAL
    assert b"aligned" in lib.ezops_hip_last_error()
    assert lib.ezops_qwen3_decode_step_bf16((_hip.Qwen3LayerParams * 1)(p), 1, None, 0, 0, None, None, 0, None,
                                            odd, 1 << 30, None) == _hip.EINVAL
    assert b"aligned" in lib.ezops_hip_last_error()
    assert lib.ezops_qwen3_prefill_bf16(ctypes.byref(p), 16, d, 16, None, 0, 0, odd, 1 << 30, None) == _hip.EINVAL
    assert b"aligned" in lib.ezops_hip_last_error()


def test_batched_linear_rejects_huge_k():
    lib = _hip.lib()
    d, K = 4096, 1 << 26
    rc = lib.ezops_linear_bf16(d, K, d, d, 16, 8, 16, K, None)
    assert rc == _hip.EINVAL and b"2^26" in lib.ezops_hip_last_error()
