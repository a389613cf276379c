"""Importing this package registers the single ``hip`` backend of every op."""

from . import (  # noqa: F401
    attn_decode,
    fused_o_proj_ffn,
    fused_qk_norm_rope,
    gemv,
    qwen3_dense_decode,
    reduce,
    rmsnorm,
    softmax,
)
