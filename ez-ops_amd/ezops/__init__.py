"""ez-ops decode-path ops on a single MI355X HIP backend.

Same public API as the reference package (ezops/__init__.py:1-17) for the
decode hot path: op specs, the kernel registry, and the ``hip`` backend
registered under every op name.
"""

from . import kernels as _kernels  # noqa: F401  (registers the hip backend)
from .ops.attn_decode import AttnDecodeOp
from .ops.base_op import Op
from .ops.fused_o_proj_ffn import FusedOProjFfnOp
from .ops.fused_qk_norm_rope import FusedQkNormRopeOp
from .ops.gemv import GemvOp
from .ops.paged_attn_decode import PagedAttnDecodeOp
from .ops.prefill_attn import PrefillAttnOp
from .ops.qwen3_decode_step import Qwen3DecodeStepOp
from .ops.qwen3_dense_decode import Qwen3DenseDecodeOp
from .ops.qwen3_prefill import Qwen3PrefillOp
from .ops.reduce import ReduceOp
from .ops.rmsnorm import RmsNormOp
from .ops.softmax import SoftmaxOp
from .ops.utils.roofline import RooflineResult
from .registry import get_kernel, list_backends, list_ops, register_kernel

__all__ = [
    "AttnDecodeOp", "FusedOProjFfnOp", "FusedQkNormRopeOp", "GemvOp", "Op", "PagedAttnDecodeOp",
    "PrefillAttnOp", "Qwen3DecodeStepOp", "Qwen3DenseDecodeOp", "Qwen3PrefillOp", "ReduceOp", "RmsNormOp",
    "RooflineResult", "SoftmaxOp", "get_kernel", "list_backends", "list_ops", "register_kernel",
]
