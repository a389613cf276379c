from .attn_decode import AttnDecodeOp
from .base_op import Op
from .fused_o_proj_ffn import FusedOProjFfnOp
from .fused_qk_norm_rope import FusedQkNormRopeOp
from .gemv import GemvOp
from .paged_attn_decode import PagedAttnDecodeOp
from .prefill_attn import PrefillAttnOp
from .qwen3_decode_step import Qwen3DecodeStepOp
from .qwen3_dense_decode import Qwen3DenseDecodeOp
from .qwen3_prefill import Qwen3PrefillOp
from .reduce import ReduceOp
from .rmsnorm import RmsNormOp
from .softmax import SoftmaxOp
from .utils.roofline import RooflineResult

__all__ = [
    "AttnDecodeOp", "FusedOProjFfnOp", "FusedQkNormRopeOp", "GemvOp", "Op", "PagedAttnDecodeOp",
    "PrefillAttnOp", "Qwen3DecodeStepOp", "Qwen3DenseDecodeOp", "Qwen3PrefillOp", "ReduceOp", "RmsNormOp",
    "RooflineResult", "SoftmaxOp",
]
