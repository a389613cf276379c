from . import fused_o_proj_ffn_hip  # noqa: F401
