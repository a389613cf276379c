from . import fused_qk_norm_rope_hip  # noqa: F401
