from . import attn_decode_hip  # noqa: F401
