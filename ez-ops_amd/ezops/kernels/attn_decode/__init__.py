from . import attn_decode_hip, paged_attn_decode_hip, prefill_attn_hip  # noqa: F401
