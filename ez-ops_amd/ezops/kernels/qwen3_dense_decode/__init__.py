from . import qwen3_decode_step_hip, qwen3_dense_decode_hip, qwen3_prefill_hip  # noqa: F401
