from . import qwen3_dense_decode_hip  # noqa: F401
