from . import softmax_hip  # noqa: F401
