from . import gemv_hip  # noqa: F401
