from . import rmsnorm_hip  # noqa: F401
