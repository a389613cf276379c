from . import reduce_hip  # noqa: F401
