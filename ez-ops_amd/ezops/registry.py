"""Op-name/backend -> kernel-class registry.

Mirrors the reference's registry contract (ezops/registry.py:4-54): a
``(op_name, backend)`` key maps to one kernel class, duplicate keys raise
ValueError, the class is stamped with ``op_name``/``backend``, and lookups of
an unknown key raise KeyError naming the backends that do exist.  The
reference wraps ``__call__`` in a TileLang cache-naming scope
(registry.py:24-30); there is no JIT cache in this backend, so classes are
registered unchanged.
"""

_KERNEL_REGISTRY: dict[tuple[str, str], type] = {}


def register_kernel(op_name: str, backend: str):
    def decorator(cls):
        key = (op_name, backend)
        prev = _KERNEL_REGISTRY.get(key)
        if prev is not None:
            raise ValueError(
                f"Kernel already registered for ({op_name!r}, {backend!r}): {prev.__name__}"
            )
        cls.op_name = op_name
        cls.backend = backend
        _KERNEL_REGISTRY[key] = cls
        return cls

    return decorator


def get_kernel(op_name: str, backend: str) -> type:
    try:
        return _KERNEL_REGISTRY[(op_name, backend)]
    except KeyError:
        have = list_backends(op_name)
        raise KeyError(
            f"No kernel registered for ({op_name!r}, {backend!r}). "
            f"Available backends for {op_name!r}: {have!r}"
        ) from None


def list_backends(op_name: str) -> list[str]:
    return [b for (n, b) in _KERNEL_REGISTRY if n == op_name]


def list_ops() -> list[str]:
    return sorted({n for (n, _) in _KERNEL_REGISTRY})
