"""Choice between the custom ops and the ATen fallbacks.

Follows relmo's ``src/relmo/ops/mp_dispatch.py:15-36``: ``RELM_MP_ENABLE=0``
selects the fallback; otherwise the library is loaded and checked once, and a
failure either raises (``RELM_MP_FALLBACK=error``, the default here) or falls
back to ATen (``RELM_MP_FALLBACK=python``).
"""

from __future__ import annotations

from .mp_runtime import (
    ensure_loaded,
    ensure_runtime_compat_once,
    env_bool_any,
    fallback_mode,
    ops_namespace,
    torch,
)


def should_use_custom(op_name: str) -> bool:
    """Whether ``op_name`` runs on the custom op library under the current policy."""

    if not env_bool_any(("RELM_MP_ENABLE",), True):
        return False
    try:
        ensure_runtime_compat_once()
    except Exception as exc:
        if fallback_mode() == "error":
            raise RuntimeError(f"Custom mp op {op_name} is unavailable.") from exc
        return False
    return True


def namespace_has_op(op_name: str) -> bool:
    if torch is None:
        return False
    try:
        ensure_loaded()
    except Exception:
        return False
    return hasattr(ops_namespace(), op_name)


def require_available_custom_op(op_name: str) -> None:
    """Raise under the ``error`` fallback policy: the loaded library lacks ``op_name``."""

    if fallback_mode() == "error":
        raise RuntimeError(f"Custom mp op {op_name} is unavailable in the loaded relm_mp library.")


def use_custom_namespace_op(
    op_name: str,
    *,
    tensor: object | None = None,
    require_cuda: bool = False,
) -> bool:
    """Whether ``op_name`` is called directly on ``torch.ops.relm_mp``."""

    if require_cuda and (tensor is None or not bool(getattr(tensor, "is_cuda", False))):
        return False
    return should_use_custom(op_name) and namespace_has_op(op_name)


def dispatch_namespace_op(
    op_name: str,
    *args,
    fallback,
    tensor: object | None = None,
    require_cuda: bool = False,
    enforce_fallback_policy: bool = True,
):
    """Call ``torch.ops.relm_mp.<op_name>`` or ``fallback`` with ``args``.

    Follows ``src/relmo/ops/mp_dispatch.py:47-81``: the library op when the
    policy allows it and the library has it; otherwise the fallback, except that
    under the ``error`` policy a library without the op raises.
    """

    if use_custom_namespace_op(op_name, tensor=tensor, require_cuda=require_cuda):
        return getattr(ops_namespace(), op_name)(*args)
    if enforce_fallback_policy and should_use_custom(op_name):
        require_available_custom_op(op_name)
    return fallback(*args)


__all__ = [
    "dispatch_namespace_op",
    "namespace_has_op",
    "ops_namespace",
    "require_available_custom_op",
    "should_use_custom",
    "use_custom_namespace_op",
]
