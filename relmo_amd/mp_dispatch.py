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


__all__ = ["namespace_has_op", "ops_namespace", "should_use_custom"]
