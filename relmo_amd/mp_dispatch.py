"""Routing of the facade's calls: the ``relm_mp`` library or the ATen fallbacks.

Every facade function asks one question, :func:`library_op`: which callable of
the library serves this op for this tensor, or ``None`` when the fallback runs.
The answer follows relmo's dispatch policy (``src/relmo/ops/mp_dispatch.py:15-78``),
whose environment variables and error messages are the contract callers match:

* ``RELM_MP_ENABLE=0`` routes every op to its fallback;
* otherwise the library is loaded and checked against the running torch once;
  if that fails, the fallback policy (:func:`mp_runtime.fallback_mode`)
  either raises ``Custom mp op <name> is unavailable.`` or routes to the
  fallback;
* an op the loaded library does not register (the optional pack and LGAN
  ops) runs its fallback, or raises
  ``Custom mp op <name> is unavailable in the loaded relm_mp library.`` under
  the ``error`` policy;
* ``gpu_only`` ops (the LGAN reductions) run on the library for GPU tensors
  only.

The policy depends on the tensor: with ``RELM_MP_FALLBACK`` unset, CPU tensors
fall back quietly as in relmo, GPU tensors raise (a GPU run never drops to
ATen without saying so).
"""

from __future__ import annotations

from .mp_runtime import ensure_runtime_compat_once, env_bool_any, fallback_mode, ops_namespace


def _on_gpu(tensor: object | None) -> bool:
    return bool(getattr(tensor, "is_cuda", False))


def library_ready(op_name: str, tensor: object | None = None) -> bool:
    """Whether the policy lets ``op_name`` run on the library at all.

    Raises ``RuntimeError`` where the library is wanted but unusable and the
    policy for ``tensor`` is ``error``.
    """

    if not env_bool_any(("RELM_MP_ENABLE",), True):
        return False
    try:
        ensure_runtime_compat_once()
    except Exception as exc:
        if fallback_mode(tensor) == "error":
            raise RuntimeError(f"Custom mp op {op_name} is unavailable.") from exc
        return False
    return True


def library_op(op_name: str, *, tensor: object | None = None, gpu_only: bool = False):
    """The library's ``torch.ops.relm_mp.<op_name>``, or ``None`` where the fallback runs."""

    if gpu_only and not _on_gpu(tensor):
        return None
    if not library_ready(op_name, tensor):
        return None
    op = getattr(ops_namespace(), op_name, None)
    if op is None and fallback_mode(tensor) == "error":
        raise RuntimeError(f"Custom mp op {op_name} is unavailable in the loaded relm_mp library.")
    return op


def run_op(op_name: str, *args, fallback, tensor: object | None = None, gpu_only: bool = False):
    """``op_name(*args)`` on the library, or ``fallback(*args)`` where the policy says so."""

    op = library_op(op_name, tensor=tensor, gpu_only=gpu_only)
    return fallback(*args) if op is None else op(*args)


__all__ = ["library_op", "library_ready", "run_op"]
