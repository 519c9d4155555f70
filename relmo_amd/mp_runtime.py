"""Loading of ``relm_mp_ops.so`` and the runtime compatibility policy.

Behaviour follows relmo's ``src/relmo/ops/mp_runtime.py``:

* ``torch`` is imported lazily-tolerant: without torch the module still
  imports, ``available()`` is False and the ops raise ``ModuleNotFoundError``
  (mp_runtime.py:21-42);
* environment flags ``RELM_MP_ENABLE``, ``RELM_MP_FALLBACK`` (``python`` |
  ``error``) and ``RELM_MP_TORCH_VERSION_POLICY`` (``forward`` | ``strict``)
  keep their meaning (mp_runtime.py:44-69).  One deliberate difference: with
  ``RELM_MP_FALLBACK`` unset (or invalid) the policy is relmo's ``python`` for
  CPU tensors but ``error`` for GPU tensors, so a GPU run never falls back to
  ATen silently when the HIP library is missing; setting the variable applies
  it to every tensor, as in relmo;
* the library is found by globbing ``relm_mp_ops*.so`` / ``librelm_mp_ops*.so``
  in the package directory (mp_runtime.py:97-125), loaded with
  ``torch.ops.load_library`` and must register every op of
  ``REQUIRED_NAMESPACE_OPS`` (mp_runtime.py:128-159);
* ``build_info()`` is parsed as ``k=v;`` pairs and checked against the running
  torch (mp_runtime.py:175-228).
"""

from __future__ import annotations

import os
import re
import warnings
from pathlib import Path

from .mp_constants import REQUIRED_NAMESPACE_OPS

try:  # pragma: no cover - exercised only where torch is missing
    import torch
except Exception as exc:  # pragma: no cover
    torch = None
    TORCH_IMPORT_ERROR: Exception | None = exc
else:
    TORCH_IMPORT_ERROR = None

_LIB_LOADED = False
_LIB_LOAD_ERROR: Exception | None = None
_LIB_PATH: Path | None = None
_BUILD_INFO_CACHE: dict[str, str] | None = None
_OPS_NAMESPACE = "relm_mp"
_RUNTIME_COMPAT_VALIDATED = False

_FALSE_WORDS = frozenset({"0", "false", "no", "off"})
_MAJOR_MINOR = re.compile(r"^(\d+)\.(\d+)")

_FALLBACK_MODES = frozenset({"python", "error"})


def require_torch(feature_name: str) -> None:
    if torch is None:
        raise ModuleNotFoundError(f"{feature_name} requires torch.") from TORCH_IMPORT_ERROR


def env_bool_any(names: tuple[str, ...], default: bool) -> bool:
    """First set variable of ``names`` read as a boolean; ``default`` if none is set."""

    for name in names:
        raw = os.getenv(name)
        if raw is not None:
            return raw.strip().lower() not in _FALSE_WORDS
    return default


def env_first(names: tuple[str, ...], default: str | None = None) -> str | None:
    for name in names:
        raw = os.getenv(name)
        if raw is not None:
            return raw
    return default


def _choice(name: str, allowed: frozenset[str], default: str) -> str:
    raw = (env_first((name,), default) or default).strip().lower()
    return raw if raw in allowed else default


def fallback_mode(tensor: object | None = None) -> str:
    """``python`` or ``error`` for ops on ``tensor``: ``RELM_MP_FALLBACK`` where it
    names one of them, else ``error`` for GPU tensors and ``python`` otherwise."""

    raw = env_first(("RELM_MP_FALLBACK",))
    if raw is not None and raw.strip().lower() in _FALLBACK_MODES:
        return raw.strip().lower()
    return "error" if getattr(tensor, "is_cuda", False) else "python"


def torch_version_policy() -> str:
    return _choice("RELM_MP_TORCH_VERSION_POLICY", frozenset({"forward", "strict"}), "forward")


def runtime_cuda_tag() -> str:
    """``cu<ver>`` for CUDA builds of torch; ``cpu`` otherwise (ROCm included)."""

    require_torch("mp runtime compatibility checks")
    cuda = getattr(torch.version, "cuda", None)
    if not cuda:
        return "cpu"
    return "cu" + str(cuda).replace(".", "")


def major_minor(version: str) -> tuple[int, int]:
    match = _MAJOR_MINOR.match(version)
    if match is None:
        raise RuntimeError(f"Could not parse torch version {version!r}.")
    return int(match.group(1)), int(match.group(2))


def parse_build_info(raw: str) -> dict[str, str]:
    info: dict[str, str] = {}
    for item in raw.split(";"):
        key, sep, value = item.partition("=")
        if sep:
            info[key.strip()] = value.strip()
    return info


def package_dir() -> Path:
    return Path(__file__).resolve().parent


def candidate_libraries() -> list[Path]:
    patterns = ("relm_mp_ops*.so", "librelm_mp_ops*.so")
    found: list[Path] = []
    seen: set[Path] = set()
    for pattern in patterns:
        for path in sorted(package_dir().glob(pattern)):
            resolved = path.resolve()
            if resolved not in seen:
                seen.add(resolved)
                found.append(resolved)
    return found


def ensure_loaded() -> None:
    """Load the op library once; raise if none of the candidates is usable."""

    global _LIB_LOADED, _LIB_LOAD_ERROR, _LIB_PATH
    if _LIB_LOADED:
        return
    require_torch("relmo_amd.mp")
    last_error: Exception | None = None
    for candidate in candidate_libraries():
        try:
            torch.ops.load_library(str(candidate))
            namespace = getattr(torch.ops, _OPS_NAMESPACE, None)
            missing = [op for op in REQUIRED_NAMESPACE_OPS if not hasattr(namespace, op)]
            if namespace is None or missing:
                raise RuntimeError(f"Loaded {candidate} but torch.ops.relm_mp is incomplete.")
        except Exception as exc:  # pragma: no cover - depends on the local build
            last_error = exc
            continue
        _LIB_LOADED = True
        _LIB_LOAD_ERROR = None
        _LIB_PATH = candidate
        return
    _LIB_LOAD_ERROR = last_error
    if last_error is not None:
        raise RuntimeError("Failed to load relm_mp custom op library.") from last_error
    raise FileNotFoundError(
        "Could not find relm_mp custom op library in the relmo_amd package directory "
        "(build it with `python -m relmo_amd.csrc.build`)."
    )


def loaded_library() -> Path | None:
    return _LIB_PATH


def ops_namespace():
    require_torch("mp custom ops")
    return getattr(torch.ops, _OPS_NAMESPACE)


def ensure_runtime_compat_once() -> None:
    global _RUNTIME_COMPAT_VALIDATED
    if not _RUNTIME_COMPAT_VALIDATED:
        assert_runtime_compat()
        _RUNTIME_COMPAT_VALIDATED = True


def assert_runtime_compat() -> dict[str, str]:
    """Raise if the running torch cannot use the loaded library; return its build info."""

    global _BUILD_INFO_CACHE
    require_torch("mp compatibility checks")
    ensure_loaded()
    if _BUILD_INFO_CACHE is None:
        _BUILD_INFO_CACHE = parse_build_info(ops_namespace().build_info())
    info = _BUILD_INFO_CACHE

    build_torch = info.get("build_torch")
    if not build_torch:
        raise RuntimeError("mp build metadata is missing build_torch.")
    runtime_torch = str(torch.__version__)
    built = major_minor(build_torch)
    running = major_minor(runtime_torch)
    if built != running:
        if torch_version_policy() == "strict":
            raise RuntimeError(
                f"mp torch version mismatch: built against {build_torch}, runtime is "
                f"{runtime_torch}. Expected matching major.minor."
            )
        if built[0] != running[0]:
            raise RuntimeError(
                f"mp torch major version mismatch: built against {build_torch}, "
                f"runtime is {runtime_torch}."
            )
        if running < built:
            raise RuntimeError(
                f"mp torch runtime is older than the build torch: built against {build_torch}, "
                f"runtime is {runtime_torch}. Rebuild against the older torch or upgrade the "
                "runtime torch."
            )
        warnings.warn(
            f"mp torch version drift: built against {build_torch}, runtime is {runtime_torch}. "
            "Continuing because RELM_MP_TORCH_VERSION_POLICY=forward. "
            "Treat this as compatibility-by-test, not ABI-guaranteed.",
            RuntimeWarning,
            stacklevel=2,
        )

    build_tag = info.get("build_cuda_tag", "cpu")
    running_tag = runtime_cuda_tag()
    if build_tag != "cpu" and build_tag != running_tag:
        raise RuntimeError(f"mp CUDA tag mismatch: built for {build_tag}, runtime is {running_tag}.")
    return info


def available() -> bool:
    """True when the op library loads and fits the running torch."""

    if torch is None:
        return False
    try:
        ensure_loaded()
        assert_runtime_compat()
    except Exception:
        return False
    return True


__all__ = [
    "TORCH_IMPORT_ERROR",
    "assert_runtime_compat",
    "available",
    "candidate_libraries",
    "ensure_loaded",
    "ensure_runtime_compat_once",
    "env_bool_any",
    "env_first",
    "fallback_mode",
    "loaded_library",
    "major_minor",
    "ops_namespace",
    "parse_build_info",
    "require_torch",
    "runtime_cuda_tag",
    "torch",
    "torch_version_policy",
]
