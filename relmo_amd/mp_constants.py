"""Codes shared by the loader, the dispatch policy and the fallbacks.

Values follow relmo's ``src/relmo/ops/mp_constants.py:7-26`` so that callers
passing integer modes keep working.
"""

from __future__ import annotations

from typing import Final

MODE_SUM: Final[int] = 0
MODE_LOGSUMEXP: Final[int] = 1
MODE_MEAN: Final[int] = 2

PW_IDENTITY: Final[int] = 0
PW_RELU: Final[int] = 1
PW_MISH: Final[int] = 2
PW_GELU_NONE: Final[int] = 3
PW_GELU_TANH: Final[int] = 4
PW_SILU: Final[int] = 5
PW_TANH: Final[int] = 6

# Ops the loaded library must provide (mp_constants.py:19-26 of the reference).
REQUIRED_NAMESPACE_OPS: Final[tuple[str, ...]] = (
    "fanout_scatter",
    "fanout_scatter_backward",
    "fanin_reduce",
    "fanin_reduce_sum_backward",
    "fanin_reduce_logsumexp_backward",
    "build_info",
)

_ACTIVATION_CODES: Final[dict[str, int]] = {
    "identity": PW_IDENTITY,
    "relu": PW_RELU,
    "mish": PW_MISH,
    "silu": PW_SILU,
    "tanh": PW_TANH,
}


def activation_code(signature: tuple[object, ...] | None) -> int | None:
    """Integer code of an activation signature such as ``("gelu", "tanh")``.

    Returns ``None`` for an empty signature or an activation without a code
    (reference: ``mp_constants.py:37-60``).
    """

    if not signature:
        return None
    kind = str(signature[0])
    if kind == "gelu":
        approximate = str(signature[1]) if len(signature) > 1 else "none"
        return {"none": PW_GELU_NONE, "tanh": PW_GELU_TANH}.get(approximate)
    return _ACTIVATION_CODES.get(kind)
