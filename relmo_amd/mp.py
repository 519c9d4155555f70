"""Public op facade: the API of relmo's ``relmo.ops.mp`` for this path.

``fanout_scatter`` and ``fanin_reduce`` keep the reference's signatures and
dispatch (``src/relmo/ops/mp.py:43-70``): modes other than sum (0) and
logsumexp (1) go to the ATen fallback, which raises ``ValueError``; otherwise
the custom ops run through autograd Functions unless the policy selects the
fallback.
"""

from __future__ import annotations

from .mp_autograd import (
    _FaninReduceLogSumExpFunction,
    _FaninReduceSumFunction,
    _FanoutScatterFunction,
)
from .mp_constants import MODE_LOGSUMEXP, MODE_MEAN, MODE_SUM, activation_code
from .mp_dispatch import should_use_custom
from .mp_pack import fanin_reduce_python, fanout_scatter_python
from .mp_runtime import TORCH_IMPORT_ERROR, assert_runtime_compat, available, require_torch, torch


def fanout_scatter(
    x_cat: torch.Tensor,
    src_global_idx: torch.Tensor,
    flat_dst: torch.Tensor,
    out_rows: int,
) -> torch.Tensor:
    """``out[flat_dst[e]] = x_cat[src_global_idx[e]]``; other rows are zero."""

    require_torch("fanout_scatter")
    if should_use_custom("fanout_scatter"):
        return _FanoutScatterFunction.apply(x_cat, src_global_idx, flat_dst, int(out_rows))
    return fanout_scatter_python(x_cat, src_global_idx, flat_dst, int(out_rows))


def fanin_reduce(
    rel_flat: torch.Tensor,
    flat_src: torch.Tensor,
    dst_idx: torch.Tensor,
    dim_size: int,
    mode: int,
) -> torch.Tensor:
    """Reduce ``rel_flat[flat_src[e]]`` onto ``dst_idx[e]``: sum (0) or logsumexp (1)."""

    require_torch("fanin_reduce")
    mode = int(mode)
    if mode not in (MODE_SUM, MODE_LOGSUMEXP):
        return fanin_reduce_python(rel_flat, flat_src, dst_idx, int(dim_size), mode)
    if should_use_custom("fanin_reduce"):
        fn = _FaninReduceSumFunction if mode == MODE_SUM else _FaninReduceLogSumExpFunction
        return fn.apply(rel_flat, flat_src, dst_idx, int(dim_size))
    return fanin_reduce_python(rel_flat, flat_src, dst_idx, int(dim_size), mode)


__all__ = [
    "MODE_LOGSUMEXP",
    "MODE_MEAN",
    "MODE_SUM",
    "TORCH_IMPORT_ERROR",
    "activation_code",
    "assert_runtime_compat",
    "available",
    "fanin_reduce",
    "fanout_scatter",
]
