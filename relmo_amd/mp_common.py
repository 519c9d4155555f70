"""Argument checks and concatenation helpers of the ATen fallbacks.

Restates relmo's ``src/relmo/ops/mp_common.py:14-97`` (messages included), so
the fallbacks raise ``ValueError`` exactly where the reference's do.
"""

from __future__ import annotations

from typing import Sequence

from .mp_runtime import torch


def _shape(tensor: torch.Tensor) -> tuple[int, ...]:
    return tuple(int(v) for v in tensor.shape)


def require_non_empty(op_name: str, values: Sequence[object], what: str) -> None:
    if not values:
        raise ValueError(f"{op_name} requires at least one {what}.")


def require_matching_lengths(op_name: str, *named: tuple[str, Sequence[object]]) -> None:
    if not named:
        return
    expected = len(named[0][1])
    if any(len(seq) != expected for _, seq in named[1:]):
        got = ", ".join(f"{name}={len(seq)}" for name, seq in named)
        raise ValueError(f"{op_name} expects matching sequence lengths, got {got}.")


def require_rank(op_name: str, name: str, tensor: torch.Tensor, rank: int) -> None:
    if tensor.dim() != rank:
        raise ValueError(f"{op_name} expects {name} to be rank-{rank}, got shape {_shape(tensor)}.")


def require_int64(op_name: str, name: str, tensor: torch.Tensor) -> None:
    if tensor.dtype != torch.int64:
        raise ValueError(f"{op_name} expects {name} to have dtype int64, got {tensor.dtype}.")


def require_positive_arity(op_name: str, arity: int) -> int:
    value = int(arity)
    if value <= 0:
        raise ValueError(f"{op_name} expects arity > 0.")
    return value


def cat_or_single(parts: Sequence[torch.Tensor], *, dim: int = 0) -> torch.Tensor:
    """The only part itself, else ``torch.cat``."""

    return parts[0] if len(parts) == 1 else torch.cat(list(parts), dim=dim)


def cat_or_empty(parts: Sequence[torch.Tensor], *, empty: torch.Tensor, dim: int = 0) -> torch.Tensor:
    return empty if not parts else cat_or_single(parts, dim=dim)


def empty_index(device) -> torch.Tensor:
    return torch.empty(0, device=device, dtype=torch.int64)


def indexed_sum_or_mean(source_embeddings, source_index, target_index, dim_size: int, mode: int,
                        *, op_name: str):
    """Rows ``target_index[e]`` of a [dim_size, emb] result receive
    ``source_embeddings[source_index[e]]``: summed, or averaged over the messages
    of each row in mean mode (``mp_common.py:88-118``)."""

    from .mp_constants import MODE_MEAN, MODE_SUM

    if mode not in (MODE_SUM, MODE_MEAN):
        raise ValueError(f"{op_name} supports only sum and mean modes.")
    out = source_embeddings.new_zeros((int(dim_size), int(source_embeddings.size(-1))))
    if int(source_index.numel()) == 0 or int(dim_size) == 0:
        return out
    out.index_add_(0, target_index, source_embeddings.index_select(0, source_index))
    if mode == MODE_MEAN:
        counts = out.new_zeros((int(dim_size), 1))
        counts.index_add_(
            0, target_index,
            torch.ones((int(target_index.numel()), 1), device=out.device, dtype=out.dtype),
        )
        out = out / counts.clamp_min_(1.0)
    return out


__all__ = [
    "cat_or_empty",
    "cat_or_single",
    "empty_index",
    "indexed_sum_or_mean",
    "require_int64",
    "require_matching_lengths",
    "require_non_empty",
    "require_positive_arity",
    "require_rank",
]
