"""ATen formulations of the two ops (the reference's ``python_only`` path).

Restates relmo's ``src/relmo/ops/mp_pack.py:19-63``: ``index_select`` +
``index_copy_`` for the fanout, ``index_add_`` for the sum fanin and the
``scatter_reduce_(amax)`` / ``exp`` / ``scatter_add_`` / ``log`` sequence for
the logsumexp fanin.  Autograd differentiates these directly.
"""

from __future__ import annotations

from .mp_constants import MODE_LOGSUMEXP, MODE_SUM
from .mp_runtime import torch


def fanout_scatter_python(
    x_cat: torch.Tensor,
    src_global_idx: torch.Tensor,
    flat_dst: torch.Tensor,
    out_rows: int,
) -> torch.Tensor:
    out = x_cat.new_zeros((int(out_rows), int(x_cat.size(-1))))
    if src_global_idx.numel() == 0 or int(out_rows) == 0:
        return out
    return out.index_copy(0, flat_dst, x_cat.index_select(0, src_global_idx))


def fanin_reduce_python(
    rel_flat: torch.Tensor,
    flat_src: torch.Tensor,
    dst_idx: torch.Tensor,
    dim_size: int,
    mode: int,
) -> torch.Tensor:
    rows = int(dim_size)
    emb = int(rel_flat.size(-1))
    if mode == MODE_SUM:
        out = rel_flat.new_zeros((rows, emb))
        if flat_src.numel() == 0 or rows == 0:
            return out
        return out.index_add(0, dst_idx, rel_flat.index_select(0, flat_src))
    if mode == MODE_LOGSUMEXP:
        neg_inf = float("-inf")
        if flat_src.numel() == 0 or rows == 0:
            return rel_flat.new_full((rows, emb), neg_inf)
        msgs = rel_flat.index_select(0, flat_src)
        scatter_index = dst_idx.view(-1, 1).expand(-1, emb)
        seg_max = rel_flat.new_full((rows, emb), neg_inf).scatter_reduce(
            0, scatter_index, msgs, reduce="amax", include_self=True
        )
        shifted = (msgs - seg_max.index_select(0, dst_idx)).exp()
        seg_sum = rel_flat.new_zeros((rows, emb)).scatter_add(0, scatter_index, shifted)
        return seg_sum.log() + seg_max
    raise ValueError(f"Unsupported fanin mode {mode!r}. Supported: 0=sum, 1=logsumexp.")


__all__ = ["fanin_reduce_python", "fanout_scatter_python"]
