"""ATen formulations of the ops (the reference's ``python_only`` path).

Restates relmo's ``src/relmo/ops/mp_pack.py``: ``index_select`` +
``index_copy_`` for the fanout, ``index_add_`` for the sum fanin and the
``scatter_reduce_(amax)`` / ``exp`` / ``scatter_add_`` / ``log`` sequence for
the logsumexp fanin (:19-63); tensor arithmetic and ``cat`` for the four pack
ops (:66-282), with their ``ValueError`` messages.  Autograd differentiates
these directly.
"""

from __future__ import annotations

from .mp_common import (
    cat_or_empty,
    cat_or_single,
    empty_index,
    require_int64,
    require_matching_lengths,
    require_non_empty,
    require_positive_arity,
    require_rank,
)
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


def _index_pair(op_name, first_name, first, second_name, second) -> None:
    for name, t in ((first_name, first), (second_name, second)):
        require_rank(op_name, name, t, 1)
    for name, t in ((first_name, first), (second_name, second)):
        require_int64(op_name, name, t)


def _pack_multi(op_name, what, names, values, first_parts, second_parts, per_part):
    value_name, first_name, second_name = names
    require_non_empty(op_name, values, what)
    require_matching_lengths(
        op_name,
        (f"{value_name}_parts", values),
        (f"{first_name}_parts", first_parts),
        (f"{second_name}_parts", second_parts),
    )
    firsts, seconds = [], []
    row_offset = 0
    for value, first, second in zip(values, first_parts, second_parts, strict=True):
        require_rank(op_name, what, value, 2)
        _index_pair(op_name, first_name, first, second_name, second)
        if first.numel() != second.numel():
            raise ValueError(
                f"{op_name} expects {first_name} and {second_name} lengths to match per {per_part}."
            )
        firsts.append(first + int(row_offset))
        seconds.append(second)
        row_offset += int(value.size(0))
    return cat_or_single(values), cat_or_single(firsts), cat_or_single(seconds)


def fanout_pack_multi_python(x_parts, src_idx_parts, flat_dst_parts):
    """``(cat(x), cat(src + row offset of its part), cat(flat_dst))`` (mp_pack.py:66-103)."""

    return _pack_multi(
        "fanout_pack_multi",
        "source tensor",
        ("x", "src_idx", "flat_dst"),
        x_parts,
        src_idx_parts,
        flat_dst_parts,
        "source",
    )


def fanin_pack_multi_python(rel_parts, flat_src_parts, dst_idx_parts):
    """``(cat(rel), cat(flat_src + row offset of its part), cat(dst))`` (mp_pack.py:106-148)."""

    return _pack_multi(
        "fanin_pack_multi",
        "relation tensor",
        ("rel", "flat_src", "dst_idx"),
        rel_parts,
        flat_src_parts,
        dst_idx_parts,
        "relation tensor",
    )


def _row_offsets(op_name, what, values) -> list[int]:
    offsets, row_offset = [], 0
    for value in values:
        require_rank(op_name, what, value, 2)
        offsets.append(int(row_offset))
        row_offset += int(value.size(0))
    return offsets


def _checked_edge_part(op_name, edge_src, edge_dst, part, num_parts, part_kind) -> int:
    _index_pair(op_name, "edge_src", edge_src, "edge_dst", edge_dst)
    if edge_src.numel() != edge_dst.numel():
        raise ValueError(f"{op_name} expects edge src/dst lengths to match.")
    part_i = int(part)
    if not 0 <= part_i < num_parts:
        raise ValueError(f"{op_name} {part_kind} out of range: {part_i!r}.")
    return part_i


def _checked_slot(op_name, arity, pos) -> tuple[int, int]:
    arity_i = require_positive_arity(op_name, arity)
    pos_i = int(pos)
    if not 0 <= pos_i < arity_i:
        raise ValueError(f"{op_name} expects pos in [0, arity), got pos={pos_i} arity={arity_i}.")
    return arity_i, pos_i


def fanout_pack_from_edges_python(
    x_parts, edge_src_parts, edge_dst_parts, src_part_ids, arity_parts, pos_parts, slot_offset_parts
):
    """Edge part i: src + row offset of x part ``src_part_ids[i]`` and
    ``slot_offset + dst * arity + pos`` (mp_pack.py:151-217)."""

    op_name = "fanout_pack_from_edges"
    require_non_empty(op_name, x_parts, "source tensor")
    require_matching_lengths(
        op_name,
        ("edge_src_parts", edge_src_parts),
        ("edge_dst_parts", edge_dst_parts),
        ("src_part_ids", src_part_ids),
        ("arity_parts", arity_parts),
        ("pos_parts", pos_parts),
        ("slot_offset_parts", slot_offset_parts),
    )
    offsets = _row_offsets(op_name, "source tensor", x_parts)
    x_cat = cat_or_single(x_parts)
    srcs, dsts = [], []
    for edge_src, edge_dst, part, arity, pos, slot_offset in zip(
        edge_src_parts, edge_dst_parts, src_part_ids, arity_parts, pos_parts, slot_offset_parts,
        strict=True,
    ):
        part_i = _checked_edge_part(op_name, edge_src, edge_dst, part, len(x_parts), "src_part_ids")
        arity_i, pos_i = _checked_slot(op_name, arity, pos)
        srcs.append(edge_src + offsets[part_i])
        dsts.append(int(slot_offset) + edge_dst * arity_i + pos_i)
    empty = empty_index(x_parts[0].device)
    return x_cat, cat_or_empty(srcs, empty=empty), cat_or_empty(dsts, empty=empty)


def fanin_pack_from_edges_python(
    rel_parts, edge_src_parts, edge_dst_parts, rel_part_ids, arity_parts, pos_parts, mode
):
    """Edge part i: ``src * arity + pos`` (mode 0, relation rows) or ``src``
    (mode 1, label rows), plus the row offset of rel part ``rel_part_ids[i]``;
    dst unchanged (mp_pack.py:220-282)."""

    op_name = "fanin_pack_from_edges"
    require_non_empty(op_name, rel_parts, "relation tensor")
    require_matching_lengths(
        op_name,
        ("edge_src_parts", edge_src_parts),
        ("edge_dst_parts", edge_dst_parts),
        ("rel_part_ids", rel_part_ids),
        ("arity_parts", arity_parts),
        ("pos_parts", pos_parts),
    )
    mode_i = int(mode)
    if mode_i not in (0, 1):
        raise ValueError(f"{op_name} expects mode in {{0,1}}, got {mode_i!r}.")
    offsets = _row_offsets(op_name, "relation tensor", rel_parts)
    rel_cat = cat_or_single(rel_parts)
    srcs, dsts = [], []
    for edge_src, edge_dst, part, arity, pos in zip(
        edge_src_parts, edge_dst_parts, rel_part_ids, arity_parts, pos_parts, strict=True
    ):
        part_i = _checked_edge_part(op_name, edge_src, edge_dst, part, len(rel_parts), "rel_part_ids")
        if mode_i == 1:
            local = edge_src
        else:
            arity_i, pos_i = _checked_slot(op_name, arity, pos)
            local = edge_src * arity_i + pos_i
        srcs.append(local + offsets[part_i])
        dsts.append(edge_dst)
    empty = empty_index(rel_parts[0].device)
    return rel_cat, cat_or_empty(srcs, empty=empty), cat_or_empty(dsts, empty=empty)


__all__ = [
    "fanin_pack_from_edges_python",
    "fanin_pack_multi_python",
    "fanin_reduce_python",
    "fanout_pack_from_edges_python",
    "fanout_pack_multi_python",
    "fanout_scatter_python",
]
