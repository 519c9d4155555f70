"""numpy restatement of relmo's four pack ops (index arithmetic + concatenation).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the pack ops;
the product package (``relmo_amd``) never imports it.

Each function follows the reference's ATen implementation in
``src/_ops/mp/mp_ops.cpp`` (cited per function) on numpy arrays: value parts
are concatenated along rows, index parts are shifted / scaled with int64
arithmetic (wrapping modulo 2^64 like torch's) and concatenated in part order.
Argument validation is the op's concern and is not restated here.

Parity status (how each function is pinned, see tests/test_oracle.py):
  fanout_pack_multi       pinned: the reference test's inputs with outputs
                          worked out by hand; round trip (src_global - offset
                          of its part recovers src, lengths add up)
  fanin_pack_multi        pinned: as above
  fanout_pack_from_edges  pinned: the reference test's inputs with outputs
                          worked out by hand; decoding (flat_dst - slot_offset)
                          divmod arity == (dst, pos); arity 1 / pos 0 / slot 0
                          reduces it to fanout_pack_multi
  fanin_pack_from_edges   pinned: the reference test's inputs (both modes) with
                          outputs worked out by hand; decoding divmod arity in
                          mode 0; mode 1 equals fanin_pack_multi
"""

from __future__ import annotations

import numpy as np


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


def _row_offsets(values) -> list[int]:
    offsets, row = [], 0
    for v in values:
        offsets.append(row)
        row += int(np.asarray(v).shape[0])
    return offsets


def _cat_values(values) -> np.ndarray:
    return np.concatenate([np.asarray(v) for v in values], axis=0)


def _cat_index(parts) -> np.ndarray:
    return np.concatenate(parts) if parts else np.zeros(0, dtype=np.int64)


def fanout_pack_multi(x_parts, src_idx_parts, flat_dst_parts):
    """mp_ops.cpp:412-484: src + row offset of its x part; flat_dst as given."""

    offsets = _row_offsets(x_parts)
    src = [_i64(s) + np.int64(o) for s, o in zip(src_idx_parts, offsets)]
    return _cat_values(x_parts), _cat_index(src), _cat_index([_i64(d) for d in flat_dst_parts])


def fanin_pack_multi(rel_parts, flat_src_parts, dst_idx_parts):
    """mp_ops.cpp:486-570: flat_src + row offset of its rel part; dst_idx as given."""

    offsets = _row_offsets(rel_parts)
    src = [_i64(s) + np.int64(o) for s, o in zip(flat_src_parts, offsets)]
    return _cat_values(rel_parts), _cat_index(src), _cat_index([_i64(d) for d in dst_idx_parts])


def fanout_pack_from_edges(x_parts, edge_src_parts, edge_dst_parts, src_part_ids, arity_parts,
                           pos_parts, slot_offset_parts):
    """mp_ops.cpp:2511-2634: src + offset of x part src_part_ids[i];
    flat_dst = slot_offset + dst * arity + pos."""

    offsets = _row_offsets(x_parts)
    src, dst = [], []
    with np.errstate(over="ignore"):
        for s, d, part, arity, pos, slot in zip(edge_src_parts, edge_dst_parts, src_part_ids,
                                                arity_parts, pos_parts, slot_offset_parts):
            src.append(_i64(s) + np.int64(offsets[int(part)]))
            dst.append(np.int64(slot) + _i64(d) * np.int64(arity) + np.int64(pos))
    return _cat_values(x_parts), _cat_index(src), _cat_index(dst)


def fanin_pack_from_edges(rel_parts, edge_src_parts, edge_dst_parts, rel_part_ids, arity_parts,
                          pos_parts, mode: int):
    """mp_ops.cpp:2636-2772: (src * arity + pos) + offset of rel part
    rel_part_ids[i] in mode 0, src + offset in mode 1; dst as given."""

    offsets = _row_offsets(rel_parts)
    src = []
    with np.errstate(over="ignore"):
        for s, part, arity, pos in zip(edge_src_parts, rel_part_ids, arity_parts, pos_parts):
            local = _i64(s) if int(mode) == 1 else _i64(s) * np.int64(arity) + np.int64(pos)
            src.append(local + np.int64(offsets[int(part)]))
    return _cat_values(rel_parts), _cat_index(src), _cat_index([_i64(d) for d in edge_dst_parts])


__all__ = [
    "fanin_pack_from_edges",
    "fanin_pack_multi",
    "fanout_pack_from_edges",
    "fanout_pack_multi",
]
