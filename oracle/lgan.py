"""numpy restatement of relmo's LGAN indexed reductions.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the LGAN ops;
the product package (``relmo_amd``) never imports it.

Follows the reference's CPU path in ``src/_ops/mp/mp_ops.cpp`` (cited per
function), the same ATen sequence on numpy arrays: ``index_add_`` is
``np.add.at`` (sequential over the index, so sums add in edge order), counts
are accumulated in the value dtype, divisions and additions happen in the
same order and dtype.

Parity status (how each function is pinned, see tests/test_oracle.py):
  lgan_pool_reduce                    pinned: the reference library (oracle/_ref)
                                      bit-exact on golden cases; float64 dense-matrix
                                      truth; mean of equal rows is the row
  lgan_pool_reduce_backward           pinned: reference library bit-exact; adjoint
                                      identity <g, F(x)> = <F^T(g), x> in float64
  lgan_relation_graph_step            pinned: as lgan_pool_reduce
  lgan_relation_graph_step_backward   pinned: as lgan_pool_reduce_backward
"""

from __future__ import annotations

import numpy as np

MODE_SUM = 0
MODE_MEAN = 2


def _idx(a) -> np.ndarray:
    return np.asarray(a).astype(np.int64, copy=False)


def indexed_sum_or_mean(src_rows, src_index, dst_index, dim_size: int, mode: int) -> np.ndarray:
    """mp_ops.cpp:3439-3462 (aggregate_indexed): out[dst[e]] += src_rows[src[e]],
    divided by max(1, messages per row) in mean mode."""

    src_rows = np.asarray(src_rows)
    out = np.zeros((int(dim_size), src_rows.shape[1]), dtype=src_rows.dtype)
    s, d = _idx(src_index), _idx(dst_index)
    if s.size == 0 or d.size == 0 or int(dim_size) == 0:
        return out
    np.add.at(out, d, src_rows[s])
    if mode == MODE_MEAN:
        count = np.zeros((int(dim_size), 1), dtype=src_rows.dtype)
        np.add.at(count, d, np.ones((d.size, 1), dtype=src_rows.dtype))
        out = out / np.maximum(count, src_rows.dtype.type(1))
    return out


def aggregate_reverse(grad_rows, src_index, dst_index, src_rows: int, mode: int) -> np.ndarray:
    """mp_ops.cpp:3538-3561 (aggregate_reverse): grad_src[src[e]] += grad_rows[dst[e]]
    (divided per message by max(1, messages into dst[e]) in mean mode)."""

    grad_rows = np.asarray(grad_rows)
    out = np.zeros((int(src_rows), grad_rows.shape[1]), dtype=grad_rows.dtype)
    s, d = _idx(src_index), _idx(dst_index)
    if s.size == 0 or d.size == 0 or int(src_rows) == 0:
        return out
    gathered = grad_rows[d]
    if mode == MODE_MEAN:
        counts = np.zeros((grad_rows.shape[0], 1), dtype=grad_rows.dtype)
        np.add.at(counts, d, np.ones((d.size, 1), dtype=grad_rows.dtype))
        gathered = gathered / np.maximum(counts[d], grad_rows.dtype.type(1))
    np.add.at(out, s, gathered)
    return out


def _arity_divisor(arities, dtype) -> np.ndarray:
    return np.maximum(_idx(arities).astype(dtype), np.dtype(dtype).type(1)).reshape(-1, 1)


def lgan_pool_reduce(slot_messages, slot_to_relation_instance, relation_instance_arities, rr_src,
                     rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, entity_dim_size: int, mode: int):
    """mp_ops.cpp:3350-3469: slot messages summed per relation instance and
    divided by its arity (at least 1), then the relation-relation step."""

    slot = np.asarray(slot_messages)
    K = _idx(relation_instance_arities).size
    rpx = np.zeros((K, slot.shape[1]), dtype=slot.dtype)
    if slot.size > 0:
        np.add.at(rpx, _idx(slot_to_relation_instance), slot)
        rpx = rpx / _arity_divisor(relation_instance_arities, slot.dtype)
    return _relation_step(rpx, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, entity_dim_size,
                          mode, K)


def _relation_step(rpx, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, entity_dim_size, mode, K):
    rpx = rpx + indexed_sum_or_mean(rpx, rr_src, rr_dst, K, mode)
    tn = indexed_sum_or_mean(rpx, tn_rel, tn_ent, entity_dim_size, mode)
    nn = indexed_sum_or_mean(rpx, nn_rel, nn_ent, entity_dim_size, mode)
    return rpx, tn, nn


def lgan_relation_graph_step(relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent,
                             entity_dim_size: int, mode: int):
    """mp_ops.cpp:3574-3656: x + aggregate(x; rr), then its aggregation onto entities."""

    x = np.asarray(relation_pair_x)
    return _relation_step(x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, entity_dim_size,
                          mode, x.shape[0])


def lgan_relation_graph_step_backward(grad_relation_pair_x, grad_tn_msgs, grad_nn_msgs, rr_src,
                                      rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, relation_count: int,
                                      mode: int):
    """mp_ops.cpp:3658-3743: g1 = g + T^T grad_tn + N^T grad_nn; g1 + R^T g1."""

    g = np.asarray(grad_relation_pair_x)
    g1 = (g + aggregate_reverse(grad_tn_msgs, tn_rel, tn_ent, relation_count, mode)) \
        + aggregate_reverse(grad_nn_msgs, nn_rel, nn_ent, relation_count, mode)
    return g1 + aggregate_reverse(g1, rr_src, rr_dst, relation_count, mode)


def lgan_pool_reduce_backward(grad_relation_pair_x, grad_tn_msgs, grad_nn_msgs,
                              slot_to_relation_instance, relation_instance_arities, rr_src, rr_dst,
                              tn_rel, tn_ent, nn_rel, nn_ent, relation_count: int, mode: int):
    """mp_ops.cpp:3471-3572: the step's backward, then each slot takes its
    relation instance's gradient divided by the arity (at least 1)."""

    g = lgan_relation_graph_step_backward(grad_relation_pair_x, grad_tn_msgs, grad_nn_msgs, rr_src,
                                          rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, relation_count,
                                          mode)
    s2r = _idx(slot_to_relation_instance)
    return g[s2r] / _arity_divisor(relation_instance_arities, g.dtype)[s2r]


__all__ = [
    "aggregate_reverse",
    "indexed_sum_or_mean",
    "lgan_pool_reduce",
    "lgan_pool_reduce_backward",
    "lgan_relation_graph_step",
    "lgan_relation_graph_step_backward",
]
