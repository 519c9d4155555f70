"""ATen formulations of the LGAN indexed reductions (the reference's
``python_only`` path, ``src/relmo/ops/mp_fallbacks.py:28-123``).

Autograd differentiates these directly; the autograd Functions of
``mp_autograd`` use them for tensors that do not take the custom ops (CPU
tensors) and for their backward in that case.
"""

from __future__ import annotations

from .mp_common import indexed_sum_or_mean, require_rank
from .mp_runtime import torch


def _relation_step(relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent,
                   entity_dim_size, mode, relation_count, op_name):
    relation_pair_x = relation_pair_x + indexed_sum_or_mean(
        relation_pair_x, rr_src, rr_dst, relation_count, mode, op_name=op_name)
    tn_msgs = indexed_sum_or_mean(relation_pair_x, tn_rel, tn_ent, int(entity_dim_size), mode,
                                  op_name=op_name)
    nn_msgs = indexed_sum_or_mean(relation_pair_x, nn_rel, nn_ent, int(entity_dim_size), mode,
                                  op_name=op_name)
    return relation_pair_x, tn_msgs, nn_msgs


def lgan_pool_reduce_python(slot_messages, slot_to_relation_instance, relation_instance_arities,
                            rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, entity_dim_size: int,
                            mode: int):
    """Slots summed per relation instance and divided by its arity (at least
    1), then one residual relation-relation step and the entity aggregations."""

    op_name = "lgan_pool_reduce"
    require_rank(op_name, "slot_messages", slot_messages, 2)
    relation_count = int(relation_instance_arities.numel())
    relation_pair_x = slot_messages.new_zeros((relation_count, int(slot_messages.size(-1))))
    if int(slot_messages.numel()) > 0:
        relation_pair_x.index_add_(0, slot_to_relation_instance, slot_messages)
        arity = relation_instance_arities.to(device=slot_messages.device, dtype=slot_messages.dtype)
        relation_pair_x = relation_pair_x / arity.view(-1, 1).clamp_min_(1.0)
    return _relation_step(relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent,
                          entity_dim_size, mode, relation_count, op_name)


def lgan_relation_graph_step_python(relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel,
                                    nn_ent, entity_dim_size: int, mode: int):
    """``x + aggregate(x; rr)`` and its aggregations onto entities (tn, nn)."""

    op_name = "lgan_relation_graph_step"
    require_rank(op_name, "relation_pair_x", relation_pair_x, 2)
    return _relation_step(relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent,
                          entity_dim_size, mode, int(relation_pair_x.size(0)), op_name)


__all__ = ["lgan_pool_reduce_python", "lgan_relation_graph_step_python"]
