"""Public op facade: the API of relmo's ``relmo.ops.mp`` for this path.

``fanout_scatter`` and ``fanin_reduce`` keep the reference's signatures and
dispatch (``src/relmo/ops/mp.py:43-70``): modes other than sum (0) and
logsumexp (1) go to the ATen fallback, which raises ``ValueError``; otherwise
the custom ops run through autograd Functions unless the policy selects the
fallback.  The four pack ops (``mp.py:73-146``) call ``torch.ops.relm_mp``
directly, or their ATen fallbacks, as ``mp_dispatch.run_op`` routes them.  The
LGAN reductions (``_lgan_pool_reduce``, ``_lgan_relation_graph_step``,
``mp.py:394-525``) run the custom ops for CUDA tensors and their ATen fallbacks
otherwise.
"""

from __future__ import annotations

import contextlib

from .mp_autograd import (
    _FaninReduceLogSumExpFunction,
    _FaninReduceSumFunction,
    _FanoutConcatFunction,
    _FanoutScatterFunction,
    _LGANPoolReduceFunction,
    _LGANRelationGraphStepFunction,
)
from .mp_constants import MODE_LOGSUMEXP, MODE_MEAN, MODE_SUM, activation_code
from .mp_dispatch import library_op, library_ready, run_op
from .mp_pack import (
    fanin_pack_from_edges_python,
    fanin_pack_multi_python,
    fanin_reduce_python,
    fanout_pack_from_edges_python,
    fanout_pack_multi_python,
    fanout_scatter_python,
)
from .mp_runtime import TORCH_IMPORT_ERROR, assert_runtime_compat, available, ops_namespace, require_torch, torch


def _first(parts):
    """The tensor whose device sets the fallback policy of a pack op."""

    return parts[0] if parts else None


def fanout_scatter(
    x_cat: torch.Tensor,
    src_global_idx: torch.Tensor,
    flat_dst: torch.Tensor,
    out_rows: int,
) -> torch.Tensor:
    """``out[flat_dst[e]] = x_cat[src_global_idx[e]]``; other rows are zero."""

    require_torch("fanout_scatter")
    if library_ready("fanout_scatter", x_cat):
        return _FanoutScatterFunction.apply(x_cat, src_global_idx, flat_dst, int(out_rows))
    return fanout_scatter_python(x_cat, src_global_idx, flat_dst, int(out_rows))


def fanout_concat(
    prefix: torch.Tensor,
    x_cat: torch.Tensor,
    src_global_idx: torch.Tensor,
    flat_dst: torch.Tensor,
    slots: int,
) -> torch.Tensor:
    """``cat([prefix, fanout_scatter(x_cat, src_global_idx, flat_dst, n * slots).view(n, slots * D)], 1)``
    with ``n = prefix.size(0)``, in one pass.

    The central layer's input assembly (relmo ``models/hetero_mp/fused.py:299-375``:
    fanout into ``args_flat``, reshape, copy into ``all_inputs`` after the context
    columns), with the fanout rows written straight into the argument slots and
    the backward reading them from the gradient in place.  No counterpart in
    relmo's facade; without the ``fanout_scatter_into`` op it runs that composition.
    """

    require_torch("fanout_concat")
    slots = int(slots)
    if library_op("fanout_scatter_into", tensor=x_cat) is not None:
        return _FanoutConcatFunction.apply(prefix, x_cat, src_global_idx, flat_dst, slots)
    nodes = int(prefix.size(0))
    args = fanout_scatter(x_cat, src_global_idx, flat_dst, nodes * slots)
    return torch.cat([prefix, args.view(nodes, slots * int(x_cat.size(1)))], dim=1)


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
    if library_ready("fanin_reduce", rel_flat):
        fn = _FaninReduceSumFunction if mode == MODE_SUM else _FaninReduceLogSumExpFunction
        return fn.apply(rel_flat, flat_src, dst_idx, int(dim_size))
    return fanin_reduce_python(rel_flat, flat_src, dst_idx, int(dim_size), mode)


def fanout_pack_multi(
    x_parts: list[torch.Tensor],
    src_idx_parts: list[torch.Tensor],
    flat_dst_parts: list[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Concatenate source parts for one ``fanout_scatter``: ``(x_cat, src_global_idx, flat_dst)``."""

    require_torch("fanout_pack_multi")
    return run_op(
        "fanout_pack_multi", x_parts, src_idx_parts, flat_dst_parts,
        fallback=fanout_pack_multi_python, tensor=_first(x_parts),
    )


def fanin_pack_multi(
    rel_parts: list[torch.Tensor],
    flat_src_parts: list[torch.Tensor],
    dst_idx_parts: list[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Concatenate relation parts for one ``fanin_reduce``: ``(rel_flat, flat_src, dst_idx)``."""

    require_torch("fanin_pack_multi")
    return run_op(
        "fanin_pack_multi", rel_parts, flat_src_parts, dst_idx_parts,
        fallback=fanin_pack_multi_python, tensor=_first(rel_parts),
    )


def fanout_pack_from_edges(
    x_parts: list[torch.Tensor],
    edge_src_parts: list[torch.Tensor],
    edge_dst_parts: list[torch.Tensor],
    src_part_ids: list[int],
    arity_parts: list[int],
    pos_parts: list[int],
    slot_offset_parts: list[int],
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fanout operands from per-relation edge lists: ``flat_dst = slot_offset + dst * arity + pos``."""

    require_torch("fanout_pack_from_edges")
    return run_op(
        "fanout_pack_from_edges", x_parts, edge_src_parts, edge_dst_parts, src_part_ids,
        arity_parts, pos_parts, slot_offset_parts,
        fallback=fanout_pack_from_edges_python, tensor=_first(x_parts),
    )


def fanin_pack_from_edges(
    rel_parts: list[torch.Tensor],
    edge_src_parts: list[torch.Tensor],
    edge_dst_parts: list[torch.Tensor],
    rel_part_ids: list[int],
    arity_parts: list[int],
    pos_parts: list[int],
    mode: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fanin operands from per-relation edge lists: ``flat_src = src * arity + pos`` (mode 0)
    or ``src`` (mode 1), plus the part's row offset."""

    require_torch("fanin_pack_from_edges")
    return run_op(
        "fanin_pack_from_edges", rel_parts, edge_src_parts, edge_dst_parts, rel_part_ids,
        arity_parts, pos_parts, int(mode),
        fallback=fanin_pack_from_edges_python, tensor=_first(rel_parts),
    )


def _resolve_lgan_mode(op_name: str, mode: str) -> int:
    key = str(mode).strip().lower()
    if key == "sum":
        return MODE_SUM
    if key == "mean":
        return MODE_MEAN
    raise ValueError(f"{op_name} supports only mode='sum' or mode='mean'.")


def _lgan_pool_reduce(slot_messages, slot_to_relation_instance, relation_instance_arities, rr_src,
                      rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, *, entity_dim_size: int, mode: str):
    """Pool slot messages to relation instances and run the RR / TN / NN
    reductions (``mp.py:468-497``): ``(relation_pair_x, tn_msgs, nn_msgs)``."""

    require_torch("_lgan_pool_reduce")
    return _LGANPoolReduceFunction.apply(
        slot_messages, slot_to_relation_instance, relation_instance_arities, rr_src, rr_dst,
        tn_rel, tn_ent, nn_rel, nn_ent, int(entity_dim_size),
        int(_resolve_lgan_mode("_lgan_pool_reduce", mode)),
    )


def _lgan_relation_graph_step(relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, *,
                              entity_dim_size: int, mode: str):
    """RR / TN / NN propagation on pooled relation-instance embeddings (``mp.py:500-525``)."""

    require_torch("_lgan_relation_graph_step")
    return _LGANRelationGraphStepFunction.apply(
        relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, int(entity_dim_size),
        int(_resolve_lgan_mode("_lgan_relation_graph_step", mode)),
    )


@contextlib.contextmanager
def plan_scope():
    """Trust scope for the library's index plans (no counterpart in relmo).

    Every op call compares its index tensors with the plans it could reuse
    (a device pass over the indices), so that a plan is never served for
    indices that changed - also through ``.data`` or a raw pointer, which
    leave the tensor's version unchanged.  Inside this scope the caller
    promises that no index tensor passed to the ops is written; a plan built
    or compared equal in the scope is then served again for the very same
    tensors (same tensor object, version, data pointer and size) without the
    comparison, and the tensors are released when the outermost scope closes.
    Scopes nest and hold for the whole process (the backward's calls on
    autograd's threads included).  Without the library loaded the scope does
    nothing."""

    ns = ops_namespace() if library_ready("plan_trust_enter") else None
    enter = getattr(ns, "plan_trust_enter", None) if ns is not None else None
    if enter is None:
        yield
        return
    enter()
    try:
        yield
    finally:
        ns.plan_trust_exit()


__all__ = [
    "MODE_LOGSUMEXP",
    "MODE_MEAN",
    "MODE_SUM",
    "TORCH_IMPORT_ERROR",
    "activation_code",
    "assert_runtime_compat",
    "available",
    "fanin_pack_from_edges",
    "fanin_pack_multi",
    "fanin_reduce",
    "fanout_concat",
    "fanout_pack_from_edges",
    "fanout_pack_multi",
    "fanout_scatter",
    "plan_scope",
]
