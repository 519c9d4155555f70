"""Autograd wrappers around the ``relm_mp`` ops.

The forward passes save what relmo's ``src/relmo/ops/mp_autograd.py:110-191``
saves (index tensors and row counts; the logsumexp also keeps ``rel_flat`` and
its output) and the backward passes call the explicit ``*_backward`` ops, so
both directions run on the custom library.  The fanin functions also keep the
index plan the forward ran on (``fanin_reduce_planned``, an opaque
``torch.classes.relm_mp.PlanRef``) and hand it to the backward op of the same
call, which then needs neither a new plan nor a cache lookup.
"""

from __future__ import annotations

from .mp_constants import MODE_LOGSUMEXP, MODE_SUM
from .mp_runtime import ops_namespace, torch


def _planned_ops(ns) -> bool:
    """Whether the loaded library hands index plans from forward to backward."""

    return hasattr(ns, "fanin_reduce_planned")


if torch is not None:

    class _FanoutScatterFunction(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x_cat, src_global_idx, flat_dst, out_rows):
            ctx.save_for_backward(src_global_idx, flat_dst)
            ctx.x_rows = int(x_cat.size(0))
            return ops_namespace().fanout_scatter(x_cat, src_global_idx, flat_dst, int(out_rows))

        @staticmethod
        def backward(ctx, grad_out):
            src_global_idx, flat_dst = ctx.saved_tensors
            grad_x = ops_namespace().fanout_scatter_backward(
                grad_out, src_global_idx, flat_dst, ctx.x_rows
            )
            return grad_x, None, None, None

    def _fanin_forward(ctx, rel_flat, flat_src, dst_idx, dim_size, mode):
        ns = ops_namespace()
        ctx.plan = None
        if _planned_ops(ns):
            out, ctx.plan = ns.fanin_reduce_planned(rel_flat, flat_src, dst_idx, int(dim_size), mode)
            return out
        return ns.fanin_reduce(rel_flat, flat_src, dst_idx, int(dim_size), mode)

    class _FaninReduceSumFunction(torch.autograd.Function):
        @staticmethod
        def forward(ctx, rel_flat, flat_src, dst_idx, dim_size):
            ctx.save_for_backward(flat_src, dst_idx)
            ctx.rel_rows = int(rel_flat.size(0))
            return _fanin_forward(ctx, rel_flat, flat_src, dst_idx, dim_size, MODE_SUM)

        @staticmethod
        def backward(ctx, grad_out):
            flat_src, dst_idx = ctx.saved_tensors
            ns = ops_namespace()
            if ctx.plan is not None:
                grad_rel = ns.fanin_reduce_sum_backward_planned(
                    grad_out, flat_src, dst_idx, ctx.rel_rows, ctx.plan
                )
            else:
                grad_rel = ns.fanin_reduce_sum_backward(grad_out, flat_src, dst_idx, ctx.rel_rows)
            return grad_rel, None, None, None

    class _FaninReduceLogSumExpFunction(torch.autograd.Function):
        @staticmethod
        def forward(ctx, rel_flat, flat_src, dst_idx, dim_size):
            ctx.rel_rows = int(rel_flat.size(0))
            out = _fanin_forward(ctx, rel_flat, flat_src, dst_idx, dim_size, MODE_LOGSUMEXP)
            ctx.save_for_backward(rel_flat, flat_src, dst_idx, out)
            return out

        @staticmethod
        def backward(ctx, grad_out):
            rel_flat, flat_src, dst_idx, out = ctx.saved_tensors
            ns = ops_namespace()
            if ctx.plan is not None:
                grad_rel = ns.fanin_reduce_logsumexp_backward_planned(
                    grad_out, rel_flat, flat_src, dst_idx, out, ctx.rel_rows, ctx.plan
                )
            else:
                grad_rel = ns.fanin_reduce_logsumexp_backward(
                    grad_out, rel_flat, flat_src, dst_idx, out, ctx.rel_rows
                )
            return grad_rel, None, None, None

    class _FanoutConcatFunction(torch.autograd.Function):
        """``[prefix | fanout rows in `slots` argument slots per line]`` in one
        pass (``fanout_scatter_into``); the backward reads the argument
        columns of the incoming gradient in place (``fanout_scatter_backward_from``)."""

        @staticmethod
        def forward(ctx, prefix, x_cat, src_global_idx, flat_dst, slots):
            nodes, cols = int(prefix.size(0)), int(prefix.size(1))
            emb = int(x_cat.size(1))
            out = prefix.new_empty((nodes, cols + slots * emb))
            out[:, :cols] = prefix
            ops_namespace().fanout_scatter_into(x_cat, src_global_idx, flat_dst, out, cols, slots)
            ctx.save_for_backward(src_global_idx, flat_dst)
            ctx.shape = (int(x_cat.size(0)), cols, slots, emb)
            return out

        @staticmethod
        def backward(ctx, grad):
            src_global_idx, flat_dst = ctx.saved_tensors
            x_rows, cols, slots, emb = ctx.shape
            grad_prefix = grad[:, :cols] if ctx.needs_input_grad[0] else None
            grad_x = None
            if ctx.needs_input_grad[1]:
                grad_x = ops_namespace().fanout_scatter_backward_from(
                    grad, src_global_idx, flat_dst, x_rows, cols, slots, emb
                )
            return grad_prefix, grad_x, None, None, None

else:  # pragma: no cover - torch missing
    _FanoutScatterFunction = None
    _FaninReduceSumFunction = None
    _FaninReduceLogSumExpFunction = None
    _FanoutConcatFunction = None


# ---- LGAN indexed reductions ---------------------------------------------------
#
# As relmo's mp_autograd.py:194-537: CUDA tensors run the custom forward op and,
# in the backward, the custom backward op (missing output gradients become
# zeros); other tensors run the ATen fallback, differentiated by autograd.

def _zeros_or(grad, rows: int, like):
    if grad is not None:
        return grad
    return torch.zeros((int(rows), int(like.size(-1))), device=like.device, dtype=like.dtype)


if torch is not None:
    from .mp_dispatch import library_op
    from .mp_fallbacks import lgan_pool_reduce_python, lgan_relation_graph_step_python

    def _custom(tensor, op_name: str) -> bool:
        return library_op(op_name, tensor=tensor, gpu_only=True) is not None

    def _fallback_grad(fn, x, args, grads):
        with torch.enable_grad():
            x_req = x.detach().requires_grad_(True)
            outputs = fn(x_req, *args)
            grads = tuple(g if g is not None else torch.zeros_like(o) for g, o in zip(grads, outputs))
            (grad_x,) = torch.autograd.grad(outputs, (x_req,), grad_outputs=grads, allow_unused=True)
        return grad_x

    class _LGANPoolReduceFunction(torch.autograd.Function):
        @staticmethod
        def forward(ctx, slot_messages, slot_to_relation_instance, relation_instance_arities,
                    rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, entity_dim_size, mode):
            ctx.entity_dim_size, ctx.mode = int(entity_dim_size), int(mode)
            ctx.save_for_backward(slot_messages, slot_to_relation_instance,
                                  relation_instance_arities, rr_src, rr_dst, tn_rel, tn_ent,
                                  nn_rel, nn_ent)
            ctx.used_custom = _custom(slot_messages, "lgan_pool_reduce")
            fn = ops_namespace().lgan_pool_reduce if ctx.used_custom else lgan_pool_reduce_python
            return fn(slot_messages, slot_to_relation_instance, relation_instance_arities, rr_src,
                      rr_dst, tn_rel, tn_ent, nn_rel, nn_ent, ctx.entity_dim_size, ctx.mode)

        @staticmethod
        def backward(ctx, grad_rpx, grad_tn, grad_nn):
            slot, s2r, arity, *edges = ctx.saved_tensors
            none = (None,) * 10
            if (grad_rpx is None and grad_tn is None and grad_nn is None) or not ctx.needs_input_grad[0]:
                return (None, *none)
            K = int(arity.numel())
            if ctx.used_custom and _custom(slot, "lgan_pool_reduce_backward"):
                grad = ops_namespace().lgan_pool_reduce_backward(
                    _zeros_or(grad_rpx, K, slot), _zeros_or(grad_tn, ctx.entity_dim_size, slot),
                    _zeros_or(grad_nn, ctx.entity_dim_size, slot), s2r, arity, *edges, K, ctx.mode)
                return (grad, *none)
            grad = _fallback_grad(
                lambda x, *a: lgan_pool_reduce_python(x, *a),
                slot, (s2r, arity, *edges, ctx.entity_dim_size, ctx.mode), (grad_rpx, grad_tn, grad_nn))
            return (grad, *none)

    class _LGANRelationGraphStepFunction(torch.autograd.Function):
        @staticmethod
        def forward(ctx, relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent,
                    entity_dim_size, mode):
            ctx.entity_dim_size, ctx.mode = int(entity_dim_size), int(mode)
            ctx.save_for_backward(relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent)
            ctx.used_custom = _custom(relation_pair_x, "lgan_relation_graph_step")
            fn = (ops_namespace().lgan_relation_graph_step if ctx.used_custom
                  else lgan_relation_graph_step_python)
            return fn(relation_pair_x, rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent,
                      ctx.entity_dim_size, ctx.mode)

        @staticmethod
        def backward(ctx, grad_rpx, grad_tn, grad_nn):
            x, *edges = ctx.saved_tensors
            none = (None,) * 8
            if (grad_rpx is None and grad_tn is None and grad_nn is None) or not ctx.needs_input_grad[0]:
                return (None, *none)
            K = int(x.size(0))
            if ctx.used_custom and _custom(x, "lgan_relation_graph_step_backward"):
                grad = ops_namespace().lgan_relation_graph_step_backward(
                    _zeros_or(grad_rpx, K, x), _zeros_or(grad_tn, ctx.entity_dim_size, x),
                    _zeros_or(grad_nn, ctx.entity_dim_size, x), *edges, K, ctx.mode)
                return (grad, *none)
            grad = _fallback_grad(
                lambda v, *a: lgan_relation_graph_step_python(v, *a),
                x, (*edges, ctx.entity_dim_size, ctx.mode), (grad_rpx, grad_tn, grad_nn))
            return (grad, *none)


if torch is None:  # the facade still imports; its functions raise in require_torch first
    _FanoutScatterFunction = _FaninReduceSumFunction = _FaninReduceLogSumExpFunction = None
    _FanoutConcatFunction = None
    _LGANPoolReduceFunction = _LGANRelationGraphStepFunction = None
