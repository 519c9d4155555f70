"""Autograd wrappers around the ``relm_mp`` ops.

The forward passes save what relmo's ``src/relmo/ops/mp_autograd.py:110-191``
saves (index tensors and row counts; the logsumexp also keeps ``rel_flat`` and
its output) and the backward passes call the explicit ``*_backward`` ops, so
both directions run on the custom library.  The index tensors reach the
backward as the same tensor objects, which lets the library reuse the index
plan it built in the forward.
"""

from __future__ import annotations

from .mp_constants import MODE_LOGSUMEXP, MODE_SUM
from .mp_runtime import ops_namespace, torch

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

    class _FaninReduceSumFunction(torch.autograd.Function):
        @staticmethod
        def forward(ctx, rel_flat, flat_src, dst_idx, dim_size):
            ctx.save_for_backward(flat_src, dst_idx)
            ctx.rel_rows = int(rel_flat.size(0))
            return ops_namespace().fanin_reduce(rel_flat, flat_src, dst_idx, int(dim_size), MODE_SUM)

        @staticmethod
        def backward(ctx, grad_out):
            flat_src, dst_idx = ctx.saved_tensors
            grad_rel = ops_namespace().fanin_reduce_sum_backward(
                grad_out, flat_src, dst_idx, ctx.rel_rows
            )
            return grad_rel, None, None, None

    class _FaninReduceLogSumExpFunction(torch.autograd.Function):
        @staticmethod
        def forward(ctx, rel_flat, flat_src, dst_idx, dim_size):
            ctx.rel_rows = int(rel_flat.size(0))
            out = ops_namespace().fanin_reduce(
                rel_flat, flat_src, dst_idx, int(dim_size), MODE_LOGSUMEXP
            )
            ctx.save_for_backward(rel_flat, flat_src, dst_idx, out)
            return out

        @staticmethod
        def backward(ctx, grad_out):
            rel_flat, flat_src, dst_idx, out = ctx.saved_tensors
            grad_rel = ops_namespace().fanin_reduce_logsumexp_backward(
                grad_out, rel_flat, flat_src, dst_idx, out, ctx.rel_rows
            )
            return grad_rel, None, None, None

else:  # pragma: no cover - torch missing
    _FanoutScatterFunction = None
    _FaninReduceSumFunction = None
    _FaninReduceLogSumExpFunction = None
