"""The reference's model-level callers of the ops, restated in plain torch.

relmo's RelationalGNN (``rel_layer_mode="fast_fused"``,
src/relmo/models/relational_gnn.py:124-535 with
src/relmo/models/hetero_mp/fast_fused.py:26-300) and CentralizedRelationalGNN
(``central_layer_mode="fused"``, relational_gnn.py:552-846 with
hetero_mp/fused.py:121-406) are built on torch_geometric, which is not
available here.  This module keeps their computation on the hot path - the
slot layout that feeds ``fanout_scatter`` / ``fanin_reduce``, the relation and
central MLPs, the embedding update - over a plain batch description, so that a
training step of either model can be timed (graphs/sec) and compared between
the HIP op lane and the ATen lane.

Batch: one object node type; ``relations`` maps predicate -> arity; ``atoms``
maps predicate -> int64 [n, arity] global object ids (arity-0 predicates are
skipped, as in relational_gnn.py:322-326).
"""

from __future__ import annotations

import contextlib
import math
from dataclasses import dataclass

import torch
from torch import Tensor, nn
from torch.utils.checkpoint import checkpoint

from . import mp
from .mp_dispatch import library_op


@dataclass
class RelationalBatch:
    num_graphs: int
    num_objects: int
    relations: dict[str, int]
    atoms: dict[str, Tensor]


def _graph_atoms(gen: torch.Generator, obj_offsets: Tensor, obj_counts: Tensor, n_per_graph: Tensor,
                 arity: int) -> Tensor:
    """Arguments uniform within each graph: [sum(n_per_graph), arity] global ids."""

    graph_of_atom = torch.repeat_interleave(torch.arange(n_per_graph.numel()), n_per_graph)
    u = torch.rand(int(graph_of_atom.numel()), arity, generator=gen, dtype=torch.float64)
    local = (u * obj_counts[graph_of_atom].unsqueeze(1).double()).long()
    local = torch.minimum(local, (obj_counts[graph_of_atom] - 1).unsqueeze(1))
    return obj_offsets[graph_of_atom].unsqueeze(1) + local


def synthetic_c4(device, seed: int = 0, num_graphs: int = 512) -> RelationalBatch:
    """200 objects per graph, predicates of arity
    0, 1, 2, 2, 3 with 400 atoms each per graph, uniform arguments."""

    gen = torch.Generator().manual_seed(seed)
    objs = torch.full((num_graphs,), 200, dtype=torch.long)
    offsets = torch.cumsum(objs, 0) - objs
    relations = {"p0": 0, "p1": 1, "p2": 2, "p3": 2, "p4": 3}
    atoms = {}
    for name, arity in relations.items():
        if arity == 0:
            continue
        per = torch.full((num_graphs,), 400, dtype=torch.long)
        atoms[name] = _graph_atoms(gen, offsets, objs, per, arity).to(device)
    return RelationalBatch(num_graphs, int(objs.sum()), relations, atoms)


def synthetic_c5(device, seed: int = 0, num_graphs: int = 2048) -> RelationalBatch:
    """64-512 objects per graph, 8 predicates of arity
    1-3, 1000-4000 atoms per graph split uniformly at random over the
    predicates, uniform arguments within each graph."""

    gen = torch.Generator().manual_seed(seed)
    objs = torch.randint(64, 513, (num_graphs,), generator=gen)
    offsets = torch.cumsum(objs, 0) - objs
    relations = {f"r{i}": int(torch.randint(1, 4, (1,), generator=gen)) for i in range(8)}
    total_atoms = torch.randint(1000, 4001, (num_graphs,), generator=gen)
    # split every graph's atoms over the predicates (multinomial, uniform)
    pick = torch.multinomial(torch.full((8,), 1.0 / 8), int(total_atoms.sum()), replacement=True,
                             generator=gen)
    graph_of = torch.repeat_interleave(torch.arange(num_graphs), total_atoms)
    counts = torch.zeros(num_graphs, 8, dtype=torch.long)
    counts.index_put_((graph_of, pick), torch.ones_like(pick), accumulate=True)
    atoms = {}
    for i, (name, arity) in enumerate(relations.items()):
        atoms[name] = _graph_atoms(gen, offsets, objs, counts[:, i], arity).to(device)
    return RelationalBatch(num_graphs, int(objs.sum()), relations, atoms)


# ---- modules (relmo/models/mlp.py, residual.py, film.py) ---------------------------------


def weight_grad(grad_out: Tensor, inp: Tensor, chunk: int | None = None) -> Tensor:
    """grad_out^T @ inp for a Linear's weight: [K, out] x [K, in] -> [out, in].

    The weight gradients of these models reduce over all atoms or relation
    nodes (K up to 5 M) into a few hundred columns.  The library GEMM picks a
    handful of output tiles and walks all of K in each (C4: 0.40-0.53 ms per
    weight of 32 x 32 to 96 x 96 over 204,800 atoms; C5's 384 x 398 weight
    over 5 M nodes: 21 ms); here K is split into chunks that run as one
    batched product (chunk x in by chunk x out per batch entry), then summed:
    31-61 us for C4's weights, 14 ms for C5's.  The input's chunks are read in
    place as transposed views (the left operand), the gradient's as they are
    (column slices of wider matrices included: only unit column strides are
    needed).  Another summation order than one GEMM: equal up to fp32
    rounding.  Chunks default to 2048 rows for weights of at most 64 x 64
    entries, 4096 up to 256 x 256, 32768 above."""

    K = inp.size(0)
    out_f, in_f = grad_out.size(1), inp.size(1)
    if chunk is None:
        entries = out_f * in_f
        chunk = 2048 if entries <= 64 * 64 else (4096 if entries <= 256 * 256 else 32768)
    if K < 8 * chunk or inp.stride(1) != 1 or grad_out.stride(1) != 1:
        return grad_out.t().matmul(inp)
    b = K // chunk
    main = b * chunk
    w = torch.bmm(inp[:main].unflatten(0, (b, chunk)).transpose(1, 2),
                  grad_out[:main].unflatten(0, (b, chunk))).sum(0).t()
    if main < K:
        w = w + grad_out[main:].t().matmul(inp[main:])
    return w


def _narrow_nt(t: Tensor, inner: int, cols: int) -> bool:
    """Whether t @ b^T (inner size `inner`, `cols` output columns) goes to the
    library's mm_nt (rocBLAS): float32 on the GPU with 64 to 128 inner and at
    most 128 output columns, where rocBLAS streams at about the HBM rate and
    hipBLASLt runs 2-3x slower (C4's relation MLPs: 23 against 55 us for a
    204,800 x 64 by 64 x 64 product, 43 against 85 us at 96).  With fewer than
    64 inner columns rocBLAS is the slower one."""

    return (64 <= inner <= 128 and cols <= 128 and t.dtype == torch.float32
            and library_op("mm_nt", tensor=t, gpu_only=True) is not None)


def matmul_nt(a: Tensor, b: Tensor) -> Tensor:
    """a @ b^T for a [M, K], b [N, K] (_narrow_nt picks the library)."""

    if _narrow_nt(a, a.size(1), b.size(0)):
        return torch.ops.relm_mp.mm_nt(a, b)
    return a.matmul(b.t())


# Contiguous transposes of the weights, shared by the layers of one training
# step (shared_weight_transposes): {id(weight): (weight, version, transpose)}.
_TRANSPOSES: dict | None = None


@contextlib.contextmanager
def shared_weight_transposes():
    """Within the block, the input gradients of the narrow products reuse one
    contiguous transpose per weight (the layers of a RelationalGNN share their
    MLPs: ten layers, one transpose each instead of ten).  An entry is used
    only for the same weight object at the same version; the block holds
    them until it ends.  Process wide, like mp.plan_scope, so that the
    backward's calls on autograd's threads see it."""

    global _TRANSPOSES
    prev = _TRANSPOSES
    _TRANSPOSES = {}
    try:
        yield
    finally:
        _TRANSPOSES = prev


def _transposed(weight: Tensor) -> Tensor:
    cache = _TRANSPOSES
    if cache is None:
        return weight.t().contiguous()
    hit = cache.get(id(weight))
    if hit is not None and hit[0] is weight and hit[1] == weight._version:
        return hit[2]
    wt = weight.detach().t().contiguous()
    cache[id(weight)] = (weight, weight._version, wt)
    return wt


def _input_grad(grad: Tensor, weight: Tensor, x: Tensor) -> Tensor:
    """grad @ weight ([M, out] x [out, in]) shaped as x."""

    g2 = grad.reshape(-1, grad.size(-1))
    if _narrow_nt(g2, weight.size(0), weight.size(1)):
        return torch.ops.relm_mp.mm_nt(g2, _transposed(weight)).view(*x.shape[:-1], weight.size(1))
    return grad.matmul(weight)


class _Linear(torch.autograd.Function):
    """F.linear with the weight gradient of weight_grad; narrow products
    through matmul_nt (the bias then added in place)."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Tensor | None) -> Tensor:
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        if x.dim() == 2 and _narrow_nt(x, weight.size(1), weight.size(0)):
            y = torch.ops.relm_mp.mm_nt(x, weight)
            return y.add_(bias) if bias is not None else y
        return nn.functional.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, grad: Tensor):
        x, weight = ctx.saved_tensors
        # no copies: x may be a column slice of a wider matrix (the GEMMs take
        # its row stride as it is)
        g2 = grad.reshape(-1, grad.size(-1))
        x2 = x.reshape(-1, x.size(-1))
        gx = _input_grad(grad, weight, x) if ctx.needs_input_grad[0] else None
        gw = weight_grad(g2, x2) if ctx.needs_input_grad[1] else None
        gb = g2.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return gx, gw, gb


def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    """F.linear; on the GPU with the weight gradient of weight_grad."""

    if torch.is_grad_enabled() and x.is_cuda:
        return _Linear.apply(x, weight, bias)
    return nn.functional.linear(x, weight, bias)


class _FilmMish(torch.autograd.Function):
    """mish(beta[k] + gamma[k] * (s + add[k])) over the row ranges k of s (range
    k = rows [starts[k], starts[k + 1])), in one pass of the library's kernel
    (torch.ops.relm_mp.film_mish); the backward reads s and the gradient once
    (film_mish_backward), and the gradient of add is gamma times beta's."""

    @staticmethod
    def forward(ctx, s: Tensor, gamma: Tensor, beta: Tensor, add: Tensor | None, starts: list[int]) -> Tensor:
        ctx.starts = starts
        ctx.save_for_backward(s, gamma, beta, add)
        return torch.ops.relm_mp.film_mish(s, starts, gamma, beta, add)

    @staticmethod
    def backward(ctx, grad: Tensor):
        s, gamma, beta, add = ctx.saved_tensors
        ds, dg, db = torch.ops.relm_mp.film_mish_backward(grad, s, ctx.starts, gamma, beta, add)
        da = gamma * db if add is not None and ctx.needs_input_grad[3] else None
        return ds, dg, db, da, None


class _FilmMishLinear(torch.autograd.Function):
    """out(film_mish(s)): the FiLM step with Mish and the Linear after it,
    keeping only s for the backward - the Mish output that the Linear's weight
    gradient needs is recomputed there by one more pass of the fused kernel
    (selective recomputation: the step's other activations are never kept)."""

    @staticmethod
    def forward(ctx, s: Tensor, gamma: Tensor, beta: Tensor, add: Tensor | None, starts: list[int],
                weight: Tensor, bias: Tensor | None) -> Tensor:
        ctx.starts = starts
        ctx.has_bias = bias is not None
        ctx.save_for_backward(s, gamma, beta, add, weight)
        h = torch.ops.relm_mp.film_mish(s, starts, gamma, beta, add)
        return nn.functional.linear(h, weight, bias)

    @staticmethod
    def backward(ctx, grad: Tensor):
        s, gamma, beta, add, weight = ctx.saved_tensors
        h = torch.ops.relm_mp.film_mish(s, ctx.starts, gamma, beta, add)
        g2 = grad.reshape(-1, grad.size(-1))
        gw = weight_grad(g2, h) if ctx.needs_input_grad[5] else None
        gb = g2.sum(0) if ctx.has_bias and ctx.needs_input_grad[6] else None
        del h
        ds, dg, db = torch.ops.relm_mp.film_mish_backward(grad.matmul(weight), s, ctx.starts, gamma, beta,
                                                          add)
        da = gamma * db if add is not None and ctx.needs_input_grad[3] else None
        return ds, dg, db, da, None, gw, gb


class Linear(nn.Linear):
    """nn.Linear whose weight gradient splits long reductions (weight_grad)."""

    def forward(self, x: Tensor) -> Tensor:
        return linear(x, self.weight, self.bias)


_UNIT_FILM: dict[tuple[torch.device, int], tuple[Tensor, Tensor]] = {}


def _unit_film(like: Tensor) -> tuple[Tensor, Tensor]:
    """gamma = 1 and beta = 0 for one row range of like's width: the fused
    FiLM kernel then computes plain Mish (0 + 1 * u == u exactly)."""

    key = (like.device, like.size(-1))
    pair = _UNIT_FILM.get(key)
    if pair is None:
        pair = (torch.ones(1, like.size(-1), device=like.device, dtype=torch.float32),
                torch.zeros(1, like.size(-1), device=like.device, dtype=torch.float32))
        _UNIT_FILM[key] = pair
    return pair


class _LinearMish(torch.autograd.Function):
    """mish(linear(x, weight, bias)) with Mish in the library's fused FiLM
    kernel (one row range, unit scale; torch.ops.relm_mp.film_mish).  Narrow
    products run through mm_nt without the bias, which the kernel then adds
    as its shift (mish(bias + u)); otherwise the GEMM adds it and the shift is
    zero.  The pre-activation u is kept; the backward reads it and the
    gradient once (film_mish_backward), which also yields the bias gradient -
    the column sums of the gradient at the Mish input - so no separate
    reduction runs for it."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Tensor | None) -> Tensor:
        x2 = x.reshape(-1, x.size(-1))
        one, zero = _unit_film(weight[:, 0])
        if _narrow_nt(x2, weight.size(1), weight.size(0)):
            u = torch.ops.relm_mp.mm_nt(x2, weight)
            shift = bias.unsqueeze(0) if bias is not None else zero
        else:
            u = nn.functional.linear(x2, weight, bias)
            shift = zero
        ctx.has_bias = bias is not None
        ctx.save_for_backward(x, weight, u, shift)
        y = torch.ops.relm_mp.film_mish(u, [0, u.size(0)], one, shift, None)
        return y.view(*x.shape[:-1], weight.size(0))

    @staticmethod
    def backward(ctx, grad: Tensor):
        x, weight, u, shift = ctx.saved_tensors
        one, _zero = _unit_film(weight[:, 0])
        du, _dg, db = torch.ops.relm_mp.film_mish_backward(grad.reshape(u.shape), u, [0, u.size(0)],
                                                           one, shift, None)
        x2 = x.reshape(-1, x.size(-1))
        gx = _input_grad(du, weight, x) if ctx.needs_input_grad[0] else None
        gw = weight_grad(du, x2) if ctx.needs_input_grad[1] else None
        gb = db[0] if ctx.has_bias and ctx.needs_input_grad[2] else None
        return gx, gw, gb


class MishMLP(nn.Sequential):
    """nn.Sequential of Linear and Mish layers (mlp.py's layer order and
    parameter names) where, in float32 on the GPU with the library loaded, a
    Linear followed by Mish runs as one autograd node (_LinearMish): torch's
    Mish costs three transcendental functions per element and its backward
    more, the fused kernel one exp and one division, and the bias gradient
    comes with the Mish backward."""

    def forward(self, x: Tensor) -> Tensor:
        mods = list(self)
        fused = (x.is_cuda and x.dtype == torch.float32
                 and library_op("film_mish", tensor=x, gpu_only=True) is not None)
        i = 0
        while i < len(mods):
            m = mods[i]
            if (fused and isinstance(m, nn.Linear) and i + 1 < len(mods)
                    and isinstance(mods[i + 1], nn.Mish) and x.size(-1) == m.in_features):
                x = _LinearMish.apply(x, m.weight, m.bias)
                i += 2
            else:
                x = m(x)
                i += 1
        return x


class _ResidualConcat(torch.autograd.Function):
    """cat_i(bases[i] + ys[i]) along the rows: each part's residual addition
    written straight into its rows of the result (the per-predicate relation
    outputs without a separate concatenation pass); the backward hands each
    part's rows of the gradient to both of its inputs.  bases[i] and ys[i]
    are [n_i, w_i] with w_i a multiple of the result's width d."""

    @staticmethod
    def forward(ctx, d: int, n: int, *parts: Tensor) -> Tensor:
        bases, ys = parts[:n], parts[n:]
        rows = [b.numel() // d for b in bases]
        ctx.d, ctx.shapes, ctx.rows = d, [b.shape for b in bases], rows
        out = bases[0].new_empty(sum(rows), d)
        off = 0
        for b, y, r in zip(bases, ys, rows):
            torch.add(b, y, out=out[off:off + r].view(b.shape))
            off += r
        return out

    @staticmethod
    def backward(ctx, grad: Tensor):
        grads, off = [], 0
        for shape, r in zip(ctx.shapes, ctx.rows):
            grads.append(grad[off:off + r].reshape(shape))
            off += r
        return (None, None, *grads, *grads)


class Residual(nn.Module):
    """x[..., -width:] + f(x) (residual.py:4-31 with truncate_right=False)."""

    def __init__(self, module: nn.Module, width: int | None = None):
        super().__init__()
        self.module = module
        self.width = width

    def forward(self, x: Tensor) -> Tensor:
        base = x if self.width is None or x.size(-1) == self.width else x[..., -self.width:]
        return base + self.module(x)


def arity_mlp(feature: int, arity: int, layers: int) -> nn.Module:
    """ArityMLPFactory(feature_size, residual=True, layers=L)(arity)
    (mlp.py:127-246): Linear + Mish per hidden layer of width arity * feature."""

    width = feature * arity
    mods: list[nn.Module] = []
    dims = [width] * (layers + 1) + [width]
    for i in range(len(dims) - 1):
        mods.append(Linear(dims[i], dims[i + 1]))
        if i < len(dims) - 2:
            mods.append(nn.Mish())
    return Residual(MishMLP(*mods), width)


def simple_mlp(in_size: int, hidden: int, out_size: int) -> nn.Module:
    """SimpleMLP (mlp.py:50-79): Linear, Mish, Linear."""

    return MishMLP(Linear(in_size, hidden), nn.Mish(), Linear(hidden, out_size))


class FiLMConcatMLP(nn.Module):
    """FiLM-conditioned MLP on [cond | features] (film.py:10-195): each hidden
    layer is Linear -> gamma(c) * h + beta(c) -> Mish, then an output Linear."""

    def __init__(self, in_dim: int, cond_dim: int, hidden: list[int], out_dim: int):
        super().__init__()
        self.cond_dim = cond_dim
        self.lins = nn.ModuleList()
        self.gammas = nn.ModuleList()
        self.betas = nn.ModuleList()
        prev = in_dim
        for h in hidden:
            self.lins.append(Linear(prev, h))
            self.gammas.append(Linear(cond_dim, h))
            self.betas.append(Linear(cond_dim, h))
            prev = h
        self.out = Linear(prev, out_dim)
        self.act = nn.Mish()

    def forward(self, x: Tensor) -> Tensor:
        cond, h = x[..., : self.cond_dim], x[..., self.cond_dim:]
        for lin, g, b in zip(self.lins, self.gammas, self.betas):
            h = self.act(g(cond) * lin(h) + b(cond))
        return self.out(h)


def _object_degrees(obj: Tensor, num_objects: int) -> Tensor:
    """Messages per object (the fanin segment sizes)."""

    return torch.bincount(obj, minlength=num_objects)


def fanin_objects(mode: int, rel_flat: Tensor, r: dict, num_objects: int) -> Tensor:
    """Aggregation of the slot messages onto the objects as the reference's
    layers do it (fused.py:381-404, fast_fused.py:280-296): sum and logsumexp
    through ``fanin_reduce``, mean as PyG's MeanAggregation (the sum divided by
    max(count, 1)); objects without messages get 0, as from PyG's aggregators
    (the op's logsumexp leaves -inf there, which is replaced - NaN and +inf
    results of objects with messages pass through unchanged)."""

    # the fanin edge list: the fanout's (slot, object) pairs unless the routing
    # packed its own (RelationalGNN's batched lane)
    src, dst = r.get("fanin_src", r["flat"]), r.get("fanin_dst", r["obj"])
    if mode == mp.MODE_MEAN:
        total = mp.fanin_reduce(rel_flat, src, dst, num_objects, mp.MODE_SUM)
        return total / r["deg"].clamp_min(1).to(total.dtype).unsqueeze(1)
    msgs = mp.fanin_reduce(rel_flat, src, dst, num_objects, mode)
    if mode == mp.MODE_LOGSUMEXP:
        msgs = msgs.masked_fill((r["deg"] == 0).unsqueeze(1), 0.0)
    return msgs


# ---- RelationalGNN, fast fused relation layer ------------------------------------------


class RelationalGNN(nn.Module):
    """RelationalGNN with the fast fused relation layer: per layer, gather the
    argument embeddings of every atom into slots (fanout_scatter), apply the
    predicate's residual MLP, reduce the slot outputs back to objects
    (fanin_reduce: sum or logsumexp), update X <- X + updater([X, m]).

    ``lane="batched"`` routes as the batched_cached lane (BatchedFanOutMP /
    BatchedFanInMP with the pack ops enabled): the slot and object indices of
    both ops come from ``fanout_pack_from_edges`` and
    ``fanin_pack_from_edges`` over per-(predicate, position) edge lists, made
    once per batch and reused by every layer.  The two lanes route the same
    edges in the same order, so their indices and steps agree exactly."""

    def __init__(self, embedding_size: int, num_layers: int, relations: dict[str, int], mode: int,
                 mlp_layers: int = 2, lane: str = "fast_fused"):
        super().__init__()
        if lane not in ("fast_fused", "batched"):
            raise ValueError(f"unknown RelationalGNN lane {lane!r} (fast_fused or batched)")
        self.lane = lane
        self.d = embedding_size
        self.num_layers = num_layers
        self.mode = mode
        self.relations = {p: a for p, a in relations.items() if a > 0}
        self.rel_mlps = nn.ModuleDict({p: arity_mlp(embedding_size, a, mlp_layers)
                                       for p, a in self.relations.items()})
        self.updater = simple_mlp(2 * embedding_size, 2 * embedding_size, embedding_size)

    def routing(self, batch: RelationalBatch) -> dict:
        """fast_fused.py:79-177: slots ordered by predicate name, slot of
        (atom, pos) = offset + atom * arity + pos; fanout edges listed per
        predicate then position, fanin edges the same way."""

        if self.lane == "batched":
            return self._routing_batched(batch)
        meta, flat, obj = [], [], []
        total = 0
        for pred in sorted(self.relations):
            args = batch.atoms.get(pred)
            if args is None or args.numel() == 0:
                continue
            n, arity = int(args.size(0)), self.relations[pred]
            meta.append((pred, n, arity, total))
            atom = torch.arange(n, device=args.device)
            for pos in range(arity):
                flat.append(total + atom * arity + pos)
                obj.append(args[:, pos])
            total += n * arity
        flat_t = torch.cat(flat) if flat else torch.zeros(0, dtype=torch.long)
        obj_t = torch.cat(obj) if obj else torch.zeros(0, dtype=torch.long)
        # the fanin pair (flat_src, dst) is the same edge list as the fanout pair
        return {"meta": meta, "total": total, "flat": flat_t, "obj": obj_t,
                "deg": _object_degrees(obj_t, batch.num_objects)}

    def _routing_batched(self, batch: RelationalBatch) -> dict:
        """batched.py:121-257 (the fanout's packed plan) and the relation lane
        of BatchedFanInMP (its packed fanin plan): one edge list per
        (predicate, position) - argument object -> atom for the fanout, atom ->
        object for the fanin - packed by the pack ops into the operands of
        fanout_scatter (object row, slot_offset + atom * arity + pos) and of
        fanin_reduce (relation row atom * arity + pos after the predicate's
        rows, object).  Only the index outputs are kept: the reference packs
        with the layer's tensors, whose values the layers pass again."""

        meta, objs, atoms, part_of, arities, positions, offsets = [], [], [], [], [], [], []
        total = 0
        for pred in sorted(self.relations):
            args = batch.atoms.get(pred)
            if args is None or args.numel() == 0:
                continue
            n, arity = int(args.size(0)), self.relations[pred]
            atom = torch.arange(n, device=args.device)
            for pos in range(arity):
                objs.append(args[:, pos])
                atoms.append(atom)
                part_of.append(len(meta))
                arities.append(arity)
                positions.append(pos)
                offsets.append(total)
            meta.append((pred, n, arity, total))
            total += n * arity
        dev = next(iter(self.updater.parameters())).device
        if not meta:
            empty = torch.zeros(0, dtype=torch.long, device=dev)
            return {"meta": meta, "total": 0, "flat": empty, "obj": empty, "fanin_src": empty,
                    "fanin_dst": empty, "deg": torch.zeros(batch.num_objects, dtype=torch.long, device=dev)}
        # index computations only: one-column stand-ins for the value parts
        x_stub = torch.zeros(batch.num_objects, 1, device=dev)
        rel_stubs = [torch.zeros(n * arity, 1, device=dev) for _p, n, arity, _o in meta]
        _x, obj_t, flat_t = mp.fanout_pack_from_edges([x_stub], objs, atoms, [0] * len(objs), arities,
                                                      positions, offsets)
        _r, fanin_src, fanin_dst = mp.fanin_pack_from_edges(rel_stubs, atoms, objs, part_of, arities,
                                                            positions, 0)
        return {"meta": meta, "total": total, "flat": flat_t, "obj": obj_t, "fanin_src": fanin_src,
                "fanin_dst": fanin_dst, "deg": _object_degrees(fanin_dst, batch.num_objects)}

    def forward(self, batch: RelationalBatch, routing: dict | None = None) -> Tensor:
        r = routing or self.routing(batch)
        ref = next(iter(self.updater.parameters()))
        x = ref.new_zeros(batch.num_objects, self.d)
        for _ in range(self.num_layers):
            args = mp.fanout_scatter(x, r["obj"], r["flat"], r["total"])
            # split, not slices: the backward of split concatenates the parts'
            # gradients once, where each slice's would be a zero-filled full
            # copy, summed over the predicates
            parts = args.split([n * arity for _p, n, arity, _o in r["meta"]])
            # each predicate's residual MLP, its residual addition written
            # straight into the relation rows (_ResidualConcat)
            feats = [part.view(n, arity * self.d) for (_p, n, arity, _o), part in zip(r["meta"], parts)]
            ys = [self.rel_mlps[pred].module(feat) for (pred, _n, _a, _o), feat in zip(r["meta"], feats)]
            rel_flat = _ResidualConcat.apply(self.d, len(feats), *feats, *ys)
            msgs = fanin_objects(self.mode, rel_flat, r, batch.num_objects)
            x = x + self.updater(torch.cat([x, msgs], dim=1))
        return x


# ---- CentralizedRelationalGNN, fused central layer -------------------------------------


class CentralizedRelationalGNN(nn.Module):
    """CentralizedRelationalGNN with the fused central layer: every atom's
    arguments in max_arity padded slots, one central FiLM MLP conditioned on a
    learned relation embedding plus the slot mask, fanin over the padded slot
    layout, the same object update as RelationalGNN."""

    def __init__(self, embedding_size: int, num_layers: int, relations: dict[str, int], mode: int,
                 condition_dim: int | None = None, slot_mask: bool = True,
                 recompute_central: bool = False, gather_first_linear: bool = False,
                 sum_before_output: bool = False):
        super().__init__()
        self.d = embedding_size
        # evaluate the central MLP's first Linear per object and gather it per
        # relation node instead of assembling [cond | mask | slots] (_central_gathered)
        self.gather_first_linear = gather_first_linear
        # sum and mean aggregation with the gathered first Linear: add up the
        # hidden rows per (object, slot position) before the output Linear
        # (_central_messages)
        self.sum_before_output = sum_before_output
        # recompute the central module's hidden activations in the backward
        # (~4x the slot tensor, ~40 GB per layer at 2048 graphs): with the
        # fused FiLM step only its Mish output (_FilmMishLinear), otherwise the
        # whole module from its saved input (activation checkpointing)
        self.recompute_central = recompute_central
        self.num_layers = num_layers
        self.mode = mode
        self.relations = dict(relations)
        self.cond_index = {p: i for i, p in enumerate(self.relations)}
        self.max_arity = max(self.relations.values(), default=0)
        self.cond_dim = condition_dim or max(1, int(math.sqrt(embedding_size)))
        self.mask_dim = self.max_arity if slot_mask else 0
        self.cond = nn.Embedding(len(self.relations), self.cond_dim)
        feat_in = self.max_arity * embedding_size + self.mask_dim
        out = self.max_arity * embedding_size
        hidden = max(feat_in + self.cond_dim, out)
        # relational_gnn.py:757-787: residual FiLM MLP, condition first ("pre")
        self.central = Residual(FiLMConcatMLP(feat_in, self.cond_dim, [hidden], out), out)
        mask = torch.zeros(len(self.relations), self.max_arity)
        for p, a in self.relations.items():
            mask[self.cond_index[p], :a] = 1.0
        self.register_buffer("slot_mask", mask, persistent=False)
        self.updater = simple_mlp(2 * embedding_size, 2 * embedding_size, embedding_size)

    def routing(self, batch: RelationalBatch) -> dict:
        """fused.py:133-232: relation nodes ordered by predicate name; slot of
        (node, pos) = node * max_arity + pos."""

        meta, flat, obj = [], [], []
        start = 0
        for pred in sorted(self.relations):
            args = batch.atoms.get(pred)
            if args is None or args.numel() == 0 or self.relations[pred] == 0:
                continue
            n, arity = int(args.size(0)), self.relations[pred]
            meta.append((pred, start, n, arity, self.cond_index[pred]))
            node = torch.arange(n, device=args.device) + start
            for pos in range(arity):
                flat.append(node * self.max_arity + pos)
                obj.append(args[:, pos])
            start += n
        obj_t, flat_t = torch.cat(obj), torch.cat(flat)
        ma = self.max_arity
        # the slot edges of the gathered first Linear: slot (node, pos) reads
        # row obj * max_arity + pos of the per-object products
        slot_src = obj_t * ma + flat_t % ma
        return {"meta": meta, "nodes": start, "flat": flat_t, "obj": obj_t,
                "deg": _object_degrees(obj_t, batch.num_objects),
                "slot_src": slot_src, "slot_node": flat_t // ma,
                # edges per (object, slot position), for the output bias
                "slot_count": torch.bincount(slot_src, minlength=batch.num_objects * ma).view(-1, ma)}

    def _film_fused(self, t: Tensor, r: dict) -> bool:
        """Whether the FiLM steps run on the library's fused kernel (float32 on
        the GPU, at most 16 predicate ranges)."""

        return (t.dtype == torch.float32 and len(r["meta"]) <= 16
                and library_op("film_mish", tensor=t, gpu_only=True) is not None)

    def _hidden_pad(self, t: Tensor, r: dict) -> int:
        """Zero columns appended to the hidden width on the fused path (one
        hidden layer) to make it a multiple of 4: rows of 398 floats are only
        8-byte aligned, rows of 400 take 16-byte lanes in the gathers and the
        FiLM kernels (C5: a 398-wide gather-sum of 10.8 M rows 5.4 ms, 400-wide
        3.9 ms).  The padding columns stay exactly zero through the Linear
        (zero weight rows and bias), FiLM (zero gamma and beta: mish(0) = 0)
        and the output Linear (zero weight columns); F.pad's backward drops
        their gradients."""

        film = self.central.module
        if len(film.lins) != 1 or not self._film_fused(t, r):
            return 0
        return -film.lins[0].out_features % 4

    def _hidden_gathered(self, x: Tensor, r: dict, *, fused_output: bool) -> tuple[Tensor, Tensor | None, int]:
        """The central module's last hidden activation per relation node from
        the gathered first Linear (see _central_gathered), with `pad` zero
        columns appended (_hidden_pad).  With fused_output (selective
        recomputation on the fused kernel, one hidden layer) the last FiLM step
        and the output Linear run as one node and the second value is the
        output Linear's result instead."""

        film = self.central.module
        ma, d, md = self.max_arity, self.d, self.mask_dim
        lin = film.lins[0]
        pad = self._hidden_pad(x, r)
        width = lin.out_features + pad
        nodes = r["nodes"]
        table = self.cond.weight
        w, b = lin.weight, lin.bias
        if pad:
            w, b = nn.functional.pad(w, (0, 0, 0, pad)), nn.functional.pad(b, (0, pad))
        if md:
            const = torch.addmm(b, self.slot_mask, w[:, :md].t())  # [predicates, width]
        else:
            const = b.unsqueeze(0).expand(table.size(0), width)
        w_slots = w[:, md:].reshape(width, ma, d).transpose(0, 1).reshape(ma * width, d)
        per_object = linear(x, w_slots).view(-1, width)  # row obj * ma + a: x[obj] @ W_a^T
        s = mp.fanin_reduce(per_object, r["slot_src"], r["slot_node"], nodes, 0)

        sizes = [n for _p, _s, n, _a, _c in r["meta"]]
        if self._film_fused(s, r):
            # the FiLM steps as one kernel each: tables in range order
            order = torch.tensor([ci for _p, _s, _n, _a, ci in r["meta"]], device=s.device)
            starts = [st for _p, st, _n, _a, _c in r["meta"]] + [nodes]
            gamma, beta = film.gammas[0](table)[order], film.betas[0](table)[order]
            if pad:
                gamma, beta = nn.functional.pad(gamma, (0, pad)), nn.functional.pad(beta, (0, pad))
            if fused_output:
                w_out = nn.functional.pad(film.out.weight, (0, pad)) if pad else film.out.weight
                return s, _FilmMishLinear.apply(s, gamma, beta, const[order], starts, w_out,
                                                film.out.bias), pad
            h = _FilmMish.apply(s, gamma, beta, const[order], starts)
            for lin_k, g_k, b_k in zip(film.lins[1:], film.gammas[1:], film.betas[1:]):
                h = _FilmMish.apply(lin_k(h), g_k(table)[order], b_k(table)[order], None, starts)
            return h, None, pad

        def film_step(pre: Tensor, gamma: Tensor, beta: Tensor, add: Tensor | None) -> Tensor:
            # torch.split, not slicing: the backward of a split is one
            # concatenation, that of each slice a zero-filled full-size gradient
            parts = []
            for v, (_p, _s, _n, _a, ci) in zip(torch.split(pre, sizes), r["meta"]):
                parts.append(film.act(torch.addcmul(beta[ci], gamma[ci], v if add is None else v + add[ci])))
            return torch.cat(parts) if len(parts) > 1 else parts[0]

        h = film_step(s, film.gammas[0](table), film.betas[0](table), const)
        for lin_k, g_k, b_k in zip(film.lins[1:], film.gammas[1:], film.betas[1:]):
            h = film_step(lin_k(h), g_k(table), b_k(table), None)
        return h, None, 0

    def _central_messages(self, x: Tensor, r: dict, num_objects: int) -> Tensor:
        """Sum (or mean) of the central module's outputs over each object's
        slots, without the outputs: the output Linear is linear in the hidden
        rows, so the hidden rows are first added up per (object, slot position)
        - a fanin sum over the slot edges into [objects * max_arity, hidden] -
        and the Linear runs once per object on those sums with the slot
        positions' weight blocks side by side ([objects, max_arity * hidden] @
        [max_arity * hidden, d]).  The output bias enters once per edge (edge
        counts per (object, position) times the position's bias) and the
        residual - the slot itself, x[object] - deg(object) times.  At C5 the
        output Linear then runs over 0.59 M objects instead of 5.07 M nodes
        (0.18 instead of 1.55 TFLOP per pass), and the [nodes, max_arity * d]
        outputs and the dense slot table are never written.  Equals fanin of
        _central_gathered's result up to fp32 rounding (another summation
        order)."""

        film = self.central.module
        ma, d = self.max_arity, self.d
        h, _, pad = self._hidden_gathered(x, r, fused_output=False)
        hidden = h.size(1)
        hsum = mp.fanin_reduce(h, r["slot_node"], r["slot_src"], num_objects * ma, 0).view(num_objects,
                                                                                          ma * hidden)
        w_out = nn.functional.pad(film.out.weight, (0, pad)) if pad else film.out.weight
        w_pos = w_out.view(ma, d, hidden).transpose(0, 1).reshape(d, ma * hidden)
        count = r["slot_count"].to(x.dtype)
        base = torch.addmm(r["deg"].to(x.dtype).unsqueeze(1) * x, count, film.out.bias.view(ma, d))
        msgs = base + linear(hsum, w_pos)
        if self.mode == mp.MODE_MEAN:
            msgs = msgs / r["deg"].clamp_min(1).to(msgs.dtype).unsqueeze(1)
        return msgs

    def _central_gathered(self, x: Tensor, r: dict) -> Tensor:
        """The central module on [cond | slot mask | slots] per relation node,
        without assembling that input (fused.py:311-375 assembles it, then runs
        the module).  Its first Linear is linear in each slot: the weight
        columns of slot position a are applied once per object (x @ W_a^T for
        all positions in one GEMM) and each node adds the products of the
        objects in its slots - a fanin sum over the slot edges (at most
        max_arity messages per node, in slot order).  The condition and mask
        columns are constant per predicate, so their part of the Linear and
        FiLM's gamma / beta are evaluated on the per-predicate table and
        broadcast over each predicate's range of nodes (nodes are ordered by
        predicate; a broadcast's backward is a sum over the range, where a
        gather by node would accumulate millions of rows into a handful).  On
        the GPU in float32 each FiLM step with its Mish is one kernel over all
        ranges (torch.ops.relm_mp.film_mish, _FilmMish).
        The result equals self.central(input) up to fp32 rounding (another
        summation order)."""

        film = self.central.module
        ma, d = self.max_arity, self.d
        fused_output = (self.recompute_central and len(film.lins) == 1 and torch.is_grad_enabled()
                        and self._film_fused(x, r))
        h, out, pad = self._hidden_gathered(x, r, fused_output=fused_output)
        if out is None:
            out = film.out(h) if not pad else linear(h, nn.functional.pad(film.out.weight, (0, pad)),
                                                     film.out.bias)
        # Residual: the slots themselves (the fanout into a dense slot table)
        slots = mp.fanout_scatter(x, r["obj"], r["flat"], r["nodes"] * ma).view(r["nodes"], ma * d)
        return slots + out

    def forward(self, batch: RelationalBatch, routing: dict | None = None) -> Tensor:
        r = routing or self.routing(batch)
        ref = self.cond.weight
        x = ref.new_zeros(batch.num_objects, self.d)
        nodes, ma, d = r["nodes"], self.max_arity, self.d
        recompute = self.recompute_central and torch.is_grad_enabled()
        if self.gather_first_linear:
            aggregated = self.sum_before_output and self.mode in (mp.MODE_SUM, mp.MODE_MEAN)
            for _ in range(self.num_layers):
                if aggregated:
                    if recompute and not self._film_fused(x, r):
                        msgs = checkpoint(self._central_messages, x, r, batch.num_objects, use_reentrant=False)
                    else:
                        msgs = self._central_messages(x, r, batch.num_objects)
                    x = x + self.updater(torch.cat([x, msgs], dim=1))
                    continue
                # with the fused FiLM step the recomputation is selective
                # (_FilmMishLinear keeps the gathered sums only); otherwise the
                # whole central module is recomputed in the backward
                if recompute and not self._film_fused(x, r):
                    outputs = checkpoint(self._central_gathered, x, r, use_reentrant=False)
                else:
                    outputs = self._central_gathered(x, r)
                msgs = fanin_objects(self.mode, outputs.reshape(nodes * ma, d), r, batch.num_objects)
                x = x + self.updater(torch.cat([x, msgs], dim=1))
            return x
        # context columns [cond | slot mask] per relation node, built once per
        # forward and shared by the layers (fused.py:311-340)
        cond_rows = torch.cat([torch.full((n,), ci, dtype=torch.long, device=ref.device)
                               for _p, _s, n, _a, ci in r["meta"]])
        ctx = [self.cond(cond_rows)]
        if self.mask_dim:
            ctx.append(self.slot_mask[cond_rows])
        context = torch.cat(ctx, dim=1)
        for _ in range(self.num_layers):
            # [context | argument slots]: the fanout writes into the slots directly
            inp = mp.fanout_concat(context, x, r["obj"], r["flat"], ma)
            if recompute:
                outputs = checkpoint(self.central, inp, use_reentrant=False)
            else:
                outputs = self.central(inp)
            out_flat = outputs.reshape(nodes * ma, d)
            msgs = fanin_objects(self.mode, out_flat, r, batch.num_objects)
            x = x + self.updater(torch.cat([x, msgs], dim=1))
        return x


def train_step(model: nn.Module, batch: RelationalBatch, routing: dict) -> Tensor:
    """Forward + backward of loss = mean(out^2), as the reference's benchmark
    (scripts/benchmark_relational_models.py:287-295).  The routing's index
    tensors are built once per batch and never written during the step, so
    the step runs in one mp.plan_scope: each layer after the first reuses
    the index plans of the first without comparing the indices again; the
    layers' shared MLP weights are transposed once (shared_weight_transposes)."""

    model.zero_grad(set_to_none=True)
    with mp.plan_scope(), shared_weight_transposes():
        out = model(batch, routing)
        loss = out.square().mean()
        loss.backward()
    return loss.detach()


__all__ = [
    "CentralizedRelationalGNN",
    "RelationalBatch",
    "RelationalGNN",
    "synthetic_c4",
    "synthetic_c5",
    "train_step",
]
