#!/usr/bin/env python3
"""Benchmark of the relational message-passing hot path on one MI355X.

Headline ("C2"): fanin_reduce logsumexp forward +
backward through the public API (relmo_amd.mp + autograd) - 1,048,576
objects, D = 32, 16,777,216 messages ~ N(0, 2^2), Zipf(1.1) destinations.
One step = forward + backward over the whole batch, with the index plans
rebuilt in every step (the plan cache is cleared first), so the figure covers
the whole op call.  value = algorithmic bytes per step / time per step, in the
steady state: the first 20-30 steps of a process run up to 2% slower (the
same kernels take longer, the backward kernel included), so the default is
30 untimed warmup steps before the timed ones.

The JSON line also carries
  roofline      - the dominant kernel (logsumexp backward in edge order: flat_src
                  is the identity, so no index plan; one launch per step) timed
                  with HIP events on its stream around each timed step's
                  backward;
  cpu_baseline  - the reference's own CPU op library (oracle/_ref) on the
                  full C2 inputs (the job's thread share; 1 thread and a
                  1/8-scale sample of both CPU lanes in its variants);
  extra         - kernel-only rates with cached plans, C2 with sum, C3 fanout
                  forward + backward, C1 latencies, the pack ops (index
                  preparation) and the LGAN pooling step against their ATen
                  formulation, C4 / C5 model training steps (graphs/sec).

usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--only c2|c2sum|c2perm|c3|c1|c4|c5|pack|lgan|copy]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

PEAK_HBM_GBS = 8000.0
METRIC = "fanout/fanin fwd+bwd HBM GB/s (% of peak); RelationalGNN graphs/sec, 1 GPU"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gbs(nbytes: float, seconds: float) -> float:
    return nbytes / seconds / 1e9


def timed(fn, steps: int, warmup: int, sync) -> float:
    """Average seconds per call of fn over `steps` calls after `warmup` calls,
    bracketed by device synchronisation."""

    for _ in range(warmup):
        fn()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    sync()
    return (time.perf_counter() - t0) / steps


def event_time(fn, reps: int, torch) -> float:
    """Average seconds per launch measured with HIP events on the current stream
    (the stream the library enqueues on)."""

    stream = torch.cuda.current_stream()
    fn()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / 1e3 / reps


def load_traffic(name: str) -> dict | None:
    path = REPO / "profiles" / f"{name}.json"
    if path.exists():
        return json.loads(path.read_text())
    return None


def bench_c2(torch, mp, capi, syn, steps: int, warmup: int, mode: int) -> dict:
    dev = torch.device("cuda", 0)
    d = syn.c2_fanin(dev)
    rel, flat_src, dst, grad_out, K = d["rel"], d["flat_src"], d["dst"], d["grad_out"], d["dim_size"]
    E, D = rel.shape
    ns = torch.ops.relm_mp
    rel.requires_grad_(True)
    deg = torch.bincount(dst, minlength=K)
    info = {"max_degree": int(deg.max()), "empty_objects": int((deg == 0).sum()),
            "objects_over_64": int((deg > 64).sum())}
    if mode == 1:
        b_fwd, b_bwd = syn.bytes_fanin_fwd(E, D, K), syn.bytes_fanin_lse_bwd(E, D, K, E)
    else:
        b_fwd, b_bwd = syn.bytes_fanin_fwd(E, D, K), syn.bytes_fanin_sum_bwd(E, D, K, E)

    # The backward of every step (one launch: flat_src is the identity, so the
    # edge-order kernel runs without a plan) is bracketed by HIP events on the
    # stream it runs on, so the roofline kernel is timed inside the timed steps.
    stream = torch.cuda.current_stream()
    bwd_events = []

    def step_uncached():
        ns.plan_cache_clear()
        out = mp.fanin_reduce(rel, flat_src, dst, K, mode)
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        torch.autograd.grad(out, rel, grad_out)
        ev1.record(stream)
        bwd_events.append((ev0, ev1))

    def step_cached():
        out = mp.fanin_reduce(rel, flat_src, dst, K, mode)
        torch.autograd.grad(out, rel, grad_out)

    # The same topology handed over in new index tensors every step (a caller
    # that rebuilds its routing per forward): the plan cache matches the
    # contents against the cached plan's snapshot instead of rebuilding.
    fresh = iter([(flat_src.clone(), dst.clone()) for _ in range(steps + warmup)])

    def step_same_topology():
        s_idx, d_idx = next(fresh)
        out = mp.fanin_reduce(rel, s_idx, d_idx, K, mode)
        torch.autograd.grad(out, rel, grad_out)

    # A new topology every step with the cache kept: every forward compares
    # the new indices with the cached plans of the same shape (a mismatch ends
    # the comparison after the first tiles), then builds and keeps its plan.
    shifted = iter([(dst + i) % K for i in range(1, steps + warmup + 1)])

    def step_new_topology():
        out = mp.fanin_reduce(rel, flat_src, next(shifted), K, mode)
        torch.autograd.grad(out, rel, grad_out)

    # flat_src injective but not the identity, plans rebuilt every step: the
    # forward's CSR plan, and in the backward the inverse map of flat_src,
    # built from the forward plan's int32 snapshot (k_inv_scatter,
    # k_inv_verify), for k_lse_bwd_inv / k_gather_inv over it.
    #  * the callers' layout (fused.py:183-190): edges grouped by (predicate,
    #    argument position), atoms in order within a group, flat_src =
    #    (atom + predicate offset) * max_arity + position - here arity-2
    #    predicates, E / 2 atoms, flat_src[k * E/2 + a] = 2a + k;
    #  * a seeded random permutation: the worst case for both index maps.
    flat_callers = callers_flat_src(torch, E, 2, dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    flat_perm = torch.randperm(E, device=dev, generator=gen)

    def step_callers():
        ns.plan_cache_clear()
        out = mp.fanin_reduce(rel, flat_callers, dst, K, mode)
        torch.autograd.grad(out, rel, grad_out)

    def step_permuted():
        ns.plan_cache_clear()
        out = mp.fanin_reduce(rel, flat_perm, dst, K, mode)
        torch.autograd.grad(out, rel, grad_out)

    sync = torch.cuda.synchronize
    t_step = timed(step_uncached, steps, warmup, sync)
    t_bwd_step = statistics.fmean(a.elapsed_time(b) for a, b in bwd_events[-steps:]) / 1e3
    t_callers = timed(step_callers, steps, warmup, sync)
    t_perm = timed(step_permuted, steps, warmup, sync)
    del flat_perm, flat_callers
    t_cached = timed(step_cached, steps, warmup, sync)
    stats0 = ns.plan_cache_stats()
    t_same = timed(step_same_topology, steps, warmup, sync)
    content_hits = ns.plan_cache_stats()[2] - stats0[2]
    del fresh
    ns.plan_cache_clear()
    stats0 = ns.plan_cache_stats()
    t_new = timed(step_new_topology, steps, warmup, sync)
    stats1 = ns.plan_cache_stats()
    del shifted
    ns.plan_cache_clear()

    # Kernel-only timings with prebuilt plans, HIP events on the launch stream.
    r = rel.detach()
    fwd_plan = capi.csr_plan(dst, K, flat_src, E, "dst_idx", "flat_src", True)
    bwd_plan = capi.inv_plan(flat_src, E, dst, K, "flat_src", "dst_idx", True)
    out = capi.plan_segment_reduce(fwd_plan, r, mode)
    reps = max(steps, 10)
    t_fwd = event_time(lambda: capi.plan_segment_reduce(fwd_plan, r, mode), reps, torch)
    # what the step's backward runs: flat_src is the identity, so the backward
    # op reuses the forward's CSR plan (no inverse plan)
    assert fwd_plan.plan.gather_identity == 1
    t_bwd = event_time(lambda: capi.plan_fanin_backward_by_dst(fwd_plan, dst, mode, grad_out, E, out, r),
                       reps, torch)
    ident = capi.identity_inv_plan(E, E, K)
    if mode == 1:
        t_bwd_inv = event_time(lambda: capi.plan_logsumexp_backward(bwd_plan, grad_out, out, r, dst), reps, torch)
        t_bwd_ident = event_time(lambda: capi.plan_logsumexp_backward(ident, grad_out, out, r, dst), reps, torch)
    else:
        t_bwd_inv = event_time(lambda: capi.plan_gather_last(bwd_plan, grad_out, dst), reps, torch)
        t_bwd_ident = event_time(lambda: capi.plan_gather_last(ident, grad_out, dst), reps, torch)
    t_plan_fwd = timed(lambda: capi.csr_plan(dst, K, flat_src, E), 3, 1, sync)
    t_plan_bwd = timed(lambda: capi.inv_plan(flat_src, E, dst, K), 3, 1, sync)
    del fwd_plan, bwd_plan, out
    res = {
        "bytes_fwd": b_fwd, "bytes_bwd": b_bwd,
        "ms_step": t_step * 1e3, "gbs_step": gbs(b_fwd + b_bwd, t_step),
        "ms_step_cached_plans": t_cached * 1e3, "gbs_step_cached_plans": gbs(b_fwd + b_bwd, t_cached),
        "ms_step_same_topology_new_tensors": t_same * 1e3,
        "gbs_step_same_topology_new_tensors": gbs(b_fwd + b_bwd, t_same),
        "content_hits_same_topology": content_hits,
        "ms_step_callers_flat_src": t_callers * 1e3, "gbs_step_callers_flat_src": gbs(b_fwd + b_bwd, t_callers),
        "frac_step_callers_flat_src": gbs(b_fwd + b_bwd, t_callers) / PEAK_HBM_GBS,
        "ms_step_random_flat_src": t_perm * 1e3, "gbs_step_random_flat_src": gbs(b_fwd + b_bwd, t_perm),
        "frac_step_random_flat_src": gbs(b_fwd + b_bwd, t_perm) / PEAK_HBM_GBS,
        "ms_step_new_topology_cache_kept": t_new * 1e3,
        "gbs_step_new_topology_cache_kept": gbs(b_fwd + b_bwd, t_new),
        "misses_new_topology": stats1[3] - stats0[3],
        "plan_cache_peak_mb": stats1[5] / 2**20,
        "ms_fwd_kernels": t_fwd * 1e3, "gbs_fwd_kernels": gbs(b_fwd, t_fwd),
        "ms_bwd_in_step": t_bwd_step * 1e3, "gbs_bwd_in_step": gbs(b_bwd, t_bwd_step),
        "ms_bwd_kernel": t_bwd * 1e3, "gbs_bwd_kernel": gbs(b_bwd, t_bwd),
        "ms_bwd_kernel_inverse_plan": t_bwd_inv * 1e3, "ms_bwd_kernel_edge_order": t_bwd_ident * 1e3,
        "ms_plan_fwd_csr": t_plan_fwd * 1e3, "ms_plan_bwd_inverse": t_plan_bwd * 1e3,
        **info,
    }
    del d, rel, grad_out
    torch.cuda.empty_cache()
    return res


def callers_flat_src(torch, num_edges: int, arity: int, dev):
    """flat_src of the fused relation layer (fused.py:183-190) for predicates
    of one arity: edges grouped by argument position, atoms in order within a
    position, flat_src = atom * arity + position."""

    atoms = num_edges // arity
    a = torch.arange(atoms, device=dev, dtype=torch.int64)
    return torch.cat([a * arity + k for k in range(arity)])


def bench_c2_permuted(torch, mp, syn, steps: int, warmup: int, mode: int) -> dict:
    """C2 with the callers' flat_src layout only (callers_flat_src, arity 2;
    plans rebuilt every step): the workload of ``--only c2perm``, for kernel
    traces of that step alone."""

    dev = torch.device("cuda", 0)
    d = syn.c2_fanin(dev)
    rel, dst, grad_out, K = d["rel"], d["dst"], d["grad_out"], d["dim_size"]
    E, D = rel.shape
    ns = torch.ops.relm_mp
    rel.requires_grad_(True)
    flat_perm = callers_flat_src(torch, E, 2, dev)
    if mode == 1:
        nbytes = syn.bytes_fanin_fwd(E, D, K) + syn.bytes_fanin_lse_bwd(E, D, K, E)
    else:
        nbytes = syn.bytes_fanin_fwd(E, D, K) + syn.bytes_fanin_sum_bwd(E, D, K, E)

    def step():
        ns.plan_cache_clear()
        out = mp.fanin_reduce(rel, flat_perm, dst, K, mode)
        torch.autograd.grad(out, rel, grad_out)

    t = timed(step, steps, warmup, torch.cuda.synchronize)
    del d, rel, grad_out, flat_perm
    torch.cuda.empty_cache()
    return {"mode": mode, "ms_step": t * 1e3, "gbs_step": gbs(nbytes, t), "frac_of_peak": gbs(nbytes, t) / PEAK_HBM_GBS}


def bench_c3(torch, mp, capi, syn, steps: int, warmup: int) -> dict:
    dev = torch.device("cuda", 0)
    d = syn.c3_fanout(dev)
    x, src, flat_dst, grad_out, out_rows = d["x"], d["src"], d["flat_dst"], d["grad_out"], d["out_rows"]
    R, D = x.shape
    E = src.numel()
    ns = torch.ops.relm_mp
    x.requires_grad_(True)
    b_fwd, b_bwd = syn.bytes_fanout_fwd(E, D, out_rows), syn.bytes_fanout_bwd(E, D, R)

    def step_uncached():
        ns.plan_cache_clear()
        out = mp.fanout_scatter(x, src, flat_dst, out_rows)
        torch.autograd.grad(out, x, grad_out)

    def step_cached():
        out = mp.fanout_scatter(x, src, flat_dst, out_rows)
        torch.autograd.grad(out, x, grad_out)

    sync = torch.cuda.synchronize
    t_step = timed(step_uncached, steps, warmup, sync)
    t_cached = timed(step_cached, steps, warmup, sync)
    ns.plan_cache_clear()
    xd = x.detach()
    fwd_plan = capi.inv_plan(flat_dst, out_rows, src, R, "flat_dst", "src_global_idx", True)
    bwd_plan = capi.csr_plan(src, R, flat_dst, out_rows, "src_global_idx", "flat_dst", False)
    reps = max(steps, 10)
    t_fwd = event_time(lambda: capi.plan_gather_last(fwd_plan, xd, src), reps, torch)
    t_bwd = event_time(lambda: capi.plan_segment_reduce(bwd_plan, grad_out, 0), reps, torch)
    del fwd_plan, bwd_plan
    res = {
        "bytes_fwd": b_fwd, "bytes_bwd": b_bwd,
        "ms_step": t_step * 1e3, "gbs_step": gbs(b_fwd + b_bwd, t_step),
        "ms_step_cached_plans": t_cached * 1e3, "gbs_step_cached_plans": gbs(b_fwd + b_bwd, t_cached),
        "ms_fwd_kernel": t_fwd * 1e3, "gbs_fwd_kernel": gbs(b_fwd, t_fwd),
        "ms_bwd_kernels": t_bwd * 1e3, "gbs_bwd_kernels": gbs(b_bwd, t_bwd),
    }
    del d, x, grad_out
    torch.cuda.empty_cache()
    return res


def bench_c1(torch, mp, syn) -> dict:
    dev = torch.device("cuda", 0)
    d = syn.c1_ops(dev)
    ns = torch.ops.relm_mp
    calls = {
        "fanout_scatter": lambda: ns.fanout_scatter(d["x"], d["src"], d["flat_dst"], d["slots"]),
        "fanout_scatter_backward": lambda: ns.fanout_scatter_backward(d["grad_slots"], d["src"], d["flat_dst"], d["objects"]),
        "fanin_reduce_sum": lambda: ns.fanin_reduce(d["rel"], d["flat_src"], d["dst"], d["objects"], 0),
        "fanin_reduce_sum_backward": lambda: ns.fanin_reduce_sum_backward(d["grad_obj"], d["flat_src"], d["dst"], d["slots"]),
    }
    out = {}
    for name, fn in calls.items():
        ns.plan_cache_clear()
        out[f"us_{name}_uncached"] = timed(lambda: (ns.plan_cache_clear(), fn()), 20, 5, torch.cuda.synchronize) * 1e6
        out[f"us_{name}_cached"] = timed(fn, 50, 5, torch.cuda.synchronize) * 1e6
    ns.plan_cache_clear()
    return out


def bench_models(torch, which: str, steps: int, warmup: int) -> dict:
    """C4 (RelationalGNN, fast fused relation layer) and C5
    (CentralizedRelationalGNN, fused central layer): fp32 training step =
    forward + backward of mean(out^2) through relmo_amd.mp (HIP ops), index
    routing built once per batch as in the reference layers; graphs/sec =
    graphs / time per step.  C5 runs all 2048 graphs of its config (~5.1M
    relation nodes).  The MLP's first Linear runs per object and is gathered
    per relation node (CentralizedRelationalGNN._central_gathered: the same
    function, a ninth of its multiply-adds at C5); the FiLM step with its
    Mish and the Linear after it keep only the gathered sums (8 GB per
    layer) and recompute the Mish output in the backward with the fused
    kernel, which keeps the step under one GPU's 288 GB.  With sum and mean
    the hidden rows are added up per (object, slot position) before the
    output Linear (CentralizedRelationalGNN._central_messages: the output
    Linear over 0.59 M objects instead of 5.07 M nodes); logsumexp is not
    linear and keeps the per-node outputs.  Reported beside them: sum with
    the per-node outputs ("gathered_sum") and the step on the assembled input
    ("assembled_input_sum", the whole central module recomputed in the
    backward by activation checkpointing)."""

    from relmo_amd import consumers as C

    dev = torch.device("cuda", 0)
    if which == "c4":
        batch = C.synthetic_c4(dev)
        make = lambda mode: C.RelationalGNN(32, 10, batch.relations, mode).to(dev)
        cfg = {"graphs": batch.num_graphs, "objects": batch.num_objects, "emb": 32, "layers": 10,
               "weight_gradients": "reductions over atoms split into 2048/4096-row chunks read in place (consumers.weight_grad)",
               "narrow_products": "64-128 inner columns through rocBLAS (relm_mp::mm_nt)"}
        modes = ((0, "sum"), (1, "logsumexp"))
    else:
        log("  generating the C5 batch (2048 graphs)")
        batch = C.synthetic_c5(dev)
        make = lambda mode: C.CentralizedRelationalGNN(128, 10, batch.relations, mode, recompute_central=True,
                                                       gather_first_linear=True, sum_before_output=True).to(dev)
        cfg = {"graphs": batch.num_graphs, "objects": batch.num_objects,
               "relation_nodes": int(sum(a.size(0) for a in batch.atoms.values())), "emb": 128,
               "layers": 10,
               "central_mlp": ("hidden width padded 398 -> 400 (zero columns); logsumexp: FiLM step + Mish + Linear "
                               "keep the gathered sums, Mish output recomputed in the backward"),
               "first_linear": "per object, gathered per relation node (fanin sum over the slot edges)",
               "output_linear": "sum / mean: on the hidden rows summed per (object, slot position)"}
        modes = ((0, "sum"), (1, "logsumexp"), (2, "mean"))
    res = {"config": cfg}
    if which == "c5":
        res["structure"] = {
            "sum, logsumexp, mean": ("restructured central layer (this repository's): the first Linear per "
                                     "object, gathered per relation node; for sum / mean the output Linear on "
                                     "the hidden rows summed per (object, slot); logsumexp keeps per-node "
                                     "outputs"),
            "gathered_sum": "first Linear per object and gathered, per-node output Linear",
            "assembled_input_sum": ("the reference's CentralFusedLayerMP structure (fused.py:311-375): the "
                                    "central module on the assembled input - the like-for-like figure"),
        }
    variants = [(mode, name, True, True) for mode, name in modes]
    if which == "c5":  # per-node outputs, and the module on the assembled input (sum)
        variants += [(0, "gathered_sum", True, False), (0, "assembled_input_sum", False, False)]
    for mode, name, gathered, summed in variants:
        torch.manual_seed(0)
        model = make(mode)
        if which == "c5":
            model.gather_first_linear = gathered
            model.sum_before_output = summed
        routing = model.routing(batch)
        torch.cuda.reset_peak_memory_stats()
        t = timed(lambda: C.train_step(model, batch, routing), steps, warmup, torch.cuda.synchronize)
        res[name] = {"ms_step": t * 1e3, "graphs_per_sec": batch.num_graphs / t,
                     "peak_gb": torch.cuda.max_memory_allocated() / 1e9}
        log(f"  {which} {name}: {t * 1e3:.1f} ms per step")
        del model, routing
        torch.cuda.empty_cache()
    if which == "c4":
        res["slots"] = int(sum(a.numel() for a in batch.atoms.values()))
    return res


def bench_slots(torch, steps: int) -> dict:
    """The central layer's input assembly at a C5-like shape: 2^20 relation
    nodes x 3 argument slots of D = 128 after 14 context columns, 2^19
    objects, 2 arguments per node on average (2^21 fanout edges, slots of
    nodes with fewer arguments stay zero).  Timed, forward and forward +
    backward (random upstream gradient, gradients for the objects and the
    context): mp.fanout_concat (fanout_scatter_into / fanout_scatter_backward_from)
    against the reference's formulation (fanout_scatter into [nodes * 3, D],
    then torch.cat with the context).  Algorithmic bytes of the forward:
    the [nodes, 14 + 3 * 128] result written, the context and one object row
    per edge read, the indices read."""

    from relmo_amd import mp

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    nodes, slots, emb, ctx_cols, objects = 1 << 20, 3, 128, 14, 1 << 19
    edges = 2 * nodes
    x = torch.randn(objects, emb, device=dev, generator=gen, requires_grad=True)
    context = torch.randn(nodes, ctx_cols, device=dev, generator=gen, requires_grad=True)
    src = torch.randint(0, objects, (edges,), device=dev, generator=gen)
    dst = torch.randperm(nodes * slots, device=dev, generator=gen)[:edges]
    grad = torch.randn(nodes, ctx_cols + slots * emb, device=dev, generator=gen)

    def into():
        return mp.fanout_concat(context, x, src, dst, slots)

    def composed():
        args = mp.fanout_scatter(x, src, dst, nodes * slots)
        return torch.cat([context, args.view(nodes, slots * emb)], dim=1)

    res = {"config": {"nodes": nodes, "slots": slots, "emb": emb, "context_cols": ctx_cols,
                      "objects": objects, "edges": edges}}
    sync = torch.cuda.synchronize
    for name, fn in (("fanout_concat", into), ("fanout_then_cat", composed)):
        with torch.no_grad():
            t_f = timed(fn, steps, 2, sync)

        def step(fn=fn):
            x.grad = None
            context.grad = None
            fn().backward(grad)

        t_fb = timed(step, steps, 2, sync)
        res[name] = {"ms_fwd": t_f * 1e3, "ms_fwd_bwd": t_fb * 1e3}
    fwd_bytes = 4 * (nodes * (ctx_cols + slots * emb) + nodes * ctx_cols + edges * emb) + 16 * edges
    res["bytes_fwd"] = fwd_bytes
    res["gbs_fwd_fanout_concat"] = gbs(fwd_bytes, res["fanout_concat"]["ms_fwd"] / 1e3)
    return res


def bench_pack(torch, steps: int) -> dict:
    """Index preparation before one fanout / fanin call: fanout_pack_from_edges
    and fanin_pack_from_edges (mode 0) over 2 value parts of 2^20 x 64 f32 and
    16 edge parts (8 relations x arity 2) of 2^18 edges each (2^22 edges), as
    in a C3-sized batch.  Timed: the op through torch.ops.relm_mp (one HIP
    launch for all index parts + at::cat of the values), the same op in the
    reference's formulation (per-part tensor arithmetic + torch.cat, the ATen
    fallback, on the same GPU), and the index kernel alone (HIP events).
    Algorithmic bytes of the index kernel: 32 per edge (two int64 read, two
    written)."""

    from relmo_amd import capi, mp_pack

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    rows, emb, n_rel, arity, per = 1 << 20, 64, 8, 2, 1 << 18
    xs = [torch.randn(rows, emb, device=dev, generator=gen) for _ in range(2)]
    src = [torch.randint(0, rows, (per,), device=dev, generator=gen) for _ in range(n_rel * arity)]
    dst = [torch.randint(0, per, (per,), device=dev, generator=gen) for _ in range(n_rel * arity)]
    ids = [(r + p) % 2 for r in range(n_rel) for p in range(arity)]
    ar = [arity] * (n_rel * arity)
    pos = [p for _ in range(n_rel) for p in range(arity)]
    slot = [r * per * arity for r in range(n_rel) for _ in range(arity)]
    ns = torch.ops.relm_mp
    E = per * n_rel * arity
    idx_bytes = 32 * E
    val_bytes = 2 * sum(x.numel() * x.element_size() for x in xs)
    sync = torch.cuda.synchronize
    res = {"edges": E, "edge_parts": n_rel * arity, "value_parts": 2, "rows_per_part": rows, "emb": emb,
           "index_bytes": idx_bytes, "value_cat_bytes": val_bytes}
    for name, ours, aten in (
        ("fanout_pack_from_edges",
         lambda: ns.fanout_pack_from_edges(xs, src, dst, ids, ar, pos, slot),
         lambda: mp_pack.fanout_pack_from_edges_python(xs, src, dst, ids, ar, pos, slot)),
        ("fanin_pack_from_edges",
         lambda: ns.fanin_pack_from_edges(xs, src, dst, ids, ar, pos, 0),
         lambda: mp_pack.fanin_pack_from_edges_python(xs, src, dst, ids, ar, pos, 0)),
    ):
        t_ours = timed(ours, steps, 3, sync)
        t_aten = timed(aten, steps, 3, sync)
        res[name] = {"ms_op": t_ours * 1e3, "ms_aten_formulation": t_aten * 1e3,
                     "gbs_op": gbs(idx_bytes + val_bytes, t_ours),
                     "gbs_aten_formulation": gbs(idx_bytes + val_bytes, t_aten)}
    offsets = [0, rows]
    parts = [(s, d, 1, offsets[i], a, sl + p) for s, d, i, a, p, sl in zip(src, dst, ids, ar, pos, slot)]
    t_kernel = event_time(lambda: capi.pack_index(parts), max(steps, 20), torch)
    res["ms_index_kernel"] = t_kernel * 1e3
    res["gbs_index_kernel"] = gbs(idx_bytes, t_kernel)
    res["frac_index_kernel"] = res["gbs_index_kernel"] / PEAK_HBM_GBS
    del xs, src, dst
    torch.cuda.empty_cache()
    return res


def bench_lgan(torch, steps: int) -> dict:
    """LGAN pooling step forward + backward through relmo_amd.mp._lgan_pool_reduce
    (custom HIP ops) against the ATen formulation of the same op on the same
    GPU (the fallback, differentiated by autograd): 2^20 relation instances of
    arity 2 (2^21 slots), D = 64, 2^22 relation-relation edges, 2^21 tn and
    2^21 nn edges onto 2^19 entities, uniform random indices.  Loss = sum of
    the three outputs weighted by fixed random tensors.  Algorithmic bytes per
    forward: 4*D per slot read, per edge of each edge set (rows gathered), per
    output row written and per base row read; the backward the same over the
    transposed sets plus the slot gradients.  Timed with plans rebuilt in
    every step (cache cleared) and with plans kept."""

    from relmo_amd import mp
    from relmo_amd import mp_fallbacks

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    K, ent, D = 1 << 20, 1 << 19, 64
    E_slots, n_rr, n_tn, n_nn = 1 << 21, 1 << 22, 1 << 21, 1 << 21
    ri = lambda hi, n: torch.randint(0, hi, (n,), device=dev, generator=gen)  # noqa: E731
    slot = torch.randn(E_slots, D, device=dev, generator=gen).requires_grad_(True)
    s2r = torch.arange(E_slots, device=dev) // 2
    arity = torch.full((K,), 2, dtype=torch.long, device=dev)
    edges = [ri(K, n_rr), ri(K, n_rr), ri(K, n_tn), ri(ent, n_tn), ri(K, n_nn), ri(ent, n_nn)]
    w = [torch.randn(K, D, device=dev, generator=gen), torch.randn(ent, D, device=dev, generator=gen),
         torch.randn(ent, D, device=dev, generator=gen)]
    ns = torch.ops.relm_mp
    row = 4 * D
    fwd_bytes = row * (E_slots + K + n_rr + 2 * K + n_tn + ent + n_nn + ent)
    bwd_bytes = row * (n_tn + ent + 2 * K + n_nn + 2 * K + n_rr + 2 * K + E_slots + E_slots)
    res = {"relation_instances": K, "entities": ent, "emb": D, "slots": E_slots, "rr_edges": n_rr,
           "tn_edges": n_tn, "nn_edges": n_nn, "bytes_fwd": fwd_bytes, "bytes_bwd": bwd_bytes}

    def make_step(fn, clear):
        def step():
            if clear:
                ns.plan_cache_clear()
            outs = fn()
            torch.autograd.grad(outs, slot, w)
        return step

    sync = torch.cuda.synchronize
    for mode in ("sum", "mean"):
        custom = lambda: mp._lgan_pool_reduce(slot, s2r, arity, *edges, entity_dim_size=ent,  # noqa: E731
                                              mode=mode)
        m = 0 if mode == "sum" else 2
        aten = lambda: mp_fallbacks.lgan_pool_reduce_python(slot, s2r, arity, *edges, ent, m)  # noqa: E731
        t_unc = timed(make_step(custom, True), steps, 2, sync)
        t_cached = timed(make_step(custom, False), steps, 2, sync)
        t_aten = timed(make_step(aten, False), max(3, steps // 2), 1, sync)
        res[mode] = {"ms_step": t_unc * 1e3, "gbs_step": gbs(fwd_bytes + bwd_bytes, t_unc),
                     "ms_step_cached_plans": t_cached * 1e3,
                     "gbs_step_cached_plans": gbs(fwd_bytes + bwd_bytes, t_cached),
                     "ms_step_aten_formulation": t_aten * 1e3}
    ns.plan_cache_clear()
    del slot, edges, w
    torch.cuda.empty_cache()
    return res


def bench_copy(torch, steps: int) -> dict:
    """A plain 1 GiB device-to-device copy: the calibration kernel for the HBM
    byte counters (FETCH_SIZE / WRITE_SIZE per dispatch against 1 GiB)."""

    n = 1 << 28
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    sec = timed(lambda: b.copy_(a), max(steps, 3), 1, torch.cuda.synchronize)
    return {"bytes_read": 4 * n, "bytes_written": 4 * n, "ms": sec * 1e3, "gbs": gbs(8 * n, sec)}


def host_threads() -> int:
    """Host threads this job may use: the box's CPU share (OMP_NUM_THREADS),
    not every core the OS reports."""

    share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    return max(1, min(os.cpu_count() or 1, share))


def cpu_baseline(syn, torch) -> dict:
    """CPU baseline of the headline workload, logsumexp forward + backward on
    the host's cores:
      * headline: the reference's own CPU op library (oracle/_ref, built from
        mp_ops.cpp) on the full C2 inputs ``value`` is measured on (the same
        seeded tensors, generated on the GPU and copied to the host), once at
        the job's thread share and once at 1 thread, as the reference's bench
        pins (benchmark_mp_ops.py:634-638);
      * variants: the same library and relmo's python_only path (ATen
        index_select / scatter_reduce / exp / scatter_add / log and autograd,
        mirrored by relmo_amd.mp_pack) on a 1/8-scale C2 sample (131,072
        objects, 2,097,152 messages) at 1 thread and at the job's share.
    Falls back to the C oracle (1 thread, 1/8 sample) where oracle/_ref is
    absent."""

    import numpy as np

    from oracle import oracle, ref_runner
    from relmo_amd import mp
    from relmo_amd import mp_pack

    full = host_threads()
    variants = []
    headline = None
    if ref_runner.available():
        d = syn.c2_fanin(torch.device("cuda", 0))
        Kf, (Ef, Df) = d["dim_size"], d["rel"].shape
        out_f = mp.fanin_reduce(d["rel"], d["flat_src"], d["dst"], Kf, 1)
        arrays = {"rel": d["rel"].cpu().numpy(), "src": d["flat_src"].cpu().numpy(),
                  "dst": d["dst"].cpu().numpy(), "g": d["grad_out"].cpu().numpy(), "out": out_f.cpu().numpy()}
        del d, out_f
        torch.cuda.empty_cache()
        nbytes_f = syn.bytes_fanin_fwd(Ef, Df, Kf) + syn.bytes_fanin_lse_bwd(Ef, Df, Kf, Ef)
        calls = []
        for th in (full, 1):
            calls += [{"op": "fanin_reduce", "tensors": ["rel", "src", "dst"], "ints": [Kf, 1], "repeat": 1,
                       "warmup": 0, "threads": th, "keep": False},
                      {"op": "fanin_reduce_logsumexp_backward", "tensors": ["g", "rel", "src", "dst", "out"],
                       "ints": [Ef], "repeat": 1, "warmup": 0, "threads": th, "keep": False}]
        res = ref_runner.run_reference(calls, arrays, timeout=900.0)
        del arrays
        for i in (0, 2):
            if "error" in res[i] or "error" in res[i + 1]:
                raise RuntimeError(f"reference library: {res[i].get('error') or res[i + 1].get('error')}")
            t = res[i]["times"][0] + res[i + 1]["times"][0]
            threads = res[i]["threads"]
            entry = {"kind": "reference relm_mp_ops CPU lane, full C2", "threads": threads,
                     "seconds": round(t, 4), "value": round(gbs(nbytes_f, t), 3)}
            if headline is None:
                headline = {"value": entry["value"], "unit": "GB/s", "cores": threads, "kind": "reference",
                            "sample": (f"C2 in full, the inputs value is measured on (K={Kf}, E={Ef}, D={Df}, "
                                       f"Zipf(1.1) dst), logsumexp fwd+bwd; reference CPU lane (ATen "
                                       f"sequences, mp_ops.cpp:2981-3036), {threads} threads, one run, "
                                       f"{t:.3f} s per fwd+bwd")}
            else:
                variants.append(entry)

    K, E, D = 1 << 17, 1 << 21, 32
    rng = np.random.default_rng(0)
    ranks = np.arange(1, K + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -1.1)
    cdf /= cdf[-1]
    dst = rng.permutation(K)[np.minimum(np.searchsorted(cdf, rng.random(E), side="right"), K - 1)]
    rel = (2.0 * rng.standard_normal((E, D))).astype(np.float32)
    flat_src = np.arange(E, dtype=np.int64)
    g = rng.standard_normal((K, D)).astype(np.float32)
    nbytes = syn.bytes_fanin_fwd(E, D, K) + syn.bytes_fanin_lse_bwd(E, D, K, E)
    sample = f"C2 at 1/8 scale: K={K}, E={E}, D={D}, Zipf(1.1) dst, logsumexp fwd+bwd"

    # python_only: ATen forward + autograd backward, in this process on CPU tensors
    rel_t = torch.from_numpy(rel)
    src_t, dst_t, g_t = torch.from_numpy(flat_src), torch.from_numpy(dst), torch.from_numpy(g)

    def aten_step():
        r = rel_t.clone().requires_grad_(True)
        out = mp_pack.fanin_reduce_python(r, src_t, dst_t, K, 1)
        torch.autograd.grad(out, r, g_t)

    saved = torch.get_num_threads()
    for th in (1, full):
        torch.set_num_threads(th)
        if th != 1:  # the 1-thread run is long enough to go unwarmed
            aten_step()
        t0 = time.perf_counter()
        aten_step()
        t = time.perf_counter() - t0
        variants.append({"kind": "python_only (ATen), 1/8 C2", "threads": th, "seconds": round(t, 4),
                         "value": round(gbs(nbytes, t), 3)})
    torch.set_num_threads(saved)

    if headline is not None:
        out = oracle.fanin_reduce_logsumexp(rel, flat_src, dst, K)
        arrays = {"rel": rel, "src": flat_src, "dst": dst, "g": g, "out": out}
        for th, reps, warm in ((1, 1, 0), (full, 3, 1)):
            calls = [
                {"op": "fanin_reduce", "tensors": ["rel", "src", "dst"], "ints": [K, 1], "repeat": reps,
                 "warmup": warm, "threads": th},
                {"op": "fanin_reduce_logsumexp_backward", "tensors": ["g", "rel", "src", "dst", "out"],
                 "ints": [E], "repeat": reps, "warmup": warm, "threads": th},
            ]
            res = ref_runner.run_reference(calls, arrays)
            t = statistics.median(res[0]["times"]) + statistics.median(res[1]["times"])
            variants.append({"kind": "reference relm_mp_ops CPU lane, 1/8 C2", "threads": res[0]["threads"],
                             "seconds": round(t, 4), "value": round(gbs(nbytes, t), 3)})
        headline["variants"] = variants
        headline["sample_1_8"] = sample
        headline["host"] = host_info(torch)
        return headline
    t0 = time.perf_counter()
    out = oracle.fanin_reduce_logsumexp(rel, flat_src, dst, K)
    oracle.fanin_reduce_logsumexp_backward(g, rel, flat_src, dst, out, E)
    t = time.perf_counter() - t0
    return {"value": round(gbs(nbytes, t), 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": sample + f"; C oracle, 1 thread, {t:.3f} s per fwd+bwd", "variants": variants,
            "host": host_info(torch)}


def host_info(torch) -> dict:
    """The host the CPU baselines ran on."""

    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        rocm = Path("/opt/rocm/.info/version").read_text().strip()
    except OSError:
        rocm = None
    return {"cpu_model": cpu, "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "job_threads": host_threads(), "torch": torch.__version__, "hip": torch.version.hip,
            "rocm": rocm}


def cpu_full(torch, syn, parts: set[str]) -> dict:
    """The full CPU baseline plan, on the host's cores (``--cpu-full``; minutes
    of CPU work, so not part of the default run):

      * C1 in full - the reference's CPU op library (oracle/_ref) per op,
        median of 80 calls after 20 warmup (benchmark_mp_ops.py:74-117 with
        one call per sample), and relmo's python_only ATen lane (forward, and
        forward + autograd backward) - at 1 thread and at the job's share;
      * C2 (logsumexp and sum) and C3 (fanout) at full size, once per thread
        count, the same two lanes;
      * C4 (512 graphs) and C5 (a 64-graph sample of its 2048) training steps
        on the ATen model path (RELM_MP_ENABLE=0), at the job's share,
        graphs/sec of one step after one warmup step."""

    from oracle import ref_runner

    full = host_threads()
    threads = (1, full)
    have_ref = ref_runner.available()
    res: dict = {"host": host_info(torch), "threads": list(threads), "reference_lane": have_ref}

    def aten(fn, th, reps, warm):
        saved = torch.get_num_threads()
        torch.set_num_threads(th)
        try:
            for _ in range(warm):
                fn()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
        finally:
            torch.set_num_threads(saved)
        return statistics.median(ts)

    def ref(specs, arrays, reps, warm):
        """{threads: {name: median seconds}} for the reference library's ops."""

        calls = [{"op": op, "tensors": ts, "ints": ints, "repeat": reps, "warmup": warm, "threads": th,
                  "keep": False} for th in threads for _name, op, ts, ints in specs]
        out = ref_runner.run_reference(calls, arrays, timeout=1800.0)
        got: dict = {}
        for call, r in zip(calls, out):
            if "error" in r:
                raise RuntimeError(f"reference {call['op']}: {r['error']}")
        i = 0
        for th in threads:
            got[th] = {}
            for name, *_ in specs:
                got[th][name] = statistics.median(out[i]["times"])
                i += 1
        return got

    def grad_of(fn, leaf, g):
        def step():
            x = leaf.clone().requires_grad_(True)
            torch.autograd.grad(fn(x), x, g)
        return step

    if "c1" in parts:
        res["c1"] = cpu_c1(torch, syn, aten, ref, grad_of, threads, have_ref)
    if "c2" in parts:
        res["c2"] = cpu_c2(torch, syn, ref, threads, have_ref)
    if "c3" in parts:
        res["c3"] = cpu_c3(torch, syn, ref, threads, have_ref)
    if parts & {"c4", "c5"}:
        res.update(cpu_models(torch, full, parts))
    return res


def cpu_c1(torch, syn, aten, ref, grad_of, threads, have_ref) -> dict:
    from relmo_amd import mp_pack

    log("CPU C1 ...")
    d = syn.c1_ops("cpu")
    objects, slots = d["objects"], d["slots"]
    c1: dict = {"python_only_us": {}}
    py = {
        "fanout_scatter": lambda: mp_pack.fanout_scatter_python(d["x"], d["src"], d["flat_dst"], slots),
        "fanout_scatter_fwd_bwd": grad_of(
            lambda x: mp_pack.fanout_scatter_python(x, d["src"], d["flat_dst"], slots), d["x"], d["grad_slots"]),
        "fanin_reduce_sum": lambda: mp_pack.fanin_reduce_python(d["rel"], d["flat_src"], d["dst"], objects, 0),
        "fanin_reduce_sum_fwd_bwd": grad_of(
            lambda r: mp_pack.fanin_reduce_python(r, d["flat_src"], d["dst"], objects, 0), d["rel"], d["grad_obj"]),
    }
    for th in threads:
        c1["python_only_us"][th] = {k: round(aten(fn, th, 80, 20) * 1e6, 1) for k, fn in py.items()}
    if have_ref:
        arrays = {k: v.numpy() for k, v in d.items() if isinstance(v, torch.Tensor)}
        specs = [("fanout_scatter", "fanout_scatter", ["x", "src", "flat_dst"], [slots]),
                 ("fanout_scatter_backward", "fanout_scatter_backward", ["grad_slots", "src", "flat_dst"], [objects]),
                 ("fanin_reduce_sum", "fanin_reduce", ["rel", "flat_src", "dst"], [objects, 0]),
                 ("fanin_reduce_sum_backward", "fanin_reduce_sum_backward", ["grad_obj", "flat_src", "dst"], [slots])]
        got = ref(specs, arrays, 80, 20)
        c1["reference_us"] = {th: {k: round(v * 1e6, 1) for k, v in got[th].items()} for th in threads}
    return c1


def cpu_c2(torch, syn, ref, threads, have_ref) -> dict:
    from relmo_amd import mp_pack

    log("CPU C2 ...")
    d = syn.c2_fanin("cpu")
    K, E, D = d["dim_size"], d["rel"].size(0), d["rel"].size(1)
    lse_bytes = syn.bytes_fanin_fwd(E, D, K) + syn.bytes_fanin_lse_bwd(E, D, K, E)
    sum_bytes = syn.bytes_fanin_fwd(E, D, K) + syn.bytes_fanin_sum_bwd(E, D, K, E)
    c2: dict = {"bytes_lse_fwd_bwd": lse_bytes, "bytes_sum_fwd_bwd": sum_bytes, "python_only_s": {}}
    saved = torch.get_num_threads()
    for th in threads:
        c2["python_only_s"][th] = {}
        torch.set_num_threads(th)
        for mode, m in (("logsumexp", 1), ("sum", 0)):
            # forward, then the autograd backward, each reported as it ends
            r = d["rel"].clone().requires_grad_(True)
            t0 = time.perf_counter()
            out = mp_pack.fanin_reduce_python(r, d["flat_src"], d["dst"], K, m)
            fwd = time.perf_counter() - t0
            log(f"  python_only C2 {mode} forward, {th} threads: {fwd:.2f} s")
            t0 = time.perf_counter()
            torch.autograd.grad(out, r, d["grad_out"])
            bwd = time.perf_counter() - t0
            log(f"  python_only C2 {mode} backward, {th} threads: {bwd:.2f} s")
            del r, out
            c2["python_only_s"][th][f"{mode}_fwd"] = round(fwd, 3)
            c2["python_only_s"][th][f"{mode}_bwd"] = round(bwd, 3)
            c2["python_only_s"][th][f"{mode}_fwd_bwd"] = round(fwd + bwd, 3)
    torch.set_num_threads(saved)
    if have_ref:
        out = mp_pack.fanin_reduce_python(d["rel"], d["flat_src"], d["dst"], K, 1)
        arrays = {"rel": d["rel"].numpy(), "src": d["flat_src"].numpy(), "dst": d["dst"].numpy(),
                  "g": d["grad_out"].numpy(), "out": out.numpy()}
        specs = [("logsumexp_fwd", "fanin_reduce", ["rel", "src", "dst"], [K, 1]),
                 ("logsumexp_bwd", "fanin_reduce_logsumexp_backward", ["g", "rel", "src", "dst", "out"], [E]),
                 ("sum_fwd", "fanin_reduce", ["rel", "src", "dst"], [K, 0]),
                 ("sum_bwd", "fanin_reduce_sum_backward", ["g", "src", "dst"], [E])]
        got = ref(specs, arrays, 1, 0)
        c2["reference_s"] = {th: {k: round(v, 3) for k, v in got[th].items()} for th in threads}
        c2["reference_gbs"] = {th: {
            "logsumexp_fwd_bwd": round(gbs(lse_bytes, got[th]["logsumexp_fwd"] + got[th]["logsumexp_bwd"]), 3),
            "sum_fwd_bwd": round(gbs(sum_bytes, got[th]["sum_fwd"] + got[th]["sum_bwd"]), 3)} for th in threads}
        del arrays, out
    c2["python_only_gbs"] = {th: {"logsumexp_fwd_bwd": round(gbs(lse_bytes, v["logsumexp_fwd_bwd"]), 3),
                                  "sum_fwd_bwd": round(gbs(sum_bytes, v["sum_fwd_bwd"]), 3)}
                             for th, v in c2["python_only_s"].items()}
    return c2


def cpu_c3(torch, syn, ref, threads, have_ref) -> dict:
    from relmo_amd import mp_pack

    log("CPU C3 ...")
    d = syn.c3_fanout("cpu")
    R, D = d["x"].shape
    S = d["out_rows"]
    c3_bytes = syn.bytes_fanout_fwd(S, D, S) + syn.bytes_fanout_bwd(S, D, R)
    c3: dict = {"bytes_fwd_bwd": c3_bytes, "python_only_s": {}}
    saved = torch.get_num_threads()
    for th in threads:
        torch.set_num_threads(th)
        x = d["x"].clone().requires_grad_(True)
        t0 = time.perf_counter()
        out = mp_pack.fanout_scatter_python(x, d["src"], d["flat_dst"], S)
        fwd = time.perf_counter() - t0
        log(f"  python_only C3 forward, {th} threads: {fwd:.2f} s")
        t0 = time.perf_counter()
        torch.autograd.grad(out, x, d["grad_out"])
        bwd = time.perf_counter() - t0
        log(f"  python_only C3 backward, {th} threads: {bwd:.2f} s")
        del x, out
        c3["python_only_s"][th] = round(fwd + bwd, 3)
    torch.set_num_threads(saved)
    if have_ref:
        arrays = {"x": d["x"].numpy(), "src": d["src"].numpy(), "flat": d["flat_dst"].numpy(),
                  "g": d["grad_out"].numpy()}
        specs = [("fanout_fwd", "fanout_scatter", ["x", "src", "flat"], [S]),
                 ("fanout_bwd", "fanout_scatter_backward", ["g", "src", "flat"], [R])]
        got = ref(specs, arrays, 1, 0)
        c3["reference_s"] = {th: {k: round(v, 3) for k, v in got[th].items()} for th in threads}
        c3["reference_gbs"] = {th: round(gbs(c3_bytes, got[th]["fanout_fwd"] + got[th]["fanout_bwd"]), 3)
                               for th in threads}
        del arrays
    c3["python_only_gbs"] = {th: round(gbs(c3_bytes, v), 3) for th, v in c3["python_only_s"].items()}
    return c3


def cpu_models(torch, full: int, parts: set[str]) -> dict:
    """C4 / C5 training steps on the ATen model path at `full` threads."""

    from relmo_amd import consumers as C

    res = {}
    saved_env = os.environ.get("RELM_MP_ENABLE")
    os.environ["RELM_MP_ENABLE"] = "0"
    saved_threads = torch.get_num_threads()
    torch.set_num_threads(full)
    try:
        for name, batch_fn, make, modes in (
            ("c4", lambda: C.synthetic_c4("cpu"), lambda b, m: C.RelationalGNN(32, 10, b.relations, m),
             ((0, "sum"), (1, "logsumexp"))),
            ("c5", lambda: C.synthetic_c5("cpu", num_graphs=64),
             lambda b, m: C.CentralizedRelationalGNN(128, 10, b.relations, m),
             ((0, "sum"), (1, "logsumexp"), (2, "mean"))),
        ):
            if name not in parts:
                continue
            log(f"CPU {name} ...")
            batch = batch_fn()
            entry: dict = {"graphs": batch.num_graphs, "objects": batch.num_objects, "threads": full}
            for m, mode in modes:
                torch.manual_seed(0)
                model = make(batch, m)
                routing = model.routing(batch)
                C.train_step(model, batch, routing)
                t0 = time.perf_counter()
                C.train_step(model, batch, routing)
                t = time.perf_counter() - t0
                entry[mode] = {"s_step": round(t, 3), "graphs_per_sec": round(batch.num_graphs / t, 2)}
                log(f"  {name} {mode}: {t:.2f} s per step")
            res[name] = entry
    finally:
        torch.set_num_threads(saved_threads)
        if saved_env is None:
            os.environ.pop("RELM_MP_ENABLE", None)
        else:
            os.environ["RELM_MP_ENABLE"] = saved_env
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--only", choices=["c2", "c2sum", "c2perm", "c3", "c1", "c4", "c5", "pack", "lgan", "slots",
                                       "copy"],
                    default=None,
                    help="run one workload only and print its figures (for profiling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-full", nargs="?", const="c1,c2,c3,c4,c5", default=None, metavar="PARTS",
                    help="run the full CPU baseline plan on the host's cores and print it: all of "
                         "C1-C5, or the comma-separated parts named")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the op library has no multi-GPU path; one GPU holds a whole C2 / C3 batch).", file=sys.stderr)
        return 2

    os.environ["RELM_MP_FALLBACK"] = "error"
    import torch

    from relmo_amd import capi, mp
    from relmo_amd import synthetic as syn

    if args.cpu_full:
        parts = {p.strip().lower() for p in args.cpu_full.split(",") if p.strip()}
        unknown = parts - {"c1", "c2", "c3", "c4", "c5"}
        if unknown:
            print(f"--cpu-full: unknown parts {sorted(unknown)}", file=sys.stderr)
            return 2
        print(json.dumps({"cpu_full": cpu_full(torch, syn, parts)}), flush=True)
        return 0

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if not mp.available():
        raise RuntimeError("relm_mp_ops.so failed to load")

    if args.only:
        fn = {"c2": lambda: bench_c2(torch, mp, capi, syn, args.steps, args.warmup, 1),
              "c2sum": lambda: bench_c2(torch, mp, capi, syn, args.steps, args.warmup, 0),
              "c2perm": lambda: bench_c2_permuted(torch, mp, syn, args.steps, args.warmup, 1),
              "c3": lambda: bench_c3(torch, mp, capi, syn, args.steps, args.warmup),
              "c1": lambda: bench_c1(torch, mp, syn),
              "c4": lambda: bench_models(torch, "c4", args.steps, args.warmup),
              "c5": lambda: bench_models(torch, "c5", args.steps, args.warmup),
              "pack": lambda: bench_pack(torch, args.steps),
              "lgan": lambda: bench_lgan(torch, args.steps),
              "slots": lambda: bench_slots(torch, args.steps),
              "copy": lambda: bench_copy(torch, args.steps)}[args.only]
        print(json.dumps({args.only: fn()}), flush=True)
        return 0

    log("C2 logsumexp fwd+bwd ...")
    c2 = bench_c2(torch, mp, capi, syn, args.steps, args.warmup, 1)
    log(f"  {c2['gbs_step']:.0f} GB/s per step; dominant kernel {c2['gbs_bwd_kernel']:.0f} GB/s")
    extra = {"c2_logsumexp": c2}
    log("C2 sum fwd+bwd ...")
    extra["c2_sum"] = bench_c2(torch, mp, capi, syn, max(5, args.steps // 2), 2, 0)
    log("C3 fanout fwd+bwd ...")
    extra["c3_fanout"] = bench_c3(torch, mp, capi, syn, max(5, args.steps // 2), 2)
    log("C1 latencies ...")
    extra["c1_latency_us"] = bench_c1(torch, mp, syn)
    log("pack ops (index preparation) ...")
    extra["pack"] = bench_pack(torch, max(5, args.steps // 2))
    log("LGAN pooling step ...")
    extra["lgan"] = bench_lgan(torch, max(5, args.steps // 2))
    log("fanout into argument slots ...")
    extra["slots"] = bench_slots(torch, max(5, args.steps // 2))
    log("C4 RelationalGNN training step ...")
    extra["c4_relational_gnn"] = bench_models(torch, "c4", 5, 2)
    log("C5 CentralizedRelationalGNN training step ...")
    extra["c5_centralized_gnn"] = bench_models(torch, "c5", 3, 1)

    baseline = None
    if not args.no_cpu_baseline:
        log("CPU baseline ...")
        baseline = cpu_baseline(syn, torch)

    kernel = "k_lse_bwd_inv"
    traffic = load_traffic("c2_logsumexp_backward_traffic")
    if traffic is not None and not traffic.get("kernel", "").startswith(kernel):
        traffic = None
    bwd_bytes = c2["bytes_bwd"]
    # the backward launches of the timed steps (HIP events around each)
    achieved = gbs(bwd_bytes, c2["ms_bwd_in_step"] / 1e3)
    roofline = {
        "bound": "hbm",
        "kernel": f"{kernel} (fanin_reduce_logsumexp_backward, identity flat_src: edge order, no plan)",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": traffic.get("bytes_per_launch") if traffic else None,
    }
    ms = c2["ms_step"]
    line = {
        "metric": METRIC,
        "value": round(c2["gbs_step"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "C2: fanin_reduce logsumexp fwd+bwd, 1,048,576 objects, D=32, 16,777,216 messages "
                        "~N(0,2^2), Zipf(1.1) destinations (unsorted), plans rebuilt every step",
            "objects": 1 << 20, "messages": 1 << 24, "emb": 32,
            "bytes_per_step": c2["bytes_fwd"] + c2["bytes_bwd"],
            "frac_of_peak": round(c2["gbs_step"] / PEAK_HBM_GBS, 4),
        },
        "roofline": roofline,
        "cpu_baseline": baseline,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
