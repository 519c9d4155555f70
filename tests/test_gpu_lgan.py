"""GPU parity of the LGAN indexed reductions (lgan_pool_reduce,
lgan_relation_graph_step and their backward ops): the HIP path (CSR segment
sums + relm_mp_rows_scale epilogues) against the reference's golden fixtures
and the numpy oracle (oracle/lgan.py).

Bars: destinations with at most 64 messages add in edge order, like the
reference's index_add_, so those results are bit-exact; the cases with a
destination of more than 64 messages (hub folding order) are compared with the
float64 truth: |got - truth| <= 8 * eps32 * F(|inputs|), F the same op (every
op here is a linear map with nonnegative coefficients, so F(|inputs|) bounds
the sum of the magnitudes of all terms of an output)."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import lgan as lgan_oracle
from tests.conftest import pack_args

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    os.environ["RELM_MP_FALLBACK"] = "error"
    from relmo_amd import mp_runtime

    mp_runtime.ensure_loaded()
    yield


@pytest.fixture(scope="module")
def ops():
    return torch.ops.relm_mp


def test_lgan_ops_reproduce_golden_on_gpu(ops, lgan_golden) -> None:
    cases, arrays = lgan_golden
    for case in cases:
        _log(f"lgan golden case {case['name']}")
        args = pack_args(case, arrays, DEV)
        fn = getattr(ops, case["op"])
        if "error" in case:
            with pytest.raises((RuntimeError, ValueError, IndexError)) as info:
                fn(*args)
            if "out of bounds" not in case["error"]:  # index checks are the plan builds' own
                assert str(info.value).splitlines()[0] == case["error"], case["name"]
            continue
        got = fn(*args)
        torch.cuda.synchronize()
        got = got if isinstance(got, (tuple, list)) else (got,)
        for g, name in zip(got, case["expected"]):
            assert g.is_cuda, case["name"]
            g = g.cpu().numpy()
            want = arrays[name]
            assert g.dtype == want.dtype and g.shape == want.shape, case["name"]
            if case["name"].startswith("b_"):
                _within_fp32_bound(case, arrays, g, want, case["expected"].index(name))
            else:
                assert np.array_equal(g, want), case["name"]


LGAN_FNS = {
    "lgan_pool_reduce": lgan_oracle.lgan_pool_reduce,
    "lgan_pool_reduce_backward": lgan_oracle.lgan_pool_reduce_backward,
    "lgan_relation_graph_step": lgan_oracle.lgan_relation_graph_step,
    "lgan_relation_graph_step_backward": lgan_oracle.lgan_relation_graph_step_backward,
}


def _within_fp32_bound(case: dict, arrays: dict, got: np.ndarray, want: np.ndarray, k: int) -> None:
    def run(transform):
        args = []
        for spec in case["args"]:
            if "int" in spec:
                args.append(spec["int"])
                continue
            a = arrays[spec["tensor"]]
            args.append(transform(a) if a.dtype.kind == "f" else a)
        out = LGAN_FNS[case["op"]](*args)
        return (out if isinstance(out, tuple) else (out,))[k]

    truth = run(lambda a: a.astype(np.float64))
    bound = 8 * np.finfo(np.float32).eps * run(lambda a: np.abs(a).astype(np.float64)) + 1e-30
    assert np.all(np.abs(got - truth) <= bound), case["name"]
    assert np.all(np.abs(want - truth) <= bound), case["name"]


def _graph(seed: int, K=50_000, ent=20_000, E=120_000, D=32, n_rr=200_000, n_tn=80_000,
           n_nn=60_000, dtype=torch.float32):
    rng = np.random.default_rng(seed)
    host = dict(
        slot=rng.standard_normal((E, D)).astype(np.float32 if dtype == torch.float32 else np.float64),
        s2r=rng.integers(0, K, E), arity=rng.integers(0, 4, K),
        edges=[rng.integers(0, b, n) for b, n in
               [(K, n_rr), (K, n_rr), (K, n_tn), (ent, n_tn), (K, n_nn), (ent, n_nn)]])
    dev = dict(slot=torch.from_numpy(host["slot"]).to(DEV), s2r=torch.from_numpy(host["s2r"]).to(DEV),
               arity=torch.from_numpy(host["arity"]).to(DEV),
               edges=[torch.from_numpy(e).to(DEV) for e in host["edges"]])
    return host, dev, K, ent


@pytest.mark.parametrize("mode", [0, 2])
def test_lgan_random_graph_matches_oracle(ops, mode) -> None:
    host, dev, K, ent = _graph(50 + mode)
    _log(f"lgan random graph mode {mode}: pool + step forward and backward")
    outs = ops.lgan_pool_reduce(dev["slot"], dev["s2r"], dev["arity"], *dev["edges"], ent, mode)
    want = lgan_oracle.lgan_pool_reduce(host["slot"], host["s2r"], host["arity"], *host["edges"],
                                        ent, mode)
    for g, w in zip(outs, want):
        assert np.array_equal(g.cpu().numpy(), w)
    step = ops.lgan_relation_graph_step(outs[0], *dev["edges"], ent, mode)
    want_step = lgan_oracle.lgan_relation_graph_step(want[0], *host["edges"], ent, mode)
    for g, w in zip(step, want_step):
        assert np.array_equal(g.cpu().numpy(), w)
    rng = np.random.default_rng(60 + mode)
    gh = [rng.standard_normal(o.shape).astype(np.float32) for o in want]
    gd = [torch.from_numpy(g).to(DEV) for g in gh]
    grad = ops.lgan_pool_reduce_backward(*gd, dev["s2r"], dev["arity"], *dev["edges"], K, mode)
    want_grad = lgan_oracle.lgan_pool_reduce_backward(*gh, host["s2r"], host["arity"],
                                                      *host["edges"], K, mode)
    assert np.array_equal(grad.cpu().numpy(), want_grad)
    grad_step = ops.lgan_relation_graph_step_backward(*gd, *dev["edges"], K, mode)
    want_step_grad = lgan_oracle.lgan_relation_graph_step_backward(*gh, *host["edges"], K, mode)
    assert np.array_equal(grad_step.cpu().numpy(), want_step_grad)


@pytest.mark.parametrize("mode", ["sum", "mean"])
def test_lgan_facade_autograd_on_gpu(mode) -> None:
    """CUDA tensors run the custom forward and backward ops; gradients equal the
    CPU fallback's autograd and pass gradcheck in float64."""

    from relmo_amd import mp

    ns = torch.ops.relm_mp
    host, dev, K, ent = _graph(70, K=400, ent=150, E=900, D=5, n_rr=1500, n_tn=700, n_nn=500,
                               dtype=torch.float64)
    grads = []
    for where in ("cpu", DEV):
        slot = torch.from_numpy(host["slot"]).to(where).requires_grad_(True)
        idx = [torch.from_numpy(a).to(where) for a in (host["s2r"], host["arity"], *host["edges"])]
        outs = mp._lgan_pool_reduce(slot, *idx, entity_dim_size=ent, mode=mode)
        step = mp._lgan_relation_graph_step(outs[0], *idx[2:], entity_dim_size=ent, mode=mode)
        loss = sum((o * o).sum() for o in (*outs[1:], *step))
        (g,) = torch.autograd.grad(loss, slot)
        grads.append(g.cpu())
    torch.testing.assert_close(grads[1], grads[0], rtol=1e-12, atol=1e-12)
    before = ns.plan_cache_stats()
    idx = dev["edges"]
    x = torch.randn(K, 3, dtype=torch.float64, device=DEV, requires_grad=True)
    assert torch.autograd.gradcheck(
        lambda v: mp._lgan_relation_graph_step(v, *idx, entity_dim_size=ent, mode=mode), (x,))
    after = ns.plan_cache_stats()
    assert after[1] > before[1]  # the backward reused the forward's plans


def test_lgan_empty_and_degenerate_on_gpu(ops) -> None:
    x = torch.randn(6, 4, device=DEV)
    empty = torch.zeros(0, dtype=torch.long, device=DEV)
    upd, tn, nn = ops.lgan_relation_graph_step(-x.abs(), empty, empty, empty, empty, empty, empty, 3, 2)
    assert torch.equal(upd, -x.abs() + 0.0) and not tn.any() and not nn.any() and tn.shape == (3, 4)
    assert (torch.signbit(upd) == torch.signbit(-x.abs() + 0.0)).all()
    rpx, tn, _ = ops.lgan_pool_reduce(torch.zeros(0, 4, device=DEV), empty,
                                      torch.ones(5, dtype=torch.long, device=DEV),
                                      empty, empty, empty, empty, empty, empty, 0, 0)
    assert rpx.shape == (5, 4) and not rpx.any() and tn.shape == (0, 4)
    with pytest.raises(RuntimeError, match="out of bounds"):
        ops.lgan_relation_graph_step(x, torch.tensor([0, 6], device=DEV), torch.tensor([1, 2], device=DEV),
                                     empty, empty, empty, empty, 3, 0)
    with pytest.raises(RuntimeError, match="slot_to_relation_instance index out of bounds"):
        ops.lgan_pool_reduce(torch.ones(2, 4, device=DEV), torch.tensor([0, 0], device=DEV),
                             torch.zeros(0, dtype=torch.long, device=DEV),
                             empty, empty, empty, empty, empty, empty, 3, 0)
    with pytest.raises(RuntimeError, match="slot_to_relation_instance index out of bounds"):
        ops.lgan_pool_reduce_backward(x, torch.zeros(3, 4, device=DEV), torch.zeros(3, 4, device=DEV),
                                      torch.tensor([0, 6], device=DEV),
                                      torch.ones(6, dtype=torch.long, device=DEV),
                                      empty, empty, empty, empty, empty, empty, 6, 0)


@pytest.mark.parametrize("seed", range(8))
def test_lgan_random_shapes_match_oracle(ops, seed) -> None:
    """Random small shapes: D from 1 to 70 (odd widths take the scalar path),
    float32 / float64, int32 / int64 indices, empty edge sets, both modes."""

    rng = np.random.default_rng(100 + seed)
    K, ent, E = int(rng.integers(1, 300)), int(rng.integers(0, 120)), int(rng.integers(0, 700))
    D = int(rng.choice([1, 3, 4, 7, 16, 33, 64, 70]))
    dtype = np.float64 if seed % 3 == 0 else np.float32
    itype = np.int32 if seed % 2 else np.int64
    n = [int(rng.integers(0, 900)) if rng.random() > 0.15 else 0 for _ in range(3)]
    if ent == 0:
        n[1] = n[2] = 0
    edges = [rng.integers(0, K, n[0]), rng.integers(0, K, n[0]),
             rng.integers(0, K, n[1]), rng.integers(0, max(ent, 1), n[1]),
             rng.integers(0, K, n[2]), rng.integers(0, max(ent, 1), n[2])]
    edges = [e.astype(itype) for e in edges]
    slot = rng.standard_normal((E, D)).astype(dtype)
    s2r = rng.integers(0, K, E).astype(itype)
    arity = rng.integers(-1, 4, K)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    for mode in (0, 2):
        _log(f"lgan random seed {seed} mode {mode}: K={K} ent={ent} E={E} D={D} {dtype.__name__} {itype.__name__}")
        got = ops.lgan_pool_reduce(t(slot), t(s2r), t(arity), *map(t, edges), ent, mode)
        want = lgan_oracle.lgan_pool_reduce(slot, s2r, arity, *edges, ent, mode)
        for g, w in zip(got, want):
            np.testing.assert_allclose(g.cpu().numpy(), w, rtol=1e-5 if dtype == np.float32 else 1e-12,
                                       atol=1e-5 if dtype == np.float32 else 1e-12)
        gr = [rng.standard_normal(w.shape).astype(dtype) for w in want]
        grad = ops.lgan_pool_reduce_backward(*map(t, gr), t(s2r), t(arity), *map(t, edges), K, mode)
        want_g = lgan_oracle.lgan_pool_reduce_backward(*gr, s2r, arity, *edges, K, mode)
        np.testing.assert_allclose(grad.cpu().numpy(), want_g, rtol=1e-5 if dtype == np.float32 else 1e-12,
                                   atol=1e-5 if dtype == np.float32 else 1e-12)


@pytest.mark.parametrize("emb,skew", [(64, False), (6, False), (32, True)])
def test_divided_sum_equals_scaled_rows_then_sum(emb, skew) -> None:
    """relm_mp_plan_segment_sum_msgdiv (each gathered row divided by its count as
    it is loaded) equals the two-pass formulation it replaces - the rows divided
    by relm_mp_rows_scale, then the plain segment sum - bit for bit, with a base
    row added, over a skewed index set (hub chunks) and over uniform indices."""

    from relmo_amd import capi

    _log(f"divided sum emb={emb} skew={skew}")
    rng = np.random.default_rng(7 + emb)
    src_rows, tgt_rows, n = 3000, 2500, 60_000
    if skew:
        t = np.minimum(rng.pareto(0.6, n).astype(np.int64), tgt_rows - 1)
        s = np.minimum(rng.pareto(0.6, n).astype(np.int64), src_rows - 1)
    else:
        t = rng.integers(0, tgt_rows, n)
        s = rng.integers(0, src_rows, n)
    tt, st = torch.from_numpy(t).to(DEV), torch.from_numpy(s).to(DEV)
    grad = torch.from_numpy(rng.standard_normal((tgt_rows, emb)).astype(np.float32)).to(DEV)
    base = torch.from_numpy(rng.standard_normal((src_rows, emb)).astype(np.float32)).to(DEV)
    fwd = capi.csr_plan(tt, tgt_rows, st, src_rows)   # keyed by the table's rows: their counts
    rev = capi.csr_plan(st, src_rows, tt, tgt_rows)   # the transposed sum
    got = capi.plan_segment_sum_msgdiv(rev, grad, fwd, base)
    scaled = capi.rows_scale(grad, tgt_rows, emb, grad, div_kind=capi.DIV_SEGMENT, div_offsets=fwd.offsets)
    want = capi.plan_segment_sum_scaled(rev, scaled, 0, None, base)
    assert torch.equal(got, want)
    # float64 truth: within this module's 8 eps32 times the op on the magnitudes
    # for the uniform sets (a count off by one there moves a term by ~4%); the
    # skewed set sums ~2e4 messages into one row through 64-message sequential
    # slices, so its bound is 1e-4 of the magnitudes
    counts = np.maximum(np.bincount(t, minlength=tgt_rows), 1).astype(np.float64)
    g64, b64 = grad.double().cpu().numpy(), base.double().cpu().numpy()
    truth, mag = b64.copy(), np.abs(b64)
    np.add.at(truth, s, g64[t] / counts[t][:, None])
    np.add.at(mag, s, np.abs(g64[t]) / counts[t][:, None])
    tol = 1e-4 if skew else 8 * np.finfo(np.float32).eps
    assert np.all(np.abs(got.double().cpu().numpy() - truth) <= tol * mag)
