"""GPU tests of the fused FiLM step with Mish (torch.ops.relm_mp.film_mish and
its backward; C ABI relm_mp_film_mish*): against the same function in float64
through torch autograd, and bit for bit against torch's own fp32 ops."""

from __future__ import annotations

import os
import sys

import pytest
import torch

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


def _reference(s, gamma, beta, add, starts):
    """float64: mish(beta[k] + gamma[k] * (s + add[k])) per range, through autograd."""

    parts = []
    for k in range(len(starts) - 1):
        v = s[starts[k]:starts[k + 1]]
        t = v + add[k] if add is not None else v
        parts.append(torch.nn.functional.mish(beta[k] + gamma[k] * t))
    return torch.cat(parts)


@pytest.mark.parametrize("width,starts,with_add", [
    (398, [0, 1000, 1000, 5123, 6000], True),   # an empty range; 8-byte lanes
    (398, [0, 513], False),                     # one range, one block plus a row
    (7, [0, 3, 700, 1536, 1537], True),         # odd width: 4-byte lanes
    (600, [0, 2048, 4096], True),               # 300 column pairs: 3 row phases
    (2500, [0, 700, 701, 1500], True),          # more column pairs than threads: one phase, looped
])
def test_film_mish_against_float64(width, starts, with_add) -> None:
    from relmo_amd import capi

    _log(f"film_mish width={width} starts={starts} add={with_add}")
    g = torch.Generator(device=DEV).manual_seed(width + len(starts))
    k, rows = len(starts) - 1, starts[-1]
    s = 2.0 * torch.randn(rows, width, device=DEV, generator=g)
    gamma = torch.randn(k, width, device=DEV, generator=g)
    beta = torch.randn(k, width, device=DEV, generator=g)
    add = torch.randn(k, width, device=DEV, generator=g) if with_add else None
    dy = torch.randn(rows, width, device=DEV, generator=g)

    ops = torch.ops.relm_mp
    y = ops.film_mish(s, starts, gamma, beta, add)
    ds, dg, db = ops.film_mish_backward(dy, s, starts, gamma, beta, add)

    leaves = [t.double().requires_grad_(True) for t in (s, gamma, beta) + ((add,) if with_add else ())]
    y64 = _reference(leaves[0], leaves[1], leaves[2], leaves[3] if with_add else None, starts)
    grads = torch.autograd.grad(y64, leaves, dy.double())
    torch.testing.assert_close(y.double(), y64.detach(), rtol=2e-6, atol=2e-6)
    torch.testing.assert_close(ds.double(), grads[0], rtol=1e-5, atol=1e-5)
    # per-range column sums over up to thousands of rows: fp32 terms added in
    # fp64 (within each 512-row block, then over the blocks), rounded once
    torch.testing.assert_close(dg.double(), grads[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(db.double(), grads[2], rtol=1e-5, atol=1e-4)
    if with_add:
        torch.testing.assert_close((gamma * db).double(), grads[3], rtol=1e-5, atol=1e-4)

    # bit for bit what torch's own ops give in fp32 (addcmul, then Mish, per
    # range, and autograd through them): the kernel uses their formulation
    sl = s.clone().requires_grad_(True)
    parts = [torch.nn.functional.mish(torch.addcmul(beta[r], gamma[r], v + add[r] if with_add else v))
             for r, v in enumerate(torch.split(sl, [starts[r + 1] - starts[r] for r in range(k)]))]
    y32 = torch.cat(parts)
    (ds32,) = torch.autograd.grad(y32, sl, dy)
    assert torch.equal(y, y32.detach())
    assert torch.equal(ds, ds32)

    # the C ABI gives the same bits as the torch op
    assert torch.equal(capi.film_mish(s, starts, gamma, beta, add), y)
    ds2, partial = capi.film_mish_backward(dy, s, starts, gamma, beta, add)
    assert torch.equal(ds2, ds)
    b0 = 0
    for r in range(k):
        nb = -(-(starts[r + 1] - starts[r]) // 512)
        if nb:
            assert partial.dtype == torch.float64
            assert torch.equal(partial[b0:b0 + nb, 1].sum(0).float(), db[r])
        b0 += nb


@pytest.mark.parametrize("lo_bits,hi_bits,step", [
    (0x41000000, 0x7F800000, 97),    # [8, inf): the saturated side (mish(u) = u from u = 10 on)
    (0xC2A00000, 0xC3800000, 5),     # [-256, -80]: exp(u) denormal, then 0 (from u = -104 on)
    (0xC0000000, 0xC2A00000, 41),    # [-80, -2]
    (0x00000000, 0x41000000, 401),   # [0, 8)
])
def test_film_mish_bitwise_against_torch_over_float_ranges(lo_bits: int, hi_bits: int, step: int) -> None:
    """Mish and its gradient on sweeps of fp32 values (every step-th bit
    pattern of the range, with its ends and the infinities): the fused kernels
    give torch's own fp32 results bit for bit, including past the thresholds
    where they skip the transcendental calls."""

    ops = torch.ops.relm_mp
    bits = torch.arange(lo_bits, hi_bits, step, dtype=torch.int64, device=DEV)
    bits = torch.cat([bits, torch.tensor([lo_bits, hi_bits - 1], device=DEV)])
    u = bits.to(torch.int32).view(torch.float32)
    u = torch.cat([u, torch.tensor([float("inf"), -float("inf")], device=DEV)])
    n = u.numel() // 64 * 64
    u = u[:n].view(-1, 64).contiguous()
    one = torch.ones(1, 64, device=DEV)
    zero = torch.zeros(1, 64, device=DEV)
    dy = torch.randn(u.shape, device=DEV, generator=torch.Generator(device=DEV).manual_seed(7))
    y = ops.film_mish(u, [0, u.size(0)], one, zero, None)
    ds, _, _ = ops.film_mish_backward(dy, u, [0, u.size(0)], one, zero, None)
    x = u.clone().requires_grad_(True)
    y32 = torch.nn.functional.mish(torch.addcmul(zero[0], one[0], x))
    (ds32,) = torch.autograd.grad(y32, x, dy)
    same = (y == y32.detach()) | (torch.isnan(y) & torch.isnan(y32.detach()))
    assert bool(same.all()), u[~same][:8].tolist()
    same = (ds == ds32) | (torch.isnan(ds) & torch.isnan(ds32))
    assert bool(same.all()), u[~same][:8].tolist()


def test_film_mish_extremes_and_errors() -> None:
    """Large and very negative pre-activations (Mish is u and 0 there), and
    ranges that do not cover the rows."""

    ops = torch.ops.relm_mp
    u = torch.tensor([[-200.0, -30.0, -5.0, 0.0, 5.0, 19.0, 21.0, 300.0]], device=DEV)
    one = torch.ones(1, 8, device=DEV)
    y = ops.film_mish(u, [0, 1], one, torch.zeros(1, 8, device=DEV), None)
    want = torch.nn.functional.mish(u.double())
    torch.testing.assert_close(y.double(), want, rtol=2e-6, atol=1e-12)
    ds, _, _ = ops.film_mish_backward(torch.ones_like(u), u, [0, 1], one, torch.zeros(1, 8, device=DEV), None)
    x = u.double().requires_grad_(True)
    (gx,) = torch.autograd.grad(torch.nn.functional.mish(x).sum(), x)
    torch.testing.assert_close(ds.double(), gx, rtol=1e-5, atol=1e-7)
    with pytest.raises(RuntimeError, match="cover the rows"):
        ops.film_mish(u, [0, 2], one, one, None)
    with pytest.raises(RuntimeError, match="row ranges"):
        ops.film_mish(u, [0], one, one, None)


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_selective_recompute_matches_stored_activations(mode: int, monkeypatch) -> None:
    """The gathered central module with recomputation (the fused FiLM step and
    the Linear after it keep only the gathered sums; the Mish output is
    recomputed in the backward) gives the loss and gradients of the same
    module that keeps its activations."""

    from relmo_amd import consumers as C

    monkeypatch.setenv("RELM_MP_ENABLE", "1")
    batch = C.synthetic_c5(DEV, seed=11, num_graphs=64)
    results = []
    for recompute in (False, True):
        _log(f"central module mode={mode} recompute={recompute}: {batch.num_objects} objects")
        torch.manual_seed(0)
        m = C.CentralizedRelationalGNN(128, 4, batch.relations, mode, gather_first_linear=True,
                                       recompute_central=recompute).to(DEV)
        routing = m.routing(batch)
        loss = float(C.train_step(m, batch, routing))
        grads = {k: p.grad.detach().clone() for k, p in m.named_parameters() if p.grad is not None}
        results.append((loss, grads))
    (l0, g0), (l1, g1) = results
    assert l0 == l1
    assert g0.keys() == g1.keys()
    for k in g0:
        torch.testing.assert_close(g1[k], g0[k], rtol=1e-6, atol=1e-7, msg=lambda m, k=k: f"{k}: {m}")


def _node_names(fn, seen=None) -> set[str]:
    seen = set() if seen is None else seen
    if fn is None or id(fn) in seen:
        return set()
    seen.add(id(fn))
    names = {type(fn).__name__}
    for nxt, _ in fn.next_functions:
        names |= _node_names(nxt, seen)
    return names


def _max_err(a, b) -> float:
    return float((a.double() - b).abs().max())


@pytest.mark.parametrize("width,rows", [(32, 5000), (64, 4099), (96, 20000), (398, 1537)])
def test_linear_mish_against_float64(width: int, rows: int) -> None:
    """MishMLP (Linear + Mish pairs as one node on the fused kernel, the bias
    gradient from its backward) against the same layers in float64 through
    torch; its error at most a few times that of the same layers in float32
    through torch."""

    import copy

    from torch import nn

    from relmo_amd import consumers as C

    _log(f"linear+mish width={width} rows={rows}")
    torch.manual_seed(width)
    mlp = C.MishMLP(C.Linear(width, width), nn.Mish(), C.Linear(width, width), nn.Mish(),
                    C.Linear(width, width)).to(DEV)
    x = torch.randn(rows, width, device=DEV, requires_grad=True)
    g = torch.randn(rows, width, device=DEV)
    y = mlp(x)
    assert "_LinearMishBackward" in _node_names(y.grad_fn)
    got = [y, *torch.autograd.grad(y, [x, *mlp.parameters()], g)]
    y32 = nn.Sequential.forward(mlp, x)
    assert "_LinearMishBackward" not in _node_names(y32.grad_fn)
    plain = [y32, *torch.autograd.grad(y32, [x, *mlp.parameters()], g)]
    m64 = copy.deepcopy(mlp).double()
    x64 = x.detach().double().requires_grad_(True)
    y64 = nn.Sequential.forward(m64, x64)
    truth = [y64, *torch.autograd.grad(y64, [x64, *m64.parameters()], g.double())]
    names = ["y", "dx"] + [n for n, _ in mlp.named_parameters()]
    for name, a, b, t in zip(names, got, plain, truth):
        e_fused, e_plain = _max_err(a, t), _max_err(b, t)
        scale = float(t.abs().max())
        _log(f"  {name}: fused {e_fused:.3g} torch {e_plain:.3g} (scale {scale:.3g})")
        assert e_fused <= 8 * e_plain + 32 * 1.2e-7 * scale, name



@pytest.mark.parametrize("m,k,n,slice_cols", [(204800, 64, 64, False), (20000, 96, 96, False),
                                              (5000, 128, 32, False), (3001, 64, 128, True),
                                              (0, 64, 64, False), (7, 0, 5, False)])
def test_mm_nt_against_float64(m: int, k: int, n: int, slice_cols: bool) -> None:
    """torch.ops.relm_mp.mm_nt (a @ b^T through hipBLAS on torch's handle):
    against float64, the same bits on a second call, and a column slice of a
    wider matrix read in place."""

    _log(f"mm_nt m={m} k={k} n={n} slice={slice_cols}")
    g = torch.Generator(device=DEV).manual_seed(m + k + n)
    if slice_cols:
        wide = torch.randn(m, k + 14, device=DEV, generator=g)
        a = wide[:, 14:]
        assert a.stride(0) == k + 14
    else:
        a = torch.randn(m, k, device=DEV, generator=g)
    b = torch.randn(n, k, device=DEV, generator=g)
    out = torch.ops.relm_mp.mm_nt(a, b)
    assert out.shape == (m, n) and out.is_contiguous()
    want = a.double() @ b.double().t()
    # fp32 products and sums over k terms of |a||b| ~ 1
    torch.testing.assert_close(out.double(), want, rtol=0, atol=4 * 1.2e-7 * max(k, 1) * 4)
    assert torch.equal(torch.ops.relm_mp.mm_nt(a, b), out)
    with pytest.raises(RuntimeError, match="mm_nt"):
        torch.ops.relm_mp.mm_nt(a, b[:, :-1] if k > 0 else torch.zeros(n, 1, device=DEV))
