"""GPU parity of the pack ops (fanout/fanin_pack_multi, fanout/fanin_pack_from_edges):
the HIP index-packing kernel through the C ABI (relmo_amd.capi) and through the
torch binding, against the reference's golden fixtures and the numpy oracle
(oracle/pack.py).  Index outputs are integer work: bit-exact."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import pack as pack_oracle
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


def _wrap(a: np.ndarray, mul: int, add: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        return a.astype(np.int64) * np.int64(mul) + np.int64(add)


def test_pack_ops_reproduce_golden_on_gpu(ops, pack_golden) -> None:
    cases, arrays = pack_golden
    for case in cases:
        _log(f"pack golden case {case['name']}")
        args = pack_args(case, arrays, DEV)
        fn = getattr(ops, case["op"])
        if "error" in case:
            with pytest.raises((RuntimeError, ValueError)) as info:
                fn(*args)
            assert str(info.value).splitlines()[0] == case["error"], case["name"]
            continue
        got = fn(*args)
        torch.cuda.synchronize()
        for g, name in zip(got, case["expected"]):
            assert g.is_cuda, case["name"]
            want = arrays[name]
            g = g.detach().cpu().numpy()
            assert g.dtype == want.dtype and g.shape == want.shape, case["name"]
            assert np.array_equal(g, want), case["name"]


@pytest.mark.parametrize("write_b", [True, False])
def test_pack_index_c_abi_matches_numpy(write_b) -> None:
    from relmo_amd import capi

    rng = np.random.default_rng(21 + write_b)
    sizes = [0, 1, 255, 1023, 1024, 1025, 4097, 100_003] + [int(v) for v in rng.integers(0, 3000, 14)]
    parts, host = [], []
    for n in sizes:  # 22 parts: two launches of at most 16
        a = rng.integers(-(2**40), 2**40, n)
        b = rng.integers(-(2**62), 2**62, n)
        coef = [int(v) for v in rng.integers(-(2**31), 2**31, 4)]
        parts.append((torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV), *coef))
        host.append((a, b, *coef))
    _log(f"pack_index C ABI: {len(parts)} parts, {sum(sizes)} pairs, write_b={write_b}")
    out_a, out_b = capi.pack_index(parts, write_b=write_b)
    torch.cuda.synchronize()
    want_a = np.concatenate([_wrap(a, am, aa) for a, _, am, aa, _, _ in host])
    assert np.array_equal(out_a.cpu().numpy(), want_a)
    if write_b:
        want_b = np.concatenate([_wrap(b, bm, ba) for _, b, _, _, bm, ba in host])
        assert np.array_equal(out_b.cpu().numpy(), want_b)
    else:
        assert out_b is None


def test_pack_index_c_abi_rejects_bad_parts() -> None:
    import ctypes

    from relmo_amd import capi

    part = capi.IndexPart(None, None, 5, 1, 0, 1, 0)
    out = torch.empty(5, dtype=torch.int64, device=DEV)
    rc = capi.lib().relm_mp_pack_index(ctypes.byref(part), 1, out.data_ptr(), out.data_ptr(), None)
    assert rc == capi.ERR_INVALID_ARGUMENT and "bad index part" in capi.last_error()
    rc = capi.lib().relm_mp_pack_index(None, -1, out.data_ptr(), None, None)
    assert rc == capi.ERR_INVALID_ARGUMENT


def test_pack_from_edges_large_parts_match_oracle(ops) -> None:
    """Edge lists of the size of one relation batch (millions of edges per part)."""

    rng = np.random.default_rng(23)
    rows = [700_000, 300_000, 1_000_000]
    xs = [torch.empty((r, 4), device=DEV) for r in rows]
    lens = [3_000_001, 1, 2_500_000, 0, 1_200_007]
    ids = [2, 0, 1, 0, 2]
    arity, pos, slot = [3, 1, 2, 4, 5], [2, 0, 1, 3, 4], [0, 9_000_003, 9_000_004, 14_000_004, 14_000_004]
    src = [rng.integers(0, rows[p], n) for p, n in zip(ids, lens)]
    dst = [rng.integers(0, 3_000_001, n) for n in lens]
    src_t = [torch.from_numpy(s).to(DEV) for s in src]
    dst_t = [torch.from_numpy(d).to(DEV) for d in dst]
    xs_np = [np.zeros((r, 0), np.float32) for r in rows]  # the oracle needs only the row counts
    _log("pack large: fanout_pack_from_edges 5 parts, 6.7M edges")
    _, s_out, d_out = ops.fanout_pack_from_edges(xs, src_t, dst_t, ids, arity, pos, slot)
    _, s_want, d_want = pack_oracle.fanout_pack_from_edges(xs_np, src, dst, ids, arity, pos, slot)
    assert np.array_equal(s_out.cpu().numpy(), s_want)
    assert np.array_equal(d_out.cpu().numpy(), d_want)
    for mode in (0, 1):
        _log(f"pack large: fanin_pack_from_edges mode {mode}")
        _, f_out, g_out = ops.fanin_pack_from_edges(xs, src_t, dst_t, ids, arity, pos, mode)
        _, f_want, g_want = pack_oracle.fanin_pack_from_edges(xs_np, src, dst, ids, arity, pos, mode)
        assert np.array_equal(f_out.cpu().numpy(), f_want)
        assert np.array_equal(g_out.cpu().numpy(), g_want)


def test_pack_single_part_aliasing_on_gpu(ops) -> None:
    x = torch.randn(4, 3, device=DEV)
    src = torch.tensor([0, 2, 3], device=DEV)
    dst = torch.tensor([5, 1, 0], device=DEV)
    for op in (ops.fanout_pack_multi, ops.fanin_pack_multi):
        v, a, b = op([x], [src], [dst])
        assert v.data_ptr() == x.data_ptr() and b.data_ptr() == dst.data_ptr()
        assert a.data_ptr() != src.data_ptr() and torch.equal(a, src)
    _, a, b = ops.fanout_pack_from_edges([x], [src], [dst], [0], [2], [1], [3])
    assert torch.equal(a, src) and torch.equal(b, 3 + dst * 2 + 1)
    _, a, b = ops.fanin_pack_from_edges([x], [src], [dst], [0], [2], [1], 0)
    assert b.data_ptr() == dst.data_ptr() and torch.equal(a, src * 2 + 1)


def test_pack_strided_index_views_on_gpu(ops) -> None:
    base = torch.arange(40, device=DEV).view(20, 2)
    src, dst = base[:, 0], base[:, 1]
    xs = [torch.randn(50, 2, device=DEV), torch.randn(5, 2, device=DEV)]
    _, a, b = ops.fanout_pack_from_edges(xs, [src, dst], [dst, src], [1, 0], [3, 2], [1, 0], [7, 9])
    assert torch.equal(a, torch.cat([src + 50, dst]))
    assert torch.equal(b, torch.cat([7 + dst * 3 + 1, 9 + src * 2]))


@pytest.mark.parametrize("mode", [0, 1])
def test_pack_then_reduce_gradients_on_gpu(mode) -> None:
    """The reference's pack -> fanout / fanin -> backward tests on the GPU
    (tests/python/test_mp_ops.py:353-600), checked against the same chain on
    the CPU lane."""

    from relmo_amd import mp

    torch.manual_seed(5)
    xs_cpu = [torch.randn(5, 3, dtype=torch.float64), torch.randn(4, 3, dtype=torch.float64)]
    src = [torch.tensor([0, 2, 4]), torch.tensor([1, 3]), torch.tensor([2, 0])]
    dst = [torch.tensor([1, 0, 2]), torch.tensor([3, 1]), torch.tensor([0, 2])]
    meta = ([0, 1, 0], [2, 3, 2], [0, 1, 1], [0, 8, 0])
    grads = []
    for dev in ("cpu", DEV):
        xs = [x.detach().to(dev).requires_grad_(True) for x in xs_cpu]
        x_cat, s, d = mp.fanout_pack_from_edges(xs, [t.to(dev) for t in src],
                                                [t.to(dev) for t in dst], *meta)
        out = mp.fanout_scatter(x_cat, s, d, 20)
        rel_cat, fs, fd = mp.fanin_pack_from_edges(
            [out[:10], out[10:]], [torch.tensor([0, 2, 1], device=dev), torch.tensor([1, 2], device=dev)],
            [torch.tensor([1, 0, 2], device=dev), torch.tensor([2, 1], device=dev)],
            [0, 1], [2, 3] if mode == 0 else [1, 1], [1, 2] if mode == 0 else [0, 0], mode)
        red = mp.fanin_reduce(rel_cat, fs, fd, 3, 0)
        red.square().sum().backward()
        grads.append([x.grad.cpu() for x in xs])
    for g_cpu, g_gpu in zip(*grads):
        assert torch.equal(g_cpu, g_gpu)


@pytest.mark.parametrize("seed", range(6))
def test_pack_random_layouts_match_oracle(ops, seed) -> None:
    rng = np.random.default_rng(200 + seed)
    n_values, n_parts = int(rng.integers(1, 6)), int(rng.integers(1, 40))
    rows = [int(r) for r in rng.integers(1, 5000, n_values)]
    xs = [torch.zeros((r, 2), device=DEV) for r in rows]
    xs_np = [np.zeros((r, 0), np.float32) for r in rows]
    lens = [int(v) if rng.random() > 0.2 else 0 for v in rng.integers(0, 20000, n_parts)]
    ids = [int(v) for v in rng.integers(0, n_values, n_parts)]
    arity = [int(v) for v in rng.integers(1, 6, n_parts)]
    pos = [int(rng.integers(0, a)) for a in arity]
    slot = [int(v) for v in rng.integers(-(2**40), 2**40, n_parts)]
    src = [rng.integers(-(2**50), 2**50, n) for n in lens]
    dst = [rng.integers(-(2**50), 2**50, n) for n in lens]
    st, dt = [torch.from_numpy(a).to(DEV) for a in src], [torch.from_numpy(a).to(DEV) for a in dst]
    _log(f"pack random seed {seed}: {n_parts} parts, {sum(lens)} pairs")
    got = ops.fanout_pack_from_edges(xs, st, dt, ids, arity, pos, slot)
    want = pack_oracle.fanout_pack_from_edges(xs_np, src, dst, ids, arity, pos, slot)
    for g, w in zip(got[1:], want[1:]):
        assert np.array_equal(g.cpu().numpy(), w)
    for mode in (0, 1):
        got = ops.fanin_pack_from_edges(xs, st, dt, ids, arity, pos, mode)
        want = pack_oracle.fanin_pack_from_edges(xs_np, src, dst, ids, arity, pos, mode)
        for g, w in zip(got[1:], want[1:]):
            assert np.array_equal(g.cpu().numpy(), w)
    k = min(n_values, n_parts)
    for op, fn in ((ops.fanout_pack_multi, pack_oracle.fanout_pack_multi),
                   (ops.fanin_pack_multi, pack_oracle.fanin_pack_multi)):
        got = op(xs[:k], st[:k], dt[:k])
        want = fn(xs_np[:k], src[:k], dst[:k])
        for g, w in zip(got[1:], want[1:]):
            assert np.array_equal(g.cpu().numpy(), w)
