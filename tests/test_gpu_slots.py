"""GPU parity of the fanout written straight into argument slots (the central
input assembly of relmo/models/hetero_mp/fused.py:299-375): the grouped-row
entry points of the C ABI (relm_mp_plan_gather_last_grouped,
relm_mp_plan_segment_sum_grouped), the torch ops fanout_scatter_into /
fanout_scatter_backward_from and the autograd facade mp.fanout_concat, against
the numpy oracle (oracle.fanout_into_slots / fanout_backward_from_slots) and
against the dense ops on the same indices.  Gathers are bit-exact; the
backward sums are bit-exact against the dense backward (same plan, same
order) and against the oracle where no object collects more than 64 slots."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import oracle

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


def _case(seed: int, lines: int, slots: int, d: int, x_rows: int, n: int, dtype=torch.float32,
          zipf: bool = False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(x_rows, d, dtype=dtype, generator=g)
    if zipf:
        rng = np.random.default_rng(seed)
        src = torch.from_numpy(np.minimum(rng.zipf(1.3, n) - 1, x_rows - 1).astype(np.int64))
    else:
        src = torch.randint(0, x_rows, (n,), generator=g)
    dst = torch.randint(0, lines * slots, (n,), generator=g)
    return x, src, dst


# (lines, slots, D, col_offset, extra columns): 16-byte aligned rows, 8-byte
# aligned ones (the C5 layout: 14 context columns, 3 slots of 128) and
# unaligned ones (odd offsets or strides: 4 bytes per lane)
LAYOUTS = [(1000, 3, 32, 12, 4), (777, 2, 64, 11, 3), (500, 1, 128, 0, 0), (3000, 3, 20, 7, 1),
           (64, 4, 5, 3, 2), (2000, 3, 128, 14, 0), (1500, 2, 32, 6, 2),
           # rows wider than one row group covers (two column slices)
           (200, 2, 300, 6, 2), (150, 3, 520, 0, 0)]


@pytest.mark.parametrize("lines,slots,d,col,extra", LAYOUTS)
@pytest.mark.parametrize("kind", ["inverse", "csr"])
def test_grouped_gather_c_abi(lines, slots, d, col, extra, kind) -> None:
    from relmo_amd import capi

    _log(f"grouped gather {kind} lines={lines} slots={slots} D={d} col={col}")
    x, src, dst = _case(lines + d, lines, slots, d, 300, lines * slots // 2)
    width = col + slots * d + extra
    out = torch.randn(lines, width, generator=torch.Generator().manual_seed(1))
    want = oracle.fanout_into_slots(x.numpy(), src.numpy(), dst.numpy(), out.numpy(), col, slots)
    xg, sg, dg, og = x.to(DEV), src.to(DEV), dst.to(DEV), out.to(DEV)
    if kind == "inverse":
        bp = capi.inv_plan(dg, lines * slots, sg, 300)
        capi.plan_gather_last_grouped(bp, xg, og, col, slots, gathers=sg)
    else:
        bp = capi.csr_plan(dg, lines * slots, sg, 300)
        capi.plan_gather_last_grouped(bp, xg, og, col, slots)
    torch.cuda.synchronize()
    assert np.array_equal(og.cpu().numpy(), want)


@pytest.mark.parametrize("lines,slots,d,col,extra", [(400, 3, 32, 6, 2), (300, 2, 7, 1, 0), (100, 2, 200, 4, 0)])
def test_grouped_layouts_in_float64(lines, slots, d, col, extra) -> None:
    from relmo_amd import capi

    _log(f"grouped float64 lines={lines} slots={slots} D={d} col={col}")
    x, src, dst = _case(lines + 3 * d, lines, slots, d, 250, lines * slots, dtype=torch.float64)
    width = col + slots * d + extra
    out = torch.randn(lines, width, dtype=torch.float64, generator=torch.Generator().manual_seed(4))
    want = oracle.fanout_into_slots(x.numpy(), src.numpy(), dst.numpy(), out.numpy(), col, slots)
    xg, sg, dg, og = x.to(DEV), src.to(DEV), dst.to(DEV), out.to(DEV)
    bp = capi.inv_plan(dg, lines * slots, sg, 250)
    capi.plan_gather_last_grouped(bp, xg, og, col, slots, gathers=sg)
    csr = capi.csr_plan(sg, 250, dg, lines * slots)
    got = capi.plan_segment_sum_grouped(csr, og, col, slots, d)
    torch.cuda.synchronize()
    assert np.array_equal(og.cpu().numpy(), want)
    ref = oracle.fanout_backward_from_slots(want, src.numpy(), dst.numpy(), 250, col, slots, d)
    counts = np.bincount(src.numpy(), minlength=250)
    short = counts <= 64
    assert np.array_equal(got.cpu().numpy()[short], ref[short])
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("lines,slots,d,col,extra", LAYOUTS)
def test_grouped_sum_matches_dense_and_oracle(lines, slots, d, col, extra) -> None:
    from relmo_amd import capi

    _log(f"grouped sum lines={lines} slots={slots} D={d} col={col}")
    x_rows = 2000
    n = lines * slots
    _, src, dst = _case(7 + d, lines, slots, d, x_rows, n, zipf=True)
    width = col + slots * d + extra
    grad = torch.randn(lines, width, generator=torch.Generator().manual_seed(2))
    gg, sg, dg = grad.to(DEV), src.to(DEV), dst.to(DEV)
    bp = capi.csr_plan(sg, x_rows, dg, n)
    got = capi.plan_segment_sum_grouped(bp, gg, col, slots, d)
    dense = gg[:, col:col + slots * d].contiguous().view(n, d)
    ref = capi.plan_segment_reduce(bp, dense, 0)
    torch.cuda.synchronize()
    counts = np.bincount(src.numpy(), minlength=x_rows)
    short = counts <= 64
    # the same row geometry (16-byte aligned slot rows) folds hub chunks in the
    # same order as the dense layout; otherwise only segments of at most 64
    # messages (summed in edge order either way) are bit-identical
    if col % 4 == 0 and width % 4 == 0 and d % 4 == 0:
        assert torch.equal(got, ref)
    else:
        assert np.array_equal(got.cpu().numpy()[short], ref.cpu().numpy()[short])
    want = oracle.fanout_backward_from_slots(grad.numpy(), src.numpy(), dst.numpy(), x_rows, col,
                                             slots, d)
    assert np.array_equal(got.cpu().numpy()[short], want[short])
    truth, absum = oracle.segment_sum_truth(
        np.ascontiguousarray(grad.numpy()[:, col:col + slots * d]).reshape(n, d).astype(np.float64),
        dst.numpy(), src.numpy(), x_rows)
    assert np.all(np.abs(got.cpu().numpy() - truth) <= 8 * np.finfo(np.float32).eps * absum + 1e-30)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_torch_ops_match_composition(ops, dtype) -> None:
    _log(f"fanout_scatter_into / backward_from {dtype}")
    lines, slots, d, col = 5000, 3, 32, 14
    x, src, dst = _case(3, lines, slots, d, 4000, 12000, dtype)
    xg, sg, dg = x.to(DEV), src.to(DEV), dst.to(DEV)
    big = torch.randn(lines, col + slots * d + 9, dtype=dtype, device=DEV)
    keep = big.clone()
    version = big._version
    ops.fanout_scatter_into(xg, sg, dg, big, col, slots)
    assert big._version > version  # an in-place change for autograd's checks
    rows = ops.fanout_scatter(xg, sg, dg, lines * slots)
    assert torch.equal(big[:, col:col + slots * d], rows.view(lines, slots * d))
    assert torch.equal(big[:, :col], keep[:, :col]) and torch.equal(big[:, col + slots * d:],
                                                                    keep[:, col + slots * d:])
    grad = torch.randn(lines, col + slots * d + 9, dtype=dtype, device=DEV)
    got = ops.fanout_scatter_backward_from(grad, sg, dg, 4000, col, slots, d)
    ref = ops.fanout_scatter_backward(grad[:, col:col + slots * d].reshape(lines * slots, d), sg, dg, 4000)
    assert torch.equal(got, ref)
    # a column slice as the destination (lines 3 apart in a wider matrix), a
    # transposed gradient (no unit column stride: read through a copy)
    wide = torch.zeros(lines, 2 * (col + slots * d), dtype=dtype, device=DEV)
    view = wide[:, 5:5 + col + slots * d]
    ops.fanout_scatter_into(xg, sg, dg, view, col, slots)
    assert torch.equal(view[:, col:col + slots * d], rows.view(lines, slots * d))
    assert torch.count_nonzero(wide[:, :5 + col]) == 0
    gt = grad.t().contiguous().t()
    assert torch.equal(ops.fanout_scatter_backward_from(gt, sg, dg, 4000, col, slots, d), ref)
    torch.cuda.synchronize()


def test_empty_and_error_cases(ops) -> None:
    x = torch.randn(10, 8, device=DEV)
    e = torch.zeros(0, dtype=torch.int64, device=DEV)
    out = torch.full((4, 3 + 2 * 8), 7.0, device=DEV)
    ops.fanout_scatter_into(x, e, e, out, 3, 2)
    assert torch.count_nonzero(out[:, 3:]) == 0 and bool((out[:, :3] == 7.0).all())
    g = ops.fanout_scatter_backward_from(out, e, e, 10, 3, 2, 8)
    assert g.shape == (10, 8) and torch.count_nonzero(g) == 0
    bad = torch.tensor([0, 8], device=DEV)
    with pytest.raises(RuntimeError, match=r"flat_dst index out of bounds: 8 not in \[0, 8\)"):
        ops.fanout_scatter_into(x, torch.tensor([0, 1], device=DEV), bad, out, 3, 2)
    with pytest.raises(RuntimeError, match="exceed the"):
        ops.fanout_scatter_into(x, e, e, out, 4, 2)


def test_fanout_concat_autograd_on_gpu(mp_env) -> None:
    from relmo_amd import mp

    _log("fanout_concat autograd")
    gen = torch.Generator().manual_seed(21)
    prefix = torch.randn(300, 5, dtype=torch.float64, generator=gen)
    x = torch.randn(80, 4, dtype=torch.float64, generator=gen)
    src = torch.randint(0, 80, (700,), generator=gen)
    dst = torch.randperm(900, generator=gen)[:700]  # distinct slots: the op's backward is the true one
    p_g = prefix.to(DEV).requires_grad_()
    x_g = x.to(DEV).requires_grad_()
    out = mp.fanout_concat(p_g, x_g, src.to(DEV), dst.to(DEV), 3)
    w = torch.randn(out.shape, dtype=torch.float64, generator=gen)
    (out * w.to(DEV)).sum().backward()
    p_c = prefix.clone().requires_grad_()
    x_c = x.clone().requires_grad_()
    rows = torch.zeros(900, 4, dtype=torch.float64).index_copy(0, dst, x_c[src])
    ref = torch.cat([p_c, rows.view(300, 12)], 1)
    (ref * w).sum().backward()
    assert torch.equal(out.detach().cpu(), ref.detach())
    torch.testing.assert_close(p_g.grad.cpu(), p_c.grad, rtol=0, atol=0)
    torch.testing.assert_close(x_g.grad.cpu(), x_c.grad, rtol=1e-12, atol=1e-12)


def test_grouped_entry_points_reject_bad_layouts() -> None:
    import ctypes

    from relmo_amd import capi

    x = torch.randn(10, 8, device=DEV)
    dst = torch.arange(12, device=DEV)
    src = torch.randint(0, 10, (12,), device=DEV)
    out = torch.zeros(4, 3 * 8, device=DEV)
    inv = capi.inv_plan(dst, 12, src, 10)
    lib = capi.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def gather(group, stride):
        return lib.relm_mp_plan_gather_last_grouped(capi.F32, ctypes.byref(inv.plan), src.data_ptr(),
                                                     x.data_ptr(), 8, group, stride, out.data_ptr(), stream)

    assert gather(0, 24) == capi.ERR_INVALID_ARGUMENT and "group" in capi.last_error()
    assert gather(3, 23) == capi.ERR_INVALID_ARGUMENT and "group_stride" in capi.last_error()
    assert gather(5, 40) == capi.ERR_INVALID_ARGUMENT and "multiple" in capi.last_error()
    assert gather(3, 24) == capi.OK
    csr = capi.csr_plan(src, 10, dst, 12)
    scratch = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    g = torch.zeros(10, 8, device=DEV)
    rc = lib.relm_mp_plan_segment_sum_grouped(capi.F32, ctypes.byref(csr.plan), out.data_ptr(), 10, 8, 3, 24,
                                              g.data_ptr(), scratch.data_ptr(), scratch.numel(), stream)
    assert rc == capi.ERR_INVALID_ARGUMENT and "multiple" in capi.last_error()
    rc = lib.relm_mp_plan_segment_sum_grouped(capi.F32, ctypes.byref(csr.plan), out.data_ptr(), 9, 8, 3, 24,
                                              g.data_ptr(), scratch.data_ptr(), scratch.numel(), stream)
    assert rc == capi.ERR_INVALID_ARGUMENT and "table_rows" in capi.last_error()
    torch.cuda.synchronize()
    want = oracle.fanout_into_slots(x.cpu().numpy(), src.cpu().numpy(), dst.cpu().numpy(),
                                    np.zeros((4, 24), np.float32), 0, 3)
    assert np.array_equal(out.cpu().numpy(), want)
