"""GPU parity of the HIP path against the oracle and the reference's golden
fixtures.  Every test calls the kernels through the C ABI (relmo_amd.capi) or
through the torch binding, never through a CPU path.

Bars: fanout copies and sums over segments of at most 64 messages are
bit-exact (the kernels add in edge order like the reference's CPU loop);
longer segments are compared with the float64 truth within
4 * eps32 * sum|terms|; logsumexp within rtol 1e-4 (exp/log differ by ulps).
"""

from __future__ import annotations

import hashlib
import json
import os
import re
import sys

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.conftest import GOLDEN, REPO

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS32 = float(np.finfo(np.float32).eps)


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    os.environ["RELM_MP_FALLBACK"] = "error"
    from relmo_amd import capi, mp

    assert mp.available(), "relm_mp_ops.so failed to load"
    capi.lib()
    yield


def _t(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _np(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _is_lse(case: dict) -> bool:
    return case["op"] == "fanin_reduce_logsumexp_backward" or (
        case["op"] == "fanin_reduce" and case["ints"][1] == 1
    )


def _assert_lse_close(got: np.ndarray, want: np.ndarray, name: str) -> None:
    assert np.array_equal(np.isnan(got), np.isnan(want)), name
    assert np.array_equal(np.isneginf(got), np.isneginf(want)), name
    assert np.array_equal(np.isposinf(got), np.isposinf(want)), name
    fin = np.isfinite(want)
    np.testing.assert_allclose(got[fin], want[fin], rtol=1e-4, atol=1e-6, err_msg=name)


# (table, read index, write index) positions in each summing op's arguments
_SUM_OPS = {
    "fanout_scatter_backward": (0, 2, 1),
    "fanin_reduce": (0, 1, 2),
    "fanin_reduce_sum_backward": (0, 2, 1),
}


def _assert_sum_parity(op: str, args: list, got: np.ndarray, want: np.ndarray, name: str) -> None:
    """Rows with at most 64 messages: bit-exact.  Longer (hub) rows: within
    4 * eps32 * sum|terms| of the float64 truth, a bound the reference's own
    sequential sum also meets."""

    t, r, w = _SUM_OPS[op]
    table, read, write = args[t], args[r], args[w]
    deg = np.bincount(write, minlength=got.shape[0])
    short = deg <= 64
    assert np.array_equal(got[short], want[short], equal_nan=True), name
    if (~short).any():
        truth, absum = oracle.segment_sum_truth(table, read, write, got.shape[0])
        bound = 4 * EPS32 * absum[~short] + 1e-30
        assert np.all(np.abs(got[~short] - truth[~short]) <= bound), name
        assert np.all(np.abs(want[~short] - truth[~short]) <= bound), name


def test_product_libraries_are_the_in_tree_builds() -> None:
    from relmo_amd import capi, mp_runtime

    lib = mp_runtime.loaded_library()
    assert lib is not None and lib.parent == capi.LIB_PATH.parent
    maps = open("/proc/self/maps").read()
    assert "relmo_amd/relm_mp_ops.so" in maps and "relmo_amd/librelm_mp_hip.so" in maps
    assert len({line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}) == 1


@pytest.mark.parametrize("via", ["capi", "torch"])
def test_golden_cases(golden, via: str) -> None:
    from relmo_amd import capi

    ns = torch.ops.relm_mp
    fns = {
        "capi": {
            "fanout_scatter": capi.fanout_scatter,
            "fanout_scatter_backward": capi.fanout_scatter_backward,
            "fanin_reduce": capi.fanin_reduce,
            "fanin_reduce_sum_backward": capi.fanin_reduce_sum_backward,
            "fanin_reduce_logsumexp_backward": capi.fanin_reduce_logsumexp_backward,
        },
        "torch": {op: getattr(ns, op) for op in (
            "fanout_scatter", "fanout_scatter_backward", "fanin_reduce",
            "fanin_reduce_sum_backward", "fanin_reduce_logsumexp_backward")},
    }[via]
    cases, arrays = golden
    for case in cases:
        _log(f"golden[{via}] {case['name']}")
        args = [_t(arrays[n]) for n in case["tensors"]] + list(case["ints"])
        if "error" in case:
            if via == "capi" and _is_lse(case):
                # the C ABI reports every bad index with the loop message; the
                # torch ops restate the ATen errors of the reference's
                # logsumexp sequences
                with pytest.raises(RuntimeError, match="index out of bounds"):
                    fns[case["op"]](*args)
                continue
            with pytest.raises((RuntimeError, ValueError, IndexError)) as info:
                fns[case["op"]](*args)
                torch.cuda.synchronize()
            assert str(info.value).splitlines()[0] == case["error"], case["name"]
            assert (case.get("error_type") == "IndexError") == isinstance(info.value, IndexError), case["name"]
            continue
        got = _np(fns[case["op"]](*args))
        want = arrays[case["expected"]]
        assert got.shape == want.shape and got.dtype == want.dtype, case["name"]
        if _is_lse(case):
            _assert_lse_close(got, want, case["name"])
        elif case["op"] in _SUM_OPS and not (case["op"] == "fanin_reduce" and case["ints"][1] != 0):
            np_args = [arrays[n] for n in case["tensors"]]
            _assert_sum_parity(case["op"], np_args, got, want, case["name"])
        else:
            assert np.array_equal(got, want, equal_nan=True), case["name"]


def test_c1_outputs_match_reference_digests() -> None:
    from relmo_amd import capi
    from tests.golden.c1_config import c1_inputs

    a = {k: _t(v) for k, v in c1_inputs().items()}
    digests = json.loads((GOLDEN / "c1_digests.json").read_text())
    outs = {
        "fanout_scatter": capi.fanout_scatter(a["x"], a["src"], a["flat_dst"], a["src"].numel()),
        "fanout_scatter_backward": capi.fanout_scatter_backward(a["grad_slots"], a["src"], a["flat_dst"], a["x"].size(0)),
        "fanin_reduce": capi.fanin_reduce(a["rel"], a["flat_src"], a["dst"], a["x"].size(0), 0),
        "fanin_reduce_sum_backward": capi.fanin_reduce_sum_backward(a["grad_obj"], a["flat_src"], a["dst"], a["rel"].size(0)),
    }
    for op, out in outs.items():
        _log(f"C1 {op}")
        assert hashlib.sha256(_np(out).tobytes()).hexdigest() == digests[op], op


@pytest.mark.parametrize(
    "num_keys,num_edges,skew",
    [(1, 1000, False), (2, 5000, False), (300, 1, False), (4096, 98304, False),
     (50_000, 400_000, True), ((1 << 20) + 3, 300_000, False), (70_000, 4096 * 3 + 17, True),
     # three sort passes; several tiles per sort chunk (more tiles than resident workgroups)
     ((1 << 23) + 1, 200_000, False), (1 << 20, 5_000_003, True), ((1 << 21) - 7, 4_000_000, False),
     # 15 to 20-bit keys over 2^20 edges and more, a partial last tile of 5 keys
     (1 << 15, 2_000_000, False), ((1 << 18) + 5, 1 << 20, True), (1 << 20, 16_384 * 70 + 5, False)],
)
def test_csr_plan_is_the_stable_counting_order(num_keys: int, num_edges: int, skew: bool) -> None:
    from relmo_amd import capi

    _log(f"csr plan keys={num_keys} edges={num_edges} skew={skew}")
    rng = np.random.default_rng(num_keys + num_edges)
    if skew:
        keys = np.minimum((rng.pareto(0.6, num_edges)).astype(np.int64), num_keys - 1)
    else:
        keys = rng.integers(0, num_keys, num_edges)
    bp = capi.csr_plan(_t(keys), num_keys, None, num_edges)
    offsets, perm = oracle.csr_build(keys, num_keys)
    assert np.array_equal(_np(bp.offsets), offsets)
    assert np.array_equal(_np(bp.gather_sorted), perm)
    assert np.array_equal(_np(bp.keys_sorted), keys[perm])
    deg = np.diff(offsets)
    hub, chunk = bp.plan.hub_threshold, bp.plan.chunk_size
    assert bp.plan.max_degree == deg.max()
    assert bp.plan.num_hubs == int((deg > hub).sum())
    nch = (deg[deg > hub] + chunk - 1) // chunk
    assert bp.plan.num_chunks == int(nch.sum())
    assert bp.plan.num_multi_hubs == int((nch > 1).sum())
    got_multi = bp.mem[bp.plan.multi_hubs - bp.mem.data_ptr():][: 4 * int((nch > 1).sum())].view(torch.int32) \
        if (nch > 1).any() else torch.zeros(0, dtype=torch.int32)
    assert np.array_equal(_np(got_multi), np.flatnonzero(nch > 1))
    # hubs are listed in key order; items start at the first key of their position range
    hub_keys = np.flatnonzero(deg > hub)
    got_hubs = bp.mem[bp.plan.hub_key - bp.mem.data_ptr():][: 4 * hub_keys.size].view(torch.int32)
    assert np.array_equal(_np(got_hubs), hub_keys)
    # walk items: balanced by weight 1 + messages of non-hub keys, RELM_MP_ITEM_SIZE units each
    item = int(re.search(r"#define RELM_MP_ITEM_SIZE (\d+)", (REPO / "include" / "relm_mp.h").read_text()).group(1))
    weight = 1 + np.where((deg > 0) & (deg <= hub), deg, 0)
    W = np.concatenate([[0], np.cumsum(weight)])
    assert bp.plan.num_items == W[-1] // item + 1
    items = np.searchsorted(W[:-1], np.arange(bp.plan.num_items) * item, side="left")
    items = np.append(items, num_keys)
    assert np.array_equal(_np(bp.item_first), items)
    # short-segment index: the non-hub segments back to back in key order
    short = (deg > 0) & (deg <= hub)
    short_off = W - np.arange(num_keys + 1)
    assert np.array_equal(_np(bp.short_off), short_off)
    assert bp.plan.num_short == int(deg[short].sum())
    mask = np.repeat(short, deg)
    assert np.array_equal(_np(bp.short_gather), perm[mask])
    assert np.array_equal(_np(bp.item_short), short_off[items])


@pytest.mark.parametrize("num_keys,num_edges", [(4096, 98304), (50_000, 1_000_000), (7, 5)])
def test_async_csr_plan_computes_before_its_counts_are_read(num_keys: int, num_edges: int) -> None:
    """A plan whose build returned after validation (statistics still on the
    device) gives the same results as a fully built one; reading the counts
    afterwards gives the same statistics."""

    from relmo_amd import capi

    _log(f"async csr plan keys={num_keys} edges={num_edges}")
    rng = np.random.default_rng(num_keys)
    keys = np.minimum(rng.pareto(0.7, num_edges).astype(np.int64), num_keys - 1)
    table = _t(rng.standard_normal((num_edges, 32)).astype(np.float32))
    kt = _t(keys)
    sync = capi.csr_plan(kt, num_keys, None, num_edges)
    fast = capi.csr_plan(kt, num_keys, None, num_edges, wait_counts=False)
    p = fast.plan
    assert (p.max_degree, p.num_hubs, p.num_chunks, p.num_multi_hubs, p.num_items, p.num_short) == (-1,) * 6
    assert p.gather_identity == 1 and p.counts
    for mode in (0, 1):
        want = capi.plan_segment_reduce(sync, table, mode)
        got = capi.plan_segment_reduce(fast, table, mode)
        assert np.array_equal(_np(got), _np(want), equal_nan=True), mode
    capi.read_counts(fast, kt)
    q = sync.plan
    assert (p.max_degree, p.num_hubs, p.num_chunks, p.num_multi_hubs, p.num_items, p.num_short) == \
        (q.max_degree, q.num_hubs, q.num_chunks, q.num_multi_hubs, q.num_items, q.num_short)
    bad = keys.copy()
    bad[num_edges // 2] = num_keys
    with pytest.raises((RuntimeError, ValueError), match=rf"key index out of bounds: {num_keys} not in"):
        capi.csr_plan(_t(bad), num_keys, None, num_edges, wait_counts=False)
    # several bad indices in different sort tiles: the one of the smallest
    # edge is reported, for the keys and for the gathered indices
    if num_edges >= 3:
        bad[num_edges // 3] = num_keys + 5
        bad[num_edges - 1] = -2
        with pytest.raises((RuntimeError, ValueError), match=rf"key index out of bounds: {num_keys + 5} not in"):
            capi.csr_plan(_t(bad), num_keys, None, num_edges)
        gathers = np.arange(num_edges, dtype=np.int64)
        gathers[num_edges - 1] = num_edges + 9
        gathers[num_edges // 2] = -1
        gathers[num_edges // 3 + 1] = num_edges
        with pytest.raises((RuntimeError, ValueError), match=rf"gather index out of bounds: {num_edges} not in"):
            capi.csr_plan(kt, num_keys, _t(gathers), num_edges)


@pytest.mark.parametrize("large", [True, False])
def test_csr_plan_gathers_in_mixed_tiles(large: bool) -> None:
    """Gathered indices equal to their edge ids in some first-pass tiles and
    not in others: the first scatter generates the values of the former and
    reads the latter."""

    from relmo_amd import capi

    num_keys = (1 << 20) if large else 3000
    n = 3_000_001 if large else 300_001
    _log(f"csr plan mixed gather tiles keys={num_keys} edges={n}")
    rng = np.random.default_rng(5 + large)
    keys = rng.integers(0, num_keys, n)
    gathers = np.arange(n)
    tiles = rng.random((n + 4095) // 4096) < 0.5
    for t in np.flatnonzero(tiles):
        lo, hi = 4096 * t, min(4096 * (t + 1), n)
        gathers[lo:hi] = rng.permutation(gathers[lo:hi])
    bp = capi.csr_plan(_t(keys), num_keys, _t(gathers), n)
    offsets, perm = oracle.csr_build(keys, num_keys)
    assert np.array_equal(_np(bp.offsets), offsets)
    assert np.array_equal(_np(bp.gather_sorted), gathers[perm])
    assert bp.plan.gather_identity == 0


def test_inverse_plan_matches_oracle() -> None:
    from relmo_amd import capi

    rng = np.random.default_rng(11)
    for n, k in [(1000, 5000), (100_000, 100_000), (300_000, 50_000)]:
        keys = rng.permutation(k)[:n] if n <= k else rng.integers(0, k, n)
        bp = capi.inv_plan(_t(keys), k, None, 0)
        inv, coll = oracle.inverse_build(keys, k)
        assert np.array_equal(_np(bp.inv), inv)
        assert bp.plan.collisions == coll
        assert bool(bp.plan.inv)
    # identity keys: the plan is marked as the identity (no inv array)
    for n, k in [(5000, 5000), (4000, 6000)]:
        bp = capi.inv_plan(_t(np.arange(n)), k, None, 0)
        assert not bp.plan.inv and bp.plan.collisions == 0
        assert np.array_equal(_np(bp.inv), oracle.inverse_build(np.arange(n), k)[0])


@pytest.mark.parametrize("identity", [True, False])
def test_async_inverse_plan_gathers_before_validation(identity: bool) -> None:
    """An inverse plan whose validation is still pending already serves the
    gather (identity flag read on the device); validating gives the same
    statistics as a waiting build, and a bad index is reported by validate."""

    from relmo_amd import capi

    rng = np.random.default_rng(5)
    n, k, rows = 50_000, 60_000, 7000
    keys = np.arange(n) if identity else rng.integers(0, k, n)
    gathers = rng.integers(0, rows, n)
    table = _t(rng.standard_normal((rows, 32)).astype(np.float32))
    kt, gt = _t(keys), _t(gathers)
    want_plan = capi.inv_plan(kt, k, gt, rows)
    want = capi.plan_gather_last(want_plan, table, gt)
    bp = capi.inv_plan(kt, k, gt, rows, wait=False)
    assert bp.plan.collisions == -1 and bp.plan.inv
    got = capi.plan_gather_last(bp, table, gt)
    # a second build while a validation is pending is refused
    with pytest.raises(RuntimeError, match="not been validated"):
        capi.inv_plan(kt, k, gt, rows)
    capi.validate(bp)
    assert np.array_equal(_np(got), _np(want))
    assert bp.plan.collisions == want_plan.plan.collisions
    assert bool(bp.plan.inv) == bool(want_plan.plan.inv) == (not identity)
    bad = gathers.copy()
    bad[n // 3] = rows + 2
    bt = _t(bad)  # the index arrays must live until validate() reads the bad value back
    bp = capi.inv_plan(kt, k, bt, rows, gather_name="src_global_idx", wait=False)
    capi.plan_gather_last(bp, table, bt)
    with pytest.raises(RuntimeError, match=rf"src_global_idx index out of bounds: {rows + 2} not in \[0, {rows}\)\."):
        capi.validate(bp)
    capi.validate(bp)  # nothing pending any more


def _segments_bounded(keys: np.ndarray, bound: int = 64) -> bool:
    return keys.size == 0 or np.bincount(keys).max() <= bound


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("emb", [1, 2, 3, 4, 5, 6, 32, 64, 128, 200, 300, 398])
def test_random_parity_all_ops(dtype, emb: int) -> None:
    from relmo_amd import capi

    _log(f"random parity dtype={dtype.__name__} emb={emb}")
    rng = np.random.default_rng(emb * 7 + (dtype == np.float64))
    x_rows, slots, objs = 900, 5000, 700
    x = rng.standard_normal((x_rows, emb)).astype(dtype)
    src = rng.integers(0, x_rows, slots)
    flat_dst = rng.permutation(slots + 300)[:slots]  # injective with untouched rows
    out_rows = slots + 300
    g_slots = rng.standard_normal((out_rows, emb)).astype(dtype)
    rel = rng.standard_normal((slots, emb)).astype(dtype)
    flat_src = rng.permutation(slots)
    dst = rng.integers(0, objs, slots)
    g_obj = rng.standard_normal((objs, emb)).astype(dtype)

    got = _np(capi.fanout_scatter(_t(x), _t(src), _t(flat_dst), out_rows))
    assert np.array_equal(got, oracle.fanout_scatter(x, src, flat_dst, out_rows))
    got = _np(capi.fanout_scatter_backward(_t(g_slots), _t(src), _t(flat_dst), x_rows))
    assert _segments_bounded(src)
    assert np.array_equal(got, oracle.fanout_scatter_backward(g_slots, src, flat_dst, x_rows))
    got = _np(capi.fanin_reduce(_t(rel), _t(flat_src), _t(dst), objs, 0))
    assert np.array_equal(got, oracle.fanin_reduce_sum(rel, flat_src, dst, objs))
    got = _np(capi.fanin_reduce_sum_backward(_t(g_obj), _t(flat_src), _t(dst), slots))
    assert np.array_equal(got, oracle.fanin_reduce_sum_backward(g_obj, flat_src, dst, slots))
    lse = _np(capi.fanin_reduce(_t(rel), _t(flat_src), _t(dst), objs, 1))
    want = oracle.fanin_reduce_logsumexp(rel, flat_src, dst, objs)
    _assert_lse_close(lse, want, "lse fwd")
    got = _np(capi.fanin_reduce_logsumexp_backward(_t(g_obj), _t(rel), _t(flat_src), _t(dst), _t(want), slots))
    ref = oracle.fanin_reduce_logsumexp_backward(g_obj, rel, flat_src, dst, want, slots)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-6)
    # duplicated flat_src: the backward ops take the CSR (sorted) lane
    flat_dup = rng.integers(0, slots // 2, slots)
    got = _np(capi.fanin_reduce_sum_backward(_t(g_obj), _t(flat_dup), _t(dst), slots))
    assert np.array_equal(got, oracle.fanin_reduce_sum_backward(g_obj, flat_dup, dst, slots))
    got = _np(capi.fanin_reduce_logsumexp_backward(_t(g_obj), _t(rel), _t(flat_dup), _t(dst), _t(want), slots))
    ref = oracle.fanin_reduce_logsumexp_backward(g_obj, rel, flat_dup, dst, want, slots)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-6)


def _zipf_keys(rng, num_keys: int, n: int, s: float = 1.1) -> np.ndarray:
    ranks = np.arange(1, num_keys + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    r = np.searchsorted(cdf, rng.random(n), side="right")
    return rng.permutation(num_keys)[np.minimum(r, num_keys - 1)]


def _chunk_size() -> int:
    return int(re.search(r"#define RELM_MP_CHUNK_SIZE (\d+)", (REPO / "include" / "relm_mp.h").read_text()).group(1))


@pytest.mark.parametrize("emb", [32, 6, 64, 128])
def test_hub_segments_against_float64_truth(emb: int) -> None:
    """Hubs of many chunks (the chunk kernel, then the combine kernel) against
    float64 truth at every row geometry the hub kernels are built for: emb 32
    (8 lanes of 16 bytes per row), 64 (16 lanes), 128 (32 lanes), and emb 6
    (rows of an even number of floats that is not a multiple of 4: 8 bytes per
    lane)."""

    from relmo_amd import capi

    rng = np.random.default_rng(12)
    num_keys, n = 20_000, 600_000
    dst = _zipf_keys(rng, num_keys, n)
    rel = (2.0 * rng.standard_normal((n, emb))).astype(np.float32)
    flat_src = rng.permutation(n)
    deg = np.bincount(dst, minlength=num_keys)
    chunk = _chunk_size()
    assert (deg > 3 * chunk).sum() >= 3, "several hubs of more than three chunks"
    short = deg <= 64
    hub = deg > 64
    got = _np(capi.fanin_reduce(_t(rel), _t(flat_src), _t(dst), num_keys, 0))
    want = oracle.fanin_reduce_sum(rel, flat_src, dst, num_keys)
    truth, absum = oracle.segment_sum_truth(rel, flat_src, dst, num_keys)
    assert np.array_equal(got[short], want[short])
    assert np.all(np.abs(got - truth) <= 4 * EPS32 * absum + 1e-30)
    lse = _np(capi.fanin_reduce(_t(rel), _t(flat_src), _t(dst), num_keys, 1))
    lse_truth = oracle.fanin_logsumexp_truth(rel, flat_src, dst, num_keys)
    _assert_lse_close(lse, lse_truth.astype(np.float32), "lse vs truth")
    _assert_lse_close(lse, oracle.fanin_reduce_logsumexp(rel, flat_src, dst, num_keys), "lse vs oracle")
    # hub rows alone, ten times tighter than the op tolerance
    np.testing.assert_allclose(lse[hub], lse_truth[hub], rtol=1e-5, atol=1e-6, err_msg="lse hubs vs truth")
    # fanout backward with hub rows on the source side
    src = _zipf_keys(rng, 5000, n)
    assert (np.bincount(src, minlength=5000) > 3 * chunk).sum() >= 3
    g = rng.standard_normal((n, emb)).astype(np.float32)
    slots = np.arange(n)
    got = _np(capi.fanout_scatter_backward(_t(g), _t(src), _t(slots), 5000))
    truth, absum = oracle.segment_sum_truth(g, slots, src, 5000)
    assert np.all(np.abs(got - truth) <= 4 * EPS32 * absum + 1e-30)


def test_results_are_deterministic() -> None:
    from relmo_amd import capi

    rng = np.random.default_rng(13)
    num_keys, n, emb = 10_000, 400_000, 64
    dst = _t(_zipf_keys(rng, num_keys, n))
    rel = _t(rng.standard_normal((n, emb)).astype(np.float32))
    flat_src = _t(rng.permutation(n))
    for mode in (0, 1):
        a = capi.fanin_reduce(rel, flat_src, dst, num_keys, mode)
        b = capi.fanin_reduce(rel, flat_src, dst, num_keys, mode)
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), mode


def test_autograd_facade_on_gpu(mp_env) -> None:
    from relmo_amd import mp

    rng = np.random.default_rng(14)
    x = torch.tensor(rng.standard_normal((50, 8)), dtype=torch.float32, device=DEV, requires_grad=True)
    src = _t(rng.integers(0, 50, 300))
    flat_dst = _t(rng.permutation(300))
    slots = mp.fanout_scatter(x, src, flat_dst, 300)
    dst = _t(rng.integers(0, 50, 300))
    agg = mp.fanin_reduce(slots, flat_dst, dst, 50, 1) + mp.fanin_reduce(slots, flat_dst, dst, 50, 0)
    loss = torch.where(torch.isfinite(agg), agg, torch.zeros_like(agg)).sum()
    loss.backward()
    x_ref = x.detach().cpu().double().requires_grad_(True)
    from relmo_amd.mp_pack import fanin_reduce_python, fanout_scatter_python

    s = fanout_scatter_python(x_ref, src.cpu(), flat_dst.cpu(), 300)
    a = fanin_reduce_python(s, flat_dst.cpu(), dst.cpu(), 50, 1) + fanin_reduce_python(s, flat_dst.cpu(), dst.cpu(), 50, 0)
    torch.where(torch.isfinite(a), a, torch.zeros_like(a)).sum().backward()
    np.testing.assert_allclose(_np(x.grad), x_ref.grad.numpy(), rtol=1e-4, atol=1e-5)


def test_gradcheck_float64_on_gpu(mp_env) -> None:
    from relmo_amd import mp

    x = torch.randn(6, 3, dtype=torch.float64, device=DEV, requires_grad=True)
    src = torch.tensor([0, 5, 2, 1], device=DEV)
    flat_dst = torch.tensor([1, 0, 3, 2], device=DEV)
    assert torch.autograd.gradcheck(lambda t: mp.fanout_scatter(t, src, flat_dst, 5), (x,), eps=1e-6, atol=1e-4, rtol=1e-3)
    rel = torch.randn(8, 4, dtype=torch.float64, device=DEV, requires_grad=True)
    fs = torch.tensor([0, 2, 5, 7, 1, 3], device=DEV)
    di = torch.tensor([1, 0, 3, 2, 0, 1], device=DEV)
    assert torch.autograd.gradcheck(lambda t: mp.fanin_reduce(t, fs, di, 4, 1), (rel,), eps=1e-6, atol=1e-4, rtol=1e-3)
    assert torch.autograd.gradcheck(lambda t: mp.fanin_reduce(t, fs[:5], di[:5], 5, 0), (rel,), eps=1e-6, atol=1e-4, rtol=1e-3)


def test_noncontiguous_and_plan_cache_reuse(mp_env) -> None:
    from relmo_amd import mp

    ns = torch.ops.relm_mp
    base = torch.randn(4, 6, device=DEV)
    x = base.transpose(0, 1)
    src = torch.tensor([0, 4, 2, 5], device=DEV)
    flat_dst = torch.tensor([2, 1, 0, 3], device=DEV)
    out = mp.fanout_scatter(x, src, flat_dst, 5)
    want = oracle.fanout_scatter(x.cpu().numpy(), src.cpu().numpy(), flat_dst.cpu().numpy(), 5)
    assert np.array_equal(_np(out), want)
    # the cached plan must not survive an in-place change of the index tensor
    ns.plan_cache_clear()
    rel = torch.randn(10, 4, device=DEV)
    fs = torch.tensor([0, 2, 7, 5, 2, 1], device=DEV)
    di = torch.tensor([1, 0, 2, 2, 1, 0], device=DEV)
    a = ns.fanin_reduce(rel, fs, di, 4, 0)
    assert ns.plan_cache_size() >= 1
    di[0] = 3
    b = ns.fanin_reduce(rel, fs, di, 4, 0)
    want = oracle.fanin_reduce_sum(rel.cpu().numpy(), fs.cpu().numpy(), di.cpu().numpy(), 4)
    assert np.array_equal(_np(b), want)
    assert not torch.equal(a, b)


@pytest.mark.parametrize("emb", [3, 32, 64])
def test_backward_by_dst_over_the_forward_plan(emb: int) -> None:
    """With flat_src = arange, the fanin backward runs over the forward's CSR
    plan: identical to the oracle (sum: exact copies) and to the inverse-plan
    lane; rows past the messages are zero."""

    from relmo_amd import capi

    _log(f"backward by dst emb={emb}")
    rng = np.random.default_rng(40 + emb)
    num_keys, n = 3000, 50_000
    dst = _zipf_keys(rng, num_keys, n)
    flat_src = np.arange(n)
    rel_rows = n + 17
    rel = (2.0 * rng.standard_normal((rel_rows, emb))).astype(np.float32)
    g = rng.standard_normal((num_keys, emb)).astype(np.float32)
    bp = capi.csr_plan(_t(dst), num_keys, _t(flat_src), rel_rows, "dst_idx", "flat_src", True)
    assert bp.plan.gather_identity == 1
    got = _np(capi.plan_fanin_backward_by_dst(bp, _t(dst), 0, _t(g), rel_rows))
    assert np.array_equal(got, oracle.fanin_reduce_sum_backward(g, flat_src, dst, rel_rows))
    out = oracle.fanin_reduce_logsumexp(rel, flat_src, dst, num_keys)
    got = _np(capi.plan_fanin_backward_by_dst(bp, _t(dst), 1, _t(g), rel_rows, _t(out), _t(rel)))
    ref = oracle.fanin_reduce_logsumexp_backward(g, rel, flat_src, dst, out, rel_rows)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-6)
    inv_lane = _np(capi.fanin_reduce_logsumexp_backward(_t(g), _t(rel), _t(flat_src), _t(dst), _t(out), rel_rows))
    assert np.array_equal(got, inv_lane)
    ident = capi.identity_inv_plan(rel_rows, n, num_keys)
    got = _np(capi.plan_logsumexp_backward(ident, _t(g), _t(out), _t(rel), _t(dst)))
    assert np.array_equal(got, inv_lane)
    # a permuted flat_src is not the identity: the plan says so and the entry point refuses
    bp2 = capi.csr_plan(_t(dst), num_keys, _t(rng.permutation(n)), rel_rows, "dst_idx", "flat_src", True)
    assert bp2.plan.gather_identity == 0
    with pytest.raises(RuntimeError, match="identity"):
        capi.plan_fanin_backward_by_dst(bp2, _t(dst), 0, _t(g), rel_rows)


def test_backward_by_dst_with_plain_snapshot_tiles() -> None:
    """The backward over the forward's CSR plan reads the destinations from the
    plan's int32 snapshot, where tiles of 4096 edges whose destinations are the
    edge ids are flagged instead of stored: destinations equal to the edge ids
    except in one tile and the partial last one give the same results as the
    int64 lane and the oracle."""

    from relmo_amd import capi

    rng = np.random.default_rng(77)
    n, num_keys, emb = 50_000, 60_000, 32
    dst = np.arange(n)
    dst[3 * 4096:4 * 4096] = rng.integers(0, num_keys, 4096)
    dst[-100:] = rng.integers(0, num_keys, 100)
    flat_src = np.arange(n)
    rel = (2.0 * rng.standard_normal((n, emb))).astype(np.float32)
    g = rng.standard_normal((num_keys, emb)).astype(np.float32)
    bp = capi.csr_plan(_t(dst), num_keys, _t(flat_src), n, "dst_idx", "flat_src", True)
    assert bp.plan.gather_identity == 1
    got = _np(capi.plan_fanin_backward_by_dst(bp, _t(dst), 0, _t(g), n))
    assert np.array_equal(got, oracle.fanin_reduce_sum_backward(g, flat_src, dst, n))
    out = oracle.fanin_reduce_logsumexp(rel, flat_src, dst, num_keys)
    got = _np(capi.plan_fanin_backward_by_dst(bp, _t(dst), 1, _t(g), n, _t(out), _t(rel)))
    ident = capi.identity_inv_plan(n, n, num_keys)
    assert np.array_equal(got, _np(capi.plan_logsumexp_backward(ident, _t(g), _t(out), _t(rel), _t(dst))))
    np.testing.assert_allclose(got, oracle.fanin_reduce_logsumexp_backward(g, rel, flat_src, dst, out, n),
                               rtol=1e-4, atol=1e-6)


def _injective_flat_src(rng, layout: str, n: int):
    """(flat_src, rel_rows) of n edges, injective and not the identity."""

    if layout in ("callers", "callers_full"):  # fused.py:183-190, arity 2: position-major, flat = 2 atom + pos
        a = np.arange(n // 2)
        # "callers_full": as many message rows as edges (a permutation: no map fill, edge-order sum)
        return np.concatenate([2 * a, 2 * a + 1]), n + (17 if layout == "callers" else 0)
    if layout == "gaps":  # arity 2 in a max-arity-3 row layout: every third row has no edge
        a = np.arange(n // 2)
        return np.concatenate([3 * a, 3 * a + 1]), 3 * (n // 2)
    if layout == "partly_plain":  # the edge ids except one 4096-edge tile and the last edges
        f = np.arange(n)
        f[4096:2 * 4096] = f[4096:2 * 4096][rng.permutation(4096)]
        f[-50:] = f[-50:][::-1]
        return f, n
    return rng.permutation(n), n + (17 if layout == "random" else 0)


@pytest.mark.parametrize("layout", ["callers", "callers_full", "gaps", "partly_plain", "random", "random_full"])
@pytest.mark.parametrize("emb", [6, 32, 64])
def test_backward_by_src_over_the_forward_plan(layout: str, emb: int) -> None:
    """flat_src injective but not the identity: the fanin backward builds the
    inverse map of flat_src from the forward plan's snapshot, without atomics,
    reports no collision, and equals the oracle (sum: exact copies) and the
    inverse-plan lane bit for bit; rows that no edge reads are zero.  With as
    many rows as edges the map is built without its initial fill, and the sum
    runs in edge order over the snapshots.  A flat_src that repeats an index
    reports collisions."""

    from relmo_amd import capi

    _log(f"backward by src layout={layout} emb={emb}")
    rng = np.random.default_rng(50 + emb)
    num_keys, n = 3000, 50_000
    dst = _zipf_keys(rng, num_keys, n)
    flat_src, rel_rows = _injective_flat_src(rng, layout, n)
    assert np.unique(flat_src).size == n and flat_src.max() < rel_rows
    rel = (2.0 * rng.standard_normal((rel_rows, emb))).astype(np.float32)
    g = rng.standard_normal((num_keys, emb)).astype(np.float32)
    bp = capi.csr_plan(_t(dst), num_keys, _t(flat_src), rel_rows, "dst_idx", "flat_src", True)
    assert bp.plan.gather_identity == 0
    got, coll = capi.plan_fanin_backward_by_src(bp, 0, _t(g), rel_rows)
    assert coll == 0
    assert np.array_equal(_np(got), oracle.fanin_reduce_sum_backward(g, flat_src, dst, rel_rows))
    out = oracle.fanin_reduce_logsumexp(rel, flat_src, dst, num_keys)
    got, coll = capi.plan_fanin_backward_by_src(bp, 1, _t(g), rel_rows, _t(out), _t(rel))
    assert coll == 0
    got = _np(got)
    np.testing.assert_allclose(got, oracle.fanin_reduce_logsumexp_backward(g, rel, flat_src, dst, out, rel_rows),
                               rtol=1e-4, atol=1e-6)
    inv_lane = _np(capi.fanin_reduce_logsumexp_backward(_t(g), _t(rel), _t(flat_src), _t(dst), _t(out), rel_rows))
    assert np.array_equal(got, inv_lane)
    # one repeated index: counted as a collision
    flat_dup = flat_src.copy()
    flat_dup[5] = flat_dup[n - 3]
    bp2 = capi.csr_plan(_t(dst), num_keys, _t(flat_dup), rel_rows, "dst_idx", "flat_src", True)
    _, coll = capi.plan_fanin_backward_by_src(bp2, 0, _t(g), rel_rows)
    assert coll > 0


@pytest.mark.parametrize("layout", ["callers", "callers_full", "random", "random_full", "repeats"])
def test_facade_backward_with_injective_flat_src(layout: str, mp_env) -> None:
    """Autograd through the facade with a flat_src that is not the identity:
    the backward runs over the forward's plan (inverse map from its snapshot)
    when flat_src is injective, and over its own CSR plan when it repeats; the
    gradients equal those of a second step over the cached plan, the ops
    called without any cached plan, and the oracle."""

    from relmo_amd import mp

    ns = torch.ops.relm_mp
    rng = np.random.default_rng(42)
    num_keys, n, emb = 2000, 40_000, 32
    dst_np = _zipf_keys(rng, num_keys, n)
    if layout == "repeats":
        flat_np, rows = rng.integers(0, n, n), n
    else:
        flat_np, rows = _injective_flat_src(rng, layout, n)
    dst, flat_src = _t(dst_np), _t(flat_np)
    g = _t(rng.standard_normal((num_keys, emb)).astype(np.float32))
    for mode in (0, 1):
        rel = _t((2.0 * rng.standard_normal((rows, emb))).astype(np.float32)).requires_grad_(True)
        ns.plan_cache_clear()
        out = mp.fanin_reduce(rel, flat_src, dst, num_keys, mode)
        (cached,) = torch.autograd.grad(out, rel, g)
        # a second step over the cached forward plan: the inverse map kept
        # with it (injective) or its recorded collision (repeats)
        out2 = mp.fanin_reduce(rel, flat_src, dst, num_keys, mode)
        (again,) = torch.autograd.grad(out2, rel, g)
        assert torch.equal(again, cached), mode
        ns.plan_cache_clear()
        if mode == 0:
            fresh = ns.fanin_reduce_sum_backward(g, flat_src, dst, rows)
        else:
            fresh = ns.fanin_reduce_logsumexp_backward(g, rel.detach(), flat_src, dst, out.detach(), rows)
        assert torch.equal(cached, fresh), mode
        if mode == 0:
            want = oracle.fanin_reduce_sum_backward(_np(g), flat_np, dst_np, rows)
        else:
            want = oracle.fanin_reduce_logsumexp_backward(_np(g), _np(rel.detach()), flat_np, dst_np,
                                                          _np(out.detach()), rows)
        np.testing.assert_allclose(_np(cached), want, rtol=1e-4, atol=1e-6)


def test_facade_backward_reuses_forward_plan(mp_env) -> None:
    """Autograd through the facade with flat_src = arange: the backward finds the
    forward's plan in the cache; results equal those computed without it."""

    from relmo_amd import mp

    ns = torch.ops.relm_mp
    rng = np.random.default_rng(41)
    num_keys, n, emb = 2000, 40_000, 32
    dst = _t(_zipf_keys(rng, num_keys, n))
    flat_src = torch.arange(n, device=DEV)
    g = _t(rng.standard_normal((num_keys, emb)).astype(np.float32))
    for mode in (0, 1):
        rel = _t((2.0 * rng.standard_normal((n, emb))).astype(np.float32)).requires_grad_(True)
        ns.plan_cache_clear()
        out = mp.fanin_reduce(rel, flat_src, dst, num_keys, mode)
        (cached,) = torch.autograd.grad(out, rel, g)
        ns.plan_cache_clear()
        if mode == 0:
            fresh = ns.fanin_reduce_sum_backward(g, flat_src, dst, n)
        else:
            fresh = ns.fanin_reduce_logsumexp_backward(g, rel.detach(), flat_src, dst, out.detach(), n)
        assert torch.equal(cached, fresh), mode
        want = (oracle.fanin_reduce_sum_backward(_np(g), _np(flat_src), _np(dst), n) if mode == 0 else
                oracle.fanin_reduce_logsumexp_backward(_np(g), _np(rel.detach()), _np(flat_src), _np(dst),
                                                       _np(out.detach()), n))
        np.testing.assert_allclose(_np(cached), want, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("model", ["relational", "centralized"])
@pytest.mark.parametrize("mode", [0, 1])
def test_model_training_step_matches_aten_lane(model: str, mode: int, monkeypatch) -> None:
    """The reference's model-level callers (C4 / C5 structure, small batch):
    the HIP op lane and the ATen lane give the same loss, output and
    parameter gradients."""

    from relmo_amd import consumers as C

    _log(f"model {model} mode={mode}")
    if model == "relational":
        batch = C.synthetic_c4(DEV, seed=3, num_graphs=6)
        make = lambda: C.RelationalGNN(32, 3, batch.relations, mode).to(DEV)
    else:
        batch = C.synthetic_c5(DEV, seed=3, num_graphs=4)
        make = lambda: C.CentralizedRelationalGNN(16, 3, batch.relations, mode).to(DEV)
    torch.manual_seed(0)
    m = make()
    routing = m.routing(batch)
    monkeypatch.setenv("RELM_MP_ENABLE", "1")
    loss = C.train_step(m, batch, routing)
    grads = {k: p.grad.clone() for k, p in m.named_parameters() if p.grad is not None}
    monkeypatch.setenv("RELM_MP_ENABLE", "0")
    loss_ref = C.train_step(m, batch, routing)
    assert torch.allclose(loss, loss_ref, rtol=1e-4, atol=1e-6)
    for k, p in m.named_parameters():
        if p.grad is None:
            continue
        torch.testing.assert_close(grads[k], p.grad, rtol=2e-3, atol=1e-5, msg=k)
