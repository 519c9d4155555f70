"""Pins the C oracle: golden fixtures of the reference library, the reference
library itself where it is built, numpy brute force, closed forms and
invariants chosen so that a dropped term, a wrong index or a transposed
operand fails one of them."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle, ref_runner

ORACLE_OPS = {
    "fanout_scatter": oracle.fanout_scatter,
    "fanout_scatter_backward": oracle.fanout_scatter_backward,
    "fanin_reduce": oracle.fanin_reduce,
    "fanin_reduce_sum_backward": oracle.fanin_reduce_sum_backward,
    "fanin_reduce_logsumexp_backward": oracle.fanin_reduce_logsumexp_backward,
}


def _is_logsumexp(case: dict) -> bool:
    return case["op"] == "fanin_reduce_logsumexp_backward" or (
        case["op"] == "fanin_reduce" and case["ints"][1] == 1
    )


def test_oracle_matches_every_golden_case(golden) -> None:
    cases, arrays = golden
    for case in cases:
        args = [arrays[n] for n in case["tensors"]] + list(case["ints"])
        fn = ORACLE_OPS[case["op"]]
        if "error" in case:
            with pytest.raises((RuntimeError, ValueError, IndexError)) as info:
                fn(*args)
            assert str(info.value) == case["error"], case["name"]
            assert (case.get("error_type") == "IndexError") == isinstance(info.value, IndexError), case["name"]
            continue
        got = fn(*args)
        want = arrays[case["expected"]]
        assert got.dtype == want.dtype and got.shape == want.shape, case["name"]
        if _is_logsumexp(case):
            # The reference computes exp/log with ATen's vectorised kernels,
            # the oracle with libm: agreement to a few ulp.
            np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-6, equal_nan=True, err_msg=case["name"])
            assert np.array_equal(np.isnan(got), np.isnan(want)), case["name"]
            assert np.array_equal(np.isneginf(got), np.isneginf(want)), case["name"]
        else:
            assert np.array_equal(got, want, equal_nan=True), case["name"]


def test_oracle_c1_digests() -> None:
    import hashlib
    import json

    from tests.conftest import GOLDEN
    from tests.golden.c1_config import c1_inputs

    a = c1_inputs()
    digests = json.loads((GOLDEN / "c1_digests.json").read_text())
    outs = {
        "fanout_scatter": oracle.fanout_scatter(a["x"], a["src"], a["flat_dst"], a["src"].size),
        "fanout_scatter_backward": oracle.fanout_scatter_backward(a["grad_slots"], a["src"], a["flat_dst"], a["x"].shape[0]),
        "fanin_reduce": oracle.fanin_reduce_sum(a["rel"], a["flat_src"], a["dst"], a["x"].shape[0]),
        "fanin_reduce_sum_backward": oracle.fanin_reduce_sum_backward(a["grad_obj"], a["flat_src"], a["dst"], a["rel"].shape[0]),
    }
    for op, out in outs.items():
        assert hashlib.sha256(np.ascontiguousarray(out).tobytes()).hexdigest() == digests[op], op


def test_fanout_matches_brute_force_with_duplicates() -> None:
    rng = np.random.default_rng(1)
    x = rng.standard_normal((30, 7)).astype(np.float32)
    src = rng.integers(0, 30, 200)
    dst = rng.integers(0, 50, 200)
    want = np.zeros((50, 7), np.float32)
    for e in range(200):
        want[dst[e]] = x[src[e]]
    assert np.array_equal(oracle.fanout_scatter(x, src, dst, 50), want)


def test_sums_match_float64_truth_and_conserve_mass() -> None:
    rng = np.random.default_rng(2)
    rel = rng.standard_normal((400, 5)).astype(np.float32)
    src = rng.integers(0, 400, 1000)
    dst = rng.integers(0, 37, 1000)
    out = oracle.fanin_reduce_sum(rel, src, dst, 37)
    truth, absum = oracle.segment_sum_truth(rel, src, dst, 37)
    assert np.all(np.abs(out - truth) <= 1e-6 * absum + 1e-30)
    # conservation: the total over all rows equals the total over all messages
    np.testing.assert_allclose(out.astype(np.float64).sum(0), rel[src].astype(np.float64).sum(0), rtol=1e-5)
    # linearity: f(2a + b) == 2 f(a) + f(b) in float64
    rel64 = rel.astype(np.float64)
    b64 = rng.standard_normal(rel64.shape)
    lhs = oracle.fanin_reduce_sum(2 * rel64 + b64, src, dst, 37)
    rhs = 2 * oracle.fanin_reduce_sum(rel64, src, dst, 37) + oracle.fanin_reduce_sum(b64, src, dst, 37)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-12, atol=1e-12)
    # fanout backward is the adjoint of fanout: <fanout(x), g> == <x, fanout_bwd(g)>
    x = rng.standard_normal((400, 5))
    g = rng.standard_normal((1000, 5))
    slot = np.arange(1000)
    lhs = np.sum(oracle.fanout_scatter(x, src, slot, 1000) * g)
    rhs = np.sum(x * oracle.fanout_scatter_backward(g, src, slot, 400))
    assert abs(lhs - rhs) < 1e-9 * max(1.0, abs(lhs))


def test_slot_oracle_matches_elementwise_loop_and_is_adjoint() -> None:
    """fanout_into_slots against a loop over edges and elements (line
    flat_dst // slots, column col + (flat_dst % slots) * D + c, last edge
    wins), and fanout_backward_from_slots as its adjoint over the slot
    columns."""

    rng = np.random.default_rng(11)
    lines, slots, d, col, width = 23, 3, 5, 4, 4 + 3 * 5 + 2
    x = rng.standard_normal((17, d))
    src = rng.integers(0, 17, 90)
    dst = rng.integers(0, lines * slots, 90)  # duplicates and empty slots
    out = rng.standard_normal((lines, width))
    want = out.copy()
    want[:, col:col + slots * d] = 0.0
    for e in range(src.size):
        line, slot = divmod(int(dst[e]), slots)
        for c in range(d):
            want[line, col + slot * d + c] = x[src[e], c]
    got = oracle.fanout_into_slots(x, src, dst, out, col, slots)
    assert np.array_equal(got, want)
    # adjoint over the slot columns (edges with distinct destinations)
    dst1 = rng.permutation(lines * slots)[:40]
    src1 = rng.integers(0, 17, 40)
    g = rng.standard_normal((lines, width))
    fwd = oracle.fanout_into_slots(x, src1, dst1, np.zeros((lines, width)), col, slots)
    lhs = np.sum(fwd * g)
    rhs = np.sum(x * oracle.fanout_backward_from_slots(g, src1, dst1, 17, col, slots, d))
    assert abs(lhs - rhs) < 1e-10 * max(1.0, abs(lhs))


def test_sum_backward_is_adjoint_of_sum() -> None:
    rng = np.random.default_rng(3)
    rel = rng.standard_normal((60, 4))
    src = rng.integers(0, 60, 150)  # duplicates on purpose
    dst = rng.integers(0, 9, 150)
    g = rng.standard_normal((9, 4))
    lhs = np.sum(oracle.fanin_reduce_sum(rel, src, dst, 9) * g)
    rhs = np.sum(rel * oracle.fanin_reduce_sum_backward(g, src, dst, 60))
    assert abs(lhs - rhs) < 1e-10 * max(1.0, abs(lhs))


def test_logsumexp_closed_forms() -> None:
    rng = np.random.default_rng(4)
    rel = rng.standard_normal((10, 3)).astype(np.float64)
    # single message: log(exp(x - x)) + x == x exactly
    out = oracle.fanin_reduce_logsumexp(rel, [7], [2], 4)
    assert np.array_equal(out[2], rel[7])
    assert np.all(np.isneginf(out[[0, 1, 3]]))
    # n equal values c -> c + log n
    c = np.full((5, 3), 1.25)
    out = oracle.fanin_reduce_logsumexp(c, np.arange(5), np.zeros(5, np.int64), 1)
    np.testing.assert_allclose(out[0], 1.25 + np.log(5.0), rtol=1e-15)
    # shift invariance and bounds max <= lse <= max + log n
    src = rng.integers(0, 10, 40)
    dst = rng.integers(0, 6, 40)
    a = oracle.fanin_reduce_logsumexp(rel, src, dst, 6)
    b = oracle.fanin_reduce_logsumexp(rel + 3.5, src, dst, 6)
    np.testing.assert_allclose(b, a + 3.5, rtol=1e-13)
    for d in range(6):
        sel = rel[src[dst == d]]
        if len(sel):
            assert np.all(sel.max(0) <= a[d] + 1e-12) and np.all(a[d] <= sel.max(0) + np.log(len(sel)) + 1e-12)
            np.testing.assert_allclose(a[d], np.log(np.exp(sel).sum(0)), rtol=1e-13)
    # all -inf row -> NaN (exp(-inf - -inf)); +inf -> NaN; NaN propagates
    v = np.array([[-np.inf, 0.0, np.nan], [-np.inf, np.inf, 1.0]])
    out = oracle.fanin_reduce_logsumexp(v, [0, 1], [0, 0], 1)
    assert np.isnan(out[0]).all()


def test_logsumexp_backward_weights_sum_to_one_and_match_finite_differences() -> None:
    rng = np.random.default_rng(5)
    rel = rng.standard_normal((30, 4))
    src = rng.permutation(30)[:25]
    dst = rng.integers(0, 7, 25)
    out = oracle.fanin_reduce_logsumexp(rel, src, dst, 7)
    ones = np.ones((7, 4))
    g = oracle.fanin_reduce_logsumexp_backward(ones, rel, src, dst, out, 30)
    for d in range(7):
        if (dst == d).any():
            np.testing.assert_allclose(g[src[dst == d]].sum(0), 1.0, rtol=1e-12)
    gout = rng.standard_normal((7, 4))
    gout[np.bincount(dst, minlength=7) == 0] = 0.0  # rows without messages hold -inf
    grad = oracle.fanin_reduce_logsumexp_backward(gout, rel, src, dst, out, 30)
    live = np.bincount(dst, minlength=7) > 0
    eps = 1e-6
    for r, k in [(src[0], 0), (src[3], 2), (src[10], 3)]:
        plus, minus = rel.copy(), rel.copy()
        plus[r, k] += eps
        minus[r, k] -= eps
        fd = (np.sum((gout * oracle.fanin_reduce_logsumexp(plus, src, dst, 7))[live])
              - np.sum((gout * oracle.fanin_reduce_logsumexp(minus, src, dst, 7))[live])) / (2 * eps)
        assert abs(fd - grad[r, k]) < 1e-6


def test_csr_and_inverse_builders_match_numpy() -> None:
    rng = np.random.default_rng(6)
    keys = rng.integers(0, 300, 5000)
    offsets, perm = oracle.csr_build(keys, 300)
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(keys, minlength=300))]))
    assert np.array_equal(perm, np.argsort(keys, kind="stable"))
    inv, coll = oracle.inverse_build(keys, 300)
    want = np.full(300, -1)
    for e, k in enumerate(keys):
        want[k] = e
    assert np.array_equal(inv, want)
    assert coll == 5000 - len(np.unique(keys))


@pytest.mark.skipif(not ref_runner.available(), reason="oracle/_ref not built")
def test_oracle_matches_reference_library_on_random_inputs() -> None:
    rng = np.random.default_rng(7)
    arrays = {
        "x": rng.standard_normal((500, 16)).astype(np.float32),
        "src": rng.integers(0, 500, 3000),
        "dst": rng.integers(0, 900, 3000),
        "g": rng.standard_normal((900, 16)).astype(np.float32),
        "rel": (2 * rng.standard_normal((3000, 16))).astype(np.float32),
        "fsrc": rng.permutation(3000),
        "fdst": rng.integers(0, 64, 3000),
        "gk": rng.standard_normal((64, 16)).astype(np.float32),
    }
    lse = oracle.fanin_reduce_logsumexp(arrays["rel"], arrays["fsrc"], arrays["fdst"], 64)
    arrays["lse"] = lse
    calls = [
        {"op": "fanout_scatter", "tensors": ["x", "src", "dst"], "ints": [900]},
        {"op": "fanout_scatter_backward", "tensors": ["g", "src", "dst"], "ints": [500]},
        {"op": "fanin_reduce", "tensors": ["rel", "fsrc", "fdst"], "ints": [64, 0]},
        {"op": "fanin_reduce", "tensors": ["rel", "fsrc", "fdst"], "ints": [64, 1]},
        {"op": "fanin_reduce_sum_backward", "tensors": ["gk", "fsrc", "fdst"], "ints": [3000]},
        {"op": "fanin_reduce_logsumexp_backward", "tensors": ["gk", "rel", "fsrc", "fdst", "lse"], "ints": [3000]},
    ]
    res = ref_runner.run_reference(calls, arrays)
    a = arrays
    assert np.array_equal(res[0]["out"], oracle.fanout_scatter(a["x"], a["src"], a["dst"], 900))
    assert np.array_equal(res[1]["out"], oracle.fanout_scatter_backward(a["g"], a["src"], a["dst"], 500))
    assert np.array_equal(res[2]["out"], oracle.fanin_reduce_sum(a["rel"], a["fsrc"], a["fdst"], 64))
    np.testing.assert_allclose(res[3]["out"], lse, rtol=2e-6)
    assert np.array_equal(res[4]["out"], oracle.fanin_reduce_sum_backward(a["gk"], a["fsrc"], a["fdst"], 3000))
    np.testing.assert_allclose(
        res[5]["out"],
        oracle.fanin_reduce_logsumexp_backward(a["gk"], a["rel"], a["fsrc"], a["fdst"], lse, 3000),
        rtol=2e-6, atol=1e-7,
    )


# ---- pack ops (oracle/pack.py) ------------------------------------------------------------
#
# Known answers: the inputs of the reference's own tests
# (tests/python/test_mp_ops.py:353-600) with the outputs worked out by hand
# from the op definitions (row offsets 0, 5 for x parts of 5 and 4 rows; 0, 6
# for rel parts of 6 and 3 rows).

from oracle import pack as pack_oracle  # noqa: E402


def _xs():
    return [np.zeros((5, 3), np.float32), np.ones((4, 3), np.float32)]


def _rels():
    return [np.zeros((6, 4), np.float32), np.ones((3, 4), np.float32)]


def test_pack_oracle_known_answers() -> None:
    x_cat, src, dst = pack_oracle.fanout_pack_multi(_xs(), [[0, 2, 4], [1, 3]], [[3, 1, 5], [0, 4]])
    assert x_cat.shape == (9, 3) and x_cat[5:].all() and not x_cat[:5].any()
    assert src.tolist() == [0, 2, 4, 6, 8] and dst.tolist() == [3, 1, 5, 0, 4]

    rel_cat, src, dst = pack_oracle.fanin_pack_multi(_rels(), [[0, 2, 5], [1, 2]], [[1, 0, 2], [2, 1]])
    assert rel_cat.shape == (9, 4)
    assert src.tolist() == [0, 2, 5, 7, 8] and dst.tolist() == [1, 0, 2, 2, 1]

    _, src, dst = pack_oracle.fanout_pack_from_edges(
        _xs(), [[0, 2, 4], [1, 3], [2, 0]], [[1, 0, 2], [3, 1], [0, 2]],
        [0, 1, 0], [2, 3, 2], [0, 1, 1], [0, 8, 0],
    )
    # part 0: dst*2+0; part 1: 8 + dst*3 + 1, src + 5; part 2: dst*2+1
    assert src.tolist() == [0, 2, 4, 6, 8, 2, 0]
    assert dst.tolist() == [2, 0, 4, 18, 12, 1, 5]

    _, src, dst = pack_oracle.fanin_pack_from_edges(
        _rels(), [[0, 2, 1], [1, 2]], [[1, 0, 2], [2, 1]], [0, 1], [1, 1], [0, 0], 1)
    assert src.tolist() == [0, 2, 1, 7, 8] and dst.tolist() == [1, 0, 2, 2, 1]
    _, src, dst = pack_oracle.fanin_pack_from_edges(
        _rels(), [[0, 2, 1], [0, 0]], [[1, 0, 2], [2, 1]], [0, 1], [2, 3], [1, 2], 0)
    # part 0: src*2+1; part 1: src*3+2+6
    assert src.tolist() == [1, 5, 3, 8, 8] and dst.tolist() == [1, 0, 2, 2, 1]


def _random_edge_parts(rng, n_values, n_parts, max_len=300):
    rows = [int(r) for r in rng.integers(1, 50, n_values)]
    values = [rng.standard_normal((r, 3)).astype(np.float32) for r in rows]
    lens = [int(v) for v in rng.integers(0, max_len, n_parts)]
    lens[0] = 0  # an empty part
    part_ids = [int(v) for v in rng.integers(0, n_values, n_parts)]
    arity = [int(v) for v in rng.integers(1, 5, n_parts)]
    pos = [int(rng.integers(0, a)) for a in arity]
    slot = [int(v) for v in rng.integers(0, 10_000, n_parts)]
    src = [rng.integers(0, rows[p], n) for p, n in zip(part_ids, lens)]
    dst = [rng.integers(0, 1000, n) for n in lens]
    return values, src, dst, part_ids, arity, pos, slot


def test_pack_oracle_invariants() -> None:
    rng = np.random.default_rng(11)
    values, src, dst, ids, arity, pos, slot = _random_edge_parts(rng, 4, 9)
    offsets = np.cumsum([0] + [v.shape[0] for v in values])
    x_cat, s_out, d_out = pack_oracle.fanout_pack_from_edges(values, src, dst, ids, arity, pos, slot)
    assert np.array_equal(x_cat, np.concatenate(values))
    bounds = np.cumsum([0] + [len(s) for s in src])
    for i in range(len(src)):
        seg = slice(bounds[i], bounds[i + 1])
        assert np.array_equal(s_out[seg] - offsets[ids[i]], src[i])
        q, r = np.divmod(d_out[seg] - slot[i], arity[i])
        assert np.array_equal(q, dst[i]) and (r == pos[i]).all()
        # the gathered rows are the rows of the named part
        assert np.array_equal(x_cat[s_out[seg]], values[ids[i]][src[i]])
    # arity 1, pos 0, slot 0 and parts in order: fanout_pack_multi
    k = len(values)
    multi = pack_oracle.fanout_pack_multi(values, src[:k], dst[:k])
    edges = pack_oracle.fanout_pack_from_edges(values, src[:k], dst[:k], list(range(k)), [1] * k,
                                               [0] * k, [0] * k)
    for m, e in zip(multi, edges):
        assert np.array_equal(m, e)

    _, f_src, f_dst = pack_oracle.fanin_pack_from_edges(values, src, dst, ids, arity, pos, 0)
    for i in range(len(src)):
        seg = slice(bounds[i], bounds[i + 1])
        q, r = np.divmod(f_src[seg] - offsets[ids[i]], arity[i])
        assert np.array_equal(q, src[i]) and (r == pos[i]).all()
        assert np.array_equal(f_dst[seg], dst[i])
    label = pack_oracle.fanin_pack_from_edges(values, src[:k], dst[:k], list(range(k)), arity[:k],
                                              pos[:k], 1)
    for m, e in zip(pack_oracle.fanin_pack_multi(values, src[:k], dst[:k]), label):
        assert np.array_equal(m, e)
    # int64 arithmetic wraps as torch's does
    _, s_big, d_big = pack_oracle.fanout_pack_from_edges(
        values[:1], [np.array([0])], [np.array([2**62])], [0], [4], [1], [5])
    assert d_big.tolist() == [(5 + 2**64 + 1) % 2**64]


def _pack_calls(values, src, dst, ids, arity, pos, slot):
    arrays = {f"v{i}": v for i, v in enumerate(values)}
    arrays.update({f"s{i}": np.asarray(s, np.int64) for i, s in enumerate(src)})
    arrays.update({f"d{i}": np.asarray(d, np.int64) for i, d in enumerate(dst)})
    vn = [f"v{i}" for i in range(len(values))]
    sn = [f"s{i}" for i in range(len(src))]
    dn = [f"d{i}" for i in range(len(dst))]
    k = len(values)
    calls = [
        {"op": "fanout_pack_multi", "args": [{"tensors": vn}, {"tensors": sn[:k]}, {"tensors": dn[:k]}]},
        {"op": "fanin_pack_multi", "args": [{"tensors": vn}, {"tensors": sn[:k]}, {"tensors": dn[:k]}]},
        {"op": "fanout_pack_from_edges", "args": [{"tensors": vn}, {"tensors": sn}, {"tensors": dn},
                                                  {"ints": ids}, {"ints": arity}, {"ints": pos},
                                                  {"ints": slot}]},
        {"op": "fanin_pack_from_edges", "args": [{"tensors": vn}, {"tensors": sn}, {"tensors": dn},
                                                 {"ints": ids}, {"ints": arity}, {"ints": pos},
                                                 {"int": 0}]},
        {"op": "fanin_pack_from_edges", "args": [{"tensors": vn}, {"tensors": sn}, {"tensors": dn},
                                                 {"ints": ids}, {"ints": arity}, {"ints": pos},
                                                 {"int": 1}]},
    ]
    expected = [
        pack_oracle.fanout_pack_multi(values, src[:k], dst[:k]),
        pack_oracle.fanin_pack_multi(values, src[:k], dst[:k]),
        pack_oracle.fanout_pack_from_edges(values, src, dst, ids, arity, pos, slot),
        pack_oracle.fanin_pack_from_edges(values, src, dst, ids, arity, pos, 0),
        pack_oracle.fanin_pack_from_edges(values, src, dst, ids, arity, pos, 1),
    ]
    return arrays, calls, expected


@pytest.mark.skipif(not ref_runner.available(), reason="oracle/_ref not built")
def test_pack_oracle_matches_reference_library() -> None:
    rng = np.random.default_rng(12)
    for n_values, n_parts in [(1, 1), (3, 5), (4, 20)]:
        case = _random_edge_parts(rng, n_values, n_parts)
        arrays, calls, expected = _pack_calls(*case)
        for res, want in zip(ref_runner.run_reference(calls, arrays), expected):
            assert "error" not in res, res
            for got, w in zip(res["outs"], want):
                assert got.dtype == w.dtype and np.array_equal(got, w), res["op"]


def test_pack_oracle_matches_every_golden_case(pack_golden) -> None:
    cases, arrays = pack_golden
    fns = {
        "fanout_pack_multi": pack_oracle.fanout_pack_multi,
        "fanin_pack_multi": pack_oracle.fanin_pack_multi,
        "fanout_pack_from_edges": pack_oracle.fanout_pack_from_edges,
        "fanin_pack_from_edges": pack_oracle.fanin_pack_from_edges,
    }
    checked = 0
    for case in cases:
        if "error" in case:
            continue
        args = []
        for spec in case["args"]:
            if "tensors" in spec:
                args.append([arrays[n] for n in spec["tensors"]])
            else:
                args.append(spec.get("ints", spec.get("int")))
        got = fns[case["op"]](*args)
        for g, name in zip(got, case["expected"]):
            want = arrays[name]
            assert g.dtype == want.dtype and g.shape == want.shape, case["name"]
            assert np.array_equal(g, want), case["name"]
        checked += 1
    assert checked >= 30


# ---- LGAN indexed reductions (oracle/lgan.py) ---------------------------------------------

from oracle import lgan as lgan_oracle  # noqa: E402

LGAN_FNS = {
    "lgan_pool_reduce": lgan_oracle.lgan_pool_reduce,
    "lgan_pool_reduce_backward": lgan_oracle.lgan_pool_reduce_backward,
    "lgan_relation_graph_step": lgan_oracle.lgan_relation_graph_step,
    "lgan_relation_graph_step_backward": lgan_oracle.lgan_relation_graph_step_backward,
}


def _np_args(case: dict, arrays: dict) -> list:
    return [arrays[s["tensor"]] if "tensor" in s else s["int"] for s in case["args"]]


def test_lgan_oracle_matches_every_golden_case(lgan_golden) -> None:
    cases, arrays = lgan_golden
    checked = 0
    for case in cases:
        if "error" in case:
            continue
        got = LGAN_FNS[case["op"]](*_np_args(case, arrays))
        got = got if isinstance(got, tuple) else (got,)
        for g, name in zip(got, case["expected"]):
            want = arrays[name]
            assert g.dtype == want.dtype and g.shape == want.shape, case["name"]
            assert np.array_equal(g, want), case["name"]
        checked += 1
    assert checked >= 40


def _dense(src, dst, rows, cols, mode):
    """Matrix M with (M x)[d] = aggregate of x[src[e]] over dst[e] == d."""

    m = np.zeros((rows, cols))
    for s, d in zip(src, dst):
        m[d, s] += 1.0
    if mode == 2:
        m /= np.maximum(m.sum(axis=1, keepdims=True), 1.0)
    return m


def _random_lgan(rng, K=30, ent=17, E=70, D=4):
    return dict(
        slot=rng.standard_normal((E, D)), s2r=rng.integers(0, K, E), arity=rng.integers(-1, 4, K),
        rr=(rng.integers(0, K, 90), rng.integers(0, K, 90)),
        tn=(rng.integers(0, K, 60), rng.integers(0, ent, 60)),
        nn=(rng.integers(0, K, 40), rng.integers(0, ent, 40)), K=K, ent=ent, E=E, D=D)


@pytest.mark.parametrize("mode", [0, 2])
def test_lgan_oracle_against_dense_matrices(mode) -> None:
    """float64 truth: the ops are linear maps; build their matrices densely."""

    rng = np.random.default_rng(31 + mode)
    r = _random_lgan(rng)
    K, ent, E = r["K"], r["ent"], r["E"]
    P = np.zeros((K, E))
    P[r["s2r"], np.arange(E)] = 1.0
    P /= np.maximum(r["arity"], 1)[:, None]
    R = np.eye(K) + _dense(*r["rr"], K, K, mode)
    T, N = _dense(*r["tn"], ent, K, mode), _dense(*r["nn"], ent, K, mode)
    rpx, tn, nn = lgan_oracle.lgan_pool_reduce(r["slot"], r["s2r"], r["arity"], *r["rr"], *r["tn"],
                                              *r["nn"], ent, mode)
    x = R @ (P @ r["slot"])
    np.testing.assert_allclose(rpx, x, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(tn, T @ x, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(nn, N @ x, rtol=1e-12, atol=1e-12)
    # the backward ops are the transposed maps
    g = rng.standard_normal((K, r["D"]))
    gt, gn = rng.standard_normal((ent, r["D"])), rng.standard_normal((ent, r["D"]))
    grad = lgan_oracle.lgan_pool_reduce_backward(g, gt, gn, r["s2r"], r["arity"], *r["rr"], *r["tn"],
                                                 *r["nn"], K, mode)
    want = P.T @ (R.T @ (g + T.T @ gt + N.T @ gn))
    np.testing.assert_allclose(grad, want, rtol=1e-12, atol=1e-12)
    step_grad = lgan_oracle.lgan_relation_graph_step_backward(g, gt, gn, *r["rr"], *r["tn"], *r["nn"],
                                                              K, mode)
    np.testing.assert_allclose(step_grad, R.T @ (g + T.T @ gt + N.T @ gn), rtol=1e-12, atol=1e-12)


def test_lgan_oracle_mean_of_equal_rows() -> None:
    """mean mode: every entity that receives messages from identical rows gets that row."""

    rng = np.random.default_rng(33)
    row = rng.standard_normal(6)
    x = np.tile(row, (20, 1))
    src, dst = rng.integers(0, 20, 50), rng.integers(0, 9, 50)
    out = lgan_oracle.indexed_sum_or_mean(x, src, dst, 9, 2)
    hit = np.bincount(dst, minlength=9) > 0
    np.testing.assert_allclose(out[hit], np.tile(row, (hit.sum(), 1)), rtol=1e-15)
    assert not out[~hit].any()
