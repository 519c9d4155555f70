"""Writes the golden fixtures under tests/golden/ from relmo's own CPU op library.

The expected outputs come from ``oracle/_ref/relm_mp_ops_ref.so`` - the
reference's ``src/_ops/mp/mp_ops.cpp`` compiled unchanged (``make -C oracle
ref``) - run through ``oracle/ref_runner.py``.  Inputs are seeded
(numpy PCG64), and the index vectors include the fixed ones of the
reference's tests (tests/python/test_mp_ops.py:176-342).

Run from the repository root where /root/reference is present:
    python tests/golden/make_golden.py
Outputs: tests/golden/reference_cases.npz (arrays) and
tests/golden/reference_cases.json (cases: op, argument names, ints, expected
output name or error), plus c1_digests.json (sha256 of the reference outputs
of the CPU-runnable op micro-benchmark configuration).
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

from oracle import ref_runner  # noqa: E402
from tests.golden.c1_config import c1_inputs  # noqa: E402


class Builder:
    def __init__(self, seed: int = 0):
        self.rng = np.random.default_rng(seed)
        self.arrays: dict[str, np.ndarray] = {}
        self.cases: list[dict] = []

    def arr(self, name: str, value) -> str:
        self.arrays[name] = np.ascontiguousarray(value)
        return name

    def randn(self, name: str, shape, dtype=np.float32, scale=1.0) -> str:
        return self.arr(name, (scale * self.rng.standard_normal(shape)).astype(dtype))

    def idx(self, name: str, values) -> str:
        return self.arr(name, np.asarray(values, dtype=np.int64))

    def case(self, name: str, op: str, tensors: list[str], ints: list[int]) -> None:
        self.cases.append({"name": name, "op": op, "tensors": tensors, "ints": ints})


def add_reference_test_vectors(b: Builder) -> None:
    """Index vectors of the reference tests, with seeded values."""

    # test_fanout_scatter_parity (test_mp_ops.py:199-205)
    b.randn("t1_x", (7, 5))
    b.idx("t1_src", [0, 3, 5, 2, 3])
    b.idx("t1_dst", [4, 1, 0, 2, 3])
    b.case("t1_fanout", "fanout_scatter", ["t1_x", "t1_src", "t1_dst"], [6])
    b.randn("t1_g", (6, 5))
    b.case("t1_fanout_bwd", "fanout_scatter_backward", ["t1_g", "t1_src", "t1_dst"], [7])
    # test_fanout_scatter_grad_parity (:219-223)
    b.randn("t2_x", (8, 4))
    b.idx("t2_src", [0, 5, 2, 6])
    b.idx("t2_dst", [1, 0, 3, 2])
    b.case("t2_fanout", "fanout_scatter", ["t2_x", "t2_src", "t2_dst"], [5])
    b.arr("t2_g", np.ones((5, 4), dtype=np.float32))
    b.case("t2_fanout_bwd", "fanout_scatter_backward", ["t2_g", "t2_src", "t2_dst"], [8])
    # test_fanin_reduce_parity (:244-250)
    b.randn("t3_rel", (10, 4))
    b.idx("t3_src", [0, 2, 7, 5, 2, 1])
    b.idx("t3_dst", [1, 0, 2, 2, 1, 0])
    for mode in (0, 1):
        b.case(f"t3_fanin_m{mode}", "fanin_reduce", ["t3_rel", "t3_src", "t3_dst"], [4, mode])
    b.randn("t3_g", (4, 4))
    b.case("t3_fanin_sum_bwd", "fanin_reduce_sum_backward", ["t3_g", "t3_src", "t3_dst"], [10])
    # test_fanin_reduce_grad_parity (:267-272)
    b.randn("t4_rel", (12, 3))
    b.idx("t4_src", [0, 1, 8, 4, 9, 10])
    b.idx("t4_dst", [2, 0, 1, 1, 0, 2])
    for mode in (0, 1):
        b.case(f"t4_fanin_m{mode}", "fanin_reduce", ["t4_rel", "t4_src", "t4_dst"], [5, mode])
    b.arr("t4_g", np.ones((5, 3), dtype=np.float32))
    b.case("t4_fanin_sum_bwd", "fanin_reduce_sum_backward", ["t4_g", "t4_src", "t4_dst"], [12])
    # test_python_fallback_path (:176-186)
    b.randn("t5_x", (6, 3))
    b.idx("t5_src", [0, 4, 1])
    b.idx("t5_dst", [3, 0, 1])
    b.case("t5_fanout", "fanout_scatter", ["t5_x", "t5_src", "t5_dst"], [5])
    b.randn("t5_rel", (8, 3))
    b.idx("t5_fsrc", [0, 2, 4, 1])
    b.idx("t5_fdst", [2, 0, 1, 0])
    for mode in (0, 1):
        b.case(f"t5_fanin_m{mode}", "fanin_reduce", ["t5_rel", "t5_fsrc", "t5_fdst"], [4, mode])
    # gradcheck vectors in float64 (:308-342)
    b.randn("t6_x", (6, 3), np.float64)
    b.idx("t6_src", [0, 5, 2, 1])
    b.idx("t6_dst", [1, 0, 3, 2])
    b.case("t6_fanout_f64", "fanout_scatter", ["t6_x", "t6_src", "t6_dst"], [5])
    b.randn("t7_rel", (8, 4), np.float64)
    b.idx("t7_src", [0, 2, 5, 7, 1])
    b.idx("t7_dst", [1, 0, 3, 2, 0])
    b.case("t7_fanin_sum_f64", "fanin_reduce", ["t7_rel", "t7_src", "t7_dst"], [5, 0])
    b.idx("t8_src", [0, 2, 5, 7, 1, 3])
    b.idx("t8_dst", [1, 0, 3, 2, 0, 1])
    b.case("t8_fanin_lse_f64", "fanin_reduce", ["t7_rel", "t8_src", "t8_dst"], [4, 1])
    # noncontiguous input (:292-296): the values of base.T, stored contiguous
    base = b.rng.standard_normal((4, 6)).astype(np.float32)
    b.arr("t9_x", base.T.copy())
    b.idx("t9_src", [0, 4, 2, 5])
    b.idx("t9_dst", [2, 1, 0, 3])
    b.case("t9_fanout", "fanout_scatter", ["t9_x", "t9_src", "t9_dst"], [5])


def add_edge_cases(b: Builder) -> None:
    """Duplicates, empty rows, long segments, special values, bounds errors."""

    # duplicated flat_dst: the last edge wins
    b.randn("e1_x", (9, 6))
    b.idx("e1_src", [1, 2, 3, 4, 5, 6, 7])
    b.idx("e1_dst", [0, 3, 0, 3, 5, 0, 2])
    b.case("e1_fanout_dup", "fanout_scatter", ["e1_x", "e1_src", "e1_dst"], [7])
    b.randn("e1_g", (7, 6))
    b.case("e1_fanout_bwd_dup", "fanout_scatter_backward", ["e1_g", "e1_src", "e1_dst"], [9])
    # duplicated flat_src in the sum backward; dst rows without messages
    b.randn("e2_rel", (20, 5))
    b.idx("e2_src", [3, 3, 7, 1, 3, 7, 19, 0])
    b.idx("e2_dst", [0, 2, 2, 5, 2, 0, 5, 6])
    for mode in (0, 1):
        b.case(f"e2_fanin_m{mode}", "fanin_reduce", ["e2_rel", "e2_src", "e2_dst"], [8, mode])
    b.randn("e2_g", (8, 5))
    b.case("e2_fanin_sum_bwd_dup", "fanin_reduce_sum_backward", ["e2_g", "e2_src", "e2_dst"], [20])
    # long segments (hub path: > 64 messages to one row), D = 32
    n = 700
    b.randn("e3_rel", (n, 32), scale=2.0)
    dst = np.where(b.rng.random(n) < 0.6, 2, b.rng.integers(0, 11, n))
    dst[:5] = 9
    b.idx("e3_src", b.rng.permutation(n))
    b.idx("e3_dst", dst)
    for mode in (0, 1):
        b.case(f"e3_fanin_hub_m{mode}", "fanin_reduce", ["e3_rel", "e3_src", "e3_dst"], [11, mode])
    b.randn("e3_g", (11, 32))
    b.case("e3_fanin_sum_bwd", "fanin_reduce_sum_backward", ["e3_g", "e3_src", "e3_dst"], [n])
    b.idx("e3_fsrc", b.rng.integers(0, 50, n))
    b.idx("e3_fdst", b.rng.permutation(n))
    b.randn("e3_gx", (n, 32))
    b.case("e3_fanout_bwd_hub", "fanout_scatter_backward", ["e3_gx", "e3_fsrc", "e3_fdst"], [50])
    # logsumexp special values: -inf rows, +inf, NaN
    rel = b.rng.standard_normal((12, 4)).astype(np.float32)
    rel[0, :] = -np.inf
    rel[1, :] = -np.inf
    rel[2, 0] = np.inf
    rel[3, 1] = np.nan
    rel[4, 2] = -np.inf
    b.arr("e4_rel", rel)
    b.idx("e4_src", [0, 1, 2, 5, 3, 6, 4, 7, 8])
    b.idx("e4_dst", [0, 0, 1, 1, 2, 2, 3, 3, 3])
    b.case("e4_lse_special", "fanin_reduce", ["e4_rel", "e4_src", "e4_dst"], [5, 1])
    b.case("e4_sum_special", "fanin_reduce", ["e4_rel", "e4_src", "e4_dst"], [5, 0])
    # NaN or -inf in the leading messages of a segment, finite ones after them
    # (a NaN anywhere makes the logsumexp NaN; -inf messages add nothing)
    lead = b.rng.standard_normal((20, 4)).astype(np.float32)
    lead[0:4, :] = -np.inf
    lead[0, 0] = np.nan
    lead[2, 2] = np.nan
    b.arr("e9_rel", lead)
    b.idx("e9_src", np.arange(20))
    b.idx("e9_dst", np.zeros(20, dtype=np.int64))
    b.case("e9_lse_nan_lead", "fanin_reduce", ["e9_rel", "e9_src", "e9_dst"], [1, 1])
    hub = b.rng.standard_normal((300, 32)).astype(np.float32)
    hub[:256, :] = -np.inf
    hub[17, 3] = np.nan
    hub[299, 5] = np.nan
    b.arr("e9_hub", hub)
    b.idx("e9_hsrc", np.arange(300))
    b.idx("e9_hdst", np.zeros(300, dtype=np.int64))
    b.case("e9_lse_nan_hub", "fanin_reduce", ["e9_hub", "e9_hsrc", "e9_hdst"], [2, 1])
    # widths that are not multiples of the vector width
    for d in (1, 3, 7, 65):
        b.randn(f"e5_x{d}", (13, d))
        b.idx(f"e5_src{d}", b.rng.integers(0, 13, 40))
        b.idx(f"e5_dst{d}", b.rng.integers(0, 9, 40))
        b.case(f"e5_fanin_sum_d{d}", "fanin_reduce", [f"e5_x{d}", f"e5_src{d}", f"e5_dst{d}"], [9, 0])
        b.case(f"e5_fanin_lse_d{d}", "fanin_reduce", [f"e5_x{d}", f"e5_src{d}", f"e5_dst{d}"], [9, 1])
    # logsumexp backward (injective and duplicated flat_src)
    b.randn("e6_rel", (16, 8))
    b.idx("e6_src", [4, 9, 1, 15, 0, 7])
    b.idx("e6_dst", [0, 2, 2, 1, 0, 0])
    b.case("e6_lse_fwd", "fanin_reduce", ["e6_rel", "e6_src", "e6_dst"], [3, 1])
    b.idx("e6_src_dup", [4, 9, 4, 15, 9, 4])
    b.case("e6_lse_fwd_dup", "fanin_reduce", ["e6_rel", "e6_src_dup", "e6_dst"], [3, 1])
    # bounds errors (message and check order)
    b.idx("e7_bad_src", [0, 3, 9, 2, 3])
    b.idx("e7_bad_dst", [4, 1, 0, 8, 3])
    b.case("e7_err_fanout_src", "fanout_scatter", ["t1_x", "e7_bad_src", "t1_dst"], [6])
    b.case("e7_err_fanout_dst", "fanout_scatter", ["t1_x", "t1_src", "e7_bad_dst"], [6])
    b.case("e7_err_fanout_both", "fanout_scatter", ["t1_x", "e7_bad_src", "e7_bad_dst"], [6])
    b.idx("e7_neg", [0, 2, -1, 5, 2, 1])
    b.case("e7_err_fanin_neg_src", "fanin_reduce", ["t3_rel", "e7_neg", "t3_dst"], [4, 0])
    b.idx("e7_big_dst", [1, 0, 2, 4, 1, 0])
    b.case("e7_err_fanin_dst", "fanin_reduce", ["t3_rel", "t3_src", "e7_big_dst"], [4, 0])
    b.case("e7_err_fanout_bwd", "fanout_scatter_backward", ["t1_g", "e7_bad_src", "e7_bad_dst"], [7])
    b.case("e7_err_sum_bwd", "fanin_reduce_sum_backward", ["t3_g", "e7_neg", "e7_big_dst"], [10])
    b.case("e7_err_mode", "fanin_reduce", ["t3_rel", "t3_src", "t3_dst"], [4, 2])
    # logsumexp runs as ATen calls in the reference's CPU lane: their errors, in call order
    b.case("e7_err_lse_neg_src", "fanin_reduce", ["t3_rel", "e7_neg", "t3_dst"], [4, 1])
    b.case("e7_err_lse_dst", "fanin_reduce", ["t3_rel", "t3_src", "e7_big_dst"], [4, 1])
    b.case("e7_err_lse_both", "fanin_reduce", ["t3_rel", "e7_neg", "e7_big_dst"], [4, 1])
    # empty inputs
    b.arr("e8_empty_idx", np.zeros(0, dtype=np.int64))
    b.case("e8_fanout_empty", "fanout_scatter", ["t1_x", "e8_empty_idx", "e8_empty_idx"], [6])
    b.case("e8_fanin_lse_empty", "fanin_reduce", ["t3_rel", "e8_empty_idx", "e8_empty_idx"], [4, 1])
    b.case("e8_fanout_zero_rows", "fanout_scatter", ["t1_x", "e8_empty_idx", "e8_empty_idx"], [0])


def add_logsumexp_backward_cases(b: Builder, outputs: dict[str, np.ndarray]) -> None:
    """Backward of the logsumexp forward cases, fed the reference's own forward
    output (the saved ``out``, mp_autograd.py:175) and a seeded upstream gradient."""

    forward = {
        "t3_fanin_m1": ("t3_rel", "t3_src", "t3_dst"),
        "t4_fanin_m1": ("t4_rel", "t4_src", "t4_dst"),
        "e3_fanin_hub_m1": ("e3_rel", "e3_src", "e3_dst"),
        "e6_lse_fwd": ("e6_rel", "e6_src", "e6_dst"),
        "e6_lse_fwd_dup": ("e6_rel", "e6_src_dup", "e6_dst"),
        "t8_fanin_lse_f64": ("t7_rel", "t8_src", "t8_dst"),
    }
    new_cases = []
    for fwd_name, (rel, src, dst) in forward.items():
        out = outputs["expected_" + fwd_name]
        out_name = b.arr(f"{fwd_name}_out", out)
        g_name = b.arr(f"{fwd_name}_gout", b.rng.standard_normal(out.shape).astype(out.dtype))
        rel_rows = b.arrays[rel].shape[0]
        new_cases.append({"name": f"{fwd_name}_bwd", "op": "fanin_reduce_logsumexp_backward",
                          "tensors": [g_name, rel, src, dst, out_name], "ints": [rel_rows]})
    calls = [{"op": c["op"], "tensors": c["tensors"], "ints": c["ints"]} for c in new_cases]
    for case, res in zip(new_cases, ref_runner.run_reference(calls, b.arrays)):
        assert "error" not in res, res
        outputs["expected_" + case["name"]] = res["out"]
        case["expected"] = "expected_" + case["name"]
        b.cases.append(case)
    # bad indices in the backward (e6: 16 rel rows, 3 objects, 6 messages): a
    # message row past rel_flat, an object past out, a message row inside
    # rel_flat but past rel_rows
    b.idx("e9_src_past_rel", [4, 9, 1, 16, 0, 7])
    b.idx("e9_dst_past_out", [0, 2, 3, 1, 0, 0])
    errors = [
        ("e9_err_lse_bwd_src", ["e6_lse_fwd_gout", "e6_rel", "e9_src_past_rel", "e6_dst", "e6_lse_fwd_out"], [16]),
        ("e9_err_lse_bwd_dst", ["e6_lse_fwd_gout", "e6_rel", "e6_src", "e9_dst_past_out", "e6_lse_fwd_out"], [16]),
        ("e9_err_lse_bwd_rows", ["e6_lse_fwd_gout", "e6_rel", "e6_src", "e6_dst", "e6_lse_fwd_out"], [8]),
    ]
    calls = [{"op": "fanin_reduce_logsumexp_backward", "tensors": t, "ints": i} for _n, t, i in errors]
    for (name, tensors, ints), res in zip(errors, ref_runner.run_reference(calls, b.arrays)):
        assert "error" in res, (name, res)
        b.cases.append({"name": name, "op": "fanin_reduce_logsumexp_backward", "tensors": tensors,
                        "ints": ints, "error": res["error"], "error_type": res["error_type"]})


def main() -> None:
    b = Builder(seed=20261201)
    add_reference_test_vectors(b)
    add_edge_cases(b)
    calls = [{"op": c["op"], "tensors": c["tensors"], "ints": c["ints"]} for c in b.cases]
    results = ref_runner.run_reference(calls, b.arrays)
    outputs = {}
    for case, res in zip(b.cases, results):
        if "error" in res:
            case["error"] = res["error"]
            case["error_type"] = res["error_type"]
        else:
            name = "expected_" + case["name"]
            outputs[name] = res["out"]
            case["expected"] = name
    add_logsumexp_backward_cases(b, outputs)
    np.savez_compressed(HERE / "reference_cases.npz", **b.arrays, **outputs)
    (HERE / "reference_cases.json").write_text(json.dumps(b.cases, indent=1) + "\n")

    # C1 (op micro-bench, CPU-runnable): digests of the reference outputs.
    arrays = c1_inputs()
    c1_calls = [
        {"op": "fanout_scatter", "tensors": ["x", "src", "flat_dst"], "ints": [arrays["src"].size]},
        {"op": "fanout_scatter_backward", "tensors": ["grad_slots", "src", "flat_dst"], "ints": [arrays["x"].shape[0]]},
        {"op": "fanin_reduce", "tensors": ["rel", "flat_src", "dst"], "ints": [arrays["x"].shape[0], 0]},
        {"op": "fanin_reduce_sum_backward", "tensors": ["grad_obj", "flat_src", "dst"], "ints": [arrays["rel"].shape[0]]},
    ]
    res = ref_runner.run_reference(c1_calls, arrays)
    digests = {
        c["op"]: hashlib.sha256(np.ascontiguousarray(r["out"]).tobytes()).hexdigest()
        for c, r in zip(c1_calls, res)
    }
    (HERE / "c1_digests.json").write_text(json.dumps(digests, indent=1) + "\n")
    print(f"{len(b.cases)} cases, {len(outputs)} outputs; C1 digests: {len(digests)}")


if __name__ == "__main__":
    main()
