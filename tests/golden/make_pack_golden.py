"""Writes the pack-op golden fixtures under tests/golden/ from relmo's own CPU op library.

The expected outputs and error messages come from
``oracle/_ref/relm_mp_ops_ref.so`` (the reference's ``src/_ops/mp/mp_ops.cpp``
compiled unchanged by ``make -C oracle ref``) through
``oracle/ref_runner.py``.  Cases: the inputs of the reference's pack tests
(tests/python/test_mp_ops.py:353-600), seeded multi-part layouts (empty parts,
more than 16 parts, one part, int64 wrap-around, negative entries) and
invalid arguments (message and order of the checks).

Run from the repository root where /root/reference is present:
    python tests/golden/make_pack_golden.py
Outputs: tests/golden/pack_cases.npz (arrays) and tests/golden/pack_cases.json
(cases: op, argument specs as taken by ref_runner.run_reference, expected
output names or the error's first line).
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

from oracle import ref_runner  # noqa: E402


class Builder:
    def __init__(self, seed: int):
        self.rng = np.random.default_rng(seed)
        self.arrays: dict[str, np.ndarray] = {}
        self.cases: list[dict] = []

    def put(self, name: str, value) -> str:
        self.arrays[name] = np.ascontiguousarray(value)
        return name

    def values(self, prefix: str, rows: list[int], emb: int = 3, dtype=np.float32) -> list[str]:
        return [self.put(f"{prefix}_v{i}", self.rng.standard_normal((r, emb)).astype(dtype))
                for i, r in enumerate(rows)]

    def index(self, prefix: str, parts: list) -> list[str]:
        return [self.put(f"{prefix}{i}", np.asarray(p, dtype=np.int64)) for i, p in enumerate(parts)]

    def multi(self, name: str, op: str, vals: list[str], first: list[str], second: list[str]) -> None:
        self.cases.append({"name": name, "op": op,
                           "args": [{"tensors": vals}, {"tensors": first}, {"tensors": second}]})

    def edges(self, name: str, op: str, vals, src, dst, ids, arity, pos, last) -> None:
        tail = {"ints": list(last)} if op == "fanout_pack_from_edges" else {"int": int(last)}
        self.cases.append({"name": name, "op": op, "args": [
            {"tensors": vals}, {"tensors": src}, {"tensors": dst}, {"ints": list(ids)},
            {"ints": list(arity)}, {"ints": list(pos)}, tail]})


def add_reference_test_inputs(b: Builder) -> None:
    xs = b.values("t1", [5, 4])
    b.multi("t1_fanout_multi", "fanout_pack_multi", xs, b.index("t1_s", [[0, 2, 4], [1, 3]]),
            b.index("t1_d", [[3, 1, 5], [0, 4]]))
    rels = b.values("t2", [6, 3], emb=4)
    b.multi("t2_fanin_multi", "fanin_pack_multi", rels, b.index("t2_s", [[0, 2, 5], [1, 2]]),
            b.index("t2_d", [[1, 0, 2], [2, 1]]))
    b.edges("t3_fanout_edges", "fanout_pack_from_edges", xs,
            b.index("t3_s", [[0, 2, 4], [1, 3], [2, 0]]), b.index("t3_d", [[1, 0, 2], [3, 1], [0, 2]]),
            [0, 1, 0], [2, 3, 2], [0, 1, 1], [0, 8, 0])
    b.edges("t4_fanin_edges_m1", "fanin_pack_from_edges", rels,
            b.index("t4_s", [[0, 2, 1], [1, 2]]), b.index("t4_d", [[1, 0, 2], [2, 1]]),
            [0, 1], [1, 1], [0, 0], 1)
    b.edges("t4_fanin_edges_m0", "fanin_pack_from_edges", rels,
            b.index("t4r_s", [[0, 2, 1], [0, 0]]), b.index("t4_d", [[1, 0, 2], [2, 1]]),
            [0, 1], [2, 3], [1, 2], 0)


def add_layouts(b: Builder) -> None:
    rng = b.rng
    for tag, n_values, n_parts, max_len in [("r1", 1, 1, 500), ("r5", 3, 5, 300),
                                           ("r20", 4, 20, 200), ("r40", 6, 40, 800)]:
        rows = [int(v) for v in rng.integers(1, 60, n_values)]
        vals = b.values(tag, rows, emb=int(rng.integers(1, 9)))
        lens = [int(v) for v in rng.integers(0, max_len, n_parts)]
        if n_parts > 2:
            lens[1] = 0
        ids = [int(v) for v in rng.integers(0, n_values, n_parts)]
        arity = [int(v) for v in rng.integers(1, 6, n_parts)]
        pos = [int(rng.integers(0, a)) for a in arity]
        slot = [int(v) for v in rng.integers(0, 1 << 40, n_parts)]
        src = b.index(f"{tag}_s", [rng.integers(0, rows[p], n) for p, n in zip(ids, lens)])
        dst = b.index(f"{tag}_d", [rng.integers(0, 5000, n) for n in lens])
        k = min(n_values, n_parts)
        b.multi(f"{tag}_fanout_multi", "fanout_pack_multi", vals[:k], src[:k], dst[:k])
        b.multi(f"{tag}_fanin_multi", "fanin_pack_multi", vals[:k], src[:k], dst[:k])
        b.edges(f"{tag}_fanout_edges", "fanout_pack_from_edges", vals, src, dst, ids, arity, pos, slot)
        for mode in (0, 1):
            b.edges(f"{tag}_fanin_edges_m{mode}", "fanin_pack_from_edges", vals, src, dst, ids,
                    arity, pos, mode)
    # no edge parts; negative entries and int64 wrap-around pass through the arithmetic
    vals = b.values("z", [3, 2])
    b.edges("z_fanout_no_edges", "fanout_pack_from_edges", vals, [], [], [], [], [], [])
    b.edges("z_fanin_no_edges", "fanin_pack_from_edges", vals, [], [], [], [], [], 0)
    big = b.index("w_d", [[-1, 2**62, 2**63 - 1, -(2**63)]])
    neg = b.index("w_s", [[-3, 0, 1, -(2**63)]])
    b.edges("w_fanout_wrap", "fanout_pack_from_edges", vals, neg, big, [1], [4], [3],
            [2**62])
    b.edges("w_fanin_wrap", "fanin_pack_from_edges", vals, big, neg, [1], [7], [6], 0)
    b.multi("w_fanin_multi_neg", "fanin_pack_multi", vals[1:], neg, big)


def add_errors(b: Builder) -> None:
    vals = b.values("e", [4, 3])
    v64 = b.put("e_v64", np.zeros((2, 3), np.float64))
    v_emb = b.put("e_vemb", np.zeros((2, 5), np.float32))
    v_rank = b.put("e_v1d", np.zeros(4, np.float32))
    s = b.index("e_s", [[0, 1], [2]])
    d = b.index("e_d", [[1, 0], [3]])
    i32 = b.put("e_i32", np.zeros(2, np.int32))
    i2d = b.put("e_i2d", np.zeros((2, 1), np.int64))
    short = b.put("e_short", np.zeros(1, np.int64))
    for op in ("fanout_pack_multi", "fanin_pack_multi"):
        b.multi(f"err_{op}_empty", op, [], [], [])
        b.multi(f"err_{op}_lengths", op, vals, s, d[:1])
        b.multi(f"err_{op}_rank0", op, [v_rank], s[:1], d[:1])
        b.multi(f"err_{op}_rank1", op, [vals[0], v_rank], s, d)
        b.multi(f"err_{op}_dtype", op, [vals[0], v64], s, d)
        b.multi(f"err_{op}_emb", op, [vals[0], v_emb], s, d)
        b.multi(f"err_{op}_int32_first", op, vals, [s[0], i32], d)
        b.multi(f"err_{op}_int32_second", op, vals, s, [d[0], i32])
        b.multi(f"err_{op}_2d_index", op, vals, [i2d, s[1]], d)
        b.multi(f"err_{op}_part_len", op, vals, s, [short, d[1]])
    fe, fi = "fanout_pack_from_edges", "fanin_pack_from_edges"
    b.edges("err_fe_empty", fe, [], s, d, [0, 1], [1, 1], [0, 0], [0, 0])
    b.edges("err_fe_lengths", fe, vals, s, d[:1], [0, 1], [1, 1], [0, 0], [0, 0])
    b.edges("err_fe_meta", fe, vals, s, d, [0], [1, 1], [0, 0], [0, 0])
    b.edges("err_fe_slot_meta", fe, vals, s, d, [0, 1], [1, 1], [0, 0], [0])
    b.edges("err_fe_dtype", fe, [vals[0], v64], s, d, [0, 1], [1, 1], [0, 0], [0, 0])
    b.edges("err_fe_emb", fe, [vals[0], v_emb], s, d, [0, 1], [1, 1], [0, 0], [0, 0])
    b.edges("err_fe_part_id", fe, vals, s, d, [0, 2], [1, 1], [0, 0], [0, 0])
    b.edges("err_fe_part_id_neg", fe, vals, s, d, [-1, 0], [1, 1], [0, 0], [0, 0])
    b.edges("err_fe_arity", fe, vals, s, d, [0, 1], [1, 0], [0, 0], [0, 0])
    b.edges("err_fe_pos", fe, vals, s, d, [0, 1], [2, 2], [0, 2], [0, 0])
    b.edges("err_fe_pos_neg", fe, vals, s, d, [0, 1], [2, 2], [-1, 0], [0, 0])
    b.edges("err_fe_int32", fe, vals, [s[0], i32], d, [0, 1], [1, 1], [0, 0], [0, 0])
    b.edges("err_fe_part_len", fe, vals, s, [short, d[1]], [0, 1], [1, 1], [0, 0], [0, 0])
    b.edges("err_fi_empty", fi, [], s, d, [0, 1], [1, 1], [0, 0], 0)
    b.edges("err_fi_mode", fi, vals, s, d, [0, 1], [1, 1], [0, 0], 2)
    b.edges("err_fi_lengths", fi, vals, s, d[:1], [0, 1], [1, 1], [0, 0], 0)
    b.edges("err_fi_meta", fi, vals, s, d, [0, 1], [1], [0, 0], 1)
    b.edges("err_fi_dtype", fi, [vals[0], v64], s, d, [0, 1], [1, 1], [0, 0], 0)
    b.edges("err_fi_emb", fi, [vals[0], v_emb], s, d, [0, 1], [1, 1], [0, 0], 0)
    b.edges("err_fi_part_id", fi, vals, s, d, [0, 5], [1, 1], [0, 0], 1)
    b.edges("err_fi_arity_m0", fi, vals, s, d, [0, 1], [1, 0], [0, 0], 0)
    b.edges("ok_fi_arity_m1", fi, vals, s, d, [0, 1], [0, -4], [7, -1], 1)
    b.edges("err_fi_pos_m0", fi, vals, s, d, [0, 1], [3, 3], [0, 3], 0)
    b.edges("err_fi_int32", fi, vals, s, [d[0], i32], [0, 1], [1, 1], [0, 0], 0)
    b.edges("err_fi_part_len", fi, vals, [s[0], short], d, [0, 1], [1, 1], [0, 0], 1)


def main() -> None:
    b = Builder(seed=20261202)
    add_reference_test_inputs(b)
    add_layouts(b)
    add_errors(b)
    calls = [{"op": c["op"], "args": c["args"]} for c in b.cases]
    outputs: dict[str, np.ndarray] = {}
    for case, res in zip(b.cases, ref_runner.run_reference(calls, b.arrays)):
        if "error" in res:
            case["error"] = res["error"]
            case["error_type"] = res["error_type"]
            continue
        names = []
        for k, out in enumerate(res["outs"]):
            names.append(f"expected_{case['name']}_{k}")
            outputs[names[-1]] = out
        case["expected"] = names
    np.savez_compressed(HERE / "pack_cases.npz", **b.arrays, **outputs)
    (HERE / "pack_cases.json").write_text(json.dumps(b.cases, indent=1) + "\n")
    n_err = sum("error" in c for c in b.cases)
    print(f"{len(b.cases)} pack cases ({n_err} errors), {len(outputs)} outputs")


if __name__ == "__main__":
    main()
