"""Writes the LGAN-op golden fixtures under tests/golden/ from relmo's own CPU op library.

Expected outputs and error messages come from ``oracle/_ref/relm_mp_ops_ref.so``
(the reference's ``src/_ops/mp/mp_ops.cpp`` compiled unchanged by ``make -C
oracle ref``) through ``oracle/ref_runner.py``: ``lgan_pool_reduce``,
``lgan_relation_graph_step`` and their backward ops in sum (0) and mean (2)
mode, float32 and float64, int64 and int32 indices, duplicates, destinations
with more than 64 messages, empty index sets, zero / negative arities, no
entities, and invalid arguments (message and order of the checks).

Run from the repository root where /root/reference is present:
    python tests/golden/make_lgan_golden.py
Outputs: tests/golden/lgan_cases.npz and tests/golden/lgan_cases.json (same
layout as pack_cases.*).
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

IDX = ("rr_src", "rr_dst", "tn_rel", "tn_ent", "nn_rel", "nn_ent")


class Builder:
    def __init__(self, seed: int):
        self.rng = np.random.default_rng(seed)
        self.arrays: dict[str, np.ndarray] = {}
        self.cases: list[dict] = []

    def put(self, name: str, value) -> str:
        self.arrays[name] = np.ascontiguousarray(value)
        return name

    def case(self, name: str, op: str, tensors: list[str], ints: list[int]) -> None:
        args = [{"tensor": t} for t in tensors] + [{"int": int(v)} for v in ints]
        self.cases.append({"name": name, "op": op, "args": args})


def graph(b: Builder, tag: str, K: int, ent: int, E_slots: int, n_rr: int, n_tn: int, n_nn: int,
          D: int, dtype, idx_dtype=np.int64, hub: bool = False) -> dict[str, str]:
    rng = b.rng
    g = {
        "slot": b.put(f"{tag}_slot", (2 * rng.standard_normal((E_slots, D))).astype(dtype)),
        "s2r": b.put(f"{tag}_s2r", rng.integers(0, max(K, 1), E_slots).astype(idx_dtype)),
        "arity": b.put(f"{tag}_arity", rng.integers(-1, 4, K).astype(np.int64)),
        "x": b.put(f"{tag}_x", rng.standard_normal((K, D)).astype(dtype)),
    }
    sizes = {"rr": (n_rr, K, K), "tn": (n_tn, K, ent), "nn": (n_nn, K, ent)}
    for kind, (n, src_bound, dst_bound) in sizes.items():
        src = rng.integers(0, max(src_bound, 1), n)
        dst = rng.integers(0, max(dst_bound, 1), n)
        if hub and n > 200:
            dst[: n // 2] = 0  # one destination with more than 64 messages
        names = {"rr": ("rr_src", "rr_dst"), "tn": ("tn_rel", "tn_ent"), "nn": ("nn_rel", "nn_ent")}[kind]
        g[names[0]] = b.put(f"{tag}_{names[0]}", src.astype(idx_dtype))
        g[names[1]] = b.put(f"{tag}_{names[1]}", dst.astype(idx_dtype))
    g["g_rpx"] = b.put(f"{tag}_g_rpx", rng.standard_normal((K, D)).astype(dtype))
    g["g_tn"] = b.put(f"{tag}_g_tn", rng.standard_normal((ent, D)).astype(dtype))
    g["g_nn"] = b.put(f"{tag}_g_nn", rng.standard_normal((ent, D)).astype(dtype))
    return g


def add_all_ops(b: Builder, tag: str, g: dict, K: int, ent: int, modes=(0, 2)) -> None:
    idx = [g[n] for n in IDX]
    for mode in modes:
        b.case(f"{tag}_pool_m{mode}", "lgan_pool_reduce", [g["slot"], g["s2r"], g["arity"], *idx],
               [ent, mode])
        b.case(f"{tag}_pool_bwd_m{mode}", "lgan_pool_reduce_backward",
               [g["g_rpx"], g["g_tn"], g["g_nn"], g["s2r"], g["arity"], *idx], [K, mode])
        b.case(f"{tag}_step_m{mode}", "lgan_relation_graph_step", [g["x"], *idx], [ent, mode])
        b.case(f"{tag}_step_bwd_m{mode}", "lgan_relation_graph_step_backward",
               [g["g_rpx"], g["g_tn"], g["g_nn"], *idx], [K, mode])


def add_cases(b: Builder) -> None:
    g = graph(b, "a", K=40, ent=25, E_slots=90, n_rr=120, n_tn=80, n_nn=70, D=5, dtype=np.float32)
    add_all_ops(b, "a", g, 40, 25)
    g = graph(b, "b", K=300, ent=64, E_slots=700, n_rr=2000, n_tn=1500, n_nn=900, D=16,
              dtype=np.float32, hub=True)
    add_all_ops(b, "b", g, 300, 64)
    g = graph(b, "c", K=50, ent=30, E_slots=120, n_rr=150, n_tn=100, n_nn=90, D=3,
              dtype=np.float64, idx_dtype=np.int32)
    add_all_ops(b, "c", g, 50, 30)
    # empty index sets, no entities, no slots
    e = graph(b, "e", K=20, ent=10, E_slots=0, n_rr=0, n_tn=30, n_nn=0, D=4, dtype=np.float32)
    add_all_ops(b, "e", e, 20, 10)
    z = graph(b, "z", K=12, ent=0, E_slots=30, n_rr=40, n_tn=0, n_nn=0, D=2, dtype=np.float32)
    add_all_ops(b, "z", z, 12, 0)


def add_errors(b: Builder) -> None:
    g = graph(b, "r", K=10, ent=6, E_slots=20, n_rr=15, n_tn=12, n_nn=9, D=3, dtype=np.float32)
    idx = [g[n] for n in IDX]
    i16 = b.put("r_i16", np.zeros(15, np.int16))
    a32 = b.put("r_arity32", np.ones(10, np.int32))
    short = b.put("r_short", np.zeros(3, np.int64))
    bad_hi = b.put("r_bad_hi", np.full(12, 6, np.int64))
    v1d = b.put("r_v1d", np.zeros(10, np.float32))
    pool = lambda *t: [t[0], g["s2r"], g["arity"], *t[1:]]  # noqa: E731
    b.case("err_pool_mode1", "lgan_pool_reduce", pool(g["slot"], *idx), [6, 1])
    b.case("err_pool_rank", "lgan_pool_reduce", pool(v1d, *idx), [6, 0])
    b.case("err_pool_arity_dtype", "lgan_pool_reduce", [g["slot"], g["s2r"], a32, *idx], [6, 0])
    b.case("err_pool_idx_dtype", "lgan_pool_reduce", pool(g["slot"], i16, *idx[1:]), [6, 0])
    b.case("err_pool_slot_len", "lgan_pool_reduce", [g["slot"], short, g["arity"], *idx], [6, 0])
    b.case("err_pool_tn_len", "lgan_pool_reduce", pool(g["slot"], *idx[:2], short, *idx[3:]), [6, 0])
    b.case("err_pool_nn_len", "lgan_pool_reduce", pool(g["slot"], *idx[:4], short, idx[5]), [6, 0])
    b.case("err_pool_rr_len", "lgan_pool_reduce", pool(g["slot"], short, *idx[1:]), [6, 0])
    b.case("err_pool_ent_neg", "lgan_pool_reduce", pool(g["slot"], *idx), [-1, 0])
    b.case("err_pool_tn_ent_range", "lgan_pool_reduce", pool(g["slot"], *idx[:3], bad_hi, *idx[4:]), [6, 0])
    b.case("err_step_mode", "lgan_relation_graph_step", [g["x"], *idx], [6, 3])
    b.case("err_step_rank", "lgan_relation_graph_step", [v1d, *idx], [6, 0])
    b.case("err_step_rr_len", "lgan_relation_graph_step", [g["x"], short, *idx[1:]], [6, 0])
    b.case("err_step_ent_neg", "lgan_relation_graph_step", [g["x"], *idx], [-2, 2])
    bwd = [g["g_rpx"], g["g_tn"], g["g_nn"]]
    b.case("err_step_bwd_mode", "lgan_relation_graph_step_backward", [*bwd, *idx], [10, 1])
    b.case("err_step_bwd_count", "lgan_relation_graph_step_backward", [*bwd, *idx], [-1, 0])
    b.case("err_step_bwd_rank", "lgan_relation_graph_step_backward", [v1d, *bwd[1:], *idx], [10, 0])
    b.case("err_pool_bwd_mode", "lgan_pool_reduce_backward", [*bwd, g["s2r"], g["arity"], *idx], [10, 5])
    b.case("err_pool_bwd_arity", "lgan_pool_reduce_backward", [*bwd, g["s2r"], a32, *idx], [10, 0])


def main() -> None:
    b = Builder(seed=20261203)
    add_cases(b)
    add_errors(b)
    calls = [{"op": c["op"], "args": c["args"]} for c in b.cases]
    outputs: dict[str, np.ndarray] = {}
    for case, res in zip(b.cases, ref_runner.run_reference(calls, b.arrays)):
        if "error" in res:
            case["error"] = res["error"]
            case["error_type"] = res["error_type"]
            continue
        outs = res["outs"] if "outs" in res else [res["out"]]
        case["expected"] = []
        for k, out in enumerate(outs):
            case["expected"].append(f"expected_{case['name']}_{k}")
            outputs[case["expected"][-1]] = out
    np.savez_compressed(HERE / "lgan_cases.npz", **b.arrays, **outputs)
    (HERE / "lgan_cases.json").write_text(json.dumps(b.cases, indent=1) + "\n")
    n_err = sum("error" in c for c in b.cases)
    print(f"{len(b.cases)} LGAN cases ({n_err} errors), {len(outputs)} outputs")


if __name__ == "__main__":
    main()
