"""Runs relmo's own CPU op library (``oracle/_ref/relm_mp_ops_ref.so``, built by
``make -C oracle ref`` from the reference's ``src/_ops/mp/mp_ops.cpp``) in a
child process.

TEST INFRASTRUCTURE ONLY (golden fixtures, oracle pinning, bench.py's
``cpu_baseline``).  The reference library registers the same
``torch.ops.relm_mp`` namespace as the product library, so it always runs in
its own process.  Arrays travel as ``.npz`` (no pickle), parameters as JSON.

Parent side:  ``run_reference(calls, arrays)``
Child side:   ``python oracle/ref_runner.py <request_dir>``
"""

from __future__ import annotations

import json
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF_LIB = HERE / "_ref" / "relm_mp_ops_ref.so"

OPS = {
    "fanout_scatter": 3,
    "fanout_scatter_backward": 3,
    "fanin_reduce": 3,
    "fanin_reduce_sum_backward": 3,
    "fanin_reduce_logsumexp_backward": 5,
    # list-argument ops: called with "args" (see run_reference)
    "fanout_pack_multi": 0,
    "fanin_pack_multi": 0,
    "fanout_pack_from_edges": 0,
    "fanin_pack_from_edges": 0,
    "lgan_pool_reduce": 0,
    "lgan_pool_reduce_backward": 0,
    "lgan_relation_graph_step": 0,
    "lgan_relation_graph_step_backward": 0,
}


def available() -> bool:
    return REF_LIB.exists()


def run_reference(calls: list[dict], arrays: dict[str, np.ndarray], timeout: float = 600.0) -> list[dict]:
    """Each call: {"op", "tensors": [names], "ints": [...], optional "repeat",
    "warmup", "threads", "keep"}, or {"op", "args": [spec, ...]} with each spec
    one of {"tensor": name}, {"tensors": [names]}, {"int": v}, {"ints": [v, ...]}.
    Returns per call {"out": ndarray} ({"outs": [ndarray, ...]} for an op
    returning a tuple; neither with "keep": false, for timing runs) or
    {"error": str}, plus "times" (seconds per repetition) when "repeat" is
    given."""

    if not available():
        raise FileNotFoundError(f"{REF_LIB} is missing; run `make -C oracle ref` where the reference is present")
    with tempfile.TemporaryDirectory(prefix="relm_ref_") as tmp:
        tmpd = Path(tmp)
        np.savez(tmpd / "inputs.npz", **arrays)
        (tmpd / "request.json").write_text(json.dumps(calls))
        # the child's stderr passes through: timing runs report each call
        proc = subprocess.run(
            [sys.executable, str(Path(__file__).resolve()), str(tmpd)],
            stdout=subprocess.PIPE, text=True, timeout=timeout,
        )
        if proc.returncode != 0:
            raise RuntimeError(f"reference runner failed (exit {proc.returncode}):\n{proc.stdout}")
        meta = json.loads((tmpd / "result.json").read_text())
        outs = np.load(tmpd / "outputs.npz", allow_pickle=False)
        results = []
        for i, m in enumerate(meta):
            r = dict(m)
            if f"out_{i}" in outs.files:
                r["out"] = outs[f"out_{i}"]
            if "num_outs" in r:
                r["outs"] = [outs[f"out_{i}_{k}"] for k in range(r["num_outs"])]
            results.append(r)
        return results


def _child(req_dir: Path) -> None:
    import torch

    torch.ops.load_library(str(REF_LIB))
    ns = torch.ops.relm_mp
    calls = json.loads((req_dir / "request.json").read_text())
    arrays = np.load(req_dir / "inputs.npz", allow_pickle=False)
    outputs: dict[str, np.ndarray] = {}
    meta: list[dict] = []
    for i, call in enumerate(calls):
        op = call["op"]
        if op not in OPS:
            raise ValueError(f"unknown op {op}")
        def tensor(name):
            return torch.from_numpy(np.array(arrays[name]))

        if "args" in call:
            tensors, ints = [], []
            for spec in call["args"]:
                if "tensor" in spec:
                    tensors.append(tensor(spec["tensor"]))
                elif "tensors" in spec:
                    tensors.append([tensor(n) for n in spec["tensors"]])
                elif "int" in spec:
                    tensors.append(int(spec["int"]))
                else:
                    tensors.append([int(v) for v in spec["ints"]])
        else:
            tensors = [tensor(name) for name in call["tensors"]]
            ints = [int(v) for v in call.get("ints", [])]
        threads = call.get("threads")
        if threads:
            torch.set_num_threads(int(threads))
        entry: dict = {"op": op, "threads": torch.get_num_threads()}
        fn = getattr(ns, op)
        try:
            t0 = time.perf_counter()
            out = fn(*tensors, *ints)
            first = time.perf_counter() - t0
        except Exception as exc:  # the reference's error is part of the result
            entry["error"] = str(exc).splitlines()[0]
            entry["error_type"] = type(exc).__name__
            meta.append(entry)
            continue
        if not call.get("keep", True):
            pass
        elif isinstance(out, (tuple, list)):
            entry["num_outs"] = len(out)
            for k, o in enumerate(out):
                outputs[f"out_{i}_{k}"] = o.detach().numpy()
        else:
            outputs[f"out_{i}"] = out.numpy()
        repeat = int(call.get("repeat", 0))
        if repeat:
            warmup = int(call.get("warmup", 1))
            for _ in range(warmup):
                fn(*tensors, *ints)
            # without warmup the output-producing call is the first timed one
            times = [] if warmup else [first]
            while len(times) < repeat:
                t0 = time.perf_counter()
                fn(*tensors, *ints)
                times.append(time.perf_counter() - t0)
            entry["times"] = times
            print(f"reference {op}: {len(times)} timed calls at {entry['threads']} threads, "
                  f"median {sorted(times)[len(times) // 2]:.4f} s", file=sys.stderr, flush=True)
        meta.append(entry)
    np.savez(req_dir / "outputs.npz", **outputs)
    (req_dir / "result.json").write_text(json.dumps(meta))


if __name__ == "__main__":
    _child(Path(sys.argv[1]))
