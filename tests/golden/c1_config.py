"""Seeded inputs of the CPU-runnable op micro-benchmark configuration (C1).

X [4096, 32] ~ N(0, 1); three predicates of arity 2 with 16384 atoms each give
98,304 atom-argument slots; each slot's object index is uniform over the 4096
objects (slot order: predicate, atom, position).  fanout_scatter gathers X
into the slots (flat_dst = arange); fanin_reduce(sum) sends random N(0, 1)
slot messages back to their argument objects (flat_src = arange, dst = the
slot's object).  numpy's PCG64 stream makes the inputs identical everywhere.
"""

from __future__ import annotations

import numpy as np

OBJECTS = 4096
EMB = 32
PREDICATES = 3
ARITY = 2
ATOMS = 16384
SLOTS = PREDICATES * ARITY * ATOMS  # 98,304


def c1_inputs(seed: int = 0) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((OBJECTS, EMB)).astype(np.float32)
    src = rng.integers(0, OBJECTS, SLOTS, dtype=np.int64)
    flat_dst = np.arange(SLOTS, dtype=np.int64)
    rel = rng.standard_normal((SLOTS, EMB)).astype(np.float32)
    grad_slots = rng.standard_normal((SLOTS, EMB)).astype(np.float32)
    grad_obj = rng.standard_normal((OBJECTS, EMB)).astype(np.float32)
    return {
        "x": x,
        "src": src,
        "flat_dst": flat_dst,
        "rel": rel,
        "flat_src": flat_dst.copy(),
        "dst": src.copy(),
        "grad_slots": grad_slots,
        "grad_obj": grad_obj,
    }
