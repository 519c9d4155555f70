"""Seeded synthetic inputs of the op benchmark configurations.

C1  op micro-bench: X [4096, 32]; 3 predicates x arity 2 x 16,384 atoms =
    98,304 slots with uniform object arguments.
C2  fanin logsumexp: 1,048,576 objects, D = 32, 16,777,216 messages ~ N(0, 2^2)
    (sigma = 2; the config's "N(0, 2)" read as a standard deviation), message i
    read from rel row i (flat_src = arange), destinations Zipf(s = 1.1) over
    object ranks through a seeded permutation of object ids, unsorted.
C3  fanout: X [2,097,152, 64]; predicates of arity 1, 2, 2, 3 with 2,097,152
    atoms each = 16,777,216 slots with uniform arguments, flat_dst = arange.

Generated directly on the target device with torch generators (no host copy).
"""

from __future__ import annotations

import torch


def zipf_destinations(num_keys: int, num_edges: int, s: float, gen: torch.Generator, device) -> torch.Tensor:
    """Truncated Zipf(s) over ranks 1..num_keys by inverse-CDF sampling, mapped
    to object ids through a random permutation (so hubs are scattered)."""

    ranks = torch.arange(1, num_keys + 1, dtype=torch.float64, device=device)
    cdf = torch.cumsum(ranks.pow(-s), 0)
    cdf /= cdf[-1].clone()
    u = torch.rand(num_edges, dtype=torch.float64, device=device, generator=gen)
    r = torch.searchsorted(cdf, u, right=True).clamp_(max=num_keys - 1)
    perm = torch.randperm(num_keys, device=device, generator=gen)
    return perm[r]


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def c2_fanin(device, seed: int = 0, num_keys: int = 1 << 20, num_edges: int = 1 << 24, emb: int = 32,
             sigma: float = 2.0) -> dict[str, torch.Tensor | int]:
    gen = _gen(device, seed)
    rel = torch.randn(num_edges, emb, device=device, generator=gen).mul_(sigma)
    dst = zipf_destinations(num_keys, num_edges, 1.1, gen, device)
    flat_src = torch.arange(num_edges, device=device)
    grad_out = torch.randn(num_keys, emb, device=device, generator=gen)
    return {"rel": rel, "flat_src": flat_src, "dst": dst, "grad_out": grad_out, "dim_size": num_keys}


def c3_fanout(device, seed: int = 0, x_rows: int = 1 << 21, atoms: int = 1 << 21, emb: int = 64,
              arities: tuple[int, ...] = (1, 2, 2, 3)) -> dict[str, torch.Tensor | int]:
    gen = _gen(device, seed)
    slots = atoms * sum(arities)
    x = torch.randn(x_rows, emb, device=device, generator=gen)
    src = torch.randint(0, x_rows, (slots,), device=device, generator=gen)
    flat_dst = torch.arange(slots, device=device)
    grad_out = torch.randn(slots, emb, device=device, generator=gen)
    return {"x": x, "src": src, "flat_dst": flat_dst, "grad_out": grad_out, "out_rows": slots}


def c1_ops(device, seed: int = 0) -> dict[str, torch.Tensor | int]:
    gen = _gen(device, seed)
    objects, emb, slots = 4096, 32, 3 * 2 * 16384
    x = torch.randn(objects, emb, device=device, generator=gen)
    src = torch.randint(0, objects, (slots,), device=device, generator=gen)
    flat = torch.arange(slots, device=device)
    rel = torch.randn(slots, emb, device=device, generator=gen)
    return {"x": x, "src": src, "flat_dst": flat, "rel": rel, "flat_src": flat, "dst": src,
            "grad_slots": torch.randn(slots, emb, device=device, generator=gen),
            "grad_obj": torch.randn(objects, emb, device=device, generator=gen),
            "objects": objects, "slots": slots}


# Algorithmic bytes (fp32 values, int64 indices; each index array read once,
# gathered rows once per message, keyed / output rows once).
def bytes_fanout_fwd(E: int, D: int, out_rows: int) -> int:
    return 4 * E * D + 4 * out_rows * D + 16 * E


def bytes_fanout_bwd(E: int, D: int, x_rows: int) -> int:
    return 4 * E * D + 4 * x_rows * D + 16 * E


def bytes_fanin_fwd(E: int, D: int, K: int) -> int:
    return 4 * E * D + 4 * K * D + 16 * E


def bytes_fanin_sum_bwd(E: int, D: int, K: int, R: int) -> int:
    return 4 * K * D + 4 * R * D + 16 * E


def bytes_fanin_lse_bwd(E: int, D: int, K: int, R: int) -> int:
    return 4 * E * D + 8 * K * D + 4 * R * D + 16 * E
