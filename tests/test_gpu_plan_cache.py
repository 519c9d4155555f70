"""GPU tests of plan reuse by index content: the C ABI's relm_mp_index_match
and the torch binding's plan cache, which serves a plan for new index tensors
whose contents equal those a cached plan was built from (the same topology
rebuilt in every forward), and never for different or modified indices."""

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
    torch.ops.relm_mp.plan_cache_clear()


def _stats() -> dict[str, int]:
    entries, identity, content, misses = torch.ops.relm_mp.plan_cache_stats()
    return {"entries": entries, "identity": identity, "content": content, "misses": misses}


def _delta(before: dict, after: dict) -> dict:
    return {k: after[k] - before[k] for k in before}


@pytest.mark.parametrize("n", [0, 1, 2047, 2048, 5_000_011])
def test_index_match_c_abi(n) -> None:
    from relmo_amd import capi

    g = torch.Generator(device=DEV)
    g.manual_seed(n)
    keys = torch.randint(0, 1 << 40, (n,), device=DEV, generator=g)
    gathers = torch.randint(0, 1 << 40, (n,), device=DEV, generator=g)
    cands = [(keys.clone(), gathers.clone())]
    if n > 0:
        for pos in sorted({0, n // 2, n - 1}):
            k2 = keys.clone()
            k2[pos] += 1
            g2 = gathers.clone()
            g2[pos] -= 1
            cands += [(k2, gathers.clone()), (keys.clone(), g2)]
    cands = cands[:8]
    _log(f"index_match n={n} candidates={len(cands)}")
    got = capi.index_match(keys, gathers, cands)
    torch.cuda.synchronize()
    assert got == [bool(torch.equal(k, keys) and torch.equal(gg, gathers)) for k, gg in cands]
    assert got[0] and (n == 0 or not any(got[1:]))
    # keys only: candidates whose keys are equal match whatever their gathers
    got_k = capi.index_match(keys, None, [(k, None) for k, _ in cands])
    assert got_k == [bool(torch.equal(k, keys)) for k, _ in cands]


def _fanin_case(seed: int, K: int = 20_000, E: int = 200_000, D: int = 32):
    # ~10 messages per destination (none near the 64-message hub threshold), so
    # sums add in edge order and match the oracle bit for bit
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    rel = torch.randn(E, D, device=DEV, generator=g)
    src = torch.randperm(E, device=DEV, generator=g)
    dst = torch.randint(0, K, (E,), device=DEV, generator=g)
    return rel, src, dst, K


def test_content_hit_reuses_the_forward_plan(mp_env) -> None:
    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, src, dst, K = _fanin_case(1)
    outs = []
    for step in range(3):  # the "same topology, new tensors" of consecutive forwards
        r = rel.clone().requires_grad_(True)
        before = _stats()
        out = mp.fanin_reduce(r, src.clone(), dst.clone(), K, 1)
        (grad,) = torch.autograd.grad(out, r, torch.ones_like(out))
        d = _delta(before, _stats())
        _log(f"content cache step {step}: {d}")
        if step > 0:  # forward CSR plan and backward inverse plan both served by content
            assert d["content"] == 2 and d["misses"] == 0 and d["entries"] == 0, d
        outs.append((out.detach(), grad))
    for out, grad in outs[1:]:
        assert torch.equal(out, outs[0][0]) and torch.equal(grad, outs[0][1])
    want = oracle.fanin_reduce_logsumexp(rel.cpu().numpy(), src.cpu().numpy(), dst.cpu().numpy(), K)
    np.testing.assert_allclose(outs[0][0].cpu().numpy(), want, rtol=1e-4, atol=1e-6)


def test_content_miss_on_different_indices(mp_env) -> None:
    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, src, dst, K = _fanin_case(2)
    mp.fanin_reduce(rel, src, dst, K, 0)
    for name, (s2, d2) in {
        "dst last": (src.clone(), torch.cat([dst[:-1], (dst[-1:] + 1) % K])),
        "src first": (torch.cat([src[1:2], src[:1], src[2:]]), dst.clone()),
    }.items():
        before = _stats()
        out = mp.fanin_reduce(rel, s2, d2, K, 0)
        d = _delta(before, _stats())
        assert d["content"] == 0 and d["misses"] >= 1, (name, d)
        want = oracle.fanin_reduce_sum(rel.cpu().numpy(), s2.cpu().numpy(), d2.cpu().numpy(), K)
        assert np.array_equal(out.cpu().numpy(), want), name


def test_content_cache_drops_entries_modified_in_place(mp_env) -> None:
    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, src, dst, K = _fanin_case(3)
    original = dst.clone()
    mp.fanin_reduce(rel, src, dst, K, 0)
    dst.copy_(torch.flip(original, [0]))  # the cached entry's tensor now holds other indices
    before = _stats()
    out = mp.fanin_reduce(rel, src, original.clone(), K, 0)
    d = _delta(before, _stats())
    assert d["content"] == 0 and d["identity"] == 0, d
    want = oracle.fanin_reduce_sum(rel.cpu().numpy(), src.cpu().numpy(), original.cpu().numpy(), K)
    assert np.array_equal(out.cpu().numpy(), want)


def test_content_hit_for_fanout_and_strided_indices(mp_env) -> None:
    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    g = torch.Generator(device=DEV)
    g.manual_seed(4)
    R, slots, D = 5000, 40_000, 16
    x = torch.randn(R, D, device=DEV, generator=g)
    pairs = torch.stack([torch.randint(0, R, (slots,), device=DEV, generator=g),
                         torch.randperm(slots, device=DEV, generator=g)], dim=1)
    src, dst = pairs[:, 0], pairs[:, 1]  # strided views: each call copies them
    assert not src.is_contiguous()
    first = mp.fanout_scatter(x, src, dst, slots)
    before = _stats()
    second = mp.fanout_scatter(x, src, dst, slots)
    d = _delta(before, _stats())
    assert d["content"] == 1, d
    assert torch.equal(first, second)
    want = oracle.fanout_scatter(x.cpu().numpy(), src.cpu().numpy(), dst.cpu().numpy(), slots)
    assert np.array_equal(second.cpu().numpy(), want)
