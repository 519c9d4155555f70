"""GPU tests of plan reuse: the C ABI's relm_mp_plan_match (index arrays against
the snapshot a plan keeps of the indices it was built from) and the torch
binding's plan cache, which serves a plan only for index arrays equal to that
snapshot - for new tensors of equal content (the same topology rebuilt in every
forward), never for different indices, whether they were changed in place,
through ``.data`` (no version-counter bump) or on another stream."""

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
    """Cache counters; "hits" counts every plan served.  Whether a hit counts as
    "same" (last used with the same tensor objects) or "other" is only the
    cache's ordering hint: a new tensor can occupy a freed tensor's address."""

    entries, same, other, misses, kept, peak, trusted = torch.ops.relm_mp.plan_cache_stats()
    return {"entries": entries, "same": same, "other": other, "hits": same + other, "misses": misses,
            "trusted": trusted}


def _delta(before: dict, after: dict) -> dict:
    return {k: after[k] - before[k] for k in before}


@pytest.mark.parametrize("n", [0, 1, 4095, 4096, 4097, 5_000_011])
def test_plan_match_c_abi(n) -> None:
    """Snapshots of CSR and inverse plans against equal and altered indices:
    random tiles (stored) and tiles whose gathers are the edge ids (flagged)."""

    from relmo_amd import capi

    g = torch.Generator(device=DEV)
    g.manual_seed(n)
    K = max(n // 3, 1)
    keys = torch.randint(0, K, (n,), device=DEV, generator=g)
    gathers = torch.arange(n, device=DEV)
    if n > 8192:  # one stored tile in the middle, the others plain
        gathers[4096:8192] = torch.randint(0, n, (4096,), device=DEV, generator=g)
    plans = [capi.csr_plan(keys, K, gathers, n),
             capi.inv_plan(keys, K, gathers, n, snapshot=True)]
    torch.cuda.synchronize()
    _log(f"plan_match n={n}")
    assert capi.plan_match(keys.clone(), gathers.clone(), plans) == [True, True]
    assert capi.plan_match(keys.clone(), None, plans) == [True, True]
    if n == 0:
        return
    for pos in sorted({0, n // 2, n - 1, min(n - 1, 5000)}):
        k2 = keys.clone()
        k2[pos] = (k2[pos] + 1) % (K + 1)
        g2 = gathers.clone()
        g2[pos] += 1
        assert capi.plan_match(k2, gathers, plans) == [False, False], ("key", pos)
        assert capi.plan_match(keys, g2, plans) == [False, False], ("gather", pos)
        assert capi.plan_match(keys, None, plans) == [True, True]
    # another length never matches; a plan without a snapshot is refused
    if n > 1:
        assert capi.plan_match(keys[:-1].clone(), gathers[:-1].clone(), plans) == [False, False]
    bare = capi.inv_plan(keys, K, gathers, n)
    with pytest.raises(RuntimeError, match="snapshot"):
        capi.plan_match(keys, gathers, [bare])


def _fanin_case(seed: int, K: int = 20_000, E: int = 200_000, D: int = 32):
    # ~10 messages per destination (none near the 64-message hub threshold), so
    # sums add in edge order and match the oracle bit for bit
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    rel = torch.randn(E, D, device=DEV, generator=g)
    src = torch.randperm(E, device=DEV, generator=g)
    dst = torch.randint(0, K, (E,), device=DEV, generator=g)
    return rel, src, dst, K


def _want_sum(rel, src, dst, K):
    return oracle.fanin_reduce_sum(rel.cpu().numpy(), src.cpu().numpy(), dst.cpu().numpy(), K)


def test_content_hit_for_new_tensors_and_handoff(mp_env) -> None:
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
        # the forward's CSR plan: built once, then served by content; the
        # backward gets it from the autograd function and (flat_src is a
        # permutation) builds the inverse map of flat_src from that plan's
        # snapshot - kept with the plan, so no plan of its own is looked up
        if step == 0:
            assert d["misses"] == 1 and d["entries"] == 1, d
        else:
            assert d["hits"] == 1 and d["misses"] == 0 and d["entries"] == 0, d
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
        assert d["hits"] == 0 and d["misses"] >= 1, (name, d)
        assert np.array_equal(out.cpu().numpy(), _want_sum(rel, s2, d2, K)), name


@pytest.mark.parametrize("how", ["in_place", "data", "raw_pointer"])
def test_index_written_after_the_build_gets_a_new_plan(mp_env, how) -> None:
    """The same tensor objects called again after their indices changed: a write
    that bumps the version counter, one through ``.data`` that does not, and one
    into the storage by a kernel that autograd never sees (a view created
    before, written after) - every one must give the new indices' result."""

    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, src, dst, K = _fanin_case(3)
    first = mp.fanin_reduce(rel, src, dst, K, 0)
    assert np.array_equal(first.cpu().numpy(), _want_sum(rel, src, dst, K))
    new_dst = torch.flip(dst, [0]).contiguous()
    version = dst._version
    if how == "in_place":
        dst.copy_(new_dst)
        assert dst._version != version
    elif how == "data":
        dst.data[:] = new_dst
        assert dst._version == version  # the hole a version check alone would miss
    else:
        alias = torch.from_dlpack(torch.utils.dlpack.to_dlpack(dst.detach()))
        alias.copy_(new_dst)
        assert dst._version == version
    assert torch.equal(dst, new_dst)
    before = _stats()
    out = mp.fanin_reduce(rel, src, dst, K, 0)
    d = _delta(before, _stats())
    _log(f"{how}: {d}")
    assert d["hits"] == 0 and d["misses"] == 1, d
    assert np.array_equal(out.cpu().numpy(), _want_sum(rel, src, new_dst, K))


def test_raw_schema_backward_finds_the_forward_plan(mp_env) -> None:
    """The reference's own autograd functions call the plain schemas; the
    backward then finds the forward's plan by content (the same tensors)."""

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, _, dst, K = _fanin_case(5)
    src = torch.arange(rel.size(0), device=DEV)
    out = ns.fanin_reduce(rel, src, dst, K, 1)
    g = torch.randn_like(out)
    before = _stats()
    got = ns.fanin_reduce_logsumexp_backward(g, rel, src, dst, out, rel.size(0))
    d = _delta(before, _stats())
    assert d["hits"] == 1 and d["misses"] == 0, d
    want = oracle.fanin_reduce_logsumexp_backward(
        g.cpu().numpy(), rel.cpu().numpy(), src.cpu().numpy(), dst.cpu().numpy(),
        out.cpu().numpy(), rel.size(0))
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-4, atol=1e-6)


def test_plan_built_on_one_stream_reused_on_another(mp_env) -> None:
    """A plan built on stream A and served on stream B: B waits for A's build
    (the cached entry is inserted before A has run it) and the plan memory is
    recorded for B, so dropping the entry while B still works is safe."""

    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, src, dst, K = _fanin_case(6, K=200_000, E=2_000_000)
    want = _want_sum(rel, src, dst, K)
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(a):
        torch.cuda._sleep(20_000_000)  # keeps A busy, so the build is still queued
        out_a = mp.fanin_reduce(rel, src, dst, K, 0)
    with torch.cuda.stream(b):
        before = _stats()
        out_b = mp.fanin_reduce(rel, src.clone(), dst.clone(), K, 0)
        d = _delta(before, _stats())
        ns.plan_cache_clear()  # drops the entry while B's kernels may still run
        out_b2 = out_b * 1.0
    torch.cuda.synchronize()
    assert d["hits"] == 1, d
    assert np.array_equal(out_a.cpu().numpy(), want)
    assert np.array_equal(out_b2.cpu().numpy(), want)


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
    assert d["hits"] == 1, d
    assert torch.equal(first, second)
    want = oracle.fanout_scatter(x.cpu().numpy(), src.cpu().numpy(), dst.cpu().numpy(), slots)
    assert np.array_equal(second.cpu().numpy(), want)


def test_cache_memory_stays_bounded(mp_env) -> None:
    """New topologies every call: entries are evicted to the memory bound and
    the kept / peak byte counts are reported."""

    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    for seed in range(12):
        rel, src, dst, K = _fanin_case(100 + seed)
        mp.fanin_reduce(rel, src, dst, K, 0)
    entries, _, _, _, kept, peak, _trusted = ns.plan_cache_stats()
    limit = int(os.environ.get("RELM_MP_PLAN_CACHE_MB", "2048")) << 20
    assert 0 < kept <= peak <= limit and entries >= 1


def test_inference_mode_indices(mp_env) -> None:
    """Index tensors made under torch.inference_mode() keep no version counter:
    the cache builds, keeps and serves plans for them as for other tensors
    (fanin sum and fanout, the second call of each a content hit)."""

    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, src, dst, K = _fanin_case(3)
    with torch.inference_mode():
        s2, d2 = src.clone(), dst.clone()
        before = _stats()
        a = mp.fanin_reduce(rel, s2, d2, K, 0)
        b = mp.fanin_reduce(rel, s2, d2, K, 0)
        f1 = mp.fanout_scatter(rel, s2, d2, K)
        f2 = mp.fanout_scatter(rel, s2, d2, K)
        d = _delta(before, _stats())
    _log(f"inference-mode indices: {d}")
    assert d["hits"] >= 2, d
    assert torch.equal(a, b) and torch.equal(f1, f2)
    assert np.array_equal(a.cpu().numpy(), _want_sum(rel, src, dst, K))
    want = oracle.fanout_scatter(rel.cpu().numpy(), src.cpu().numpy(), dst.cpu().numpy(), K)
    assert np.array_equal(f1.cpu().numpy(), want)


def test_trust_scope_serves_the_same_tensors_without_comparing(mp_env) -> None:
    """In an mp.plan_scope the plan of a call is served again for the very same
    index tensors without the device comparison (counted as "trusted"); new
    tensors of equal content are still compared, and after the scope a write
    through .data is seen again."""

    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, src, dst, K = _fanin_case(7)
    want = _want_sum(rel, src, dst, K)
    with mp.plan_scope():
        with mp.plan_scope():  # nested: the outer scope keeps the records
            before = _stats()
            first = mp.fanin_reduce(rel, src, dst, K, 0)
            d = _delta(before, _stats())
            assert d["trusted"] == 0 and d["misses"] == 1, d
        for rep in range(3):
            before = _stats()
            out = mp.fanin_reduce(rel, src, dst, K, 0)
            d = _delta(before, _stats())
            _log(f"trust scope call {rep}: {d}")
            assert d["trusted"] == 1 and d["hits"] == 0 and d["misses"] == 0, d
            assert torch.equal(out, first)
        before = _stats()
        out = mp.fanin_reduce(rel, src.clone(), dst.clone(), K, 0)
        d = _delta(before, _stats())
        assert d["trusted"] == 0 and d["hits"] == 1, d
        assert torch.equal(out, first)
    assert np.array_equal(first.cpu().numpy(), want)
    # scope closed: the same tensors are compared again, so an untracked write is seen
    new_dst = torch.flip(dst, [0]).contiguous()
    dst.data[:] = new_dst
    before = _stats()
    out = mp.fanin_reduce(rel, src, dst, K, 0)
    d = _delta(before, _stats())
    assert d["trusted"] == 0 and d["misses"] == 1, d
    assert np.array_equal(out.cpu().numpy(), _want_sum(rel, src, new_dst, K))


def test_trust_scope_closes_on_error(mp_env) -> None:
    from relmo_amd import mp

    ns = torch.ops.relm_mp
    ns.plan_cache_clear()
    rel, src, dst, K = _fanin_case(8)
    with pytest.raises(ValueError, match="boom"):
        with mp.plan_scope():
            mp.fanin_reduce(rel, src, dst, K, 0)
            raise ValueError("boom")
    before = _stats()
    mp.fanin_reduce(rel, src, dst, K, 0)
    d = _delta(before, _stats())
    assert d["trusted"] == 0 and d["hits"] == 1, d

