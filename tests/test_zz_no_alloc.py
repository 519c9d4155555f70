"""GPU test of relm_mp_fanin_reduce_noalloc, the entry point that allocates
nothing: through the C ABI, its results equal relm_mp_fanin_reduce's (the
workspace entry point, same kernels) bit for bit, on consecutive calls that
reuse the library's device scratch with a smaller input second, on two
streams back to back, and a call beyond the scratch size is refused before
anything is launched."""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")


def _case(seed: int, K: int, E: int, D: int, dtype, hub: int):
    """Uniform destinations plus one hub of `hub` messages (many hub chunks),
    messages gathered through a random permutation."""

    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    rel = 2.0 * torch.randn(E, D, device=DEV, generator=g, dtype=dtype)
    dst = torch.randint(0, K, (E,), device=DEV, generator=g)
    dst[torch.randperm(E, device=DEV, generator=g)[:hub]] = 7
    src = torch.randperm(E, device=DEV, generator=g)
    return rel, src, dst


# (seed, objects, messages, emb, dtype, hub size, mode); the second call is
# the smaller one, on the scratch the first has just filled
CALLS = [
    (1, 60_000, 1_200_000, 32, torch.float32, 200_000, 1),
    (2, 3_000, 50_000, 8, torch.float32, 5_000, 0),
    (3, 10_000, 300_000, 16, torch.float64, 20_000, 1),
]


def test_noalloc_matches_the_workspace_entry_point() -> None:
    from relmo_amd import capi

    for seed, K, E, D, dtype, hub, mode in CALLS:
        need = capi.lib().relm_mp_fanin_reduce_workspace_size(E, K, D, capi._dtype(torch.empty(0, dtype=dtype)))
        assert need <= capi.NOALLOC_SCRATCH_BYTES, need
        _log(f"noalloc seed={seed} K={K} E={E} D={D} {dtype} hub={hub} mode={mode} scratch={need}")
        rel, src, dst = _case(seed, K, E, D, dtype, hub)
        got = capi.fanin_reduce_noalloc(rel, src, dst, K, mode)
        want = capi.fanin_reduce(rel, src, dst, K, mode)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (seed, (got - want).abs().max().item())


def test_noalloc_calls_on_two_streams_are_ordered() -> None:
    """A call on one stream returns with its kernels still queued; the next
    call, on another stream, builds its plan in the same device scratch.  The
    library orders the second behind the first (an event per device), so both
    results equal the workspace entry point's."""

    from relmo_amd import capi

    a = _case(4, 60_000, 1_200_000, 32, torch.float32, 200_000)
    b = _case(5, 3_000, 50_000, 32, torch.float32, 5_000)
    want_a = capi.fanin_reduce(*a, 60_000, 1)
    want_b = capi.fanin_reduce(*b, 3_000, 1)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        with torch.cuda.stream(s1):
            got_a = capi.fanin_reduce_noalloc(*a, 60_000, 1)
        with torch.cuda.stream(s2):
            got_b = capi.fanin_reduce_noalloc(*b, 3_000, 1)
        torch.cuda.synchronize()
        assert torch.equal(got_a, want_a)
        assert torch.equal(got_b, want_b)


def test_noalloc_refuses_calls_beyond_its_scratch() -> None:
    from relmo_amd import capi

    E, K, D = 4_000_000, 1_000, 32
    need = capi.lib().relm_mp_fanin_reduce_workspace_size(E, K, D, capi.F32)
    assert need > capi.NOALLOC_SCRATCH_BYTES
    # valid arguments of the claimed sizes (every index in bounds), so that a
    # call that is not refused shows up as a changed `out`, never as a fault
    rel = torch.zeros(1, D, device=DEV)
    idx = torch.zeros(E, dtype=torch.int64, device=DEV)
    out = torch.full((K, D), 5.0, device=DEV)
    rc = capi.lib().relm_mp_fanin_reduce_noalloc(
        capi.F32, rel.data_ptr(), rel.size(0), D, idx.data_ptr(), idx.data_ptr(), E, K, 0, out.data_ptr(),
        capi._stream(rel))
    assert rc == capi.ERR_WORKSPACE
    assert "relm_mp_fanin_reduce_noalloc" in capi.last_error() and "workspace" in capi.last_error()
    torch.cuda.synchronize()
    assert bool((out == 5.0).all())  # nothing was launched
