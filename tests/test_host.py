"""Host-side checks that run without a GPU: the C ABI library loads and exports
exactly what include/relm_mp.h declares, the ctypes plan mirror matches the C
struct, the torch binding's CPU lane and the python_only path reproduce the
reference's golden fixtures, the runtime / dispatch policy follows relmo's
mp_runtime.py / mp_dispatch.py, and the autograd facade differentiates
correctly (CPU lane, float64 gradcheck).  No kernel is launched here.
"""

from __future__ import annotations

import ctypes
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.conftest import REPO

HEADER = REPO / "include" / "relm_mp.h"
EPS32 = float(np.finfo(np.float32).eps)


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^(?:size_t|int|int64_t|const char\*)\s+(relm_mp_\w+)\s*\(", text, re.M))


def _hip_library():
    from relmo_amd import capi

    if not capi.LIB_PATH.exists():
        pytest.skip("librelm_mp_hip.so is not built (run __graft_entry__.build())")
    return capi


def test_header_declares_the_reference_ops() -> None:
    names = _declared_functions()
    for op in ("fanout_scatter", "fanout_scatter_backward", "fanin_reduce",
               "fanin_reduce_sum_backward", "fanin_reduce_logsumexp_backward"):
        assert f"relm_mp_{op}" in names and f"relm_mp_{op}_workspace_size" in names
    assert {"relm_mp_last_error", "relm_mp_build_info"} <= names


def test_library_exports_exactly_the_header_symbols() -> None:
    capi = _hip_library()
    declared = _declared_functions()
    nm = subprocess.run(["nm", "-D", "--defined-only", str(capi.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T relm_mp_" in line}
    assert exported == declared
    assert set(capi.EXPORTED_SYMBOLS) == declared
    lib = ctypes.CDLL(str(capi.LIB_PATH))
    for name in declared:
        assert getattr(lib, name) is not None


@pytest.mark.parametrize("struct", ["relm_mp_plan", "relm_mp_index_part"])
def test_struct_layouts_match_header(tmp_path, struct) -> None:
    from relmo_amd import capi

    mirror = {"relm_mp_plan": capi.Plan, "relm_mp_index_part": capi.IndexPart}[struct]
    fields = [name for name, _ in mirror._fields_]
    prog = tmp_path / "layout.c"
    body = "\n".join(f'    printf("{f} %zu\\n", offsetof({struct}, {f}));' for f in fields)
    prog.write_text(
        "#include <stddef.h>\n#include <stdio.h>\n#include \"relm_mp.h\"\n"
        f"int main(void) {{\n    printf(\"sizeof %zu\\n\", sizeof({struct}));\n{body}\n    return 0;\n}}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{HEADER.parent}", str(prog), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                        check=True).stdout.splitlines())
    assert int(out["sizeof"]) == ctypes.sizeof(mirror)
    for f in fields:
        assert int(out[f]) == getattr(mirror, f).offset, f


# ---- torch binding, CPU lane -------------------------------------------------------------


@pytest.fixture(scope="module")
def ops():
    from relmo_amd import mp_runtime

    mp_runtime.ensure_loaded()
    return torch.ops.relm_mp


def _cpu_sum_parity(op: str, args: list, got: np.ndarray, want: np.ndarray, name: str) -> None:
    positions = {"fanout_scatter_backward": (0, 2, 1), "fanin_reduce": (0, 1, 2),
                 "fanin_reduce_sum_backward": (0, 2, 1)}
    t, r, w = positions[op]
    truth, absum = oracle.segment_sum_truth(args[t], args[r], args[w], got.shape[0])
    special = ~np.isfinite(want) | ~np.isfinite(truth)
    assert np.array_equal(got[special], want[special], equal_nan=True), name
    bound = 4 * EPS32 * absum[~special] + 1e-30
    assert np.all(np.abs(got[~special] - truth[~special]) <= bound), name
    assert np.all(np.abs(want[~special] - truth[~special]) <= bound), name


def _check_case(fn, case: dict, arrays: dict, exact: bool) -> None:
    args = [torch.from_numpy(arrays[n]) for n in case["tensors"]] + list(case["ints"])
    if "error" in case:
        with pytest.raises((RuntimeError, ValueError, IndexError)) as info:
            fn(*args)
        assert str(info.value).splitlines()[0] == case["error"], case["name"]
        assert (case.get("error_type") == "IndexError") == isinstance(info.value, IndexError), case["name"]
        return
    got = fn(*args).numpy()
    want = arrays[case["expected"]]
    assert got.shape == want.shape and got.dtype == want.dtype, case["name"]
    lse = case["op"] == "fanin_reduce_logsumexp_backward" or (
        case["op"] == "fanin_reduce" and case["ints"][1] == 1)
    if exact and not lse:
        assert np.array_equal(got, want, equal_nan=True), case["name"]
    elif lse:
        assert np.array_equal(np.isnan(got), np.isnan(want)), case["name"]
        assert np.array_equal(np.isinf(got), np.isinf(want)), case["name"]
        fin = np.isfinite(want)
        np.testing.assert_allclose(got[fin], want[fin], rtol=1e-5, atol=1e-6, err_msg=case["name"])
    elif case["op"] == "fanout_scatter":
        assert np.array_equal(got, want), case["name"]
    else:
        np_args = [arrays[n] for n in case["tensors"]]
        _cpu_sum_parity(case["op"], np_args, got, want, case["name"])


def test_cpu_lane_reproduces_golden_bit_exact(ops, golden) -> None:
    """The CPU lane is the reference's sequential loops: identical bits for
    copies and sums, the same ATen sequence for logsumexp."""

    cases, arrays = golden
    for case in cases:
        _check_case(getattr(ops, case["op"]), case, arrays, exact=True)


def test_python_only_path_reproduces_golden(monkeypatch, golden) -> None:
    from relmo_amd import mp_pack

    cases, arrays = golden
    fns = {
        "fanout_scatter": mp_pack.fanout_scatter_python,
        "fanin_reduce": mp_pack.fanin_reduce_python,
    }
    checked = 0
    for case in cases:
        if case["op"] not in fns or "error" in case:
            continue
        _check_case(fns[case["op"]], case, arrays, exact=False)
        checked += 1
    assert checked > 10


def test_cpu_lane_rejects_bad_arguments(ops) -> None:
    x = torch.randn(4, 3)
    idx = torch.tensor([0, 1, 2])
    with pytest.raises(RuntimeError, match="must have equal length"):
        ops.fanout_scatter(x, idx, idx[:2], 3)
    with pytest.raises(RuntimeError, match="must have dtype torch.int64"):
        ops.fanout_scatter(x, idx.int(), idx, 3)
    # std::invalid_argument, as in the reference (torch surfaces it as ValueError)
    with pytest.raises((RuntimeError, ValueError), match="Unsupported fanin_reduce mode"):
        ops.fanin_reduce(x, idx, idx, 4, 2)
    with pytest.raises(RuntimeError, match=r"src_global_idx index out of bounds: 4 not in \[0, 4\)\."):
        ops.fanout_scatter(x, torch.tensor([0, 4]), torch.tensor([0, 1]), 2)


def test_cpu_lane_empty_inputs(ops) -> None:
    rel = torch.randn(0, 5)
    empty = torch.zeros(0, dtype=torch.long)
    assert torch.equal(ops.fanin_reduce(rel, empty, empty, 3, 0), torch.zeros(3, 5))
    assert torch.equal(ops.fanin_reduce(rel, empty, empty, 3, 1), torch.full((3, 5), float("-inf")))
    assert ops.fanout_scatter(torch.randn(2, 4), empty, empty, 0).shape == (0, 4)


def test_build_info_is_rocm_compatible(ops) -> None:
    from relmo_amd import mp_runtime

    info = mp_runtime.parse_build_info(ops.build_info())
    assert info["build_cuda_tag"] == "cpu"
    assert mp_runtime.major_minor(info["build_torch"]) == mp_runtime.major_minor(torch.__version__)
    assert info["arch"] == "gfx950" and "hip" in info
    assert mp_runtime.assert_runtime_compat()["build_cuda_tag"] == "cpu"


# ---- runtime / dispatch policy (mirrors relmo's test_mp_runtime.py) -------------------------


def test_parse_build_info_and_versions() -> None:
    from relmo_amd import mp_runtime

    assert mp_runtime.parse_build_info("a=1; b = x ;junk;c=") == {"a": "1", "b": "x", "c": ""}
    assert mp_runtime.major_minor("2.10.0+rocm7.0") == (2, 10)
    with pytest.raises(RuntimeError):
        mp_runtime.major_minor("nightly")
    assert mp_runtime.runtime_cuda_tag() == ("cpu" if torch.version.cuda is None else
                                             "cu" + torch.version.cuda.replace(".", ""))


def test_env_policies(monkeypatch) -> None:
    from relmo_amd import mp_runtime

    monkeypatch.delenv("RELM_MP_FALLBACK", raising=False)
    assert mp_runtime.fallback_mode() == "python"
    assert mp_runtime.fallback_mode(torch.empty(0)) == "python"
    gpu_like = type("GpuTensor", (), {"is_cuda": True})()
    assert mp_runtime.fallback_mode(gpu_like) == "error"
    monkeypatch.setenv("RELM_MP_FALLBACK", "PYTHON")
    assert mp_runtime.fallback_mode() == "python"
    monkeypatch.setenv("RELM_MP_TORCH_VERSION_POLICY", "strict")
    assert mp_runtime.torch_version_policy() == "strict"
    # unknown values fall back to the default, as in relmo's mp_runtime.py:60-69
    monkeypatch.setenv("RELM_MP_TORCH_VERSION_POLICY", "bogus")
    assert mp_runtime.torch_version_policy() == "forward"
    monkeypatch.setenv("RELM_MP_FALLBACK", "bogus")
    assert mp_runtime.fallback_mode() == "python"
    assert mp_runtime.fallback_mode(gpu_like) == "error"


def _fake_build(monkeypatch, info: str) -> None:
    from relmo_amd import mp_runtime

    class _NS:
        @staticmethod
        def build_info() -> str:
            return info

    monkeypatch.setattr(mp_runtime, "_BUILD_INFO_CACHE", None)
    monkeypatch.setattr(mp_runtime, "ensure_loaded", lambda: None)
    monkeypatch.setattr(mp_runtime, "ops_namespace", lambda: _NS)


def test_compat_rejects_mismatched_builds(monkeypatch) -> None:
    from relmo_amd import mp_runtime

    major, minor = mp_runtime.major_minor(torch.__version__)
    _fake_build(monkeypatch, "build_cuda_tag=cpu")
    with pytest.raises(RuntimeError, match="missing build_torch"):
        mp_runtime.assert_runtime_compat()
    _fake_build(monkeypatch, f"build_torch={major + 1}.0.0;build_cuda_tag=cpu")
    with pytest.raises(RuntimeError, match="major version mismatch"):
        mp_runtime.assert_runtime_compat()
    _fake_build(monkeypatch, f"build_torch={major}.{minor + 1}.0;build_cuda_tag=cpu")
    with pytest.raises(RuntimeError, match="older than the build torch"):
        mp_runtime.assert_runtime_compat()
    _fake_build(monkeypatch, f"build_torch={major}.{minor}.0;build_cuda_tag=cu999")
    with pytest.raises(RuntimeError, match="CUDA tag mismatch"):
        mp_runtime.assert_runtime_compat()
    if minor > 0:
        _fake_build(monkeypatch, f"build_torch={major}.{minor - 1}.0;build_cuda_tag=cpu")
        with pytest.warns(RuntimeWarning, match="version drift"):
            mp_runtime.assert_runtime_compat()
        monkeypatch.setenv("RELM_MP_TORCH_VERSION_POLICY", "strict")
        _fake_build(monkeypatch, f"build_torch={major}.{minor - 1}.0;build_cuda_tag=cpu")
        with pytest.raises(RuntimeError, match="Expected matching major.minor"):
            mp_runtime.assert_runtime_compat()


def test_dispatch_policy(monkeypatch) -> None:
    from relmo_amd import mp_dispatch, mp_runtime

    gpu_like = type("GpuTensor", (), {"is_cuda": True})()
    monkeypatch.setenv("RELM_MP_ENABLE", "0")
    assert mp_dispatch.library_ready("fanin_reduce") is False
    assert mp_dispatch.library_op("fanin_pack_multi") is None

    def broken() -> None:
        raise RuntimeError("library missing")

    monkeypatch.setenv("RELM_MP_ENABLE", "1")
    monkeypatch.setattr(mp_dispatch, "ensure_runtime_compat_once", broken)
    monkeypatch.setenv("RELM_MP_FALLBACK", "error")
    with pytest.raises(RuntimeError, match="Custom mp op fanin_reduce is unavailable"):
        mp_dispatch.library_ready("fanin_reduce")
    monkeypatch.setenv("RELM_MP_FALLBACK", "python")
    assert mp_dispatch.library_ready("fanin_reduce") is False
    assert mp_dispatch.library_ready("fanin_reduce", gpu_like) is False
    # unset: relmo's quiet fallback for CPU tensors, an error for GPU tensors
    monkeypatch.delenv("RELM_MP_FALLBACK")
    assert mp_dispatch.library_ready("fanin_reduce", torch.empty(0)) is False
    with pytest.raises(RuntimeError, match="Custom mp op fanin_reduce is unavailable"):
        mp_dispatch.library_ready("fanin_reduce", gpu_like)
    calls = []
    assert mp_dispatch.run_op("fanin_pack_multi", 1, 2, fallback=lambda *a: calls.append(a) or "fb") == "fb"
    assert calls == [(1, 2)]
    assert mp_runtime.candidate_libraries()[0].name.startswith("relm_mp_ops")


def test_dispatch_routes_to_the_library(monkeypatch) -> None:
    from relmo_amd import mp_dispatch

    monkeypatch.setenv("RELM_MP_ENABLE", "1")
    monkeypatch.setenv("RELM_MP_FALLBACK", "error")
    op = mp_dispatch.library_op("fanin_pack_multi")
    assert op is torch.ops.relm_mp.fanin_pack_multi
    # gpu-only ops stay on the fallback for CPU tensors, without an error
    assert mp_dispatch.library_op("lgan_pool_reduce", tensor=torch.empty(0), gpu_only=True) is None
    with pytest.raises(RuntimeError, match="unavailable in the loaded relm_mp library"):
        mp_dispatch.library_op("no_such_op")
    monkeypatch.setenv("RELM_MP_FALLBACK", "python")
    assert mp_dispatch.library_op("no_such_op") is None


def test_facade_public_names() -> None:
    from relmo_amd import mp

    for name in mp.__all__:
        assert hasattr(mp, name), name
    assert (mp.MODE_SUM, mp.MODE_LOGSUMEXP, mp.MODE_MEAN) == (0, 1, 2)
    with pytest.raises(ValueError):
        mp.fanin_reduce(torch.randn(2, 3), torch.tensor([0, 1]), torch.tensor([0, 0]), 1, mode=2)


# ---- autograd facade on the CPU lane -----------------------------------------------------


def test_autograd_matches_aten_on_cpu(mp_env) -> None:
    from relmo_amd import mp

    gen = torch.Generator().manual_seed(3)
    x = torch.randn(6, 4, dtype=torch.float64, generator=gen, requires_grad=True)
    src = torch.tensor([0, 2, 2, 5, 1, 0, 3])
    flat = torch.tensor([3, 0, 6, 1, 2, 5, 4])
    assert torch.autograd.gradcheck(lambda t: mp.fanout_scatter(t, src, flat, 7), (x,))
    rel = torch.randn(7, 4, dtype=torch.float64, generator=gen, requires_grad=True)
    fs = torch.tensor([0, 1, 2, 3, 4, 5, 6])
    di = torch.tensor([1, 1, 0, 3, 1, 0, 3])
    assert torch.autograd.gradcheck(lambda t: mp.fanin_reduce(t, fs, di, 4, 0), (rel,))
    assert torch.autograd.gradcheck(lambda t: mp.fanin_reduce(t, fs, di, 4, 1)[[0, 1, 3]], (rel,))
    out = mp.fanin_reduce(rel, fs, di, 4, 1)
    ref = torch.full((4, 4), float("-inf"), dtype=torch.float64).index_reduce(
        0, di, rel, "amax", include_self=True)
    ref = torch.zeros(4, 4, dtype=torch.float64).index_add(0, di, (rel - ref[di]).exp()).log() + ref
    torch.testing.assert_close(out, ref)


def test_model_consumers_cpu_lane_matches_aten(monkeypatch) -> None:
    """The C4 / C5 model structure on CPU tensors: the torch binding's CPU
    lane and the ATen (python_only) lane give the same loss."""

    from relmo_amd import consumers as C

    for make_batch, make_model in (
        (lambda: C.synthetic_c4("cpu", seed=1, num_graphs=3),
         lambda b, mode: C.RelationalGNN(16, 2, b.relations, mode)),
        (lambda: C.synthetic_c5("cpu", seed=1, num_graphs=2),
         lambda b, mode: C.CentralizedRelationalGNN(8, 2, b.relations, mode)),
    ):
        batch = make_batch()
        for mode in (0, 1, 2):
            torch.manual_seed(0)
            model = make_model(batch, mode)
            routing = model.routing(batch)
            monkeypatch.setenv("RELM_MP_ENABLE", "1")
            a = C.train_step(model, batch, routing)
            monkeypatch.setenv("RELM_MP_ENABLE", "0")
            b = C.train_step(model, batch, routing)
            assert torch.allclose(a, b, rtol=1e-5, atol=1e-7), (mode, float(a), float(b))


@pytest.mark.parametrize("enable", ["1", "0"])
def test_relational_gnn_batched_lane(monkeypatch, enable: str) -> None:
    """The batched lane's routing, packed by fanout_pack_from_edges and
    fanin_pack_from_edges (the library's CPU lane, or the Python fallbacks with
    the library off), equals the fast fused lane's index for index, and one
    training step of either lane gives the same loss and gradients bit for bit
    (sum, logsumexp, mean)."""

    from relmo_amd import consumers as C

    monkeypatch.setenv("RELM_MP_ENABLE", enable)
    batch = C.synthetic_c4("cpu", seed=2, num_graphs=3)
    for mode in (0, 1, 2):
        runs = []
        for lane in ("fast_fused", "batched"):
            torch.manual_seed(0)
            model = C.RelationalGNN(16, 2, batch.relations, mode, lane=lane)
            r = model.routing(batch)
            loss = C.train_step(model, batch, r)
            runs.append((r, loss, {k: p.grad.clone() for k, p in model.named_parameters()}))
        (ra, la, ga), (rb, lb, gb) = runs
        for key in ("flat", "obj", "deg"):
            assert torch.equal(ra[key], rb[key]), key
        assert torch.equal(rb["fanin_src"], ra["flat"]) and torch.equal(rb["fanin_dst"], ra["obj"])
        assert torch.equal(la, lb), mode
        for k in ga:
            assert torch.equal(ga[k], gb[k]), (mode, k)
    with pytest.raises(ValueError, match="lane"):
        C.RelationalGNN(16, 2, batch.relations, 0, lane="modular")


def test_central_recompute_matches_stored_activations() -> None:
    """Recomputing the central module in the backward (activation
    checkpointing) gives the same loss and gradients as keeping its
    activations."""

    from relmo_amd import consumers as C

    batch = C.synthetic_c5("cpu", seed=2, num_graphs=2)
    for mode in (0, 1, 2):
        grads = []
        for recompute in (False, True):
            torch.manual_seed(0)
            model = C.CentralizedRelationalGNN(8, 2, batch.relations, mode, recompute_central=recompute)
            loss = C.train_step(model, batch, model.routing(batch))
            grads.append((loss, [p.grad.clone() for p in model.parameters()]))
        (la, ga), (lb, gb) = grads
        assert torch.equal(la, lb), mode
        for a, b in zip(ga, gb):
            torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_central_first_linear_gathered_per_object(dtype) -> None:
    """The central MLP with its first Linear evaluated per object and gathered
    per relation node equals the module run on the assembled input: float64
    to 1e-12, float32 to a few ulps of the activations, for every mode, with
    and without recomputation in the backward; so does the path that adds up
    the hidden rows per (object, slot) before the output Linear (sum and mean;
    logsumexp keeps the gathered path)."""

    from relmo_amd import consumers as C

    batch = C.synthetic_c5("cpu", seed=3, num_graphs=2)
    tol = {torch.float64: (1e-10, 1e-12), torch.float32: (2e-4, 1e-6)}[dtype]
    for mode in (0, 1, 2):
        runs = []
        for gathered, recompute, summed in ((False, False, False), (True, False, False), (True, True, False),
                                            (True, False, True), (True, True, True)):
            torch.manual_seed(0)
            model = C.CentralizedRelationalGNN(8, 2, batch.relations, mode, recompute_central=recompute,
                                               gather_first_linear=gathered,
                                               sum_before_output=summed).to(dtype)
            loss = C.train_step(model, batch, model.routing(batch))
            runs.append((loss, [p.grad.clone() for p in model.parameters()]))
        (la, ga), *others = runs
        for lb, gb in others:
            torch.testing.assert_close(lb, la, rtol=tol[0], atol=tol[1])
            for a, b in zip(ga, gb):
                torch.testing.assert_close(b, a, rtol=tol[0], atol=tol[1])


@pytest.mark.parametrize("K", [0, 5, 127, 128, 129, 1000])
def test_split_weight_gradient(K: int) -> None:
    """The chunked weight gradient equals grad_out^T @ inp (chunks of 16 rows
    here, so every K above 128 takes the batched path, with and without a
    remainder)."""

    from relmo_amd.consumers import weight_grad

    g = torch.Generator().manual_seed(K)
    for out_f, in_f in ((7, 5), (5, 7)):  # either operand the narrower one
        go = torch.randn(K, out_f, generator=g, dtype=torch.float64)
        x = torch.randn(K, in_f + 3, generator=g, dtype=torch.float64)[:, 3:]  # a column slice
        torch.testing.assert_close(weight_grad(go, x, chunk=16), go.t() @ x, rtol=1e-12, atol=1e-12)
    # weights of more than 256 x 256 entries, contiguous input or a column slice
    go = torch.randn(K, 300, generator=g, dtype=torch.float64)
    x = torch.randn(K, 260, generator=g, dtype=torch.float64)
    torch.testing.assert_close(weight_grad(go, x, chunk=16), go.t() @ x, rtol=1e-12, atol=1e-12)
    xs = torch.randn(K, 263, generator=g, dtype=torch.float64)[:, 3:]
    torch.testing.assert_close(weight_grad(go, xs, chunk=16), go.t() @ xs, rtol=1e-12, atol=1e-12)
    # a column-strided gradient, and one whose columns are not contiguous
    gs = torch.randn(K, 305, generator=g, dtype=torch.float64)[:, 5:]
    torch.testing.assert_close(weight_grad(gs, xs, chunk=16), gs.t() @ xs, rtol=1e-12, atol=1e-12)
    gt = torch.randn(300, K, generator=g, dtype=torch.float64).t()
    torch.testing.assert_close(weight_grad(gt, x, chunk=16), gt.t() @ x, rtol=1e-12, atol=1e-12)


def test_model_fanin_masks_only_objects_without_messages(mp_env) -> None:
    """Objects without messages get 0 (PyG's aggregators); a NaN or +inf in an
    object's messages still reaches that object's aggregate."""

    from relmo_amd import consumers as C

    rel = torch.tensor([[1.0, 2.0], [float("nan"), 0.0], [float("inf"), 3.0], [4.0, 5.0]])
    r = {"flat": torch.arange(4), "obj": torch.tensor([0, 0, 1, 3])}
    r["deg"] = torch.bincount(r["obj"], minlength=5)
    lse = C.fanin_objects(1, rel, r, 5)
    # relmo's logsumexp (ATen sequence) turns a +inf message into NaN
    assert torch.isnan(lse[0, 0]) and torch.isnan(lse[1, 0])
    assert torch.equal(lse[2], torch.zeros(2)) and torch.equal(lse[4], torch.zeros(2))
    assert torch.equal(lse[3], rel[3])
    mean = C.fanin_objects(2, rel, r, 5)
    assert torch.isnan(mean[0, 0]) and mean[0, 1] == 1.0
    assert torch.equal(mean[3], rel[3]) and torch.equal(mean[2], torch.zeros(2))


# ---- pack ops on the CPU lane ----------------------------------------------------------------

from tests.conftest import pack_args  # noqa: E402


def _check_pack_case(fn, case: dict, arrays: dict, device: str = "cpu", errors: bool = True) -> bool:
    args = pack_args(case, arrays, device)
    if "error" in case:
        if not errors:
            return False
        with pytest.raises((RuntimeError, ValueError)) as info:
            fn(*args)
        assert str(info.value).splitlines()[0] == case["error"], case["name"]
        return True
    got = fn(*args)
    assert len(got) == len(case["expected"]) == 3, case["name"]
    for g, name in zip(got, case["expected"]):
        want = arrays[name]
        assert str(g.device).startswith(device), case["name"]
        g = g.detach().cpu().numpy()
        assert g.dtype == want.dtype and g.shape == want.shape, case["name"]
        assert np.array_equal(g, want), case["name"]
    return True


def test_pack_cpu_lane_reproduces_golden(ops, pack_golden) -> None:
    """Outputs bit-exact, and each invalid call raises the reference's message."""

    cases, arrays = pack_golden
    for case in cases:
        _check_pack_case(getattr(ops, case["op"]), case, arrays)


def test_pack_python_fallbacks_reproduce_golden(pack_golden) -> None:
    from relmo_amd import mp_pack

    cases, arrays = pack_golden
    checked = sum(
        _check_pack_case(getattr(mp_pack, case["op"] + "_python"), case, arrays, errors=False)
        for case in cases
    )
    assert checked >= 30


def test_pack_python_fallback_messages() -> None:
    from relmo_amd import mp_pack

    x = [torch.zeros(3, 2)]
    s = [torch.tensor([0, 1])]
    with pytest.raises(ValueError, match="fanout_pack_multi requires at least one source tensor."):
        mp_pack.fanout_pack_multi_python([], [], [])
    with pytest.raises(ValueError, match="expects matching sequence lengths, got x_parts=1, "
                                         "src_idx_parts=1, flat_dst_parts=0"):
        mp_pack.fanout_pack_multi_python(x, s, [])
    with pytest.raises(ValueError, match="expects src_idx to have dtype int64"):
        mp_pack.fanout_pack_multi_python(x, [s[0].int()], s)
    with pytest.raises(ValueError, match=r"expects pos in \[0, arity\), got pos=2 arity=2"):
        mp_pack.fanout_pack_from_edges_python(x, s, s, [0], [2], [2], [0])
    with pytest.raises(ValueError, match="rel_part_ids out of range: 1"):
        mp_pack.fanin_pack_from_edges_python(x, s, s, [1], [1], [0], 1)
    with pytest.raises(ValueError, match=r"expects mode in \{0,1\}, got 3"):
        mp_pack.fanin_pack_from_edges_python(x, s, s, [0], [1], [0], 3)


def test_pack_single_part_aliasing(ops) -> None:
    """One part: the values tensor comes back as is, so does the second index
    tensor where the op applies no arithmetic to it; the first index output is
    always a new tensor (mp_ops.cpp:480-483, 565-568, 2630-2633, 2767-2770)."""

    x = torch.randn(4, 3)
    src, dst = torch.tensor([0, 2, 3]), torch.tensor([5, 1, 0])
    for op in (ops.fanout_pack_multi, ops.fanin_pack_multi):
        v, a, b = op([x], [src], [dst])
        assert v is x or v.data_ptr() == x.data_ptr()
        assert b.data_ptr() == dst.data_ptr() and a.data_ptr() != src.data_ptr()
        assert torch.equal(a, src)
    v, a, b = ops.fanout_pack_from_edges([x], [src], [dst], [0], [1], [0], [0])
    assert a.data_ptr() != src.data_ptr() and b.data_ptr() != dst.data_ptr()
    for mode in (0, 1):
        v, a, b = ops.fanin_pack_from_edges([x], [src], [dst], [0], [1], [0], mode)
        assert b.data_ptr() == dst.data_ptr() and a.data_ptr() != src.data_ptr()
    # two parts: everything concatenated into new tensors
    v, a, b = ops.fanout_pack_multi([x, x], [src, src], [dst, dst])
    assert v.data_ptr() != x.data_ptr() and torch.equal(b, torch.cat([dst, dst]))


def test_pack_accepts_strided_index_views(ops) -> None:
    base = torch.arange(20).view(10, 2)
    src, dst = base[:, 0], base[:, 1]
    assert not src.is_contiguous()
    x = [torch.randn(30, 2), torch.randn(5, 2)]
    _, a, b = ops.fanout_pack_from_edges(x, [src, dst], [dst, src], [1, 0], [3, 2], [1, 0], [7, 9])
    assert torch.equal(a, torch.cat([src + 30, dst]))
    assert torch.equal(b, torch.cat([7 + dst * 3 + 1, 9 + src * 2]))


def test_pack_facade_dispatch_and_grad(mp_env) -> None:
    """The reference's pack -> fanout / fanin -> backward test on the CPU lane
    (tests/python/test_mp_ops.py:353-600): gradients reach every value part."""

    from relmo_amd import mp

    torch.manual_seed(3)
    xs = [torch.randn(5, 3, dtype=torch.float64, requires_grad=True),
          torch.randn(4, 3, dtype=torch.float64, requires_grad=True)]
    src = [torch.tensor([0, 2, 4, 4]), torch.tensor([1, 3])]
    dst = [torch.tensor([1, 0, 2, 3]), torch.tensor([3, 1])]
    x_cat, s, d = mp.fanout_pack_from_edges(xs, src, dst, [0, 1], [2, 3], [0, 1], [0, 8])
    out = mp.fanout_scatter(x_cat, s, d, 20)
    w = torch.randn_like(out)
    (out * w).sum().backward()
    for x, si, di, arity, pos, slot in zip(xs, src, dst, [2, 3], [0, 1], [0, 8]):
        want = torch.zeros_like(x).index_add_(0, si, w[slot + di * arity + pos])
        assert torch.equal(x.grad, want)
    rels = [torch.randn(6, 4, dtype=torch.float64, requires_grad=True),
            torch.randn(3, 4, dtype=torch.float64, requires_grad=True)]
    fsrc = [torch.tensor([0, 2, 5]), torch.tensor([1, 2])]
    fdst = [torch.tensor([1, 0, 2]), torch.tensor([2, 1])]

    def packed_lse(a, b):
        r_cat, fs, fd = mp.fanin_pack_multi([a, b], fsrc, fdst)
        return mp.fanin_reduce(r_cat, fs, fd, 3, 1)

    assert torch.autograd.gradcheck(packed_lse, tuple(rels))


# ---- LGAN indexed reductions on the CPU lane --------------------------------------------------

LGAN_OUTPUTS = {"lgan_pool_reduce": 3, "lgan_relation_graph_step": 3,
                "lgan_pool_reduce_backward": 1, "lgan_relation_graph_step_backward": 1}


def _check_lgan_case(fn, case: dict, arrays: dict, device: str = "cpu", errors: bool = True) -> bool:
    args = pack_args(case, arrays, device)
    if "error" in case:
        if not errors:
            return False
        with pytest.raises((RuntimeError, ValueError, IndexError)) as info:
            fn(*args)
        assert str(info.value).splitlines()[0] == case["error"], case["name"]
        return True
    got = fn(*args)
    got = got if isinstance(got, (tuple, list)) else (got,)
    assert len(got) == LGAN_OUTPUTS[case["op"]] == len(case["expected"]), case["name"]
    for g, name in zip(got, case["expected"]):
        assert str(g.device).startswith(device), case["name"]
        g = g.detach().cpu().numpy()
        want = arrays[name]
        assert g.dtype == want.dtype and g.shape == want.shape, case["name"]
        assert np.array_equal(g, want), case["name"]
    return True


def test_lgan_cpu_lane_reproduces_golden(ops, lgan_golden) -> None:
    cases, arrays = lgan_golden
    for case in cases:
        _check_lgan_case(getattr(ops, case["op"]), case, arrays)


def test_lgan_python_fallbacks_reproduce_golden(lgan_golden) -> None:
    from relmo_amd import mp_fallbacks

    cases, arrays = lgan_golden
    fns = {"lgan_pool_reduce": mp_fallbacks.lgan_pool_reduce_python,
           "lgan_relation_graph_step": mp_fallbacks.lgan_relation_graph_step_python}
    checked = sum(_check_lgan_case(fns[c["op"]], c, arrays, errors=False)
                  for c in cases if c["op"] in fns)
    assert checked >= 20


@pytest.mark.parametrize("mode", ["sum", "mean"])
def test_lgan_facade_autograd_on_cpu(mode) -> None:
    """CPU tensors take the ATen fallback; gradients equal the backward ops'
    (reference library semantics, pinned by the golden cases) and pass gradcheck."""

    from relmo_amd import mp

    rng = np.random.default_rng(41)
    K, ent, E, D = 25, 11, 60, 3
    s2r = torch.from_numpy(rng.integers(0, K, E))
    arity = torch.from_numpy(rng.integers(0, 4, K))
    edges = [torch.from_numpy(rng.integers(0, b, n)) for b, n in
             [(K, 70), (K, 70), (K, 40), (ent, 40), (K, 30), (ent, 30)]]
    slot = torch.randn(E, D, dtype=torch.float64, requires_grad=True)
    outs = mp._lgan_pool_reduce(slot, s2r, arity, *edges, entity_dim_size=ent, mode=mode)
    gs = [torch.randn_like(o) for o in outs]
    (grad,) = torch.autograd.grad(outs, slot, gs)
    m = 0 if mode == "sum" else 2
    want = torch.ops.relm_mp.lgan_pool_reduce_backward(*gs, s2r, arity, *edges, K, m)
    torch.testing.assert_close(grad, want, rtol=1e-12, atol=1e-12)
    assert torch.autograd.gradcheck(
        lambda x: mp._lgan_relation_graph_step(x, *edges, entity_dim_size=ent, mode=mode),
        (torch.randn(K, D, dtype=torch.float64, requires_grad=True),))
    with pytest.raises(ValueError, match="supports only mode='sum' or mode='mean'"):
        mp._lgan_relation_graph_step(slot, *edges, entity_dim_size=ent, mode="max")


def test_facade_imports_without_torch() -> None:
    """As relmo's facade (tests/python/test_mp_module_layout.py:21-60): without
    torch the module imports, available() is False and the ops fail lazily."""

    code = """
import builtins, importlib, sys
real_import = builtins.__import__
def fake_import(name, globals=None, locals=None, fromlist=(), level=0):
    if name == "torch" or name.startswith("torch."):
        raise ModuleNotFoundError("simulated missing torch")
    return real_import(name, globals, locals, fromlist, level)
builtins.__import__ = fake_import
for key in list(sys.modules):
    if key == "torch" or key.startswith("torch.") or key.startswith("relmo_amd"):
        sys.modules.pop(key, None)
mp = importlib.import_module("relmo_amd.mp")
assert mp.torch is None and mp.available() is False
assert mp.activation_code(("relu",)) == 1
calls = [lambda: mp.fanout_scatter(None, None, None, 0), lambda: mp.fanin_reduce(None, None, None, 0, 0),
         lambda: mp.fanout_pack_multi([], [], []),
         lambda: mp._lgan_relation_graph_step(None, None, None, None, None, None, None,
                                              entity_dim_size=0, mode="sum")]
for call in calls:
    try:
        call()
    except ModuleNotFoundError as exc:
        assert "requires torch" in str(exc)
    else:
        raise AssertionError("no lazy failure")
"""
    proc = subprocess.run([sys.executable, "-c", code], cwd=str(REPO), capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr or proc.stdout


# ---- fanout into argument slots (CPU lane) ----------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_fanout_slots_cpu_lane_matches_oracle(ops, dtype) -> None:
    gen = torch.Generator().manual_seed(12)
    lines, slots, d, col = 40, 3, 6, 5
    x = torch.randn(25, d, dtype=dtype, generator=gen)
    src = torch.randint(0, 25, (100,), generator=gen)
    dst = torch.randint(0, lines * slots, (100,), generator=gen)
    out = torch.randn(lines, col + slots * d + 3, dtype=dtype, generator=gen)
    want = oracle.fanout_into_slots(x.numpy(), src.numpy(), dst.numpy(), out.numpy(), col, slots)
    version = out._version
    ops.fanout_scatter_into(x, src, dst, out, col, slots)
    assert np.array_equal(out.numpy(), want)
    assert out._version > version
    grad = torch.randn(lines, col + slots * d + 3, dtype=dtype, generator=gen)
    got = ops.fanout_scatter_backward_from(grad, src, dst, 25, col, slots, d)
    want = oracle.fanout_backward_from_slots(grad.numpy(), src.numpy(), dst.numpy(), 25, col, slots, d)
    assert np.array_equal(got.numpy(), want)
    with pytest.raises(RuntimeError, match="exceed the"):
        ops.fanout_scatter_into(x, src, dst, out, col + 4, slots)
    with pytest.raises(RuntimeError, match="flat_dst index out of bounds"):
        ops.fanout_scatter_into(x, src, dst, out[:10], col, slots)


def test_fanout_concat_autograd_on_cpu(mp_env) -> None:
    from relmo_amd import mp

    gen = torch.Generator().manual_seed(13)
    prefix = torch.randn(9, 4, dtype=torch.float64, generator=gen, requires_grad=True)
    x = torch.randn(7, 3, dtype=torch.float64, generator=gen, requires_grad=True)
    src = torch.randint(0, 7, (14,), generator=gen)
    dst = torch.randperm(9 * 2, generator=gen)[:14]
    got = mp.fanout_concat(prefix, x, src, dst, 2)
    want = torch.cat([prefix, mp.fanout_scatter(x, src, dst, 18).view(9, 6)], dim=1)
    assert torch.equal(got, want)
    assert torch.autograd.gradcheck(lambda p, t: mp.fanout_concat(p, t, src, dst, 2), (prefix, x))


if __name__ == "__main__":  # pragma: no cover
    sys.exit(pytest.main([__file__, "-q"]))


def test_planned_ops_on_the_cpu_lane(ops) -> None:
    """fanin_reduce_planned returns the plain op's result and an empty plan
    handle on the CPU lane; the *_planned backward ops then equal the plain
    backward ops, and the autograd facade uses them."""

    gen = torch.Generator().manual_seed(11)
    rel = torch.randn(9, 3, dtype=torch.float64, generator=gen)
    src = torch.tensor([0, 2, 4, 6, 8, 1, 3])
    dst = torch.tensor([1, 1, 0, 3, 1, 0, 3])
    g = torch.randn(4, 3, dtype=torch.float64, generator=gen)
    for mode in (0, 1):
        out, plan = ops.fanin_reduce_planned(rel, src, dst, 4, mode)
        assert isinstance(plan, torch.ScriptObject)
        assert torch.equal(out, ops.fanin_reduce(rel, src, dst, 4, mode))
        if mode == 0:
            got = ops.fanin_reduce_sum_backward_planned(g, src, dst, 9, plan)
            want = ops.fanin_reduce_sum_backward(g, src, dst, 9)
        else:
            got = ops.fanin_reduce_logsumexp_backward_planned(g, rel, src, dst, out, 9, plan)
            want = ops.fanin_reduce_logsumexp_backward(g, rel, src, dst, out, 9)
        assert torch.equal(got, want)
    with pytest.raises((RuntimeError, ValueError), match="Unsupported fanin_reduce mode"):
        ops.fanin_reduce_planned(rel, src, dst, 4, 2)


def test_plan_scope_nests_and_survives_errors() -> None:
    """mp.plan_scope enters and leaves the library's trust scope (CPU: nothing
    is served from it; the calls only have to balance)."""

    import torch

    from relmo_amd import mp

    with mp.plan_scope():
        with mp.plan_scope():
            pass
    with pytest.raises(KeyError):
        with mp.plan_scope():
            raise KeyError("x")
    stats = torch.ops.relm_mp.plan_cache_stats()
    assert len(stats) == 7 and stats[6] == 0


def test_relational_gnn_residual_concat_matches_modules() -> None:
    """RelationalGNN writes each predicate's residual MLP output straight into
    the relation rows (_ResidualConcat): the same loss and gradients as
    calling the Residual modules and concatenating their outputs (float64,
    CPU, sum and logsumexp)."""

    import torch

    from relmo_amd import consumers as C
    from relmo_amd import mp

    batch = C.synthetic_c4("cpu", seed=2, num_graphs=3)
    for mode in (0, 1):
        torch.manual_seed(0)
        model = C.RelationalGNN(8, 2, batch.relations, mode).double()
        r = model.routing(batch)
        loss = C.train_step(model, batch, r)
        got = {k: p.grad.clone() for k, p in model.named_parameters()}

        def reference_forward():
            x = torch.zeros(batch.num_objects, model.d, dtype=torch.float64)
            for _ in range(model.num_layers):
                args = mp.fanout_scatter(x, r["obj"], r["flat"], r["total"])
                outs = [model.rel_mlps[pred](args[off:off + n * a].view(n, a * model.d)).view(n * a, model.d)
                        for pred, n, a, off in r["meta"]]
                msgs = C.fanin_objects(mode, torch.cat(outs), r, batch.num_objects)
                x = x + model.updater(torch.cat([x, msgs], dim=1))
            return x

        model.zero_grad(set_to_none=True)
        ref_loss = reference_forward().square().mean()
        ref_loss.backward()
        torch.testing.assert_close(loss, ref_loss.detach(), rtol=1e-12, atol=1e-14)
        for k, p in model.named_parameters():
            torch.testing.assert_close(got[k], p.grad, rtol=1e-10, atol=1e-13, msg=lambda m, k=k: f"{k}: {m}")
