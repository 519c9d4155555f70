from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
GOLDEN = REPO / "tests" / "golden"
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def golden() -> tuple[list[dict], dict[str, np.ndarray]]:
    cases = json.loads((GOLDEN / "reference_cases.json").read_text())
    with np.load(GOLDEN / "reference_cases.npz", allow_pickle=False) as data:
        arrays = {k: data[k] for k in data.files}
    return cases, arrays


@pytest.fixture(scope="session")
def pack_golden() -> tuple[list[dict], dict[str, np.ndarray]]:
    """Pack-op cases written by tests/golden/make_pack_golden.py."""

    cases = json.loads((GOLDEN / "pack_cases.json").read_text())
    with np.load(GOLDEN / "pack_cases.npz", allow_pickle=False) as data:
        arrays = {k: data[k] for k in data.files}
    return cases, arrays


@pytest.fixture(scope="session")
def lgan_golden() -> tuple[list[dict], dict[str, np.ndarray]]:
    """LGAN-op cases written by tests/golden/make_lgan_golden.py."""

    cases = json.loads((GOLDEN / "lgan_cases.json").read_text())
    with np.load(GOLDEN / "lgan_cases.npz", allow_pickle=False) as data:
        arrays = {k: data[k] for k in data.files}
    return cases, arrays


def pack_args(case: dict, arrays: dict[str, np.ndarray], device: str = "cpu") -> list:
    """Arguments of a pack case as torch objects (tensor lists, int lists, ints)."""

    import torch

    def tensor(name: str):
        return torch.from_numpy(np.array(arrays[name])).to(device)

    args: list = []
    for spec in case["args"]:
        if "tensors" in spec:
            args.append([tensor(n) for n in spec["tensors"]])
        elif "tensor" in spec:
            args.append(tensor(spec["tensor"]))
        elif "ints" in spec:
            args.append([int(v) for v in spec["ints"]])
        else:
            args.append(int(spec["int"]))
    return args


@pytest.fixture
def mp_env(monkeypatch: pytest.MonkeyPatch):
    """Custom ops on, and a missing library raises instead of falling back."""

    monkeypatch.setenv("RELM_MP_ENABLE", "1")
    monkeypatch.setenv("RELM_MP_FALLBACK", "error")
    yield


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def require_gpu() -> None:
    if not gpu_available():
        pytest.skip("no GPU visible")


os.environ.setdefault("PYTHONHASHSEED", "0")
