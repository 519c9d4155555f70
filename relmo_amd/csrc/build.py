"""Builds the two shared libraries of relmo_amd in-tree.

* ``relmo_amd/librelm_mp_hip.so`` - the HIP kernels for gfx950 and their C ABI
  (``include/relm_mp.h``), compiled with hipcc; no torch dependency.
* ``relmo_amd/relm_mp_ops.so`` - the ``torch.library`` binding (namespace
  ``relm_mp``), compiled with g++ against the installed torch and linked to the
  HIP library through ``$ORIGIN``.

Run ``python -m relmo_amd.csrc.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import shlex
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent.parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("RELM_MP_OFFLOAD_ARCH", "gfx950")

HIP_SOURCES = ["plan_kernels.hip", "reduce_kernels.hip", "pack_kernels.hip", "match_kernels.hip",
               "film_kernels.hip",
               "capi.hip"]
HIP_LIB = PKG_DIR / "librelm_mp_hip.so"
TORCH_EXT = PKG_DIR / "relm_mp_ops.so"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # Packed FP32 instructions are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-parameter",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        sys.stderr.write(proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {cmd[0]}")
    noise = "packed-fp32-ops"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line).strip()
    if err and verbose:
        sys.stderr.write(err + "\n")


def build_hip_lib(verbose: bool = False) -> Path:
    hipcc = str(ROCM / "bin" / "hipcc")
    obj_dir = PKG_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    objs = [str(obj_dir / (Path(src).stem + ".o")) for src in HIP_SOURCES]
    # one hipcc per source, run side by side (each is single-threaded)
    jobs = max(1, min(len(HIP_SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(lambda so: _run([hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c",
                                       str(CSRC / so[0]), "-o", so[1]], verbose),
                      zip(HIP_SOURCES, objs)))
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-Wl,-soname,librelm_mp_hip.so", "-o", str(tmp)], verbose)
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_torch_ext(verbose: bool = False) -> Path:
    import torch

    tdir = Path(torch.__file__).resolve().parent
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"),
        "-std=c++17",
        "-O2",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-parameter",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        f'-DRELM_MP_BUILD_TORCH_VERSION="{torch.__version__}"',
        f"-I{INCLUDE}",
        f"-I{tdir / 'include'}",
        f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
        f"-I{ROCM / 'include'}",
        str(CSRC / "relm_mp_ops.cpp"),
        f"-L{PKG_DIR}",
        "-lrelm_mp_hip",
        f"-L{tdir / 'lib'}",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-lc10",
        "-lc10_hip",
        "-lhipblas",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{tdir / 'lib'}",
        "-o",
        str(TORCH_EXT.with_suffix(".so.tmp")),
    ]
    _run(cmd, verbose)
    os.replace(TORCH_EXT.with_suffix(".so.tmp"), TORCH_EXT)
    return TORCH_EXT


def build(verbose: bool = False) -> list[Path]:
    return [build_hip_lib(verbose), build_torch_ext(verbose)]


if __name__ == "__main__":
    for path in build(verbose="-v" in sys.argv):
        print(path)
