"""Build of the HIP decode-step library (``libmkd_decode.so``), in-tree.

The reference JIT-compiles a torch extension with nvcc
(``backends/megakernel/build.py:59-93``). Here the kernels are plain HIP
compiled once by ``hipcc`` for gfx950 into a C-ABI shared library next to this
file; Python binds it with ctypes (:mod:`.native`). Build flags:

* ``--offload-arch=gfx950 -O3 -std=c++17 -fPIC -shared``;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps packed-FP32 VALU
  instructions out of the generated code;
* ``MKD_ARCH`` overrides the architecture (for experiments only).
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG_ROOT = HERE.parents[2]          # decode-fusion-boundary_amd/
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_NAME = "libmkd_decode.so"
LIB_PATH = HERE / LIB_NAME
SOURCES = ("mkd_decode.hip",)
TORCH_OPS_NAME = "libmkd_torch_ops.so"
TORCH_OPS_PATH = HERE / TORCH_OPS_NAME
TORCH_OPS_SOURCE = "mkd_torch_ops.cpp"
HEADERS = ("mkd_common.h", "mkd_tasks.h")


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else "hipcc"


def compile_command(out: Path = LIB_PATH) -> list[str]:
    arch = os.environ.get("MKD_ARCH", "gfx950")
    return [
        hipcc(),
        f"--offload-arch={arch}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # Each kernel starts on a 4 KiB boundary, so its instruction-cache set
        # mapping no longer depends on the size of the kernels placed before it:
        # the batch-8 kernel (larger than the 64 KiB instruction cache two CUs
        # share) measured 834 vs 862 us per step with identical code at two
        # offsets, and 833 us aligned.
        "-falign-functions=4096",
        f"-I{INCLUDE}",
        "-o", str(out),
        *[str(CSRC / s) for s in SOURCES],
    ]


def torch_ops_command(out: Path = TORCH_OPS_PATH) -> list[str]:
    """Host-only C++ compile of the torch operator shim against the installed
    PyTorch-ROCm headers and libraries, linked to ``libmkd_decode.so`` (found
    next to it at run time through ``$ORIGIN``)."""

    import torch

    tdir = Path(torch.__file__).resolve().parent
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    abi = int(torch.compiled_with_cxx11_abi())
    return [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-I{INCLUDE}", f"-I{tdir / 'include'}", f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
        f"-I{rocm}/include",
        "-o", str(out), str(CSRC / TORCH_OPS_SOURCE),
        f"-L{HERE}", "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN",
        f"-L{tdir / 'lib'}", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_hip",
        f"-Wl,-rpath,{tdir / 'lib'}", f"-L{rocm}/lib", "-lamdhip64",
    ]


def _run(cmd: list[str], out: Path, final: Path, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd))
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed ({proc.returncode}):\n{proc.stderr[-4000:]}")
    os.replace(out, final)


def build(verbose: bool = False, torch_ops: bool = True) -> Path:
    """Compile the library and, unless ``torch_ops`` is False, the torch
    operator shim (always; the caller decides when to rebuild)."""

    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run(compile_command(tmp), tmp, LIB_PATH, verbose)
    if torch_ops:
        tmp = TORCH_OPS_PATH.with_suffix(".so.tmp")
        _run(torch_ops_command(tmp), tmp, TORCH_OPS_PATH, verbose)
    return LIB_PATH


def library_path() -> Path:
    return LIB_PATH


def get_extension():
    """Load the built library (build it if it is missing). Mirrors the reference
    ``get_extension()`` entry point name."""

    from . import native

    if not LIB_PATH.exists():
        build()
    return native.load()
