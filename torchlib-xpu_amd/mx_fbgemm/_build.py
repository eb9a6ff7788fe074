"""In-tree build of the two native libraries of mx_fbgemm.

* ``lib/libmx_fbgemm_kernels.so`` -- the hand-written gfx950 HIP kernels and
  their C-ABI (``include/mx_fbgemm.h``), built with hipcc, no torch types.
* ``lib/mx_fbgemm_ops.so`` -- the PyTorch-ROCm extension that registers the
  ``torch.ops.fbgemm.*`` schemas and calls the C-ABI; built with g++ against
  the installed torch and linked to the kernel library through ``$ORIGIN``.

The build always recompiles (it is the "does it build" check); callers that
only need the libraries load what is already there.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
PROJ_DIR = PKG_DIR.parent  # torchlib-xpu_amd/
REPO_DIR = PROJ_DIR.parent
CSRC = PROJ_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
BUILD_DIR = PROJ_DIR / "_build"
LIB_DIR = PKG_DIR / "lib"

KERNEL_LIB = LIB_DIR / "libmx_fbgemm_kernels.so"
OPS_LIB = LIB_DIR / "mx_fbgemm_ops.so"

HIP_SOURCES = ["abi.hip", "jagged.hip", "tbe_fwd.hip", "tbe_bwd.hip", "nbit_fwd.hip",
               "bounds_check.hip", "codec.hip", "vbe.hip", "sparse_ops.hip"]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed FP32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wextra",
    "-Werror",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def _hipcc() -> str:
    exe = ROCM / "bin" / "hipcc"
    return str(exe) if exe.exists() else "hipcc"


def build_kernels(verbose: bool = False, jobs: int | None = None) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([_hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c",
                     str(CSRC / src), "-o", str(obj)])
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        for fut in [ex.submit(_run, c, verbose) for c in cmds]:
            fut.result()
    tmp = KERNEL_LIB.with_suffix(".so.tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o",
          str(tmp)], verbose)
    os.replace(tmp, KERNEL_LIB)
    return KERNEL_LIB


def build_ops(verbose: bool = False) -> Path:
    import torch
    from torch.utils import cpp_extension

    LIB_DIR.mkdir(parents=True, exist_ok=True)
    inc = [f"-I{p}" for p in cpp_extension.include_paths()]
    libdirs = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS_LIB.with_suffix(".so.tmp")
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Werror",
        "-Wno-unused-parameter",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=mx_fbgemm_ops", "-DTORCH_API_INCLUDE_EXTENSION_H",
        *inc, f"-I{ROCM / 'include'}", f"-I{INCLUDE}",
        str(CSRC / "ops.cpp"), "-o", str(tmp),
        *[f"-L{d}" for d in libdirs], f"-L{LIB_DIR}",
        "-lmx_fbgemm_kernels", "-ltorch_hip", "-lc10_hip", "-ltorch_cpu", "-lc10", "-ltorch",
        "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs],
    ]
    _run(cmd, verbose)
    os.replace(tmp, OPS_LIB)
    return OPS_LIB


def build(verbose: bool = False) -> None:
    if not shutil.which(_hipcc()) and not Path(_hipcc()).exists():
        raise RuntimeError("hipcc not found; set ROCM_PATH")
    build_kernels(verbose)
    build_ops(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(f"built {KERNEL_LIB} and {OPS_LIB}")
