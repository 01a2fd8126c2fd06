"""Build the gfx950 kernel library and the PyTorch-ROCm extension in-tree.

Outputs (git-ignored, shipped with the source tree):
  gdsllm_amd/libgdsllm_amd.so                  hipcc, every csrc/*.hip, C ABI of include/gdsllm_amd.h
  gdsllm_amd/runtime/gds_io_ext<EXT_SUFFIX>    g++, csrc/gds_io_ext.cpp, links the library above

Every call recompiles from source (the "does it build" check), in parallel.
Run as `python -m gdsllm_amd.build`.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD_DIR = PKG / "_build"
LIB = PKG / "libgdsllm_amd.so"
EXT = PKG / "runtime" / ("gds_io_ext" + sysconfig.get_config_var("EXT_SUFFIX"))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"-I{INCLUDE}",
    # no packed fp32 instructions anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        # hipcc's host pass warns that it does not know the packed-fp32 feature: noise
        err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{err}\n{res.stdout}")


def hipcc() -> str:
    path = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build gdsllm_amd)")
    return path


def build_library(verbose: bool = False, jobs: int = 0) -> Path:
    """Compile csrc/*.hip for gfx950 and link libgdsllm_amd.so."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    cc = hipcc()
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [cc, *HIPCC_FLAGS, "-c", str(s), "-o", str(o)], verbose) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_extension(verbose: bool = False) -> Path:
    """Compile the torch binding (plain C++, no device code) against the library."""
    import torch
    import torch.utils.cpp_extension as ce

    py_inc = sysconfig.get_paths()["include"]
    incs = [str(INCLUDE), py_inc, *ce.include_paths("cuda")]
    libdirs = ce.library_paths("cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = EXT.with_name(EXT.name + ".tmp")
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        str(CSRC / "gds_io_ext.cpp"), "-o", str(tmp),
        *[f"-I{i}" for i in incs],
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=gds_io_ext", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-Wno-deprecated-declarations",
        *[f"-L{d}" for d in libdirs], f"-L{PKG}",
        "-lgdsllm_amd", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN/..", *[f"-Wl,-rpath,{d}" for d in libdirs],
    ]
    _run(cmd, verbose)
    os.replace(tmp, EXT)
    return EXT


def build_all(verbose: bool = False) -> None:
    build_library(verbose)
    build_extension(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print(f"built {LIB.relative_to(ROOT)} and {EXT.relative_to(ROOT)}")
