"""Build libace_hip.so (the C-ABI of the HIP kernels) for gfx950 with hipcc,
and _ace_autograd.so (the loss call and its backward node in C++ over that
C-ABI) with g++ against torch's headers.

    python ace-kernels_amd/build.py            # compile + link
    python ace-kernels_amd/build.py --check    # also print kernel resource usage

Each translation unit under csrc/ is compiled to an object in parallel, then
linked into ace_kernels/libace_hip.so, next to the Python package that loads
it.  Every HIP compile line carries
``-Xclang -target-feature -Xclang -packed-fp32-ops`` (no packed fp32 VALU) and
``-ffp-contract=off`` (no implicit FMA contraction: the probabilities and bin
weights must be rounded exactly as written).
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
OUT_DIR = HERE / "ace_kernels"
LIB = OUT_DIR / "libace_hip.so"
AUTOGRAD_SRC = CSRC / "ace_autograd.cpp"
AUTOGRAD_LIB = OUT_DIR / "_ace_autograd.so"
OBJ_DIR = HERE / "_build"

ARCH = os.environ.get("ACE_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def _compile(src: Path, extra: list, incremental: bool = False) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    if incremental and obj.exists():
        deps = [src, *CSRC.glob("*.hpp"), *INCLUDE.glob("*.h")]
        if obj.stat().st_mtime > max(d.stat().st_mtime for d in deps):
            return obj
    cmd = [hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stderr}")
    return obj


def _build_autograd(incremental: bool = False) -> Path:
    """g++ -shared ace_autograd.cpp -> ace_kernels/_ace_autograd.so (a Python
    extension module: pybind11 and torch's headers; host code only, it calls
    libace_hip.so through entry points handed over at load time)."""
    out = AUTOGRAD_LIB
    if incremental and out.exists():
        deps = [AUTOGRAD_SRC, *INCLUDE.glob("*.h")]
        if out.stat().st_mtime > max(d.stat().st_mtime for d in deps):
            return out
    import sysconfig

    import torch
    from torch.utils.cpp_extension import include_paths

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    tmp = out.with_suffix(".so.tmp")
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
        str(AUTOGRAD_SRC), "-o", str(tmp),
        f"-I{sysconfig.get_paths()['include']}", *(f"-I{p}" for p in include_paths()),
        f"-I{INCLUDE}", "-I/opt/rocm/include",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_ace_autograd", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        f"-Wl,-rpath,{torch_lib}",
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for {AUTOGRAD_SRC.name}:\n{' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False, extra: list | None = None, incremental: bool = False) -> Path:
    """Compile every csrc/*.hip and link ace_kernels/libace_hip.so, and build
    ace_kernels/_ace_autograd.so; return the library's path.
    ``incremental``: skip objects newer than their source and every header."""
    extra = list(extra or [])
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources) + 1, max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as pool:
        autograd = pool.submit(_build_autograd, incremental)
        objs = list(pool.map(lambda s: _compile(s, extra, incremental), sources))
        autograd.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources, and {AUTOGRAD_LIB}")
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true", help="print register/LDS usage (-Rpass-analysis)")
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only objects older than their source or a header")
    args = ap.parse_args()
    extra = ["-Rpass-analysis=kernel-resource-usage"] if args.check else []
    if args.check:
        OBJ_DIR.mkdir(exist_ok=True)
        for src in sorted(CSRC.glob("*.hip")):
            cmd = [hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(OBJ_DIR / (src.stem + ".o"))]
            res = subprocess.run(cmd, capture_output=True, text=True)
            sys.stdout.write(res.stderr)
    build(verbose=True, incremental=args.incremental)
    return 0


if __name__ == "__main__":
    sys.exit(main())
