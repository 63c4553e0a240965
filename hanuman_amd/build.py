"""Builds ``libhanuman_moe.so`` (the C-ABI library of HIP kernels) in-tree.

Plain ``hipcc`` for gfx950: every ``csrc/*.hip`` file is compiled to an object
in ``hanuman_amd/_build`` (in parallel), then linked into
``hanuman_amd/libhanuman_moe.so``.  Run ``python -m hanuman_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libhanuman_moe.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-gpu-rdc",
    # Packed fp32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Router gates rely on correctly rounded float32 division.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build hanuman_amd")
    return path


# Per-file flags.  gemm.hip: no wave-level aggregation of atomics (the fused
# launch's claims are made by one lane and their results are read a K step
# later; the aggregation would read the result, and wait for every memory
# operation in flight, right after the atomic).
FILE_FLAGS = {
    "gemm.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, flush=True)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fno-gpu-rdc", *map(str, objs),
           "-o", str(tmp), "-Wl,-rpath,/opt/rocm/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


XLA_FFI_SRC = PKG / "xla_ffi" / "hmoe_xla_ffi.cc"
XLA_FFI_LIB = PKG / "xla_ffi" / "libhanuman_moe_xla.so"


def build_xla_ffi(verbose: bool = False) -> Path | None:
    """Compiles the XLA FFI handlers (``xla_ffi/hmoe_xla_ffi.cc``) against
    JAX's FFI headers and links them to ``libhanuman_moe.so``; returns None
    (and builds nothing) when JAX is not importable, since the headers ship
    with it."""
    import importlib.util
    if importlib.util.find_spec("jax") is None:
        if verbose:
            print("xla_ffi: jax is not importable here; the handlers are not built", flush=True)
        return None
    import jax  # noqa: PLC0415
    inc = jax.ffi.include_dir()
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-shared",
           f"-I{inc}", f"-I{ROOT / 'include'}", str(XLA_FFI_SRC), f"-L{PKG}", "-lhanuman_moe",
           "-Wl,-rpath,$ORIGIN/..", "-o", str(XLA_FFI_LIB)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"xla_ffi build failed:\n{r.stdout}{r.stderr}")
    return XLA_FFI_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    build_xla_ffi(verbose=True)
