"""Build recipe for libwmx_attn.so (gfx950) from white_matter_amd/csrc.

Each .hip translation unit is compiled with hipcc for gfx950 only, then the
objects are linked into one shared library next to this file. Packed-FP32
instructions are disabled for all device code.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
REPO = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = REPO / "include"
LIBRARY = PACKAGE / "lib" / "libwmx_attn.so"
OPS_LIBRARY = PACKAGE / "lib" / "libwmx_torch.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _torch_flags() -> tuple[list[str], list[str]]:
    import torch

    root = Path(torch.__file__).resolve().parent
    lib = root / "lib"
    compile_flags = [
        "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
        "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        f"-I{root / 'include'}", f"-I{root / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
        "-I/opt/rocm/include", f"-I{INCLUDE}",
    ]
    link_flags = [
        f"-L{LIBRARY.parent}", "-lwmx_attn", f"-L{lib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{lib}",
    ]
    return compile_flags, link_flags


def build_ops(verbose: bool = False) -> Path:
    """Compile the C++ operator registrations (csrc/torch_ops.cpp, host code
    only) against libtorch and libwmx_attn.so into libwmx_torch.so."""
    compile_flags, link_flags = _torch_flags()
    tmp = OPS_LIBRARY.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), *compile_flags, "-shared", str(CSRC / "torch_ops.cpp"), "-o", str(tmp), *link_flags]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"building libwmx_torch.so failed:\n{proc.stderr}")
    os.replace(tmp, OPS_LIBRARY)
    return OPS_LIBRARY


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950, link libwmx_attn.so, then build the
    C++ operator library on top of it."""
    hipcc = _hipcc()
    out_dir = LIBRARY.parent
    obj_dir = out_dir / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        objects = list(pool.map(compile_one, sources()))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    build_ops(verbose)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
