"""Build `libkvfp8.so` (the gfx950 HIP kernels and their C ABI) in-tree with hipcc.

Usage: python -m aiproj_amd.build   (or aiproj_amd.build.build()).
The library lands next to this file, so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
LIBRARY = PACKAGE_DIR / "libkvfp8.so"
OBJ_DIR = PACKAGE_DIR / "_build"
# Fast-call Python bindings of the per-step entry points (csrc/pyfast.c), a CPython
# extension linked to LIBRARY; _native falls back to ctypes where it is absent.
FAST_EXT = PACKAGE_DIR / ("_kvfp8_fast" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))

ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code.
# -fhip-fp32-correctly-rounded-divide-sqrt: IEEE float32 division, which the
# bit-exact quantizer relies on (scale = amax / 448, code = e4m3(x / scale)).
# No fast-math: the quantizer's NaN/zero handling must follow IEEE.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the kvfp8 HIP library cannot be built")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libkvfp8.so (always rebuilds)."""
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    build_fast_ext(verbose)
    return LIBRARY


def build_fast_ext(verbose: bool = False) -> Path:
    """Compile csrc/pyfast.c into the CPython extension FAST_EXT, linked to libkvfp8.so
    in the same directory (found at run time through an $ORIGIN rpath)."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no host C compiler for the fast-call extension")
    tmp = FAST_EXT.with_suffix(".tmp")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           str(CSRC / "pyfast.c"), f"-L{PACKAGE_DIR}", "-lkvfp8", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"fast-call extension failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, FAST_EXT)
    if verbose:
        print(f"built {FAST_EXT}")
    return FAST_EXT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
