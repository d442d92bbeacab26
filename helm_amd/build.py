"""Build libhelm_mi355x.so (gfx950) in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object in parallel, then linked into
``helm_amd/libhelm_mi355x.so``.  The host-side page walk of
perform_streaming_attention (``csrc/page_walk.c``) is built with gcc as the
CPython module ``helm_amd._page_walk``.  Run as ``python -m helm_amd.build``
(``--incremental``: recompile only sources changed since their object).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ_DIR = PKG / "_build"
LIB_NAME = "libhelm_mi355x.so"
LIB_PATH = PKG / LIB_NAME
ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled for all device code (the host pass warns that
# it does not know the feature; that warning is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(hipcc: str, src: pathlib.Path) -> pathlib.Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def _stale(src: pathlib.Path, deps) -> bool:
    obj = OBJ_DIR / (src.stem + ".o")
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return any(d.stat().st_mtime > t for d in (src, *deps))


def build_page_walk(verbose: bool = False) -> pathlib.Path:
    """Compile csrc/page_walk.c into the extension module helm_amd/_page_walk."""
    import sysconfig
    out = PKG / ("_page_walk" + sysconfig.get_config_var("EXT_SUFFIX"))
    cc = os.environ.get("CC") or shutil.which("gcc") or "gcc"
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", "-Werror", f"-I{sysconfig.get_paths()['include']}",
           str(CSRC / "page_walk.c"), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"[helm_amd.build] {out}")
    return out


def build(verbose: bool = False, incremental: bool = False) -> pathlib.Path:
    """Compile every HIP source and link the shared library; returns its path.
    With `incremental`, only sources newer than their object (or whose shared
    headers changed) are recompiled."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    deps = [*CSRC.glob("*.h"), PKG.parent / "include" / "helm_mi355x.h"]
    todo = [s for s in sources if not incremental or _stale(s, deps)]
    jobs = max(1, min(len(todo), 8, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda s: _compile(hipcc, s), todo))
    objs = [OBJ_DIR / (s.stem + ".o") for s in sources]
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[helm_amd.build] {LIB_PATH} ({len(objs)} objects)")
    build_page_walk(verbose)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv)
    sys.exit(0)
