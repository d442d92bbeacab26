"""Build the reference's own CPU GEMV into oracle/_ref/ — TEST INFRASTRUCTURE ONLY.

The reference's only native code is helm/kernels/fp16_gemv.cpp, a pybind11
torch extension (helm_fp16_linear).  The reference builds it at import time with
torch.utils.cpp_extension.load and the flags -O3 -march=native -ffast-math
-fopenmp (helm/kernels/__init__.py:37-46).  This recipe compiles that one source
file where it lies under /root/reference with g++ directly, against the torch
headers and libraries installed with torch, into
oracle/_ref/helm_fp16_gemv_ref<python extension suffix> (the reference's
flags) and oracle/_ref/helm_fp16_gemv_ref_strict<suffix> (the same without
-ffast-math).  -march=native is replaced by -mavx2 -mfma -mf16c (the
instruction sets the file's intrinsics use), so the modules also run on a host
CPU other than this one.

The module is a checker and a CPU baseline, never a product path:
tests/test_oracle_linear.py compares the oracle's C restatement
(gemv_ref.c) with it, and bench.py's cpu_baseline may time it.  Nothing is
copied out of the reference: the source is read in place, and only the
compiled module is written (into oracle/_ref/, which git ignores).

Usage: python -m oracle.build_ref   (a no-op when /root/reference is absent)
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import pathlib
import subprocess
import sys
import sysconfig
from typing import Optional

HERE = pathlib.Path(__file__).resolve().parent
REF_SRC = pathlib.Path("/root/reference/helm/kernels/fp16_gemv.cpp")
OUT_DIR = HERE / "_ref"
SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
# module name -> floating-point flags: the reference's own (-ffast-math lets the
# compiler reassociate the final accumulator and horizontal sums), and the same
# source with the summation order as written (no -ffast-math)
VARIANTS = {"helm_fp16_gemv_ref": ["-ffast-math"], "helm_fp16_gemv_ref_strict": []}


def _path(module: str) -> pathlib.Path:
    return OUT_DIR / (module + SUFFIX)


def build(verbose: bool = False, force: bool = False) -> Optional[pathlib.Path]:
    """Compile the reference's fp16_gemv.cpp into oracle/_ref/ (both variants;
    skipped for a module newer than the source and this recipe unless `force`);
    None when the reference tree is not present (the GPU host uses the modules
    built here)."""
    if not REF_SRC.exists():
        return None
    from torch.utils import cpp_extension as ce
    OUT_DIR.mkdir(exist_ok=True)
    inc = [f"-I{p}" for p in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}"]
    libdirs = ce.library_paths()
    newest = max(REF_SRC.stat().st_mtime, pathlib.Path(__file__).stat().st_mtime)
    for module, fp_flags in VARIANTS.items():
        out = _path(module)
        if not force and out.exists() and out.stat().st_mtime > newest:
            continue
        obj = OUT_DIR / (module + ".o")
        # compile with the floating-point flags, link without them: linking with
        # -ffast-math would add the start-up code that sets flush-to-zero /
        # denormals-are-zero for the whole process that loads the module
        compile_cmd = ["g++", "-O3", "-mavx2", "-mfma", "-mf16c", *fp_flags, "-fopenmp",
                       "-std=c++17", "-fPIC", f"-DTORCH_EXTENSION_NAME={module}",
                       "-DTORCH_API_INCLUDE_EXTENSION_H", "-D_GLIBCXX_USE_CXX11_ABI=1", *inc, "-c",
                       str(REF_SRC), "-o", str(obj)]
        link_cmd = ["g++", "-shared", "-fPIC", str(obj), "-o", str(out) + ".tmp",
                    *[f"-L{d}" for d in libdirs], *[f"-Wl,-rpath,{d}" for d in libdirs], "-lc10",
                    "-ltorch", "-ltorch_cpu", "-ltorch_python", "-fopenmp"]
        for cmd in (compile_cmd, link_cmd):
            proc = subprocess.run(cmd, capture_output=True, text=True)
            if proc.returncode != 0:
                raise RuntimeError(f"reference GEMV build failed: {' '.join(cmd)}\n{proc.stderr[-4000:]}")
        obj.unlink()
        pathlib.Path(str(out) + ".tmp").replace(out)
        if verbose:
            print(f"[oracle.build_ref] {out}")
    return _path("helm_fp16_gemv_ref")


def load(strict: bool = False):
    """The built reference module (exposes helm_fp16_linear), or None: the
    reference's own flags, or with `strict` the same source without -ffast-math."""
    module = "helm_fp16_gemv_ref_strict" if strict else "helm_fp16_gemv_ref"
    out = _path(module)
    if not out.exists():
        return None
    import torch  # noqa: F401  (the module links against torch's libraries)
    loader = importlib.machinery.ExtensionFileLoader(module, str(out))
    spec = importlib.util.spec_from_file_location(module, str(out), loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    return mod


if __name__ == "__main__":
    built = build(verbose=True)
    if built is None:
        print("[oracle.build_ref] /root/reference not present; nothing built")
    sys.exit(0)
