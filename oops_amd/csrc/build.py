"""Build ``oops_amd/lib/liboops_amd.so`` from the HIP sources with hipcc for gfx950.

The library is a plain C-ABI shared object.  It is linked against the HIP
runtime that PyTorch-ROCm ships (``torch/lib/libamdhip64.so``, which has no
SONAME, so the dependency is recorded as ``libamdhip64.so``); a process that
already imported torch then resolves it to torch's copy, so a single HIP
runtime serves both.  Without torch the loader falls back to ``/opt/rocm/lib``
through the RUNPATH.

Usage: ``python -m oops_amd.csrc.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
REPO = PKG.parent
LIB_DIR = PKG / "lib"
OBJ_DIR = REPO / "_build" / "oops_amd"
LIB_NAME = "liboops_amd.so"

SOURCES = (
    "attn_fwd.hip",
    "attn_fwd_fast.hip",
    "attn_bwd.hip",
    "attn_bwd_fast.hip",
    "attn_bwd_fused.hip",
    "gate.hip",
    "trimul.hip",
    "trimul_f32.hip",
    "reduce.hip",
    "capi.cpp",
)
FAST_MATH_SOURCES = ("attn_fwd_fast.hip", "attn_bwd_fast.hip", "attn_bwd_fused.hip")
ARCH = "gfx950"


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the oops_amd HIP library cannot be built")


def _torch_lib_dir() -> Path | None:
    try:
        import importlib.util

        spec = importlib.util.find_spec("torch")
    except Exception:  # pragma: no cover - torch absent
        return None
    if spec is None or spec.origin is None:
        return None
    lib = Path(spec.origin).parent / "lib"
    return lib if (lib / "libamdhip64.so").exists() else None


def _compile(src: str, hipcc: str, extra: list[str]) -> Path:
    obj = OBJ_DIR / (Path(src).stem + ".o")
    cmd = [
        hipcc,
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-mcode-object-version=5",
        # gfx950: keep fp32 arithmetic on scalar-lane VALU ops
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        "-I",
        str(REPO / "include"),
        *extra,
        "-c",
        str(HERE / src),
        "-o",
        str(obj),
    ]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    if src in FAST_MATH_SOURCES:
        # min/max without NaN canonicalisation (the kernels select masked
        # scores explicitly and never test for NaN)
        cmd[1:1] = ["-mno-amdgpu-ieee", "-fno-honor-nans"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr[-8000:]}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library; returns its path."""

    hipcc = _hipcc()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    extra = [f for f in os.environ.get("OOPS_HIPCC_FLAGS", "").split() if f]
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as pool:
        objs = list(pool.map(lambda s: _compile(s, hipcc, extra), SOURCES))
    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    # Host link with the system C++ driver: the device code is already embedded
    # in each object, and hipcc's own link line would add /opt/rocm's runtime.
    link = [shutil.which("g++") or "c++", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    torch_lib = _torch_lib_dir()
    rpaths = []
    if torch_lib is not None:
        # record the dependency as "libamdhip64.so" (torch's copy has no SONAME)
        link += ["-Wl,--no-as-needed", str(torch_lib / "libamdhip64.so")]
        rpaths.append(str(torch_lib))
    else:
        link += ["-L/opt/rocm/lib", "-lamdhip64"]
    rpaths.append("/opt/rocm/lib")
    link += [f"-Wl,-rpath,{':'.join(rpaths)}", "-Wl,--enable-new-dtags"]
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-8000:]}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build()
    sys.exit(0)
