"""Build libmxgg.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

The shared library lands next to this file so that it travels with the
source tree; nothing is installed into site-packages.
"""
from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR.parent / "csrc"
INCLUDE_DIR = PKG_DIR.parent.parent / "include"
BUILD_DIR = PKG_DIR.parent / "_build"
LIB_PATH = PKG_DIR / "libmxgg.so"

SOURCES = ["capi.hip", "quant.hip", "swiglu.hip", "route.hip", "groups.hip", "gemm.hip"]
HEADERS = ["mxgg_internal.h", "mx_device.h"]

ARCH = os.environ.get("MXGG_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep v_pk_{add,mul,fma}_f32 out of the generated code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
]


def hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return cand


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line.
    out = "\n".join(
        ln for ln in proc.stdout.splitlines()
        if "packed-fp32-ops" not in ln and "--hip-link" not in ln
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build(verbose: bool = True) -> Path:
    """Compile every HIP source for gfx950 and link libmxgg.so (always rebuilds)."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([cc, *HIPCC_FLAGS, "-c", str(CSRC_DIR / src), "-o", str(obj)])
    with _cf.ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[mxfp8gg] built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
