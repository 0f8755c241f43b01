"""Compile the HIP kernels + C ABI into ``mla_kv_quant_amd/librolaq_mla.so`` (gfx950).

Usage: ``python -m mla_kv_quant_amd.build`` (or ``__graft_entry__.build()``).
Cross-compiles without a GPU. Packed FP32 instructions are disabled for the
device code (``-packed-fp32-ops``); hipcc's host pass warns about the unknown
feature, which is harmless.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
ROOT = HERE.parent
LIB = HERE / "librolaq_mla.so"
SOURCES = ["api.cpp", "pack.hip", "writer.hip", "decode.hip", "extend.hip", "assemble.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")


def common_flags() -> list[str]:
    return [
        "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", str(ROOT / "include"), "-I", str(CSRC),
        "-Wall", "-Wno-unused-function",
    ]


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    cc = hipcc()
    objdir = HERE / "_obj"
    objdir.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = objdir / (src + ".o")
        objs.append(obj)
        lang = ["-x", "hip"] if src.endswith(".hip") else ["-x", "hip"]
        cmds.append([cc, *common_flags(), *lang, "-c", str(CSRC / src), "-o", str(obj)])

    def run(cmd):
        res = subprocess.run(cmd, capture_output=True, text=True)
        out = (res.stdout + res.stderr).strip()
        # hipcc's host pass does not know the device-only feature; drop that noise
        lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and "not a recognized feature" not in ln]
        return res.returncode, "\n".join(lines), cmd

    with ThreadPoolExecutor(max_workers=jobs or min(8, len(cmds))) as ex:
        results = list(ex.map(run, cmds))
    for rc, out, cmd in results:
        if verbose and out:
            print(out, file=sys.stderr)
        if rc != 0:
            raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{out}")
    tmp = LIB.with_suffix(".so.tmp")
    link = [cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(link, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(link)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
