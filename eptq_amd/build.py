"""Build ``eptq_amd/_lib/libeptq_hip.so`` for gfx950 with hipcc (in-tree).

Usage: ``python -m eptq_amd.build``.  Compiles every time it is called.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
SOURCES = ["abi.hip", "dequant.hip", "matvec.hip", "decode.hip", "decode_mfma.hip", "gemm.hip", "llama_ops.hip"]
OUT = ROOT / "_lib" / "libeptq_hip.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # IEEE fp32 everywhere: no multiply-add contraction (bit-exact dequant).
    "-ffp-contract=off",
    # Keep the compiler from emitting packed fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def _finish(proc, what):
    _, err = proc.communicate()
    errs = "\n".join(l for l in err.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {what} ({proc.returncode}):\n{errs}")


def build(verbose: bool = False) -> Path:
    """Compile the sources in parallel (one object each), then link."""
    OUT.parent.mkdir(parents=True, exist_ok=True)
    objdir = OUT.parent / "obj"
    objdir.mkdir(exist_ok=True)
    inc = [f"-I{REPO / 'include'}", f"-I{ROOT / 'csrc'}"]
    objs, procs = [], []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        objs.append(str(obj))
        procs.append((_run([hipcc(), *HIPCC_FLAGS, *inc, "-c", str(ROOT / "csrc" / src), "-o", str(obj)],
                           verbose), src))
    for proc, src in procs:
        _finish(proc, src)
    tmp = OUT.with_suffix(".so.tmp")
    _finish(_run([hipcc(), *HIPCC_FLAGS, "-shared", *objs, "-o", str(tmp)], verbose), "link")
    os.replace(tmp, OUT)
    shutil.rmtree(objdir, ignore_errors=True)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
