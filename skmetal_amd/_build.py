"""Build libskmetal_hip.so (gfx950) in-tree with hipcc.

Used by ``__graft_entry__.build()`` and ``python -m skmetal_amd._build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libskmetal_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    # keep the compiler from emitting packed fp32 VALU ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# MFMA accumulators in VGPRs: keeps the runtime-loop-carried accumulators of
# the assign kernel in place instead of rotating them through AGPRs with
# v_accvgpr_* copies
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
# (source, extra flags): the fused kernel keeps its accumulators in AGPRs
SOURCES = [
    ("kmeans_kernels.hip", VGPR_FORM),
    ("fused_kernels.hip", []),
    ("split_kernels.hip", []),
    ("plusplus_kernels.hip", []),
    ("transform_kernels.hip", []),
    ("sample_kernels.hip", []),
    ("skmetal_hip.hip", VGPR_FORM),
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build libskmetal_hip.so")
    return path


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _finish(proc, verbose):
    out, _ = proc.communicate()
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in out.splitlines() if noise not in ln and ln.strip()]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs))


def build(verbose: bool = False) -> Path:
    """Compile every source to an object (in parallel), then link the library."""
    tmp = LIB.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="skmetal_hip_build_") as bdir:
        objs, procs = [], []
        for src, extra in SOURCES:
            obj = str(Path(bdir) / (Path(src).stem + ".o"))
            objs.append(obj)
            procs.append(_run([hipcc(), *HIPCC_FLAGS, *extra, f"-I{ROOT / 'include'}", "-c", str(CSRC / src),
                               "-o", obj], verbose))
        for p in procs:
            _finish(p, verbose)
        _finish(_run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *objs, "-o", str(tmp)], verbose),
                verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
