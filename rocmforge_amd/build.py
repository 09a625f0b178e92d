"""Build librocmforge_cdna4.so (all HIP kernels + C-ABI launchers) in-tree.

hipcc cross-compiles for gfx950 without a GPU.  Every HIP source is built
with packed-FP32 instruction selection disabled (the compiler flag below),
and the library is linked as one shared object that exports exactly the
symbols declared in include/rocmforge_cdna4.h.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "librocmforge_cdna4.so"
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
SOURCES = ["runtime.hip", "gemv_q4k.hip", "gemv_q6k.hip", "gemm_qk.hip", "model_ops.hip", "mfma_peak.hip",
           "dispatch.cpp"]
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-pass-failed",
]


# Per-source extras.  model_ops.hip: the prefill attention (its only MFMA
# kernel) rescales and reads its accumulators with VALU every key tile; with
# them in AGPRs each tile paid ~350 accvgpr moves, in VGPRs none.
EXTRA = {"model_ops.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = []
    srcs = [s for s in SOURCES if (CSRC / s).exists()]
    procs = []
    for s in srcs:
        obj = BUILD / (Path(s).stem + ".o")
        cmd = [HIPCC, *FLAGS, *EXTRA.get(s, []), "-c", str(CSRC / s), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
        objs.append(str(obj))
    for cmd, p in procs:
        _, err = p.communicate()
        if p.returncode != 0:
            err = "\n".join(l for l in err.splitlines() if "packed-fp32-ops" not in l)
            raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *objs])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
