"""Build libflower_amd.so in-tree with hipcc for gfx950.

    python -m flower_amd._build          # compile all HIP sources into flower_amd/libflower_amd.so

The product: one shared object, C ABI only (include/flower_amd.h). Beside it, and never linked
into it, the diagnostics library flower_amd/libflower_amd_diag.so (csrc/diag/flw_diag.h: device
arithmetic checks and the issue-cost probe that tests and bench.py load). Every HIP source is
compiled with packed FP32 instructions disabled (``-target-feature -packed-fp32-ops``); sources
compile in parallel into ``_build/`` and are linked with ``hipcc -shared``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJDIR = os.path.join(ROOT, "_build")
LIB = os.path.join(HERE, "libflower_amd.so")
DIAG_LIB = os.path.join(HERE, "libflower_amd_diag.so")
SOURCES = ["flw_error.hip", "flw_quant.hip", "flw_swa.hip", "flw_swa_bf16.hip", "flw_gemm.hip", "flw_heads.hip", "flw_norm_act.hip"]
# The diagnostics library: its own source plus its own copy of the error / timing state.
DIAG_SOURCES = ["diag/flw_diag.hip"]
ARCH = os.environ.get("FLW_OFFLOAD_ARCH", "gfx950")

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]
# Attention: MFMA accumulators in ordinary VGPRs (the online-softmax rescale works on them in
# place instead of copying through AGPRs), and no IEEE mode, since in IEEE mode every fmax operand
# of the row max is first re-quietened (one extra VALU op per score); NaN inputs still give NaN
# rows without it. The other sources keep the compiler's default forms.
PER_SOURCE = {"flw_swa.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-fno-honor-nans", "-mno-amdgpu-ieee"]}
NOISE = "'-packed-fp32-ops' is not a recognized feature"


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libflower_amd")


def _run_all(cmds, verbose):
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    errors = []
    for cmd, pr in procs:
        _, err = pr.communicate()
        err = "\n".join(l for l in err.splitlines() if NOISE not in l)
        if pr.returncode != 0:
            errors.append(f"{cmd[-3] if len(cmd) > 3 else cmd}: hipcc failed ({pr.returncode}):\n{err}")
        elif verbose and err.strip():
            print(err, file=sys.stderr)
    if errors:
        raise RuntimeError("\n".join(errors))


def _obj(source: str) -> str:
    return os.path.join(OBJDIR, os.path.basename(source).replace(".hip", ".o"))


def build(verbose: bool = False) -> str:
    """Compile every source and link both libraries; returns the product library's path."""
    os.makedirs(OBJDIR, exist_ok=True)
    cc = hipcc()
    cmds = [[cc, *COMMON, *PER_SOURCE.get(s, []), "-c", os.path.join(CSRC, s), "-o", _obj(s)]
            for s in SOURCES + DIAG_SOURCES]
    _run_all(cmds, verbose)
    links = []
    for lib, srcs in ((LIB, SOURCES), (DIAG_LIB, DIAG_SOURCES + ["flw_error.hip"])):
        links.append([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(_obj, srcs), "-o", lib + ".tmp"])
    _run_all(links, verbose)
    for lib in (LIB, DIAG_LIB):
        os.replace(lib + ".tmp", lib)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
