"""Builds the gfx950 HIP library liblamq_hip.so in-tree from csrc/*.hip with hipcc.

    python -m lookatmyquant_amd.build

Every translation unit is compiled with -ffp-contract=off (each rounding step is the one written in the
source; fused multiply-adds appear only where fma() is called) and with packed FP32 instructions disabled.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "liblamq_hip.so"
ARCH = os.environ.get("LAMQ_OFFLOAD_ARCH", "gfx950")

FLAGS = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-ffp-contract=off", "-fno-fast-math",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]


# Per-file additions. The fp64 MFMA kernels keep their accumulators in VGPR-form MFMAs (-amdgpu-mfma-vgpr-form): left
# to itself, the register allocator carries them around the k-loop in VGPRs and copies them into AGPRs every stage,
# and AGPR-form f64 MFMAs measured at half the rate of VGPR-form ones (34.7 against 68.6 TFLOP/s on a pure MFMA loop).
# The trellis searches never produce a NaN (costs are finite or +inf, and inf - inf never forms), so they are
# built with -fno-honor-nans: a group's minimum is then a v_min/v_min3 tree, which needs no compare masks and spares
# the hazard waits of compare-select pairs.
FILE_FLAGS = {"ldlq.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"], "chol.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
              "rht.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
              "viterbi.hip": ["-fno-honor-nans"], "viterbi16.hip": ["-fno-honor-nans"]}


def hipcc() -> str:
    h = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(h).exists():
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    return h


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip to an object and link liblamq_hip.so; always recompiles."""
    srcs = sorted(CSRC.glob("*.hip"))
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [cc, *FLAGS, *FILE_FLAGS.get(src.name, []), "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
        if verbose and err.strip():
            print(err, file=sys.stderr)
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    r = subprocess.run([cc, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
