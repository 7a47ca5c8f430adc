"""Builds libinferbit_amd/_build/libibhip.so (gfx950) with hipcc, in-tree.

Usage: python -m libinferbit_amd.build   (or libinferbit_amd.build.build())
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libibhip.so")

SOURCES = ["ibh_runtime.hip", "ibh_gemv.hip", "ibh_mfma.hip", "ibh_rows.hip", "ibh_tile.hip", "ibh_probe.hip", "ibh_attn.hip", "ibh_pq.hip", "ibh_int4g.hip", "ibh_v5.hip", "ibh_decode.hip", "ibh_exact.hip", "ibh_gemm.hip", "ibh_host.cpp", "ibh_spec.cpp", "ibh_sample.cpp", "ibh_v5_sample.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Results must not depend on the compiler fusing a*b+c: every fused
    # multiply-add in the kernels is written as fmaf().
    "-ffp-contract=off",
    # Packed fp32 VALU ops are kept out of the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{ROOT}/include",
]


# Per-source additions.  The prefill GEMM keeps its 96 int32 accumulators in
# VGPRs: with the AGPR form the register allocator copies every accumulator
# through v_accvgpr moves on each K step.
EXTRA_FLAGS = {
    "ibh_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libinferbit_amd")
    return p


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
    return r.returncode


def build(verbose: bool = False) -> str:
    """Compiles every source to an object (in parallel), then links the .so."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OUT_DIR, exist_ok=True)
    cc = hipcc()
    objs = [os.path.join(OUT_DIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(s, []), "-c", os.path.join(CSRC, s), "-o", o]
            for s, o in zip(SOURCES, objs)]
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as ex:
        codes = list(ex.map(lambda c: _run(c, verbose), cmds))
    if any(codes):
        raise RuntimeError("hipcc failed building libibhip.so: " +
                           ", ".join(s for s, c in zip(SOURCES, codes) if c))
    tmp = LIB + ".tmp"
    if _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose):
        raise RuntimeError("hipcc failed linking libibhip.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
