"""Build the LVSA HIP library (gfx950) in-tree with hipcc.

    python -m longvideosparseattention_amd.build_lib [--verbose]

Produces ``longvideosparseattention_amd/_lib/liblvsa_amd.so``: the C-ABI
declared in ``include/lvsa_amd.h``.  It links only the HIP runtime (no torch),
so any host language can bind it.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB_DIR = PKG / "_lib"
LIB = LIB_DIR / "liblvsa_amd.so"
SOURCES = ["lvsa_mask.hip", "lvsa_attn.hip"]
ARCH = os.environ.get("LVSA_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    f"--offload-arch={ARCH}",
    # Keep hipcc from forming packed fp32 ops (v_pk_fma_f32 & co.).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in arch VGPRs (the softmax reads them with VALU); AGPRs are
    # then left to the register allocator for spills of long-lived values.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-fvisibility=hidden",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build liblvsa_amd.so)")


def build(verbose: bool = False) -> Path:
    LIB_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}",
           *[str(CSRC / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)
    os.replace(tmp, LIB)
    return LIB


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(verbose=args.verbose)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
