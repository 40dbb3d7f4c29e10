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
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB_DIR = PKG / "_lib"
LIB = LIB_DIR / "liblvsa_amd.so"
ARCH = os.environ.get("LVSA_OFFLOAD_ARCH", "gfx950")
# Translation units and their extra flags: one unit per attention head size,
# each with the machine scheduler measured fastest for it.  max-ILP: about 2%
# faster on the D = 128 configurations (slower on 64 and 96).  iterative-maxocc:
# the 4-wave kernels, about 6% faster at D = 192 and 21% at D = 256.
MAXOCC = ["-mllvm", "-amdgpu-sched-strategy=iterative-maxocc"]
SOURCES = {
    "lvsa_mask.hip": [],
    "lvsa_attn.hip": [],
    "lvsa_noalloc.hip": [],
    "lvsa_attn_d64.hip": [],
    "lvsa_attn_d96.hip": [],
    "lvsa_attn_d128.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "lvsa_attn_d192.hip": MAXOCC,
    "lvsa_attn_d256.hip": MAXOCC,
    "lvsa_attn_f32.hip": [],
}

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
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


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _finish(proc, what, verbose):
    out, _ = proc.communicate()
    msgs = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {what} ({proc.returncode}):\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)


def build(verbose: bool = False) -> Path:
    """Compile every translation unit (in parallel) and link the shared library."""
    LIB_DIR.mkdir(exist_ok=True)
    # the hand-scheduled key loop of the single-stream D = 128 kernel
    subprocess.run([sys.executable, str(CSRC / "gen_stream_asm.py")], check=True)
    tmp = LIB.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="lvsa_build_") as objdir:
        jobs = []
        for src, extra in SOURCES.items():
            obj = str(Path(objdir) / (Path(src).stem + ".o"))
            cmd = [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src), "-o", obj]
            jobs.append((src, obj, _run(cmd, verbose)))
        for src, _, proc in jobs:
            _finish(proc, src, verbose)
        link = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *[o for _, o, _ in jobs], "-o", str(tmp)]
        _finish(_run(link, verbose), "link", verbose)
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
