"""The single-stream kernel's work-queue map, checked on the host.

tests/native/queue_map_check.cpp includes the kernel header and runs its
queue_shape / queue_item over 20,000 random geometries (heads, batches,
tiles, text chunks, split counts): every video tile is taken exactly once
(whole, or as its two key-range halves in one partial slot that the merge
kernel maps back to the same tile) and every text item exactly once.  No GPU
is used; the program is compiled with hipcc for its host code.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _hipcc():
    for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and Path(c).exists():
            return c
    return None


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_queue_map_covers_every_item_once(tmp_path):
    exe = tmp_path / "queue_map_check"
    build = subprocess.run(
        [_hipcc(), "-O1", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{ROOT / 'longvideosparseattention_amd' / 'csrc'}",
         str(ROOT / "tests" / "native" / "queue_map_check.cpp"), "-o", str(exe)],
        capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stdout + build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0 and "queue map ok" in run.stdout, run.stdout + run.stderr
