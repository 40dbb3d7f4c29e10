"""The C-ABI library (CPU only: no kernel is launched).

* liblvsa_amd.so loads and exports every function include/lvsa_amd.h declares;
* the ctypes structures have the C layout (checked against gcc's offsetof);
* the host-only sizing entry points validate their input and report errors.
"""

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from longvideosparseattention_amd import _capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "lvsa_amd.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"LVSA_API\s+[\w\s\*]*?\b(lvsa_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _capi.lib()
    names = _declared()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_capi.SIGNATURES)
    assert _capi.version() == re.search(r'LVSA_AMD_VERSION "([^"]+)"', HEADER.read_text()).group(1)


def test_struct_layout_matches_c(tmp_path):
    structs = {"lvsa_mask_params": _capi.MaskParams, "lvsa_mask_sizes": _capi.MaskSizes,
               "lvsa_mask_out": _capi.MaskOut, "lvsa_plan_params": _capi.PlanParams,
               "lvsa_plan_sizes": _capi.PlanSizes, "lvsa_attn_args": _capi.AttnArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "lvsa_amd.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    cc = subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", "-I/opt/rocm/include",
                         str(src), "-o", str(exe)], capture_output=True, text=True)
    if cc.returncode != 0:
        pytest.fail(f"gcc failed: {cc.stderr}")
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {}
    for line in filter(None, out):
        s, f, v = line.split()
        got[(s, f)] = int(v)
    for cname, py in structs.items():
        assert got[(cname, "size")] == C.sizeof(py), cname
        for fname, _ in py._fields_:
            assert got[(cname, fname)] == getattr(py, fname).offset, (cname, fname)


def test_mask_sizes_and_errors():
    lib = _capi.lib()
    p = _capi.MaskParams(T=84, P=1560, window=2, n_first=1, kfi=8, offset=0, expand=1, rank=0, world=1)
    s = _capi.MaskSizes()
    assert lib.lvsa_mask_sizes_query(C.byref(p), C.byref(s)) == 0
    assert (s.n_rows, s.n_local, s.words, s.local_seq) == (84, 84, 3, 84 * 1560)
    p.T = 0
    assert lib.lvsa_mask_sizes_query(C.byref(p), C.byref(s)) == -1
    assert b"T=0" in lib.lvsa_last_error()
    p.T, p.world = 5, 2
    p.P = 3
    assert lib.lvsa_mask_sizes_query(C.byref(p), C.byref(s)) == -1
    assert b"divisible by world" in lib.lvsa_last_error()


def test_auto_kfi_rejects_bad_arguments_without_launching():
    lib = _capi.lib()
    assert lib.lvsa_auto_kfi(0, 2, 1, 21, 1.0, 8, None) == -1
    assert b"T=0" in lib.lvsa_last_error()
    assert lib.lvsa_auto_kfi(84, -1, 1, 21, 1.0, 8, None) == -1
    assert lib.lvsa_auto_kfi(84, 2, 1, 21, 1.0, None, None) == -1
    assert lib.lvsa_auto_kfi(84, 2, 1, 21, float("nan"), 8, None) == -1
    assert b"NaN" in lib.lvsa_last_error()
    # the mask builder's device re-tune checks the same budget on the host
    p = _capi.MaskParams(T=84, P=1560, window=2, n_first=1, expand=1, rank=0, world=1, auto_kfi=1,
                         reference_frames=21, sparsity_scale=float("nan"), step=3)
    s = _capi.MaskSizes()
    assert lib.lvsa_mask_sizes_query(C.byref(p), C.byref(s)) == -1
    p.sparsity_scale, p.step = 0.5, -1
    assert lib.lvsa_mask_sizes_query(C.byref(p), C.byref(s)) == -1
    assert b"step=-1" in lib.lvsa_last_error()
    p.step = 3
    assert lib.lvsa_mask_sizes_query(C.byref(p), C.byref(s)) == 0


def test_plan_sizes():
    lib = _capi.lib()
    p = _capi.PlanParams(n_q=131040, n_k=131040, n_x=0, n_tq=0, R=1560, C=1560, q_tok0=0, k_tok0=0,
                         q_frame0=0, rel_rows=84, words=3, rel=1, block_q=128, block_k=64)
    s = _capi.PlanSizes()
    assert lib.lvsa_plan_sizes_query(C.byref(p), 17, C.byref(s)) == 0
    assert s.n_tiles == s.n_video_tiles == 1024
    assert 0 < s.max_entries <= 1024 * 2048
    p.block_q = 384                          # the 12-wave kernel's tiles (row split in 9 bits)
    assert lib.lvsa_plan_sizes_query(C.byref(p), 17, C.byref(s)) == 0
    assert s.n_video_tiles == -(-131040 // 384)
    p.block_q = 385
    assert lib.lvsa_plan_sizes_query(C.byref(p), 17, C.byref(s)) == -1


def test_attn_rejects_bad_args_without_launching():
    lib = _capi.lib()
    a = _capi.AttnArgs()
    a.D, a.dtype, a.B, a.H, a.Hkv = 80, 0, 1, 2, 2
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    assert b"head_dim 80" in lib.lvsa_last_error()
    a.D, a.block_q = 96, 128
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    assert b"head_dim 96 runs 256-row tiles" in lib.lvsa_last_error()
    a.D, a.block_q = 256, 256
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    assert b"head_dim 256 runs 128-row tiles" in lib.lvsa_last_error()
    a.D, a.block_q = 192, 384
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    assert b"head_dim 192 runs 128-row tiles (192 also 256-row" in lib.lvsa_last_error()
    a.tile_indptr = a.entries = 4096         # host checks only: nothing is launched
    a.D, a.block_q = 128, 384                # 384-row tiles: head size 64 only
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    assert b"384-row tiles need head_dim 64" in lib.lvsa_last_error()
    a.D, a.n_q, a.R, a.C = 64, 1000, 300, 300   # query frames below 383 rows
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    assert b"384-row tiles" in lib.lvsa_last_error()
    a.n_q, a.R, a.C, a.block_q = 0, 0, 0, 256
    a.tile_indptr = a.entries = None
    a.D, a.H, a.Hkv = 128, 3, 2
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -1


def _attn_args(n_q=1000, rel_rows=10, n_tq=0, n_k=1000):
    """Arguments that pass every check up to the relation bound (fake,
    aligned, non-null device pointers: nothing is launched by these tests)."""
    a = _capi.AttnArgs()
    a.D, a.dtype, a.B, a.H, a.Hkv, a.block_q = 128, 0, 1, 2, 2, 256
    a.n_q, a.n_k, a.n_tq = n_q, n_k, n_tq
    a.n_video_tiles = -(-n_q // 256)
    a.n_tiles = a.n_video_tiles + -(-n_tq // 256)
    for f in ("q", "k", "v", "o", "qt", "ot", "tile_indptr", "entries", "rel"):
        setattr(a, f, 4096)
    for f in ("q_str", "k_str", "v_str", "o_str", "qt_str", "ot_str"):
        setattr(a, f, _capi._Str3(1 << 20, 256, 128))
    a.words, a.R, a.C, a.rel_rows = 1, 100, 100, rel_rows
    return a


def test_attn_head_192_on_256_row_tiles_needs_the_dual_wide_geometry():
    """Head size 192 on 256-row tiles runs the dual-wide map only: query frames
    below 255 rows, or a short last key block that crosses a frame, are
    rejected before anything is launched."""
    lib = _capi.lib()
    a = _attn_args(n_q=1000, rel_rows=10)
    a.D = 192
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2          # R = C = 100
    assert b"build the plan with block_q 128" in lib.lvsa_last_error()
    a.R, a.C, a.rel_rows, a.k_tok0 = 300, 300, 4, 220           # (220 + 1000) % 300 = 20 < 40 tail rows
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    assert b"build the plan with block_q 128" in lib.lvsa_last_error()


def test_attn_rejects_query_rows_outside_relation():
    lib = _capi.lib()
    a = _attn_args(n_q=1000, rel_rows=9)   # rows 0..999 need relation rows 0..9
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -1
    assert b"relation rows [0, 9]" in lib.lvsa_last_error()
    a.q_frame0 = 1                          # first query row maps to relation row -1
    a.rel_rows = 11
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -1
    assert b"relation rows [-1, 8]" in lib.lvsa_last_error()


def test_attn_workspace_query_and_capacity():
    lib = _capi.lib()
    a = _attn_args(n_q=1000, rel_rows=10, n_tq=100, n_k=20000)
    n = C.c_int64(-1)
    assert lib.lvsa_attn_workspace_query(C.byref(a), C.byref(n)) == 0
    chunks = -(-(-(-20000 // 64)) // 128)           # 313 key blocks in chunks of 128
    assert chunks == 3
    text = 4 * chunks * 2 * 100 * (128 + 2)          # partial O and (max, sum) per chunk
    queues = 8 * 128                                  # one work-queue counter per 128-byte line
    # 8 video tiles: too few for the work queues, so no video split either
    assert n.value == -(-text // 256) * 256 + queues
    a.workspace, a.workspace_bytes = 4096, n.value - 16
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -3
    assert b"workspace" in lib.lvsa_last_error()
    b = _attn_args(n_q=0, rel_rows=10, n_tq=0)    # no queries: the queue counters only
    assert lib.lvsa_attn_workspace_query(C.byref(b), C.byref(n)) == 0 and n.value == queues


def test_plan_rejects_query_rows_outside_relation():
    lib = _capi.lib()
    p = _capi.PlanParams(n_q=1000, n_k=1000, n_x=0, n_tq=0, R=100, C=100, q_tok0=0, k_tok0=0,
                         q_frame0=0, rel_rows=9, words=1, rel=4096, block_q=256, block_k=64)
    s = _capi.PlanSizes()
    assert lib.lvsa_plan_sizes_query(C.byref(p), 5, C.byref(s)) == -1
    assert b"relation rows [0, 9]" in lib.lvsa_last_error()
    p.rel_rows = 10
    assert lib.lvsa_plan_sizes_query(C.byref(p), 5, C.byref(s)) == 0


def test_attn_rejects_384_row_plans_the_12_wave_kernel_cannot_run():
    """384-row tiles run only on the 12-wave single-stream kernel, whose loop
    masks "two-part" descriptors and addresses each key source with 32-bit
    byte offsets: a frame source whose short last key block crosses a frame
    boundary (keys [384, 440) over frames of 385: planned "generic"), or a
    source of 2^32 bytes or more, is rejected before anything is launched."""
    lib = _capi.lib()
    a = _attn_args(n_q=440, rel_rows=2, n_k=440)
    a.D, a.block_q, a.R, a.C = 64, 384, 385, 385
    a.n_video_tiles = a.n_tiles = 2
    a.q_str = a.o_str = a.k_str = a.v_str = _capi._Str3(1 << 20, 64, 64)
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    assert b"last key block of the frame source inside one frame" in lib.lvsa_last_error()
    a.k_tok0 = 440                                   # keys [440, 880): boundary 770 outside the tail
    a.k_str = _capi._Str3(1 << 40, 1 << 23, 64)      # 16 MiB rows: 2^32 bytes well before the end
    assert lib.lvsa_attn_fwd(C.byref(a), None) == -2
    err = lib.lvsa_last_error()
    assert b"16 MiB" in err or b"32-bit byte offsets" in err
