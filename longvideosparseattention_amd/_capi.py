"""ctypes binding of ``include/lvsa_amd.h`` (liblvsa_amd.so).

The library is the only compute path of this package: every public function
that touches tensors ends in one of these entry points, and there is no CPU
or PyTorch fallback.  If the shared library is missing, ``lib()`` raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Optional

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "_lib" / "liblvsa_amd.so"

LVSA_MAX_FRAMES = 4096
LVSA_BITMAP_WORDS = LVSA_MAX_FRAMES // 32
LVSA_BF16, LVSA_FP16, LVSA_FP32 = 0, 1, 2

STATUS = {0: "ok", -1: "invalid argument", -2: "unsupported", -3: "capacity", -4: "hip error"}

# Kernel tiling of lvsa_attn_fwd (query rows x key rows per block).
ATTN_BLOCK_Q = 128
ATTN_BLOCK_K = 64
# Static scratch of lvsa_attn_fwd_noalloc (LVSA_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 64 << 20


class LvsaError(RuntimeError):
    """A C-ABI call returned a non-zero lvsa_status."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed ({STATUS.get(code, code)}): {message}")
        self.code = code


class MaskParams(C.Structure):
    _fields_ = [
        ("T", C.c_int32), ("P", C.c_int32), ("window", C.c_int32), ("n_first", C.c_int32),
        ("kfi", C.c_int32), ("offset", C.c_int32), ("expand", C.c_int32),
        ("rank", C.c_int32), ("world", C.c_int32),
        ("guard_bits", C.c_uint32 * LVSA_BITMAP_WORDS),
        ("auto_kfi", C.c_int32), ("reference_frames", C.c_int32), ("sparsity_scale", C.c_double),
        ("step", C.c_int64),
    ]


class MaskSizes(C.Structure):
    _fields_ = [
        ("n_rows", C.c_int32), ("n_local", C.c_int32), ("words", C.c_int32), ("max_nnz", C.c_int32),
        ("local_seq", C.c_int64), ("global_token_start", C.c_int64),
    ]


class MaskOut(C.Structure):
    _fields_ = [
        ("frame_indptr", C.c_void_p), ("frame_indices", C.c_void_p), ("compact_frames", C.c_void_p),
        ("global_frames", C.c_void_p), ("window_bounds", C.c_void_p), ("rel_full", C.c_void_p),
        ("rel_window", C.c_void_p), ("info", C.c_void_p),
    ]


class PlanParams(C.Structure):
    _fields_ = [
        ("n_q", C.c_int32), ("n_k", C.c_int32), ("n_x", C.c_int32), ("n_tq", C.c_int32),
        ("R", C.c_int32), ("C", C.c_int32),
        ("q_tok0", C.c_int64), ("k_tok0", C.c_int64),
        ("q_frame0", C.c_int32), ("rel_rows", C.c_int32), ("words", C.c_int32),
        ("rel", C.c_void_p),
        ("block_q", C.c_int32), ("block_k", C.c_int32),
    ]


class PlanSizes(C.Structure):
    _fields_ = [
        ("n_tiles", C.c_int32), ("n_video_tiles", C.c_int32),
        ("max_entries", C.c_int64), ("workspace_bytes", C.c_int64),
    ]


_Str3 = C.c_int64 * 3


class AttnArgs(C.Structure):
    _fields_ = [
        ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p),
        ("kx", C.c_void_p), ("vx", C.c_void_p), ("qt", C.c_void_p),
        ("o", C.c_void_p), ("ot", C.c_void_p),
        ("lse", C.c_void_p), ("lse_t", C.c_void_p),
        ("q_str", _Str3), ("k_str", _Str3), ("v_str", _Str3), ("kx_str", _Str3),
        ("vx_str", _Str3), ("qt_str", _Str3), ("o_str", _Str3), ("ot_str", _Str3),
        ("B", C.c_int32), ("H", C.c_int32), ("Hkv", C.c_int32), ("D", C.c_int32),
        ("n_q", C.c_int32), ("n_k", C.c_int32), ("n_x", C.c_int32), ("n_tq", C.c_int32),
        ("scale", C.c_float), ("dtype", C.c_int32),
        ("block_q", C.c_int32),
        ("tile_indptr", C.c_void_p), ("entries", C.c_void_p),
        ("n_tiles", C.c_int32), ("n_video_tiles", C.c_int32),
        ("rel", C.c_void_p), ("words", C.c_int32), ("R", C.c_int32), ("C", C.c_int32),
        ("q_frame0", C.c_int32),
        ("q_tok0", C.c_int64), ("k_tok0", C.c_int64),
        ("rel_rows", C.c_int32),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_int64),
    ]


# Every symbol the header declares, with its ctypes signature.
SIGNATURES = {
    "lvsa_mask_sizes_query": (C.c_int, [C.POINTER(MaskParams), C.POINTER(MaskSizes)]),
    "lvsa_mask_build": (C.c_int, [C.POINTER(MaskParams), C.POINTER(MaskOut), C.c_void_p]),
    "lvsa_auto_kfi": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_double, C.c_void_p,
                                C.c_void_p]),
    "lvsa_plan_sizes_query": (C.c_int, [C.POINTER(PlanParams), C.c_int32, C.POINTER(PlanSizes)]),
    "lvsa_plan_build": (C.c_int, [C.POINTER(PlanParams), C.c_void_p, C.c_void_p, C.c_int64,
                                  C.c_void_p, C.c_int64, C.c_void_p]),
    "lvsa_csr_to_bitmap": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_int32,
                                     C.c_void_p, C.c_void_p]),
    "lvsa_attn_fwd": (C.c_int, [C.POINTER(AttnArgs), C.c_void_p]),
    "lvsa_attn_workspace_query": (C.c_int, [C.POINTER(AttnArgs), C.POINTER(C.c_int64)]),
    "lvsa_attn_fwd_noalloc": (C.c_int, [C.POINTER(AttnArgs), C.c_void_p]),
    "lvsa_gather_frames": (C.c_int, [C.c_void_p, C.POINTER(C.c_int64), C.c_void_p, C.POINTER(C.c_int64),
                                     C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                     C.c_int32, C.c_void_p]),
    "lvsa_version": (C.c_char_p, []),
    "lvsa_last_error": (C.c_char_p, []),
}

_LIB: Optional[C.CDLL] = None


def lib_path() -> Path:
    override = os.environ.get("LVSA_AMD_LIB")
    return Path(override) if override else LIB_PATH


def lib() -> C.CDLL:
    """Load liblvsa_amd.so (once).  Raises if it has not been built."""
    global _LIB
    if _LIB is None:
        path = lib_path()
        if not path.exists():
            raise RuntimeError(
                f"liblvsa_amd.so not found at {path}; build it with "
                "`python -m longvideosparseattention_amd.build_lib` (the HIP library is the only compute path)"
            )
        handle = C.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(fn: str, code: int) -> None:
    if code != 0:
        msg = lib().lvsa_last_error().decode(errors="replace")
        raise LvsaError(fn, code, msg)


def version() -> str:
    return lib().lvsa_version().decode()
