"""Torch-facing wrappers of the C-ABI entry points (device memory + streams).

Torch is used only for device allocation and the current stream; every
computation is one of the HIP kernels of ``liblvsa_amd.so``.  Inputs must be
device tensors: there is no CPU path.
"""

from __future__ import annotations

import ctypes as C
import math
import os
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from . import _capi as capi

_DTYPES = {torch.bfloat16: capi.LVSA_BF16, torch.float16: capi.LVSA_FP16, torch.float32: capi.LVSA_FP32}
# Head sizes of the reference plugin (LVSABackend.get_supported_head_sizes,
# backend.py:52-53), all run natively: 96 on the 128 LDS layout, 192 on the
# 256 one.
SUPPORTED_HEAD_DIMS = (64, 96, 128, 192, 256)
def kernel_head_dim(head_dim: int) -> int:
    """Head size the kernel runs for ``head_dim``: every supported size natively."""
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim {head_dim} not supported by the gfx950 kernel (supported: {SUPPORTED_HEAD_DIMS})")
    return head_dim


def stream_tail_crosses_frame(n_q: int, n_k: int, k_tok0: int, key_rows: int) -> bool:
    """Whether the short last key block of a frame-structured source of ``n_k``
    rows starting at token ``k_tok0`` crosses a frame boundary (frames of
    ``key_rows`` tokens).  The plan builder describes such a block as
    "generic", which the single-stream kernels do not handle; the C entry
    point makes the same test (``stream_tail_crosses_frame``)."""
    B = capi.ATTN_BLOCK_K
    if n_q == 0 or n_k <= 0 or key_rows <= 0:
        return False
    t = n_k - B * ((n_k - 1) // B)
    e = (k_tok0 + n_k) % key_rows
    return t < B and 0 < e < t


def attn_block_q(head_dim: int = 128, dtype: Optional[torch.dtype] = None, frame_rows: int = 0,
                 key_rows: int = 0, n_k: int = 0, k_tok0: int = 0, video_rows: bool = True) -> int:
    """Query rows per attention tile, i.e. which kernel a plan is built for.

    256 for head sizes 64, 96 and 128 in 16-bit: the single-stream kernels
    (head size 64: the dual map, 4 waves of 64 rows, two work-groups per CU)
    when query frames span at least 255 rows and key frames at least 64, the
    8-wave ping-pong kernel otherwise.  256 for 192 in 16-bit where the
    single-stream kernel's dual-wide map (4 waves of 64 rows) takes the
    geometry: query frames of at least 255 rows (``frame_rows``), key frames
    of at least 64 (``key_rows``), and a key source of ``n_k`` rows from
    token ``k_tok0`` whose short last block lies in one frame, or for a plan
    without video query rows (``video_rows=False``: dense calls, whose rows
    are text-query tiles that touch no frame).  128 for 192 otherwise and
    for 256: the single-stream kernel's wide map (4 waves, one
    per SIMD, when query frames span at least 127 rows and key frames at
    least 64) or else the 4-wave kernel; and 128 for fp32 inputs at every
    head size (the fp32 kernel).

    ``LVSA_ATTN_BLOCK_Q`` (128, 256 or 384) overrides the choice for 64 and
    128 in 16-bit, and 128 that for 192, for comparisons; so does
    ``LVSA_ATTN_KERNEL=pp`` for 192 (the 4-wave kernel's 128-row tiles).
    384 selects the 12-wave single-stream kernel (head size 64, three waves
    of 32 rows per SIMD) where the geometry allows it (query frames of at
    least 383 rows, the key conditions above); 256 otherwise."""
    kd = kernel_head_dim(head_dim)
    if dtype == torch.float32:
        return 128
    env = os.environ.get("LVSA_ATTN_BLOCK_Q")
    if kd == 192:
        if env == "128" or os.environ.get("LVSA_ATTN_KERNEL") == "pp":
            return 128
        ok = not video_rows or (frame_rows >= 255 and key_rows >= capi.ATTN_BLOCK_K and
                                not stream_tail_crosses_frame(1, n_k, k_tok0, key_rows))
        return 256 if ok else 128
    if kd >= 192:
        return 128
    if kd == 96:
        return 256
    if env == "384":
        ok = (kd == 64 and frame_rows >= 383 and key_rows >= capi.ATTN_BLOCK_K and
              not stream_tail_crosses_frame(1, n_k, k_tok0, key_rows))
        return 384 if ok else 256
    if env:
        return int(env)
    return 256


def stream12_sources_ok(*srcs: Optional[torch.Tensor], limit: int = 1 << 32) -> bool:
    """Whether the single-stream kernel can address these key / value
    sources: its copies use one buffer resource per source with 32-bit byte
    offsets (sources below ``limit`` bytes: 2^32, or 2^31 at head size 192,
    whose lanes of a row's unused chunks add 0x7FFF0000), and 24-bit lane
    offsets (row x row stride in bytes).  The C entry point rejects a 384-row
    plan, or a 256-row plan at head size 192, otherwise."""
    for t in srcs:
        if t is None or t.shape[1] == 0:
            continue
        row = t.stride(1) * t.element_size()
        if (t.shape[1] + capi.ATTN_BLOCK_K) * row >= limit or row >= (1 << 24):
            return False
    return True


def dual_wide_ok(plan: "BlockPlan", *srcs: Optional[torch.Tensor]) -> bool:
    """Whether a call at head size 192 can run ``plan``'s 256-row tiles (the
    dual-wide map, the only kernel for them): frames of at least 255 query
    and 64 key rows, the frame source's short last key block inside one
    frame, addressable sources, and no ``LVSA_ATTN_KERNEL=pp``.  The C entry
    point makes the same test."""
    p = plan.params
    geom = p.n_q == 0 or (p.R >= 255 and p.C >= capi.ATTN_BLOCK_K and
                          not stream_tail_crosses_frame(p.n_q, p.n_k, p.k_tok0, p.C))
    return (geom and os.environ.get("LVSA_ATTN_KERNEL") != "pp" and
            stream12_sources_ok(*srcs, limit=1 << 31))


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_device(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise RuntimeError(
            f"{name} must be a GPU (HIP) tensor: the LVSA MI355X backend has no CPU path "
            f"(got {getattr(t, 'device', type(t))})"
        )


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ───────────────────────────── mask builder ────────────────────────────────


@dataclass
class DeviceMask:
    """Device outputs of ``lvsa_mask_build`` (see include/lvsa_amd.h)."""

    frame_indptr: torch.Tensor      # [n_rows+1] int32
    frame_indices: torch.Tensor     # [max_nnz] int32 (first nnz valid)
    compact_frames: torch.Tensor    # [T] int32
    global_frames: torch.Tensor     # [T] int32
    window_bounds: torch.Tensor     # [T, 2] int32
    rel_full: torch.Tensor          # [n_local, words] int32 (uint32 bit patterns)
    rel_window: torch.Tensor        # [n_local, words]
    info: torch.Tensor              # [8] int32
    n_rows: int
    n_local: int
    words: int
    local_seq: int
    global_token_start: int


def mask_params(T: int, P: int, W: int, n_first: int, kfi: Optional[int], offset: int = 0,
                expand: bool = True, rank: int = 0, world: int = 1,
                guards: Sequence[int] = (), auto_step: Optional[int] = None,
                reference_frames: int = 21, sparsity_scale: float = 1.0) -> capi.MaskParams:
    """Parameters of ``lvsa_mask_build``.  With ``auto_step`` set, the kernel
    derives kfi itself (``compute_auto_kfi`` of the window, ``reference_frames``
    and ``sparsity_scale``) and rotates by ``auto_step % kfi``; ``kfi`` and
    ``offset`` are then ignored."""
    if not 1 <= T <= capi.LVSA_MAX_FRAMES:
        raise ValueError(f"total_latent_frames={T} outside [1, {capi.LVSA_MAX_FRAMES}]")
    p = capi.MaskParams()
    p.T, p.P, p.window, p.n_first = T, P, W, n_first
    p.kfi = int(kfi) if (kfi is not None and kfi > 0) else 0
    p.offset, p.expand, p.rank, p.world = int(offset), int(bool(expand)), rank, world
    for g in guards:
        if 0 <= g < T:
            p.guard_bits[g >> 5] |= 1 << (g & 31)
    p.reference_frames, p.sparsity_scale = int(reference_frames), float(sparsity_scale)
    if auto_step is not None:
        p.auto_kfi, p.step = 1, int(auto_step)
    return p


def auto_kfi(T: int, W: int, n_first: int, reference_frames: int = 21, sparsity_scale: float = 1.0,
             device: Optional[torch.device] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``compute_auto_kfi`` on the GPU (``lvsa_auto_kfi``): a one-element
    int32 device tensor, written on the current stream."""
    if out is None:
        device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("lvsa_auto_kfi runs on the GPU only")
        out = torch.empty(1, dtype=torch.int32, device=device)
    _require_device(out, "kfi output")
    with torch.cuda.device(out.device):
        capi.check("lvsa_auto_kfi", capi.lib().lvsa_auto_kfi(
            int(T), int(W), int(n_first), int(reference_frames), float(sparsity_scale), out.data_ptr(),
            _stream(out.device)))
    return out


def mask_sizes(p: capi.MaskParams) -> capi.MaskSizes:
    s = capi.MaskSizes()
    capi.check("lvsa_mask_sizes_query", capi.lib().lvsa_mask_sizes_query(C.byref(p), C.byref(s)))
    return s


def mask_build(p: capi.MaskParams, device: torch.device) -> DeviceMask:
    device = torch.device(device)
    if device.type != "cuda":
        raise RuntimeError("lvsa_mask_build runs on the GPU only")
    s = mask_sizes(p)
    i32 = dict(dtype=torch.int32, device=device)
    T = p.T
    dm = DeviceMask(
        frame_indptr=torch.empty(s.n_rows + 1, **i32),
        frame_indices=torch.empty(max(s.max_nnz, 1), **i32),
        compact_frames=torch.empty(T, **i32),
        global_frames=torch.empty(T, **i32),
        window_bounds=torch.empty(T, 2, **i32),
        rel_full=torch.empty(s.n_local, s.words, **i32),
        rel_window=torch.empty(s.n_local, s.words, **i32),
        info=torch.empty(8, **i32),
        n_rows=s.n_rows, n_local=s.n_local, words=s.words,
        local_seq=s.local_seq, global_token_start=s.global_token_start,
    )
    out = capi.MaskOut(
        dm.frame_indptr.data_ptr(), dm.frame_indices.data_ptr(), dm.compact_frames.data_ptr(),
        dm.global_frames.data_ptr(), dm.window_bounds.data_ptr(), dm.rel_full.data_ptr(),
        dm.rel_window.data_ptr(), dm.info.data_ptr(),
    )
    with torch.cuda.device(device):
        capi.check("lvsa_mask_build", capi.lib().lvsa_mask_build(C.byref(p), C.byref(out), _stream(device)))
    return dm


# ────────────────────────────── block plan ─────────────────────────────────


@dataclass
class BlockPlan:
    """Block-sparse CSR over query tiles (``lvsa_plan_build``)."""

    tile_indptr: torch.Tensor   # [n_tiles+1] int32
    entries: torch.Tensor       # [max_entries, 2] int32 (uint32 bit patterns)
    status: torch.Tensor        # [4] int32: overflow flag, true entry count
    n_tiles: int
    n_video_tiles: int
    params: capi.PlanParams
    rel: Optional[torch.Tensor]  # keeps the relation bitmap alive
    max_row_frames: int = 0
    _verified: bool = False
    _fallback: Optional["BlockPlan"] = None
    _fallback_ready: Optional[torch.cuda.Event] = None

    @property
    def block_q(self) -> int:
        return self.params.block_q

    @property
    def block_k(self) -> int:
        return self.params.block_k

    def with_smaller_tiles(self) -> "BlockPlan":
        """The same relation planned for the next smaller tiles (built once, on
        the current stream): 256 rows for a 384-row plan when a call's key
        sources exceed the 12-wave kernel's addressing, 128 for a 256-row plan
        at head size 192 when a call does not fit the dual-wide map."""
        if self.block_q == 128:
            return self
        smaller = 256 if self.block_q == 384 else 128
        dev = self.tile_indptr.device
        capturing = torch.cuda.is_current_stream_capturing()
        if self._fallback is None:
            p = self.params
            self._fallback = plan_build(
                self.rel, n_q=p.n_q, n_k=p.n_k, n_x=p.n_x, n_tq=p.n_tq, R=p.R, Cf=p.C, q_tok0=p.q_tok0,
                k_tok0=p.k_tok0, q_frame0=p.q_frame0, max_row_frames=self.max_row_frames, block_q=smaller,
                block_k=p.block_k, device=dev)
            if not capturing:
                self._fallback_ready = torch.cuda.Event()
                self._fallback_ready.record(torch.cuda.current_stream(dev))
        elif self._fallback_ready is not None and not capturing:
            s = torch.cuda.current_stream(dev)   # a plan shared between streams: order after its build
            s.wait_event(self._fallback_ready)
            for t in (self._fallback.tile_indptr, self._fallback.entries, self._fallback.status):
                t.record_stream(s)
        return self._fallback

    def verify(self) -> None:
        """Raise if the plan overflowed its entry capacity (``status[0]``).

        Checked once, at the first use outside stream capture (one host
        synchronisation per plan; plans are cached and reused by every layer).
        The capacity comes from ``max_row_frames``: a value below the
        relation's true row maximum would otherwise truncate the key lists."""
        if self._verified or torch.cuda.is_current_stream_capturing():
            return
        overflow, total = (int(x) for x in self.status[:2].tolist())
        if overflow:
            raise RuntimeError(
                f"lvsa_plan_build: {total} block entries exceed the capacity {self.entries.shape[0]} "
                f"(max_row_frames below the relation's row maximum)")
        self._verified = True


def plan_build(rel: Optional[torch.Tensor], *, n_q: int, n_k: int, n_x: int = 0, n_tq: int = 0,
               R: int = 1, Cf: int = 1, q_tok0: int = 0, k_tok0: int = 0, q_frame0: int = 0,
               max_row_frames: int = 0, block_q: Optional[int] = None, block_k: int = capi.ATTN_BLOCK_K,
               head_dim: int = 128, device: Optional[torch.device] = None,
               dtype: Optional[torch.dtype] = None) -> BlockPlan:
    """Refine a frame relation (bitmap rows x words, int32) to token blocks.

    ``block_q`` defaults to the tile height of the kernel that serves
    ``head_dim`` and ``dtype`` (see :func:`attn_block_q`; without frame
    geometry, except for a plan without video query rows)."""
    if rel is not None:
        _require_device(rel, "relation bitmap")
        device = rel.device
        rel = rel.contiguous()
    if device is None or torch.device(device).type != "cuda":
        raise RuntimeError("lvsa_plan_build runs on the GPU only")
    device = torch.device(device)
    if block_q is None:
        block_q = attn_block_q(head_dim, dtype, video_rows=n_q > 0)
    p = capi.PlanParams()
    p.n_q, p.n_k, p.n_x, p.n_tq = n_q, n_k, n_x, n_tq
    p.R, p.C = R, Cf
    p.q_tok0, p.k_tok0, p.q_frame0 = q_tok0, k_tok0, q_frame0
    p.rel_rows = rel.shape[0] if rel is not None else 0
    p.words = rel.shape[1] if rel is not None else 0
    p.rel = rel.data_ptr() if rel is not None else None
    p.block_q, p.block_k = block_q, block_k
    sz = capi.PlanSizes()
    capi.check("lvsa_plan_sizes_query", capi.lib().lvsa_plan_sizes_query(C.byref(p), max_row_frames, C.byref(sz)))
    i32 = dict(dtype=torch.int32, device=device)
    indptr = torch.empty(sz.n_tiles + 1, **i32)
    entries = torch.empty(max(sz.max_entries, 1), 2, **i32)
    status = torch.empty(max(sz.workspace_bytes // 4, 4), **i32)
    with torch.cuda.device(device):
        capi.check("lvsa_plan_build", capi.lib().lvsa_plan_build(
            C.byref(p), indptr.data_ptr(), entries.data_ptr(), sz.max_entries,
            status.data_ptr(), status.numel() * 4, _stream(device)))
    return BlockPlan(indptr, entries, status, sz.n_tiles, sz.n_video_tiles, p, rel, max_row_frames)


# ─────────────────────────── attention forward ─────────────────────────────


def _prep(t: torch.Tensor, name: str, dtype: torch.dtype) -> torch.Tensor:
    _require_device(t, name)
    if t.dim() != 4:
        raise ValueError(f"{name} must be [B, S, H, D], got shape {tuple(t.shape)}")
    if t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * t.element_size()) % 16 == 0
                                                              for s in t.stride()[:3])
    # The kernel reads 16-byte row chunks; other layouts are repacked on the device.
    return t if ok else t.clone(memory_format=torch.contiguous_format)


def _str3(t: Optional[torch.Tensor]):
    return capi._Str3(*(t.stride()[:3] if t is not None else (0, 0, 0)))


@dataclass
class AttnCall:
    """The C-ABI arguments of one attention call and the tensors they point to
    (repacked inputs and fresh outputs are kept alive here)."""

    args: capi.AttnArgs
    out: torch.Tensor
    out_t: Optional[torch.Tensor]
    lse: Optional[torch.Tensor]
    lse_t: Optional[torch.Tensor]
    tensors: tuple


def attn_args(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan: BlockPlan, *,
              kx: Optional[torch.Tensor] = None, vx: Optional[torch.Tensor] = None,
              qt: Optional[torch.Tensor] = None, scale: Optional[float] = None,
              return_lse: bool = False, out: Optional[torch.Tensor] = None,
              out_t: Optional[torch.Tensor] = None) -> AttnCall:
    """Validate an attention call and fill its ``lvsa_attn_args`` (no workspace)."""
    dtype = q.dtype
    if dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {dtype}: bf16, fp16 or fp32 inputs")
    q = _prep(q, "query", dtype)
    k = _prep(k, "key", dtype)
    v = _prep(v, "value", dtype)
    B, n_q, H, D = q.shape
    Hkv = k.shape[2]
    kernel_head_dim(D)  # raises for an unsupported head size
    if k.shape[0] != B or k.shape[3] != D or v.shape != k.shape:
        raise ValueError(f"key/value shapes {tuple(k.shape)} / {tuple(v.shape)} do not match query {tuple(q.shape)}")
    if H % Hkv:
        raise ValueError(f"num heads {H} must be a multiple of kv heads {Hkv}")
    n_x = 0
    if kx is not None and kx.shape[1] > 0:
        kx = _prep(kx, "extra key", dtype)
        vx = _prep(vx, "extra value", dtype)
        if kx.shape[0] != B or kx.shape[2] != Hkv or kx.shape[3] != D or vx.shape != kx.shape:
            raise ValueError("extra key/value shape mismatch")
        n_x = kx.shape[1]
    else:
        kx = vx = None
    n_tq = 0
    if qt is not None and qt.shape[1] > 0:
        qt = _prep(qt, "text query", dtype)
        if qt.shape[0] != B or qt.shape[2] != H or qt.shape[3] != D:
            raise ValueError("text query shape mismatch")
        n_tq = qt.shape[1]
    else:
        qt = None
    if plan.block_q == 384 and not stream12_sources_ok(k, v, kx, vx):
        plan = plan.with_smaller_tiles()
    elif plan.block_q == 256 and D == 192 and not dual_wide_ok(plan, k, v, kx, vx):
        plan = plan.with_smaller_tiles()
    pp = plan.params
    if plan.block_k != capi.ATTN_BLOCK_K:
        raise ValueError(f"plan built with block_k={plan.block_k}; the attention kernels walk key blocks of "
                         f"{capi.ATTN_BLOCK_K} rows")
    if (pp.n_q, pp.n_k, pp.n_x, pp.n_tq) != (n_q, k.shape[1], n_x, n_tq):
        raise ValueError(
            f"plan built for (n_q, n_k, n_x, n_tq)={(pp.n_q, pp.n_k, pp.n_x, pp.n_tq)}, "
            f"called with {(n_q, k.shape[1], n_x, n_tq)}")
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    if qt is not None and out_t is None:
        out_t = torch.empty_like(qt, memory_format=torch.contiguous_format)
    lse = torch.empty(B, H, n_q, dtype=torch.float32, device=q.device) if return_lse else None
    lse_t = (torch.empty(B, H, n_tq, dtype=torch.float32, device=q.device)
             if (return_lse and qt is not None) else None)
    a = capi.AttnArgs()
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.kx, a.vx, a.qt = _ptr(kx), _ptr(vx), _ptr(qt)
    a.o, a.ot = out.data_ptr(), _ptr(out_t)
    a.lse, a.lse_t = _ptr(lse), _ptr(lse_t)
    a.q_str, a.k_str, a.v_str = _str3(q), _str3(k), _str3(v)
    a.kx_str, a.vx_str, a.qt_str = _str3(kx), _str3(vx), _str3(qt)
    a.o_str, a.ot_str = _str3(out), _str3(out_t)
    a.B, a.H, a.Hkv, a.D = B, H, Hkv, D
    a.n_q, a.n_k, a.n_x, a.n_tq = n_q, k.shape[1], n_x, n_tq
    a.scale = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    a.dtype = _DTYPES[dtype]
    a.block_q = plan.block_q
    a.tile_indptr, a.entries = plan.tile_indptr.data_ptr(), plan.entries.data_ptr()
    a.n_tiles, a.n_video_tiles = plan.n_tiles, plan.n_video_tiles
    a.rel = pp.rel
    a.words, a.R, a.C, a.q_frame0 = pp.words, pp.R, pp.C, pp.q_frame0
    a.q_tok0, a.k_tok0 = pp.q_tok0, pp.k_tok0
    a.rel_rows = pp.rel_rows
    plan.verify()
    return AttnCall(a, out, out_t, lse, lse_t, (q, k, v, kx, vx, qt, plan))


def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan: BlockPlan, *,
             kx: Optional[torch.Tensor] = None, vx: Optional[torch.Tensor] = None,
             qt: Optional[torch.Tensor] = None, scale: Optional[float] = None,
             return_lse: bool = False, out: Optional[torch.Tensor] = None,
             out_t: Optional[torch.Tensor] = None, scratch: bool = True
             ) -> Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Block-sparse attention over ``plan``: returns ``(o, o_text, lse, lse_text)``.

    ``lse`` is the natural-log log-sum-exp ``[B, H, S]`` (fp32) when requested.
    ``scratch`` (the default) passes the call's device scratch: the counters of
    the work queues that balance the single-stream kernel's work-groups over
    the XCDs, and the partials that let long text-query tiles run as key-range
    chunks merged by log-sum-exp.  ``False`` launches one work-group per work
    item and runs each text tile whole.
    """
    call = attn_args(q, k, v, plan, kx=kx, vx=vx, qt=qt, scale=scale, return_lse=return_lse, out=out,
                     out_t=out_t)
    a = call.args
    ws_bytes = C.c_int64(0)
    capi.check("lvsa_attn_workspace_query", capi.lib().lvsa_attn_workspace_query(C.byref(a), C.byref(ws_bytes)))
    ws = None
    if ws_bytes.value > 0 and scratch:
        # work-queue counters (zeroed by the call) and the text-split partials
        ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=call.out.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes.value
    with torch.cuda.device(call.out.device):
        capi.check("lvsa_attn_fwd", capi.lib().lvsa_attn_fwd(C.byref(a), _stream(call.out.device)))
    return call.out, call.out_t, call.lse, call.lse_t


# ───────────────────────────── frame gather ────────────────────────────────


def gather_frames(src: torch.Tensor, frames: torch.Tensor, P: int) -> torch.Tensor:
    """``dst[b, i*P + t] = src[b, frames[i]*P + t]`` on the GPU."""
    _require_device(src, "source")
    if src.dim() != 4:
        raise ValueError("source must be [B, S, H, D]")
    if src.stride(-1) != 1:
        src = src.contiguous()
    frames = frames.to(device=src.device, dtype=torch.int32)
    B, _, H, D = src.shape
    n = frames.numel()
    dst = src.new_empty(B, n * P, H, D)
    if n == 0:
        return dst
    es = src.element_size()
    if es not in (2, 4):
        raise TypeError(f"unsupported element size {es}")
    sstr = (C.c_int64 * 3)(*src.stride()[:3])
    dstr = (C.c_int64 * 3)(*dst.stride()[:3])
    with torch.cuda.device(src.device):
        capi.check("lvsa_gather_frames", capi.lib().lvsa_gather_frames(
            src.data_ptr(), sstr, dst.data_ptr(), dstr, frames.data_ptr(), n, P, B, H, D, es,
            _stream(src.device)))
    return dst


def csr_to_bitmap(indptr: torch.Tensor, indices: torch.Tensor, n_cols: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block CSR -> relation bitmap ``[n_rows, ceil(n_cols/32)]`` (int32 words) on the GPU.

    Returns ``(bitmap, status)``; ``status[0] == 1`` flags out-of-range columns.
    """
    _require_device(indptr, "indptr")
    device = indptr.device
    indptr = indptr.to(dtype=torch.int32).contiguous()
    indices = indices.to(device=device, dtype=torch.int32).contiguous()
    n_rows = indptr.numel() - 1
    words = max(1, -(-n_cols // 32))
    bitmap = torch.empty(max(n_rows, 1), words, dtype=torch.int32, device=device)
    status = torch.empty(4, dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        capi.check("lvsa_csr_to_bitmap", capi.lib().lvsa_csr_to_bitmap(
            indptr.data_ptr(), indices.data_ptr() if indices.numel() else None, n_rows, n_cols,
            bitmap.data_ptr(), words, status.data_ptr(), _stream(device)))
    return bitmap[:n_rows], status
