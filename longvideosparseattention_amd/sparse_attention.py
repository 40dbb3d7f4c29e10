"""LVSA sparse windowed attention — MI355X (HIP) implementation of the reference API.

Mirrors ``lvsa/sparse_attention.py`` of LVSA v1.2.0: the same public names,
argument order, return shapes/dtypes and error behaviour, so callers switch by
changing the import.  What changes is underneath:

* the frame-level block CSR (``fi_indptr`` / ``fi_indices``) and the frame
  relation are built on the GPU by ``lvsa_mask_build`` (bit-exact with the
  reference's ``_build_flashinfer_csr``); host-side fields (global set,
  window bounds, per-frame token ranges) stay plain Python as in the
  reference, because callers read them;
* ``lvsa_sdpa`` and the FlashInfer backend run the hand-written gfx950
  block-sparse attention kernel (``lvsa_attn_fwd``) in one launch instead of
  a per-frame ``cat`` + SDPA loop or a FlashInfer plan;
* ``lvsa_attention`` adds the zero-copy fused form: global and window frames
  are read in place from ``key``/``value`` by frame index, text keys are
  always-attended extra rows and text queries are dense rows of the same
  launch.

There is no CPU path: tensor entry points require GPU tensors and raise
otherwise.
"""

from __future__ import annotations

import math
import os
import sys
import threading
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Any, Dict, Iterator, List, Optional, Set, Tuple

import torch

from . import hip_ops

# ═══════════════════════════════════════════════════════════════════════════════
# Pattern helpers (host; same semantics as lvsa/sparse_attention.py:40-216)
# ═══════════════════════════════════════════════════════════════════════════════


def adaptive_window_bounds(f: int, W: int, T: int) -> Tuple[int, int]:
    """Window of constant width ``min(2W+1, T)`` around frame ``f``, shifted
    inward at the sequence edges (``lvsa/sparse_attention.py:40-47``)."""
    start = f - W
    if start > T - 1 - 2 * W:
        start = T - 1 - 2 * W
    end = f + W
    if end < 2 * W:
        end = 2 * W
    return (start if start > 0 else 0), (end if end < T - 1 else T - 1)


def _outward(lo: int, hi: int, T: int) -> Iterator[int]:
    """Frames outside ``[lo, hi]`` in the order the expansion visits them:
    left, right, left, right, ... continuing on one side once the other is
    exhausted."""
    left, right = lo - 1, hi + 1
    while left >= 0 or right <= T - 1:
        if left >= 0:
            yield left
            left -= 1
        if right <= T - 1:
            yield right
            right += 1


def expanded_window_bounds(
    f: int, W: int, T: int,
    global_set: Set[int],
    global_count: int,
) -> Tuple[int, int]:
    """Expand the adaptive window until it holds ``min(2W+1, T-|G|)`` non-global
    frames (``lvsa/sparse_attention.py:50-86``).

    Total unique attended frames = ``|G| + min(2W+1, T-|G|)``.
    """
    lo, hi = adaptive_window_bounds(f, W, T)
    target = min(2 * W + 1, T - global_count)
    count = sum(1 for x in range(lo, hi + 1) if x not in global_set)
    if count >= target:
        return lo, hi
    for x in _outward(lo, hi, T):
        if x < lo:
            lo = x
        else:
            hi = x
        if x not in global_set:
            count += 1
            if count >= target:
                break
    return lo, hi


def get_window_bounds(
    f: int, W: int, T: int,
    expand: bool,
    global_set: Set[int],
    global_count: int,
) -> Tuple[int, int]:
    """Expanded or adaptive bounds; ``W == 0`` (globals-only) gives the empty
    range ``(f, f-1)`` (``lvsa/sparse_attention.py:89-104``)."""
    if W == 0:
        return f, f - 1
    if expand:
        return expanded_window_bounds(f, W, T, global_set, global_count)
    return adaptive_window_bounds(f, W, T)


def compute_boundary_guard_frames(
    total_frames: int,
    local_seq: int,
    num_patches: int,
    world: int,
    window_size: int,
) -> List[int]:
    """Frames within ±W of each context-parallel token split
    (``lvsa/sparse_attention.py:107-129``)."""
    guards: Set[int] = set()
    for r in range(1, world):
        centre = (r * local_seq) // num_patches
        guards.update(range(max(0, centre - window_size), min(total_frames, centre + window_size + 1)))
    return sorted(guards)


def compute_auto_kfi(
    total_frames: int,
    window_size: int,
    n_first_frames: int,
    reference_frames: int = 21,
    sparsity_scale: float = 1.0,
) -> int:
    """Keyframe interval giving ≈ ``reference_frames·sparsity_scale`` attended
    frames per query (``lvsa/sparse_attention.py:132-195``): the larger of the
    strict interval (largest kfi whose anchor set reaches the global budget)
    and the closed-form fallback."""
    T, W, n = total_frames, window_size, n_first_frames
    budget = max(n + 1, int(reference_frames * sparsity_scale))
    if T <= budget:
        return 1
    globals_needed = max(n, min(budget, T) - min(2 * W + 1, T))
    anchors = set(range(min(n, T)))
    strict = 1
    for kfi in range(T, 0, -1):
        if len(anchors.union(range(0, T, kfi))) >= globals_needed:
            strict = kfi
            break
    mandatory = 2 * W + n
    fallback = math.ceil(max(T - mandatory, budget - mandatory) / max(budget - mandatory, 1))
    return max(strict, fallback)


def compute_global_indices(
    total_frames: int,
    n_first_frames: int,
    key_frame_interval: Optional[int],
    offset: int = 0,
) -> List[int]:
    """Sorted global (anchor) frames: ``0..n_first-1`` plus ``ceil(T/kfi)``
    keyframes ``(offset + i·kfi) mod T`` (``lvsa/sparse_attention.py:198-216``)."""
    T = total_frames
    flags = bytearray(T)
    for i in range(min(n_first_frames, T)):
        flags[i] = 1
    if key_frame_interval is not None and key_frame_interval > 0:
        for i in range(-(-T // key_frame_interval)):
            flags[(offset + i * key_frame_interval) % T] = 1
    return [i for i in range(T) if flags[i]]


def print_attention_mask_compact(
    total_frames: int,
    window_size: int,
    global_set: Set[int],
    expand_window: bool,
    file=None,
) -> None:
    """One character per key frame: ``G`` global, ``W`` window, ``X`` both,
    ``.`` skipped; each row ends with its attended count
    (``lvsa/sparse_attention.py:219-278``)."""
    T = total_frames
    width = len(str(T - 1)) if T > 1 else 1
    print(" " * (width + 2) + "".join(str(k % 10) if k % 5 == 0 else " " for k in range(T)), file=file)
    counts = []
    for f in range(T):
        lo, hi = get_window_bounds(f, window_size, T, expand_window, global_set, len(global_set))
        win = set(range(lo, hi + 1)) if lo <= hi else set()
        glyph = {(True, True): "X", (True, False): "G", (False, True): "W", (False, False): "."}
        row = "".join(glyph[(k in global_set, k in win)] for k in range(T))
        counts.append(len(global_set | win))
        print(f"{f:>{width}} |{row}| {counts[-1]}", file=file)
    if counts:
        print(f"G=global W=window X=both .=skip  min={min(counts)} max={max(counts)} "
              f"avg={sum(counts) / len(counts):.1f}/{T}", file=file)


# ═══════════════════════════════════════════════════════════════════════════════
# LVSAMetadata
# ═══════════════════════════════════════════════════════════════════════════════


@dataclass
class _DeviceState:
    """The device mask and block plans of one pattern on one GPU.

    A pattern is shared (``LVSAMetadata.build`` returns one instance per set of
    arguments), so its tensors can be built on one stream and read on others.
    Every build records ``ready`` on its stream and bumps ``version``; a stream
    that has not joined the current version first waits for ``ready`` and
    registers itself with the caching allocator (``record_stream``), so an
    evicted pattern's memory is not reused while that stream may still read
    it.  Not done under stream capture: build a pattern before capturing it.
    """

    mask: hip_ops.DeviceMask
    plans: Dict[Tuple, hip_ops.BlockPlan] = field(default_factory=dict)
    ready: Optional[torch.cuda.Event] = None
    version: int = 0
    joined: Dict[int, int] = field(default_factory=dict)   # stream handle -> version it has waited for

    def _tensors(self):
        m = self.mask
        ts = [m.frame_indptr, m.frame_indices, m.compact_frames, m.global_frames, m.window_bounds, m.rel_full,
              m.rel_window, m.info]
        for p in self.plans.values():
            ts += [p.tile_indptr, p.entries, p.status]
            if p._fallback is not None:
                ts += [p._fallback.tile_indptr, p._fallback.entries, p._fallback.status]
        return ts

    def built(self, device: torch.device) -> None:
        """Mark a build just enqueued on the current stream of ``device``."""
        if torch.cuda.is_current_stream_capturing():
            return
        s = torch.cuda.current_stream(device)
        if self.ready is None:
            self.ready = torch.cuda.Event()
        self.ready.record(s)
        self.version += 1
        self.joined[s.cuda_stream] = self.version

    def join(self, device: torch.device) -> None:
        """Order the current stream of ``device`` after every build so far."""
        if self.ready is None or torch.cuda.is_current_stream_capturing():
            return
        s = torch.cuda.current_stream(device)
        if self.joined.get(s.cuda_stream, 0) == self.version:
            return
        s.wait_event(self.ready)
        for t in self._tensors():
            t.record_stream(s)
        self.joined[s.cuda_stream] = self.version


# Patterns built by LVSAMetadata.build, shared by every caller that asks for
# the same one.  The reference's plugin hooks (``attention_impl.py:387-419``,
# ``hunyuan_hook.py:185-215``) keep one pattern per attention layer and rebuild
# it at every denoising step; with the cache the layers of a step share one
# build, one device mask and one set of block plans.
_BUILD_CACHE: "OrderedDict[tuple, LVSAMetadata]" = OrderedDict()
_BUILD_LOCK = threading.Lock()


def _build_cache_size() -> int:
    """Patterns kept (LRU): ``LVSA_METADATA_CACHE``, default 16; 0 turns the cache off."""
    try:
        return max(0, int(os.environ.get("LVSA_METADATA_CACHE", "16")))
    except ValueError:
        return 16


def clear_metadata_cache() -> None:
    """Drop every cached pattern (and with it, once unreferenced, its device mask and plans)."""
    with _BUILD_LOCK:
        _BUILD_CACHE.clear()


@dataclass
class LVSAMetadata:
    """Pre-computed sparse attention pattern (``lvsa/sparse_attention.py:286-333``).

    Host fields are plain Python (callers read them).  The FlashInfer CSR
    (``fi_indptr`` / ``fi_indices``) and the frame relation live on the GPU:
    they are produced by the ``lvsa_mask_build`` kernel on first use on a
    device (``ensure_device`` or any attention call) and returned as device
    int32 tensors.

    ``build`` returns one shared instance per set of pattern arguments (and
    current GPU), so an instance is read-only, as the reference's callers
    treat it.
    """

    # ── Pattern config ──
    total_latent_frames: int
    num_patches: int
    window_size: int
    n_first_frames: int
    key_frame_interval: Optional[int]
    expand_window: bool
    rank: int
    world: int

    # ── Derived geometry ──
    local_seq: int
    global_token_start: int
    global_indices: List[int]
    global_set: Set[int]
    local_frames: List[Tuple[int, int, int]]
    window_ctx: Dict[int, List[Tuple[int, int]]]

    # ── Frame-level tables ──
    global_frame_mask: torch.Tensor
    window_bounds: torch.Tensor
    attended_C: int

    # ── FlashInfer CSR geometry ──
    fi_M: int
    fi_N: int
    fi_MB: int
    fi_compact_n: int
    fi_global_copies: List[Tuple[int, int]]
    fi_local_copies: List[Tuple[int, int]]

    keyframe_offset: int = 0
    boundary_guards: List[int] = field(default_factory=list)
    fi_nnz: int = 0
    max_row_frames: int = 0
    _attended_rows: List[List[int]] = field(default_factory=list, repr=False)
    _device_state: Dict[str, _DeviceState] = field(default_factory=dict, repr=False)
    _home_device: Optional[torch.device] = field(default=None, repr=False)

    @classmethod
    @torch.compiler.disable
    def build(
        cls,
        total_latent_frames: int,
        num_patches: int,
        window_size: int,
        n_first_frames: int,
        key_frame_interval: Optional[int],
        rank: int,
        world: int,
        expand_window: bool = True,
        keyframe_offset: int = 0,
        boundary_guards: Optional[List[int]] = None,
        reference_frames: int = 21,
        sparsity_scale: float = 1.0,
    ) -> "LVSAMetadata":
        """Derive the host-side pattern state (``lvsa/sparse_attention.py:335-484``).

        ``key_frame_interval`` is used verbatim (callers wanting auto-scaling
        call ``compute_auto_kfi`` first); ``reference_frames`` and
        ``sparsity_scale`` are accepted for signature compatibility.

        Repeated arguments return the instance built first (an LRU of
        ``LVSA_METADATA_CACHE`` patterns, default 16, keyed also by the current
        GPU), with the device mask and plans it has already built.
        """
        guards_key = tuple(sorted(set(boundary_guards or [])))
        dev = torch.cuda.current_device() if torch.cuda.is_available() else -1
        key = (total_latent_frames, num_patches, window_size, n_first_frames, key_frame_interval, rank, world,
               bool(expand_window), keyframe_offset, guards_key, dev)
        size = _build_cache_size()
        if size:
            with _BUILD_LOCK:
                hit = _BUILD_CACHE.get(key)
                if hit is not None:
                    _BUILD_CACHE.move_to_end(key)
                    return hit
        m = cls._build(total_latent_frames, num_patches, window_size, n_first_frames, key_frame_interval, rank,
                       world, expand_window, keyframe_offset, boundary_guards)
        if size:
            with _BUILD_LOCK:
                m = _BUILD_CACHE.setdefault(key, m)
                _BUILD_CACHE.move_to_end(key)
                while len(_BUILD_CACHE) > size:
                    _BUILD_CACHE.popitem(last=False)
        return m

    @classmethod
    def _build(cls, total_latent_frames: int, num_patches: int, window_size: int, n_first_frames: int,
               key_frame_interval: Optional[int], rank: int, world: int, expand_window: bool,
               keyframe_offset: int, boundary_guards: Optional[List[int]]) -> "LVSAMetadata":
        T, P, W = total_latent_frames, num_patches, window_size
        total_seq = T * P
        assert total_seq % world == 0, (
            f"total_seq={total_seq} (T={T} x P={P}) must be divisible by world={world}."
        )
        local_seq = total_seq // world
        gts = rank * local_seq
        kfi = key_frame_interval
        guards = sorted(set(boundary_guards or []))
        G = sorted(set(compute_global_indices(T, n_first_frames, kfi, keyframe_offset)) | set(guards))
        Gs = set(G)
        nG = len(G)
        bounds = [get_window_bounds(f, W, T, expand_window, Gs, nG) for f in range(T)]

        def on_rank(fr: int) -> Tuple[int, int]:
            return max(fr * P, gts) - gts, min((fr + 1) * P, gts + local_seq) - gts

        first, last = gts // P, (gts + local_seq - 1) // P
        local_frames = [(fr, *on_rank(fr)) for fr in range(first, last + 1)]
        window_ctx: Dict[int, List[Tuple[int, int]]] = {}
        for fr, _, _ in local_frames:
            lo, hi = bounds[fr]
            window_ctx[fr] = [on_rank(wf) for wf in range(lo, hi + 1)
                              if wf not in Gs and on_rank(wf)[0] < on_rank(wf)[1]]

        attended_rows = []
        for fr in range(first, last + 1):
            lo, hi = bounds[fr]
            attended_rows.append(sorted(Gs.union(range(lo, hi + 1))))
        attended_C = max(len(r) for r in attended_rows)

        # CSR geometry: MB rows from the first local frame; compact ids number
        # the union of all rows (lvsa/sparse_attention.py:550-635).
        MB = -(-local_seq // P)
        union: Set[int] = set()
        nnz = 0
        row_max = 0
        for qi in range(MB):
            fr = first + qi
            lo, hi = bounds[fr]
            row = Gs | {wf for wf in range(lo, hi + 1) if wf not in Gs and on_rank(wf)[0] < on_rank(wf)[1]}
            union |= row
            nnz += len(row)
            row_max = max(row_max, len(row))
        compact = sorted(union)
        gpos = {g: i for i, g in enumerate(G)}
        gcop = [(gpos[fr] * P, ci * P) for ci, fr in enumerate(compact) if fr in Gs]
        lcop = [(fr * P - gts, ci * P) for ci, fr in enumerate(compact) if fr not in Gs]

        gmask = torch.zeros(T, dtype=torch.int8)
        if G:
            gmask[torch.tensor(G)] = 1
        return cls(
            total_latent_frames=T, num_patches=P, window_size=W, n_first_frames=n_first_frames,
            key_frame_interval=kfi, expand_window=expand_window, rank=rank, world=world,
            local_seq=local_seq, global_token_start=gts, global_indices=G, global_set=Gs,
            local_frames=local_frames, window_ctx=window_ctx,
            global_frame_mask=gmask, window_bounds=torch.tensor(bounds, dtype=torch.int32).reshape(T, 2),
            attended_C=attended_C,
            fi_M=MB * P, fi_N=len(compact) * P, fi_MB=MB, fi_compact_n=len(compact),
            fi_global_copies=gcop, fi_local_copies=lcop,
            keyframe_offset=keyframe_offset, boundary_guards=guards, fi_nnz=nnz,
            max_row_frames=row_max, _attended_rows=attended_rows,
        )

    # ── Lazily materialised tables of the reference API ──

    @property
    def attended_indices(self) -> torch.Tensor:
        """``[T_local, C]`` attended frames per local frame, padded with the row's last value."""
        C = self.attended_C
        rows = [r + [r[-1]] * (C - len(r)) for r in self._attended_rows]
        return torch.tensor(rows, dtype=torch.int32).reshape(len(rows), C)

    def _frame_token_index(self, frames: List[int], base: torch.Tensor) -> torch.Tensor:
        P = self.num_patches
        if not frames:
            return torch.empty(0, dtype=torch.long)
        t = torch.arange(P, dtype=torch.long)
        return (base[:, None] * P + t[None, :]).reshape(-1)

    @property
    def global_src_idx(self) -> torch.Tensor:
        G = self.global_indices
        return self._frame_token_index(G, torch.arange(len(G), dtype=torch.long))

    @property
    def global_dst_idx(self) -> torch.Tensor:
        G = self.global_indices
        return self._frame_token_index(G, torch.tensor(G, dtype=torch.long))

    def _local_nonglobal(self) -> List[Tuple[int, int]]:
        return [(s, e) for fr, s, e in self.local_frames if fr not in self.global_set and s < e]

    @property
    def local_src_idx(self) -> torch.Tensor:
        parts = [torch.arange(s, e, dtype=torch.long) for s, e in self._local_nonglobal()]
        return torch.cat(parts) if parts else torch.empty(0, dtype=torch.long)

    @property
    def local_dst_idx(self) -> torch.Tensor:
        g = self.global_token_start
        parts = [torch.arange(s + g, e + g, dtype=torch.long) for s, e in self._local_nonglobal()]
        return torch.cat(parts) if parts else torch.empty(0, dtype=torch.long)

    # ── Device state ──

    def _mask_params(self):
        return hip_ops.mask_params(
            self.total_latent_frames, self.num_patches, self.window_size, self.n_first_frames,
            self.key_frame_interval, self.keyframe_offset, self.expand_window, self.rank, self.world,
            self.boundary_guards)

    def device_state(self, device: Optional[torch.device] = None) -> _DeviceState:
        """Build (once per device) the GPU mask: CSR + relation bitmaps."""
        if device is None:
            device = self._home_device
        if device is None:
            if not torch.cuda.is_available():
                raise RuntimeError("LVSAMetadata device tensors need a GPU (the mask is built by a HIP kernel)")
            device = torch.device("cuda", torch.cuda.current_device())
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        key = str(device)
        st = self._device_state.get(key)
        if st is None:
            st = _DeviceState(hip_ops.mask_build(self._mask_params(), device))
            st.built(device)
            self._device_state[key] = st
        st.join(device)
        return st

    def ensure_device(self, device: torch.device) -> None:
        """Build the device-side mask on ``device`` (idempotent).

        The reference moves its index tensors here; this implementation
        builds the CSR and relation bitmaps on the device with the mask kernel
        and makes ``device`` the home of ``fi_indptr`` / ``fi_indices``.  A CPU
        device is a no-op (host fields are always available).
        """
        device = torch.device(device)
        if device.type == "cpu":
            return
        self.device_state(device)
        self._home_device = device

    @property
    def fi_indptr(self) -> torch.Tensor:
        return self.device_state().mask.frame_indptr

    @property
    def fi_indices(self) -> torch.Tensor:
        return self.device_state().mask.frame_indices[: self.fi_nnz]

    @property
    def compact_frames(self) -> torch.Tensor:
        return self.device_state().mask.compact_frames[: self.fi_compact_n]

    # ── Block plans (cached per device and call geometry) ──

    def window_plan(self, device: torch.device, n_q: int, n_k: int, n_extra: int,
                    head_dim: int = 128, dtype: Optional[torch.dtype] = None) -> hip_ops.BlockPlan:
        """Plan for ``lvsa_sdpa`` semantics: every query row attends all extra
        rows (``k_global``) plus the non-global window frames of its frame."""
        st = self.device_state(device)
        block_q = hip_ops.attn_block_q(head_dim, dtype, self.num_patches, self.num_patches, n_k=n_k,
                                       k_tok0=self.global_token_start)
        key = ("window", n_q, n_k, n_extra, block_q)
        plan = st.plans.get(key)
        if plan is None:
            P, gts = self.num_patches, self.global_token_start
            plan = hip_ops.plan_build(
                st.mask.rel_window, n_q=n_q, n_k=n_k, n_x=n_extra, R=P, Cf=P, q_tok0=gts, k_tok0=gts,
                q_frame0=gts // P, max_row_frames=max(1, 2 * self.window_size + 1), block_q=block_q)
            st.plans[key] = plan
            st.built(st.mask.info.device)
        return plan

    def full_plan(self, device: torch.device, n_q: int, n_k: int, n_text_k: int, n_text_q: int,
                  head_dim: int = 128, dtype: Optional[torch.dtype] = None) -> hip_ops.BlockPlan:
        """Zero-copy plan: query rows attend their global + window frames of
        ``key`` directly, all text keys, and text queries attend everything."""
        if self.world != 1:
            raise NotImplementedError("zero-copy LVSA attention needs the whole sequence on one GPU (world=1)")
        st = self.device_state(device)
        block_q = hip_ops.attn_block_q(head_dim, dtype, self.num_patches, self.num_patches, n_k=n_k)
        key = ("full", n_q, n_k, n_text_k, n_text_q, block_q)
        plan = st.plans.get(key)
        if plan is None:
            P = self.num_patches
            plan = hip_ops.plan_build(
                st.mask.rel_full, n_q=n_q, n_k=n_k, n_x=n_text_k, n_tq=n_text_q, R=P, Cf=P,
                max_row_frames=max(1, self.max_row_frames), block_q=block_q)
            st.plans[key] = plan
            st.built(st.mask.info.device)
        return plan


# ═══════════════════════════════════════════════════════════════════════════════
# Backends
# ═══════════════════════════════════════════════════════════════════════════════

_COMPUTE_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _compute_dtype(t: torch.Tensor) -> torch.dtype:
    """The caller's dtype, as the reference computes (``lvsa/sparse_attention.py:670,
    689-704``): bf16 and fp16 on the 16-bit MFMA kernels, fp32 on the fp32
    kernel; other types (fp64) run in fp32 and are cast back."""
    return t.dtype if t.dtype in _COMPUTE_DTYPES else torch.float32


def _check_local_seq(query: torch.Tensor, metadata: LVSAMetadata) -> None:
    # The metadata's relation has one row per local frame; the kernels map
    # query row r to frame (global_token_start + r) // P, so the query length
    # must be the metadata's local sequence (the reference slices
    # metadata.local_frames out of it, lvsa/sparse_attention.py:668-675).
    if query.dim() != 4 or query.shape[1] != metadata.local_seq:
        raise ValueError(f"query has shape {tuple(query.shape)}; the metadata describes [B, "
                         f"local_seq={metadata.local_seq}, H, D]")


def _as(t: Optional[torch.Tensor], dtype: torch.dtype) -> Optional[torch.Tensor]:
    return None if t is None or t.dtype == dtype else t.to(dtype)


def lvsa_sdpa(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    k_global: torch.Tensor,
    v_global: torch.Tensor,
    metadata: LVSAMetadata,
    attention_backend: Any = None,
) -> torch.Tensor:
    """Block-sparse LVSA with the semantics of the reference's per-frame loop
    (``lvsa/sparse_attention.py:643-706``), as one HIP kernel launch.

    Every query token of local frame ``f`` attends all rows of ``k_global``
    (pre-gathered global frames, plus any appended text) and the non-global
    window frames of ``f`` read in place from ``key``/``value``.

    query : [B, local_seq, H, D];  key, value, k_global, v_global : [B, *, H_kv, D]
        ``H_kv`` may divide ``H`` (grouped-query attention, handled natively).
    ``attention_backend`` is accepted for signature compatibility and ignored.
    Returns a new tensor with the dtype of ``query``, computed in that dtype
    (fp64 in fp32).
    """
    _check_local_seq(query, metadata)
    hip_ops._require_device(query, "query")
    dt = _compute_dtype(query)
    plan = metadata.window_plan(query.device, query.shape[1], key.shape[1], k_global.shape[1], query.shape[-1],
                                dt)
    q, k, v, kg, vg = (x if x.dtype == dt else x.to(dt) for x in (query, key, value, k_global, v_global))
    out, _, _, _ = hip_ops.attn_fwd(q, k, v, plan, kx=kg, vx=vg)
    return out if out.dtype == query.dtype else out.to(query.dtype)


def lvsa_flashinfer(
    query_padded: torch.Tensor,
    k_compact: torch.Tensor,
    v_compact: torch.Tensor,
    fi_wrapper: Any,
    local_seq: int,
    fi_M: int,
) -> torch.Tensor:
    """Block-sparse LVSA through a planned block-sparse wrapper
    (``lvsa/sparse_attention.py:709-742``).

    ``fi_wrapper`` is a :class:`~longvideosparseattention_amd.block_sparse.BlockSparseAttentionWrapper`
    (the HIP replacement of FlashInfer's wrapper) planned with the metadata's
    CSR; ``query_padded`` is ``[B, M, H, D]`` with ``M = MB·P``.
    """
    B = query_padded.shape[0]
    H, D = query_padded.shape[2], query_padded.shape[3]
    if hasattr(fi_wrapper, "run_batched"):
        # this package's wrapper: the whole batch in one launch (the reference
        # runs one FlashInfer call per batch element)
        return fi_wrapper.run_batched(query_padded, k_compact, v_compact)[:, :local_seq]
    output = query_padded.new_empty(B, fi_M, H, D)
    for b in range(B):
        output[b] = fi_wrapper.run(query_padded[b], k_compact[b], v_compact[b])
    return output[:, :local_seq]


def sparse_windowed_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    k_global: torch.Tensor,
    v_global: torch.Tensor,
    metadata: LVSAMetadata,
    backend: str = "sdpa",
    *,
    k_compact: Optional[torch.Tensor] = None,
    v_compact: Optional[torch.Tensor] = None,
    fi_wrapper: Optional[Any] = None,
    attention_backend: Any = None,
) -> torch.Tensor:
    """Top-level dispatcher (``lvsa/sparse_attention.py:750-788``).

    ``backend="sdpa"`` (default, also ``"hip"``) runs :func:`lvsa_sdpa`;
    ``backend="flashinfer"`` runs :func:`lvsa_flashinfer` and requires the
    pre-filled compact buffers and a planned wrapper.
    """
    if backend == "flashinfer":
        assert k_compact is not None and v_compact is not None and fi_wrapper is not None, (
            "FlashInfer backend requires k_compact, v_compact, and fi_wrapper"
        )
        return lvsa_flashinfer(query, k_compact, v_compact, fi_wrapper, metadata.local_seq, metadata.fi_M)
    return lvsa_sdpa(query, key, value, k_global, v_global, metadata, attention_backend)


def lvsa_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    metadata: LVSAMetadata,
    *,
    k_text: Optional[torch.Tensor] = None,
    v_text: Optional[torch.Tensor] = None,
    q_text: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    return_lse: bool = False,
):
    """Zero-copy fused LVSA attention (one launch).

    Video queries attend the global and window frames of their frame, read in
    place from ``key``/``value`` (no ``build_global_kv`` copy), plus every
    text key; text queries (``q_text``) attend all video and text keys
    densely — the joint-text semantics of the reference's processor
    (``lvsa/lvsa_processor.py:545-591``) and FlashInfer runner
    (``flashinfer_runner.py:96-198``) without the LSE merge.

    Returns ``out`` or ``(out, out_text)`` when ``q_text`` is given; with
    ``return_lse`` the natural-log LSE ``[B, H, S]`` tensors are appended.
    """
    _check_local_seq(query, metadata)
    hip_ops._require_device(query, "query")
    dt = _compute_dtype(query)
    n_tk = 0 if k_text is None else k_text.shape[1]
    n_tq = 0 if q_text is None else q_text.shape[1]
    plan = metadata.full_plan(query.device, query.shape[1], key.shape[1], n_tk, n_tq, query.shape[-1], dt)
    cast = lambda x: x if (x is None or x.dtype == dt) else x.to(dt)  # noqa: E731
    out, out_t, lse, lse_t = hip_ops.attn_fwd(
        cast(query), cast(key), cast(value), plan, kx=cast(k_text), vx=cast(v_text), qt=cast(q_text),
        scale=scale, return_lse=return_lse)
    if out.dtype != query.dtype:
        out = out.to(query.dtype)
        out_t = None if out_t is None else out_t.to(query.dtype)
    res = (out,) if q_text is None else (out, out_t)
    if return_lse:
        res = res + ((lse,) if q_text is None else (lse, lse_t))
    return res[0] if len(res) == 1 else res
