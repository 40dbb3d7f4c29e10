"""Stateful LVSA attention processor on the gfx950 kernels.

Mirror of ``DistributedLVSAProcessor`` (``lvsa/lvsa_processor.py:68-913``):
the same constructor, the step / window / sparsity controls that rebuild the
pattern (``set_step`` ``:317-331``, ``set_window_size`` ``:288-315``,
``set_sparsity_scale`` ``:333-360``, ``_rebuild_for_current_params``
``:362-405``), the geometry guard with its dense fallback (``:529-582``,
``:611-641``), the dual-stream encoder queries (``:586-591``, ``:710-735``)
and the model-agnostic ``__call__`` that delegates projections, RoPE,
cross-attention and output formatting to an adapter (``:454-609``).

What changes is the attention itself: one fused launch per call
(:func:`~longvideosparseattention_amd.sparse_attention.lvsa_attention`)
covers the video queries over their global and window frames plus every
encoder key, and the encoder queries over all keys.  The global K/V buffer,
its all-reduce and the FlashInfer compact copies are not needed: the kernel
reads global frames in place.  ``_use_flashinfer`` is kept (the reference's
``lvsa/parallel.py:160`` sets it) and selects the same kernel, since both
reference backends compute the same attention.

Only ``world == 1`` runs: the K/V of another rank's frames would need the
collectives this build leaves out.  ``adapter`` is duck-typed; the
reference's default (``WanAdapter``, built on diffusers) is not part of this
package, so ``__call__`` needs one (``attention`` does not).
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Any, Optional, Tuple

import torch

from . import hip_ops
from .global_kv import build_global_kv
from .sparse_attention import (
    LVSAMetadata,
    _compute_dtype,
    adaptive_window_bounds,
    compute_auto_kfi,
    compute_boundary_guard_frames,
    compute_global_indices,
    expanded_window_bounds,
    get_window_bounds,
    lvsa_attention,
    lvsa_sdpa,
    print_attention_mask_compact,
)


class DistributedLVSAProcessor:
    """Block-sparse LVSA self-attention with keyframe rotation (see module doc)."""

    _attention_backend = None
    _parallel_config = None
    # Parameter sets (window, kfi, sparsity) whose patterns stay cached: the
    # current one and the one before it (denoising schedules alternate a
    # windowed and a globals-only band); older sets and their device masks
    # and plans are dropped, as the reference drops its state on a rebuild.
    _PATTERN_SETS = 2

    def __init__(
        self,
        total_num_latent_frames: int,
        num_patches: int,
        window_size: int,
        n_first_frames: int,
        key_frame_interval: Optional[int],
        rank: int,
        world: int,
        expand_window: bool = True,
        adapter: Optional[Any] = None,
        sparsity_scale: float = 1.0,
        reference_frames: int = 21,
    ) -> None:
        self.total_num_frames = total_num_latent_frames
        self.num_patches = num_patches
        self.window_size = window_size
        self.n_first_frames = n_first_frames
        self.rank = rank
        self.world = world
        self._expand_window = expand_window
        self._sparsity_scale = sparsity_scale
        self._reference_frames = reference_frames
        self.adapter = adapter
        self._use_flashinfer = False
        self._geometry_warned = False
        self._dense_plans = {}
        self._pattern_cache: "OrderedDict[tuple, dict]" = OrderedDict()
        # Boundary guards stay fixed across rotations (lvsa_processor.py:135-140).
        self._boundary_guards = compute_boundary_guard_frames(
            total_num_latent_frames, total_num_latent_frames * num_patches // world,
            num_patches, world, window_size)
        self.key_frame_interval = key_frame_interval
        self._current_offset = 0
        self._metadata = self._build(0)
        self._copy_metadata_to_self()
        self._log_config()

    # ── pattern state ──────────────────────────────────────────────────────

    def _build(self, offset: int) -> LVSAMetadata:
        """The pattern for ``offset`` under the current window / kfi / sparsity.

        Patterns are kept per parameter set: a denoising run cycles through
        ``kfi`` offsets, so every rotation after the first cycle reuses the
        metadata together with its device mask and block plans."""
        params = (self.window_size, self.key_frame_interval, self._sparsity_scale)
        per_offset = self._pattern_cache.get(params)
        if per_offset is None:
            per_offset = self._pattern_cache[params] = {}
            while len(self._pattern_cache) > self._PATTERN_SETS:
                self._pattern_cache.popitem(last=False)
        else:
            self._pattern_cache.move_to_end(params)
        meta = per_offset.get(offset)
        if meta is None:
            meta = per_offset[offset] = self._build_uncached(offset)
        return meta

    def _build_uncached(self, offset: int) -> LVSAMetadata:
        return LVSAMetadata.build(
            total_latent_frames=self.total_num_frames, num_patches=self.num_patches,
            window_size=self.window_size, n_first_frames=self.n_first_frames,
            key_frame_interval=self.key_frame_interval, rank=self.rank, world=self.world,
            expand_window=self._expand_window, keyframe_offset=offset,
            boundary_guards=self._boundary_guards, reference_frames=self._reference_frames,
            sparsity_scale=self._sparsity_scale)

    def _copy_metadata_to_self(self) -> None:
        """The reference exposes the metadata fields as processor attributes
        (lvsa_processor.py:203-233); the device CSR stays on the metadata."""
        m = self._metadata
        self.local_seq = m.local_seq
        self.global_token_start = m.global_token_start
        self.key_frame_interval = m.key_frame_interval
        self._global_indices = m.global_indices
        self._global_set = m.global_set
        self._local_frames = m.local_frames
        self._window_ctx = m.window_ctx
        self._global_frame_mask = m.global_frame_mask
        self._window_bounds = m.window_bounds
        self._attended_C = m.attended_C
        self._fi_M, self._fi_N, self._fi_MB = m.fi_M, m.fi_N, m.fi_MB
        self._fi_compact_n = m.fi_compact_n
        self._fi_global_copies = m.fi_global_copies
        self._fi_local_copies = m.fi_local_copies

    # Index tensors are derived on first access (the CSR by the mask kernel,
    # on the GPU), so they are read through the metadata, not copied.
    _attended_indices = property(lambda self: self._metadata.attended_indices)
    _global_src_idx = property(lambda self: self._metadata.global_src_idx)
    _global_dst_idx = property(lambda self: self._metadata.global_dst_idx)
    _local_src_idx = property(lambda self: self._metadata.local_src_idx)
    _local_dst_idx = property(lambda self: self._metadata.local_dst_idx)
    _fi_indptr = property(lambda self: self._metadata.fi_indptr)
    _fi_indices = property(lambda self: self._metadata.fi_indices)

    @property
    def metadata(self) -> LVSAMetadata:
        return self._metadata

    def _log_config(self) -> None:
        """One summary line on rank 0 (lvsa_processor.py:178-201)."""
        if self.rank != 0:
            return
        P, T = self.num_patches, self.total_num_frames
        first, last = self.global_token_start // P, (self.global_token_start + self.local_seq - 1) // P
        lo, hi = self._get_window_bounds((first + last) // 2, self.window_size, T)
        attended = len(self._global_set | set(range(lo, hi + 1)))
        print(f"[LVSA] total_lat_frames={T}  local_seq={self.local_seq}  rank0_frames~[{first},{last}]  "
              f"window={self.window_size}  n_first={self.n_first_frames}  "
              f"kfi={self.key_frame_interval or 'none'}  global_count={len(self._global_indices)}  "
              f"attended_per_frame={attended}/{T}")

    def _rebuild_for_current_params(self, offset: int) -> None:
        self._current_offset = offset
        self._metadata = self._build(offset)
        self._copy_metadata_to_self()

    def set_step(self, step_idx: int) -> None:
        """Rotate the periodic keyframes: offset = step_idx % kfi; nothing to
        do without keyframes or when the offset is unchanged."""
        if not self.key_frame_interval:
            return
        offset = step_idx % self.key_frame_interval
        if offset == self._current_offset:
            return
        self._rebuild_for_current_params(offset)

    def _derive_kfi(self) -> int:
        """``compute_auto_kfi`` for the current window and budget.  With a GPU
        present it runs as ``lvsa_auto_kfi`` on the device (one 4-byte read
        back, since the host pattern fields depend on it); host-only processes
        (no HIP device) evaluate the reference's formula in Python."""
        if torch.cuda.is_available():
            kfi = hip_ops.auto_kfi(self.total_num_frames, self.window_size, self.n_first_frames,
                                   self._reference_frames, self._sparsity_scale)
            return int(kfi.item())
        return compute_auto_kfi(
            self.total_num_frames, self.window_size, self.n_first_frames,
            reference_frames=self._reference_frames, sparsity_scale=self._sparsity_scale)

    def _retune_kfi(self) -> None:
        self.key_frame_interval = self._derive_kfi()
        old_offset = self._current_offset
        self._current_offset = -1
        self._rebuild_for_current_params(old_offset)

    def set_window_size(self, new_window_size: int) -> None:
        """Switch the window (0: globals only); kfi is re-derived for the new
        budget split and the pattern rebuilt."""
        if new_window_size == self.window_size:
            return
        self.window_size = new_window_size
        self._retune_kfi()

    def set_sparsity_scale(self, new_sparsity_scale: float) -> None:
        """< 1.0: fewer attended frames, > 1.0: more; kfi is re-derived."""
        if new_sparsity_scale == self._sparsity_scale:
            return
        self._sparsity_scale = new_sparsity_scale
        self._retune_kfi()

    def _get_window_bounds(self, f: int, W: int, T: int) -> Tuple[int, int]:
        return get_window_bounds(f, W, T, self._expand_window, self._global_set, len(self._global_indices))

    def _expanded_window_bounds(self, f: int, W: int, T: int) -> Tuple[int, int]:
        return expanded_window_bounds(f, W, T, self._global_set, len(self._global_indices))

    # Static delegators of the reference (lvsa_processor.py:414-448).
    _adaptive_window_bounds = staticmethod(adaptive_window_bounds)
    _compute_boundary_guard_frames = staticmethod(compute_boundary_guard_frames)
    _compute_auto_kfi = staticmethod(compute_auto_kfi)
    _compute_global_indices = staticmethod(compute_global_indices)

    def print_attention_mask(self) -> None:
        """T x T frame matrix: G = global, W = window, X = both, . = not attended."""
        T, W = self.total_num_frames, self.window_size
        print("Q\\K " + "".join(f"{k:>3}" for k in range(T)))
        print("    " + "---" * T)
        counts = []
        for f in range(T):
            lo, hi = self._get_window_bounds(f, W, T)
            win = set(range(lo, hi + 1))
            cells = ["  X" if (k in self._global_set and k in win) else "  G" if k in self._global_set
                     else "  W" if k in win else "  ." for k in range(T)]
            counts.append(len(self._global_set | win))
            print(f"{f:>3} |" + "".join(cells) + f"  | {counts[-1]}/{T}")
        print("    " + "---" * T)
        print(f"Legend: G=global, W=window, X=both  |  attended min={min(counts)} max={max(counts)} "
              f"avg={sum(counts) / len(counts):.1f}")

    def print_attention_mask_compact(self) -> None:
        print_attention_mask_compact(total_frames=self.total_num_frames, window_size=self.window_size,
                                     global_set=self._global_set, expand_window=self._expand_window)

    # ── attention ──────────────────────────────────────────────────────────

    def _geometry_matches(self, local_seq: int) -> bool:
        return self.num_patches > 0 and local_seq * self.world == self.total_num_frames * self.num_patches

    def _warn_geometry_mismatch_once(self, local_seq: int) -> None:
        if self._geometry_warned:
            return
        self._geometry_warned = True
        if self.rank == 0:
            print(f"[LVSA] WARNING geometry mismatch: runtime self-attention seq={local_seq} "
                  f"(world={self.world}) != configured T_lat*P={self.total_num_frames * self.num_patches} "
                  f"-> falling back to DENSE attention.", flush=True)

    def _dense(self, query, key, value, enc_q, enc_k, enc_v):
        """Dense attention of the video (and encoder) queries over all video
        and encoder keys, one launch: every query row is a dense "text query"
        tile of the kernel, the encoder keys its extra key range."""
        L, S = query.shape[1], key.shape[1]
        n_x = 0 if enc_k is None else enc_k.shape[1]
        qt = query if enc_q is None else torch.cat([query, enc_q], 1)
        dt = _compute_dtype(query)
        pkey = (query.device, qt.shape[1], S, n_x, query.shape[-1], dt)
        plan = self._dense_plans.get(pkey)
        if plan is None:
            plan = hip_ops.plan_build(None, n_q=0, n_k=S, n_x=n_x, n_tq=qt.shape[1], head_dim=query.shape[-1],
                                      device=query.device, dtype=dt)
            self._dense_plans[pkey] = plan
        cast = lambda x: None if x is None else x.to(dt)  # noqa: E731
        empty_q = qt.new_empty(qt.shape[0], 0, qt.shape[2], qt.shape[3], dtype=dt)
        _, o, _, _ = hip_ops.attn_fwd(empty_q, cast(key), cast(value), plan, kx=cast(enc_k), vx=cast(enc_v),
                                      qt=cast(qt))
        o = o.to(query.dtype)
        return o[:, :L], (None if enc_q is None else o[:, L:])

    def attention(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                  enc_q: Optional[torch.Tensor] = None, enc_k: Optional[torch.Tensor] = None,
                  enc_v: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """The attention of ``__call__`` on projected tensors ``[B, S, H, D]``:
        returns ``(video_out, encoder_out)``.  Video queries attend their
        global and window frames plus every encoder key; encoder queries
        attend all keys (one launch).  A sequence that is not the configured
        frame grid falls back to dense attention."""
        if self.world != 1:
            raise NotImplementedError(
                "DistributedLVSAProcessor on this build runs world == 1: the K/V of other ranks' global "
                "frames need collectives that are not part of it")
        local_seq = query.shape[1]
        if not self._geometry_matches(local_seq):
            self._warn_geometry_mismatch_once(local_seq)
            return self._dense(query, key, value, enc_q, enc_k, enc_v)
        res = lvsa_attention(query, key, value, self._metadata, k_text=enc_k, v_text=enc_v, q_text=enc_q)
        if enc_q is None:
            return res, None
        return res[0], res[1]

    # Reference-shaped pieces of the attention (lvsa_processor.py:643-913), for
    # callers that drive the steps themselves; ``attention`` fuses them.

    def _build_global_kv(self, key: torch.Tensor, value: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Global-frame K/V ``[B, G*P, Hkv, D]`` gathered by the copy kernel."""
        if self.world != 1:
            raise NotImplementedError("the global K/V of other ranks needs a collective (world == 1 only)")
        return build_global_kv(key, value, self._global_indices, self.num_patches)

    def _compute_full_attention(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
        """Dense attention of ``query`` over ``key``/``value`` (one launch)."""
        return self._dense(query, key, value, None, None, None)[0]

    def _compute_lvsa(self, query, key, value, k_global, v_global, encoder_hidden_states=None):
        """Video queries over ``k_global`` (+ any appended encoder K/V) and
        their window frames; the SDPA loop and the FlashInfer plan of the
        reference compute the same attention, so both flags run this."""
        return lvsa_sdpa(query, key, value, k_global, v_global, self._metadata)

    _compute_lvsa_sdpa = _compute_lvsa
    _compute_lvsa_flashinfer = _compute_lvsa

    def __call__(
        self,
        attn: Any,
        hidden_states: torch.Tensor,
        encoder_hidden_states: Optional[torch.Tensor] = None,
        attention_mask: Optional[torch.Tensor] = None,
        rotary_emb: Optional[Any] = None,
        image_rotary_emb: Optional[Any] = None,
        **kwargs,
    ) -> Any:
        adapter = self.adapter
        if adapter is None:
            raise RuntimeError("DistributedLVSAProcessor.__call__ needs a model adapter "
                               "(extract_qkv / apply_rotary / output_projection ...); use attention() "
                               "for projected tensors")
        if rotary_emb is None and image_rotary_emb is not None:
            rotary_emb = image_rotary_emb
        encoder_hidden_states_img = None
        if encoder_hidden_states is not None:
            encoder_hidden_states, encoder_hidden_states_img = adapter.split_encoder_for_cross_attn(
                attn, encoder_hidden_states)
        query, key, value = adapter.extract_qkv(attn, hidden_states, encoder_hidden_states)
        query_dtype = query.dtype
        enc_q = enc_k = enc_v = None
        encoder_seq_len = 0
        if encoder_hidden_states is not None:
            enc_qkv = adapter.extract_encoder_qkv(attn, encoder_hidden_states)
            if enc_qkv is not None:
                enc_q, enc_k, enc_v = enc_qkv
                encoder_seq_len = enc_q.shape[1]
        local_seq = hidden_states.shape[1]
        query, key = adapter.apply_rotary(query, key, rotary_emb, local_seq, self.rank, self.world)
        hidden_states, enc_output = self.attention(query, key, value, enc_q, enc_k, enc_v)
        cross_out = adapter.cross_attention(attn, query, encoder_hidden_states_img, self._attention_backend)
        if cross_out is not None:
            hidden_states = hidden_states + cross_out
        hidden_states = adapter.output_projection(attn, hidden_states, query_dtype)
        if enc_output is not None:
            return adapter.format_output(attn, hidden_states, enc_output, encoder_seq_len, query_dtype)
        return hidden_states
