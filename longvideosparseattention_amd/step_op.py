"""The per-step LVSA attention as one PyTorch custom operator.

``torch.ops.lvsa_amd.step_attention`` runs the attention of a denoising step
from scalars: the frame geometry and the step index.  Inside the operator:

* the keyframe offset is ``step % key_frame_interval``
  (``lvsa/lvsa_processor.py:317-331``);
* the pattern state comes from a cache keyed by the geometry and the offset:
  host fields, the device CSR from ``lvsa_mask_build`` and the block plan
  from ``lvsa_plan_build``;
* the attention is one ``lvsa_attn_fwd`` launch (``lvsa_attention``): video
  rows over their global and window frames plus every text key, text rows
  over everything.

The reference runs this path under ``torch.compiler.disable``
(``lvsa-vllm-omni/lvsa_vllm_omni/attention_impl.py:298, 352``;
``lvsa/sparse_attention.py:336``). Its metadata build is data-dependent
Python, so it breaks the graph, and with the step baked in as a constant it
recompiles every step. As a custom operator with a shape-only fake
implementation, the attention stays inside a ``torch.compile`` graph. The
step travels as a one-element CPU tensor, so its value is data, not a guard,
and successive steps reuse one compiled graph.
"""
from functools import lru_cache
from typing import Optional, Tuple

import torch

from . import sparse_attention as _sa

__all__ = ["step_attention"]


@lru_cache(maxsize=64)
def _metadata(T: int, P: int, W: int, n_first: int, kfi: int, offset: int, expand: bool) -> _sa.LVSAMetadata:
    """Pattern state of one (geometry, offset); its device mask and plans are cached inside."""
    return _sa.LVSAMetadata.build(
        total_latent_frames=T, num_patches=P, window_size=W, n_first_frames=n_first,
        key_frame_interval=kfi if kfi > 0 else None, rank=0, world=1,
        expand_window=expand, keyframe_offset=offset)


def _text_out_shape(query: torch.Tensor, q_text: torch.Tensor):
    return (query.shape[0], q_text.shape[1], query.shape[2], query.shape[3])


@torch.library.custom_op("lvsa_amd::step_attention", mutates_args=(), device_types="cuda")
def step_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   k_text: torch.Tensor, v_text: torch.Tensor, q_text: torch.Tensor, step: torch.Tensor,
                   total_latent_frames: int, num_patches: int, window_size: int, n_first_frames: int,
                   key_frame_interval: int, expand_window: bool = True,
                   scale: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """LVSA attention of one denoising step: returns ``(out, out_text)``.

    ``query``/``key``/``value`` are ``[B, T*P, H(kv), D]`` video tokens; the
    ``*_text`` tensors are ``[B, n, H(kv), D]`` text tokens, ``n`` possibly
    0; ``step`` is a one-element CPU integer tensor; ``key_frame_interval``
    <= 0 means no keyframe grid.  ``out_text`` is ``[B, n_text_queries, H,
    D]``.
    """
    if step.device.type != "cpu" or step.numel() != 1:
        raise ValueError("step must be a one-element CPU tensor (the denoising step index)")
    kfi = int(key_frame_interval)
    offset = int(step.item()) % kfi if kfi > 0 else 0
    meta = _metadata(int(total_latent_frames), int(num_patches), int(window_size), int(n_first_frames),
                     kfi, offset, bool(expand_window))
    n_tk, n_tq = k_text.shape[1], q_text.shape[1]
    res = _sa.lvsa_attention(
        query, key, value, meta,
        k_text=k_text if n_tk else None, v_text=v_text if n_tk else None,
        q_text=q_text if n_tq else None, scale=scale)
    if n_tq:
        return res[0], res[1]
    return res, query.new_empty(_text_out_shape(query, q_text))


@step_attention.register_fake
def _step_attention_fake(query, key, value, k_text, v_text, q_text, step, total_latent_frames, num_patches,
                         window_size, n_first_frames, key_frame_interval, expand_window=True, scale=None):
    if query.shape[1] != total_latent_frames * num_patches:
        raise ValueError(f"query has {query.shape[1]} tokens, geometry gives {total_latent_frames * num_patches}")
    return query.new_empty(query.shape), query.new_empty(_text_out_shape(query, q_text))
