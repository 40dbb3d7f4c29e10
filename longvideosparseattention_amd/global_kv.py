"""Global-frame K/V extraction (``lvsa-vllm-omni/lvsa_vllm_omni/global_kv.py``).

``build_global_kv`` packs the K/V rows of the global frames with the HIP
frame-gather kernel.  The fused ``lvsa_attention`` path does not need it (it
addresses global frames in place); it is kept for callers of the reference
API that pass ``k_global``/``v_global`` to ``lvsa_sdpa``.
"""

from __future__ import annotations

from typing import List, Tuple

import torch

from . import hip_ops

_FRAME_LISTS = {}


def _frames_on(device: torch.device, frames: List[int]) -> torch.Tensor:
    key = (str(device), tuple(frames))
    t = _FRAME_LISTS.get(key)
    if t is None:
        t = torch.tensor(frames, dtype=torch.int32).to(device)
        if len(_FRAME_LISTS) > 256:
            _FRAME_LISTS.clear()
        _FRAME_LISTS[key] = t
    return t


def build_global_kv(
    key: torch.Tensor,
    value: torch.Tensor,
    global_indices: List[int],
    num_patches: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """K/V tokens of the global frames: ``[B, len(global_indices)·P, H, D]`` each.

    ``key``/``value`` are ``[B, seq_len, H, D]`` GPU tensors.
    """
    B, _, H, D = key.shape
    if not global_indices:
        return key.new_empty(B, 0, H, D), value.new_empty(B, 0, H, D)
    frames = _frames_on(key.device, list(global_indices))
    return (hip_ops.gather_frames(key, frames, num_patches),
            hip_ops.gather_frames(value, frames, num_patches))
