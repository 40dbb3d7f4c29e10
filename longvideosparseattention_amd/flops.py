"""Algorithmic work of one LVSA attention call (for throughput reporting).

``F_block = 4·B·H·D·[Σ_active |q_blk|·|k_blk| + N_v·N_t + N_t·(N_v+N_t)]``:
active block pairs of the canonical ``b x b`` tiling of the video sequence
(a pair is active iff any token pair in it is allowed by the frame rule;
``|·|`` counts real tokens of a tail block), text keys dense for video
queries and text queries dense over everything.  The token-exact variant
replaces the block area by the mask's token count.

The block area is read from the device block plan at ``(b, b)`` built by
``lvsa_plan_build`` (the same refinement the attention kernel runs on).
"""

from __future__ import annotations

from typing import Tuple

import torch

from . import hip_ops


def active_block_area(metadata, device: torch.device, block: int) -> int:
    """Σ over active canonical (block x block) pairs of |q_blk|·|k_blk| (video part)."""
    st = metadata.device_state(device)
    N = metadata.total_latent_frames * metadata.num_patches
    P = metadata.num_patches
    plan = hip_ops.plan_build(st.mask.rel_full, n_q=N, n_k=N, R=P, Cf=P,
                              max_row_frames=max(1, metadata.max_row_frames), block_q=block, block_k=block)
    indptr = plan.tile_indptr.long()
    counts = indptr[1:] - indptr[:-1]
    nnz = int(indptr[-1].item())
    tiles = torch.arange(plan.n_tiles, device=device)
    qsz = torch.clamp(N - tiles * block, max=block)
    cols = plan.entries[:nnz, 0].long() & 0x7FFFFFFF
    ksz = torch.clamp(N - cols * block, max=block)
    rows = torch.repeat_interleave(qsz, counts)
    return int((rows * ksz).sum().item())


def attention_flops(metadata, device: torch.device, block: int, H: int, D: int, n_text: int = 0,
                    batch: int = 1) -> Tuple[int, int]:
    """``(F_block, F_token_exact)`` of one call on the full (world=1) sequence."""
    N = metadata.total_latent_frames * metadata.num_patches
    P = metadata.num_patches
    area = active_block_area(metadata, device, block)
    exact = metadata.fi_nnz * P * P
    text = N * n_text + n_text * (N + n_text)
    k = 4 * batch * H * D
    return k * (area + text), k * (exact + text)
