"""fp32 reference attention for the LVSA hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module; the product never does.

Two independent formulations of the same mathematics (softmax attention
restricted to the LVSA frame mask, scale 1/sqrt(D), GQA by head grouping):

* ``masked_sdpa``       — explicit boolean token mask, one softmax over all
                          keys (small shapes: the mask is dense);
* ``per_frame_sdpa``    — restates ``lvsa_sdpa`` (``lvsa/sparse_attention.py:643-706``):
                          for every query frame, gather the always-attended
                          extra rows (``k_global`` / text) and the key frames
                          of its relation row, then dense fp32 attention.

Both run in fp32 on whatever device their inputs live on (CPU here, the GPU
on the box for the large BASELINE shapes) and return ``(out, lse)`` with the
natural-log log-sum-exp.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Set, Tuple

import torch


def _expand_kv(k: torch.Tensor, H: int) -> torch.Tensor:
    Hkv = k.shape[2]
    if Hkv == H:
        return k
    return k.repeat_interleave(H // Hkv, dim=2)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    mask: Optional[torch.Tensor] = None, scale: Optional[float] = None
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax attention in fp32.  q [B,Sq,H,D], k/v [B,Sk,Hkv,D], mask [Sq,Sk] bool.

    Written out (matmul, max-shifted exp, normalise) rather than through a
    library kernel so the LSE comes for free and nothing is fused.
    """
    B, Sq, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    qf = q.float().permute(0, 2, 1, 3).contiguous()                 # [B,H,Sq,D]
    kf = _expand_kv(k.float(), H).permute(0, 2, 3, 1).contiguous()  # [B,H,D,Sk]
    vf = _expand_kv(v.float(), H).permute(0, 2, 1, 3).contiguous()  # [B,H,Sk,D]
    s = torch.matmul(qf, kf) * scale                                # [B,H,Sq,Sk]
    if mask is not None:
        s = s.masked_fill(~mask.to(s.device)[None, None], float("-inf"))
    m = s.amax(dim=-1, keepdim=True)
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    p = torch.exp(s - m)
    l = p.sum(dim=-1, keepdim=True)
    o = torch.matmul(p, vf) / l
    lse = (m + torch.log(l)).squeeze(-1)                            # [B,H,Sq]
    return o.permute(0, 2, 1, 3).contiguous(), lse


def masked_sdpa(q, k, v, mask, scale=None):
    """Explicit-mask formulation (small shapes)."""
    return dense_attention(q, k, v, mask, scale)


def per_frame_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   rows: Sequence[Set[int]], P: int,
                   k_extra: Optional[torch.Tensor] = None, v_extra: Optional[torch.Tensor] = None,
                   scale: Optional[float] = None, frames: Optional[Sequence[int]] = None,
                   ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-query-frame gather + dense fp32 attention (the ``lvsa_sdpa`` loop).

    ``rows[f]`` is the set of key frames of ``k``/``v`` that query frame ``f``
    attends; ``k_extra``/``v_extra`` rows are attended by every query.  With
    ``frames`` given, only those query frames are computed (the other output
    rows stay NaN) — used for spot checks at the large shapes.
    """
    B, S, H, D = q.shape
    out = torch.full((B, S, H, D), float("nan"), dtype=torch.float32, device=q.device)
    lse = torch.full((B, H, S), float("nan"), dtype=torch.float32, device=q.device)
    n_frames = -(-S // P)
    for f in (range(n_frames) if frames is None else frames):
        qs, qe = f * P, min((f + 1) * P, S)
        parts_k, parts_v = [], []
        if k_extra is not None and k_extra.shape[1] > 0:
            parts_k.append(k_extra)
            parts_v.append(v_extra)
        for g in sorted(rows[f]):
            ks, ke = g * P, min((g + 1) * P, k.shape[1])
            if ks < ke:
                parts_k.append(k[:, ks:ke])
                parts_v.append(v[:, ks:ke])
        kc = torch.cat(parts_k, dim=1)
        vc = torch.cat(parts_v, dim=1)
        o, l = dense_attention(q[:, qs:qe], kc, vc, None, scale)
        out[:, qs:qe] = o
        lse[:, :, qs:qe] = l
    return out, lse


def text_row_attention(q_text, k, v, k_text, v_text, scale=None):
    """Dense text-query rows over ``cat(video K, text K)`` (lvsa/lvsa_processor.py:710-735)."""
    return dense_attention(q_text, torch.cat([k, k_text], 1), torch.cat([v, v_text], 1), None, scale)
