"""Block-sparse attention wrapper and dual-stream runner (HIP).

Replaces the two FlashInfer entry points LVSA uses
(``lvsa/lvsa_processor.py:768-913``,
``lvsa-vllm-omni/lvsa_vllm_omni/flashinfer_runner.py``):

* :class:`BlockSparseAttentionWrapper` — ``plan(indptr, indices, M, N, R, C,
  num_qo_heads, num_kv_heads, head_dim, ...)`` / ``run(q, k, v,
  return_lse=...)`` over an ``R x C`` block CSR, computed by the gfx950
  block-sparse kernel.  As in FlashInfer, ``lse`` is returned in base 2.
* :func:`single_prefill_with_kv_cache` — dense (non-causal) attention with
  optional base-2 LSE, used for the text/und term.
* :class:`HipDualStreamRunner` — the ``FlashInferDualStreamRunner.run``
  contract: sparse generated-token attention plus the dense text/und term.
  Here both are one fused launch (text keys are always-attended extra rows),
  so the log-sum-exp merge of the reference is not needed.
"""

from __future__ import annotations

import math
from typing import Any, Optional

import torch

from . import hip_ops
from .sparse_attention import LVSAMetadata, lvsa_sdpa

_LN2 = math.log(2.0)


def _torch_dtype(x: Any) -> Optional[torch.dtype]:
    """FlashInfer's ``q_data_type`` (a torch dtype or its name) as a torch dtype."""
    if isinstance(x, torch.dtype) or x is None:
        return x
    return getattr(torch, str(x).replace("torch.", ""), None)


class BlockSparseAttentionWrapper:
    """HIP block-sparse attention over a block CSR (FlashInfer-compatible subset).

    ``float_workspace_buffer`` is accepted for signature compatibility; the
    plan lives on the device, and the only scratch (for split text tiles) is
    taken per call from torch's caching allocator.
    """

    def __init__(self, float_workspace_buffer: Optional[torch.Tensor] = None, backend: str = "auto"):
        self._workspace = float_workspace_buffer
        self._plan: Optional[hip_ops.BlockPlan] = None
        self._bitmap: Optional[torch.Tensor] = None
        self._shape = None
        self._scale: Optional[float] = None

    def plan(self, indptr: torch.Tensor, indices: torch.Tensor, M: int, N: int, R: int, C: int,
             num_qo_heads: int, num_kv_heads: int, head_dim: int, mask: Optional[torch.Tensor] = None,
             packed_mask: Optional[torch.Tensor] = None, causal: bool = False,
             pos_encoding_mode: str = "NONE", use_fp16_qk_reduction: bool = False,
             logits_soft_cap: Optional[float] = None, sm_scale: Optional[float] = None,
             rope_scale: Optional[float] = None, rope_theta: Optional[float] = None,
             q_data_type: Any = "float16", kv_data_type: Any = None, o_data_type: Any = None,
             non_blocking: bool = True) -> None:
        """Plan block-sparse attention: query block ``i`` (rows ``[iR, (i+1)R)``)
        attends key blocks ``indices[indptr[i]:indptr[i+1]]`` (rows
        ``[jC, (j+1)C)``)."""
        if mask is not None or packed_mask is not None or causal:
            raise NotImplementedError("custom masks and causal masking are not part of the LVSA path")
        if pos_encoding_mode not in ("NONE", None) or logits_soft_cap:
            raise NotImplementedError("positional encoding / soft cap are not part of the LVSA path")
        if num_qo_heads % num_kv_heads:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        if M % R or N % C:
            raise ValueError(f"M={M} / N={N} must be multiples of the block sizes R={R} / C={C}")
        if indptr.numel() - 1 != M // R:
            raise ValueError(f"indptr has {indptr.numel() - 1} rows, M/R = {M // R} query blocks")
        device = indptr.device if indptr.device.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
        indptr = indptr.to(device)
        indices = indices.to(device)
        n_blocks_k = N // C
        self._bitmap, status = hip_ops.csr_to_bitmap(indptr, indices, n_blocks_k)
        self._plans = {}
        self._plan_args = dict(n_q=M, n_k=N, R=R, Cf=C, max_row_frames=max(1, n_blocks_k), device=device)
        self._plan = self._plan_for(head_dim, _torch_dtype(q_data_type))
        self._shape = (M, N, num_qo_heads, num_kv_heads, head_dim)
        self._scale = sm_scale
        self._status = status
        self._status_checked = False

    def _plan_for(self, head_dim: int, dtype: Optional[torch.dtype]) -> hip_ops.BlockPlan:
        # one block plan per tile height: fp32 runs 128-row tiles
        block_q = hip_ops.attn_block_q(head_dim, dtype, self._plan_args["R"], self._plan_args["Cf"],
                                       n_k=self._plan_args["n_k"])
        plan = self._plans.get(block_q)
        if plan is None:
            plan = hip_ops.plan_build(self._bitmap, block_q=block_q, **self._plan_args)
            self._plans[block_q] = plan
        return plan

    def _check_columns(self) -> None:
        # status[0] of csr_to_bitmap flags column ids outside [0, N/C): such a
        # CSR names blocks that do not exist.  Read once per plan, outside
        # stream capture (the plan is reused by every run()).
        if self._status_checked or torch.cuda.is_current_stream_capturing():
            return
        if int(self._status[0].item()):
            raise ValueError("indices hold column ids outside [0, N/C)")
        self._status_checked = True

    def run(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: Optional[torch.Tensor] = None,
            lse: Optional[torch.Tensor] = None, return_lse: bool = False):
        """``q [M, H, D]``, ``k``/``v`` ``[N, H_kv, D]`` → ``o [M, H, D]`` (and base-2 ``lse [M, H]``)."""
        if self._plan is None:
            raise RuntimeError("plan() must be called before run()")
        M, N, H, Hkv, D = self._shape
        if q.shape != (M, H, D) or k.shape != (N, Hkv, D) or v.shape != (N, Hkv, D):
            raise ValueError(f"run() shapes {tuple(q.shape)}, {tuple(k.shape)} do not match the plan {self._shape}")
        self._check_columns()
        self._plan = self._plan_for(D, q.dtype)
        o, _, lse_n, _ = hip_ops.attn_fwd(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), self._plan,
                                          scale=self._scale, return_lse=return_lse)
        o = o[0]
        if out is not None:
            out.copy_(o)
            o = out
        if not return_lse:
            return o
        lse2 = (lse_n[0].transpose(0, 1) / _LN2).contiguous()
        if lse is not None:
            lse.copy_(lse2)
            lse2 = lse
        return o, lse2


    def run_batched(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """``run`` over a batch in one launch: ``q [B, M, H, D]``, ``k``/``v``
        ``[B, N, H_kv, D]`` → ``o [B, M, H, D]``.  Every batch element uses the
        planned block pattern (the kernel's batch index is a grid dimension)."""
        if self._plan is None:
            raise RuntimeError("plan() must be called before run()")
        M, N, H, Hkv, D = self._shape
        B = q.shape[0]
        if q.shape != (B, M, H, D) or k.shape != (B, N, Hkv, D) or v.shape != (B, N, Hkv, D):
            raise ValueError(f"run_batched() shapes {tuple(q.shape)}, {tuple(k.shape)} do not match the plan "
                             f"{self._shape} with a leading batch")
        self._check_columns()
        self._plan = self._plan_for(D, q.dtype)
        o, _, _, _ = hip_ops.attn_fwd(q, k, v, self._plan, scale=self._scale)
        return o


_DENSE_PLANS = {}


def single_prefill_with_kv_cache(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                                 sm_scale: Optional[float] = None, return_lse: bool = False, **unused):
    """Dense attention ``q [L, H, D]`` over ``k``/``v`` ``[S, H_kv, D]`` (base-2 LSE ``[L, H]``)."""
    if causal:
        raise NotImplementedError("causal prefill is not part of the LVSA path")
    hip_ops._require_device(q, "q")
    key = (q.device, q.shape[0], k.shape[0], hip_ops.attn_block_q(q.shape[-1], q.dtype, video_rows=False))
    plan = _DENSE_PLANS.get(key)
    if plan is None:
        plan = hip_ops.plan_build(None, n_q=0, n_k=k.shape[0], n_tq=q.shape[0], head_dim=q.shape[-1],
                                  device=q.device, dtype=q.dtype)
        _DENSE_PLANS[key] = plan
    # Dense rows are the kernel's "text query" tiles: every key block, no mask.
    qt = q.unsqueeze(0)
    empty_q = q.new_empty(1, 0, q.shape[1], q.shape[2])
    _, o, _, lse_t = hip_ops.attn_fwd(empty_q, k.unsqueeze(0), v.unsqueeze(0), plan, qt=qt, scale=sm_scale,
                                      return_lse=return_lse)
    o = o[0]
    if not return_lse:
        return o
    return o, (lse_t[0].transpose(0, 1) / _LN2).contiguous()


class HipDualStreamRunner:
    """Sparse generated-token attention + dense und/text keys, one launch.

    Same contract as ``FlashInferDualStreamRunner.run``
    (``flashinfer_runner.py:96-198``): ``k_global``/``v_global`` are the
    global-frame K/V (``build_global_kv``) with the und/text K/V appended;
    GQA is native (``H_kv`` divides ``H``).
    """

    def run(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, k_global: torch.Tensor,
            v_global: torch.Tensor, metadata: LVSAMetadata) -> torch.Tensor:
        return lvsa_sdpa(query, key, value, k_global, v_global, metadata)


_SHARED_RUNNER: Optional[HipDualStreamRunner] = None


def get_shared_runner() -> HipDualStreamRunner:
    """Process-wide runner shared by all attention layers (``flashinfer_runner.py:39-55``)."""
    global _SHARED_RUNNER
    if _SHARED_RUNNER is None:
        _SHARED_RUNNER = HipDualStreamRunner()
    return _SHARED_RUNNER
