"""Module aliases that bind the reference's imports to this package.

The reference imports FlashInfer by name and gates its FlashInfer backends on
that import (``lvsa/lvsa_processor.py:30-34``,
``lvsa-vllm-omni/lvsa_vllm_omni/flashinfer_runner.py:21-26``,
``attention_impl.py:454-468``); its SDPA backends import
``lvsa.sparse_attention`` and ``lvsa_vllm_omni.global_kv``.  ``install()``
registers modules under those names in ``sys.modules`` before the reference
is imported, so every backend of the reference runs the HIP kernels:

* ``flashinfer``: ``BlockSparseAttentionWrapper`` and
  ``single_prefill_with_kv_cache`` of :mod:`.block_sparse` (the subset of
  FlashInfer's API the reference calls);
* ``lvsa_vllm_omni.flashinfer_runner``: ``FLASHINFER_AVAILABLE = True``,
  ``FlashInferDualStreamRunner`` (the one-launch
  :class:`~.block_sparse.HipDualStreamRunner`) and ``get_shared_runner``;
* ``lvsa.sparse_attention`` and ``lvsa_vllm_omni.global_kv``: this package's
  :mod:`.sparse_attention` and :mod:`.global_kv`.

Nothing here is imported by the package itself.
"""

from __future__ import annotations

import sys
import types
from typing import Dict, Iterable, Optional

from . import block_sparse, global_kv, sparse_attention

__all__ = ["flashinfer_module", "flashinfer_runner_module", "modules", "install"]


def flashinfer_module() -> types.ModuleType:
    """A module named ``flashinfer`` with the two entry points the reference uses."""
    m = types.ModuleType("flashinfer", "LVSA HIP kernels under FlashInfer's names (gfx950)")
    m.BlockSparseAttentionWrapper = block_sparse.BlockSparseAttentionWrapper
    m.single_prefill_with_kv_cache = block_sparse.single_prefill_with_kv_cache
    m.__version__ = "lvsa-amd"
    return m


def flashinfer_runner_module() -> types.ModuleType:
    """``lvsa_vllm_omni.flashinfer_runner`` with the HIP runner behind its names."""
    m = types.ModuleType("lvsa_vllm_omni.flashinfer_runner", "HIP dual-stream runner (one launch, no LSE merge)")
    m.FLASHINFER_AVAILABLE = True
    m.FlashInferDualStreamRunner = block_sparse.HipDualStreamRunner
    m.get_shared_runner = block_sparse.get_shared_runner
    return m


def modules() -> Dict[str, types.ModuleType]:
    """Every alias :func:`install` registers, by module name."""
    return {
        "flashinfer": flashinfer_module(),
        "lvsa.sparse_attention": sparse_attention,
        "lvsa_vllm_omni.global_kv": global_kv,
        "lvsa_vllm_omni.flashinfer_runner": flashinfer_runner_module(),
    }


def install(names: Optional[Iterable[str]] = None, *, replace: bool = False) -> Dict[str, types.ModuleType]:
    """Register the aliases (all of them, or ``names``) in ``sys.modules``.

    Call it before importing the reference.  A module already imported under
    one of these names is left alone unless ``replace`` is set (a real
    FlashInfer in the process, or a reference module already bound).
    Returns the modules registered by this call."""
    table = modules()
    chosen = table if names is None else {n: table[n] for n in names}
    done = {}
    for name, mod in chosen.items():
        if name in sys.modules and not replace:
            continue
        sys.modules[name] = mod
        done[name] = mod
    return done
