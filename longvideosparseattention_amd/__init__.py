"""LVSA (Long-Video Sparse Attention) hot path, MI355X-native.

Drop-in replacement for the attention path of ``lvsa`` (JiusiServe/
LongVideoSparseAttention v1.2.0): the same public names as
``lvsa.sparse_attention`` (and the plugin's ``build_global_kv`` /
FlashInfer runner), computed by hand-written gfx950 HIP kernels behind the C
ABI of ``include/lvsa_amd.h``.

Exports are lazy (like ``lvsa/__init__.py``) so that importing the package
needs neither the HIP library nor a GPU.
"""

__version__ = "0.1.0"

_SPARSE = (
    "sparse_windowed_attention", "LVSAMetadata", "lvsa_sdpa", "lvsa_flashinfer", "lvsa_attention",
    "adaptive_window_bounds", "expanded_window_bounds", "get_window_bounds",
    "compute_boundary_guard_frames", "compute_auto_kfi", "compute_global_indices",
    "print_attention_mask_compact",
)
_BLOCK = ("BlockSparseAttentionWrapper", "single_prefill_with_kv_cache", "HipDualStreamRunner",
          "get_shared_runner")


def __getattr__(name):
    if name in _SPARSE:
        from . import sparse_attention as m
    elif name in _BLOCK:
        from . import block_sparse as m
    elif name == "build_global_kv":
        from . import global_kv as m
    elif name == "DistributedLVSAProcessor":
        from . import processor as m
    elif name == "step_attention":
        from . import step_op as m
    else:
        raise AttributeError(f"module 'longvideosparseattention_amd' has no attribute {name!r}")
    value = getattr(m, name)
    globals()[name] = value
    return value


__all__ = list(_SPARSE) + list(_BLOCK) + ["build_global_kv", "DistributedLVSAProcessor", "step_attention"]
