"""Host-side API of the package (CPU only): helpers and LVSAMetadata host
fields against the golden vectors; the reference's own unit-test contracts;
error behaviour; no CPU compute path."""

import io

import pytest
import torch

import longvideosparseattention_amd as lv
from longvideosparseattention_amd import sparse_attention as sa


def _meta(a):
    return sa.LVSAMetadata.build(
        total_latent_frames=a["T"], num_patches=a["P"], window_size=a["W"], n_first_frames=a["n_first"],
        key_frame_interval=a["kfi"], rank=a["rank"], world=a["world"], expand_window=a["expand"],
        keyframe_offset=a["offset"], boundary_guards=a["guards"])


def test_helpers_match_golden(golden):
    for rec in golden["windows"]:
        G = set(rec["G"])
        assert list(sa.get_window_bounds(rec["f"], rec["W"], rec["T"], rec["expand"], G, len(G))) == rec["bounds"]
    for rec in golden["auto_kfi"]:
        assert sa.compute_auto_kfi(rec["T"], rec["W"], rec["n_first"], reference_frames=rec["ref"],
                                   sparsity_scale=rec["scale"]) == rec["kfi"]


def test_metadata_host_fields_match_golden(golden):
    for rec in golden["random"] + golden["baseline"]:
        a = rec["args"]
        m = _meta(a)
        tag = str(a)
        assert m.global_indices == rec["global_indices"], tag
        assert m.window_bounds.tolist() == rec["window_bounds"], tag
        assert (m.fi_M, m.fi_N, m.fi_MB, m.fi_compact_n) == (rec["fi_M"], rec["fi_N"], rec["fi_MB"],
                                                             rec["fi_compact_n"]), tag
        assert m.fi_nnz == rec["fi_indptr"][-1], tag
        assert (m.local_seq, m.global_token_start) == (rec["local_seq"], rec["global_token_start"]), tag
        if "local_frames" in rec:
            assert [list(x) for x in m.local_frames] == rec["local_frames"], tag
            assert {str(k): [list(p) for p in v] for k, v in m.window_ctx.items()} == rec["window_ctx"], tag
            assert m.attended_indices.tolist() == rec["attended_indices"], tag
            assert m.attended_C == rec["attended_C"], tag
            assert [list(x) for x in m.fi_global_copies] == rec["fi_global_copies"], tag
            assert [list(x) for x in m.fi_local_copies] == rec["fi_local_copies"], tag
            assert m.global_frame_mask.tolist() == rec["global_frame_mask"], tag


# Contracts of tests/test_sparse_attention.py:22-133 (host fields only).
class TestLVSAMetadataBuild:
    def _build(self, T=21, P=30, W=3, n_first=1, kfi=4, rank=0, world=1, expand=True):
        return lv.LVSAMetadata.build(total_latent_frames=T, num_patches=P, window_size=W, n_first_frames=n_first,
                                     key_frame_interval=kfi, rank=rank, world=world, expand_window=expand)

    def test_basic_build(self):
        m = self._build()
        assert (m.total_latent_frames, m.num_patches, m.local_seq, m.global_token_start) == (21, 30, 630, 0)

    def test_local_frames_cover_local_seq(self):
        m = self._build()
        assert sum(e - s for _, s, e in m.local_frames) == m.local_seq

    def test_window_ctx_excludes_globals(self):
        m = self._build()
        for f, parts in m.window_ctx.items():
            for s, e in parts:
                for t in range(s, e, m.num_patches):
                    assert (m.global_token_start + t) // m.num_patches not in m.global_set

    def test_tables(self):
        m = self._build()
        assert m.global_frame_mask.shape == (21,) and m.window_bounds.shape == (21, 2)
        assert m.attended_indices.shape == (len(m.local_frames), m.attended_C)
        assert len(m.fi_global_copies) + len(m.fi_local_copies) == m.fi_compact_n
        assert m.global_src_idx.numel() == len(m.global_indices) * 30
        assert torch.equal(m.global_dst_idx[:30], torch.arange(30))

    def test_multi_gpu_rank1(self):
        m = self._build(rank=1, world=2)
        assert m.global_token_start == m.local_seq == 21 * 30 // 2

    def test_indivisible_world_asserts(self):
        with pytest.raises(AssertionError, match="must be divisible by world"):
            self._build(T=5, P=3, world=2)

    def test_boundary_guards_and_rotation(self):
        m = lv.LVSAMetadata.build(total_latent_frames=21, num_patches=30, window_size=3, n_first_frames=1,
                                  key_frame_interval=4, rank=0, world=1, boundary_guards=[5, 10, 15])
        assert {5, 10, 15} <= m.global_set
        m0 = self._build()
        m1 = lv.LVSAMetadata.build(total_latent_frames=21, num_patches=30, window_size=3, n_first_frames=1,
                                   key_frame_interval=4, rank=0, world=1, keyframe_offset=1)
        assert m0.global_indices != m1.global_indices
        assert len(m0.global_indices) == len(m1.global_indices)

    def test_kfi_used_verbatim(self):
        # tests/test_sparse_attention.py:590-611
        m = lv.LVSAMetadata.build(total_latent_frames=33, num_patches=30, window_size=3, n_first_frames=1,
                                  key_frame_interval=1, rank=0, world=1, reference_frames=33)
        assert m.key_frame_interval == 1 and len(m.global_set) == 33

    def test_ensure_device_cpu_is_noop(self):
        m = self._build()
        m.ensure_device(torch.device("cpu"))


def test_flashinfer_backend_requires_buffers():
    # tests/test_sparse_attention.py:284-292
    m = lv.LVSAMetadata.build(total_latent_frames=5, num_patches=4, window_size=1, n_first_frames=1,
                              key_frame_interval=None, rank=0, world=1)
    q = k = v = kg = vg = torch.randn(1, 20, 2, 8)
    with pytest.raises(AssertionError, match="FlashInfer backend requires"):
        lv.sparse_windowed_attention(q, k, v, kg, vg, m, backend="flashinfer")


def test_no_cpu_compute_path():
    m = lv.LVSAMetadata.build(total_latent_frames=5, num_patches=4, window_size=1, n_first_frames=1,
                              key_frame_interval=None, rank=0, world=1)
    q = torch.randn(1, 20, 2, 64)
    with pytest.raises(RuntimeError, match="no CPU path"):
        lv.lvsa_sdpa(q, q, q, q[:, :4], q[:, :4], m)
    with pytest.raises(RuntimeError, match="no CPU path"):
        lv.lvsa_attention(q, q, q, m)


def test_print_mask_compact():
    buf = io.StringIO()
    sa.print_attention_mask_compact(10, 2, {0, 3, 6, 9}, True, file=buf)
    lines = buf.getvalue().splitlines()
    assert len(lines) == 12 and "G=global" in lines[-1]
    assert lines[1].startswith("0 |") and lines[1].endswith(f"| {len(lines[1].split('|')[1]) - lines[1].split('|')[1].count('.')}")


def test_lazy_exports():
    for name in lv.__all__:
        assert getattr(lv, name) is not None
    with pytest.raises(AttributeError):
        lv.does_not_exist


def test_head_sizes_of_the_plugin():
    """The reference plugin's head sizes (backend.py:52-53) all map onto a kernel:
    every size runs natively; 96 on 256-row tiles, 192 on 256-row tiles
    where the dual-wide map takes the geometry and 128-row ones otherwise,
    256 on 128-row tiles."""
    from longvideosparseattention_amd import hip_ops

    assert hip_ops.SUPPORTED_HEAD_DIMS == (64, 96, 128, 192, 256)
    assert [hip_ops.kernel_head_dim(d) for d in (64, 96, 128, 192, 256)] == [64, 96, 128, 192, 256]
    assert hip_ops.attn_block_q(256) == 128 and hip_ops.attn_block_q(192) == 128   # no geometry: 128
    assert hip_ops.attn_block_q(96) == 256
    # head size 64: 256-row tiles (the dual map); fp32: 128
    assert hip_ops.attn_block_q(64, torch.bfloat16, 1350, 1350) == 256
    assert hip_ops.attn_block_q(64, torch.float16, 383, 64) == 256
    assert hip_ops.attn_block_q(64, torch.float32, 1350, 1350) == 128
    assert hip_ops.attn_block_q(128, torch.bfloat16, 1560, 1560) == 256
    with pytest.raises(ValueError, match="head_dim 80"):
        hip_ops.kernel_head_dim(80)


def test_block_q_head_192(monkeypatch):
    """Head size 192 in 16-bit: 256-row tiles (the dual-wide map) for query
    frames >= 255 rows, key frames >= 64 and a short last key block inside
    one frame; 128-row tiles (the wide map or the 4-wave kernel) otherwise,
    for fp32, and with LVSA_ATTN_BLOCK_Q=128 or LVSA_ATTN_KERNEL=pp."""
    from longvideosparseattention_amd import hip_ops

    monkeypatch.delenv("LVSA_ATTN_BLOCK_Q", raising=False)
    monkeypatch.delenv("LVSA_ATTN_KERNEL", raising=False)
    assert hip_ops.attn_block_q(192, torch.bfloat16, 1560, 1560) == 256
    assert hip_ops.attn_block_q(192, torch.float16, 255, 64) == 256
    assert hip_ops.attn_block_q(192, torch.bfloat16, 254, 1560) == 128
    assert hip_ops.attn_block_q(192, torch.bfloat16, 1560, 63) == 128
    assert hip_ops.attn_block_q(192, torch.float32, 1560, 1560) == 128
    assert hip_ops.attn_block_q(192, torch.bfloat16, 385, 385, n_k=440, k_tok0=0) == 128
    assert hip_ops.attn_block_q(192, torch.bfloat16, 385, 385, n_k=440, k_tok0=440) == 256
    assert hip_ops.attn_block_q(256, torch.bfloat16, 1560, 1560) == 128
    # no video query rows (dense calls): no frame condition
    assert hip_ops.attn_block_q(192, torch.bfloat16, video_rows=False) == 256
    assert hip_ops.attn_block_q(192, torch.float32, video_rows=False) == 128
    assert hip_ops.attn_block_q(256, torch.bfloat16, video_rows=False) == 128
    monkeypatch.setenv("LVSA_ATTN_BLOCK_Q", "128")
    assert hip_ops.attn_block_q(192, torch.bfloat16, 1560, 1560) == 128
    monkeypatch.delenv("LVSA_ATTN_BLOCK_Q")
    monkeypatch.setenv("LVSA_ATTN_KERNEL", "pp")
    assert hip_ops.attn_block_q(192, torch.bfloat16, 1560, 1560) == 128
    assert hip_ops.attn_block_q(192, torch.bfloat16, video_rows=False) == 128


def test_dual_wide_ok_mirrors_the_entry_point(monkeypatch):
    """hip_ops.dual_wide_ok (the call-time test that sends a 256-row plan at
    head size 192 to its 128-row fallback) accepts what the C entry point
    accepts: frames, the last key block, source sizes below 2^31 bytes."""
    from longvideosparseattention_amd import _capi as capi
    from longvideosparseattention_amd import hip_ops

    monkeypatch.delenv("LVSA_ATTN_KERNEL", raising=False)

    def plan(n_q, n_k, R, C, k_tok0=0):
        p = capi.PlanParams(n_q=n_q, n_k=n_k, R=R, C=C, k_tok0=k_tok0, block_q=256, block_k=64)
        return hip_ops.BlockPlan(tile_indptr=None, entries=None, status=None, n_tiles=0, n_video_tiles=0,
                                 params=p, rel=None)

    def src(rows, row_elems):
        return torch.empty_strided((1, rows, 1, 192), (0, row_elems, 192, 1), dtype=torch.bfloat16, device="meta")

    k = src(4680, 192)
    assert hip_ops.dual_wide_ok(plan(4680, 4680, 1560, 1560), k, k, None, None)
    assert not hip_ops.dual_wide_ok(plan(4680, 4680, 254, 1560), k, k, None, None)
    assert not hip_ops.dual_wide_ok(plan(4680, 4680, 1560, 63), k, k, None, None)
    assert not hip_ops.dual_wide_ok(plan(1000, 440, 385, 385), k, k, None, None)        # tail crosses a frame
    assert hip_ops.dual_wide_ok(plan(0, 440, 0, 0), k, k, None, None)                   # text rows only
    big = (1 << 31) // (192 * 2)
    assert not hip_ops.dual_wide_ok(plan(4680, big, 1560, 1560), src(big - 63, 192), k, None, None)
    assert hip_ops.dual_wide_ok(plan(4680, big, 1560, 1560), src(big - 65, 192), k, None, None)
    monkeypatch.setenv("LVSA_ATTN_KERNEL", "pp")
    assert not hip_ops.dual_wide_ok(plan(4680, 4680, 1560, 1560), k, k, None, None)


def test_block_q_override_384(monkeypatch):
    """LVSA_ATTN_BLOCK_Q=384 selects the 12-wave kernel's 384-row tiles for
    head size 64 where the geometry allows them (query frames >= 383 rows, key
    frames >= 64, the key source's short last block inside one frame) and
    256-row tiles elsewhere."""
    from longvideosparseattention_amd import hip_ops

    monkeypatch.setenv("LVSA_ATTN_BLOCK_Q", "384")
    assert hip_ops.attn_block_q(64, torch.bfloat16, 1350, 1350) == 384
    assert hip_ops.attn_block_q(64, torch.float16, 383, 64) == 384
    assert hip_ops.attn_block_q(64, torch.bfloat16, 382, 1350) == 256
    assert hip_ops.attn_block_q(64, torch.bfloat16, 1350, 63) == 256
    assert hip_ops.attn_block_q(128, torch.bfloat16, 1560, 1560) == 256
    assert hip_ops.attn_block_q(64, torch.float32, 1350, 1350) == 128
    # a shard whose short last key block crosses a frame boundary: 256-row tiles
    assert hip_ops.attn_block_q(64, torch.bfloat16, 385, 385, n_k=440, k_tok0=0) == 256
    assert hip_ops.attn_block_q(64, torch.bfloat16, 385, 385, n_k=440, k_tok0=440) == 384
    monkeypatch.setenv("LVSA_ATTN_BLOCK_Q", "128")
    assert hip_ops.attn_block_q(64, torch.bfloat16, 1350, 1350) == 128


def _frame_parts_of_last_block(n_k, k_tok0, C, block=64):
    """Parts of the last key block as the plan builder counts them
    (lvsa_mask.hip frame_desc): the key frames its rows fall in, plus one for
    the rows past the end of the source when the block is short."""
    k0 = block * ((n_k - 1) // block)
    frames = {(k_tok0 + k) // C for k in range(k0, n_k)}
    return len(frames) + (1 if n_k - k0 < block else 0)


def test_stream_tail_test_matches_the_plan_descriptor():
    """stream_tail_crosses_frame (mirrored by the C entry point's gate of the
    single-stream kernels) is true exactly when the plan builder would make
    the source's last key block a three-part ("generic") descriptor."""
    import random

    from longvideosparseattention_amd import hip_ops

    rng = random.Random(7)
    cases = [(312, 0, 260), (440, 0, 385), (440, 440, 385), (64, 30, 64), (1, 5, 64), (320, 0, 260)]
    cases += [(rng.randint(1, 3000), rng.randint(0, 5000), rng.randint(64, 700)) for _ in range(3000)]
    hits = 0
    for n_k, k_tok0, C in cases:
        want = _frame_parts_of_last_block(n_k, k_tok0, C) >= 3
        assert hip_ops.stream_tail_crosses_frame(1, n_k, k_tok0, C) == want, (n_k, k_tok0, C)
        hits += want
    assert hits > 20
    assert not hip_ops.stream_tail_crosses_frame(0, 312, 0, 260)   # no video queries: no frame plan


def test_query_length_must_match_metadata():
    """The kernels map query row r to local frame (start + r) // P: a query
    that is not the metadata's local sequence is rejected before any device
    work (the reference slices metadata.local_frames out of the query)."""
    m = lv.LVSAMetadata.build(total_latent_frames=5, num_patches=4, window_size=1, n_first_frames=1,
                              key_frame_interval=None, rank=0, world=1)
    q = torch.randn(1, 16, 2, 64)     # 4 frames of 4, metadata has 5
    with pytest.raises(ValueError, match="local_seq=20"):
        lv.lvsa_sdpa(q, q, q, q[:, :4], q[:, :4], m)
    with pytest.raises(ValueError, match="local_seq=20"):
        lv.lvsa_attention(q, q, q, m)


def test_wrapper_rejects_csr_with_wrong_row_count():
    w = lv.BlockSparseAttentionWrapper()
    indptr = torch.tensor([0, 1, 2], dtype=torch.int32)      # 2 rows, M/R = 3
    indices = torch.tensor([0, 1], dtype=torch.int32)
    with pytest.raises(ValueError, match="M/R = 3"):
        w.plan(indptr, indices, M=192, N=128, R=64, C=64, num_qo_heads=2, num_kv_heads=2, head_dim=128)


def test_shim_binds_the_reference_import_names():
    """shim.install(): ``import flashinfer`` and the plugin's runner module
    resolve to the HIP wrapper, prefill and runner (the names the reference
    gates its FlashInfer backends on, lvsa/lvsa_processor.py:30-34,
    flashinfer_runner.py:21-26), and the SDPA path's module names to this
    package.  Runs in a fresh interpreter so sys.modules stays clean here."""
    import subprocess
    import sys
    import textwrap
    code = textwrap.dedent("""
        import sys
        sys.modules.pop("flashinfer", None)
        from longvideosparseattention_amd import shim, block_sparse, sparse_attention, global_kv
        got = shim.install()
        assert sorted(got) == ["flashinfer", "lvsa.sparse_attention", "lvsa_vllm_omni.flashinfer_runner",
                               "lvsa_vllm_omni.global_kv"], got
        import flashinfer
        assert flashinfer.BlockSparseAttentionWrapper is block_sparse.BlockSparseAttentionWrapper
        assert flashinfer.single_prefill_with_kv_cache is block_sparse.single_prefill_with_kv_cache
        from lvsa_vllm_omni.flashinfer_runner import (FLASHINFER_AVAILABLE, FlashInferDualStreamRunner,
                                                      get_shared_runner)
        assert FLASHINFER_AVAILABLE and FlashInferDualStreamRunner is block_sparse.HipDualStreamRunner
        assert get_shared_runner() is get_shared_runner()
        from lvsa.sparse_attention import lvsa_sdpa, LVSAMetadata
        assert lvsa_sdpa is sparse_attention.lvsa_sdpa
        from lvsa_vllm_omni.global_kv import build_global_kv
        assert build_global_kv is global_kv.build_global_kv
        # a second install leaves bound names alone unless asked
        assert shim.install() == {}
        assert sorted(shim.install(["flashinfer"], replace=True)) == ["flashinfer"]
        print("ok")
    """)
    root = str(__import__("pathlib").Path(__file__).resolve().parents[1])
    res = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stderr[-2000:]


def test_build_returns_one_shared_pattern_per_argument_set(monkeypatch):
    """The plugin hooks rebuild the pattern in every layer at every step
    (attention_impl.py:387-419): repeated arguments return the instance built
    first, LRU-bounded by LVSA_METADATA_CACHE (0 turns the cache off)."""
    sa.clear_metadata_cache()
    kw = dict(total_latent_frames=9, num_patches=256, window_size=1, n_first_frames=1, key_frame_interval=4,
              rank=0, world=1)
    a = lv.LVSAMetadata.build(keyframe_offset=3, **kw)
    # reference_frames / sparsity_scale do not enter the pattern (kfi is used verbatim)
    assert lv.LVSAMetadata.build(keyframe_offset=3, reference_frames=7, sparsity_scale=2.0, **kw) is a
    b = lv.LVSAMetadata.build(keyframe_offset=2, **kw)
    assert b is not a and b.global_indices == [0, 1, 2, 6] and a.global_indices == [0, 2, 3, 7]
    assert lv.LVSAMetadata.build(keyframe_offset=3, boundary_guards=[5], **kw) is not a
    assert lv.LVSAMetadata.build(keyframe_offset=3, expand_window=False, **kw) is not a

    monkeypatch.setenv("LVSA_METADATA_CACHE", "2")
    sa.clear_metadata_cache()
    ms = [lv.LVSAMetadata.build(keyframe_offset=o, **kw) for o in range(3)]
    assert lv.LVSAMetadata.build(keyframe_offset=2, **kw) is ms[2]
    assert lv.LVSAMetadata.build(keyframe_offset=0, **kw) is not ms[0]      # evicted (LRU of 2)

    monkeypatch.setenv("LVSA_METADATA_CACHE", "0")
    x, y = (lv.LVSAMetadata.build(keyframe_offset=1, **kw) for _ in range(2))
    assert x is not y and x.global_indices == y.global_indices
    sa.clear_metadata_cache()


def test_stream12_source_limits():
    """384-row plans fall back to 256-row tiles (hip_ops.attn_args) for key
    sources the 12-wave kernel cannot address: 32-bit byte offsets per source
    and 24-bit lane offsets (row stride in bytes below 16 MiB)."""
    from longvideosparseattention_amd import hip_ops

    def src(rows, row_stride):
        return torch.empty_strided((1, rows, 1, 64), (0, row_stride, 64, 1), dtype=torch.bfloat16, device="meta")

    assert hip_ops.stream12_sources_ok(src(1000, 3072), src(1000, 3072), None, None)
    assert not hip_ops.stream12_sources_ok(src(1000, 8 << 20), src(1000, 64))        # 16 MiB row stride
    assert hip_ops.stream12_sources_ok(src(100, (8 << 20) - 8))                       # just below both limits
    big = (1 << 31) // 3072                                                          # rows of 6 KiB
    assert not hip_ops.stream12_sources_ok(src(big - 63, 3072))                      # (rows + 64) * 6 KiB >= 2^32
    assert hip_ops.stream12_sources_ok(src(big - 65, 3072))
    assert hip_ops.stream12_sources_ok(src(0, 8 << 20))                              # empty source: nothing read
