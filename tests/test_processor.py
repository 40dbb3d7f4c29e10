"""Host-side behaviour of the stateful processor (no GPU).

Mirrors the intent of the reference's processor tests
(``tests/test_swa_processor.py`` classes TestGeometryGuard, TestProcessorInit,
TestDynamicReconfiguration, TestAttentionMask, TestFrameOwnership,
TestEdgeCases, TestMultiGPUConsistency, TestReferenceFramesPropagation and
``tests/test_sparse_attention.py::TestCrossCheck``).  Pattern state is
checked against the CPU oracle (``oracle/lvsa_mask.py``), which the golden
vectors pin; the attention itself runs on the GPU only (``test_gpu_processor``).
"""

import pytest
import torch

from longvideosparseattention_amd.processor import DistributedLVSAProcessor
from oracle import lvsa_mask as om


def _proc(T=21, P=30, W=3, n_first=3, kfi=4, rank=0, world=1, **kw):
    return DistributedLVSAProcessor(total_num_latent_frames=T, num_patches=P, window_size=W,
                                    n_first_frames=n_first, key_frame_interval=kfi, rank=rank, world=world, **kw)


def _oracle(proc, offset=None):
    return om.build_frame_mask(proc.total_num_frames, proc.num_patches, proc.window_size, proc.n_first_frames,
                               proc.key_frame_interval, rank=proc.rank, world=proc.world,
                               expand=proc._expand_window,
                               offset=proc._current_offset if offset is None else offset,
                               guards=proc._boundary_guards)


def _assert_matches_oracle(proc):
    ref = _oracle(proc)
    assert proc._global_indices == ref.global_indices
    assert proc.local_seq == ref.local_seq and proc.global_token_start == ref.gts
    assert proc._local_frames == ref.local_frames
    assert proc._window_ctx == ref.window_ctx
    assert proc._window_bounds.tolist() == [list(b) for b in ref.window_bounds]
    assert proc._fi_MB == ref.MB and proc._fi_compact_n == ref.compact_n
    assert proc._fi_global_copies == ref.global_copies and proc._fi_local_copies == ref.local_copies


class TestGeometryGuard:
    def test_exact_grid(self):
        assert _proc(T=21, P=30)._geometry_matches(21 * 30) is True

    def test_extra_tokens(self):
        assert _proc(T=21, P=30)._geometry_matches(21 * 30 + 100) is False

    def test_context_parallel_shard(self):
        p = _proc(T=20, P=30, world=2)
        assert p._geometry_matches(300) is True
        assert p._geometry_matches(600) is False

    def test_history_prefix(self):
        p = _proc(T=33, P=960)
        assert p._geometry_matches(33 * 960) and not p._geometry_matches(11040)


class TestInit:
    @pytest.mark.parametrize("cfg", [dict(), dict(T=41, W=3, n_first=3, kfi=8), dict(T=20, world=2, rank=1),
                                     dict(T=21, world=2, rank=0), dict(T=20, world=4, rank=3, kfi=5),
                                     dict(T=10, P=4, W=0, n_first=2, kfi=3), dict(expand_window=False)])
    def test_fields_match_oracle(self, cfg):
        _assert_matches_oracle(_proc(**cfg))

    def test_metadata_attributes_agree(self):
        p = _proc()
        m = p._metadata
        assert m.global_indices == p._global_indices and m.global_set == p._global_set
        assert m.local_frames == p._local_frames and m.local_seq == p.local_seq
        assert torch.equal(m.global_frame_mask, p._global_frame_mask)
        assert torch.equal(m.window_bounds, p._window_bounds)
        assert torch.equal(m.attended_indices, p._attended_indices)
        assert p.metadata is m

    def test_partial_frame_ownership(self):
        # 630 tokens on 2 ranks: frame 10 spans tokens 300..330, rank 0 owns 300..315.
        p = _proc(T=21, P=30, world=2, rank=0)
        (f10,) = [(s, e) for f, s, e in p._local_frames if f == 10]
        assert f10[1] - f10[0] == 15

    def test_index_tensor_lengths(self):
        p = _proc()
        assert len(p._global_src_idx) == len(p._global_dst_idx) == len(p._global_indices) * p.num_patches
        assert len(p._local_src_idx) == len(p._local_dst_idx)

    def test_global_frame_mask_and_bounds(self):
        p = _proc()
        assert p._global_frame_mask.dtype == torch.int8 and p._global_frame_mask.shape == (21,)
        assert [f for f in range(21) if p._global_frame_mask[f]] == p._global_indices
        assert p._window_bounds.dtype == torch.int32 and p._window_bounds.shape == (21, 2)
        lo, hi = p._window_bounds[:, 0], p._window_bounds[:, 1]
        assert bool(((0 <= lo) & (lo <= hi) & (hi < 21)).all())

    def test_indivisible_world(self):
        with pytest.raises(AssertionError, match="must be divisible by"):
            _proc(T=21, P=30, world=4)

    def test_logs_on_rank0_only(self, capsys):
        _proc()
        assert "[LVSA] total_lat_frames=21" in capsys.readouterr().out
        _proc(T=20, world=2, rank=1)
        assert capsys.readouterr().out == ""


class TestDynamicReconfiguration:
    def test_set_step_rotates_and_matches_oracle(self):
        p = _proc(T=21, kfi=4)
        seen = set()
        for step in range(6):
            p.set_step(step)
            assert p._current_offset == step % 4
            _assert_matches_oracle(p)
            seen.update(p._global_indices)
        # One rotation cycle makes every frame a global once.
        assert seen == set(range(21))

    def test_same_offset_keeps_metadata(self):
        p = _proc(kfi=4)
        p.set_step(1)
        m = p._metadata
        p.set_step(5)
        assert p._metadata is m

    def test_rotation_cycle_reuses_patterns(self):
        """A second cycle through the kfi offsets reuses the first cycle's metadata
        (and with it the device mask and plans); each offset still matches the oracle."""
        p = _proc(T=21, kfi=4)
        first = {}
        for step in range(4):
            p.set_step(step)
            first[step % 4] = p._metadata
        assert len({id(m) for m in first.values()}) == 4
        for step in range(4, 12):
            p.set_step(step)
            assert p._metadata is first[step % 4]
            _assert_matches_oracle(p)
        p.set_window_size(2)
        assert all(p._metadata is not m for m in first.values())
        _assert_matches_oracle(p)

    def test_no_kfi_is_noop(self):
        p = _proc(kfi=None)
        m = p._metadata
        p.set_step(5)
        assert p._metadata is m and p._current_offset == 0

    def test_window_zero_then_restore(self):
        p = _proc(T=41, P=30, W=3, n_first=3, kfi=8)
        p.set_window_size(0)
        assert p.window_size == 0 and all(parts == [] for parts in p._window_ctx.values())
        assert p.key_frame_interval == om.compute_auto_kfi(41, 0, 3)
        _assert_matches_oracle(p)
        p.set_window_size(3)
        assert any(p._window_ctx.values())
        assert p.key_frame_interval == om.compute_auto_kfi(41, 3, 3)
        _assert_matches_oracle(p)

    def test_same_window_is_noop(self):
        p = _proc(W=3)
        m = p._metadata
        p.set_window_size(3)
        assert p._metadata is m and p.key_frame_interval == 4

    def test_rebuild_keeps_offset(self):
        p = _proc(T=41, W=3, n_first=1, kfi=8)
        p.set_step(3)
        p.set_window_size(2)
        assert p._current_offset == 3
        _assert_matches_oracle(p)

    def test_sparsity_scale(self):
        p = _proc(T=81, W=3, n_first=1, kfi=None)
        p.set_sparsity_scale(0.5)
        assert p.key_frame_interval == om.compute_auto_kfi(81, 3, 1, sparsity_scale=0.5)
        _assert_matches_oracle(p)
        m = p._metadata
        p.set_sparsity_scale(0.5)
        assert p._metadata is m

    def test_pattern_cache_keeps_two_parameter_sets(self, monkeypatch):
        """Patterns of at most the current and the previous (window, kfi,
        sparsity) set stay cached; switching back to the previous set reuses
        its metadata, older sets are dropped.  (The process-wide cache of
        LVSAMetadata.build is off here, so a dropped set is built anew.)"""
        monkeypatch.setenv("LVSA_METADATA_CACHE", "0")
        p = _proc(T=81, W=3, n_first=1, kfi=None)
        for scale in (0.5, 0.7, 0.9, 1.3, 0.5):
            p.set_sparsity_scale(scale)
            assert len(p._pattern_cache) <= 2
        m = p._metadata
        p.set_window_size(0)
        p.set_window_size(3)
        assert p._metadata is m
        p.set_sparsity_scale(2.0)
        p.set_sparsity_scale(0.25)
        p.set_sparsity_scale(0.5)
        assert p._metadata is not m
        _assert_matches_oracle(p)

    def test_window_change_shrinks_compact_set(self):
        p = _proc(W=3)
        before = p._fi_compact_n
        p.set_window_size(0)
        assert p._fi_compact_n <= before


class TestReferenceFrames:
    """``reference_frames`` reaches every kfi re-derivation."""

    def _make(self, T, ref, W=3, n_first=1):
        kfi = om.compute_auto_kfi(T, W, n_first, reference_frames=ref)
        return _proc(T=T, P=30, W=W, n_first=n_first, kfi=kfi, reference_frames=ref)

    @pytest.mark.parametrize("T,ref", [(33, 33), (17, 33), (21, 21)])
    def test_up_to_reference_all_global(self, T, ref):
        p = self._make(T, ref)
        assert p.key_frame_interval == 1 and len(p._global_set) == T

    def test_globals_only_keeps_full_coverage(self):
        p = self._make(33, 33)
        p.set_window_size(0)
        assert len(p._global_set) == 33

    def test_sparsity_scale_honours_reference(self):
        p = self._make(33, 33)
        p.set_sparsity_scale(0.99)
        assert p.key_frame_interval == om.compute_auto_kfi(33, 3, 1, reference_frames=33, sparsity_scale=0.99)
        assert len(p._global_set) > p.n_first_frames

    def test_above_reference_is_sparse(self):
        assert len(self._make(65, 33)._global_set) < 65


class TestMultiRank:
    def test_ranks_cover_sequence(self):
        toks = set()
        for r in range(4):
            p = _proc(T=20, P=30, world=4, rank=r)
            for _, s, e in p._local_frames:
                toks.update(range(s + p.global_token_start, e + p.global_token_start))
        assert toks == set(range(600))

    def test_ranks_agree_on_globals_through_rotation(self):
        ps = [_proc(T=20, P=30, world=2, rank=r) for r in range(2)]
        assert ps[0]._boundary_guards == ps[1]._boundary_guards
        for step in range(4):
            for p in ps:
                p.set_step(step)
            assert ps[0]._global_set == ps[1]._global_set

    def test_attention_needs_one_rank(self):
        p = _proc(T=20, P=30, world=2)
        q = torch.zeros(1, 300, 1, 64, dtype=torch.bfloat16)
        with pytest.raises(NotImplementedError, match="world == 1"):
            p.attention(q, q, q)


class TestEdgeCases:
    def test_single_frame(self):
        p = _proc(T=1, W=0, n_first=1, kfi=None)
        assert p._global_indices == [0] and len(p._local_frames) == 1

    def test_window_wider_than_video(self):
        p = _proc(T=5, W=10, n_first=1, kfi=None)
        assert all(p._get_window_bounds(f, 10, 5) == (0, 4) for f in range(5))

    def test_all_global(self):
        assert len(_proc(T=10, W=0, n_first=1, kfi=1)._global_indices) == 10

    def test_expanded_bounds(self):
        p = _proc(T=41, W=3, n_first=3, kfi=8)
        target = min(7, 41 - len(p._global_indices))
        for f in range(41):
            lo, hi = p._expanded_window_bounds(f, 3, 41)
            assert 0 <= lo <= f <= hi < 41
            assert sum(w not in p._global_set for w in range(lo, hi + 1)) >= target

    def test_static_delegators(self):
        P = DistributedLVSAProcessor
        assert P._compute_global_indices(21, 1, 5, 2) == om.compute_global_indices(21, 1, 5, 2)
        assert P._compute_auto_kfi(81, 3, 1) == om.compute_auto_kfi(81, 3, 1)
        assert P._adaptive_window_bounds(0, 3, 21) == om.adaptive_window_bounds(0, 3, 21)
        assert P._compute_boundary_guard_frames(20, 300, 30, 2, 3) == om.compute_boundary_guard_frames(
            20, 300, 30, 2, 3)


class TestPrinting:
    def test_full_mask(self, capsys):
        p = _proc(T=10, P=4, W=2, n_first=2, kfi=3)
        p.print_attention_mask()
        out = capsys.readouterr().out
        assert "Q\\K" in out and "Legend" in out
        rows = [ln for ln in out.splitlines() if "|" in ln and ln.strip()[0].isdigit()]
        assert len(rows) == 10
        # Frame 0 row: the oracle's attended set, as G / W / X cells.
        lo, hi = om.get_window_bounds(0, 2, 10, True, set(p._global_indices), len(p._global_indices))
        cells = rows[0].split("|")[1]
        marked = {k for k in range(10) if cells[3 * k:3 * k + 3].strip() in "GWX" and cells[3 * k:3 * k + 3].strip()}
        assert marked == set(p._global_indices) | set(range(lo, hi + 1))

    def test_compact_mask(self, capsys):
        _proc(T=10, P=4, W=2, n_first=2, kfi=3).print_attention_mask_compact()
        assert "G=global" in capsys.readouterr().out


class TestCallContract:
    def test_call_without_adapter(self):
        p = _proc()
        with pytest.raises(RuntimeError, match="adapter"):
            p(None, torch.zeros(1, 630, 64))

    def test_no_cpu_attention(self):
        p = _proc(T=4, P=16, W=1, n_first=1, kfi=2)
        q = torch.zeros(1, 64, 2, 64, dtype=torch.bfloat16)
        with pytest.raises(RuntimeError):
            p.attention(q, q, q)
