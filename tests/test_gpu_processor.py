"""GPU parity of the stateful processor against the fp32 oracle.

The processor's ``__call__`` runs a toy adapter whose projections are
reshapes (``[B, S, H*D]`` <-> ``[B, S, H, D]``), so its output is the
attention itself and is compared with ``oracle/attention.py`` on the same
bf16 inputs.  Tolerance as for the kernel: max |err| <= 2e-2, mean |err| <= 2e-3.
The CSR the processor exposes (built on the GPU by the mask kernel) is
checked against ``oracle/lvsa_mask.py`` exactly, following the reference's
``tests/test_swa_processor.py::TestBuildFlashinferCSR``.
"""

import pytest
import torch

from longvideosparseattention_amd.processor import DistributedLVSAProcessor
from oracle import attention as oa
from oracle import lvsa_mask as om

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _close(got, ref, what):
    err = (got.float() - ref.to(got.device)).abs()
    mx, mn = err.max().item(), err.mean().item()
    assert mx <= MAX_ABS and mn <= MEAN_ABS, f"{what}: max {mx:.3e} mean {mn:.3e}"


def _draw(shapes, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g, dtype=torch.float32).to(torch.bfloat16) for s in shapes]


class ReshapeAdapter:
    """Adapter of the reference's ModelAdapter contract (``lvsa/adapters/base.py``)
    with identity projections; records the calls it sees."""

    def __init__(self, H, D, encoder_queries=True):
        self.H, self.D, self.encoder_queries = H, D, encoder_queries
        self.calls = []

    def _heads(self, x):
        return x.unflatten(-1, (self.H, self.D))

    def split_encoder_for_cross_attn(self, attn, enc):
        self.calls.append("split")
        return enc, None

    def extract_qkv(self, attn, hidden, enc):
        self.calls.append("qkv")
        q, k, v = hidden.chunk(3, dim=-1)
        return self._heads(q), self._heads(k), self._heads(v)

    def extract_encoder_qkv(self, attn, enc):
        self.calls.append("enc_qkv")
        if not self.encoder_queries:
            return None
        q, k, v = enc.chunk(3, dim=-1)
        return self._heads(q), self._heads(k), self._heads(v)

    def apply_rotary(self, q, k, rotary_emb, local_seq, rank, world):
        self.calls.append(("rotary", local_seq, rank, world))
        return q, k

    def cross_attention(self, attn, q, enc_img, backend):
        self.calls.append("cross")
        return None

    def output_projection(self, attn, hidden, dtype):
        self.calls.append("out")
        return hidden.flatten(-2).to(dtype)

    def format_output(self, attn, hidden, enc_out, enc_len, dtype):
        self.calls.append(("format", enc_len))
        return hidden, enc_out.flatten(-2).to(dtype)


def _proc(T, P, W, n, kfi, adapter=None):
    return DistributedLVSAProcessor(total_num_latent_frames=T, num_patches=P, window_size=W, n_first_frames=n,
                                    key_frame_interval=kfi, rank=0, world=1, adapter=adapter)


def _rows(proc):
    m = om.build_frame_mask(proc.total_num_frames, proc.num_patches, proc.window_size, proc.n_first_frames,
                            proc.key_frame_interval, offset=proc._current_offset, guards=proc._boundary_guards)
    return [set(r) for r in m.rows]


# 96-token frames run the ping-pong / 4-wave kernels, 320-token frames the
# single-stream kernels (D = 64, 96, 128)
@pytest.mark.parametrize("P", [96, 320])
@pytest.mark.parametrize("D", [64, 96, 128, 192])
@pytest.mark.parametrize("n_txt", [0, 24], ids=["video", "dual_stream"])
def test_call_matches_oracle_across_steps(n_txt, D, P, gpu):
    T, W, n, kfi, H = 13, 1, 1, 4, 2
    ad = ReshapeAdapter(H, D)
    proc = _proc(T, P, W, n, kfi, ad)
    hid, enc = _draw([(1, T * P, 3 * H * D), (1, n_txt, 3 * H * D)])
    for step in (0, 1, 6):
        proc.set_step(step)
        res = proc(None, hid.to(gpu), enc.to(gpu) if n_txt else None)
        q, k, v = (t.unflatten(-1, (H, D)).float() for t in hid.chunk(3, -1))
        if n_txt:
            qt, kt, vt = (t.unflatten(-1, (H, D)).float() for t in enc.chunk(3, -1))
            out, out_t = res
            ro, _ = oa.per_frame_sdpa(q, k, v, _rows(proc), P, k_extra=kt, v_extra=vt)
            rt, _ = oa.text_row_attention(qt, k, v, kt, vt)
            _close(out_t.unflatten(-1, (H, D)), rt, f"encoder rows, step {step}")
            assert ("format", n_txt) in ad.calls
        else:
            out = res
            ro, _ = oa.per_frame_sdpa(q, k, v, _rows(proc), P)
        assert out.shape == (1, T * P, H * D) and out.dtype == torch.bfloat16
        _close(out.unflatten(-1, (H, D)), ro, f"video rows, step {step}")
    assert ("rotary", T * P, 0, 1) in ad.calls


def test_encoder_keys_without_encoder_queries(gpu):
    """An adapter that returns no encoder q/k/v: plain video attention."""
    T, P, H, D = 8, 64, 2, 64
    proc = _proc(T, P, 1, 1, 3, ReshapeAdapter(H, D, encoder_queries=False))
    hid, enc = _draw([(1, T * P, 3 * H * D), (1, 9, 3 * H * D)])
    out = proc(None, hid.to(gpu), enc.to(gpu))
    q, k, v = (t.unflatten(-1, (H, D)).float() for t in hid.chunk(3, -1))
    ro, _ = oa.per_frame_sdpa(q, k, v, _rows(proc), P)
    _close(out.unflatten(-1, (H, D)), ro, "video rows")


def test_geometry_mismatch_falls_back_to_dense(gpu, capsys):
    T, P, H, D, extra, n_txt = 6, 64, 2, 128, 40, 17
    ad = ReshapeAdapter(H, D)
    proc = _proc(T, P, 1, 1, 3, ad)
    L = T * P + extra
    hid, enc = _draw([(1, L, 3 * H * D), (1, n_txt, 3 * H * D)], seed=3)
    out, out_t = proc(None, hid.to(gpu), enc.to(gpu))
    assert "geometry mismatch" in capsys.readouterr().out
    q, k, v = (t.unflatten(-1, (H, D)).float() for t in hid.chunk(3, -1))
    qt, kt, vt = (t.unflatten(-1, (H, D)).float() for t in enc.chunk(3, -1))
    kk, vv = torch.cat([k, kt], 1), torch.cat([v, vt], 1)
    ro, _ = oa.dense_attention(q, kk, vv)
    rt, _ = oa.dense_attention(qt, kk, vv)
    _close(out.unflatten(-1, (H, D)), ro, "dense video rows")
    _close(out_t.unflatten(-1, (H, D)), rt, "dense encoder rows")
    proc(None, hid.to(gpu), enc.to(gpu))
    assert "geometry mismatch" not in capsys.readouterr().out      # warned once


def test_reference_shaped_steps_agree_with_fused(gpu):
    """_build_global_kv + _compute_lvsa (both backend flags) vs the fused attention."""
    T, P, W, H, Hkv, D, n_txt = 11, 80, 2, 4, 2, 128, 30
    proc = _proc(T, P, W, 1, 4)
    q, k, v, kt, vt = (x.to(gpu) for x in _draw([(1, T * P, H, D), (1, T * P, Hkv, D), (1, T * P, Hkv, D),
                                                  (1, n_txt, Hkv, D), (1, n_txt, Hkv, D)], seed=5))
    fused, _ = proc.attention(q, k, v, enc_k=kt, enc_v=vt)
    kg, vg = proc._build_global_kv(k, v)
    assert kg.shape[1] == len(proc._global_indices) * P
    kg, vg = torch.cat([kg, kt], 1), torch.cat([vg, vt], 1)
    for flag in (False, True):
        proc._use_flashinfer = flag
        out = proc._compute_lvsa(q, k, v, kg, vg, None)
        _close(out, fused.float(), f"_compute_lvsa flashinfer={flag}")
    ro, _ = oa.per_frame_sdpa(q.float(), k.float(), v.float(), _rows(proc), P, k_extra=kt.float(),
                              v_extra=vt.float())
    _close(fused, ro, "fused")
    dense = proc._compute_full_attention(q[:, :100], k, v)
    rd, _ = oa.dense_attention(q[:, :100].float(), k.float(), v.float())
    _close(dense, rd, "_compute_full_attention")


@pytest.mark.parametrize("cfg", [dict(T=21, P=30, W=3, n=3, kfi=4), dict(T=10, P=4, W=0, n=2, kfi=3),
                                 dict(T=21, P=30, W=3, n=3, kfi=4, world=2, rank=1),
                                 dict(T=20, P=30, W=3, n=3, kfi=4, world=4, rank=2),
                                 dict(T=1, P=4, W=0, n=1, kfi=None), dict(T=8, P=4, W=0, n=1, kfi=1)],
                         ids=["wan_like", "globals_only", "rank1_of_2", "rank2_of_4", "one_frame", "all_global"])
def test_processor_csr_matches_oracle(cfg, gpu):
    world, rank = cfg.get("world", 1), cfg.get("rank", 0)
    proc = DistributedLVSAProcessor(total_num_latent_frames=cfg["T"], num_patches=cfg["P"],
                                    window_size=cfg["W"], n_first_frames=cfg["n"], key_frame_interval=cfg["kfi"],
                                    rank=rank, world=world)
    for step in (0, 1):
        proc.set_step(step)
        ref = om.build_frame_mask(cfg["T"], cfg["P"], cfg["W"], cfg["n"], proc.key_frame_interval, rank=rank,
                                  world=world, offset=proc._current_offset, guards=proc._boundary_guards)
        assert proc._fi_indptr.tolist() == ref.indptr
        assert proc._fi_indices.tolist() == ref.indices
        assert len(proc._fi_indptr) == proc._fi_MB + 1
        nG = len(proc._global_indices)
        for qi in range(proc._fi_MB):
            a, b = proc._fi_indptr[qi].item(), proc._fi_indptr[qi + 1].item()
            row = proc._fi_indices[a:b].tolist()
            assert row == sorted(row) and b - a >= nG
            assert all(0 <= c < proc._fi_compact_n for c in row)
        if cfg["W"] == 0:
            assert proc._fi_compact_n == nG


def test_retune_derives_kfi_on_the_device(gpu, monkeypatch):
    """set_window_size / set_sparsity_scale take kfi from lvsa_auto_kfi, not
    from the host formula (lvsa/lvsa_processor.py:288-360)."""
    import longvideosparseattention_amd.processor as proc_mod

    def _host_formula(*a, **k):
        raise AssertionError("host compute_auto_kfi called")

    p = DistributedLVSAProcessor(40, 16, 2, 2, 4, 0, 1, reference_frames=21)
    monkeypatch.setattr(proc_mod, "compute_auto_kfi", _host_formula)
    p.set_sparsity_scale(0.6)
    assert p.key_frame_interval == om.compute_auto_kfi(40, 2, 2, reference_frames=21, sparsity_scale=0.6)
    p.set_window_size(0)
    assert p.key_frame_interval == om.compute_auto_kfi(40, 0, 2, reference_frames=21, sparsity_scale=0.6)
    ref = om.build_frame_mask(40, 16, 0, 2, p.key_frame_interval, offset=0)
    assert p._global_indices == ref.global_indices
