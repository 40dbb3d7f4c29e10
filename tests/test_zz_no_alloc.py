"""lvsa_attn_fwd_noalloc (static device scratch, no allocation) against
lvsa_attn_fwd with a caller workspace, through the C ABI.

Both run the same kernels, the same text-tile split and, at head size 64, the
same split of the queues' last video tiles, so the outputs must match bit for
bit.  Two calls in a row, the second on a smaller input, show
that the shared scratch left by the first call does not leak into the second.
"""

import ctypes as C

import pytest
import torch

import longvideosparseattention_amd as lv
from longvideosparseattention_amd import _capi, hip_ops
from oracle import attention as oa


def _inputs(T, P, H, D, n_txt, seed):
    g = torch.Generator().manual_seed(seed)
    N = T * P
    shapes = [(1, N, H, D)] * 3 + [(1, n_txt, H, D)] * 3
    return [torch.randn(*s, generator=g).to(torch.bfloat16) for s in shapes]


def _noalloc(gpu, m, q, k, v, qt, kt, vt):
    N, n_txt, D = q.shape[1], qt.shape[1], q.shape[3]
    plan = m.full_plan(gpu, N, N, n_txt, n_txt, D)
    call = hip_ops.attn_args(q, k, v, plan, kx=kt, vx=vt, qt=qt, return_lse=True)
    need = C.c_int64(0)
    _capi.check("lvsa_attn_workspace_query",
                _capi.lib().lvsa_attn_workspace_query(C.byref(call.args), C.byref(need)))
    assert 0 < need.value <= _capi.NOALLOC_SCRATCH_BYTES   # the split (and so the scratch) is in use
    stream = torch.cuda.current_stream(gpu).cuda_stream
    _capi.check("lvsa_attn_fwd_noalloc", _capi.lib().lvsa_attn_fwd_noalloc(C.byref(call.args), stream))
    return call.out, call.out_t, call.lse, call.lse_t


@pytest.mark.gpu
@pytest.mark.parametrize("D", [128, 64, 96, 192, 256])
def test_noalloc_matches_workspace_entry_point(D, gpu):
    # second call: smaller input.  Head size 64 takes 8 heads in the first
    # call: enough tiles for its two work-groups per CU to run the work queues
    # and the video split, whose partials fit the static scratch too.
    shapes = [(16, 1500, 8 if D == 64 else 3, 300), (8, 1100, 2, 100)]
    for i, (T, P, H, n_txt) in enumerate(shapes):
        q, k, v, qt, kt, vt = (x.to(gpu) for x in _inputs(T, P, H, D, n_txt, seed=11 + i))
        m = lv.LVSAMetadata.build(total_latent_frames=T, num_patches=P, window_size=1, n_first_frames=1,
                                  key_frame_interval=4, rank=0, world=1, keyframe_offset=i)
        got = _noalloc(gpu, m, q, k, v, qt, kt, vt)
        want = lv.lvsa_attention(q, k, v, m, k_text=kt, v_text=vt, q_text=qt, return_lse=True)
        torch.cuda.synchronize()
        for a, b, name in zip(got, want, ("out", "out_text", "lse", "lse_text")):
            assert torch.equal(a, b), f"call {i} ({T}x{P}, {n_txt} text): {name} differs"
        rto, _ = oa.text_row_attention(qt.float().cpu(), k.float().cpu(), v.float().cpu(), kt.float().cpu(),
                                       vt.float().cpu())
        err = (got[1].float().cpu() - rto).abs()
        assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3


def test_noalloc_rejects_scratch_overflow():
    """A split that needs more than the static scratch is refused before any
    device work (host check only)."""
    a = _capi.AttnArgs()
    a.D, a.dtype, a.B, a.H, a.Hkv, a.block_q = 128, 0, 4, 64, 64, 256
    a.n_q, a.n_k, a.n_tq = 0, 400000, 4096
    rc = _capi.lib().lvsa_attn_fwd_noalloc(C.byref(a), None)
    assert rc == -3
    assert b"static" in _capi.lib().lvsa_last_error()
