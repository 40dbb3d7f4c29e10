"""``torch.ops.lvsa_amd.step_attention`` on the GPU inside ``torch.compile``.

One compiled graph (``fullgraph=True``) serves every denoising step: the step
index is a CPU tensor, so changing it neither breaks the graph nor
recompiles. Each step's outputs must equal, bit for bit, the eager
``lvsa_attention`` with that step's keyframe offset ``step % kfi``
(``lvsa/lvsa_processor.py:317-331``). That entry point is itself checked
against the fp32 oracle in ``test_gpu_attention.py``; one step here is also
checked against the oracle directly.
"""
import pytest
import torch

import longvideosparseattention_amd as lv
from longvideosparseattention_amd import step_op  # noqa: F401  (registers the operator)
from oracle import attention as oa
from oracle import lvsa_mask as om

pytestmark = pytest.mark.gpu

T, H = 10, 4
W, N_FIRST, KFI = 2, 1, 4


def _draw(shapes, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=g).to(torch.bfloat16) for s in shapes]


# 128-token frames: the ping-pong kernel; 400-token frames: the single-stream
# kernels (256-row tiles: D = 128 with 8 waves, D = 64 with the dual map)
@pytest.mark.parametrize("P", [128, 400])
@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("n_txt", [48, 0])
def test_compiled_steps_match_eager(n_txt, D, P):
    dev = torch.device("cuda", 0)
    N = T * P
    q, k, v, qt, kt, vt = (x.to(dev) for x in _draw(
        [(1, N, H, D)] * 3 + [(1, n_txt, H, D)] * 3, seed=5 + n_txt))
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    def attn(q, k, v, kt, vt, qt, step):
        return torch.ops.lvsa_amd.step_attention(q, k, v, kt, vt, qt, step, T, P, W, N_FIRST, KFI, True, None)

    f = torch.compile(attn, backend=backend, fullgraph=True)
    for step in range(6):
        o, ot = f(q, k, v, kt, vt, qt, torch.tensor(step))
        meta = lv.LVSAMetadata.build(total_latent_frames=T, num_patches=P, window_size=W, n_first_frames=N_FIRST,
                                     key_frame_interval=KFI, rank=0, world=1, keyframe_offset=step % KFI)
        if n_txt:
            ro, rot = lv.lvsa_attention(q, k, v, meta, k_text=kt, v_text=vt, q_text=qt)
            assert torch.equal(ot, rot), step
        else:
            ro = lv.lvsa_attention(q, k, v, meta)
            assert ot.shape == (1, 0, H, D)
        assert torch.equal(o, ro), step
    assert len(graphs) == 1

    # the last step against the fp32 oracle (video rows of two frames)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, N_FIRST, KFI, offset=5 % KFI).rows]
    ref, _ = oa.per_frame_sdpa(q.cpu().float(), k.cpu().float(), v.cpu().float(), rows, P,
                               k_extra=kt.cpu().float() if n_txt else None,
                               v_extra=vt.cpu().float() if n_txt else None, frames=[0, T - 1])
    got = o.float().cpu()
    for f in (0, T - 1):
        err = (got[:, f * P:(f + 1) * P] - ref[:, f * P:(f + 1) * P]).abs()
        assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, f


def test_step_must_be_cpu_scalar():
    dev = torch.device("cuda", 0)
    D, P = 128, 128
    q = torch.zeros(1, T * P, H, D, dtype=torch.bfloat16, device=dev)
    z = torch.zeros(1, 0, H, D, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="CPU"):
        torch.ops.lvsa_amd.step_attention(q, q, q, z, z, z, torch.tensor(1, device=dev), T, P, W, N_FIRST, KFI,
                                          True, None)
