"""HIP-graph capture of one denoising step's device work.

A serving loop captures the mask build, the plan build and the fused
attention forward (``lvsa_mask_build``, ``lvsa_plan_build``,
``lvsa_attn_fwd``) once per keyframe offset and replays the graph every step
(``lvsa/lvsa_processor.py:317-331`` rebuilds the pattern whenever the offset
changes).  None of the three allocates, synchronises or records a memset, so
the captured graph holds exactly their kernel launches.

Every replay is checked bit for bit against the same three calls run
eagerly on the same inputs (the kernels are deterministic), and against the
public fused entry point ``lvsa_attention``.  Between replays the test writes
new inputs into the captured buffers and runs its own eager work, with host
synchronisation.
"""
import pytest
import torch

import longvideosparseattention_amd as lv
from longvideosparseattention_amd import hip_ops

pytestmark = pytest.mark.gpu

T, H, NT = 12, 4, 64
W, N_FIRST, KFI = 2, 1, 4


def _step(meta, q, k, v, qt, kt, vt):
    """Mask, plan and attention for one offset: the device work of a step."""
    D, P = q.shape[-1], meta.num_patches
    dm = hip_ops.mask_build(meta._mask_params(), q.device)
    plan = hip_ops.plan_build(dm.rel_full, n_q=q.shape[1], n_k=k.shape[1], n_x=kt.shape[1], n_tq=qt.shape[1],
                              R=P, Cf=P, max_row_frames=max(1, meta.max_row_frames),
                              block_q=hip_ops.attn_block_q(D, q.dtype, P, P))
    o, ot, lse, lse_t = hip_ops.attn_fwd(q, k, v, plan, kx=kt, vx=vt, qt=qt, return_lse=True)
    return dict(frame_indptr=dm.frame_indptr, frame_indices=dm.frame_indices,
                tile_indptr=plan.tile_indptr, entries=plan.entries, o=o, ot=ot, lse=lse, lse_t=lse_t)


def _assert_same(a, b, what):
    """Bitwise equality; CSR payloads compared over their used prefix only."""
    assert torch.equal(a["frame_indptr"], b["frame_indptr"]), what
    nf = int(a["frame_indptr"][-1])
    assert torch.equal(a["frame_indices"][:nf], b["frame_indices"][:nf]), what
    assert torch.equal(a["tile_indptr"], b["tile_indptr"]), what
    ne = int(a["tile_indptr"][-1])
    assert ne > 0, what
    assert torch.equal(a["entries"][:ne], b["entries"][:ne]), what
    for key in ("o", "ot", "lse", "lse_t"):
        assert torch.equal(a[key], b[key]), (what, key)


# 128-token frames run the ping-pong / 4-wave kernels; 400-token frames the
# single-stream kernels (D = 128 and 96 on 256-row tiles with 8 waves, D = 64
# on 256-row tiles with the dual map's 4 waves of 64 rows), whose work-queue
# counters are zeroed by a kernel in the captured graph.
@pytest.mark.parametrize("D,offset,P", [(128, 0, 128), (128, 3, 128), (64, 1, 128), (96, 2, 128), (192, 3, 128),
                                        (256, 0, 128), (128, 1, 400), (96, 3, 400), (64, 2, 400)])
def test_step_graph_replays_match_eager(D, offset, P):
    dev = torch.device("cuda", 0)
    meta = lv.LVSAMetadata.build(total_latent_frames=T, num_patches=P, window_size=W, n_first_frames=N_FIRST,
                                 key_frame_interval=KFI, rank=0, world=1, keyframe_offset=offset)
    g = torch.Generator().manual_seed(11 + offset + D)
    N = T * P
    shapes = {"q": (1, N, H, D), "k": (1, N, H, D), "v": (1, N, H, D),
              "qt": (1, NT, H, D), "kt": (1, NT, H, D), "vt": (1, NT, H, D)}
    x = {n: torch.randn(s, generator=g).to(torch.bfloat16).to(dev) for n, s in shapes.items()}
    args = lambda: (meta, x["q"], x["k"], x["v"], x["qt"], x["kt"], x["vt"])  # noqa: E731

    # warm-up on a side stream before capture (allocator pools, lazy library load)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _step(*args())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = _step(*args())

    for rep in range(4):
        # new inputs in the captured buffers, plus unrelated eager work
        for n, s in shapes.items():
            x[n].copy_(torch.randn(s, generator=g).to(torch.bfloat16))
        scratch = (x["q"].float() * 2).sum()
        graph.replay()
        torch.cuda.synchronize()
        eager = _step(*args())
        torch.cuda.synchronize()
        _assert_same(static, eager, f"replay {rep}")
        o, ot = lv.lvsa_attention(x["q"], x["k"], x["v"], meta, k_text=x["kt"], v_text=x["vt"], q_text=x["qt"])
        assert torch.equal(o, static["o"]) and torch.equal(ot, static["ot"]), f"replay {rep}: lvsa_attention"
        assert torch.isfinite(static["o"].float()).all() and torch.isfinite(scratch)
