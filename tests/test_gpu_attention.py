"""GPU parity of the block-sparse attention kernel through every entry point.

Reference: the fp32 oracle (``oracle/attention.py``) on the same bf16-rounded
inputs.  Tolerance (bf16 output vs fp32 reference):
max |err| <= 2e-2 and mean |err| <= 2e-3.  Inputs follow the BASELINE recipe:
one CPU generator, seed 0, fp32 randn drawn in order q, k, v, then text q,
k, v, shapes [B, N, H, D], rounded to the compute dtype.
"""

import math

import pytest
import torch

import longvideosparseattention_amd as lv
from longvideosparseattention_amd import hip_ops
from oracle import attention as oa
from oracle import lvsa_mask as om

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _draw(shapes, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g, dtype=torch.float32).to(dtype) for s in shapes]


def _close(got, ref, what, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    ref = ref.to(got.device)
    sel = torch.isfinite(ref)
    err = (got.float()[sel] - ref[sel]).abs()
    assert err.numel() > 0
    mx, mn = err.max().item(), err.mean().item()
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max {mx:.3e} mean {mn:.3e}"


def _meta(T, P, W, n, kfi, off=0, rank=0, world=1, guards=None):
    return lv.LVSAMetadata.build(total_latent_frames=T, num_patches=P, window_size=W, n_first_frames=n,
                                 key_frame_interval=kfi, rank=rank, world=world, keyframe_offset=off,
                                 boundary_guards=guards)


SMALL = [
    # T, P, W, n, kfi, off, H, Hkv, D, n_txt, dtype
    (9, 256, 1, 1, 4, 3, 2, 2, 128, 0, torch.bfloat16),
    (9, 256, 1, 1, 4, 3, 2, 2, 64, 0, torch.bfloat16),
    (10, 4, 0, 2, 3, 0, 2, 2, 128, 0, torch.bfloat16),       # W=0, tiny frames -> generic masks
    (21, 30, 3, 3, 4, 2, 4, 1, 128, 0, torch.bfloat16),      # GQA 4:1, frames < block
    (9, 200, 1, 1, 4, 1, 4, 4, 128, 37, torch.bfloat16),     # text keys + text queries
    (13, 150, 1, 1, 4, 0, 3, 3, 64, 26, torch.float16),      # fp16, D=64, text
    (24, 130, 2, 1, 8, 5, 2, 2, 128, 0, torch.bfloat16),
    (6, 8, 2, 1, 1, 0, 8, 2, 128, 16, torch.bfloat16),       # kfi=1: dense
    (5, 30, 10, 1, None, 0, 2, 2, 64, 0, torch.bfloat16),    # W > T: dense
    (1, 77, 0, 1, None, 0, 2, 2, 128, 3, torch.bfloat16),    # single frame
    (17, 129, 2, 2, 5, 4, 2, 2, 128, 129, torch.float16),    # odd sizes, text tail
    (9, 200, 1, 1, 4, 1, 4, 2, 96, 37, torch.bfloat16),      # D=96 (native, 256-row tiles), GQA, text
    (13, 150, 1, 1, 4, 0, 3, 3, 96, 26, torch.float16),      # D=96, fp16, text
    (9, 256, 1, 1, 4, 3, 2, 2, 192, 0, torch.bfloat16),      # D=192 (native, 128-row tiles)
    (13, 150, 1, 1, 4, 0, 4, 2, 192, 26, torch.float16),     # D=192, fp16, GQA, text
    (9, 200, 1, 1, 4, 1, 4, 4, 256, 37, torch.bfloat16),     # D=256, text
    (13, 150, 1, 1, 4, 0, 3, 3, 256, 26, torch.float16),     # D=256, fp16, text
]


@pytest.mark.parametrize("block_q", [128, 256], ids=["tile128", "tile256"])
@pytest.mark.parametrize("cfg", SMALL, ids=[str(c[:10]) for c in SMALL])
def test_fused_attention_small(cfg, block_q, gpu, monkeypatch):
    """Both kernels (128-row tiles: 4 waves; 256-row tiles: 8 waves in two
    alternating groups) on every small configuration."""
    monkeypatch.setenv("LVSA_ATTN_BLOCK_Q", str(block_q))
    T, P, W, n, kfi, off, H, Hkv, D, n_txt, dt = cfg
    N = T * P
    m = _meta(T, P, W, n, kfi, off)
    q, k, v, qt, kt, vt = _draw([(1, N, H, D), (1, N, Hkv, D), (1, N, Hkv, D), (1, n_txt, H, D),
                                 (1, n_txt, Hkv, D), (1, n_txt, Hkv, D)], dtype=dt)
    ref_rows = [set(r) for r in om.build_frame_mask(T, P, W, n, kfi, offset=off).rows]
    args = dict(k_text=kt.to(gpu), v_text=vt.to(gpu), q_text=qt.to(gpu)) if n_txt else {}
    res = lv.lvsa_attention(q.to(gpu), k.to(gpu), v.to(gpu), m, return_lse=True, **args)
    ro, rl = oa.per_frame_sdpa(q.float(), k.float(), v.float(), ref_rows, P,
                               k_extra=kt.float() if n_txt else None, v_extra=vt.float() if n_txt else None)
    if n_txt:
        o, ot, lse, lse_t = res
        rto, rtl = oa.text_row_attention(qt.float(), k.float(), v.float(), kt.float(), vt.float())
        _close(ot, rto, "text rows")
        torch.testing.assert_close(lse_t.cpu(), rtl, atol=2e-2, rtol=0)
    else:
        o, lse = res
    assert o.dtype == dt and o.shape == q.shape
    _close(o, ro, "video rows")
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-2, rtol=0)


def _random_cfg(seed):
    """A seeded random geometry: frame sizes on and off the 64-key blocks,
    every head size, GQA, text tokens, both dtypes and both tile heights."""
    g = torch.Generator().manual_seed(1000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]  # noqa: E731
    T = int(torch.randint(1, 17, (1,), generator=g))
    P = int(torch.randint(1, 301, (1,), generator=g))
    W = pick([0, 1, 1, 2, 2, 3, 4])
    n = pick([1, 1, 2, 3])
    kfi = pick([None, 1, 2, 3, 4, 5, 8])
    off = int(torch.randint(0, 8, (1,), generator=g)) % (kfi or 1)
    D = pick([64, 96, 128, 192, 256])
    Hkv = pick([1, 2, 3])
    H = Hkv * pick([1, 2])
    n_txt = pick([0, 0, 1, 17, 64, 100])
    dt = pick([torch.bfloat16, torch.float16])
    block_q = pick([128, 256])
    return T, P, W, n, kfi, off, H, Hkv, D, n_txt, dt, block_q


@pytest.mark.parametrize("seed", range(24))
def test_random_geometries(seed, gpu, monkeypatch):
    """Seeded random geometries through ``lvsa_attention`` against the fp32
    oracle (video rows, text rows and both LSEs)."""
    T, P, W, n, kfi, off, H, Hkv, D, n_txt, dt, block_q = _random_cfg(seed)
    monkeypatch.setenv("LVSA_ATTN_BLOCK_Q", str(block_q))
    N = T * P
    m = _meta(T, P, W, n, kfi, off)
    q, k, v, qt, kt, vt = _draw([(1, N, H, D), (1, N, Hkv, D), (1, N, Hkv, D), (1, n_txt, H, D),
                                 (1, n_txt, Hkv, D), (1, n_txt, Hkv, D)], seed=seed, dtype=dt)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, n, kfi, offset=off).rows]
    args = dict(k_text=kt.to(gpu), v_text=vt.to(gpu), q_text=qt.to(gpu)) if n_txt else {}
    res = lv.lvsa_attention(q.to(gpu), k.to(gpu), v.to(gpu), m, return_lse=True, **args)
    ro, rl = oa.per_frame_sdpa(q.float(), k.float(), v.float(), rows, P,
                               k_extra=kt.float() if n_txt else None, v_extra=vt.float() if n_txt else None)
    what = f"seed {seed}: T={T} P={P} W={W} n={n} kfi={kfi} off={off} H={H}/{Hkv} D={D} txt={n_txt} {dt} bq={block_q}"
    if n_txt:
        o, ot, lse, lse_t = res
        rto, rtl = oa.text_row_attention(qt.float(), k.float(), v.float(), kt.float(), vt.float())
        _close(ot, rto, what + " text rows")
        torch.testing.assert_close(lse_t.cpu(), rtl, atol=2e-2, rtol=0, msg=what)
    else:
        o, lse = res
    assert o.dtype == dt and o.shape == q.shape
    _close(o, ro, what)
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-2, rtol=0, msg=what)


def test_repeat_call_is_bitwise_identical(gpu):
    T, P, H, D = 12, 300, 4, 128
    m = _meta(T, P, 2, 1, 4, 1)
    q, k, v = (x.to(gpu) for x in _draw([(1, T * P, H, D)] * 3))
    a = lv.lvsa_attention(q, k, v, m)
    b = lv.lvsa_attention(q, k, v, m)
    assert torch.equal(a, b)


def test_lvsa_sdpa_with_k_global_and_text(gpu):
    # The reference call path: build_global_kv + text appended -> lvsa_sdpa.
    T, P, W, H, Hkv, D, n_txt = 11, 160, 2, 4, 2, 128, 40
    m = _meta(T, P, W, 1, 4, 2)
    q, k, v, kt, vt = (x.to(gpu) for x in _draw([(1, T * P, H, D), (1, T * P, Hkv, D), (1, T * P, Hkv, D),
                                                 (1, n_txt, Hkv, D), (1, n_txt, Hkv, D)]))
    kg, vg = lv.build_global_kv(k, v, m.global_indices, P)
    kg, vg = torch.cat([kg, kt], 1), torch.cat([vg, vt], 1)
    out = lv.lvsa_sdpa(q, k, v, kg, vg, m)
    out2 = lv.sparse_windowed_attention(q, k, v, kg, vg, m, backend="sdpa")
    assert torch.equal(out, out2)
    ref = om.build_frame_mask(T, P, W, 1, 4, offset=2)
    ro, _ = oa.per_frame_sdpa(q.float(), k.float(), v.float(), om.window_only_relation(ref), P,
                              k_extra=kg.float(), v_extra=vg.float())
    _close(out, ro, "lvsa_sdpa")
    fused = lv.lvsa_attention(q, k, v, m, k_text=kt, v_text=vt)
    _close(fused, ro, "fused vs lvsa_sdpa reference")


CP_SHARDS = [
    # T, P, W, kfi, off, H, D, world, rank
    (12, 50, 2, 5, 3, 2, 128, 2, 1),
    # P >= 255 (single-stream kernels) with the shard's short last key block
    # [256, 312) crossing the frame boundary at 260: planned "generic", so
    # these run the compiler-built kernels
    (6, 260, 1, 3, 1, 2, 128, 5, 0),
    (6, 260, 1, 3, 1, 2, 64, 5, 0),
    (6, 260, 1, 3, 1, 2, 192, 5, 0),
    # P >= 383 (where head size 64 may run 384-row tiles) with a crossing
    # last block: keys [384, 440), boundary at 385
    (8, 385, 1, 3, 2, 2, 64, 7, 0),
]


@pytest.mark.parametrize("cfg", CP_SHARDS, ids=[str(c) for c in CP_SHARDS])
def test_lvsa_sdpa_context_parallel_shard(cfg, gpu):
    # one rank: local queries/keys, globals assembled from the full sequence.
    T, P, W, kfi, off, H, D, world, rank = cfg
    guards = lv.compute_boundary_guard_frames(T, T * P // world, P, world, W)
    m = _meta(T, P, W, 1, kfi, off, rank=rank, world=world, guards=guards)
    q, k, v = _draw([(1, T * P, H, D)] * 3)
    s, e = m.global_token_start, m.global_token_start + m.local_seq
    kg = torch.cat([k[:, g * P:(g + 1) * P] for g in m.global_indices], 1)
    vg = torch.cat([v[:, g * P:(g + 1) * P] for g in m.global_indices], 1)
    out = lv.lvsa_sdpa(q[:, s:e].to(gpu), k[:, s:e].to(gpu), v[:, s:e].to(gpu), kg.to(gpu), vg.to(gpu), m)
    # Oracle: the reference loop over local frames (lvsa/sparse_attention.py:674-704).
    ref = torch.full((1, m.local_seq, H, D), float("nan"))
    for f, qs, qe in m.local_frames:
        parts_k = [kg.float()] + [k[:, s + a:s + b].float() for a, b in m.window_ctx[f]]
        parts_v = [vg.float()] + [v[:, s + a:s + b].float() for a, b in m.window_ctx[f]]
        o, _ = oa.dense_attention(q[:, s + qs:s + qe].float(), torch.cat(parts_k, 1), torch.cat(parts_v, 1))
        ref[:, qs:qe] = o
    _close(out, ref, "cp shard")


def test_flashinfer_backend_and_wrapper(gpu):
    T, P, W, H, D = 9, 96, 1, 4, 128
    m = _meta(T, P, W, 1, 4, 3)
    m.ensure_device(gpu)
    q, k, v = (x.to(gpu) for x in _draw([(1, T * P, H, D)] * 3))
    kg, vg = lv.build_global_kv(k, v, m.global_indices, P)
    ck = q.new_zeros(1, m.fi_N, H, D)
    cv = q.new_zeros(1, m.fi_N, H, D)
    for src, dst in m.fi_global_copies:
        ck[:, dst:dst + P], cv[:, dst:dst + P] = kg[:, src:src + P], vg[:, src:src + P]
    for src, dst in m.fi_local_copies:
        ck[:, dst:dst + P], cv[:, dst:dst + P] = k[:, src:src + P], v[:, src:src + P]
    w = lv.BlockSparseAttentionWrapper(torch.empty(1, dtype=torch.uint8, device=gpu))
    w.plan(m.fi_indptr, m.fi_indices, M=m.fi_M, N=m.fi_N, R=P, C=P, num_qo_heads=H, num_kv_heads=H,
           head_dim=D, q_data_type="bfloat16")
    out = lv.sparse_windowed_attention(q, k, v, kg, vg, m, backend="flashinfer", k_compact=ck, v_compact=cv,
                                       fi_wrapper=w)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, 4, offset=3).rows]
    ro, rl = oa.per_frame_sdpa(q.float(), k.float(), v.float(), rows, P)
    _close(out, ro, "flashinfer backend")
    o2, lse2 = w.run(q[0], ck[0], cv[0], return_lse=True)
    torch.testing.assert_close(lse2.cpu(), (rl[0].transpose(0, 1) / math.log(2.0)).cpu(), atol=3e-2, rtol=0)


def test_flashinfer_backend_batch_of_two(gpu):
    """B = 2 (classifier-free guidance): the backend runs the batch in one
    launch (run_batched), bit for bit what one run() per element gives, and
    matches the oracle per element."""
    T, P, W, H, Hkv, D = 9, 96, 1, 4, 2, 128
    m = _meta(T, P, W, 1, 4, 2)
    m.ensure_device(gpu)
    q = _draw([(2, T * P, H, D)], seed=11)[0].to(gpu)
    k, v = (x.to(gpu) for x in _draw([(2, T * P, Hkv, D)] * 2, seed=12))
    kg, vg = lv.build_global_kv(k, v, m.global_indices, P)
    ck = k.new_zeros(2, m.fi_N, Hkv, D)
    cv = k.new_zeros(2, m.fi_N, Hkv, D)
    for src, dst in m.fi_global_copies:
        ck[:, dst:dst + P], cv[:, dst:dst + P] = kg[:, src:src + P], vg[:, src:src + P]
    for src, dst in m.fi_local_copies:
        ck[:, dst:dst + P], cv[:, dst:dst + P] = k[:, src:src + P], v[:, src:src + P]
    w = lv.BlockSparseAttentionWrapper(torch.empty(1, dtype=torch.uint8, device=gpu))
    w.plan(m.fi_indptr, m.fi_indices, M=m.fi_M, N=m.fi_N, R=P, C=P, num_qo_heads=H, num_kv_heads=Hkv,
           head_dim=D, q_data_type="bfloat16")
    qp = q.new_zeros(2, m.fi_M, H, D)
    qp[:, :m.local_seq] = q
    out = lv.sparse_windowed_attention(qp, k, v, kg, vg, m, backend="flashinfer", k_compact=ck, v_compact=cv,
                                       fi_wrapper=w)
    assert out.shape == (2, m.local_seq, H, D)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, 4, offset=2).rows]
    for b in range(2):
        assert torch.equal(out[b], w.run(qp[b], ck[b], cv[b])[:m.local_seq])
        ro, _ = oa.per_frame_sdpa(q[b:b + 1].float(), k[b:b + 1].float(), v[b:b + 1].float(), rows, P)
        _close(out[b:b + 1], ro, f"flashinfer backend batch element {b}")


def test_dual_stream_runner_gqa(gpu):
    # lvsa-vllm-omni/tests/test_flashinfer_runner.py: H=8, Hkv=2, D=128, P=8, 16 und tokens.
    H, HKV, D, P, S_UND = 8, 2, 128, 8, 16
    for T_lat, ref_frames, kfi in [(24, 6, None), (6, 6, 1)]:
        if kfi is None:
            kfi = lv.compute_auto_kfi(T_lat, 2, 1, reference_frames=ref_frames)
        m = lv.LVSAMetadata.build(total_latent_frames=T_lat, num_patches=P, window_size=2, n_first_frames=1,
                                  key_frame_interval=kfi, rank=0, world=1, reference_frames=ref_frames)
        q, k, v, ku, vu = (x.to(gpu) for x in _draw([(1, T_lat * P, H, D), (1, T_lat * P, HKV, D),
                                                     (1, T_lat * P, HKV, D), (1, S_UND, HKV, D),
                                                     (1, S_UND, HKV, D)], seed=T_lat))
        kg, vg = lv.build_global_kv(k, v, m.global_indices, P)
        kg, vg = torch.cat([kg, ku], 1), torch.cat([vg, vu], 1)
        out = lv.get_shared_runner().run(q, k, v, kg, vg, m)
        assert out.shape == q.shape and torch.isfinite(out.float()).all()
        rows = [set(r) for r in om.build_frame_mask(T_lat, P, 2, 1, kfi).rows]
        ro, _ = oa.per_frame_sdpa(q.float(), k.float(), v.float(), rows, P, k_extra=ku.float(), v_extra=vu.float())
        _close(out, ro, f"runner T={T_lat}")
        if kfi == 1:
            dense, _ = oa.dense_attention(q.float(), torch.cat([k, ku], 1).float(), torch.cat([v, vu], 1).float())
            rel = ((out.float() - dense).norm() / dense.norm()).item()
            assert rel < 2e-2


def test_build_global_kv_exact(gpu):
    # lvsa-vllm-omni/tests/test_global_kv.py
    B, T, P, H, D = 1, 5, 2, 1, 8
    k = torch.arange(T * P, dtype=torch.float32).view(1, T * P, 1, 1).expand(B, T * P, H, D).contiguous().to(gpu)
    kg, _ = lv.build_global_kv(k, k.clone(), [1, 3], P)
    assert kg[0, :, 0, 0].tolist() == [2, 3, 6, 7]
    kb = torch.randn(3, 8 * 4, 2, 8, device=gpu, dtype=torch.bfloat16)
    kg, vg = lv.build_global_kv(kb, kb, [0, 4], 4)
    for b in range(3):
        assert torch.equal(kg[b, :4], kb[b, :4]) and torch.equal(kg[b, 4:], kb[b, 16:20])
    e, _ = lv.build_global_kv(kb, kb, [], 4)
    assert e.shape == (3, 0, 2, 8)
    full, _ = lv.build_global_kv(kb, kb, list(range(8)), 4)
    assert torch.equal(full, kb)


@pytest.mark.parametrize("D", [128, 64, 96, 192, 256])
def test_single_prefill_dense(D, gpu):
    """Dense prefill at every head size (head size 192: 256-row tiles on the
    dual-wide map, which a dense plan takes whatever its length)."""
    q, k, v = (x.to(gpu) for x in _draw([(1, 300, 4, D), (1, 333, 2, D), (1, 333, 2, D)]))
    o, lse = lv.single_prefill_with_kv_cache(q[0], k[0], v[0], causal=False, return_lse=True)
    ro, rl = oa.dense_attention(q.float(), k.float(), v.float())
    _close(o.unsqueeze(0), ro, f"single_prefill D={D}")
    torch.testing.assert_close(lse.cpu(), rl[0].transpose(0, 1).cpu() / math.log(2.0), atol=3e-2, rtol=0)


def test_batch_views_and_fp32_inputs(gpu):
    T, P, W, H, D = 8, 64, 1, 2, 64
    m = _meta(T, P, W, 1, 3, 1)
    qkv = torch.randn(2, T * P, 3 * H * D, device=gpu, dtype=torch.bfloat16)
    q, k, v = (t.unflatten(-1, (H, D)) for t in qkv.chunk(3, dim=-1))   # strided views
    out = lv.lvsa_attention(q, k, v, m)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, 3, offset=1).rows]
    for b in range(2):
        ro, _ = oa.per_frame_sdpa(q[b:b + 1].float(), k[b:b + 1].float(), v[b:b + 1].float(), rows, P)
        _close(out[b:b + 1], ro, f"batch {b}")
    out32 = lv.lvsa_attention(q.float(), k.float(), v.float(), m)   # fp32 kernel, strided fp32 copies
    assert out32.dtype == torch.float32
    for b in range(2):
        ro, _ = oa.per_frame_sdpa(q[b:b + 1].float(), k[b:b + 1].float(), v[b:b + 1].float(), rows, P)
        _close(out32[b:b + 1], ro, f"fp32 batch {b}", max_abs=FP32_MAX_ABS, mean_abs=FP32_MEAN_ABS)


# fp32 callers compute in fp32 (fp32 MFMA products and accumulation, exact
# online softmax): tolerance against the fp32 oracle about 400x tighter
# than the 16-bit path's.
FP32_MAX_ABS = 5e-5
FP32_MEAN_ABS = 5e-6


def test_fp32_baseline_config_1(gpu):
    """BASELINE config 1 (fp32, 12 heads, D 128, 9 frames x 256 tokens, 1
    anchor, keyframe stride 4 rotated by step 3, window 1) through
    lvsa_sdpa and lvsa_attention, against the fp32 oracle on the CPU."""
    T, P, W, kfi, off, H, D = 9, 256, 1, 4, 3, 12, 128
    N = T * P
    q, k, v = _draw([(1, N, H, D)] * 3, dtype=torch.float32)
    m = _meta(T, P, W, 1, kfi, off)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, kfi, offset=off).rows]
    ro, rl = oa.per_frame_sdpa(q, k, v, rows, P)
    o, lse = lv.lvsa_attention(q.to(gpu), k.to(gpu), v.to(gpu), m, return_lse=True)
    assert o.dtype == torch.float32
    _close(o, ro, "fp32 lvsa_attention", max_abs=FP32_MAX_ABS, mean_abs=FP32_MEAN_ABS)
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-5, rtol=1e-6)
    # the reference's lvsa_sdpa semantics: pre-gathered globals + window frames
    kd, vd = k.to(gpu), v.to(gpu)
    kg, vg = lv.build_global_kv(kd, vd, m.global_indices, P)
    o2 = lv.lvsa_sdpa(q.to(gpu), kd, vd, kg, vg, m)
    _close(o2, ro, "fp32 lvsa_sdpa", max_abs=FP32_MAX_ABS, mean_abs=FP32_MEAN_ABS)
    # the bf16 path on the same data is within the 16-bit tolerance only
    ob = lv.lvsa_attention(*(x.to(gpu, torch.bfloat16) for x in (q, k, v)), m)
    assert (ob.float().cpu() - ro).abs().max().item() > 20 * FP32_MAX_ABS


@pytest.mark.parametrize("cfg", SMALL, ids=[str(c[:10]) for c in SMALL])
def test_fp32_small_configs(cfg, gpu):
    """fp32 over the small grid: every head size, GQA, text keys and text
    queries, W = 0 and frames below a tile (generic masks), kfi = 1."""
    T, P, W, n, kfi, off, H, Hkv, D, n_txt, _ = cfg
    N = T * P
    q, k, v, qt, kt, vt = _draw([(1, N, H, D), (1, N, Hkv, D), (1, N, Hkv, D), (1, n_txt, H, D),
                                 (1, n_txt, Hkv, D), (1, n_txt, Hkv, D)], seed=4, dtype=torch.float32)
    m = _meta(T, P, W, n, kfi, off)
    g = [x.to(gpu) for x in (q, k, v, qt, kt, vt)]
    rows = [set(r) for r in om.build_frame_mask(T, P, W, n, kfi, offset=off).rows]
    ro, rl = oa.per_frame_sdpa(q, k, v, rows, P, k_extra=kt if n_txt else None, v_extra=vt if n_txt else None)
    if n_txt:
        o, ot, lse, lse_t = lv.lvsa_attention(g[0], g[1], g[2], m, k_text=g[4], v_text=g[5], q_text=g[3],
                                              return_lse=True)
        rto, rtl = oa.text_row_attention(qt, k, v, kt, vt)
        _close(ot, rto, "fp32 text rows", max_abs=FP32_MAX_ABS, mean_abs=FP32_MEAN_ABS)
        torch.testing.assert_close(lse_t.cpu(), rtl, atol=2e-5, rtol=1e-6)
    else:
        o, lse = lv.lvsa_attention(g[0], g[1], g[2], m, return_lse=True)
    _close(o, ro, f"fp32 D={D}", max_abs=FP32_MAX_ABS, mean_abs=FP32_MEAN_ABS)
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-5, rtol=1e-6)


def test_fp32_wrapper_and_prefill(gpu):
    """fp32 through the block-sparse wrapper (planned for fp16, run in fp32:
    the wrapper re-plans for 128-row tiles) and the dense prefill."""
    R, C, nb, H, D = 64, 64, 6, 2, 128
    g = torch.Generator().manual_seed(9)
    indptr = torch.tensor([0, 2, 3, 6, 6, 8, 9], dtype=torch.int32)
    indices = torch.tensor([0, 3, 1, 5, 2, 0, 4, 1, 3], dtype=torch.int32)
    q, k, v = (torch.randn(nb * R, H, D, generator=g) for _ in range(3))
    w = lv.BlockSparseAttentionWrapper()
    w.plan(indptr.to(gpu), indices.to(gpu), nb * R, nb * C, R, C, H, H, D)
    o = w.run(q.to(gpu), k.to(gpu), v.to(gpu))
    assert o.dtype == torch.float32
    for i in range(nb):
        cols = indices[indptr[i]:indptr[i + 1]].tolist()
        rows = slice(i * R, (i + 1) * R)
        if not cols:
            assert (o[rows] == 0).all()
            continue
        kk = torch.cat([k[c * C:(c + 1) * C] for c in cols])
        vv = torch.cat([v[c * C:(c + 1) * C] for c in cols])
        ro, _ = oa.dense_attention(q[rows].unsqueeze(0), kk.unsqueeze(0), vv.unsqueeze(0))
        _close(o[rows].unsqueeze(0), ro, f"fp32 wrapper row block {i}", max_abs=FP32_MAX_ABS,
               mean_abs=FP32_MEAN_ABS)
    qd, kd, vd = (torch.randn(*s, generator=g) for s in ((70, 4, 64), (3000, 2, 64), (3000, 2, 64)))
    od = lv.single_prefill_with_kv_cache(qd.to(gpu), kd.to(gpu), vd.to(gpu))
    rd, _ = oa.dense_attention(qd.unsqueeze(0), kd.unsqueeze(0), vd.unsqueeze(0))
    _close(od.unsqueeze(0), rd, "fp32 prefill", max_abs=FP32_MAX_ABS, mean_abs=FP32_MEAN_ABS)


EXTREME = ["hot", "cold", "cold_then_hot", "hot_then_cold"]


@pytest.mark.parametrize("block_q", [128, 256], ids=["tile128", "tile256"])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("D", [64, 96, 128, 192, 256])
@pytest.mark.parametrize("pattern", EXTREME)
@pytest.mark.parametrize("P", [96, 300])
def test_extreme_logits(P, pattern, D, dt, block_q, gpu, monkeypatch):
    """Logits far from N(0,1), where the exponent offset of a row has to move.

    * hot: |s * scale| up to hundreds, so 2^(s * scale * log2 e) overflows fp32 without an offset.
    * cold: every logit very negative, so the exponentials underflow without an offset.
    * cold_then_hot / hot_then_cold: the key frames switch between the two, so a row's offset
      first settles low and must move up, or must stay while later blocks vanish.

    Frames of 300 tokens put D = 128 on the single-stream kernel, whose softmax
    skips the row max unless a block raises it (its rare path).
    """
    monkeypatch.setenv("LVSA_ATTN_BLOCK_Q", str(block_q))
    T, W, n, kfi, off, H = 9, 1, 1, 4, 1, 2
    N = T * P
    amp = 12.0 if dt == torch.bfloat16 else 5.0
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, N, H, D, generator=g)
    k = torch.randn(1, N, H, D, generator=g)
    v = torch.randn(1, N, H, D, generator=g)
    hot_q, hot_k = amp * q, amp * k
    cold_q, cold_k = amp * (q.abs() + 0.5), -amp * (k.abs() + 0.5)
    key_frame = torch.arange(N) // P
    if pattern == "hot":
        q, k = hot_q, hot_k
    elif pattern == "cold":
        q, k = cold_q, cold_k
    else:
        first_cold = pattern == "cold_then_hot"
        early = (key_frame < T // 2).view(1, N, 1, 1)
        q = cold_q if first_cold else hot_q.abs() + 0.5
        k_cold, k_hot = cold_k, amp * (k.abs() + 0.5)
        k = torch.where(early, k_cold, k_hot) if first_cold else torch.where(early, k_hot, k_cold)
    q, k, v = q.to(dt), k.to(dt), v.to(dt)
    m = _meta(T, P, W, n, kfi, off)
    o, lse = lv.lvsa_attention(q.to(gpu), k.to(gpu), v.to(gpu), m, return_lse=True)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, n, kfi, offset=off).rows]
    ro, rl = oa.per_frame_sdpa(q.float(), k.float(), v.float(), rows, P)
    assert torch.isfinite(o.float()).all() and torch.isfinite(lse).all()
    _close(o, ro, f"{pattern} D={D}")
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-2, rtol=1e-5)


def test_rejects_unsupported_head_dim(gpu):
    m = _meta(4, 16, 1, 1, 2)
    q = torch.randn(1, 64, 2, 80, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="head_dim 80"):
        lv.lvsa_attention(q, q, q, m)


# ── BASELINE shapes at full size ─────────────────────────────────────────────

BASELINE = [
    # name, T, P, W, kfi, off, H, D, n_txt, dtype, spot frames
    ("cpu", 9, 256, 1, 4, 3, 12, 128, 0, torch.float32, None),
    ("wan4x_off0", 84, 1560, 2, 8, 0, 12, 128, 0, torch.bfloat16, [0, 1, 41, 42, 82, 83]),
    ("wan4x_off5", 84, 1560, 2, 8, 5, 12, 128, 0, torch.bfloat16, [1, 13, 50, 83]),
    ("wan6x_w1", 121, 1560, 1, 8, 3, 12, 128, 0, torch.bfloat16, [0, 60, 120]),
    ("cog", 13, 1350, 1, 4, 0, 48, 64, 226, torch.bfloat16, [0, 5, 12]),
    ("hv_off2", 49, 1590, 2, 8, 2, 16, 128, 256, torch.bfloat16, [0, 24, 48]),
]


@pytest.mark.parametrize("cfg", BASELINE, ids=[c[0] for c in BASELINE])
def test_baseline_config_parity(cfg, gpu):
    name, T, P, W, kfi, off, H, D, n_txt, dt, frames = cfg
    N = T * P
    q, k, v, qt, kt, vt = _draw([(1, N, H, D), (1, N, H, D), (1, N, H, D), (1, n_txt, H, D),
                                 (1, n_txt, H, D), (1, n_txt, H, D)], dtype=dt)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    m = _meta(T, P, W, 1, kfi, off)
    if n_txt:
        o, ot = lv.lvsa_attention(qd, kd, vd, m, k_text=kt.to(gpu), v_text=vt.to(gpu), q_text=qt.to(gpu))
    else:
        o = lv.lvsa_attention(qd, kd, vd, m)
    # size-independent properties: finite, convex combination of value rows
    vmax = v.abs().max().item() if not n_txt else max(v.abs().max().item(), vt.abs().max().item())
    assert torch.isfinite(o.float()).all()
    assert o.float().abs().max().item() <= vmax * 1.01
    rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, kfi, offset=off).rows]
    ro, _ = oa.per_frame_sdpa(qd.float(), kd.float(), vd.float(), rows, P,
                              k_extra=kt.to(gpu).float() if n_txt else None,
                              v_extra=vt.to(gpu).float() if n_txt else None, frames=frames)
    _close(o, ro, name)
    if n_txt:
        rto, _ = oa.text_row_attention(qt.to(gpu).float(), kd.float(), vd.float(), kt.to(gpu).float(),
                                       vt.to(gpu).float())
        _close(ot, rto, name + " text rows")


SWEEP = [
    # name, T, P, W, kfi, H, D, n_txt, offsets (full BASELINE sizes, bf16)
    ("wan4x", 84, 1560, 2, 8, 12, 128, 0, tuple(range(8))),
    ("hv", 49, 1590, 2, 8, 16, 128, 256, tuple(range(8))),
    ("wan6x_w2", 121, 1560, 2, 8, 12, 128, 0, (0, 3, 6)),
    ("wan6x_w4", 121, 1560, 4, 8, 12, 128, 0, (1, 7)),
]


def _sweep_frames(T, P, kfi, off):
    """Query frames to compare: first / last, the rotated keyframes and their
    neighbours (rows that gain or lose a global frame with the offset), and
    the frames whose first row lies nearest above a 256-row tile edge and a
    128-row block edge."""
    fs = {0, 1, T - 1, off % T, (off + 1) % T, (off - 1) % T}
    mid = off + kfi * ((T // kfi) // 2)
    fs |= {mid % T, (mid + 1) % T}
    fs.add(min(range(1, T), key=lambda f: (f * P) % 256))
    fs.add(min(range(1, T), key=lambda f: (-(f * P)) % 128))
    return sorted(fs)


@pytest.mark.parametrize("cfg", SWEEP, ids=[c[0] for c in SWEEP])
def test_baseline_sweep_spot_frames(cfg, gpu):
    """Every keyframe rotation of Wan 4x and HunyuanVideo and the window
    sweep of Wan 6x, at full size through lvsa_attention: about 9 query
    frames per offset against the fp32 oracle, all frames by properties."""
    name, T, P, W, kfi, H, D, n_txt, offsets = cfg
    N = T * P
    g = torch.Generator(device=gpu).manual_seed(11)
    q, k, v = (torch.randn(1, N, H, D, generator=g, device=gpu).to(torch.bfloat16) for _ in range(3))
    qt, kt, vt = (torch.randn(1, n_txt, H, D, generator=g, device=gpu).to(torch.bfloat16) for _ in range(3))
    qf, kf, vf = q.float(), k.float(), v.float()
    vmax = max(v.abs().max().item(), vt.abs().max().item() if n_txt else 0.0)
    for off in offsets:
        m = _meta(T, P, W, 1, kfi, off)
        if n_txt:
            o, ot = lv.lvsa_attention(q, k, v, m, k_text=kt, v_text=vt, q_text=qt)
        else:
            o = lv.lvsa_attention(q, k, v, m)
        assert torch.isfinite(o.float()).all() and o.float().abs().max().item() <= vmax * 1.01
        rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, kfi, offset=off).rows]
        frames = _sweep_frames(T, P, kfi, off)
        ro, _ = oa.per_frame_sdpa(qf, kf, vf, rows, P, k_extra=kt.float() if n_txt else None,
                                  v_extra=vt.float() if n_txt else None, frames=frames)
        _close(o, ro, f"{name} offset {off} frames {frames}")
        if n_txt and off == offsets[0]:
            rto, _ = oa.text_row_attention(qt.float(), kf, vf, kt.float(), vt.float())
            _close(ot, rto, f"{name} text rows")


ALL_FRAMES = [
    # name, T, P, W, kfi, offsets, H, D, n_txt[, dtype[, Hkv]] (full BASELINE sizes, bf16 and Hkv = H
    # unless given).  Wan 4x, Wan 6x (window +-2), HunyuanVideo and CogVideoX at every keyframe
    # rotation; the Wan 6x window sweep points +-1 and +-4 at four rotations each.
    ("wan4x_all_offsets", 84, 1560, 2, 8, tuple(range(8)), 12, 128, 0),
    ("wan6x_w1_four_offsets", 121, 1560, 1, 8, (0, 3, 5, 7), 12, 128, 0),
    ("wan6x_w2_all_offsets", 121, 1560, 2, 8, tuple(range(8)), 12, 128, 0),
    ("wan6x_w4_four_offsets", 121, 1560, 4, 8, (1, 2, 6, 7), 12, 128, 0),
    ("hv_all_offsets", 49, 1590, 2, 8, tuple(range(8)), 16, 128, 256),
    ("cog_all_offsets", 13, 1350, 1, 4, tuple(range(4)), 48, 64, 226),
    # the plugin's other head sizes at the Wan 4x geometry (96: D = 128 LDS layout; 192: dual-wide map,
    # 256-row tiles; 256: wide map), and 192 with text rows (HunyuanVideo geometry), fp16 and GQA
    ("wan4x_d96_off6", 84, 1560, 2, 8, (6,), 12, 96, 0),
    ("wan4x_d192_off1", 84, 1560, 2, 8, (1,), 12, 192, 0),
    ("hv_d192_off3", 49, 1590, 2, 8, (3,), 16, 192, 256),
    ("wan4x_d192_f16_gqa3_off4", 84, 1560, 2, 8, (4,), 12, 192, 0, torch.float16, 4),
    ("wan4x_d256_off7", 84, 1560, 2, 8, (7,), 12, 256, 0),
    # fp16 inputs (the loops' f16 variants)
    ("wan4x_f16_off0", 84, 1560, 2, 8, (0,), 12, 128, 0, torch.float16),
    ("cog_f16_off2", 13, 1350, 1, 4, (2,), 48, 64, 226, torch.float16),
    # grouped K/V heads (3 query heads per K/V head), read in place
    ("wan4x_gqa3_off2", 84, 1560, 2, 8, (2,), 12, 128, 0, torch.bfloat16, 4),
    # batch of two (classifier-free guidance in the plugin): the batch index is a grid dimension
    ("cog_b2_off0", 13, 1350, 1, 4, (0,), 48, 64, 226, torch.bfloat16, 48, 2),
    ("wan4x_b2_off5", 84, 1560, 2, 8, (5,), 12, 128, 0, torch.bfloat16, 12, 2),
]


@pytest.mark.parametrize("cfg", ALL_FRAMES, ids=[c[0] for c in ALL_FRAMES])
def test_baseline_all_frames(cfg, gpu):
    """Every query frame (not a sample) at full size against the fp32 oracle
    (its per-frame gather and dense attention run on the GPU in fp32), with
    the LSE; text rows too.  Each listed keyframe rotation rebuilds the
    pattern (lvsa/lvsa_processor.py:317-331) on the same inputs."""
    name, T, P, W, kfi, offsets, H, D, n_txt = cfg[:9]
    dt = cfg[9] if len(cfg) > 9 else torch.bfloat16
    Hkv = cfg[10] if len(cfg) > 10 else H
    B = cfg[11] if len(cfg) > 11 else 1
    N = T * P
    g = torch.Generator(device=gpu).manual_seed(37)
    q = torch.randn(B, N, H, D, generator=g, device=gpu).to(dt)
    k, v = (torch.randn(B, N, Hkv, D, generator=g, device=gpu).to(dt) for _ in range(2))
    qt = torch.randn(B, n_txt, H, D, generator=g, device=gpu).to(dt)
    kt, vt = (torch.randn(B, n_txt, Hkv, D, generator=g, device=gpu).to(dt) for _ in range(2))
    args = dict(k_text=kt, v_text=vt, q_text=qt) if n_txt else {}
    for off in offsets:
        tag = f"{name} offset {off}"
        print(f"  {tag}", flush=True)
        m = _meta(T, P, W, 1, kfi, off)
        res = lv.lvsa_attention(q, k, v, m, return_lse=True, **args)
        o, lse = (res[0], res[2]) if n_txt else res
        rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, kfi, offset=off).rows]
        ro, rl = oa.per_frame_sdpa(q.float(), k.float(), v.float(), rows, P,
                                   k_extra=kt.float() if n_txt else None, v_extra=vt.float() if n_txt else None)
        assert not torch.isnan(ro).any()
        _close(o, ro, tag)
        torch.testing.assert_close(lse.float(), rl, atol=2e-2, rtol=0, msg=tag)
        del ro, rl
        if n_txt and off == offsets[0]:
            rto, _ = oa.text_row_attention(qt.float(), k.float(), v.float(), kt.float(), vt.float())
            _close(res[1], rto, tag + " text rows")


SUPPORT = [
    # name, T, P, W, kfi, H, D, n_txt, offsets (full BASELINE sizes, bf16; T + 1 <= D)
    ("wan4x", 84, 1560, 2, 8, 12, 128, 0, tuple(range(8))),
    ("wan6x_w0", 121, 1560, 0, 8, 12, 128, 0, (2,)),
    ("wan6x_w1", 121, 1560, 1, 8, 12, 128, 0, (3,)),
    ("wan6x_w2", 121, 1560, 2, 8, 12, 128, 0, (0, 5)),
    ("wan6x_w3", 121, 1560, 3, 8, 12, 128, 0, (6,)),
    ("wan6x_w4", 121, 1560, 4, 8, 12, 128, 0, (1, 7)),
    ("cog", 13, 1350, 1, 4, 48, 64, 226, tuple(range(4))),
    ("hv", 49, 1590, 2, 8, 16, 128, 256, tuple(range(8))),
]


@pytest.mark.parametrize("cfg", SUPPORT, ids=[c[0] for c in SUPPORT])
def test_baseline_frame_support_every_row(cfg, gpu):
    """Every query row at full size, every listed keyframe rotation: with the
    value rows of key frame t equal to the unit vector e_t (text keys: e_T),
    output coordinate d of a row is the softmax weight its row gives key
    frame d.  So a row's nonzero coordinates must be exactly the frames the
    reference's frame rule lets its query frame attend (plus the text
    keys), each weight positive, every other coordinate exactly 0 (masked
    keys and skipped blocks contribute nothing), and the weights sum to 1.
    Text-query rows attend every frame and the text."""
    name, T, P, W, kfi, H, D, n_txt, offsets = cfg
    assert T + 1 <= D
    N = T * P
    g = torch.Generator(device=gpu).manual_seed(29)
    q, k = (torch.randn(1, N, H, D, generator=g, device=gpu).to(torch.bfloat16) for _ in range(2))
    fidx = torch.arange(N, device=gpu) // P
    v = torch.zeros(1, N, H, D, device=gpu, dtype=torch.bfloat16)
    v[0, torch.arange(N, device=gpu), :, fidx] = 1.0
    args = {}
    if n_txt:
        qt, kt = (torch.randn(1, n_txt, H, D, generator=g, device=gpu).to(torch.bfloat16) for _ in range(2))
        vt = torch.zeros(1, n_txt, H, D, device=gpu, dtype=torch.bfloat16)
        vt[..., T] = 1.0
        args = dict(k_text=kt, v_text=vt, q_text=qt)
    for off in offsets:
        m = _meta(T, P, W, 1, kfi, off)
        res = lv.lvsa_attention(q, k, v, m, **args)
        o = (res[0] if n_txt else res)[0].float()                    # [N, H, D]
        allowed = torch.zeros(T, D, dtype=torch.bool)
        for i, r in enumerate(om.build_frame_mask(T, P, W, 1, kfi, offset=off).rows):
            allowed[i, sorted(r)] = True
        if n_txt:
            allowed[:, T] = True
        keep = allowed.to(gpu)[fidx][:, None, :]                      # [N, 1, D]
        what = f"{name} offset {off}"
        assert o.masked_fill(keep, 0.0).abs().max().item() == 0.0, what + ": weight on a frame outside the rule"
        assert o.masked_fill(~keep, 1.0).min().item() > 1e-4, what + ": an allowed frame got no weight"
        assert (o.sum(-1) - 1.0).abs().max().item() < 1e-2, what + ": weights do not sum to 1"
        if n_txt:
            ot = res[1][0].float()
            assert ot[..., T + 1:].abs().max().item() == 0.0 and ot[..., :T + 1].min().item() > 1e-4, what
            assert (ot.sum(-1) - 1.0).abs().max().item() < 1e-2, what


SPLIT = [
    # T, P, H, Hkv, D, n_txt, dtype, B   (text tiles of more than 128 key blocks: split into chunks)
    (8, 1100, 2, 2, 128, 100, torch.bfloat16, 1),   # 140 blocks: 2 chunks
    (24, 1100, 2, 1, 128, 300, torch.bfloat16, 2),  # 418 blocks: 4 chunks, GQA, batch 2
    (13, 1350, 3, 3, 64, 226, torch.float16, 1),    # CogVideoX frame size
    (9, 1000, 2, 2, 96, 37, torch.bfloat16, 1),
    (9, 1000, 2, 2, 256, 37, torch.bfloat16, 1),    # 128-row tiles
]


@pytest.mark.parametrize("cfg", SPLIT, ids=[str(c[:6]) for c in SPLIT])
def test_text_split_parity(cfg, gpu, monkeypatch):
    """Text-query tiles split into key-range chunks (scratch + log-sum-exp
    merge launch) against the fp32 oracle and against the unsplit launch."""
    monkeypatch.setenv("LVSA_VIDEO_SPLIT", "0")   # video tiles whole: their rows compare bit for bit
    T, P, H, Hkv, D, n_txt, dt, B = cfg
    N = T * P
    m = _meta(T, P, 1, 1, 4, 1)
    q, k, v, qt, kt, vt = _draw([(B, N, H, D), (B, N, Hkv, D), (B, N, Hkv, D), (B, n_txt, H, D),
                                 (B, n_txt, Hkv, D), (B, n_txt, Hkv, D)], seed=3, dtype=dt)
    g = [x.to(gpu) for x in (q, k, v, qt, kt, vt)]
    plan = m.full_plan(gpu, N, N, n_txt, n_txt, D)
    o1, ot1, l1, lt1 = hip_ops.attn_fwd(g[0], g[1], g[2], plan, kx=g[4], vx=g[5], qt=g[3], return_lse=True)
    o0, ot0, l0, lt0 = hip_ops.attn_fwd(g[0], g[1], g[2], plan, kx=g[4], vx=g[5], qt=g[3], return_lse=True,
                                        scratch=False)
    assert torch.equal(o1, o0) and torch.equal(l1, l0)   # video rows do not depend on the split
    for b in range(B):
        rto, rtl = oa.text_row_attention(qt[b:b + 1].float(), k[b:b + 1].float(), v[b:b + 1].float(),
                                         kt[b:b + 1].float(), vt[b:b + 1].float())
        _close(ot1[b:b + 1], rto, f"split text rows, batch {b}")
        _close(ot0[b:b + 1], rto, f"unsplit text rows, batch {b}")
        torch.testing.assert_close(lt1[b:b + 1].cpu(), rtl, atol=2e-2, rtol=0)
    _close(ot1, ot0.float(), "split vs unsplit", max_abs=8e-3, mean_abs=5e-4)


QUEUED = [
    # T, P, H, Hkv, D, n_txt, B   (well over 256 work items: the persistent work-queue launch)
    (24, 1100, 8, 2, 128, 300, 2),   # 1664 video tiles + split text chunks, GQA, batch 2
    (13, 1350, 24, 24, 64, 226, 1),  # CogVideoX frame size and text length, half the heads
    (13, 1350, 16, 4, 64, 226, 2),   # the same, GQA (16 query heads over 4) and batch 2: split tiles of both
    (40, 1560, 12, 12, 128, 0, 1),   # Wan frame size, video only
    (24, 1100, 8, 2, 192, 300, 2),   # head size 192 (the dual-wide map), GQA, split text chunks, batch 2
]


@pytest.mark.parametrize("cfg", QUEUED, ids=[str(c) for c in QUEUED])
def test_work_queues_match_static_grid(cfg, gpu, monkeypatch):
    """The single-stream kernel over the work queues (persistent work-groups,
    items stolen across XCDs) computes every whole item exactly as the launch
    with one work-group per item: with the video split off, video rows and
    LSE bit for bit (the text rows differ only by their split).  With the
    split on (the dual map of head size 64: each queue's last video tiles run
    as key-range halves merged by log-sum-exp), rows of split tiles differ by
    rounding only; spot frames, the last ones (split tiles) among them,
    against the fp32 oracle."""
    T, P, H, Hkv, D, n_txt, B = cfg
    N = T * P
    m = _meta(T, P, 2, 1, 8, 3)
    q, k, v, qt, kt, vt = _draw([(B, N, H, D), (B, N, Hkv, D), (B, N, Hkv, D), (B, n_txt, H, D),
                                 (B, n_txt, Hkv, D), (B, n_txt, Hkv, D)], seed=21)
    g = [x.to(gpu) for x in (q, k, v, qt, kt, vt)]
    plan = m.full_plan(gpu, N, N, n_txt, n_txt, D)
    kw = dict(kx=g[4], vx=g[5], qt=g[3]) if n_txt else {}
    o1, ot1, l1, lt1 = hip_ops.attn_fwd(g[0], g[1], g[2], plan, return_lse=True, **kw)
    o0, ot0, l0, lt0 = hip_ops.attn_fwd(g[0], g[1], g[2], plan, return_lse=True, scratch=False, **kw)
    monkeypatch.setenv("LVSA_VIDEO_SPLIT", "0")
    oq, otq, lq, ltq = hip_ops.attn_fwd(g[0], g[1], g[2], plan, return_lse=True, **kw)
    monkeypatch.delenv("LVSA_VIDEO_SPLIT")
    assert torch.equal(oq, o0) and torch.equal(lq, l0)
    # the split tiles: rounding of the two-way merge at most
    assert (o1.float() - o0.float()).abs().max().item() <= 4e-3, "split video tiles differ beyond rounding"
    assert (l1 - l0).abs().max().item() <= 1e-3, "split video tiles: LSE"
    assert torch.equal(o1, o0) != (D == 64), "the dual map (only) splits video tiles"
    rows = [set(r) for r in om.build_frame_mask(T, P, 2, 1, 8, offset=3).rows]
    for b in range(B):
        ro, _ = oa.per_frame_sdpa(g[0][b:b + 1].float(), g[1][b:b + 1].float(), g[2][b:b + 1].float(), rows, P,
                                  k_extra=g[4][b:b + 1].float() if n_txt else None,
                                  v_extra=g[5][b:b + 1].float() if n_txt else None, frames=[0, T // 2, T - 1])
        _close(o1[b:b + 1], ro, f"queued, batch {b}")
    if n_txt:
        _close(ot1, ot0.float(), "queued text vs unsplit", max_abs=8e-3, mean_abs=5e-4)
        rto, _ = oa.text_row_attention(g[3][:1].float(), g[1][:1].float(), g[2][:1].float(), g[4][:1].float(),
                                       g[5][:1].float())
        _close(ot1[:1], rto, "queued text rows")


TALL = [
    # T, P, W, kfi, off, H, Hkv, D, n_txt, dtype, B  (head size 64, frames >= 383 rows: 384-row tiles possible)
    (13, 1350, 1, 4, 0, 6, 6, 64, 226, torch.bfloat16, 1),     # CogVideoX frame and text sizes
    (9, 383, 2, 4, 1, 4, 2, 64, 37, torch.bfloat16, 2),        # smallest frame for 384 rows, GQA, batch 2
    (21, 700, 1, 3, 2, 3, 3, 64, 0, torch.float16, 1),         # fp16, video only, frames straddling tiles
    (16, 1500, 2, 8, 5, 8, 4, 64, 300, torch.float16, 1),      # more than 256 items: work queues
]


@pytest.mark.parametrize("cfg", TALL, ids=[str(c[:9]) for c in TALL])
def test_head64_maps_agree(cfg, gpu, monkeypatch):
    """Head size 64 has three single-stream maps for frames of >= 383 rows:
    the dual map (the default: 256-row tiles, 4 waves of 64 rows, two
    work-groups per CU), 8 waves of 32 rows on the same plan
    (LVSA_D64_WAVES=8) and 12 waves on 384-row tiles.  Per query row the
    8- and 12-wave kernels walk the same key blocks in the same order
    (blocks masked out for a row add exact zeros), so their O and LSE agree
    bit for bit.  The dual map computes each 32-row half as the 8-wave kernel
    does, except that a half also takes the exact-max path when the other
    half of its wave needs it (a rescale, rounding only).  Spot frames and
    text rows are checked against the fp32 oracle."""
    T, P, W, kfi, off, H, Hkv, D, n_txt, dt, B = cfg
    monkeypatch.setenv("LVSA_VIDEO_SPLIT", "0")   # whole tiles: the maps split different tiles
    N = T * P
    m = _meta(T, P, W, 1, kfi, off)
    q, k, v, qt, kt, vt = _draw([(B, N, H, D), (B, N, Hkv, D), (B, N, Hkv, D), (B, n_txt, H, D),
                                 (B, n_txt, Hkv, D), (B, n_txt, Hkv, D)], seed=17, dtype=dt)
    g = [x.to(gpu) for x in (q, k, v, qt, kt, vt)]
    plan = m.full_plan(gpu, N, N, n_txt, n_txt, D, dt)
    assert plan.block_q == 256
    st = m.device_state(gpu)
    plan384 = hip_ops.plan_build(st.mask.rel_full, n_q=N, n_k=N, n_x=n_txt, n_tq=n_txt, R=P, Cf=P,
                                 max_row_frames=max(1, m.max_row_frames), block_q=384)
    kw = dict(kx=g[4], vx=g[5], qt=g[3]) if n_txt else {}
    od, otd, ld, ltd = hip_ops.attn_fwd(g[0], g[1], g[2], plan, return_lse=True, **kw)
    o12, ot12, l12, lt12 = hip_ops.attn_fwd(g[0], g[1], g[2], plan384, return_lse=True, **kw)
    monkeypatch.setenv("LVSA_D64_WAVES", "8")
    o8, ot8, l8, lt8 = hip_ops.attn_fwd(g[0], g[1], g[2], plan, return_lse=True, **kw)
    monkeypatch.delenv("LVSA_D64_WAVES")
    assert torch.equal(o12, o8) and torch.equal(l12, l8), "video rows differ between 384- and 256-row tiles"
    if n_txt:
        assert torch.equal(ot12, ot8) and torch.equal(lt12, lt8), "text rows differ"
    # dual map against 8 waves: rounding of an extra rescale at most
    assert (od.float() - o8.float()).abs().max().item() <= 2e-3 and (ld - l8).abs().max().item() <= 1e-4
    if n_txt:
        assert (otd.float() - ot8.float()).abs().max().item() <= 2e-3 and (ltd - lt8).abs().max().item() <= 1e-4
    rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, kfi, offset=off).rows]
    for b in range(B):
        ro, _ = oa.per_frame_sdpa(g[0][b:b + 1].float(), g[1][b:b + 1].float(), g[2][b:b + 1].float(), rows, P,
                                  k_extra=g[4][b:b + 1].float() if n_txt else None,
                                  v_extra=g[5][b:b + 1].float() if n_txt else None, frames=[0, 1, T // 2, T - 1])
        _close(od[b:b + 1], ro, f"dual map, batch {b}")
        _close(o12[b:b + 1], ro, f"384-row tiles, batch {b}")
    if n_txt:
        rto, _ = oa.text_row_attention(g[3][:1].float(), g[1][:1].float(), g[2][:1].float(), g[4][:1].float(),
                                       g[5][:1].float())
        _close(otd[:1], rto, "dual map, text rows")
        _close(ot12[:1], rto, "384-row tiles, text rows")


@pytest.mark.parametrize("D", [128, 192])
def test_single_prefill_long_keys_split(D, gpu):
    """Dense prefill over more than 128 key blocks runs split (chunks + merge)."""
    q, k, v = (x.to(gpu) for x in _draw([(1, 70, 4, D), (1, 20000, 2, D), (1, 20000, 2, D)], seed=5))
    o, lse = lv.single_prefill_with_kv_cache(q[0], k[0], v[0], causal=False, return_lse=True)
    ro, rl = oa.dense_attention(q.float(), k.float(), v.float())
    _close(o.unsqueeze(0), ro, f"single_prefill split D={D}")
    torch.testing.assert_close(lse.cpu(), rl[0].transpose(0, 1).cpu() / math.log(2.0), atol=3e-2, rtol=0)


def test_plan_overflow_and_block_k_are_rejected(gpu):
    """A plan whose entry capacity is too small (max_row_frames below the
    relation's row maximum) raises at first use; so does a plan built for key
    blocks other than the kernels' 64 rows."""
    T, P, H, D = 12, 300, 2, 128
    m = _meta(T, P, 2, 1, 4, 1)
    m.ensure_device(gpu)
    st = m.device_state(gpu)
    q, k, v = (x.to(gpu) for x in _draw([(1, T * P, H, D)] * 3))
    bad = hip_ops.plan_build(st.mask.rel_full, n_q=T * P, n_k=T * P, R=P, Cf=P, max_row_frames=1)
    with pytest.raises(RuntimeError, match="exceed the capacity"):
        hip_ops.attn_fwd(q, k, v, bad)
    wide = hip_ops.plan_build(st.mask.rel_full, n_q=T * P, n_k=T * P, R=P, Cf=P,
                              max_row_frames=m.max_row_frames, block_k=128)
    with pytest.raises(ValueError, match="block_k=128"):
        hip_ops.attn_fwd(q, k, v, wide)
    good = hip_ops.plan_build(st.mask.rel_full, n_q=T * P, n_k=T * P, R=P, Cf=P, max_row_frames=m.max_row_frames)
    out, _, _, _ = hip_ops.attn_fwd(q, k, v, good)
    assert torch.equal(out, lv.lvsa_attention(q, k, v, m))


def test_wrapper_rejects_out_of_range_columns(gpu):
    w = lv.BlockSparseAttentionWrapper()
    indptr = torch.tensor([0, 2, 3], dtype=torch.int32)
    indices = torch.tensor([0, 5, 1], dtype=torch.int32)  # column 5 of 2
    w.plan(indptr, indices, M=128, N=128, R=64, C=64, num_qo_heads=2, num_kv_heads=2, head_dim=128)
    q, k, v = (x.to(gpu) for x in _draw([(128, 2, 128)] * 3))
    with pytest.raises(ValueError, match="outside"):
        w.run(q, k, v)


def _stream_cfg(seed, p_min=255):
    """Random geometries the single-stream kernel serves (frames of at least
    p_min tokens): window / keyframe patterns, text, GQA, both dtypes."""
    g = torch.Generator().manual_seed(2000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]  # noqa: E731
    T = int(torch.randint(1, 14, (1,), generator=g))
    P = int(torch.randint(p_min, 700, (1,), generator=g))
    W = pick([0, 1, 2, 3])
    n = pick([1, 1, 2])
    kfi = pick([None, 1, 2, 3, 4, 8])
    off = int(torch.randint(0, 8, (1,), generator=g)) % (kfi or 1)
    Hkv = pick([1, 2])
    H = Hkv * pick([1, 2])
    n_txt = pick([0, 0, 1, 37, 64, 300])
    dt = pick([torch.bfloat16, torch.float16])
    return T, P, W, n, kfi, off, H, Hkv, n_txt, dt


@pytest.mark.parametrize("D", [128, 64, 96, 192, 256])
@pytest.mark.parametrize("seed", range(16))
def test_stream_kernel_random_geometries(seed, D, gpu, monkeypatch):
    """D = 64, 96 and 128 on frames of >= 255 tokens, and D = 192 and 256 (the
    wide map, 128-row tiles) on frames of >= 127, run the hand-scheduled
    single-stream kernel; against the fp32 oracle, and the ping-pong (D >= 192:
    4-wave) kernel within bf16 rounding."""
    # the wide map's 128-row tiles take frames from 127 tokens on
    T, P, W, n, kfi, off, H, Hkv, n_txt, dt = _stream_cfg(seed, 127 if D >= 192 else 255)
    N = T * P
    m = _meta(T, P, W, n, kfi, off)
    q, k, v, qt, kt, vt = _draw([(1, N, H, D), (1, N, Hkv, D), (1, N, Hkv, D), (1, n_txt, H, D),
                                 (1, n_txt, Hkv, D), (1, n_txt, Hkv, D)], seed=seed, dtype=dt)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, n, kfi, offset=off).rows]
    args = dict(k_text=kt.to(gpu), v_text=vt.to(gpu), q_text=qt.to(gpu)) if n_txt else {}
    res = lv.lvsa_attention(q.to(gpu), k.to(gpu), v.to(gpu), m, return_lse=True, **args)
    monkeypatch.setenv("LVSA_ATTN_KERNEL", "pp")
    res_pp = lv.lvsa_attention(q.to(gpu), k.to(gpu), v.to(gpu), m, return_lse=True, **args)
    ro, rl = oa.per_frame_sdpa(q.float(), k.float(), v.float(), rows, P,
                               k_extra=kt.float() if n_txt else None, v_extra=vt.float() if n_txt else None)
    what = f"seed {seed}: D={D} T={T} P={P} W={W} n={n} kfi={kfi} off={off} H={H}/{Hkv} txt={n_txt} {dt}"
    o, lse = (res[0], res[2]) if n_txt else res
    _close(o, ro, what)
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-2, rtol=0, msg=what)
    _close(o, (res_pp[0] if n_txt else res_pp[0]).float(), what + " vs ping-pong", max_abs=8e-3, mean_abs=5e-4)
    if n_txt:
        rto, _ = oa.text_row_attention(qt.float(), k.float(), v.float(), kt.float(), vt.float())
        _close(res[1], rto, what + " text rows")


def test_shared_pattern_across_streams(gpu):
    """LVSAMetadata.build shares one pattern per set of arguments: built (mask
    and plan) on one stream and then used on another, the second stream waits
    for the build and registers itself with the allocator, and both give the
    same output bit for bit."""
    T, P, W, kfi, off, H, D = 11, 264, 1, 4, 2, 2, 128
    m = _meta(T, P, W, 1, kfi, off)
    q, k, v = (x.to(gpu) for x in _draw([(1, T * P, H, D)] * 3, seed=5))
    s1, s2 = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    s1.wait_stream(torch.cuda.current_stream(gpu))
    s2.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s1):
        o1 = lv.lvsa_attention(q, k, v, m)
    with torch.cuda.stream(s2):
        o2 = lv.lvsa_attention(q, k, v, m)
    torch.cuda.synchronize(gpu)
    st = m.device_state(gpu)
    assert st.joined.get(s1.cuda_stream) == st.version and st.joined.get(s2.cuda_stream) == st.version
    assert torch.equal(o1, o2)
    rows = [set(r) for r in om.build_frame_mask(T, P, W, 1, kfi, offset=off).rows]
    ro, _ = oa.per_frame_sdpa(q.float(), k.float(), v.float(), rows, P)
    _close(o2, ro, "second stream")
