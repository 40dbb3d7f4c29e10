"""GPU parity of the mask builder and the block plan (bit-exact).

* lvsa_mask_build vs the golden vectors of the reference (every BASELINE
  config and offset, and the random grid including context-parallel ranks
  with boundary guards) and vs the oracle's relation rows;
* lvsa_plan_build: the block CSR equals the oracle's canonical block CSR, and
  decoding every entry's mask descriptor back to tokens reproduces the
  oracle's dense token mask exactly.
"""

import random

import numpy as np
import pytest
import torch

from longvideosparseattention_amd import hip_ops
import longvideosparseattention_amd as lv
from oracle import lvsa_mask as om

pytestmark = pytest.mark.gpu


def _rows_from_bits(bm: torch.Tensor):
    out = []
    for r in bm.cpu().tolist():
        s = set()
        for w, word in enumerate(r):
            word &= 0xFFFFFFFF
            while word:
                b = (word & -word).bit_length() - 1
                s.add(32 * w + b)
                word &= word - 1
        out.append(s)
    return out


def _device_mask(a, gpu):
    p = hip_ops.mask_params(a["T"], a["P"], a["W"], a["n_first"], a["kfi"], a["offset"], a["expand"],
                            a["rank"], a["world"], a["guards"] or ())
    return hip_ops.mask_build(p, gpu)


def _check_record(rec, gpu):
    a = rec["args"]
    dm = _device_mask(a, gpu)
    info = dm.info.cpu().tolist()
    nnz, cn, ng = info[0], info[1], info[2]
    tag = str(a)
    assert dm.frame_indptr.cpu().tolist() == rec["fi_indptr"], tag
    assert dm.frame_indices[:nnz].cpu().tolist() == rec["fi_indices"], tag
    assert cn == rec["fi_compact_n"] and info[3] == rec["fi_MB"], tag
    assert dm.global_frames[:ng].cpu().tolist() == rec["global_indices"], tag
    assert dm.window_bounds.cpu().tolist() == rec["window_bounds"], tag
    return dm


def test_mask_golden_baseline(golden, gpu):
    for rec in golden["baseline"]:
        _check_record(rec, gpu)


def test_mask_golden_random_with_cp_ranks(golden, gpu):
    n_cp = 0
    for rec in golden["random"]:
        dm = _check_record(rec, gpu)
        a = rec["args"]
        n_cp += a["world"] > 1
        ref = om.build_frame_mask(a["T"], a["P"], a["W"], a["n_first"], a["kfi"], rank=a["rank"],
                                  world=a["world"], expand=a["expand"], offset=a["offset"], guards=a["guards"])
        full = _rows_from_bits(dm.rel_full)
        assert [sorted(x) for x in full[:ref.MB]] == ref.rows, str(a)
        assert _rows_from_bits(dm.rel_window) == om.window_only_relation(ref), str(a)
    assert n_cp > 50


def test_metadata_device_csr_equals_golden(golden, gpu):
    for rec in golden["baseline"][:12] + golden["random"][:60]:
        a = rec["args"]
        m = lv.LVSAMetadata.build(total_latent_frames=a["T"], num_patches=a["P"], window_size=a["W"],
                                  n_first_frames=a["n_first"], key_frame_interval=a["kfi"], rank=a["rank"],
                                  world=a["world"], expand_window=a["expand"], keyframe_offset=a["offset"],
                                  boundary_guards=a["guards"])
        m.ensure_device(gpu)
        assert m.fi_indptr.device.type == "cuda"
        assert m.fi_indptr.cpu().tolist() == rec["fi_indptr"]
        assert m.fi_indices.cpu().tolist() == rec["fi_indices"]


# ── plan ──────────────────────────────────────────────────────────────────


def _decode_plan(plan, rel_rows, P, n_q, n_k, n_x, n_tq):
    """Dense token masks [n_q + n_tq, n_k + n_x] described by the plan entries,
    interpreted exactly as the attention kernel does."""
    bq, bk = plan.block_q, plan.block_k
    mask = np.zeros((n_q + n_tq, n_k + n_x), dtype=bool)
    hits = np.zeros(mask.shape, dtype=np.int32)
    ind = plan.tile_indptr.cpu().tolist()
    ent = plan.entries.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    n_vt = plan.n_video_tiles
    T_k = -(-max(n_k, 1) // P)
    frame_rel = np.zeros((len(rel_rows), T_k), dtype=bool)
    for f, row in enumerate(rel_rows):
        for g in row:
            frame_rel[f, g] = True
    for t in range(plan.n_tiles):
        if t < n_vt:
            r0, r1, rowbase = t * bq, min(t * bq + bq, n_q), 0
        else:
            r0, r1, rowbase = (t - n_vt) * bq, min((t - n_vt) * bq + bq, n_tq), n_q
        rr = np.arange(r0, r1)[:, None]
        for e in range(ind[t], ind[t + 1]):
            w0, w1 = int(ent[e, 0]), int(ent[e, 1])
            extra = bool(w0 >> 31)
            j = w0 & 0x7FFFFFFF
            n_src = n_x if extra else n_k
            k0 = j * bk
            kk = np.arange(k0, k0 + bk)[None, :]
            kind = w1 & 3
            if kind == 0:
                ok = np.ones((rr.shape[0], kk.shape[1]), dtype=bool)
            elif kind == 1:
                bits, kb, qs = (w1 >> 2) & 0xF, (w1 >> 8) & 0xFF, (w1 >> 16) & 0xFF
                sel = 2 * ((rr - r0) >= qs) + ((kk - k0) >= kb)
                ok = ((bits >> sel) & 1).astype(bool)
            else:
                assert not extra and t < n_vt
                kf = np.minimum(kk, n_src - 1) // P
                ok = (kk < n_src) & frame_rel[rr // P, kf]
            assert not (ok & (kk >= n_src)).any(), "descriptor allows a key beyond the source"
            colbase = n_k if extra else 0
            okc = ok[:, : max(0, min(bk, n_src - k0))]
            sub = (slice(rowbase + r0, rowbase + r1), slice(colbase + k0, colbase + k0 + okc.shape[1]))
            mask[sub] |= okc
            hits[sub] += okc
    assert hits.max() <= 1, "a (query, key) pair is covered twice"
    return mask


@pytest.mark.parametrize("seed", range(12))
def test_plan_descriptors_reproduce_token_mask(seed, gpu):
    rng = random.Random(seed)
    T, P = rng.randint(1, 10), rng.choice([3, 7, 30, 64, 100, 130, 200])
    W, n, kfi, off = rng.randint(0, 2), rng.randint(1, 2), rng.choice([None, 2, 3, 4]), rng.randint(0, 3)
    n_x, n_tq = rng.choice([0, 5, 70]), rng.choice([0, 9, 130])
    ref = om.build_frame_mask(T, P, W, n, kfi, offset=off)
    dm = hip_ops.mask_build(hip_ops.mask_params(T, P, W, n, kfi, off), gpu)
    N = T * P
    plan = hip_ops.plan_build(dm.rel_full, n_q=N, n_k=N, n_x=n_x, n_tq=n_tq, R=P, Cf=P,
                              max_row_frames=ref.compact_n)
    torch.cuda.synchronize()
    assert plan.status[0].item() == 0
    rel = om.frame_relation(ref)
    got = _decode_plan(plan, rel, P, N, N, n_x, n_tq)
    want = np.zeros_like(got)
    want[:N, :N] = om.token_mask(rel, P, N, N)
    want[:N, N:] = True
    want[N:, :] = True
    assert np.array_equal(got, want)


@pytest.mark.parametrize("name,T,P,W,kfi,offs,b", [
    ("wan4x", 84, 1560, 2, 8, [0, 5], 128), ("cog", 13, 1350, 1, 4, [0], 64),
    ("hv", 49, 1590, 2, 8, [3], 128), ("wan6x_w4", 121, 1560, 4, 8, [7], 128)])
def test_plan_block_csr_at_baseline(name, T, P, W, kfi, offs, b, gpu):
    for off in offs:
        ref = om.build_frame_mask(T, P, W, 1, kfi, offset=off)
        rel = om.frame_relation(ref)
        dm = hip_ops.mask_build(hip_ops.mask_params(T, P, W, 1, kfi, off), gpu)
        N = T * P
        for bq, bk in [(128, 64), (b, b)]:
            plan = hip_ops.plan_build(dm.rel_full, n_q=N, n_k=N, R=P, Cf=P, max_row_frames=ref.compact_n,
                                      block_q=bq, block_k=bk)
            torch.cuda.synchronize()
            indptr, cols = om.block_csr(rel, P, N, N, bq, bk)
            assert plan.tile_indptr.cpu().tolist() == indptr, (name, off, bq, bk)
            got = (plan.entries[: indptr[-1], 0].cpu().numpy().astype(np.int64) & 0x7FFFFFFF).tolist()
            assert got == cols, (name, off, bq, bk)


def test_window_golden_arbitrary_global_sets(golden, gpu):
    """The reference's window bounds for 600 arbitrary global sets: each set
    goes in as boundary guards (no anchors, no keyframe grid), so the device's
    expanded-window tie-break is pinned beyond the anchor + grid sets."""
    by_pattern = {}
    for rec in golden["windows"]:
        by_pattern.setdefault((rec["T"], rec["W"], tuple(rec["G"]), rec["expand"]), []).append(rec)
    assert sum(len(v) for v in by_pattern.values()) == 600
    for (T, W, G, expand), recs in by_pattern.items():
        p = hip_ops.mask_params(T, 1, W, 0, None, 0, expand, guards=G)
        dm = hip_ops.mask_build(p, gpu)
        ng = int(dm.info[2].item())
        assert dm.global_frames[:ng].tolist() == sorted(G)
        bounds = dm.window_bounds.tolist()
        for rec in recs:
            assert bounds[rec["f"]] == rec["bounds"], rec


def test_auto_kfi_golden(golden, gpu):
    """lvsa_auto_kfi against the reference's compute_auto_kfi outputs."""
    recs = golden["auto_kfi"]
    out = torch.full((len(recs),), -7, dtype=torch.int32, device=gpu)
    for i, r in enumerate(recs):
        hip_ops.auto_kfi(r["T"], r["W"], r["n_first"], r["ref"], r["scale"], out=out[i:i + 1])
    assert out.tolist() == [r["kfi"] for r in recs]


def test_auto_kfi_sweep(gpu):
    """Both branches (strict / fallback), the dense cut-off, W = 0, no
    anchors, T well past the mask limit and budgets from scales below and
    above 1, against the oracle."""
    cases = [(T, W, n, ref, sc) for T in list(range(1, 48)) + [60, 97, 257, 1000, 4096, 9999]
             for W in (0, 1, 3, 12) for n in (0, 1, 4) for ref, sc in ((21, 1.0), (21, 0.45), (33, 1.3), (5, 3.0))]
    out = torch.empty(len(cases), dtype=torch.int32, device=gpu)
    for i, c in enumerate(cases):
        hip_ops.auto_kfi(*c, out=out[i:i + 1])
    want = [om.compute_auto_kfi(T, W, n, reference_frames=ref, sparsity_scale=sc) for T, W, n, ref, sc in cases]
    got = out.tolist()
    bad = [(c, g, w) for c, g, w in zip(cases, got, want) if g != w]
    assert not bad, bad[:5]
    assert len(set(want)) > 30


@pytest.mark.parametrize("scale", [0.5, 1.0, 1.7])
def test_mask_auto_kfi_equals_explicit(golden, scale, gpu):
    """lvsa_mask_build with the device re-tune (kfi derived in the kernel,
    offset = step % kfi) writes exactly what an explicit build with the
    oracle's kfi and offset writes, and reports that kfi in info[7]."""
    for rec in golden["baseline"][::2] + golden["random"][::20]:
        a = rec["args"]
        kfi = om.compute_auto_kfi(a["T"], a["W"], a["n_first"], sparsity_scale=scale)
        for step in (0, 5, 13):
            common = (a["T"], a["P"], a["W"], a["n_first"])
            pa = hip_ops.mask_params(*common, None, 0, a["expand"], a["rank"], a["world"], a["guards"] or (),
                                     auto_step=step, sparsity_scale=scale)
            pe = hip_ops.mask_params(*common, kfi, step % kfi, a["expand"], a["rank"], a["world"],
                                     a["guards"] or ())
            da, de = hip_ops.mask_build(pa, gpu), hip_ops.mask_build(pe, gpu)
            tag = (str(a), scale, step)
            assert int(da.info[7].item()) == kfi, tag
            nnz = int(de.info[0].item())
            assert da.info[:7].tolist() == de.info[:7].tolist(), tag
            assert torch.equal(da.frame_indptr, de.frame_indptr), tag
            assert torch.equal(da.frame_indices[:nnz], de.frame_indices[:nnz]), tag
            for f in ("compact_frames", "global_frames", "window_bounds", "rel_full", "rel_window"):
                assert torch.equal(getattr(da, f), getattr(de, f)), (f, tag)
