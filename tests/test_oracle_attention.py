"""Pin the fp32 attention oracle (CPU only).

The two oracle formulations (per-frame gather, explicit token mask) are
checked against each other and against library routines in the cases where
LVSA reduces to plain attention (kfi = 1 -> every frame global; W >= T).
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import lvsa_mask as om


def _rand(shape, g):
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def _library_sdpa(q, k, v, mask=None):
    H = q.shape[2]
    k = k.repeat_interleave(H // k.shape[2], dim=2)
    v = v.repeat_interleave(H // v.shape[2], dim=2)
    out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                         attn_mask=None if mask is None else mask)
    return out.transpose(1, 2)


def test_dense_matches_library_sdpa():
    g = torch.Generator().manual_seed(0)
    q, k, v = _rand((2, 37, 4, 32), g), _rand((2, 53, 2, 32), g), _rand((2, 53, 2, 32), g)
    o, lse = oa.dense_attention(q, k, v)
    torch.testing.assert_close(o, _library_sdpa(q, k, v), atol=1e-5, rtol=1e-5)
    kk = k.repeat_interleave(2, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", q, kk) / math.sqrt(32)
    torch.testing.assert_close(lse, torch.logsumexp(s, dim=-1), atol=1e-5, rtol=1e-5)


def test_masked_matches_library_sdpa_with_mask():
    g = torch.Generator().manual_seed(1)
    T, P = 9, 8
    m = om.build_frame_mask(T, P, 1, 1, 4, offset=3)
    mask = torch.from_numpy(om.token_mask(om.frame_relation(m), P, T * P, T * P))
    q, k, v = (_rand((1, T * P, 2, 16), g) for _ in range(3))
    o, _ = oa.masked_sdpa(q, k, v, mask)
    torch.testing.assert_close(o, _library_sdpa(q, k, v, mask), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("T,P,W,n,kfi,off,Hkv", [(9, 16, 1, 1, 4, 3, 2), (12, 10, 2, 1, 5, 4, 1),
                                                  (10, 4, 0, 2, 3, 0, 2), (21, 6, 3, 3, 4, 2, 2)])
def test_per_frame_equals_explicit_mask(T, P, W, n, kfi, off, Hkv):
    g = torch.Generator().manual_seed(T)
    m = om.build_frame_mask(T, P, W, n, kfi, offset=off)
    rel = om.frame_relation(m)
    N = T * P
    q = _rand((1, N, 2, 16), g)
    k, v = _rand((1, N, Hkv, 16), g), _rand((1, N, Hkv, 16), g)
    o1, l1 = oa.per_frame_sdpa(q, k, v, rel, P)
    o2, l2 = oa.masked_sdpa(q, k, v, torch.from_numpy(om.token_mask(rel, P, N, N)))
    torch.testing.assert_close(o1, o2, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(l1, l2, atol=1e-5, rtol=1e-5)


def test_kfi_one_reduces_to_dense_with_text():
    # lvsa-vllm-omni/tests/test_flashinfer_runner.py:108-129: every frame global -> dense.
    g = torch.Generator().manual_seed(5)
    T, P = 6, 8
    m = om.build_frame_mask(T, P, 2, 1, 1)
    assert len(m.global_indices) == T
    rel = om.frame_relation(m)
    q, k, v = _rand((1, T * P, 4, 32), g), _rand((1, T * P, 2, 32), g), _rand((1, T * P, 2, 32), g)
    kt, vt = _rand((1, 16, 2, 32), g), _rand((1, 16, 2, 32), g)
    o, _ = oa.per_frame_sdpa(q, k, v, rel, P, k_extra=kt, v_extra=vt)
    dense = _library_sdpa(q, torch.cat([k, kt], 1), torch.cat([v, vt], 1))
    torch.testing.assert_close(o, dense, atol=1e-5, rtol=1e-5)


def test_window_covering_everything_is_dense():
    g = torch.Generator().manual_seed(6)
    T, P = 5, 7
    m = om.build_frame_mask(T, P, 10, 1, None)
    q, k, v = (_rand((1, T * P, 2, 8), g) for _ in range(3))
    o, _ = oa.per_frame_sdpa(q, k, v, om.frame_relation(m), P)
    torch.testing.assert_close(o, _library_sdpa(q, k, v), atol=1e-5, rtol=1e-5)


def test_lvsa_sdpa_restatement_structure():
    # k_global (gathered globals) + window frames == the full frame relation.
    g = torch.Generator().manual_seed(8)
    T, P = 9, 8
    m = om.build_frame_mask(T, P, 1, 1, 4, offset=3)
    N = T * P
    q, k, v = (_rand((1, N, 2, 16), g) for _ in range(3))
    idx = torch.cat([torch.arange(f * P, (f + 1) * P) for f in m.global_indices])
    o1, _ = oa.per_frame_sdpa(q, k, v, om.window_only_relation(m), P, k_extra=k[:, idx], v_extra=v[:, idx])
    o2, _ = oa.per_frame_sdpa(q, k, v, om.frame_relation(m), P)
    torch.testing.assert_close(o1, o2, atol=1e-5, rtol=1e-5)
