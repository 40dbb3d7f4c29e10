"""GPU parity of the FlashInfer-style wrapper on arbitrary block CSRs.

``BlockSparseAttentionWrapper.plan`` takes any block CSR, as FlashInfer's
does (``lvsa/lvsa_processor.py:805-827``): query block ``i`` (``R`` rows)
attends key blocks ``indices[indptr[i]:indptr[i+1]]`` (``C`` rows each).
These tests use block sizes that are not multiples of the kernel's 64-key
blocks (so the plan carries partial-block masks), unsorted random column
sets, GQA, every kernel tile height and head dim, and query blocks with no
key block at all.

The oracle is the explicit-mask fp32 attention of ``oracle/attention.py`` on
the same bf16-rounded inputs; tolerance max |err| <= 2e-2, mean |err| <=
2e-3. A query row with no key gets output 0 and LSE -inf, the limit of a
softmax over an empty set (the reference's masks never produce one).
"""
import itertools
import math

import pytest
import torch

import longvideosparseattention_amd as lv
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _csr(n_qblocks, n_kblocks, empty, g):
    rows = []
    for i in range(n_qblocks):
        if i in empty:
            rows.append([])
            continue
        n = int(torch.randint(1, n_kblocks + 1, (1,), generator=g))
        rows.append(torch.randperm(n_kblocks, generator=g)[:n].tolist())  # unsorted on purpose
    indptr = torch.tensor([0] + list(itertools.accumulate(len(r) for r in rows)), dtype=torch.int32)
    indices = torch.tensor([j for r in rows for j in r], dtype=torch.int32)
    return rows, indptr, indices


# R, C = 96, 80: generic descriptors, the ping-pong / 4-wave kernels;
# R, C = 320, 300 (block_q 256): the single-stream kernels
@pytest.mark.parametrize("block_q,R,C", [(128, 96, 80), (256, 96, 80), (256, 320, 300)])
@pytest.mark.parametrize("D", [64, 96, 128, 192, 256])
def test_arbitrary_csr_with_empty_rows(D, block_q, R, C, gpu, monkeypatch):
    monkeypatch.setenv("LVSA_ATTN_BLOCK_Q", str(block_q))
    H, HKV = 4, 2
    MB, NB = 7, 9
    M, N = MB * R, NB * C
    g = torch.Generator().manual_seed(D + block_q)
    rows, indptr, indices = _csr(MB, NB, empty=(1, 4), g=g)
    q, k, v = (torch.randn(*s, generator=g).to(torch.bfloat16) for s in [(M, H, D), (N, HKV, D), (N, HKV, D)])

    w = lv.BlockSparseAttentionWrapper(torch.empty(1, dtype=torch.uint8, device=gpu))
    w.plan(indptr.to(gpu), indices.to(gpu), M=M, N=N, R=R, C=C, num_qo_heads=H, num_kv_heads=HKV,
           head_dim=D, q_data_type="bfloat16")
    o, lse = w.run(q.to(gpu), k.to(gpu), v.to(gpu), return_lse=True)
    o, lse = o.float().cpu(), lse.float().cpu()

    mask = torch.zeros(M, N, dtype=torch.bool)
    for i, r in enumerate(rows):
        for j in r:
            mask[i * R:(i + 1) * R, j * C:(j + 1) * C] = True
    ro, rl = oa.dense_attention(q[None].float(), k[None].float(), v[None].float(), mask=mask)
    live = mask.any(dim=1)
    err = (o[live] - ro[0][live]).abs()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, (err.max().item(), err.mean().item())
    # base-2 LSE, as FlashInfer returns it
    torch.testing.assert_close(lse[live], rl[0].transpose(0, 1)[live] / math.log(2.0), atol=3e-2, rtol=0)
    assert torch.all(o[~live] == 0)
    assert torch.all(torch.isneginf(lse[~live]))
