"""``torch.ops.lvsa_amd.step_attention`` on the CPU: it traces into one
``torch.compile`` graph without a break (meta tensors run the shape-only fake
implementation), successive steps reuse that graph, the fake outputs have the
real outputs' shapes and dtypes, and CPU tensors find no kernel (there is no
CPU fallback).  The GPU results are checked in ``test_gpu_step_op.py``."""
import pytest
import torch

import longvideosparseattention_amd as lv
from longvideosparseattention_amd import step_op  # noqa: F401  (registers the operator)

T, P, H, D = 4, 16, 2, 64


def _inputs(device, n_txt, dtype=torch.bfloat16):
    v = lambda n: torch.empty(1, n, H, D, device=device, dtype=dtype)  # noqa: E731
    return v(T * P), v(T * P), v(T * P), v(n_txt), v(n_txt), v(n_txt)


def _call(q, k, v, kt, vt, qt, step):
    o, ot = torch.ops.lvsa_amd.step_attention(q, k, v, kt, vt, qt, step, T, P, 1, 1, 2, True, None)
    return o * 2, ot


@pytest.mark.parametrize("n_txt", [8, 0])
def test_traces_into_one_graph(n_txt):
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    f = torch.compile(_call, backend=backend, fullgraph=True)
    x = _inputs("meta", n_txt)
    for _ in range(3):
        o, ot = f(*x, torch.empty((), dtype=torch.int64, device="meta"))
    assert len(graphs) == 1
    targets = [str(n.target) for n in graphs[0].graph.nodes if n.op == "call_function"]
    assert "lvsa_amd.step_attention" in targets
    assert o.shape == (1, T * P, H, D) and o.dtype == torch.bfloat16
    assert ot.shape == (1, n_txt, H, D)


def test_fake_shapes_follow_query_dtype():
    q, k, v, kt, vt, qt = _inputs("meta", 5, dtype=torch.float32)
    o, ot = torch.ops.lvsa_amd.step_attention(q, k, v, kt, vt, qt, torch.empty((), dtype=torch.int64, device="meta"),
                                              T, P, 1, 1, 2, True, None)
    assert o.shape == q.shape and o.dtype == torch.float32
    assert ot.shape == (1, 5, H, D) and ot.dtype == torch.float32


def test_geometry_mismatch_rejected_at_trace():
    q, k, v, kt, vt, qt = _inputs("meta", 0)
    with pytest.raises(ValueError, match="geometry"):
        torch.ops.lvsa_amd.step_attention(q, k, v, kt, vt, qt, torch.empty((), dtype=torch.int64, device="meta"),
                                          T + 1, P, 1, 1, 2, True, None)


def test_cpu_tensors_have_no_kernel():
    q, k, v, kt, vt, qt = _inputs("cpu", 0)
    with pytest.raises(NotImplementedError):
        torch.ops.lvsa_amd.step_attention(q, k, v, kt, vt, qt, torch.tensor(0), T, P, 1, 1, 2, True, None)


def test_package_export():
    assert lv.step_attention is step_op.step_attention
