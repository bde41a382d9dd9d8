"""Fused in-batch MNR loss (the train-step objective) against the oracle
(GPU): forward and both gradients, f32 and bf16 embeddings, square and
rectangular batches, a zero row, invalid arguments, graph replay."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mnr as omnr
from representax_amd import ops
from tests.helpers import rng

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _rel_l2(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("nq,nd,dim", [(64, 64, 768), (32, 32, 2048), (5, 9, 100), (1, 1, 7)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mnr_matches_oracle(nq, nd, dim, dtype):
    g = rng(500 + nq + dim)
    q = torch.from_numpy(g.standard_normal((nq, dim)).astype(np.float32)).to(DEV, dtype)
    d = torch.from_numpy(g.standard_normal((nd, dim)).astype(np.float32)).to(DEV, dtype)
    qv = q.float().cpu().numpy()
    dv = d.float().cpu().numpy()
    q.requires_grad_(True)
    d.requires_grad_(True)
    loss = ops.mnr_loss(q, d, 20.0)
    loss.backward(torch.tensor(1.5, device=DEV))
    torch.cuda.synchronize()
    want = omnr.mnr_forward(qv, dv, 20.0)
    assert loss.dtype == torch.float32
    # f32 sums in a different order than the float64 oracle
    assert abs(loss.item() - want) <= 1e-5 * max(1.0, abs(want))
    gq, gd = omnr.mnr_backward(qv, dv, 20.0, grad=1.5)
    # bf16 gradients carry one bf16 rounding (2^-9 relative)
    tol = 1e-5 if dtype == torch.float32 else 4e-3
    assert q.grad.dtype == dtype and d.grad.dtype == dtype
    assert _rel_l2(q.grad.float().cpu().numpy(), gq) <= tol
    assert _rel_l2(d.grad.float().cpu().numpy(), gd) <= tol


@pytest.mark.parametrize("nq,nd,dim", [(8, 8, 4096), (4, 8192, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mnr_at_the_kernel_limits(nq, nd, dim, dtype):
    """The largest embedding width (4096: the 16-element register array per
    thread) and the most documents (8192: a logits row in the 32 KB LDS row
    buffer), forward and both gradients."""

    test_mnr_matches_oracle(nq, nd, dim, dtype)


@pytest.mark.parametrize("q_dtype,d_dtype", [(torch.bfloat16, torch.float32),
                                             (torch.float32, torch.bfloat16)])
def test_mnr_mixed_dtypes_cast_each_set_on_its_own(q_dtype, d_dtype):
    """mnr.py:48-52 casts each embedding set to float32 separately: a bf16
    set and an f32 set meet without rounding the f32 one to bf16. Each
    gradient comes back in its own set's dtype."""

    nq, nd, dim = 24, 40, 320
    g = rng(911)
    q = torch.from_numpy(g.standard_normal((nq, dim)).astype(np.float32)).to(DEV, q_dtype)
    # f32 values with bits below bf16 precision, which a bf16 round would drop
    d = torch.from_numpy((g.standard_normal((nd, dim)) * (1 + 2.0 ** -12)).astype(np.float32)
                         ).to(DEV, d_dtype)
    qv = q.float().cpu().numpy()
    dv = d.float().cpu().numpy()
    q.requires_grad_(True)
    d.requires_grad_(True)
    loss = ops.mnr_loss(q, d, 20.0)
    loss.backward()
    torch.cuda.synchronize()
    want = omnr.mnr_forward(qv, dv, 20.0)
    assert abs(loss.item() - want) <= 1e-5 * max(1.0, abs(want))
    gq, gd = omnr.mnr_backward(qv, dv, 20.0)
    assert q.grad.dtype == q_dtype and d.grad.dtype == d_dtype
    for grad, want_g, dt in ((q.grad, gq, q_dtype), (d.grad, gd, d_dtype)):
        tol = 1e-5 if dt == torch.float32 else 4e-3
        assert _rel_l2(grad.float().cpu().numpy(), want_g) <= tol


def test_mnr_zero_row_and_orthonormal_closed_form():
    n, s = 8, 20.0
    q = torch.eye(n, 64, device=DEV) * 3.0
    d = torch.eye(n, 64, device=DEV) * 0.5
    want = float(np.log(np.exp(s) + (n - 1)) - s)
    assert abs(ops.mnr_loss(q, d, s).item() - want) <= 1e-6
    q[0] = 0.0
    q.requires_grad_(True)
    loss = ops.mnr_loss(q, d, s)
    loss.backward()
    qv = q.detach().cpu().numpy()
    gq, _ = omnr.mnr_backward(qv, d.cpu().numpy(), s)
    assert abs(loss.item() - omnr.mnr_forward(qv, d.cpu().numpy(), s)) <= 1e-5
    # the clamped row's gradient is du / 1e-12, the others go through the norm
    assert _rel_l2(q.grad.cpu().numpy(), gq) <= 1e-5


def test_mnr_is_deterministic_and_replays_in_a_graph():
    g = rng(77)
    q = torch.from_numpy(g.standard_normal((16, 128)).astype(np.float32)).to(DEV).requires_grad_(True)
    d = torch.from_numpy(g.standard_normal((16, 128)).astype(np.float32)).to(DEV).requires_grad_(True)

    def run():
        q.grad = None
        d.grad = None
        loss = ops.mnr_loss(q, d, 20.0)
        loss.backward()
        return loss.detach().clone(), q.grad.clone(), d.grad.clone()

    first = run()
    second = run()
    assert all(torch.equal(a, b) for a, b in zip(first, second))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    q.grad = None
    d.grad = None
    with torch.cuda.graph(graph):
        loss = ops.mnr_loss(q, d, 20.0)
        loss.backward()
    captured = (loss, q.grad, d.grad)
    for _ in range(3):
        for t in captured:
            t.zero_()
        run()  # eager work between the replays
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(captured, first))


def test_mnr_rejects_invalid_arguments():
    q = torch.randn(4, 8, device=DEV)
    with pytest.raises(ValueError):
        ops.mnr_loss(q, q, 0.0)
    with pytest.raises(ValueError):
        ops.mnr_loss(q, q, float("inf"))
    with pytest.raises(ValueError):
        ops.mnr_loss(q, q[:2], 1.0)
    with pytest.raises(ValueError):
        ops.mnr_loss(q, torch.randn(4, 9, device=DEV), 1.0)
    with pytest.raises(RuntimeError):
        ops.mnr_loss(q.cpu(), q.cpu(), 1.0)
