"""Pin the oracle's in-batch MNR loss against brute-force loops, closed forms,
torch's float64 logsumexp and autograd, and central finite differences
(CPU)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import mnr as omnr


def _emb(seed, n, dim):
    return np.random.default_rng(seed).standard_normal((n, dim)).astype(np.float32)


def test_forward_matches_brute_force_loops():
    q, d = _emb(1, 3, 5), _emb(2, 4, 5)
    assert abs(omnr.mnr_forward(q, d, 7.0) - omnr.mnr_forward_loops(q, d, 7.0)) < 1e-12


def test_orthonormal_closed_form():
    # q_i = d_i = e_i (scaled rows are normalised away): cosine = I, so every
    # row loss is log(e^s + (n - 1)) - s
    n, s = 6, 20.0
    q = np.eye(n, dtype=np.float32) * 3.0
    d = np.eye(n, dtype=np.float32) * 0.5
    want = math.log(math.exp(s) + (n - 1)) - s
    assert abs(omnr.mnr_forward(q, d, s) - want) < 1e-12
    # a zero row is clamped at 1e-12 and contributes cosine 0 everywhere
    q[0] = 0.0
    want0 = (math.log(n) + (n - 1) * want) / n
    assert abs(omnr.mnr_forward(q, d, s) - want0) < 1e-12


def _torch_loss(q, d, scale):
    qn = q / q.norm(dim=1, keepdim=True).clamp_min(1e-12)
    dn = d / d.norm(dim=1, keepdim=True).clamp_min(1e-12)
    logits = (qn @ dn.T) * scale
    n = q.shape[0]
    return (torch.logsumexp(logits, dim=1) - logits[torch.arange(n), torch.arange(n)]).mean()


@pytest.mark.parametrize("nq,nd,dim", [(8, 8, 16), (5, 9, 33)])
def test_forward_and_backward_match_torch_float64(nq, nd, dim):
    q, d = _emb(3, nq, dim), _emb(4, nd, dim)
    tq = torch.from_numpy(q.astype(np.float64)).requires_grad_(True)
    td = torch.from_numpy(d.astype(np.float64)).requires_grad_(True)
    loss = _torch_loss(tq, td, 20.0)
    loss.backward()
    assert abs(omnr.mnr_forward(q, d, 20.0) - loss.item()) < 1e-12
    gq, gd = omnr.mnr_backward(q, d, 20.0)
    np.testing.assert_allclose(gq, tq.grad.numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(gd, td.grad.numpy(), rtol=1e-9, atol=1e-12)


def test_backward_matches_finite_differences():
    # inputs on a 2^-8 grid and a 2^-10 step: the perturbed values stay
    # exact through the forward's float32 cast
    q = np.round(_emb(5, 4, 6) * 256) / 256
    d = np.round(_emb(6, 5, 6) * 256) / 256
    gq, gd = omnr.mnr_backward(q, d, 3.0, grad=2.0)
    h = 2.0 ** -10
    for arr, grad in ((q, gq), (d, gd)):
        for idx in [(0, 0), (1, 3), (arr.shape[0] - 1, 5)]:
            plus = arr.astype(np.float64).copy()
            minus = plus.copy()
            plus[idx] += h
            minus[idx] -= h
            if arr is q:
                fp = omnr.mnr_forward(plus, d.astype(np.float64), 3.0)
                fm = omnr.mnr_forward(minus, d.astype(np.float64), 3.0)
            else:
                fp = omnr.mnr_forward(q.astype(np.float64), plus, 3.0)
                fm = omnr.mnr_forward(q.astype(np.float64), minus, 3.0)
            assert abs(2.0 * (fp - fm) / (2 * h) - grad[idx]) < 1e-4 * max(1.0, abs(grad[idx]))


def test_invalid_arguments_raise():
    q = _emb(7, 4, 3)
    with pytest.raises(ValueError):
        omnr.mnr_forward(q, q, 0.0)
    with pytest.raises(ValueError):
        omnr.mnr_forward(q, q[:2], 1.0)
