"""In-batch multiple-negatives ranking loss (numpy restatement; test
infrastructure).

``mnr_loss_terms(queries, documents, eye, scale=scale).loss`` of
``src/representax/tasks/retrieval/mnr.py`` with query i's positive at
document i, unit weights and every row valid:

* ``_normalize`` (mnr.py:48-52): rows cast to float32 and divided by
  ``max(||row||_2, 1e-12)``;
* ``_direction_row_terms`` (mnr.py:132-158): ``cosine = q_n d_n^T``,
  ``logits = cosine * scale``, ``partition = logsumexp(logits, axis=1)``,
  ``row_loss_i = partition_i - logits_ii`` (one positive of weight 1);
* the forward loss (mnr.py:338-341): the mean of the row losses.

``mnr_backward`` is the JAX transpose of the same expressions:
``dlogits = g (softmax(logits) - I) / n_queries``, through the product and
the normalisation ``d v = (d u - u <u, d u>) / ||v||`` (``d u / 1e-12`` for
rows clamped at 1e-12).

Evaluated in float64 (``dtype``) from the float32 (or bf16-valued) inputs.
The float32 reading differs only in the order of the sums (XLA's reduction
order is not fixed by any reference test: parity unpinned for the last bits
of the float32 sums, as for the other reductions). Pinned by the tests
against brute-force loops, closed forms for orthonormal embeddings, torch's
float64 ``logsumexp`` / autograd, and central finite differences.
"""

from __future__ import annotations

import numpy as np


def _normalize(v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    norm = np.sqrt(np.sum(v * v, axis=1, keepdims=True))
    return v / np.maximum(norm, 1e-12), norm[:, 0]


def mnr_forward(queries: np.ndarray, documents: np.ndarray, scale: float = 20.0,
                dtype=np.float64) -> float:
    """The loss (mnr.py:48-52,132-158,338-341)."""

    if not (np.isfinite(scale) and scale > 0):
        raise ValueError("scale must be finite and positive")
    q = np.asarray(queries, dtype=np.float32).astype(dtype)
    d = np.asarray(documents, dtype=np.float32).astype(dtype)
    nq = q.shape[0]
    if d.shape[0] < nq:
        raise ValueError("every query needs its positive document")
    qn, _ = _normalize(q)
    dn, _ = _normalize(d)
    logits = (qn @ dn.T) * dtype(scale)
    m = logits.max(axis=1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(logits - m).sum(axis=1))
    rows = lse - logits[np.arange(nq), np.arange(nq)]
    return float(rows.mean())


def mnr_backward(queries: np.ndarray, documents: np.ndarray, scale: float = 20.0,
                 grad: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """(d queries, d documents) of ``grad * loss``, float64."""

    q = np.asarray(queries, dtype=np.float32).astype(np.float64)
    d = np.asarray(documents, dtype=np.float32).astype(np.float64)
    nq = q.shape[0]
    qn, q_norm = _normalize(q)
    dn, d_norm = _normalize(d)
    logits = (qn @ dn.T) * scale
    m = logits.max(axis=1, keepdims=True)
    p = np.exp(logits - m)
    p /= p.sum(axis=1, keepdims=True)
    dl = p.copy()
    dl[np.arange(nq), np.arange(nq)] -= 1.0
    dl *= grad / nq
    dqn = scale * dl @ dn
    ddn = scale * dl.T @ qn

    def through_norm(du, u, norm):
        out = np.empty_like(du)
        for i in range(du.shape[0]):
            if norm[i] > 1e-12:
                out[i] = (du[i] - u[i] * np.dot(u[i], du[i])) / norm[i]
            else:
                out[i] = du[i] / 1e-12
        return out

    return through_norm(dqn, qn, q_norm), through_norm(ddn, dn, d_norm)


def mnr_forward_loops(queries: np.ndarray, documents: np.ndarray, scale: float = 20.0) -> float:
    """Element-by-element float64 restatement for tiny shapes (the check
    of ``mnr_forward``)."""

    q = np.asarray(queries, dtype=np.float32).astype(np.float64)
    d = np.asarray(documents, dtype=np.float32).astype(np.float64)
    nq, dim = q.shape
    nd = d.shape[0]

    def unit(row):
        s = 0.0
        for x in row:
            s += x * x
        n = max(s ** 0.5, 1e-12)
        return [x / n for x in row]

    qs = [unit(q[i]) for i in range(nq)]
    ds = [unit(d[j]) for j in range(nd)]
    total = 0.0
    for i in range(nq):
        logits = []
        for j in range(nd):
            c = 0.0
            for e in range(dim):
                c += qs[i][e] * ds[j][e]
            logits.append(c * scale)
        m = max(logits)
        lse = m + np.log(sum(np.exp(v - m) for v in logits))
        total += lse - logits[i]
    return total / nq


__all__ = ["mnr_backward", "mnr_forward", "mnr_forward_loops"]
