"""fp64 brute-force attention on tiny inputs -- TEST INFRASTRUCTURE ONLY.

An independent formulation used to pin oracle/naive.py: explicit Python
loops over (batch, head, query, key, dim) with math.exp, no matrix products,
no torch.softmax, no repeat_interleave.  Each softmax row subtracts its own
maximum over admissible keys and divides by the explicit sum.  Only for
shapes that finish in well under a second.
"""
from __future__ import annotations

import math

import numpy as np


def brute_forward(q, k, v, *, causal: bool, sm_scale: float | None = None,
                  causal_offset: int | None = None, split: int | None = None) -> dict:
    """q (B,Hq,M,D), k/v (B,Hk,N,D) as array-likes; returns fp64 numpy arrays
    with the same keys and layouts as oracle.naive.reference_forward."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    G = Hq // Hk
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if causal_offset is None:
        causal_offset = N - M

    out = np.zeros((B, Hq, M, D))
    scores = np.full((B, Hq, M, N), -np.inf)
    weights = np.zeros((B, Hq, M, N))
    lse = np.full((B, Hq, M), -np.inf)
    for b in range(B):
        for h in range(Hq):
            hk = h // G
            for i in range(M):
                admissible = [j for j in range(N) if (not causal) or causal_offset + i >= j]
                for j in admissible:
                    acc = 0.0
                    for d in range(D):
                        acc += q[b, h, i, d] * k[b, hk, j, d]
                    scores[b, h, i, j] = acc * sm_scale
                if not admissible:
                    continue
                top = max(scores[b, h, i, j] for j in admissible)
                e = {j: math.exp(scores[b, h, i, j] - top) for j in admissible}
                total = sum(e.values())
                lse[b, h, i] = top + math.log(total)
                for j in admissible:
                    weights[b, h, i, j] = e[j] / total
                for d in range(D):
                    out[b, h, i, d] = sum(weights[b, h, i, j] * v[b, hk, j, d] for j in admissible)

    finite = np.where(np.isfinite(scores), scores, 0.0)
    res = {
        "out": out,
        "scores": scores,
        "weights": weights,
        "lse": lse,
        "total": weights.sum(axis=2),
        "row_sum": finite.sum(axis=-1),
        "col_sum": np.zeros((B, Hk, N)),
        "col_softmax": np.zeros((B, Hk, N)),
    }
    for b in range(B):
        for h in range(Hq):
            for i in range(M):
                for j in range(N):
                    res["col_sum"][b, h // G, j] += finite[b, h, i, j]
                    res["col_softmax"][b, h // G, j] += weights[b, h, i, j]
    if split is not None:
        res["cross_qk"] = np.zeros((B, Hk, split))
        res["cross_softmax"] = np.zeros((B, Hk, split))
        for b in range(B):
            for h in range(Hq):
                for i in range(split, M):
                    for j in range(split):
                        res["cross_qk"][b, h // G, j] += finite[b, h, i, j]
                        res["cross_softmax"][b, h // G, j] += weights[b, h, i, j]
    return res
