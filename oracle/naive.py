"""CPU oracle for the fused attention family -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker (or the timed CPU baseline); the product
path never imports it.

It restates, in fp32 on the CPU, the reference's naive attention
(reference_implementations.py:11-52: GQA by repeat_interleave, scores =
(q @ k^T) * sm_scale, causal mask -> -inf, softmax over keys, P @ v) and the
harness's side-product formulas:

  row sum        benchmark.py:1526-1534   masked scores (-inf -> 0) summed over keys
  column sum     benchmark.py:1573-1581   ... summed over queries; folded over the
                                          query heads of each KV group as the
                                          kernels return it (attention_with_col_sum.py:72,370)
  softmax col    attention_with_col_softmax_sum.py:224-270  softmax weights summed
                                          over queries, folded per KV group
  cross softmax  benchmark.py:1619-1646   softmax weights [split:, :split] summed
                                          over queries, folded (eps 1e-12 of
                                          attention_cross_token_softmax_sum.py:238
                                          is below fp32 resolution for l >= 1)
  cross qk       benchmark.py:1684-1693   masked scores [split:, :split] summed
                                          over queries, folded

Causal alignment.  The naive reference masks torch.triu(ones(M, N), 1), i.e.
keeps j <= i (top-left).  The kernels keep (N - M) + i >= j (bottom-right,
attention_with_scores.py:136) except the cross-token QK sum, which keeps
j <= i (attention_cross_token_qk_sum.py:138).  The two agree when M == N;
`causal_offset` selects the alignment (0 = top-left = naive reference).
Rows with no admissible key (bottom-right, M > N) give output 0 and zero
sums, as the kernels do (attention_with_scores.py:192-195).

Work is streamed per (batch, head) and per chunk of query rows so the
largest configurations fit in host memory; per-chunk partial sums are
accumulated in fp64.

attention_reference restates attention() (flash.py:32-297) in fp64: the
output, the natural-log normalizer L = m * sm_scale + ln(l) (flash.py:477-483,
-inf for rows with no admissible key), the per-query-head total attention
(total.py:120-136) and, given dO, the gradients the backward kernels compute
(flash.py:172-261), by torch autograd with dK and dV summed over each KV
head's query-head group (flash.py:258-259).
"""
from __future__ import annotations

import math
from typing import Iterable

import numpy as np
import torch

from . import philox

ALL_OUTPUTS = ("out", "scores", "row_sum", "col_sum", "col_softmax", "cross_qk", "cross_softmax")


def naive_attention_with_scores(q, k, v, causal, dropout_p=0.0, sm_scale=None):
    """fp32 CPU restatement of reference_implementations.py:11-52.

    Returns (output, scores) with masked scores set to -inf; causal masking
    is top-left aligned exactly as the reference's triu(..., diagonal=1).
    """
    if dropout_p > 0.0:
        raise NotImplementedError("the oracle has no dropout")
    q, k, v = (t.detach().to("cpu", torch.float32) for t in (q, k, v))
    B, Hq, M, D = q.shape
    Hk = k.shape[1]
    if Hq != Hk:
        assert Hq % Hk == 0
        groups = Hq // Hk
        k = torch.repeat_interleave(k, repeats=groups, dim=1)
        v = torch.repeat_interleave(v, repeats=groups, dim=1)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    scores = torch.matmul(q, k.transpose(-2, -1)) * sm_scale
    if causal:
        N = k.shape[-2]
        mask = torch.triu(torch.ones(M, N, dtype=torch.bool), diagonal=1)
        scores = scores.masked_fill(mask, float("-inf"))
    weights = torch.softmax(scores, dim=-1)
    return torch.matmul(weights, v), scores


def admissible_mask(i0: int, i1: int, N: int, causal: bool, causal_offset: int) -> torch.Tensor:
    """Boolean (i1 - i0, N) mask of admissible (query, key) pairs."""
    if not causal:
        return torch.ones(i1 - i0, N, dtype=torch.bool)
    rows = torch.arange(i0, i1).unsqueeze(1)
    cols = torch.arange(N).unsqueeze(0)
    return causal_offset + rows >= cols


def reference_forward(q, k, v, *, causal: bool, sm_scale: float | None = None,
                      causal_offset: int | None = None, split: int | None = None,
                      want: Iterable[str] = ALL_OUTPUTS, chunk: int = 1024,
                      heads: Iterable[int] | None = None, dropout=None,
                      drop_scale: float = 1.0, drop_col_softmax: bool = False) -> dict:
    """Streams the oracle over (batch, query head, row chunk).

    q: (B, Hq, M, D); k, v: (B, Hk, N, D), any dtype/device (converted to
    fp32 on the CPU).  causal_offset defaults to N - M (bottom-right).
    `heads` restricts the work to some query heads (used for bounded CPU
    timing); outputs of other heads stay zero.  Returns a dict with the
    requested entries of ALL_OUTPUTS:
      out (B,Hq,M,D) fp32, scores (B,Hq,M,N) fp32 with -inf at masked pairs,
      row_sum (B,Hq,M), col_sum / col_softmax (B,Hk,N),
      cross_qk / cross_softmax (B,Hk,split).
    dropout = (p, seed, offset) drops weight (b, h, i, j) from O (and from the
    softmax column sum when drop_col_softmax) unless oracle.philox.keep_mask
    keeps it; the row normaliser sums the weights before dropout, and O is
    multiplied by drop_scale (attention_with_scores.py:165-203).
    """
    want = set(want)
    unknown = want - set(ALL_OUTPUTS)
    if unknown:
        raise ValueError(f"unknown outputs {sorted(unknown)}")
    q, k, v = (t.detach().to("cpu", torch.float32) for t in (q, k, v))
    B, Hq, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    assert Hq % Hk == 0
    G = Hq // Hk
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if causal_offset is None:
        causal_offset = N - M
    if want & {"cross_qk", "cross_softmax"}:
        assert split is not None and 0 < split <= N

    res = {}
    if "out" in want:
        res["out"] = torch.zeros(B, Hq, M, D, dtype=torch.float32)
    if "scores" in want:
        res["scores"] = torch.empty(B, Hq, M, N, dtype=torch.float32)
    if "row_sum" in want:
        res["row_sum"] = torch.zeros(B, Hq, M, dtype=torch.float32)
    for name in ("col_sum", "col_softmax"):
        if name in want:
            res[name] = torch.zeros(B, Hk, N, dtype=torch.float64)
    for name in ("cross_qk", "cross_softmax"):
        if name in want:
            res[name] = torch.zeros(B, Hk, split, dtype=torch.float64)

    head_list = range(Hq) if heads is None else list(heads)
    for b in range(B):
        for h in head_list:
            hk = h // G
            kh, vh = k[b, hk], v[b, hk]
            for i0 in range(0, M, chunk):
                i1 = min(M, i0 + chunk)
                s = torch.matmul(q[b, h, i0:i1], kh.transpose(0, 1)) * sm_scale
                keep = admissible_mask(i0, i1, N, causal, causal_offset)
                s = s.masked_fill(~keep, float("-inf"))
                if "scores" in want:
                    res["scores"][b, h, i0:i1] = s
                s0 = torch.where(keep, s, torch.zeros((), dtype=s.dtype))
                need_p = bool(want & {"out", "col_softmax", "cross_softmax"})
                if need_p:
                    p = torch.softmax(s, dim=-1)
                    p = torch.nan_to_num(p, nan=0.0)  # rows with no admissible key
                pd = p if need_p else None
                if need_p and dropout is not None:
                    kept = philox.keep_mask(dropout[1], dropout[2], dropout[0], b, h,
                                            range(i0, i1), N, Hq, M)
                    pd = p * torch.from_numpy(kept)
                if "out" in want:
                    res["out"][b, h, i0:i1] = torch.matmul(pd, vh) * drop_scale
                if "row_sum" in want:
                    res["row_sum"][b, h, i0:i1] = s0.sum(dim=-1)
                if "col_sum" in want:
                    res["col_sum"][b, hk] += s0.sum(dim=0, dtype=torch.float64)
                if "col_softmax" in want:
                    pc = pd if drop_col_softmax else p
                    res["col_softmax"][b, hk] += pc.sum(dim=0, dtype=torch.float64)
                r0 = max(i0, split) if split is not None else i1
                if r0 < i1:
                    if "cross_qk" in want:
                        res["cross_qk"][b, hk] += s0[r0 - i0:, :split].sum(dim=0, dtype=torch.float64)
                    if "cross_softmax" in want:
                        res["cross_softmax"][b, hk] += p[r0 - i0:, :split].sum(dim=0, dtype=torch.float64)
    for name in ("col_sum", "col_softmax", "cross_qk", "cross_softmax"):
        if name in res:
            res[name] = res[name].to(torch.float32)
    return res


def scores_as_returned(scores: torch.Tensor) -> torch.Tensor:
    """The score tensor as the kernels return it: masked (-inf) -> 0
    (attention_with_scores.py:141-148)."""
    return torch.where(torch.isinf(scores) & (scores < 0), torch.zeros((), dtype=scores.dtype), scores)


# Which causal alignment each entry point uses (0 = top-left, None = N - M).
ENTRY_POINT_OFFSET = {
    "attention_with_scores": None,
    "attention_with_row_sum": None,
    "attention_with_col_sum": None,
    "attention_with_col_sum_sequential": None,
    "attention_with_softmax_col_sum": None,
    "attention_cross_token_qk_sum": 0,
    "attention_cross_token_softmax_sum": None,
    "attention_cross_token_softmax_sum_buffered": None,
}

# The side product each entry point returns, as named in reference_forward.
ENTRY_POINT_OUTPUT = {
    "attention_with_scores": "scores",
    "attention_with_row_sum": "row_sum",
    "attention_with_col_sum": "col_sum",
    "attention_with_col_sum_sequential": "col_sum",
    "attention_with_softmax_col_sum": "col_softmax",
    "attention_cross_token_qk_sum": "cross_qk",
    "attention_cross_token_softmax_sum": "cross_softmax",
    "attention_cross_token_softmax_sum_buffered": "cross_softmax",
}


# Entry points whose O is rescaled by 1/(1 - p) under dropout
# (attention_with_scores.py:200-203; flash.py:488-491); the others are not.
DROPOUT_RESCALES = {"attention_with_scores", "attention"}


def dropout_scale(p: float) -> float:
    """1.0 / (1.0 - p) as the reference's kernels compute it, in fp32."""
    return float(np.float32(1.0) / (np.float32(1.0) - np.float32(p)))


def oracle_for(entry_point: str, q, k, v, *, causal: bool, sm_scale=None, split=None,
               chunk: int = 1024, dropout=None) -> tuple[torch.Tensor, torch.Tensor]:
    """(out, side product) the named entry point must reproduce; dropout is
    None or (p, seed, offset) as the launch drew it.  The buffered cross
    softmax sum ignores dropout (attention_cross_token_softmax_sum.py:639-732).
    For rows with no admissible key (M > N, causal) the buffered entry point is
    held to the fused kernel's convention, output 0
    (attention_cross_token_softmax_sum.py:182-184): the reference's buffered
    kernel writes acc * (1 / l_i) with l_i = 0 there (:498-503, :630), NaN,
    a deviation this build makes on purpose.  Its sums mask those rows in
    both kernels (:609-620), so the side product is the same either way."""
    side = ENTRY_POINT_OUTPUT[entry_point]
    if entry_point == "attention_cross_token_softmax_sum_buffered":
        dropout = None
    scale = dropout_scale(dropout[0]) if dropout and entry_point in DROPOUT_RESCALES else 1.0
    res = reference_forward(q, k, v, causal=causal, sm_scale=sm_scale,
                            causal_offset=ENTRY_POINT_OFFSET[entry_point], split=split,
                            want=("out", side), chunk=chunk, dropout=dropout,
                            drop_scale=scale,
                            drop_col_softmax=entry_point == "attention_with_softmax_col_sum")
    out, extra = res["out"], res[side]
    if side == "scores":
        extra = scores_as_returned(extra)
    return out, extra


def attention_reference(q, k, v, do=None, *, causal: bool, sm_scale: float | None = None,
                        causal_offset: int | None = None, dropout=None) -> dict:
    """fp64 CPU restatement of attention() and its backward pass.

    Returns out (B,Hq,M,D), lse (B,Hq,M) and total (B,Hq,N) and, when do
    (shaped like out) is given, dq (like q), dk and dv (like k): the
    gradients of sum(out * do).  causal_offset defaults to N - M
    (bottom-right, flash.py:447).  dropout = (p, seed, offset): out uses the
    weights times the keep mask of oracle.philox.keep_mask and 1/(1-p)
    (flash.py:459-466, 488-491); lse and total are the undropped ones.
    """
    q, k, v = (t.detach().to("cpu", torch.float64) for t in (q, k, v))
    B, Hq, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    assert Hq % Hk == 0
    G = Hq // Hk
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if causal_offset is None:
        causal_offset = N - M
    keep = admissible_mask(0, M, N, causal, causal_offset)
    has_key = keep.any(dim=1)
    # Rows with no admissible key use every key in the exponent (finite
    # values, so autograd stays NaN-free) and are zeroed afterwards.
    use = keep | ~has_key.unsqueeze(1)
    res = {
        "out": torch.zeros(B, Hq, M, D, dtype=torch.float64),
        "lse": torch.full((B, Hq, M), float("-inf"), dtype=torch.float64),
        "total": torch.zeros(B, Hq, N, dtype=torch.float64),
    }
    grads = do is not None
    if grads:
        do = do.detach().to("cpu", torch.float64)
        res["dq"] = torch.zeros_like(q)
        res["dk"] = torch.zeros_like(k)
        res["dv"] = torch.zeros_like(v)
    row_has = has_key.to(torch.float64).unsqueeze(1)
    for b in range(B):
        for hk in range(Hk):
            hs = slice(hk * G, (hk + 1) * G)
            qg = q[b, hs].clone().requires_grad_(grads)
            kk = k[b, hk].clone().requires_grad_(grads)
            vv = v[b, hk].clone().requires_grad_(grads)
            s = torch.matmul(qg, kk.transpose(0, 1)) * sm_scale
            s = s.masked_fill(~use, float("-inf"))
            lse = torch.logsumexp(s, dim=-1, keepdim=True)
            p = torch.exp(s - lse) * row_has
            pd = p
            if dropout is not None:
                z = np.stack([philox.keep_mask(dropout[1], dropout[2], dropout[0], b, h,
                                               range(M), N, Hq, M)
                              for h in range(hk * G, (hk + 1) * G)])
                pd = p * torch.from_numpy(z).to(torch.float64) * dropout_scale(dropout[0])
            o = torch.matmul(pd, vv)
            res["out"][b, hs] = o.detach()
            res["lse"][b, hs] = torch.where(has_key, lse.detach().squeeze(-1),
                                            torch.full((), float("-inf"), dtype=torch.float64))
            res["total"][b, hs] = p.detach().sum(dim=1)
            if grads:
                gq, gk, gv = torch.autograd.grad(o, (qg, kk, vv), do[b, hs])
                res["dq"][b, hs] = gq
                res["dk"][b, hk] = gk
                res["dv"][b, hk] = gv
    return res
