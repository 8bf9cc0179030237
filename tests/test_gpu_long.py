"""A score matrix past 2 GiB in one head.  The buffer descriptors of both
score writers are based per row block, so only a row block's span needs
32-bit offsets; one head at M = N = 40000 (3.2 GB of fp16 scores, rows past
2^31 bytes from the head's first element) checks that, at the first, a
middle and the last rows against the oracle computed for those rows alone
(the reference's own int32 element arithmetic stops at 2^31 elements per
head, attention_with_scores.py:71, 112)."""
from __future__ import annotations

import pytest
import torch

import flash_attn_with_score_amd as fas
from flash_attn_with_score_amd.attention_scores import compute_attention_scores
from oracle import inputs, naive
from tests.tolerances import assert_out_close, assert_scores_close

pytestmark = pytest.mark.gpu

M = N = 40000
D = 64
ROWS = (0, M // 2 + 7, M - 64)


def test_fused_scores_past_2gib_per_head(gpu):
    print(f"[case] attention_with_scores B1 H1 M{M} N{N} D{D} causal", flush=True)
    q, k, v = inputs.make_qkv(1, 1, 1, M, N, D, dtype=torch.float16, seed=21, device=gpu)
    o, s = fas.attention_with_scores(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert s.shape == (1, 1, M, N) and s.numel() * 2 > 2**31
    for i0 in ROWS:
        ref = naive.reference_forward(q[:, :, i0:i0 + 64], k, v, causal=True, causal_offset=i0,
                                      want=("out", "scores"))
        assert_out_close(o[:, :, i0:i0 + 64], ref["out"])
        assert_scores_close(s[:, :, i0:i0 + 64], ref["scores"])


def test_scores_only_past_2gib_per_head(gpu):
    print(f"[case] compute_attention_scores B1 H1 M{M} N{N} D{D}", flush=True)
    q, k, _ = inputs.make_qkv(1, 1, 1, M, N, D, dtype=torch.float16, seed=22, device=gpu)
    s = compute_attention_scores(q, k)
    torch.cuda.synchronize()
    for i0 in ROWS:
        ref = naive.reference_forward(q[:, :, i0:i0 + 64], k, k, causal=False,
                                      want=("scores",))["scores"]
        assert_out_close(s[:, :, i0:i0 + 64], ref, "scores")
