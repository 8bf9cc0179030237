"""compute_attention_scores: the attention scores alone.

Drop-in for the reference's attention_scores.py:154-223: scores
(B, Hq, M, N) = (q @ k^T) * sm_scale in q's dtype, GQA by query-head groups,
with no mask (the reference accepts `causal` and ignores it).  One call into
the scores-only gfx950 kernel through fas_attention_scores.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _common, _native

__all__ = ["compute_attention_scores"]


def compute_attention_scores(
    q: torch.Tensor,
    k: torch.Tensor,
    causal: bool = False,
    sm_scale: float = None,
) -> torch.Tensor:
    Dq, Dk = q.shape[-1], k.shape[-1]
    assert Dq == Dk, "Q and K must have the same head_dim"
    assert Dk in {16, 32, 64, 128}, f"head_dim must be one of 16, 32, 64, 128, got {Dk}"
    B, H, M, D = q.shape
    N = k.shape[2]
    Hk = k.shape[1]
    assert H % Hk == 0, "num_heads_q must be a multiple of num_heads_k (GQA support)"
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    assert q.dtype in _native.DTYPE_CODES and k.dtype == q.dtype, "q, k must be fp16 or bf16"
    if not (q.is_cuda and k.is_cuda):
        raise RuntimeError("flash_attn_with_score_amd: q, k must be HIP device tensors")
    q, k = _common.as_kernel_operand(q), _common.as_kernel_operand(k)
    scores = torch.empty((B, H, M, N), dtype=q.dtype, device=q.device)
    # causal is accepted and ignored, as in the reference (attention_scores.py:166).
    args = _native.make_args(q, k, k, q, False, float(sm_scale))
    _common.call("fas_attention_scores", q, ctypes.byref(args), scores.data_ptr(),
                 _native.strides4(scores))
    return scores
