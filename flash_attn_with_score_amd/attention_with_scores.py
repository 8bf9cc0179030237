"""attention_with_scores: attention output plus the full score matrix.

Drop-in for the reference's attention_with_scores.py:214-333.  The gfx950
kernel writes every element of the (B, H, M, N) matrix itself, including the
causal upper triangle as zeros, so the score tensor is allocated with
torch.empty rather than zero-filled as the reference does (:284).
"""
from __future__ import annotations

import ctypes

import torch

from . import _common, _native


def attention_with_scores(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    sm_scale: float = None,
    dropout_p: float = 0.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Attention output and scores from one fused kernel.

    Args mirror attention_with_scores.py:214-237.  Returns
    (output (B, Hq, M, D), scores (B, Hq, M, N) in q.dtype), where scores
    hold (q . k) * sm_scale and causally masked positions are 0.
    """
    Dq, Dk, Dv = q.shape[-1], k.shape[-1], v.shape[-1]
    assert Dq == Dk == Dv, "feature size of q, k, v should be equal"
    assert Dk in {16, 32, 64, 128}

    B, H, M, D = q.shape
    N = k.shape[2]
    Hk, Hv = k.shape[1], v.shape[1]
    assert Hk == Hv, "num of heads in k and v should be equal"
    assert H % Hk == 0, "number of heads in q must be a multiple of that in k & v"

    _common.check_device_inputs(q, k, v, dropout_p)
    p = _common.finish_problem(q, k, v, sm_scale)
    o = _common.new_output(p.q)
    scores = torch.empty((B, H, M, N), device=q.device, dtype=q.dtype)
    args = _native.make_args(p.q, p.k, p.v, o, causal, p.sm_scale,
                             _common.draw_dropout(p.q, p.k, dropout_p))
    ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_SCORES, args, 0, q.device)
    _common.call("fas_attention_with_scores", p.q, ctypes.byref(args), scores.data_ptr(),
                 _native.strides4(scores), ws_ptr, ws_bytes)
    return o, scores
