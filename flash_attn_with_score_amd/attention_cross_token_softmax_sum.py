"""Cross-token softmax-weight sums, recomputing and buffered variants.

Drop-ins for the reference's attention_cross_token_softmax_sum.py:735-863
(attention_cross_token_softmax_sum, fused two-pass kernel :24-268) and
:639-732 (attention_cross_token_softmax_sum_buffered, kernel :434-636).
"""
from __future__ import annotations

import ctypes

import torch

from . import _common, _native

__all__ = ["attention_cross_token_softmax_sum", "attention_cross_token_softmax_sum_buffered"]


def attention_cross_token_softmax_sum_buffered(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    split: int,
    causal: bool = False,
    sm_scale: float = None,
    dropout_p: float = 0.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Same result as attention_cross_token_softmax_sum; pass 1 stores the
    scores of the region (queries >= split, keys < split) in a scratch buffer
    and pass 2 reloads them instead of recomputing q . k.

    The scratch holds only the region (the only part ever re-read; the
    reference allocates B * Hq * M * N * 4 bytes of raw fp32 scores,
    :704-705), each score as an fp16 base-2 exponent relative to its row's
    maximum over the region keys of its 64-key tile, plus those maxima:
    B * Hq * max(M - split, 0) * (split * 2 + ceil(split / 64) * 4) bytes.
    """
    Dq, Dk, Dv = q.shape[-1], k.shape[-1], v.shape[-1]
    assert Dq == Dk == Dv, "Q, K, V must have the same head_dim"
    assert Dk in {16, 32, 64, 128}

    B, H, M, D = q.shape
    N = k.shape[2]
    Hk = k.shape[1]
    Hv = v.shape[1]
    assert Hk == Hv, "K and V must have the same number of heads"
    assert H % Hk == 0, "num_heads_q must be divisible by num_heads_k"

    assert 0 < split <= N, f"Split position must be in valid range (0, {N}]"

    _common.check_device_inputs(q, k, v, dropout_p)
    p = _common.finish_problem(q, k, v, sm_scale)
    output = _common.new_output(p.q)
    cross = torch.empty((B, Hk, split), device=q.device, dtype=torch.float32)
    # The reference's buffered kernel ignores dropout_p and draws no seed.
    args = _native.make_args(p.q, p.k, p.v, output, causal, p.sm_scale)
    ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_CROSS_SOFTMAX_SUM_BUFFERED, args, split,
                                             q.device)
    _common.call("fas_attention_cross_token_softmax_sum_buffered", p.q, ctypes.byref(args),
                 int(split), cross.data_ptr(), _native.strides3(cross), ws_ptr, ws_bytes)
    return output, cross


def attention_cross_token_softmax_sum(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    split: int,
    causal: bool = False,
    sm_scale: float = None,
    dropout_p: float = 0.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (output, cross_token_softmax_sum (B, Hk, split) fp32) with
    sum[b, hk, j] = sum over queries i in [split, M) and the query heads of
    group hk of exp(s_ij - m_i) / (l_i + 1e-12), for keys j < split
    (attention_cross_token_softmax_sum.py:236-268)."""
    Dq, Dk, Dv = q.shape[-1], k.shape[-1], v.shape[-1]
    assert Dq == Dk == Dv, "Q, K, V must have the same head_dim"
    assert Dk in {16, 32, 64, 128}

    B, H, M, D = q.shape
    N = k.shape[2]
    Hk = k.shape[1]
    assert Hk == v.shape[1]
    assert H % Hk == 0

    assert 0 < split <= N, f"Split position must be in valid range (0, {N}]"

    _common.check_device_inputs(q, k, v, dropout_p)
    p = _common.finish_problem(q, k, v, sm_scale)
    output = _common.new_output(p.q)
    cross = torch.empty((B, Hk, split), device=q.device, dtype=torch.float32)
    args = _native.make_args(p.q, p.k, p.v, output, causal, p.sm_scale,
                             _common.draw_dropout(p.q, p.k, dropout_p))
    ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_CROSS_SOFTMAX_SUM, args, split,
                                             q.device)
    _common.call("fas_attention_cross_token_softmax_sum", p.q, ctypes.byref(args), int(split),
                 cross.data_ptr(), _native.strides3(cross), ws_ptr, ws_bytes)
    return output, cross
