"""attention_with_softmax_col_sum: attention output plus per-key sums of the
softmax weights.

Drop-in for the reference's attention_with_col_softmax_sum.py:274-401.  Two
passes over K: pass 1 is the online-softmax forward (O, row max m, row sum
l); pass 2 recomputes q . k and accumulates P = exp(s - m) / l per key.
Pass 2 visits key tiles in reverse order when causal.
"""
from __future__ import annotations

import ctypes

import torch

from . import _common, _native


def attention_with_softmax_col_sum(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    sm_scale: float = None,
    dropout_p: float = 0.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (output, col_sum), col_sum (B, Hk, N) fp32: for each key the
    sum over queries and group heads of the final softmax weights
    (attention_with_col_softmax_sum.py:224-270)."""
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
    col_sum = torch.empty((B, Hk, N), device=q.device, dtype=torch.float32)
    args = _native.make_args(p.q, p.k, p.v, o, causal, p.sm_scale,
                             _common.draw_dropout(p.q, p.k, dropout_p))
    ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_SOFTMAX_COL_SUM, args, 0, q.device)
    _common.call("fas_attention_with_softmax_col_sum", p.q, ctypes.byref(args), col_sum.data_ptr(),
                 _native.strides3(col_sum), ws_ptr, ws_bytes)
    return o, col_sum
