"""attention_with_row_sum: attention output plus per-query score sums.

Drop-in for the reference's attention_with_row_sum.py:204-326.
"""
from __future__ import annotations

import ctypes

import torch

from . import _common, _native


def attention_with_row_sum(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    sm_scale: float = None,
    dropout_p: float = 0.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (output, row_sum), row_sum (B, Hq, M) fp32 holding the sum over
    admissible keys of (q . k) * sm_scale (attention_with_row_sum.py:144-156).
    Query rows with no admissible key get 0 (:181-185)."""
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
    # Every element is written by the kernels (rows with no admissible key get
    # 0, attention_with_row_sum.py:185), so no zero-fill is needed.
    row_sum = torch.empty((B, H, M), device=q.device, dtype=torch.float32)
    args = _native.make_args(p.q, p.k, p.v, o, causal, p.sm_scale,
                             _common.draw_dropout(p.q, p.k, dropout_p))
    ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_ROW_SUM, args, 0, q.device)
    _common.call("fas_attention_with_row_sum", p.q, ctypes.byref(args), row_sum.data_ptr(),
                 _native.strides3(row_sum), ws_ptr, ws_bytes)
    return o, row_sum
