"""attention_cross_token_qk_sum: attention output plus cross-segment sums of
raw scores.

Drop-in for the reference's attention_cross_token_qk_sum.py:255-408.  Its
causal mask is top-left aligned (query i sees keys j <= i, :89, :138) for
both the output and the sums, unlike the other entry points.
"""
from __future__ import annotations

import ctypes

import torch

from . import _common, _native


def attention_cross_token_qk_sum(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    split: int,
    causal: bool = False,
    sm_scale: float = None,
    dropout_p: float = 0.0,
    *,
    out: torch.Tensor | None = None,
    cross_token_qk_out: torch.Tensor | None = None,
    reuse_buffers: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (output, cross_token_qk), cross_token_qk (B, Hk, split) fp32:
    cross_token_qk[b, hk, j] = sum over queries i in [split, M) and the query
    heads of group hk of masked (q_i . k_j) * sm_scale, for j < split.

    out / cross_token_qk_out are optional caller buffers, validated as in
    attention_cross_token_qk_sum.py:341-357.  The kernels overwrite every
    (B, Hk, split) element of cross_token_qk_out, so unlike the reference
    (:363) it is not zeroed first and its prior contents do not matter.
    reuse_buffers is accepted and unused, as in the reference.
    """
    Dq, Dk, Dv = q.shape[-1], k.shape[-1], v.shape[-1]
    assert Dq == Dk == Dv, "Feature dimensions of q, k, v must be equal"
    assert Dk in {16, 32, 64, 128}, f"Unsupported head_dim: {Dk}"

    B, H, M, D = q.shape
    N = k.shape[2]
    Hk, Hv = k.shape[1], v.shape[1]

    assert Hk == Hv, "Number of heads in k and v must be equal"
    assert H % Hk == 0, "Number of heads in q must be a multiple of that in k"
    assert 0 < split <= N, f"Split position must be within valid range (0, {N}]"

    _common.check_device_inputs(q, k, v, dropout_p)
    p = _common.finish_problem(q, k, v, sm_scale)

    if out is not None:
        o = out
        assert o.shape == q.shape, f"out.shape must equal q.shape, current out={o.shape}, q={q.shape}"
        assert o.device == q.device, "out.device must match q.device"
        assert o.dtype == q.dtype, "out.dtype must match q.dtype"
    else:
        o = _common.new_output(p.q)

    if cross_token_qk_out is not None:
        cross_token_qk = cross_token_qk_out
        assert cross_token_qk.shape == (B, Hk, split), (
            f"cross_token_qk_out.shape must be {(B, Hk, split)}, current is {cross_token_qk.shape}"
        )
        assert cross_token_qk.device == q.device, "cross_token_qk_out.device must match q.device"
        assert cross_token_qk.dtype == torch.float32, "cross_token_qk_out.dtype must be torch.float32"
    else:
        cross_token_qk = torch.empty((B, Hk, split), device=q.device, dtype=torch.float32)

    # A caller buffer the kernel cannot write directly (innermost stride != 1
    # or unaligned rows) is filled through a temporary.
    o_k = o if (o.stride(-1) == 1 and _common._rows_aligned(o)) else _common.new_output(p.q)
    args = _native.make_args(p.q, p.k, p.v, o_k, causal, p.sm_scale,
                             _common.draw_dropout(p.q, p.k, dropout_p))
    ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_CROSS_QK_SUM, args, split, q.device)
    _common.call("fas_attention_cross_token_qk_sum", p.q, ctypes.byref(args), int(split),
                 cross_token_qk.data_ptr(), _native.strides3(cross_token_qk), ws_ptr, ws_bytes)
    if o_k is not o:
        o.copy_(o_k)
    return o, cross_token_qk
