"""total_attention: per-key sums of the softmax weights from a saved normalizer.

Drop-in for the reference's total.py:9-48 (+ _total_attention_kernel
:51-143): given q, k and the natural-log normalizer l that attention()
returns, tot[b, h, j] = sum over query rows i of exp(q_i . k_j * sm_scale -
l[b, h, i]) over the admissible pairs (bottom-right causal mask when causal).
Runs the key-outer column-pass kernel of the softmax column sums, per query
head.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _common, _native

__all__ = ["total_attention"]


def total_attention(q, k, l, causal=False, sm_scale=None):
    Dq, Dk = q.shape[-1], k.shape[-1]
    assert Dq == Dk
    assert Dk in {16, 32, 64, 128}
    B, H, M, D = q.shape
    N = k.shape[2]
    Hk = k.shape[1]
    assert H % Hk == 0, "number of heads in q must be a multiple of that in k"
    if sm_scale is None:
        sm_scale = 1. / math.sqrt(D)
    assert q.dtype in _native.DTYPE_CODES and k.dtype == q.dtype, "q, k must be fp16 or bf16"
    if not (q.is_cuda and k.is_cuda and l.is_cuda):
        raise RuntimeError("flash_attn_with_score_amd: q, k, l must be HIP device tensors")
    assert l.dtype == torch.float32 and tuple(l.shape) == (B, H, M), "l must be (B, H, M) fp32"
    q, k = _common.as_kernel_operand(q), _common.as_kernel_operand(k)
    tot = torch.empty((B, H, N), dtype=torch.float32, device=q.device)
    args = _native.make_args(q, k, k, q, causal, float(sm_scale))
    _common.call("fas_total_attention", q, ctypes.byref(args), l.data_ptr(), _native.strides3(l),
                 tot.data_ptr(), _native.strides3(tot))
    return tot
