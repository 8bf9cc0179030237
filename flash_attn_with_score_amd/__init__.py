"""Fused flash-attention-forward family for MI355X (gfx950).

Drop-in replacements for the Python entry points of the reference's package
(__init__.py:6-39): each returns (output, side product) from one call into a
hand-written HIP kernel through the C ABI in include/fas.h.  `attention`
(flash.py) adds the FlashAttention-2 backward pass; `total.total_attention`
mirrors the reference's total.py.
"""
from .attention_with_scores import attention_with_scores
from .flash import attention
from .attention_with_col_sum import attention_with_col_sum
from .attention_with_col_sum_sequential import attention_with_col_sum_sequential
from .attention_with_col_softmax_sum import attention_with_softmax_col_sum
from .attention_cross_token_softmax_sum import (
    attention_cross_token_softmax_sum,
    attention_cross_token_softmax_sum_buffered,
)
from .attention_with_row_sum import attention_with_row_sum
from .attention_cross_token_qk_sum import attention_cross_token_qk_sum

__all__ = [
    "attention",
    "attention_with_scores",
    "attention_with_col_sum",
    "attention_with_col_sum_sequential",
    "attention_with_softmax_col_sum",
    "attention_cross_token_softmax_sum",
    "attention_cross_token_softmax_sum_buffered",
    "attention_with_row_sum",
    "attention_cross_token_qk_sum",
]
