"""Every output element is written by the kernels.

The launchers allocate outputs and workspace with torch.empty, so a kernel
that skipped some elements could still pass a parity test whenever the
caching allocator hands back stale but plausible memory.  Here each entry
point is called through the C ABI (ctypes, as flash_attn_with_score_amd/
_native.py binds it) with the output, the side product and the workspace
pre-filled with NaN (all-ones bytes), and the results must be NaN-free and
match the oracle.  The cases cover the key-split route (short query range,
fp32 partials in the workspace), causal M > N (rows with no admissible key)
and N % 8 != 0 (the element-wise score path and its zero triangle).
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from flash_attn_with_score_amd import _native
from oracle import inputs, naive
from tests.tolerances import assert_out_close, assert_scores_close, assert_sum_close

pytestmark = pytest.mark.gpu

# (B, Hq, Hk, M, N, D)
CASES = [
    (1, 4, 2, 32, 2048, 128),   # key split: 1 row block, 32 tiles
    (1, 2, 2, 600, 512, 32),    # causal M > N: 88 empty rows
    (1, 3, 1, 100, 77, 64),     # N % 8 != 0: element-wise scores, GQA 3
    (2, 4, 4, 256, 256, 16),
]

# entry point -> (variant, oracle side product, takes split, side shape fn)
SIDE = {
    "fas_attention_with_scores": (_native.VARIANT_SCORES, "scores", False),
    "fas_attention_with_row_sum": (_native.VARIANT_ROW_SUM, "row_sum", False),
    "fas_attention_with_col_sum": (_native.VARIANT_COL_SUM, "col_sum", False),
    "fas_attention_with_col_sum_sequential": (_native.VARIANT_COL_SUM_SEQUENTIAL, "col_sum", False),
    "fas_attention_with_softmax_col_sum": (_native.VARIANT_SOFTMAX_COL_SUM, "col_softmax", False),
    "fas_attention_cross_token_qk_sum": (_native.VARIANT_CROSS_QK_SUM, "cross_qk", True),
    "fas_attention_cross_token_softmax_sum": (_native.VARIANT_CROSS_SOFTMAX_SUM, "cross_softmax",
                                              True),
    "fas_attention_cross_token_softmax_sum_buffered": (
        _native.VARIANT_CROSS_SOFTMAX_SUM_BUFFERED, "cross_softmax", True),
}


def _nan(shape, dtype, dev):
    return torch.full(shape, float("nan"), dtype=dtype, device=dev)


@pytest.mark.parametrize("shape", CASES, ids=lambda s: "B{}H{}K{}M{}N{}D{}".format(*s))
@pytest.mark.parametrize("fn_name", sorted(SIDE))
def test_outputs_fully_written(fn_name, shape, gpu):
    B, Hq, Hk, M, N, D = shape
    variant, side, has_split = SIDE[fn_name]
    split = max(1, min(M, N) // 2) if has_split else 0
    print(f"[case] poison {fn_name} B{B}H{Hq}K{Hk}M{M}N{N}D{D} split={split}", flush=True)
    lib = _native.load()
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=torch.float16, seed=21)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    o = _nan((B, Hq, M, D), torch.float16, gpu)
    args = _native.make_args(qd, kd, vd, o, True, D ** -0.5)
    nbytes = lib.fas_workspace_bytes(variant, ctypes.byref(args), split)
    assert nbytes != ctypes.c_size_t(-1).value
    ws = torch.full((nbytes + 256,), 0xFF, dtype=torch.uint8, device=gpu)
    wptr = ws.data_ptr() + (-ws.data_ptr()) % 256
    stream = torch.cuda.current_stream().cuda_stream
    fn = getattr(lib, fn_name)
    if side == "scores":
        extra = _nan((B, Hq, M, N), torch.float16, gpu)
        rc = fn(ctypes.byref(args), extra.data_ptr(), _native.strides4(extra), wptr, nbytes, stream)
    else:
        ncols = {"row_sum": M, "cross_qk": split, "cross_softmax": split}.get(side, N)
        heads = Hq if side == "row_sum" else Hk
        extra = _nan((B, heads, ncols), torch.float32, gpu)
        if has_split:
            rc = fn(ctypes.byref(args), split, extra.data_ptr(), _native.strides3(extra), wptr,
                    nbytes, stream)
        else:
            rc = fn(ctypes.byref(args), extra.data_ptr(), _native.strides3(extra), wptr, nbytes,
                    stream)
    _native.check(lib, rc, fn_name)
    torch.cuda.synchronize()
    assert not torch.isnan(o).any(), f"{fn_name}: output elements left unwritten"
    assert not torch.isnan(extra).any(), f"{fn_name}: side-product elements left unwritten"
    ep = fn_name[len("fas_"):]
    ref = naive.reference_forward(q, k, v, causal=True,
                                  causal_offset=naive.ENTRY_POINT_OFFSET[ep],
                                  split=split if has_split else None, want=("out", side))
    assert_out_close(o, ref["out"])
    if side == "scores":
        assert_scores_close(extra, ref["scores"])
    else:
        assert_sum_close(extra, ref[side], side)
