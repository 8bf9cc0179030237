"""fas_attention_with_softmax_col_sum_noalloc against the allocating entry
point it mirrors.

The no-allocation entry point takes its workspace from the library's
file-scope device array (64 MiB per GPU) instead of a caller buffer.  It is
called through the C ABI and compared with fas_attention_with_softmax_col_sum
(workspace from torch) under the parity criteria: two calls in a row, the
second with a smaller problem, so stale contents of the shared array from the
first call must not leak into the second.  Also: an oversized problem is
rejected with FAS_ERR_WORKSPACE and a message, before any launch.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from flash_attn_with_score_amd import _native
from oracle import inputs
from tests.tolerances import assert_out_close, assert_sum_close

pytestmark = pytest.mark.gpu


def _call_both(lib, shape, dtype, causal, gpu, seed):
    B, Hq, Hk, M, N, D = shape
    print(f"[case] noalloc B{B}H{Hq}K{Hk}M{M}N{N}D{D} {dtype} causal={causal}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=seed, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    # Reference: the allocating entry point with a torch workspace.
    o_ref = torch.empty_like(q)
    c_ref = torch.empty((B, Hk, N), dtype=torch.float32, device=gpu)
    a = _native.make_args(q, k, v, o_ref, causal, D ** -0.5)
    nbytes = lib.fas_workspace_bytes(_native.VARIANT_SOFTMAX_COL_SUM, ctypes.byref(a), 0)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=gpu)
    wptr = ws.data_ptr() + (-ws.data_ptr()) % 256
    rc = lib.fas_attention_with_softmax_col_sum(ctypes.byref(a), c_ref.data_ptr(),
                                                _native.strides3(c_ref), wptr, nbytes, stream)
    _native.check(lib, rc, "fas_attention_with_softmax_col_sum")
    # No-allocation entry point: outputs pre-filled with NaN.
    o = torch.full_like(q, float("nan"))
    c = torch.full((B, Hk, N), float("nan"), dtype=torch.float32, device=gpu)
    a2 = _native.make_args(q, k, v, o, causal, D ** -0.5)
    rc = lib.fas_attention_with_softmax_col_sum_noalloc(ctypes.byref(a2), c.data_ptr(),
                                                        _native.strides3(c), stream)
    _native.check(lib, rc, "fas_attention_with_softmax_col_sum_noalloc")
    torch.cuda.synchronize()
    assert_out_close(o, o_ref.float())
    assert_sum_close(c, c_ref, "col_softmax noalloc")


@pytest.mark.parametrize("first,second", [
    ((1, 8, 2, 1024, 1024, 128), (1, 4, 4, 300, 300, 64)),    # GQA then MHA, smaller
    ((2, 4, 2, 32, 4096, 128), (1, 2, 1, 16, 1000, 32)),      # key-split plans
    # 128 row blocks of 256 against 64 key tiles: the allocating entry point
    # splits each block's keys 4 ways (68.7 MB of partials, past the 64 MiB
    # scratch); the no-allocation entry point must shrink the plan (3 splits).
    ((1, 128, 128, 256, 4096, 128), (1, 4, 4, 300, 300, 64)),
])
def test_noalloc_matches_allocating_entry_point(first, second, gpu):
    lib = _native.load()
    if first[1] == 128:
        q, k, v = (torch.empty((1, 128, n, 128), dtype=torch.float16) for n in (256, 4096, 4096))
        a = _native.make_args(q, k, v, q, True, 128 ** -0.5)
        full = lib.fas_workspace_bytes(_native.VARIANT_SOFTMAX_COL_SUM, ctypes.byref(a), 0)
        assert full > 64 << 20, full
    _call_both(lib, first, torch.float16, True, gpu, seed=1)
    _call_both(lib, second, torch.bfloat16, True, gpu, seed=2)


def test_noalloc_rejects_oversized_problem(gpu):
    """B*Hq*M*4 bytes of row normalizers beyond 64 MiB: rejected before any
    launch.  The arguments are otherwise valid (aligned, non-null addresses,
    contiguous strides) so that the argument checks pass; no device memory is
    touched, because the workspace check fails before any HIP call."""
    lib = _native.load()
    a = _native.AttnArgs()
    a.dtype, a.causal, a.sm_scale = 0, 1, 0.125
    B, H, S, D = 64, 64, 8192, 64
    a.batch, a.heads_q, a.heads_k, a.seqlen_q, a.seqlen_k, a.head_dim = B, H, H, S, S, D
    fake = 1 << 40  # 256-byte aligned stand-in addresses, never dereferenced
    a.q, a.k, a.v, a.out = fake, 2 * fake, 3 * fake, 4 * fake
    for name in ("q_stride", "k_stride", "v_stride", "out_stride"):
        setattr(a, name, (ctypes.c_int64 * 4)(H * S * D, S * D, D, 1))
    out = (ctypes.c_int64 * 3)(H * S, S, 1)
    rc = lib.fas_attention_with_softmax_col_sum_noalloc(ctypes.byref(a), ctypes.c_void_p(5 * fake),
                                                        out, None)
    assert rc == _native.FAS_ERR_WORKSPACE
    assert "64" in _native.last_error(lib) and "scratch" in _native.last_error(lib)
