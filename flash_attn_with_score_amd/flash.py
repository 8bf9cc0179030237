"""attention: FlashAttention-2 forward and backward as a torch.autograd.Function.

Drop-in for the reference's flash.py:32-297 (FlashAttention, attention).  The
forward pass is the family's forward kernel (kFwdPlain) writing O and the
natural-log normalizer L = m * sm_scale + ln(l) (flash.py:477-483); with
return_total_attention the key-outer column pass sums the softmax weights per
query head (total.py:9-48).  The backward pass (flash.py:172-261) runs three
gfx950 kernels through fas_attention_backward: delta = rowsum(O * dO), the
key-outer dK/dV kernel, which also stores dS when the workspace holds it, and
the query-outer dQ kernel (dQ = dS K from the stored dS, or recomputing S and
dP).  The reference's
split-KV forward (flash.py:66-136) is a scheduling choice of its Triton
kernels for small grids and gives the same O and L.
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _common, _native

__all__ = ["attention", "FlashAttention"]

# Largest keep-bit buffer (bytes) a forward with dropout holds for its
# backward pass, about B*Hq*M*N/8 (one bit per pair); past it the backward
# evaluates the random stream again, as the reference does.  The buffer lives
# from a layer's forward to its backward, so a model holds one per layer:
# the default, 64 MiB, covers B1 H32 S4096 and keeps deeper or longer models
# near the reference's O(M) saved state per head.  FAS_KEEP_BITS_MAX_BYTES
# overrides it (0 turns the buffer off).
KEEP_BITS_MAX_BYTES = int(os.environ.get("FAS_KEEP_BITS_MAX_BYTES", 64 << 20))

# Largest workspace (bytes) the backward pass allocates.  The full size holds
# dS in the input dtype for every visible (query, key) pair, about B*Hq*M*N
# bytes causal and twice that without a mask, which the dQ kernel reads
# instead of recomputing S and dP; past this limit (or when the allocation
# fails) the backward takes the smaller workspace, O(B*Hq*M) bytes, and
# recomputes.  The default, 1 GiB, holds the dS of B1 H32 S4096 causal
# (541 MB, a 7% faster backward there); B1 H32 S16384 (8.6 GB of dS) then
# recomputes at 3% more time.  FAS_BWD_WORKSPACE_MAX_BYTES overrides it
# (0: always recompute; the library's own limit is 16 GiB).
BWD_WORKSPACE_MAX_BYTES = int(os.environ.get("FAS_BWD_WORKSPACE_MAX_BYTES", 1 << 30))


def _check_inputs(q, k, v):
    Dq, Dk, Dv = q.shape[-1], k.shape[-1], v.shape[-1]
    assert Dq == Dk == Dv, "feature size of q, k, v should be equal"
    assert Dk in {16, 32, 64, 128}
    Hk, Hv = k.shape[1], v.shape[1]
    assert Hk == Hv, "num of heads in k and v should be equal"
    assert q.shape[1] % Hk == 0, "number of heads in q must be a multiple of that in k & v"


def _forward(q, k, v, causal, sm_scale, want_total, dropout_p, keep=False):
    """keep: with dropout, store the mask's bits for the backward pass
    (one bit per pair, in a buffer returned as (pointer, tensor))."""
    p = _common.finish_problem(q, k, v, sm_scale)
    o = _common.new_output(p.q)
    L = torch.empty((p.B, p.H, p.M), device=q.device, dtype=torch.float32)
    drop = _common.draw_dropout(p.q, p.k, dropout_p)
    args = _native.make_args(p.q, p.k, p.v, o, causal, p.sm_scale, drop)
    kept = (0, None)
    if keep and drop is not None:
        kptr, _, kbuf = _common.workspace(_native.VARIANT_KEEP_BITS, args, 0, q.device,
                                          limit=KEEP_BITS_MAX_BYTES)
        if kbuf is not None:
            args.keep_bits = kptr
            kept = (kptr, kbuf)
    ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_ATTENTION_FORWARD, args, 0,
                                             q.device)
    _common.call("fas_attention_forward", p.q, ctypes.byref(args), L.data_ptr(),
                 _native.strides3(L), ws_ptr, ws_bytes)
    tot = None
    if want_total:
        tot = torch.empty((p.B, p.H, p.N), device=q.device, dtype=torch.float32)
        _common.call("fas_total_attention", p.q, ctypes.byref(args), L.data_ptr(),
                     _native.strides3(L), tot.data_ptr(), _native.strides3(tot))
    return p, o, L, tot, drop, kept


class FlashAttention(torch.autograd.Function):
    """flash.py:32-261, with dropout in the forward (flash.py:59-66, 459-466,
    488-491) and the backward (:653-659, 705-731, 843-895)."""

    @staticmethod
    def forward(ctx, q, k, v, causal, sm_scale, dropout_p, return_log_normalizer,
                return_total_attention, return_seed_offset):
        _check_inputs(q, k, v)
        _common.check_device_inputs(q, k, v, dropout_p)
        # With dropout the forward keeps the mask's bits (B*Hq*M*N/8 bytes in
        # two layouts, ~N*M/4 bytes per head, up to KEEP_BITS_MAX_BYTES) so
        # that the backward reads the mask instead of evaluating the random
        # stream again; the reference regenerates it (flash.py:653-659), with
        # the same result.
        need_grad = any(ctx.needs_input_grad[:3])
        p, o, L, tot, drop, kept = _forward(q, k, v, causal, sm_scale, return_total_attention,
                                            dropout_p, keep=need_grad)
        ctx.save_for_backward(p.q, p.k, p.v, o, L)
        ctx.sm_scale = p.sm_scale
        ctx.causal = causal
        ctx.drop = drop
        ctx.keep_ptr, ctx.keep_buf = kept
        if return_log_normalizer or return_total_attention or return_seed_offset:
            # seed and offset only with dropout and return_seed_offset
            # (flash.py:161-169).
            seed = drop[1] if drop is not None and return_seed_offset else None
            offset = drop[2] if drop is not None and return_seed_offset else None
            return (o, L if return_log_normalizer else None,
                    tot if return_total_attention else None, seed, offset)
        return o

    @staticmethod
    def backward(ctx, do, *ignored):
        q, k, v, o, L = ctx.saved_tensors
        B, H, M, D = q.shape
        Hk, N = k.shape[1], k.shape[2]
        do = _common.as_kernel_operand(do)
        dq = _common.new_output(q)
        dk = torch.empty((B, Hk, N, D), dtype=k.dtype, device=q.device)
        dv = torch.empty((B, Hk, N, D), dtype=v.dtype, device=q.device)
        # The forward's (p, seed, offset): the same keep mask (flash.py:653-659),
        # read from the forward's bits when it kept them.
        args = _native.make_args(q, k, v, o, ctx.causal, ctx.sm_scale, ctx.drop,
                                 ctx.keep_ptr if ctx.keep_buf is not None else 0)
        try:
            ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_ATTENTION_BACKWARD, args, 0,
                                                     q.device, limit=BWD_WORKSPACE_MAX_BYTES)
        except torch.cuda.OutOfMemoryError:
            # The stored dS is an optimisation: without room for it the
            # backward recomputes S and dP in the dQ kernel.
            ws_ptr, ws_bytes, ws = 0, 1, None
        if ws is None and ws_bytes > 0:
            # Over the limit: the workspace without the stored dS (split != 0).
            ws_ptr, ws_bytes, ws = _common.workspace(_native.VARIANT_ATTENTION_BACKWARD, args,
                                                     1, q.device)
        _common.call("fas_attention_backward", q, ctypes.byref(args), do.data_ptr(),
                     _native.strides4(do), L.data_ptr(), _native.strides3(L), dq.data_ptr(),
                     _native.strides4(dq), dk.data_ptr(), _native.strides4(dk), dv.data_ptr(),
                     _native.strides4(dv), ws_ptr, ws_bytes)
        return dq, dk, dv, None, None, None, None, None, None


def attention(q, k, v, causal=False, sm_scale=None, dropout_p=0.0,
              return_log_normalizer=False, return_total_attention=False,
              return_seed_offset=False):
    """FlashAttention-2 (flash.py:264-297).

    q (B, Hq, M, D); k, v (B, Hk, N, D) with Hq % Hk == 0; causal masking is
    bottom-right ((N - M) + i >= j).  Returns out (B, Hq, M, D), or, when any
    return_* flag is set, (out, log_normalizer (B, Hq, M) fp32 or None,
    total_attention (B, Hq, N) fp32 or None, seed, offset), seed and offset
    being None without dropout.  Differentiable in q, k and v.
    """
    return FlashAttention.apply(q, k, v, causal, sm_scale, dropout_p, return_log_normalizer,
                                return_total_attention, return_seed_offset)
