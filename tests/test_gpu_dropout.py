"""Dropout with the reference's random stream, on the GPU.

The reference keeps weight (b, h, i, j) iff Triton's tl.rand(seed, offset +
((b*H + h)*M + i)*N + j, n_rounds=6) > p, with (seed, offset) drawn from the
device generator by dropout.py:5-15.  The kernels' keep decisions are
checked bit for bit against oracle/philox.py (itself pinned to Random123's
known-answer vectors), and every entry point's outputs against the oracle
with the reference's per-entry-point semantics: O everywhere, rescaled by
1/(1-p) only in attention_with_scores and attention; the softmax column sum
masked; other side products unaffected; the buffered cross softmax sum
ignoring dropout.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import flash_attn_with_score_amd as fas
from oracle import inputs, naive, philox
from tests.tolerances import assert_out_close, assert_scores_close, assert_sum_close

pytestmark = pytest.mark.gpu
P = 0.3


def _gen(gpu):
    torch.cuda.init()  # the generators exist once the device is initialised
    return torch.cuda.default_generators[gpu.index or 0]


def _state(gpu):
    w = _gen(gpu).get_state().view(torch.int64)
    return int(w[0]), int(w[1])


def _set_state(gpu, seed, offset):
    g = _gen(gpu)
    st = g.get_state()
    w = st.view(torch.int64)
    w[0], w[1] = seed, offset
    g.set_state(st)


def _ceil4(x):
    return (x + 3) // 4 * 4


# Offsets >= 2^31 are 64-bit: counter word 1 is the high word of offset +
# index, which carries inside the tensor for the "carry" offsets.
@pytest.mark.parametrize("offset", [0, 123456, 2**31 + 1000, 2**32 - 3000, 5 * 2**32 + 2**31,
                                    7 * 2**32 - 10000],
                         ids=["zero", "small", "wide", "carry", "wide_hi", "carry_hi"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("ep", ["attention_with_scores", "attention_with_row_sum"])
def test_keep_mask_bit_exact(ep, offset, causal, gpu):
    """With V = I (N = D) the output row i is keep_i * P_i / l_i (* scale):
    its zeros are exactly the dropped or inadmissible pairs."""
    B, H, M, N, D = 1, 3, 96, 64, 64
    seed = 0x0123456789ABCDEF
    print(f"[case] keep mask {ep} offset={offset} causal={causal}", flush=True)
    q, k, _ = inputs.make_qkv(B, H, H, M, N, D, dtype=torch.float16, seed=3, scale=0.5)
    v = torch.eye(N, D, dtype=torch.float16).expand(B, H, N, D).contiguous()
    _set_state(gpu, seed, offset)
    out, _ = getattr(fas, ep)(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, dropout_p=P)
    torch.cuda.synchronize()
    assert _state(gpu) == (seed, offset + _ceil4(B * H * M * N))
    got = (out.cpu() != 0).numpy()
    adm = naive.admissible_mask(0, M, N, causal, N - M).numpy()
    for h in range(H):
        keep = philox.keep_mask(seed, offset, P, 0, h, range(M), N, H, M)
        assert np.array_equal(got[0, h], keep & adm), f"head {h}"


EPS = ["attention_with_scores", "attention_with_row_sum", "attention_with_col_sum",
       "attention_with_col_sum_sequential", "attention_with_softmax_col_sum",
       "attention_cross_token_qk_sum", "attention_cross_token_softmax_sum"]
SHAPES = [(1, 4, 2, 200, 200, 64), (2, 3, 1, 130, 300, 128), (1, 4, 2, 32, 2048, 128)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B{}H{}K{}M{}N{}D{}".format(*s))
@pytest.mark.parametrize("ep", EPS)
def test_entry_points_with_dropout(ep, shape, causal, dtype, gpu):
    _check_entry_point(ep, shape, causal, dtype, 4096 * (1 + shape[0]), gpu)


@pytest.mark.parametrize("ep", ["attention_with_scores", "attention_with_softmax_col_sum",
                                "attention_cross_token_softmax_sum"])
def test_entry_points_wide_offset_carry(ep, gpu):
    """A 64-bit offset whose index sum carries into counter word 1 halfway
    through the tensor (forward and column-pass masks)."""
    _check_entry_point(ep, (1, 4, 2, 200, 200, 64), True, torch.float16, 2**32 - 77000, gpu)


def _check_entry_point(ep, shape, causal, dtype, offset, gpu):
    B, Hq, Hk, M, N, D = shape
    split = N // 2 if "cross" in ep else None
    seed = 2024 + len(ep)
    print(f"[case] dropout {ep} {shape} causal={causal} {dtype} offset={offset}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=11)
    _set_state(gpu, seed, offset)
    fn = getattr(fas, ep)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    if split is None:
        out, extra = fn(qd, kd, vd, causal=causal, dropout_p=P)
    else:
        out, extra = fn(qd, kd, vd, split, causal=causal, dropout_p=P)
    torch.cuda.synchronize()
    assert _state(gpu) == (seed, offset + _ceil4(B * Hq * M * N))
    ref_out, ref_extra = naive.oracle_for(ep, q, k, v, causal=causal, split=split,
                                          dropout=(P, seed, offset))
    assert_out_close(out, ref_out)
    if naive.ENTRY_POINT_OUTPUT[ep] == "scores":
        assert_scores_close(extra, ref_extra)
    else:
        assert_sum_close(extra, ref_extra, naive.ENTRY_POINT_OUTPUT[ep])


def test_buffered_ignores_dropout(gpu):
    """attention_cross_token_softmax_sum_buffered ignores dropout_p and draws
    no seed (attention_cross_token_softmax_sum.py:639-732)."""
    q, k, v = inputs.make_qkv(1, 4, 2, 300, 300, 64, dtype=torch.float16, seed=5, device=gpu)
    _set_state(gpu, 9, 100)
    o1, x1 = fas.attention_cross_token_softmax_sum_buffered(q, k, v, 150, causal=True,
                                                            dropout_p=P)
    assert _state(gpu) == (9, 100)
    o0, x0 = fas.attention_cross_token_softmax_sum_buffered(q, k, v, 150, causal=True)
    assert torch.equal(o0, o1) and torch.equal(x0, x1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("shape", [(1, 4, 2, 200, 264, 64), (2, 2, 2, 300, 160, 128),
                                   (1, 6, 2, 96, 520, 32), (1, 2, 1, 64, 300, 16)],
                         ids=lambda s: "B{}H{}K{}M{}N{}D{}".format(*s))
def test_attention_dropout(shape, dtype, gpu):
    """attention(): O with dropout and the 1/(1-p) rescale, L as without
    dropout, (seed, offset) returned, and dq, dk, dv through the same mask
    (flash.py:653-731, 843-895) against the fp64 oracle."""
    _check_attention(shape, dtype, 640, gpu)


def test_attention_dropout_wide_offset_carry(gpu):
    """The backward kernels' masks with a 64-bit offset whose index sum
    carries into counter word 1 inside the tensor."""
    _check_attention((1, 4, 2, 200, 264, 64), torch.float16, 2**32 - 100000, gpu)


def _check_attention(shape, dtype, offset, gpu):
    B, H, Hk, M, N, D = shape
    print(f"[case] attention dropout {shape} {dtype} offset={offset}", flush=True)
    q, k, v = inputs.make_qkv(B, H, Hk, M, N, D, dtype=dtype, seed=8)
    seed = 31337
    _set_state(gpu, seed, offset)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    o, L, tot, s, off = fas.attention(qd, kd, vd, causal=True, dropout_p=P,
                                      return_log_normalizer=True, return_seed_offset=True)
    torch.cuda.synchronize()
    assert (s, off) == (seed, offset)
    ref = naive.reference_forward(q, k, v, causal=True, want=("out",), dropout=(P, seed, offset),
                                  drop_scale=naive.dropout_scale(P))
    assert_out_close(o, ref["out"])
    _, L0, _, s0, off0 = fas.attention(qd, kd, vd, causal=True, return_log_normalizer=True,
                                       return_seed_offset=True)
    assert s0 is None and off0 is None
    assert torch.equal(L, L0)
    g = torch.Generator("cpu").manual_seed(21)
    do = torch.randn(q.shape, generator=g).to(dtype)
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (qd, kd, vd))
    _set_state(gpu, seed, offset)
    og = fas.attention(qg, kg, vg, causal=True, dropout_p=P)
    dq, dk, dv = torch.autograd.grad(og, (qg, kg, vg), do.to(gpu))
    torch.cuda.synchronize()
    r = naive.attention_reference(q, k, v, do, causal=True, dropout=(P, seed, offset))
    assert_out_close(og, r["out"])
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert_out_close(got, r[name])


def test_softmax_col_sum_keep_bits_match_philox(gpu):
    """The softmax column sum with dropout stores the forward pass's keep
    decisions as bits for its column pass.  The no-allocation entry point,
    whose 64 MiB scratch cannot hold them at this size, evaluates the Philox
    stream again instead: both routes must give identical bits, here with a
    64-bit offset whose index sum carries into counter word 1."""
    import ctypes

    from flash_attn_with_score_amd import _native

    B, H, M, N, D = 1, 8, 8192, 8192, 64
    print(f"[case] keep bits vs Philox B{B}H{H}M{M}N{N}D{D}", flush=True)
    lib = _native.load()
    q, k, v = inputs.make_qkv(B, H, H, M, N, D, dtype=torch.float16, seed=12, device=gpu)
    drop = (P, 4321, 2**32 - 5_000_000)
    stream = torch.cuda.current_stream().cuda_stream
    o_bits = torch.empty_like(q)
    c_bits = torch.empty((B, H, N), dtype=torch.float32, device=gpu)
    a = _native.make_args(q, k, v, o_bits, True, D ** -0.5, drop)
    nbytes = lib.fas_workspace_bytes(_native.VARIANT_SOFTMAX_COL_SUM, ctypes.byref(a), 0)
    assert nbytes > 64 << 20  # room for the keep bits
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=gpu)
    wptr = ws.data_ptr() + (-ws.data_ptr()) % 256
    rc = lib.fas_attention_with_softmax_col_sum(ctypes.byref(a), c_bits.data_ptr(),
                                                _native.strides3(c_bits), wptr, nbytes, stream)
    _native.check(lib, rc, "fas_attention_with_softmax_col_sum")
    o_phx = torch.full_like(q, float("nan"))
    c_phx = torch.full((B, H, N), float("nan"), dtype=torch.float32, device=gpu)
    a2 = _native.make_args(q, k, v, o_phx, True, D ** -0.5, drop)
    rc = lib.fas_attention_with_softmax_col_sum_noalloc(ctypes.byref(a2), c_phx.data_ptr(),
                                                        _native.strides3(c_phx), stream)
    _native.check(lib, rc, "fas_attention_with_softmax_col_sum_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(o_bits, o_phx)
    assert torch.equal(c_bits, c_phx)


@pytest.mark.parametrize("shape", [(1, 4, 2, 200, 264, 64), (2, 3, 3, 97, 1000, 128)],
                         ids=lambda s: "B{}H{}K{}M{}N{}D{}".format(*s))
def test_attention_keep_bits_match_philox(shape, gpu):
    """attention()'s forward stores the keep bits for its backward
    (keep_bits); a backward without them (keep_bits = 0) evaluates the
    Philox stream in its dK/dV kernel instead.  Both routes must give the
    same O and the same dq, dk, dv bit for bit, here with a 64-bit offset
    whose index sum carries into counter word 1."""
    from flash_attn_with_score_amd import _common, _native

    B, H, Hk, M, N, D = shape
    print(f"[case] attention keep bits vs Philox {shape}", flush=True)
    lib = _native.load()
    q, k, v = inputs.make_qkv(B, H, Hk, M, N, D, dtype=torch.float16, seed=14, device=gpu)
    do = torch.randn(q.shape, generator=torch.Generator("cpu").manual_seed(3)).half().to(gpu)
    drop = (P, 777, 2**32 - 50_000)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for keep in (True, False):
        o = torch.full_like(q, float("nan"))
        L = torch.empty((B, H, M), dtype=torch.float32, device=gpu)
        a = _native.make_args(q, k, v, o, True, D ** -0.5, drop)
        kbuf = None
        if keep:
            kptr, kbytes, kbuf = _common.workspace(_native.VARIANT_KEEP_BITS, a, 0, gpu)
            assert kbytes > 0
            a.keep_bits = kptr
        wptr, wbytes, ws = _common.workspace(_native.VARIANT_ATTENTION_FORWARD, a, 0, gpu)
        rc = lib.fas_attention_forward(ctypes.byref(a), L.data_ptr(), _native.strides3(L),
                                       wptr, wbytes, stream)
        _native.check(lib, rc, "fas_attention_forward")
        grads = [torch.full_like(t, float("nan")) for t in (q, k, v)]
        b = _native.make_args(q, k, v, o, True, D ** -0.5, drop, a.keep_bits)
        wptr, wbytes, ws2 = _common.workspace(_native.VARIANT_ATTENTION_BACKWARD, b, 0, gpu)
        rc = lib.fas_attention_backward(ctypes.byref(b), do.data_ptr(), _native.strides4(do),
                                        L.data_ptr(), _native.strides3(L),
                                        *(x for g in grads for x in (g.data_ptr(),
                                                                     _native.strides4(g))),
                                        wptr, wbytes, stream)
        _native.check(lib, rc, "fas_attention_backward")
        torch.cuda.synchronize()
        outs.append((o, *grads))
        del kbuf, ws, ws2
    for name, x, y in zip(("o", "dq", "dk", "dv"), *outs):
        assert not torch.isnan(x).any(), name
        assert torch.equal(x, y), name


def test_attention_keep_bits_cap(monkeypatch, gpu):
    """Past KEEP_BITS_MAX_BYTES attention()'s forward keeps no mask bits and
    its backward evaluates the random stream again: O, dq, dk and dv are the
    same bits either way."""
    from flash_attn_with_score_amd import flash

    B, H, Hk, M, N, D = 1, 4, 2, 200, 264, 64
    print(f"[case] attention keep-bit cap B{B}H{H}K{Hk}M{M}N{N}D{D}", flush=True)
    q, k, v = inputs.make_qkv(B, H, Hk, M, N, D, dtype=torch.bfloat16, seed=15, device=gpu)
    do = torch.randn(q.shape, generator=torch.Generator("cpu").manual_seed(4)).bfloat16().to(gpu)
    outs = []
    for cap in (flash.KEEP_BITS_MAX_BYTES, 0):
        monkeypatch.setattr(flash, "KEEP_BITS_MAX_BYTES", cap)
        _set_state(gpu, 4242, 2**32 - 30_000)
        qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        o = fas.attention(qg, kg, vg, causal=True, dropout_p=P)
        outs.append((o, *torch.autograd.grad(o, (qg, kg, vg), do)))
    torch.cuda.synchronize()
    for name, x, y in zip(("o", "dq", "dk", "dv"), *outs):
        assert torch.equal(x, y), name


def test_attention_dropout_both_dq_routes(monkeypatch, gpu):
    """attention() with dropout, the forward keeping its (key-major) mask
    bits: the default backward reads the stored dS in its dQ kernel; with
    the workspace limited below the dS (FAS_BWD_WORKSPACE_MAX_BYTES) the dQ
    kernel recomputes S and dP and, the forward having stored no row blocks
    for it, evaluates the random stream.  O, dk and dv are the same bits on
    both routes, dq of each is within the oracle tolerance (64-bit offset
    carrying into counter word 1)."""
    from flash_attn_with_score_amd import flash

    B, H, Hk, M, N, D = 1, 4, 2, 200, 264, 64
    seed, offset = 5151, 2**32 - 20_000
    print(f"[case] attention dropout dq routes B{B}H{H}K{Hk}M{M}N{N}D{D}", flush=True)
    q, k, v = inputs.make_qkv(B, H, Hk, M, N, D, dtype=torch.float16, seed=17)
    do = torch.randn(q.shape, generator=torch.Generator("cpu").manual_seed(6)).half()
    outs = []
    for limit in (flash.BWD_WORKSPACE_MAX_BYTES, 0):
        monkeypatch.setattr(flash, "BWD_WORKSPACE_MAX_BYTES", limit)
        _set_state(gpu, seed, offset)
        qg, kg, vg = (t.to(gpu).requires_grad_(True) for t in (q, k, v))
        o = fas.attention(qg, kg, vg, causal=True, dropout_p=P)
        outs.append((o, *torch.autograd.grad(o, (qg, kg, vg), do.to(gpu))))
    torch.cuda.synchronize()
    for name, x, y in zip(("o", "dq", "dk", "dv"), *outs):
        assert not torch.isnan(x).any() and not torch.isnan(y).any(), name
        if name != "dq":
            assert torch.equal(x, y), name
    r = naive.attention_reference(q, k, v, do, causal=True, dropout=(P, seed, offset))
    assert_out_close(outs[0][1], r["dq"], "dq (stored dS)")
    assert_out_close(outs[1][1], r["dq"], "dq (recomputed)")
    assert_out_close(outs[0][2], r["dk"], "dk")
    assert_out_close(outs[0][3], r["dv"], "dv")


def test_attention_backward_without_bit_workspace(gpu):
    """fas_attention_backward with dropout and no keep_bits, on the route
    that recomputes S and dP for dQ (a workspace without the stored dS):
    given a workspace short of the keep-bit part as well, the dQ kernel
    evaluates the Philox stream instead of reading the dK/dV kernel's bits;
    dq, dk and dv are the same bits either way (64-bit offset carrying into
    counter word 1).  The full workspace (stored dS, whose values carry the
    mask) gives the same dk and dv bits and dq within the oracle tolerance."""
    from flash_attn_with_score_amd import _common, _native

    B, H, Hk, M, N, D = 2, 4, 2, 150, 300, 64
    print(f"[case] backward without keep-bit workspace B{B}H{H}K{Hk}M{M}N{N}D{D}", flush=True)
    lib = _native.load()
    q, k, v = inputs.make_qkv(B, H, Hk, M, N, D, dtype=torch.float16, seed=16, device=gpu)
    do = torch.randn(q.shape, generator=torch.Generator("cpu").manual_seed(5)).half().to(gpu)
    drop = (P, 99, 2**32 - 40_000)
    stream = torch.cuda.current_stream().cuda_stream
    o = torch.empty_like(q)
    L = torch.empty((B, H, M), dtype=torch.float32, device=gpu)
    a = _native.make_args(q, k, v, o, True, D ** -0.5, drop)
    wptr, wbytes, ws = _common.workspace(_native.VARIANT_ATTENTION_FORWARD, a, 0, gpu)
    _native.check(lib, lib.fas_attention_forward(ctypes.byref(a), L.data_ptr(),
                                                 _native.strides3(L), wptr, wbytes, stream),
                  "fas_attention_forward")
    full = lib.fas_workspace_bytes(_native.VARIANT_ATTENTION_BACKWARD, ctypes.byref(a), 0)
    nods = lib.fas_workspace_bytes(_native.VARIANT_ATTENTION_BACKWARD, ctypes.byref(a), 1)
    mpad = (M + 127) // 128 * 128
    bits = (B * H * mpad * ((N + 31) // 32) * 4 + 255) // 256 * 256
    assert full > nods > bits
    outs = []
    for nbytes in (nods, nods - bits, full):
        # All-ones bytes (NaN in fp16 and fp32): no kernel may read a
        # workspace element it did not write.
        buf = torch.full((full + 256,), 255, dtype=torch.uint8, device=gpu)
        ptr = buf.data_ptr() + (-buf.data_ptr()) % 256
        grads = [torch.full_like(t, float("nan")) for t in (q, k, v)]
        rc = lib.fas_attention_backward(ctypes.byref(a), do.data_ptr(), _native.strides4(do),
                                        L.data_ptr(), _native.strides3(L),
                                        *(x for g in grads for x in (g.data_ptr(),
                                                                     _native.strides4(g))),
                                        ptr, nbytes, stream)
        _native.check(lib, rc, "fas_attention_backward")
        torch.cuda.synchronize()
        outs.append(grads)
        del buf
    for name, x, y, z in zip(("dq", "dk", "dv"), *outs):
        assert not torch.isnan(x).any() and not torch.isnan(z).any(), name
        assert torch.equal(x, y), name
        if name != "dq":
            assert torch.equal(x, z), name
    r = naive.attention_reference(q.cpu(), k.cpu(), v.cpu(), do.cpu(), causal=True,
                                  dropout=drop)
    for name, i in (("dq", 0), ("dk", 1), ("dv", 2)):
        assert_out_close(outs[0][i], r[name], name)
        assert_out_close(outs[2][i], r[name], name)
    # Short of the base part the call is refused.
    rc = lib.fas_attention_backward(ctypes.byref(a), do.data_ptr(), _native.strides4(do),
                                    L.data_ptr(), _native.strides3(L),
                                    *(x for g in outs[0] for x in (g.data_ptr(),
                                                                   _native.strides4(g))),
                                    wptr or 0, 256, stream)
    assert rc == _native.FAS_ERR_WORKSPACE
