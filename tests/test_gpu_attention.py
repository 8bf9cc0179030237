"""GPU parity of attention() (flash.py:32-297) and total_attention (total.py:9-48).

Forward: output within the output tolerance of tests/tolerances.py, the
natural-log normalizer L within 1e-3 (absolute, or relative to |L| above 1)
with -inf exactly where a row sees no key, and the per-query-head total
attention under the sum criterion.  Backward: dq, dk, dv from
torch.autograd.grad through the autograd Function, within the output
tolerance of the fp64 oracle gradients (oracle/naive.attention_reference).
Shapes cover MHA and GQA in both dK/dV modes (whole group per workgroup, and
per-head fp32 partials when that leaves too few workgroups), every head dim,
non-divisible lengths, M < N, M > N (rows with no key) and a negative
sm_scale, and both dQ routes (stored dS, recomputed S and dP).
"""
from __future__ import annotations

import pytest
import torch

import flash_attn_with_score_amd as fas
from flash_attn_with_score_amd.total import total_attention
from oracle import inputs, naive
from tests.tolerances import assert_out_close, assert_sum_close

pytestmark = pytest.mark.gpu

# (B, Hq, Hk, M, N, D, causal, sm_scale)
CASES = [
    (1, 4, 4, 256, 256, 64, True, None),
    (1, 4, 4, 256, 256, 64, False, None),
    (2, 4, 2, 200, 300, 128, True, None),     # GQA, per-head partials
    (1, 8, 1, 130, 100, 32, True, None),      # M > N: rows with no key
    (1, 2, 2, 77, 333, 16, False, None),
    (1, 3, 3, 96, 160, 128, True, -0.09),     # negative scale
    (64, 8, 4, 128, 128, 32, True, None),     # GQA, whole group per workgroup
    (1, 2, 1, 1, 64, 128, True, None),
    (1, 4, 2, 64, 96, 64, True, 0.0),         # zero scale: uniform weights
    (1, 4, 2, 32, 2048, 128, True, None),     # key-split forward
    (1, 2, 2, 600, 512, 32, True, None),      # key-split forward, rows with no key
]


def _label(c):
    B, Hq, Hk, M, N, D, causal, sc = c
    tag = "" if sc is None else ("zero" if sc == 0 else "neg")
    return f"B{B}H{Hq}K{Hk}M{M}N{N}D{D}{'c' if causal else 'f'}{tag}"


def assert_lse_close(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    neg = torch.isneginf(ref)
    assert torch.equal(torch.isneginf(got), neg), "lse: -inf pattern differs"
    fin = ~neg
    err = (got[fin] - ref[fin]).abs()
    bound = 1e-3 * torch.clamp(ref[fin].abs(), min=1.0)
    assert (err <= bound).all(), f"lse: max err {err.max().item():.3e}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=_label)
def test_attention_forward_and_backward(case, dtype, gpu):
    B, Hq, Hk, M, N, D, causal, sm_scale = case
    print(f"[case] attention {_label(case)} {dtype}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=5)
    g = torch.Generator("cpu").manual_seed(7)
    do = torch.randn(B, Hq, M, D, generator=g).to(dtype)
    qd, kd, vd = (t.to(gpu).requires_grad_(True) for t in (q, k, v))
    o, L, tot, seed, offset = fas.attention(qd, kd, vd, causal=causal, sm_scale=sm_scale,
                                            return_log_normalizer=True,
                                            return_total_attention=True)
    dq, dk, dv = torch.autograd.grad(o, (qd, kd, vd), do.to(gpu))
    torch.cuda.synchronize()
    assert seed is None and offset is None
    ref = naive.attention_reference(q, k, v, do, causal=causal, sm_scale=sm_scale)
    assert o.dtype == dtype and o.shape == q.shape
    assert_out_close(o, ref["out"])
    assert L.dtype == torch.float32 and L.shape == (B, Hq, M)
    assert_lse_close(L, ref["lse"])
    assert tot.shape == (B, Hq, N)
    assert_sum_close(tot, ref["total"], "total")
    assert dq.dtype == dtype and dq.shape == q.shape
    assert dk.shape == k.shape and dv.shape == v.shape
    assert_out_close(dq, ref["dq"], "dq")
    assert_out_close(dk, ref["dk"], "dk")
    assert_out_close(dv, ref["dv"], "dv")


# Edge shapes for the dS block layout: one key, lengths just off 32 and 256,
# M > N with rows that see no key, and a batch of several heads.
EDGE_CASES = [
    (1, 2, 2, 64, 1, 64, False, None),
    (1, 2, 2, 64, 1, 64, True, None),
    (1, 4, 1, 33, 31, 16, True, None),
    (3, 2, 2, 257, 255, 128, True, None),
    (2, 6, 3, 31, 289, 32, True, None),
    (1, 2, 2, 300, 40, 64, True, None),
]


@pytest.mark.parametrize("case", CASES + EDGE_CASES, ids=_label)
def test_attention_backward_both_dq_routes(case, monkeypatch, gpu):
    """The backward's two dQ routes: from the dS blocks the dK/dV kernel
    stores (the default workspace) and, with the workspace limited below
    them (FAS_BWD_WORKSPACE_MAX_BYTES), recomputing S and dP.  dk and dv come
    from the same dK/dV kernel and are equal bit for bit; dq of each route
    is within the output tolerance of the fp64 oracle."""
    from flash_attn_with_score_amd import flash

    B, Hq, Hk, M, N, D, causal, sm_scale = case
    print(f"[case] attention dq routes {_label(case)}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=torch.float16, seed=9)
    do = torch.randn(B, Hq, M, D, generator=torch.Generator("cpu").manual_seed(10)).half()
    grads = []
    for limit in (flash.BWD_WORKSPACE_MAX_BYTES, 0):
        monkeypatch.setattr(flash, "BWD_WORKSPACE_MAX_BYTES", limit)
        qd, kd, vd = (t.to(gpu).requires_grad_(True) for t in (q, k, v))
        o = fas.attention(qd, kd, vd, causal=causal, sm_scale=sm_scale)
        grads.append(torch.autograd.grad(o, (qd, kd, vd), do.to(gpu)))
    torch.cuda.synchronize()
    (dq0, dk0, dv0), (dq1, dk1, dv1) = grads
    assert torch.equal(dk0, dk1) and torch.equal(dv0, dv1)
    ref = naive.attention_reference(q, k, v, do, causal=causal, sm_scale=sm_scale)
    assert_out_close(dq0, ref["dq"], "dq (stored dS)")
    assert_out_close(dq1, ref["dq"], "dq (recomputed)")
    assert_out_close(dk0, ref["dk"], "dk")
    assert_out_close(dv0, ref["dv"], "dv")


def _aligned_qkv(M, N, D, dtype, v_zero, seed):
    """q and k share a large common direction (q.k ~ 144 +- 17 at D = 64),
    so with a negative sm_scale every score of a row is strongly negative and
    so is its normalizer L."""
    g = torch.Generator("cpu").manual_seed(seed)
    a = 1.5 * torch.ones(D)
    q = (a + torch.randn(1, 2, M, D, generator=g)).to(dtype)
    k = (a + torch.randn(1, 2, N, D, generator=g)).to(dtype)
    v = (torch.zeros(1, 2, N, D) if v_zero else torch.randn(1, 2, N, D, generator=g)).to(dtype)
    return q, k, v


# (dtype, sm_scale, v_zero): at -0.14 the rows' L lies in [-28, -10], so
# exp(-L) * delta passes the fp16 range; at -1.0 L < -88 and exp(-L) passes
# the fp32 range (V = 0 keeps every valid dS exactly 0, so dq must be 0).
KEY_EDGE = [
    (torch.float16, -0.14, False),
    (torch.float16, -1.0, True),
    (torch.bfloat16, -1.0, True),
]


@pytest.mark.parametrize("N", [1, 40])
@pytest.mark.parametrize("dt,sm_scale,v_zero", KEY_EDGE,
                         ids=["f16-scale0.14", "f16-scale1-v0", "bf16-scale1-v0"])
def test_attention_dq_keys_past_n_strongly_negative_lse(N, dt, sm_scale, v_zero, monkeypatch, gpu):
    """Non-causal, N % 32 != 0, rows whose normalizer L is strongly negative.
    A key past N has a zero K row, so its unmasked weight would be
    exp(-L): its dS then overflows the input type (or fp32) and the dQ
    product over the stored dS blocks gives inf * 0 = NaN.  The dK/dV kernel
    masks keys past N, so both dQ routes stay finite and match the oracle."""
    from flash_attn_with_score_amd import flash

    M, D = 64, 64
    print(f"[case] dq keys past N: N{N} {dt} scale {sm_scale} v_zero {v_zero}", flush=True)
    q, k, v = _aligned_qkv(M, N, D, dt, v_zero, seed=21)
    do = torch.randn(1, 2, M, D, generator=torch.Generator("cpu").manual_seed(22)).to(dt)
    ref = naive.attention_reference(q, k, v, do, causal=False, sm_scale=sm_scale)
    for limit in (flash.BWD_WORKSPACE_MAX_BYTES, 0):
        monkeypatch.setattr(flash, "BWD_WORKSPACE_MAX_BYTES", limit)
        qd, kd, vd = (t.to(gpu).requires_grad_(True) for t in (q, k, v))
        o = fas.attention(qd, kd, vd, causal=False, sm_scale=sm_scale)
        dq, dk, dv = torch.autograd.grad(o, (qd, kd, vd), do.to(gpu))
        torch.cuda.synchronize()
        route = "stored dS" if limit else "recomputed"
        assert_out_close(dq, ref["dq"], f"dq ({route})")
        assert_out_close(dk, ref["dk"], f"dk ({route})")
        assert_out_close(dv, ref["dv"], f"dv ({route})")


@pytest.mark.parametrize("shape", [(1, 8, 8, 2048, 2048, 128, True), (2, 8, 2, 1000, 3000, 64, False),
                                   (1, 16, 4, 3000, 1000, 32, True)],
                         ids=lambda s: "B{}H{}K{}M{}N{}D{}{}".format(*s[:6], "c" if s[6] else "f"))
def test_attention_backward_bit_reproducible(shape, gpu):
    """Three backward passes of one forward give dq, dk and dv equal bit for
    bit: no atomics, and every LDS stage of the pipelined kernels (the dQ
    kernel keeps two tiles of K and dS in flight) is complete before it is
    read.  Shapes with many key tiles per workgroup, GQA and M != N."""
    B, Hq, Hk, M, N, D, causal = shape
    print(f"[case] backward reproducible {shape}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=torch.float16, seed=11, device=gpu)
    do = torch.randn(q.shape, generator=torch.Generator("cpu").manual_seed(12)).half().to(gpu)
    qd, kd, vd = (t.requires_grad_(True) for t in (q, k, v))
    o = fas.attention(qd, kd, vd, causal=causal)
    runs = [torch.autograd.grad(o, (qd, kd, vd), do, retain_graph=True) for _ in range(3)]
    torch.cuda.synchronize()
    for name, i in (("dq", 0), ("dk", 1), ("dv", 2)):
        assert not torch.isnan(runs[0][i]).any(), name
        for r in runs[1:]:
            assert torch.equal(runs[0][i], r[i]), name


def test_attention_large_magnitude_inputs(gpu):
    """q, k, v ~ N(0, 6^2): nearly one-hot softmax rows whose two half-waves
    see very different maxima."""
    print("[case] attention large magnitude", flush=True)
    q, k, v = inputs.make_qkv(1, 4, 2, 256, 256, 128, dtype=torch.float16, seed=12, scale=6.0)
    g = torch.Generator("cpu").manual_seed(13)
    do = torch.randn(1, 4, 256, 128, generator=g).to(torch.float16)
    qd, kd, vd = (t.to(gpu).requires_grad_(True) for t in (q, k, v))
    o, L, tot, _, _ = fas.attention(qd, kd, vd, causal=True, return_log_normalizer=True,
                                    return_total_attention=True)
    dq, dk, dv = torch.autograd.grad(o, (qd, kd, vd), do.to(gpu))
    torch.cuda.synchronize()
    ref = naive.attention_reference(q, k, v, do, causal=True)
    assert_out_close(o, ref["out"])
    assert_lse_close(L, ref["lse"])
    assert_sum_close(tot, ref["total"], "total")
    assert_out_close(dv, ref["dv"], "dv")


def test_attention_plain_call_returns_tensor(gpu):
    q, k, v = inputs.make_qkv(1, 2, 2, 64, 64, 64, dtype=torch.float16, seed=1, device=gpu)
    o = fas.attention(q, k, v, causal=True)
    assert isinstance(o, torch.Tensor) and o.shape == q.shape


def test_total_attention_module_matches_forward(gpu):
    """total.total_attention from a saved normalizer equals the forward's
    return_total_attention output bit for bit (same kernel, same inputs)."""
    q, k, v = inputs.make_qkv(1, 4, 2, 192, 256, 64, dtype=torch.float16, seed=2, device=gpu)
    o, L, tot, _, _ = fas.attention(q, k, v, causal=True, return_log_normalizer=True,
                                    return_total_attention=True)
    t2 = total_attention(q, k, L, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(tot, t2)


def test_attention_backward_b1h32s1024(gpu):
    """B1 H32 S1024 D128 fp16 causal (the metric shape's heads and head dim
    at a quarter of its length): gradients against the fp64 oracle."""
    B, H, S, D = 1, 32, 1024, 128
    print("[case] attention backward B1 H32 S1024 D128 f16 causal", flush=True)
    q, k, v = inputs.make_qkv(B, H, H, S, S, D, dtype=torch.float16, seed=0)
    g = torch.Generator("cpu").manual_seed(1)
    do = torch.randn(B, H, S, D, generator=g).to(torch.float16)
    qd, kd, vd = (t.to(gpu).requires_grad_(True) for t in (q, k, v))
    o = fas.attention(qd, kd, vd, causal=True)
    dq, dk, dv = torch.autograd.grad(o, (qd, kd, vd), do.to(gpu))
    torch.cuda.synchronize()
    ref = naive.attention_reference(q, k, v, do, causal=True)
    assert_out_close(o, ref["out"])
    assert_out_close(dq, ref["dq"], "dq")
    assert_out_close(dk, ref["dk"], "dk")
    assert_out_close(dv, ref["dv"], "dv")
