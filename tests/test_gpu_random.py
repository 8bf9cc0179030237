"""Seeded random sweep over every entry point against the CPU oracle.

Each case draws, from a fixed seed, a shape (ragged M and N, M < N and
M > N, GQA groups 1 to 8, head dims 16 to 128), a dtype, the causal flag,
sm_scale (default, positive, negative), the cross-token split and the
storage layout of q, k and v ((B, H, S, D) or (B, S, H, D) viewed as
(B, H, S, D)).  The cases are fixed at collection time, so a failure names
a reproducible case; the fixed-shape tests in test_gpu_parity.py cover the
edges by name.
"""
from __future__ import annotations

import random

import pytest
import torch

import flash_attn_with_score_amd as fas
from flash_attn_with_score_amd.attention_scores import compute_attention_scores
from oracle import inputs, naive
from tests.tolerances import assert_out_close, assert_scores_close, assert_sum_close

pytestmark = pytest.mark.gpu

EPS = [
    "attention_with_scores",
    "attention_with_row_sum",
    "attention_with_col_sum",
    "attention_with_col_sum_sequential",
    "attention_with_softmax_col_sum",
    "attention_cross_token_qk_sum",
    "attention_cross_token_softmax_sum",
    "attention_cross_token_softmax_sum_buffered",
    "compute_attention_scores",
    "attention",
]


def _cases(n: int = 200, seed: int = 20241202):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        ep = EPS[i % len(EPS)]
        G = rng.choice([1, 1, 2, 3, 4, 7, 8])
        Hk = rng.choice([1, 2, 3])
        B = rng.choice([1, 1, 2])
        M = rng.choice([1, 7, 64, 100, 255, 256, 257, 390, 513])
        N = rng.choice([1, 8, 63, 64, 65, 200, 512, 700])
        D = rng.choice([16, 32, 64, 128])
        dtype = rng.choice(["f16", "bf16"])
        causal = rng.random() < 0.6
        layout = rng.choice(["bhsd", "bshd"])
        sm_scale = rng.choice([None, None, 0.07, -0.1])
        split = rng.randint(1, min(M, N)) if "cross" in ep else None
        out.append((i, ep, (B, Hk * G, Hk, M, N, D), dtype, causal, layout, sm_scale, split))
    return out


def _label(case):
    i, ep, (B, Hq, Hk, M, N, D), dtype, causal, layout, sm_scale, split = case
    return (f"{i}-{ep}-B{B}H{Hq}K{Hk}M{M}N{N}D{D}-{dtype}-{'causal' if causal else 'full'}-{layout}"
            f"-s{sm_scale}-x{split}")


def _tensors(shape, dtype, layout, seed):
    """Seeded q, k, v on the CPU (oracle/inputs.py values) in the given
    storage layout: bshd stores (B, S, H, D) and returns the (B, H, S, D) view."""
    B, Hq, Hk, M, N, D = shape
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=seed)
    if layout == "bshd":
        q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    return q, k, v


def _to_gpu(t, gpu):
    """The same storage layout on the device."""
    if t.is_contiguous():
        return t.to(gpu)
    return t.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)


@pytest.mark.parametrize("case", _cases(), ids=_label)
def test_random_case(case, gpu):
    i, ep, shape, dname, causal, layout, sm_scale, split = case
    B, Hq, Hk, M, N, D = shape
    dtype = torch.float16 if dname == "f16" else torch.bfloat16
    print(f"[case] {_label(case)}", flush=True)
    q, k, v = _tensors(shape, dtype, layout, seed=1000 + i)
    qd, kd, vd = (_to_gpu(t, gpu) for t in (q, k, v))
    assert qd.stride() == q.stride()

    if ep == "compute_attention_scores":
        got = compute_attention_scores(qd, kd, causal=causal, sm_scale=sm_scale)
        torch.cuda.synchronize()
        ref = naive.reference_forward(q, k, k, causal=False, sm_scale=sm_scale,
                                      want=("scores",))["scores"]
        assert got.dtype == dtype and got.shape == (B, Hq, M, N)
        assert_out_close(got, ref, "scores")
        return

    if ep == "attention":
        g = torch.Generator("cpu").manual_seed(7)
        do = torch.randn(B, Hq, M, D, generator=g).to(dtype)
        qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (qd, kd, vd))
        o = fas.attention(qg, kg, vg, causal=causal, sm_scale=sm_scale)
        dq, dk, dv = torch.autograd.grad(o, (qg, kg, vg), do.to(gpu))
        torch.cuda.synchronize()
        ref = naive.attention_reference(q, k, v, do, causal=causal, sm_scale=sm_scale)
        assert_out_close(o, ref["out"])
        assert_out_close(dq, ref["dq"], "dq")
        assert_out_close(dk, ref["dk"], "dk")
        assert_out_close(dv, ref["dv"], "dv")
        return

    fn = getattr(fas, ep)
    if split is None:
        out, extra = fn(qd, kd, vd, causal=causal, sm_scale=sm_scale)
    else:
        out, extra = fn(qd, kd, vd, split, causal=causal, sm_scale=sm_scale)
    torch.cuda.synchronize()
    ref_out, ref_extra = naive.oracle_for(ep, q, k, v, causal=causal, sm_scale=sm_scale,
                                          split=split)
    assert out.dtype == dtype and out.shape == q.shape
    assert_out_close(out, ref_out)
    if naive.ENTRY_POINT_OUTPUT[ep] == "scores":
        assert_scores_close(extra, ref_extra)
    else:
        assert_sum_close(extra, ref_extra, naive.ENTRY_POINT_OUTPUT[ep])


# Dropout: the same sweep over the entry points that draw the mask, with the
# generator state set to a seeded (seed, offset) -- a third of the offsets
# 64-bit, some of them carrying into counter word 1 inside the tensor -- so
# the keep-bit routes (softmax column sum, attention backward) and Philox
# evaluated in place meet ragged shapes, GQA and every head dim.
DROP_EPS = [
    "attention_with_scores",
    "attention_with_row_sum",
    "attention_with_softmax_col_sum",
    "attention_cross_token_softmax_sum",
    "attention",
]


def _drop_cases(n: int = 60, seed: int = 7331):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        ep = DROP_EPS[i % len(DROP_EPS)]
        G = rng.choice([1, 1, 2, 4])
        Hk = rng.choice([1, 2])
        B = rng.choice([1, 2])
        M = rng.choice([1, 33, 64, 100, 257, 390])
        N = rng.choice([8, 63, 64, 65, 200, 512])
        D = rng.choice([16, 32, 64, 128])
        dtype = rng.choice(["f16", "bf16"])
        causal = rng.random() < 0.6
        total = B * Hk * G * M * N
        kind = rng.choice(["small", "wide", "carry"])
        if kind == "small":
            offset = rng.randrange(0, 2**31 - total)
        elif kind == "wide":
            offset = rng.randrange(2**31, 2**40)
        else:  # 64-bit, the low word wrapping inside the tensor
            offset = (rng.randrange(1, 2**8) << 32) - rng.randrange(1, total)
        offset &= ~3  # torch's generator keeps offsets at multiples of 4
        split = rng.randint(1, min(M, N)) if "cross" in ep else None
        out.append((i, ep, (B, Hk * G, Hk, M, N, D), dtype, causal, offset, split))
    return out


def _drop_label(case):
    i, ep, (B, Hq, Hk, M, N, D), dtype, causal, offset, split = case
    return (f"{i}-{ep}-B{B}H{Hq}K{Hk}M{M}N{N}D{D}-{dtype}-{'causal' if causal else 'full'}"
            f"-o{offset}-x{split}")


@pytest.mark.parametrize("case", _drop_cases(), ids=_drop_label)
def test_random_dropout_case(case, gpu):
    i, ep, shape, dname, causal, offset, split = case
    B, Hq, Hk, M, N, D = shape
    dtype = torch.float16 if dname == "f16" else torch.bfloat16
    p_drop, seed = 0.2, 9000 + i
    print(f"[case] {_drop_label(case)}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=2000 + i)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    gen = torch.cuda.default_generators[gpu.index or 0]
    state = gen.get_state()
    state.view(torch.int64)[0], state.view(torch.int64)[1] = seed, offset
    gen.set_state(state)
    dropout = (p_drop, seed, offset)

    if ep == "attention":
        g = torch.Generator("cpu").manual_seed(7)
        do = torch.randn(B, Hq, M, D, generator=g).to(dtype)
        qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (qd, kd, vd))
        o = fas.attention(qg, kg, vg, causal=causal, dropout_p=p_drop)
        dq, dk, dv = torch.autograd.grad(o, (qg, kg, vg), do.to(gpu))
        torch.cuda.synchronize()
        ref = naive.attention_reference(q, k, v, do, causal=causal, dropout=dropout)
        assert_out_close(o, ref["out"])
        assert_out_close(dq, ref["dq"], "dq")
        assert_out_close(dk, ref["dk"], "dk")
        assert_out_close(dv, ref["dv"], "dv")
        return

    fn = getattr(fas, ep)
    if split is None:
        out, extra = fn(qd, kd, vd, causal=causal, dropout_p=p_drop)
    else:
        out, extra = fn(qd, kd, vd, split, causal=causal, dropout_p=p_drop)
    torch.cuda.synchronize()
    ref_out, ref_extra = naive.oracle_for(ep, q, k, v, causal=causal, split=split,
                                          dropout=dropout)
    assert_out_close(out, ref_out)
    if naive.ENTRY_POINT_OUTPUT[ep] == "scores":
        assert_scores_close(extra, ref_extra)
    else:
        assert_sum_close(extra, ref_extra, naive.ENTRY_POINT_OUTPUT[ep])
