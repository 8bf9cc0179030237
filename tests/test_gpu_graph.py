"""The entry points captured in a HIP graph (torch.cuda.CUDAGraph), as a
serving loop would: each graph is replayed three times, new inputs copied
into its static input tensors eagerly between the replays, and every replay
must equal the eager call on the same inputs bit for bit (the kernels are
deterministic).  The library issues no memset and no allocation of its own
inside a call, so every launch is a kernel node; workspaces come from torch's
graph pool, or, for the no-allocation entry point, from the library's device
array."""
from __future__ import annotations

import ctypes

import pytest
import torch

import flash_attn_with_score_amd as fas
from flash_attn_with_score_amd import _native
from flash_attn_with_score_amd.attention_scores import compute_attention_scores
from oracle import inputs

pytestmark = pytest.mark.gpu

SHAPE = (1, 4, 2, 200, 264, 64)  # B, Hq, Hk, M, N, D: GQA, ragged M and N
SPLIT = 100


def _noalloc(q, k, v):
    """fas_attention_with_softmax_col_sum_noalloc through the C ABI."""
    lib = _native.load()
    B, _, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    c = torch.empty((B, Hk, N), dtype=torch.float32, device=q.device)
    a = _native.make_args(q, k, v, o, True, D ** -0.5)
    rc = lib.fas_attention_with_softmax_col_sum_noalloc(
        ctypes.byref(a), c.data_ptr(), _native.strides3(c), torch.cuda.current_stream().cuda_stream)
    _native.check(lib, rc, "fas_attention_with_softmax_col_sum_noalloc")
    return o, c


CALLS = {
    "attention_with_scores": lambda q, k, v: fas.attention_with_scores(q, k, v, causal=True),
    "attention_with_row_sum": lambda q, k, v: fas.attention_with_row_sum(q, k, v, causal=True),
    "attention_with_col_sum": lambda q, k, v: fas.attention_with_col_sum(q, k, v, causal=True),
    "attention_with_softmax_col_sum":
        lambda q, k, v: fas.attention_with_softmax_col_sum(q, k, v, causal=True),
    "attention_cross_token_qk_sum":
        lambda q, k, v: fas.attention_cross_token_qk_sum(q, k, v, SPLIT, causal=True),
    "attention_cross_token_softmax_sum":
        lambda q, k, v: fas.attention_cross_token_softmax_sum(q, k, v, SPLIT, causal=True),
    "attention_cross_token_softmax_sum_buffered":
        lambda q, k, v: fas.attention_cross_token_softmax_sum_buffered(q, k, v, SPLIT, causal=True),
    "attention": lambda q, k, v: fas.attention(q, k, v, causal=True, return_log_normalizer=True)[:2],
    "compute_attention_scores": lambda q, k, v: (compute_attention_scores(q, k),),
    "softmax_col_sum_noalloc": _noalloc,
}


@pytest.mark.parametrize("name", sorted(CALLS))
def test_graph_replays_match_eager(name, gpu):
    B, H, Hk, M, N, D = SHAPE
    print(f"[case] graph {name} B{B}H{H}K{Hk}M{M}N{N}D{D}", flush=True)
    call = CALLS[name]
    static = [t.to(gpu) for t in inputs.make_qkv(B, H, Hk, M, N, D, dtype=torch.float16, seed=1)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            call(*static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = call(*static)
    for seed in (2, 3, 4):
        fresh = inputs.make_qkv(B, H, Hk, M, N, D, dtype=torch.float16, seed=seed)
        for dst, src in zip(static, fresh):
            dst.copy_(src.to(gpu))
        graph.replay()
        torch.cuda.synchronize()
        eager = call(*static)
        torch.cuda.synchronize()
        for i, (x, y) in enumerate(zip(outs, eager)):
            assert torch.equal(x, y), f"replay with inputs seed {seed}, output {i}"
    del graph


def test_graph_attention_forward_backward(gpu):
    """attention()'s forward and backward captured together (a training
    step): every replay's O and dq, dk, dv equal the eager autograd result on
    the same inputs bit for bit."""
    B, H, Hk, M, N, D = SHAPE
    print(f"[case] graph attention fwd+bwd B{B}H{H}K{Hk}M{M}N{N}D{D}", flush=True)
    q, k, v = (t.to(gpu).requires_grad_(True)
               for t in inputs.make_qkv(B, H, Hk, M, N, D, dtype=torch.bfloat16, seed=1))
    do = torch.randn(B, H, M, D, generator=torch.Generator("cpu").manual_seed(9)).bfloat16().to(gpu)

    def step():
        o = fas.attention(q, k, v, causal=True)
        o.backward(do)
        return o

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for t in (q, k, v):
                t.grad = None
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for t in (q, k, v):
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_static = step()
    for seed in (2, 3, 4):
        fresh = inputs.make_qkv(B, H, Hk, M, N, D, dtype=torch.bfloat16, seed=seed)
        with torch.no_grad():
            for dst, src in zip((q, k, v), fresh):
                dst.copy_(src.to(gpu))
        graph.replay()
        torch.cuda.synchronize()
        qe, ke, ve = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        oe = fas.attention(qe, ke, ve, causal=True)
        ge = torch.autograd.grad(oe, (qe, ke, ve), do)
        torch.cuda.synchronize()
        assert torch.equal(o_static, oe), f"O, inputs seed {seed}"
        for name, x, y in zip(("dq", "dk", "dv"), (q.grad, k.grad, v.grad), ge):
            assert torch.equal(x, y), f"{name}, inputs seed {seed}"
    del graph
