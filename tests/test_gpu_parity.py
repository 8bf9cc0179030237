"""GPU parity of every entry point against the CPU oracle (small shapes).

Each case draws seeded q/k/v on the CPU (oracle/inputs.py), runs the HIP
entry point on the device, and compares output and side product with
oracle/naive.py under the criteria of tests/tolerances.py.  Shapes cover
MHA and GQA (group sizes 1, 2, 3, 7), every head dim, non-divisible
lengths, M < N and M > N (rows with no admissible key under bottom-right
causal masking), and split at 1, at tile edges and at N.
"""
from __future__ import annotations

import sys

import pytest
import torch

import flash_attn_with_score_amd as fas
from oracle import inputs, naive
from tests.tolerances import assert_out_close, assert_scores_close, assert_sum_close

pytestmark = pytest.mark.gpu

# (B, Hq, Hk, M, N, D)
SHAPES = [
    (1, 4, 4, 256, 256, 64),
    (2, 4, 2, 200, 200, 128),
    (1, 6, 2, 96, 160, 32),
    (1, 2, 1, 160, 96, 16),
    (1, 7, 1, 130, 130, 64),
    (1, 3, 3, 64, 64, 128),
    (1, 2, 2, 1, 77, 128),
]

PLAIN_EPS = [
    "attention_with_scores",
    "attention_with_row_sum",
    "attention_with_col_sum",
    "attention_with_col_sum_sequential",
    "attention_with_softmax_col_sum",
]
CROSS_EPS = [
    "attention_cross_token_qk_sum",
    "attention_cross_token_softmax_sum",
    "attention_cross_token_softmax_sum_buffered",
]


def _label(shape):
    return "B{}H{}K{}M{}N{}D{}".format(*shape)


def _run(ep, shape, dtype, causal, gpu, split=None, seed=0, scale=1.0, sm_scale=None):
    B, Hq, Hk, M, N, D = shape
    print(f"[case] {ep} {_label(shape)} {dtype} causal={causal} split={split} scale={scale} "
          f"sm_scale={sm_scale}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=seed, scale=scale)
    fn = getattr(fas, ep)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    if split is None:
        out, extra = fn(qd, kd, vd, causal=causal, sm_scale=sm_scale)
    else:
        out, extra = fn(qd, kd, vd, split, causal=causal, sm_scale=sm_scale)
    torch.cuda.synchronize()
    side = naive.ENTRY_POINT_OUTPUT[ep]
    ref = naive.reference_forward(q, k, v, causal=causal, sm_scale=sm_scale,
                                  causal_offset=naive.ENTRY_POINT_OFFSET[ep],
                                  split=split, want=("out", side))
    assert out.dtype == dtype and out.shape == q.shape
    assert_out_close(out, ref["out"])
    if side == "scores":
        assert extra.dtype == dtype and extra.shape == (B, Hq, M, N)
        assert_scores_close(extra, ref["scores"])
    else:
        assert extra.dtype == torch.float32
        assert_sum_close(extra, ref[side], side)


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=_label)
@pytest.mark.parametrize("ep", PLAIN_EPS)
def test_plain_entry_points(ep, shape, dtype, causal, gpu):
    _run(ep, shape, dtype, causal, gpu)


# The score writer without a causal mask: many key tiles, several row blocks
# and head groups, GQA, and N a multiple of the 64-key tile.
NONCAUSAL_SCORE_SHAPES = [
    (2, 8, 4, 300, 1024, 128),
    (1, 4, 4, 600, 768, 64),
    (1, 12, 3, 513, 320, 32),
    (3, 2, 2, 64, 4096, 16),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("shape", NONCAUSAL_SCORE_SHAPES, ids=_label)
def test_scores_noncausal_many_tiles(shape, dtype, gpu):
    _run("attention_with_scores", shape, dtype, False, gpu, seed=4)


# Short query ranges against long key ranges: fewer row blocks than CUs, so
# the plain and row-sum forward split each row block's keys over several
# workgroups and merge fp32 partials (including rows with no key, M > N).
SPLIT_SHAPES = [
    (1, 4, 2, 32, 2048, 128),
    (1, 2, 1, 300, 1500, 64),
    (2, 3, 3, 17, 4000, 16),
    (1, 2, 2, 600, 512, 32),
]


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("shape", SPLIT_SHAPES, ids=_label)
@pytest.mark.parametrize("ep", PLAIN_EPS + [
    "attention_cross_token_qk_sum", "attention_cross_token_softmax_sum"])
def test_key_split_forward(ep, shape, causal, gpu):
    split = None
    if "cross" in ep:
        split = max(1, min(shape[4], shape[3]) // 2)
    _run(ep, shape, torch.float16, causal, gpu, split=split, seed=9)


@pytest.mark.parametrize("sm_scale", [0.0, 0.3, -0.2], ids=["zero", "pos", "neg"])
@pytest.mark.parametrize("ep", PLAIN_EPS + CROSS_EPS)
def test_explicit_sm_scale(ep, sm_scale, gpu):
    """sm_scale passed explicitly, including 0 (uniform weights over the
    admissible keys) and a negative value."""
    split = 100 if "cross" in ep else None
    _run(ep, (1, 4, 2, 192, 256, 64), torch.float16, True, gpu, split=split, seed=3,
         sm_scale=sm_scale)


@pytest.mark.parametrize("sm_scale", [1.0, 1.5, -3.0], ids=["one", "1.5", "neg3"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_scores_scale_above_one(sm_scale, causal, dtype, gpu):
    """sm_scale at and above 1 (and negative): the writer scales each score
    in fp32 after the q . k product, never q itself."""
    _run("attention_with_scores", (1, 4, 2, 192, 320, 64), dtype, causal, gpu, seed=13,
         sm_scale=sm_scale)


def test_scores_q_times_scale_past_fp16_range(gpu):
    """fp16 |q| up to ~4500 with sm_scale 100: q * sm_scale lies past the
    fp16 range (65504) while the scaled scores (k is tiny) stay near +-1000;
    scores and output match the oracle (the writer must not form
    q * sm_scale in the input type)."""
    dtype = torch.float16
    B, Hq, Hk, M, N, D = 1, 2, 1, 130, 200, 64
    print(f"[case] attention_with_scores q*scale past fp16 range {dtype}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=torch.float32, seed=21)
    q, k, v = (q * 1000.0).to(dtype), (k * 0.001).to(dtype), v.to(dtype)
    out, scores = fas.attention_with_scores(q.to(gpu), k.to(gpu), v.to(gpu), causal=True,
                                            sm_scale=100.0)
    torch.cuda.synchronize()
    ref = naive.reference_forward(q, k, v, causal=True, sm_scale=100.0, want=("out", "scores"))
    assert torch.isfinite(scores.float()).all()
    assert_out_close(out, ref["out"])
    assert_scores_close(scores, ref["scores"])


@pytest.mark.parametrize("ep", PLAIN_EPS + ["attention_cross_token_softmax_sum",
                                          "attention_cross_token_softmax_sum_buffered"])
def test_large_magnitude_inputs(ep, gpu):
    """q, k, v ~ N(0, 6^2): base-2 exponents spread over hundreds, so the row
    maxima of the two half-waves that share a query row differ widely.  A
    row maximum combined from one half only overflows exp2 here."""
    split = 100 if "cross" in ep else None
    _run(ep, (1, 4, 2, 256, 256, 128), torch.float16, True, gpu, split=split, seed=11, scale=6.0)


CROSS_CASES = [
    ((1, 4, 4, 256, 256, 64), 100),
    ((1, 4, 4, 256, 256, 64), 128),
    ((1, 4, 4, 256, 256, 64), 1),
    ((1, 4, 4, 256, 256, 64), 256),
    ((2, 4, 2, 200, 200, 128), 77),
    ((1, 7, 1, 130, 130, 64), 64),
    ((1, 6, 2, 96, 160, 32), 150),
    ((1, 2, 1, 160, 96, 16), 40),
]


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", CROSS_CASES, ids=lambda c: f"{_label(c[0])}s{c[1]}")
@pytest.mark.parametrize("ep", CROSS_EPS)
def test_cross_entry_points(ep, case, dtype, causal, gpu):
    shape, split = case
    _run(ep, shape, dtype, causal, gpu, split=split)


def test_scores_config2_shape(gpu):
    """B1 H32 S1024 D128 fp16 causal (8 heads checked
    against the oracle to bound CPU time; all heads checked for the causal
    zero triangle)."""
    B, H, M, D = 1, 32, 1024, 128
    q, k, v = inputs.make_qkv(B, H, H, M, M, D, dtype=torch.float16, seed=0)
    out, scores = fas.attention_with_scores(q.to(gpu), k.to(gpu), v.to(gpu), causal=True)
    torch.cuda.synchronize()
    upper = torch.triu(torch.ones(M, M, dtype=torch.bool, device=gpu), diagonal=1)
    assert (scores[:, :, upper] == 0).all()
    sel = [0, 5, 13, 31]
    ref = naive.reference_forward(q[:, sel], k[:, sel], v[:, sel], causal=True, want=("out", "scores"))
    assert_out_close(out[:, sel], ref["out"])
    assert_scores_close(scores[:, sel], ref["scores"])


# The multi-round score writers with no causal mask: every workgroup writes
# score tiles only (no zeros), so the storer waves run their copy of the key
# loop that stores between the O += P V MFMAs.  B*H*ceil(M/256) > 256
# workgroups selects the 8-wave 256-row writer; 4 heads are checked against
# the oracle, every head's row sums against attention_with_row_sum.
@pytest.mark.parametrize("shape,dtype", [
    ((1, 80, 80, 1024, 1024, 128), torch.float16),
    ((2, 48, 48, 700, 520, 64), torch.bfloat16),
], ids=["B1H80S1024D128f16", "B2H48M700N520D64bf16"])
def test_scores_noncausal_multi_round(shape, dtype, gpu):
    B, Hq, Hk, M, N, D = shape
    print(f"[case] scores non-causal multi-round {_label(shape)} {dtype}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=6)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    out, scores = fas.attention_with_scores(qd, kd, vd, causal=False)
    _, row = fas.attention_with_row_sum(qd, kd, vd, causal=False)
    torch.cuda.synchronize()
    # Sums of the stored (rounded) scores: bf16 keeps 8 significant bits.
    rs = scores.float().sum(-1)
    tol = 2e-3 if dtype == torch.float16 else 1e-2
    assert ((rs - row).abs().max() / row.abs().max()).item() < tol
    sel = [0, 7, Hq // 2 + 1, Hq - 1]
    ref = naive.reference_forward(q[-1:, sel], k[-1:, sel], v[-1:, sel], causal=False,
                                  want=("out", "scores"))
    assert_out_close(out[-1:, sel], ref["out"])
    assert_scores_close(scores[-1:, sel], ref["scores"])


def test_noncontiguous_inputs(gpu):
    """(B, S, H, D) storage viewed as (B, H, S, D): strides are honoured."""
    B, H, S, D = 1, 4, 192, 64
    g = torch.Generator("cpu").manual_seed(3)
    base = [torch.randn(B, S, H, D, generator=g).to(torch.float16) for _ in range(3)]
    q, k, v = (t.transpose(1, 2) for t in base)
    out, scores = fas.attention_with_scores(q.to(gpu), k.to(gpu), v.to(gpu), causal=True)
    ref = naive.reference_forward(q, k, v, causal=True, want=("out", "scores"))
    assert_out_close(out, ref["out"])
    assert_scores_close(scores, ref["scores"])


def test_cross_qk_out_buffers(gpu):
    B, H, S, D, split = 1, 4, 256, 64, 96
    q, k, v = inputs.make_qkv(B, H, H, S, S, D, dtype=torch.float16, seed=5)
    out = torch.full((B, H, S, D), 7.0, dtype=torch.float16, device=gpu)
    buf = torch.full((B, H, split), 3.0, dtype=torch.float32, device=gpu)
    o, x = fas.attention_cross_token_qk_sum(q.to(gpu), k.to(gpu), v.to(gpu), split, causal=True,
                                            out=out, cross_token_qk_out=buf)
    assert o is out and x is buf
    ref = naive.reference_forward(q, k, v, causal=True, causal_offset=0, split=split,
                                  want=("out", "cross_qk"))
    assert_out_close(o, ref["out"])
    assert_sum_close(x, ref["cross_qk"], "cross_qk")


SUM_EPS = [
    "attention_with_row_sum",
    "attention_with_col_sum",
    "attention_with_col_sum_sequential",
    "attention_with_softmax_col_sum",
] + CROSS_EPS


@pytest.mark.parametrize("shape", [(1, 8, 2, 512, 512, 128), (1, 7, 1, 300, 300, 64),
                                   (1, 4, 2, 32, 2048, 128), (2, 3, 3, 17, 4000, 16)],
                         ids=_label)
@pytest.mark.parametrize("ep", SUM_EPS)
def test_repeat_calls_bit_identical(ep, shape, gpu):
    """Every column is reduced by one workgroup in a fixed order (no atomics),
    and the GQA fold and the key-split combine add in a fixed order too, so
    two calls on the same inputs return identical bits -- output and sums.
    The shapes cover MHA, GQA groups of 4 and 7, and two key-split plans."""
    B, Hq, Hk, M, N, D = shape
    print(f"[case] determinism {ep} {_label(shape)}", flush=True)
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=torch.bfloat16, seed=9, device=gpu)
    fn = getattr(fas, ep)
    args = (q, k, v, max(1, min(M, N) // 2)) if "cross" in ep else (q, k, v)
    o1, a = fn(*args, causal=True)
    o2, b = fn(*args, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2), f"{ep}: output differs between calls"
    assert torch.equal(a, b), f"{ep}: side product differs between calls"


@pytest.mark.parametrize("shape", [(1, 4, 2, 96, 200, 64), (2, 2, 1, 33, 1000, 128),
                                   (1, 3, 3, 300, 70, 16), (1, 2, 2, 64, 64, 32),
                                   (1, 2, 2, 600, 520, 128), (1, 2, 1, 513, 1029, 64),
                                   # fewer keys than one 64-key group, rows past M in
                                   # the last step (16-byte and element-wise stores)
                                   (1, 2, 2, 100, 40, 32), (2, 1, 1, 70, 8, 16)],
                         ids=_label)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_compute_attention_scores(shape, dtype, gpu):
    """attention_scores.compute_attention_scores: unmasked (q . k) * sm_scale
    for every pair, causal accepted and ignored (attention_scores.py:154-223)."""
    from flash_attn_with_score_amd.attention_scores import compute_attention_scores

    B, Hq, Hk, M, N, D = shape
    print(f"[case] compute_attention_scores {_label(shape)} {dtype}", flush=True)
    q, k, _ = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=4)
    got = compute_attention_scores(q.to(gpu), k.to(gpu), causal=True)
    torch.cuda.synchronize()
    ref = naive.reference_forward(q, k, k, causal=False, want=("scores",))["scores"]
    assert got.dtype == dtype and got.shape == (B, Hq, M, N)
    assert_out_close(got, ref, "scores")



# Short query ranges (M <= 512) over many key blocks: the scores-only
# kernel keeps each head group's Q rows in LDS (32, 64, 128, 256 or 512
# rows) and every workgroup walks several 512-key blocks (16-byte stores
# only).  B*H a multiple of 8 and not (12 heads), GQA (two heads of a group
# of 4 per workgroup at M = 200), a partial last key block and last step,
# M = 1, uneven numbers of blocks per workgroup (34 blocks over 16
# workgroups), and B*H >= 256 (one workgroup per head, 2-4 blocks each) at
# D 16 to 128.
RESIDENT_Q_SHAPES = [
    (1, 32, 32, 256, 8192, 128),
    (2, 16, 4, 200, 17000, 64),
    (1, 12, 12, 37, 22600, 128),
    (1, 16, 8, 100, 16384, 128),
    (1, 32, 32, 32, 8200, 128),
    (2, 8, 2, 17, 16384, 64),
    (8, 32, 8, 1, 2048, 128),
    (4, 64, 64, 64, 520, 32),
    (2, 128, 128, 130, 1800, 16),
    (1, 32, 32, 512, 8192, 128),
    (1, 16, 16, 300, 16384, 64),
]


# GQA: a workgroup serves the largest power-of-two share of a KV head's
# query heads whose rows fit in 512 (2, 4 and 8 heads: 200, 128 and 192
# rows, including M = 1), or one head when the group size is odd (7).
RESIDENT_Q_GROUP_SHAPES = [
    (1, 32, 8, 32, 32768, 128),
    (8, 32, 8, 1, 8192, 128),
    (1, 16, 2, 24, 131072, 64),
    (1, 28, 4, 16, 32768, 128),
    (1, 16, 8, 100, 32768, 128),
]


@pytest.mark.parametrize("shape", RESIDENT_Q_SHAPES + RESIDENT_Q_GROUP_SHAPES, ids=_label)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_compute_attention_scores_resident_q(shape, dtype, gpu):
    from flash_attn_with_score_amd.attention_scores import compute_attention_scores

    B, Hq, Hk, M, N, D = shape
    print(f"[case] compute_attention_scores resident q {_label(shape)} {dtype}", flush=True)
    q, k, _ = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=14)
    got = compute_attention_scores(q.to(gpu), k.to(gpu))
    torch.cuda.synchronize()
    ref = naive.reference_forward(q, k, k, causal=False, want=("scores",))["scores"]
    assert got.dtype == dtype and got.shape == (B, Hq, M, N)
    assert_out_close(got, ref, "scores")


# attention_with_scores on the same shapes: short query ranges take the
# key-split forward for O and the masked scores-only kernel (causal: keys
# past N - M + row written as 0).
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
# (2, 32, 32, 300, 4096, 64): 128 row blocks with N >= 8 M, also split;
# (8, 32, 32, 40, 2600, 32): 256 row blocks of M = 40, split at N >= 64 M.
@pytest.mark.parametrize("shape", RESIDENT_Q_SHAPES[:6] + RESIDENT_Q_SHAPES[9:] +
                         RESIDENT_Q_GROUP_SHAPES[::2] +
                         [(2, 32, 32, 300, 4096, 64), (8, 32, 32, 40, 2600, 32)],
                         ids=_label)
def test_scores_short_query_resident_q(shape, causal, gpu):
    _run("attention_with_scores", shape, torch.float16, causal, gpu, seed=15)


# GQA packing: a forward workgroup serves all G query heads of its KV head,
# its rows interleaving the heads (virtual row = position * G + head).
# Shapes: group sizes 2, 4, 7 and 8; M not a multiple of the block's
# positions; decode-like M = 1 and M = 3 against long keys (key split);
# causal M > N (rows with no key); D 16 to 128.  The score writer packs
# groups of 2, 4 and 8 only (group 7 runs it one head per workgroup).
PACK_SHAPES = [
    (1, 8, 2, 100, 300, 64),
    (2, 8, 1, 1, 700, 128),
    (1, 14, 2, 3, 2100, 32),
    (1, 4, 1, 300, 200, 32),
    (1, 8, 1, 257, 257, 16),
    (1, 28, 4, 333, 333, 128),
    # score writer packed over 4 and 8 heads on its 16-byte store path
    # (N % 8 == 0): M > N, M < N, and a block of positions cut by M
    (1, 8, 2, 520, 512, 64),
    (1, 16, 2, 200, 1024, 128),
    (2, 8, 1, 64, 64, 32),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("shape", PACK_SHAPES, ids=_label)
@pytest.mark.parametrize("ep", PLAIN_EPS + CROSS_EPS)
def test_gqa_packed_forward(ep, shape, dtype, gpu):
    split = max(1, min(shape[3], shape[4]) // 2) if "cross" in ep else None
    _run(ep, shape, dtype, True, gpu, split=split, seed=17)


@pytest.mark.parametrize("ep", PLAIN_EPS)
def test_gqa_equals_mha_on_repeated_kv(ep, gpu):
    """The packed GQA launch and the one-head-per-workgroup MHA launch on
    K/V repeated over the group give the same output and per-query-head side
    products (column sums of the MHA call folded over each group)."""
    B, Hq, Hk, M, N, D = 1, 8, 2, 320, 320, 64
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=torch.float16, seed=5, device=gpu)
    fn = getattr(fas, ep)
    o1, x1 = fn(q, k, v, causal=True)
    kr = k.repeat_interleave(Hq // Hk, dim=1).contiguous()
    vr = v.repeat_interleave(Hq // Hk, dim=1).contiguous()
    o2, x2 = fn(q, kr, vr, causal=True)
    torch.cuda.synchronize()
    assert_out_close(o1, o2.float())
    if ep == "attention_with_scores":
        assert_out_close(x1, x2.float(), "scores")
    elif x1.shape[1] == Hk:
        assert_sum_close(x1, x2.view(B, Hk, Hq // Hk, -1).sum(2), ep)
    else:
        assert_sum_close(x1, x2, ep)


# Causal score writes whose 128-row blocks all fit in one round of workgroups
# with long rows (N >= 2048) take the key-split writer: 64-row blocks whose
# even and odd key tiles go to two wave pairs, merged at the end.  Ragged M
# and N (N % 64 != 0, a last step with one tile), M < N, M > N (rows that see
# no key), every head dim, both dtypes, a group of 3 query heads per KV head
# (the writer packs only 2, 4 or 8, so these stay unpacked) and a large input
# scale (maxima that differ between the two halves of a row's keys).
KEY_SPLIT_SHAPES = [
    (1, 2, 2, 2048, 2048, 128),
    (1, 2, 2, 2112, 2112, 64),
    (1, 1, 1, 2000, 2056, 32),
    (1, 2, 2, 100, 2048, 16),
    (1, 1, 1, 2300, 2048, 128),
    (2, 3, 1, 513, 2200, 64),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("shape", KEY_SPLIT_SHAPES, ids=_label)
def test_scores_key_split_writer(shape, dtype, gpu):
    _run("attention_with_scores", shape, dtype, True, gpu, seed=11)


def test_scores_key_split_writer_large_inputs(gpu):
    _run("attention_with_scores", (1, 2, 2, 2048, 2048, 128), torch.float16, True, gpu, seed=12,
         scale=6.0)
