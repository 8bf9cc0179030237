"""Pins the CPU oracle (oracle/naive.py) -- runs without a GPU.

The oracle is what every GPU parity test trusts, so it is checked here
against things that do not share its code:

  * golden fixtures (tests/golden/*.npz) written by oracle/brute.py, an fp64
    explicit-loop formulation of reference_implementations.py:11-52;
  * closed forms: softmax rows sum to 1; constant keys give uniform weights;
    raw-score sums over rows and over columns agree; an empty cross region
    gives zero sums; rows with no admissible key give zero output;
  * structural identities: GQA equals MHA on repeated K/V with the column
    sums folded per KV head (attention_with_col_sum.py:72,370);
  * planted mistakes: each of a wrong causal offset, a missing GQA fold, a
    doubled softmax scale and a wrong split boundary, planted in the oracle,
    makes a pin fail.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import brute, inputs, naive

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz"))

SUM_KEYS = ("row_sum", "col_sum", "col_softmax", "cross_qk", "cross_softmax")


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz")) as z:
        return {k: z[k] for k in z.files}


def run_oracle(f):
    q, k, v = (torch.from_numpy(f[n]) for n in ("q", "k", "v"))
    split = int(f["meta_split"]) if "meta_split" in f else None
    want = ["out", "scores", "row_sum", "col_sum", "col_softmax"]
    if split is not None:
        want += ["cross_qk", "cross_softmax"]
    return naive.reference_forward(q, k, v, causal=bool(f["meta_causal"]),
                                   sm_scale=float(f["meta_sm_scale"]),
                                   causal_offset=int(f["meta_causal_offset"]), split=split,
                                   want=want, chunk=37)


def check_against_fixture(name):
    f = load(name)
    res = run_oracle(f)
    np.testing.assert_allclose(res["out"].numpy(), f["out"], rtol=1e-5, atol=1e-5)
    ref_s = f["scores"]
    got_s = res["scores"].numpy()
    assert np.array_equal(np.isneginf(ref_s), np.isneginf(got_s)), f"{name}: mask differs"
    fin = np.isfinite(ref_s)
    np.testing.assert_allclose(got_s[fin], ref_s[fin], rtol=1e-5, atol=1e-5)
    for key in SUM_KEYS:
        if key in f:
            ref = f[key]
            got = res[key].numpy()
            scale = max(1.0, float(np.abs(ref).max()))
            np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5 * scale, err_msg=f"{name}:{key}")


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_matches_golden(name):
    check_against_fixture(name)


@pytest.mark.parametrize("name", ["f1_config1_causal", "f2_gqa_causal"])
def test_naive_restatement_matches_golden(name):
    """naive_attention_with_scores restates reference_implementations.py:11-52
    (top-left triu mask, -inf fill); the fixtures use offset 0, M == N."""
    f = load(name)
    q, k, v = (torch.from_numpy(f[n]) for n in ("q", "k", "v"))
    out, scores = naive.naive_attention_with_scores(q, k, v, causal=True,
                                                    sm_scale=float(f["meta_sm_scale"]))
    np.testing.assert_allclose(out.numpy(), f["out"], rtol=1e-5, atol=1e-5)
    assert np.array_equal(np.isneginf(scores.numpy()), np.isneginf(f["scores"]))


def test_fixture_config1_shape():
    f = load("f1_config1_causal")
    assert f["q"].shape == (1, 4, 256, 64) and f["out"].shape == (1, 4, 256, 64)
    assert f["scores"].shape == (1, 4, 256, 256)
    assert abs(float(f["meta_sm_scale"]) - 1 / 8) < 1e-12


# ----------------------------------------------------------- closed forms

CASES = [
    # (B, Hq, Hk, M, N, D, causal)
    (1, 4, 2, 40, 40, 16, True),
    (2, 3, 1, 33, 57, 32, True),
    (1, 2, 2, 57, 33, 16, True),   # M > N: 24 empty rows (bottom-right)
    (1, 6, 3, 29, 41, 16, False),
]


def _qkv(case, seed=0, dtype=torch.float32):
    B, Hq, Hk, M, N, D, _ = case
    return inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=dtype, seed=seed)


@pytest.mark.parametrize("case", CASES)
def test_softmax_weights_sum_to_group_rows(case):
    """sum_j col_softmax[b, hk, j] = G * (number of rows with an admissible key)."""
    B, Hq, Hk, M, N, D, causal = case
    q, k, v = _qkv(case)
    res = naive.reference_forward(q, k, v, causal=causal, want=("col_softmax",))
    nonempty = M if not causal else sum(1 for i in range(M) if (N - M) + i >= 0)
    tot = res["col_softmax"].double().sum(-1)
    assert torch.allclose(tot, torch.full_like(tot, (Hq // Hk) * nonempty), rtol=1e-5)


@pytest.mark.parametrize("case", CASES)
def test_row_and_column_raw_sums_agree(case):
    """Both side products sum every admissible scaled score exactly once."""
    B, Hq, Hk, M, N, D, causal = case
    q, k, v = _qkv(case, seed=1)
    res = naive.reference_forward(q, k, v, causal=causal, want=("row_sum", "col_sum"))
    G = Hq // Hk
    rows = res["row_sum"].double().view(B, Hk, G, M).sum((2, 3))
    cols = res["col_sum"].double().sum(-1)
    assert torch.allclose(rows, cols, rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("causal", [True, False])
def test_constant_keys_give_uniform_weights(causal):
    """Identical keys: every admissible key of row i gets weight 1/n_i, so the
    output is the mean of the admissible V rows and the softmax column sum
    is sum over rows seeing j of G/n_i."""
    B, Hq, Hk, M, N, D = 1, 4, 2, 24, 40, 16
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, seed=3)
    k = k[:, :, :1].expand(B, Hk, N, D).contiguous()
    res = naive.reference_forward(q, k, v, causal=causal, want=("out", "col_softmax"))
    off = N - M
    G = Hq // Hk
    exp_col = torch.zeros(B, Hk, N, dtype=torch.float64)
    for i in range(M):
        n_i = min(N, off + i + 1) if causal else N
        exp_col[:, :, :n_i] += G / n_i
        for h in range(Hq):
            mean_v = v[0, h // G, :n_i].double().mean(0)
            assert torch.allclose(res["out"][0, h, i].double(), mean_v, atol=1e-5)
    assert torch.allclose(res["col_softmax"].double(), exp_col, rtol=1e-5)


def test_gqa_equals_mha_with_repeated_kv():
    B, Hq, Hk, M, N, D = 1, 6, 2, 31, 45, 32
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, seed=4)
    G = Hq // Hk
    want = ("out", "row_sum", "col_sum", "col_softmax", "cross_qk", "cross_softmax")
    gqa = naive.reference_forward(q, k, v, causal=True, split=20, want=want)
    kr, vr = (torch.repeat_interleave(t, G, dim=1) for t in (k, v))
    mha = naive.reference_forward(q, kr, vr, causal=True, split=20, want=want)
    assert torch.allclose(gqa["out"], mha["out"], atol=1e-6)
    assert torch.allclose(gqa["row_sum"], mha["row_sum"], atol=1e-5)
    for key in ("col_sum", "col_softmax", "cross_qk", "cross_softmax"):
        folded = mha[key].double().view(B, Hk, G, -1).sum(2)
        assert torch.allclose(gqa[key].double(), folded, rtol=1e-5, atol=1e-4), key


def test_split_at_M_gives_zero_cross_sums():
    q, k, v = inputs.make_qkv(1, 2, 2, 32, 48, 16, seed=5)
    res = naive.reference_forward(q, k, v, causal=False, split=32,
                                  want=("cross_qk", "cross_softmax"))
    assert res["cross_qk"].abs().max() == 0 and res["cross_softmax"].abs().max() == 0


def test_empty_rows_give_zero_output_and_row_sums():
    """M > N, bottom-right causal: the first M - N rows see no key
    (attention_with_scores.py:192-195, attention_with_row_sum.py:181-185)."""
    q, k, v = inputs.make_qkv(1, 2, 2, 40, 16, 16, seed=6)
    res = naive.reference_forward(q, k, v, causal=True, want=("out", "row_sum", "scores"))
    assert res["out"][:, :, :24].abs().max() == 0
    assert res["row_sum"][:, :, :24].abs().max() == 0
    assert torch.isneginf(res["scores"][:, :, :24]).all()
    assert torch.isfinite(res["out"]).all()


def test_scores_as_returned_zero_the_mask():
    q, k, v = inputs.make_qkv(1, 1, 1, 8, 8, 16, seed=7)
    res = naive.reference_forward(q, k, v, causal=True, want=("scores",))
    s = naive.scores_as_returned(res["scores"])
    assert (s[0, 0].triu(1) == 0).all() and torch.isfinite(s).all()


def test_brute_matches_oracle_on_random_tiny_problem():
    """A second fp64 brute-force run on inputs the fixtures do not cover."""
    B, Hq, Hk, M, N, D = 2, 3, 3, 11, 13, 16
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, seed=8)
    for causal in (True, False):
        ref = brute.brute_forward(q.numpy(), k.numpy(), v.numpy(), causal=causal, split=7)
        got = naive.reference_forward(q, k, v, causal=causal, split=7)
        for key in ("out", "row_sum", "col_sum", "col_softmax", "cross_qk", "cross_softmax"):
            np.testing.assert_allclose(got[key].numpy(), ref[key], rtol=1e-5, atol=1e-5,
                                       err_msg=key)


# ------------------------------------------------- planted mistakes must fail

def test_planted_wrong_causal_offset_is_caught(monkeypatch):
    orig = naive.admissible_mask
    monkeypatch.setattr(naive, "admissible_mask",
                        lambda i0, i1, N, causal, off: orig(i0, i1, N, causal, off + 1))
    with pytest.raises(AssertionError):
        check_against_fixture("f4_m48_n80_bottomright")


def test_planted_missing_group_fold_is_caught(monkeypatch):
    """Column sums written per query head instead of summed per KV head."""
    orig = naive.reference_forward

    def mutated(q, k, v, **kw):
        res = orig(q, k, v, **kw)
        if "col_softmax" in res:
            res["col_softmax"] = res["col_softmax"] / (q.shape[1] // k.shape[1])
        return res

    monkeypatch.setattr(naive, "reference_forward", mutated)
    with pytest.raises(AssertionError):
        check_against_fixture("f2_gqa_causal")


def test_planted_doubled_scale_is_caught():
    f = load("f1_config1_causal")
    f = dict(f)
    f["meta_sm_scale"] = np.asarray(float(f["meta_sm_scale"]) * 2)
    res = run_oracle(f)
    assert not np.allclose(res["out"].numpy(), f["out"], atol=1e-3)


def test_planted_split_boundary_is_caught():
    f = dict(load("f3_cross_causal"))
    f["meta_split"] = np.asarray(int(f["meta_split"]) + 1)
    res = run_oracle(f)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(res["cross_softmax"].numpy()[..., :96],
                                   f["cross_softmax"], rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- attention()
# oracle.naive.attention_reference (flash.py:32-297 and its backward) is
# pinned by the independent fp64 loop formulation (out, L, total attention)
# and by central finite differences of sum(out * dO) through that same loop
# formulation (the gradients).

ATTN_CASES = [  # (B, Hq, Hk, M, N, D, causal)
    (1, 4, 2, 5, 7, 4, True),
    (1, 2, 1, 7, 5, 4, True),   # M > N: two rows see no key
    (2, 2, 2, 4, 6, 3, False),
]


def _attn_inputs(case, seed=3):
    B, Hq, Hk, M, N, D, causal = case
    q, k, v = inputs.make_qkv(B, Hq, Hk, M, N, D, dtype=torch.float32, seed=seed)
    g = torch.Generator("cpu").manual_seed(seed + 100)
    do = torch.randn(B, Hq, M, D, generator=g, dtype=torch.float32)
    return q.double(), k.double(), v.double(), do.double(), causal


@pytest.mark.parametrize("case", ATTN_CASES)
def test_attention_reference_forward_matches_brute_force(case):
    q, k, v, do, causal = _attn_inputs(case)
    r = naive.attention_reference(q, k, v, causal=causal, sm_scale=0.7)
    bf = brute.brute_forward(q.numpy(), k.numpy(), v.numpy(), causal=causal, sm_scale=0.7)
    np.testing.assert_allclose(r["out"].numpy(), bf["out"], atol=1e-12)
    assert np.array_equal(np.isneginf(r["lse"].numpy()), np.isneginf(bf["lse"]))
    fin = np.isfinite(bf["lse"])
    np.testing.assert_allclose(r["lse"].numpy()[fin], bf["lse"][fin], atol=1e-12)
    np.testing.assert_allclose(r["total"].numpy(), bf["total"], atol=1e-12)


def _fd_grads(q, k, v, do, causal, sm_scale, h=1e-6):
    """Central differences of sum(out * do), out from oracle/brute.py."""
    qn, kn, vn, dn = (t.numpy().copy() for t in (q, k, v, do))

    def f(qq, kk, vv):
        return float((brute.brute_forward(qq, kk, vv, causal=causal, sm_scale=sm_scale)["out"]
                      * dn).sum())

    grads = []
    for which in range(3):
        arrs = [qn, kn, vn]
        base = arrs[which]
        g = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            old = base[idx]
            base[idx] = old + h
            fp = f(*arrs)
            base[idx] = old - h
            fm = f(*arrs)
            base[idx] = old
            g[idx] = (fp - fm) / (2 * h)
        grads.append(g)
    return grads


@pytest.mark.parametrize("case", ATTN_CASES)
def test_attention_reference_gradients_match_finite_differences(case):
    q, k, v, do, causal = _attn_inputs(case)
    r = naive.attention_reference(q, k, v, do, causal=causal, sm_scale=0.7)
    gq, gk, gv = _fd_grads(q, k, v, do, causal, 0.7)
    np.testing.assert_allclose(r["dq"].numpy(), gq, atol=1e-6)
    np.testing.assert_allclose(r["dk"].numpy(), gk, atol=1e-6)
    np.testing.assert_allclose(r["dv"].numpy(), gv, atol=1e-6)


def test_planted_gradient_without_group_sum_is_caught():
    """dK taken from the first query head of each group only (a missing GQA
    fold in the backward, flash.py:258-259) must fail the finite differences."""
    case = ATTN_CASES[0]
    q, k, v, do, causal = _attn_inputs(case)
    G = q.shape[1] // k.shape[1]
    r = naive.attention_reference(q[:, ::G], k, v, do[:, ::G], causal=causal, sm_scale=0.7)
    _, gk, _ = _fd_grads(q, k, v, do, causal, 0.7)
    assert not np.allclose(r["dk"].numpy(), gk, atol=1e-6)


def test_attention_reference_dropout():
    """Dropout in the fp64 attention oracle: with every weight kept the output
    is 1/(1-p) times the undropped one; with some dropped, the autograd
    gradients match central differences of its own forward (the mask is
    fixed by (seed, offset), so the function is smooth)."""
    from oracle import philox

    case = (1, 2, 1, 5, 7, 4, True)
    q, k, v, do, causal = _attn_inputs(case)
    base = naive.attention_reference(q, k, v, causal=causal, sm_scale=0.7)
    tiny = (1e-9, 5, 0)
    assert all(philox.keep_mask(5, 0, 1e-9, 0, h, range(5), 7, 2, 5).all() for h in range(2))
    kept = naive.attention_reference(q, k, v, causal=causal, sm_scale=0.7, dropout=tiny)
    np.testing.assert_allclose(kept["out"].numpy(), base["out"].numpy() * naive.dropout_scale(1e-9),
                               rtol=1e-12)
    drop = (0.4, 12345, 64)
    r = naive.attention_reference(q, k, v, do, causal=causal, sm_scale=0.7, dropout=drop)
    assert not np.allclose(r["out"].numpy(), base["out"].numpy())
    np.testing.assert_array_equal(r["lse"].numpy(), base["lse"].numpy())

    def f(qq, kk, vv):
        o = naive.attention_reference(torch.from_numpy(qq), torch.from_numpy(kk),
                                      torch.from_numpy(vv), causal=causal, sm_scale=0.7,
                                      dropout=drop)["out"]
        return float((o.numpy() * do.numpy()).sum())

    arrs = [t.numpy().copy() for t in (q, k, v)]
    for which, name in enumerate(("dq", "dk", "dv")):
        g = np.zeros_like(arrs[which])
        for idx in np.ndindex(g.shape):
            old = arrs[which][idx]
            arrs[which][idx] = old + 1e-6
            fp = f(*arrs)
            arrs[which][idx] = old - 1e-6
            fm = f(*arrs)
            arrs[which][idx] = old
            g[idx] = (fp - fm) / 2e-6
        np.testing.assert_allclose(r[name].numpy(), g, atol=1e-6)
