"""Parity criteria for the fused attention family.

Outputs and scores: |kernel - oracle| <= 2e-2 + 2e-2 * |oracle| elementwise
(fp16/bf16 inputs against the fp32 oracle).  Masked score positions (oracle
-inf) must be exactly 0.  Sums: relative error <= 1e-3, measured both as
||d||_2 / ||ref||_2 and as max|d| <= 1e-3 * max|ref| (elementwise relative
error is ill-conditioned for raw-score sums near zero).
"""
from __future__ import annotations

import torch

OUT_ATOL = 2e-2
OUT_RTOL = 2e-2
SUM_RTOL = 1e-3


def assert_out_close(got: torch.Tensor, ref: torch.Tensor, what: str = "out") -> None:
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    err = (got - ref).abs()
    bound = OUT_ATOL + OUT_RTOL * ref.abs()
    bad = err > bound
    if bad.any():
        idx = tuple(int(i) for i in bad.nonzero()[0])
        raise AssertionError(f"{what}: {int(bad.sum())} elements out of tolerance; first at {idx}: "
                             f"got {got[idx].item()} ref {ref[idx].item()} (max err {err.max().item():.3e})")


def assert_scores_close(got: torch.Tensor, ref_masked: torch.Tensor) -> None:
    """ref_masked: oracle scores with -inf at masked positions."""
    got = got.detach().float().cpu()
    ref_masked = ref_masked.float().cpu()
    masked = torch.isinf(ref_masked) & (ref_masked < 0)
    assert (got[masked] == 0).all(), "scores: masked positions must be exactly 0"
    ref = torch.where(masked, torch.zeros(()), ref_masked)
    assert_out_close(got, ref, "scores")


def assert_sum_close(got: torch.Tensor, ref: torch.Tensor, what: str = "sum") -> None:
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    d = got - ref
    ref_norm = ref.norm().item()
    ref_max = ref.abs().max().item() if ref.numel() else 0.0
    if ref_norm == 0.0:
        assert d.abs().max().item() <= 1e-6, f"{what}: expected zeros, max |got| {got.abs().max().item()}"
        return
    rel = d.norm().item() / ref_norm
    mx = d.abs().max().item()
    assert rel <= SUM_RTOL, f"{what}: ||d||/||ref|| = {rel:.3e} > {SUM_RTOL}"
    assert mx <= SUM_RTOL * ref_max, f"{what}: max|d| = {mx:.3e} > {SUM_RTOL} * max|ref| ({ref_max:.3e})"
