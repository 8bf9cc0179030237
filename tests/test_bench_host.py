"""bench.py's host side on the CPU: the pair counts, the algorithmic FLOP and
byte model of every workload, the one-GPU refusal and the traffic figure it
reads from the committed profile."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _pairs_brute(M, N, causal, off):
    return sum(1 for i in range(M) for j in range(N) if not causal or off + i >= j)


@pytest.mark.parametrize("M,N", [(1, 1), (7, 7), (5, 9), (9, 5), (64, 100)])
@pytest.mark.parametrize("causal", [False, True])
def test_pairs_brute_force(M, N, causal):
    off = N - M
    assert bench.pairs(M, N, causal, off) == _pairs_brute(M, N, causal, off)


def test_pairs_closed_form_metric_shape():
    # Causal M = N = 4096: 4096 * 4097 / 2 admissible pairs per head.
    assert bench.pairs(4096, 4096, True, 0) == 4096 * 4097 // 2 == 8390656
    assert bench.pairs(4096, 4096, False, 0) == 4096 * 4096


@pytest.mark.parametrize("causal", [False, True])
def test_cross_pairs_brute_force(causal):
    M, N, split = 37, 37, 20
    brute = sum(1 for i in range(split, M) for j in range(split)
                if not causal or i >= j)
    assert bench.cross_pairs(M, N, split, causal, 0) == brute


def test_metric_shape_scores_bytes_and_flop():
    flop, nbytes = bench.work("scores", 1, 32, 32, 4096, 4096, 128, True, None)
    assert nbytes == 1_207_959_552  # scores 2BHMN + q, k, v, o
    assert flop == 4 * 32 * 128 * 8390656


@pytest.mark.parametrize("name", sorted(bench.WORKLOADS))
def test_every_workload_has_a_model(name):
    needs_split = bench.WORKLOADS[name][1]
    flop, nbytes = bench.work(name, 2, 8, 4, 256, 384, 64, True, 128 if needs_split else None)
    assert flop > 0 and nbytes > 0
    # q, k, v, o are always read or written once
    assert nbytes >= 2 * (2 * 2 * 8 * 256 * 64 + 2 * 2 * 4 * 384 * 64)


def test_backward_is_two_and_a_half_forwards():
    f, _ = bench.work("attention_fwd", 1, 4, 4, 128, 128, 64, True, None)
    b, _ = bench.work("attention_bwd", 1, 4, 4, 128, 128, 64, True, None)
    assert b == 2.5 * f


def test_traffic_figure_from_committed_profile():
    t, src = bench.measured_traffic(("scores", 1, 32, 32, 4096, 128, "fp16", True))
    assert src == "profiles/attn_fwd_scores_f16_b1h32s4096d128_causal.md"
    algorithmic = bench.work("scores", 1, 32, 32, 4096, 4096, 128, True, None)[1]
    assert algorithmic <= t <= 1.2 * algorithmic


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
