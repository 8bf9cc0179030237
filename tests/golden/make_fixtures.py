"""Writes the golden fixtures under tests/golden/ -- TEST INFRASTRUCTURE.

The reference ships no test vectors (its only check, benchmark.py:1241-1907,
prints errors and asserts nothing), so the fixtures are computed with
oracle/brute.py: an independent fp64 formulation of the reference's naive
attention (reference_implementations.py:11-52) with explicit loops, no matrix
products and no torch.softmax, plus the side products the kernels return.
tests/test_oracle.py checks oracle/naive.py against them.

Inputs are stored in the fixture (fp32), so the check does not depend on the
random generator of the torch build that reads them.

  F1  BASELINE config 1: B=1, H=4, S=256, D=64, fp32, causal, seed 0,
      sm_scale = 1/sqrt(64); output, scores (-inf at masked pairs), row sums
      and column sums of raw scores and of softmax weights
  F2  GQA: B=1, Hq=4, Hk=2, S=64, D=32, causal, seed 1
  F3  cross-token: B=1, Hq=2, Hk=1, M=N=128, D=16, split=96, seed 2,
      causal and non-causal, with cross-token raw and softmax sums
  F4  M != N: (M, N) = (48, 80) and (80, 48), B=1, H=2, D=16, causal
      (bottom-right aligned, and top-left as the cross-QK kernel masks)

Run: python tests/golden/make_fixtures.py   (about a minute)
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import brute  # noqa: E402


def qkv(B, Hq, Hk, M, N, D, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, M, D)).astype(np.float32)
    k = rng.standard_normal((B, Hk, N, D)).astype(np.float32)
    v = rng.standard_normal((B, Hk, N, D)).astype(np.float32)
    return q, k, v


def save(name, q, k, v, res, **meta):
    arrays = {"q": q, "k": k, "v": v}
    for key, val in res.items():
        if key == "weights":
            continue
        arrays[key] = np.asarray(val, dtype=np.float32)
    for key, val in meta.items():
        arrays["meta_" + key] = np.asarray(val)
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


def main():
    # F1: BASELINE config 1.
    q, k, v = qkv(1, 4, 4, 256, 256, 64, seed=0)
    res = brute.brute_forward(q, k, v, causal=True, sm_scale=1.0 / math.sqrt(64))
    save("f1_config1_causal", q, k, v, res, causal=1, sm_scale=1.0 / 8, causal_offset=0)

    # F2: GQA head grouping.
    q, k, v = qkv(1, 4, 2, 64, 64, 32, seed=1)
    res = brute.brute_forward(q, k, v, causal=True)
    save("f2_gqa_causal", q, k, v, res, causal=1, sm_scale=1.0 / math.sqrt(32), causal_offset=0)

    # F3: cross-token sums.
    q, k, v = qkv(1, 2, 1, 128, 128, 16, seed=2)
    for causal in (True, False):
        res = brute.brute_forward(q, k, v, causal=causal, split=96)
        save(f"f3_cross_{'causal' if causal else 'full'}", q, k, v, res, causal=int(causal),
             sm_scale=1.0 / 4, causal_offset=0, split=96)

    # F4: M != N, both causal alignments.
    for M, N in ((48, 80), (80, 48)):
        q, k, v = qkv(1, 2, 2, M, N, 16, seed=3)
        res = brute.brute_forward(q, k, v, causal=True)  # bottom-right (N - M)
        save(f"f4_m{M}_n{N}_bottomright", q, k, v, res, causal=1, sm_scale=1.0 / 4,
             causal_offset=N - M)
        res = brute.brute_forward(q, k, v, causal=True, causal_offset=0)
        save(f"f4_m{M}_n{N}_topleft", q, k, v, res, causal=1, sm_scale=1.0 / 4, causal_offset=0)


if __name__ == "__main__":
    main()
