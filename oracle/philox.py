"""Philox4x32 and Triton's tl.rand as the reference's dropout uses them --
TEST INFRASTRUCTURE ONLY (tests/ may use it as the checker; the product path
never imports it).

The reference drops attention weight (b, h, i, j) unless
tl.rand(seed, offset + rowblock_base + ..., n_rounds=6) > dropout_p
(attention_with_scores.py:70-75, 173-176; the same index in every kernel of
the family, e.g. attention_with_col_softmax_sum.py:74-78, 239-244), where
rowblock_base + local row * N + start_n + local column is the linear index
((b*H + h)*M + i)*N + j computed in Triton's int32 arithmetic.  seed and
offset come from dropout.py:5-15.

tl.rand is defined in Triton's open-source triton/language/random.py
(triton 3.x; no Triton kernel is run here):
  * randint4x(seed, offset): counter (offset low word, offset high word for a
    64-bit offset else 0, 0, 0), key (seed low word, seed high word), Philox
    of n_rounds rounds; randint keeps the first word;
  * the Philox round is Random123's philox4x32 round (Salmon, Moraes, Dror,
    Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11): multipliers
    0xD2511F53 (word 0) and 0xCD9E8D57 (word 2), Weyl key increments
    0x9E3779B9 / 0xBB67AE85;
  * uint_to_uniform_float: the word as int32 x, y = x if x >= 0 else -x - 1,
    u = float32(y) * 4.6566127342e-10 in fp32.
Pinned by tests/test_dropout_oracle.py against Random123's published
10-round known-answer vectors and the closed forms of the conversion.
"""
from __future__ import annotations

import numpy as np

M_A, M_B = 0xD2511F53, 0xCD9E8D57
W_A, W_B = 0x9E3779B9, 0xBB67AE85
_MASK = np.uint64(0xFFFFFFFF)
UNIFORM_SCALE = np.float32(4.6566127342e-10)


def philox4x32(ctr, key, rounds: int):
    """Philox4x32-`rounds` of counter words ctr (4 uint32 arrays, broadcast)
    under key (2 uint32 words): 4 uint32 arrays."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint64) & _MASK for c in ctr)
    c0, c1, c2, c3 = np.broadcast_arrays(c0, c1, c2, c3)
    k0, k1 = np.uint64(int(key[0]) & 0xFFFFFFFF), np.uint64(int(key[1]) & 0xFFFFFFFF)
    for _ in range(rounds):
        p0 = np.uint64(M_A) * c0  # 32 x 32 -> 64 bits, exact in uint64
        p2 = np.uint64(M_B) * c2
        c0, c1, c2, c3 = ((p2 >> np.uint64(32)) ^ c1 ^ k0, p2 & _MASK,
                          (p0 >> np.uint64(32)) ^ c3 ^ k1, p0 & _MASK)
        k0 = (k0 + np.uint64(W_A)) & _MASK
        k1 = (k1 + np.uint64(W_B)) & _MASK
    return tuple(x.astype(np.uint32) for x in (c0, c1, c2, c3))


def uniform(x) -> np.ndarray:
    """Triton's uint_to_uniform_float for 32-bit words, in fp32."""
    xi = np.asarray(x, dtype=np.uint32).view(np.int32).astype(np.int64)
    y = np.where(xi < 0, -xi - 1, xi)
    return y.astype(np.float32) * UNIFORM_SCALE


def tl_rand(seed: int, offsets, n_rounds: int = 6, wide: bool = False) -> np.ndarray:
    """tl.rand(seed, offsets, n_rounds): offsets are Triton int32 values
    (taken mod 2^32) unless `wide` (an int64 offset argument)."""
    off = np.asarray(offsets, dtype=np.uint64)
    lo = off & _MASK
    hi = (off >> np.uint64(32)) if wide else np.zeros_like(off)
    seed &= 0xFFFFFFFFFFFFFFFF
    x = philox4x32((lo, hi, 0, 0), (seed & 0xFFFFFFFF, seed >> 32), n_rounds)[0]
    return uniform(x)


def keep_mask(seed: int, offset: int, p: float, b: int, h: int, rows, N: int, H: int,
              M: int) -> np.ndarray:
    """Boolean (len(rows), N) keep mask of query head h of batch b: element
    (i, j) is kept iff tl.rand(seed, offset + ((b*H + h)*M + i)*N + j, 6) > p.

    With an int32 offset (< 2^31) the whole index wraps mod 2^32 as the
    reference's int32 arithmetic does.  A larger offset makes the sum int64
    (then the index itself must stay below 2^31)."""
    rows = np.asarray(rows, dtype=np.int64)
    idx = ((b * H + h) * M + rows[:, None]) * N + np.arange(N, dtype=np.int64)[None, :]
    wide = offset >= 2**31
    if wide:
        assert np.all(idx < 2**31), "the index must stay below 2^31 with a 64-bit offset"
        ctr = (np.int64(offset) + idx).astype(np.uint64)
    else:
        ctr = ((offset + idx) % 2**32).astype(np.uint64)
    return tl_rand(seed, ctr, 6, wide=wide) > np.float32(p)

