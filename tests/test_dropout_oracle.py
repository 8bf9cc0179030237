"""The dropout stream's CPU restatement (oracle/philox.py) against published
vectors and closed forms."""
import numpy as np
import pytest

from oracle import philox

# Random123's known-answer vectors for philox4x32, 10 rounds
# (Random123 distribution, examples/kat_vectors): counter, key, output.
KAT_10 = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,out", KAT_10)
def test_philox_known_answers(ctr, key, out):
    got = philox.philox4x32(ctr, key, 10)
    assert tuple(int(x) for x in got) == out


def test_planted_multiplier_swap_fails(monkeypatch):
    """Exchanging the two round multipliers (a plausible slip) breaks the vectors."""
    monkeypatch.setattr(philox, "M_A", 0xCD9E8D57)
    monkeypatch.setattr(philox, "M_B", 0xD2511F53)
    ctr, key, out = KAT_10[2]
    assert tuple(int(x) for x in philox.philox4x32(ctr, key, 10)) != out


def test_rounds_compose():
    """Philox-6 is the first 6 rounds of Philox-10 with the key advanced:
    running 4 more rounds from Philox-6's state under the key bumped 6 times
    gives Philox-10."""
    rng = np.random.default_rng(0)
    ctr = tuple(rng.integers(0, 2**32, size=64, dtype=np.uint64) for _ in range(4))
    key = (0x12345678, 0x9ABCDEF0)
    six = philox.philox4x32(ctr, key, 6)
    k6 = ((key[0] + 6 * philox.W_A) % 2**32, (key[1] + 6 * philox.W_B) % 2**32)
    ten = philox.philox4x32(six, k6, 4)
    for a, b in zip(ten, philox.philox4x32(ctr, key, 10)):
        assert np.array_equal(a, b)


def test_uniform_closed_forms():
    u = philox.uniform(np.array([0, 1, 0xFFFFFFFF, 0xFFFFFFFE, 0x7FFFFFFF, 0x80000000],
                                dtype=np.uint32))
    s = np.float32(4.6566127342e-10)
    assert u[0] == 0.0 and u[2] == 0.0          # x = 0 and x = -1 -> y = 0
    assert u[1] == s and u[3] == s              # x = 1 and x = -2 -> y = 1
    # x = 2^31 - 1 and x = -2^31 -> y = 2^31 - 1, float32 rounds it to 2^31:
    # the largest uniform, still below 1 (the scale's purpose).
    assert u[4] == u[5] == np.float32(2.0**31) * s
    assert u[4] < 1.0
    assert u.dtype == np.float32


def test_keep_fraction():
    """Kept fraction of 2^20 consecutive offsets is 1 - p within 5 sigma."""
    p = 0.3
    kept = philox.tl_rand(1234, np.arange(2**20), 6) > np.float32(p)
    n = kept.size
    assert abs(kept.mean() - (1 - p)) < 5 * np.sqrt(p * (1 - p) / n)


def test_keep_mask_index():
    """keep_mask indexes the stream by offset + ((b*H + h)*M + i)*N + j,
    wrapping mod 2^32 for int32 offsets."""
    seed, off, p = 77, 2**31 - 5, 0.5
    B, H, M, N = 1, 3, 4, 5
    m = philox.keep_mask(seed, off, p, 0, 2, range(M), N, H, M)
    idx = (2 * M + np.arange(M)[:, None]) * N + np.arange(N)[None, :]
    ref = philox.tl_rand(seed, (off + idx) % 2**32, 6) > np.float32(p)
    assert np.array_equal(m, ref)
    # a 64-bit offset uses the counter's high word
    big = 2**32 + 9
    m64 = philox.keep_mask(seed, big, p, 0, 0, range(M), N, H, M)
    lo = philox.keep_mask(seed, 9, p, 0, 0, range(M), N, H, M)
    assert not np.array_equal(m64, lo)


def test_keep_interval_form():
    """The kernels test "uniform(x) > p" as (x - (t + 1)) mod 2^32 <
    2^32 - 2t - 2, t the largest y whose uniform is <= p: the same decision
    as Triton's folding y = x or -x - 1 (x as int32), over the words where
    the two could part (around 0, +-t, 2^31) and random ones."""
    rng = np.random.default_rng(7)
    for p in (1e-6, 0.1, 0.5, 0.9, 0.999):
        # t by bisection over fp32 uniforms, as the host computes it.
        lo, hi = 0, 2**31 - 1
        while hi - lo > 1:
            mid = (lo + hi) // 2
            if philox.uniform(np.uint32(mid)) <= np.float32(p):
                lo = mid
            else:
                hi = mid
        t = lo
        edges = [0, 1, 2**31 - 1, 2**31, 2**32 - 1, t, t + 1, t + 2, 2**32 - t - 3,
                 2**32 - t - 2, 2**32 - t - 1, 2**32 - t]
        x = np.concatenate([np.array([e % 2**32 for e in edges], dtype=np.uint64),
                            rng.integers(0, 2**32, size=20000, dtype=np.uint64)])
        want = philox.uniform(x.astype(np.uint32)) > np.float32(p)
        got = ((x - np.uint64(t + 1)) % np.uint64(2**32)) < np.uint64(2**32 - 2 * t - 2)
        assert np.array_equal(got, want), p


def test_split_first_rounds():
    """The kernels' Philox-6 on counter (x0, w1, 0, 0): round 0's word-2
    product is zero and round 1's word-0 product A (w1 ^ k0) is precomputed
    per value of w1 (w1 = offset high word + carry of offset + index).  The
    split form gives Philox's word 0 for both values of the carry."""
    rng = np.random.default_rng(3)
    key = (0x89ABCDEF, 0x01234567)
    mask = 0xFFFFFFFF
    for w1 in (0, 5, 0x7FFFFFFF):
        x0 = rng.integers(0, 2**32, size=4096, dtype=np.uint64)
        want = philox.philox4x32((x0, np.uint64(w1), 0, 0), key, 6)[0].astype(np.uint64)
        pa1 = philox.M_A * ((w1 ^ key[0]) & mask)
        p0 = np.uint64(philox.M_A) * x0
        p1 = np.uint64(philox.M_B) * ((p0 >> np.uint64(32)) ^ np.uint64(key[1]))
        c0 = (p1 >> np.uint64(32)) ^ np.uint64((key[0] + philox.W_A) & mask)
        c1 = p1 & np.uint64(mask)
        c2 = np.uint64((pa1 >> 32) ^ ((key[1] + philox.W_B) & mask)) ^ (p0 & np.uint64(mask))
        c3 = np.uint64(pa1 & mask)
        c3 = np.broadcast_to(c3, x0.shape)
        k0, k1 = (key[0] + 2 * philox.W_A) & mask, (key[1] + 2 * philox.W_B) & mask
        for _ in range(4):
            pa = np.uint64(philox.M_A) * c0
            pb = np.uint64(philox.M_B) * c2
            c0, c1, c2, c3 = ((pb >> np.uint64(32)) ^ c1 ^ np.uint64(k0), pb & np.uint64(mask),
                              (pa >> np.uint64(32)) ^ c3 ^ np.uint64(k1), pa & np.uint64(mask))
            k0, k1 = (k0 + philox.W_A) & mask, (k1 + philox.W_B) & mask
        assert np.array_equal(c0, want), w1
