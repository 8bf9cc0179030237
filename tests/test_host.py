"""Host-side tests of the boundary -- run without a GPU.

  * libfas.so loads (built by __graft_entry__.build()) and exports exactly
    the functions include/fas.h declares, with the ctypes signatures of
    flash_attn_with_score_amd/_native.py;
  * fas_workspace_bytes sizes each variant's workspace as documented;
  * invalid requests are rejected with the right status and a message that
    names the entry point, before any HIP call is made;
  * the Python launchers keep the reference's asserts
    (e.g. attention_with_scores.py:240-247, attention_cross_token_qk_sum.py:298-307)
    and fail loudly instead of falling back to a CPU path;
  * the product package never imports the test oracle.
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

import flash_attn_with_score_amd as fas
from flash_attn_with_score_amd import _common, _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fas.h")

SIZE_MAX = ctypes.c_size_t(-1).value


@pytest.fixture(scope="module")
def lib():
    return _native.load()


def header_functions():
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(fas_\w+)\s*\(", text, re.M))


def test_library_loads_with_abi_version(lib):
    assert lib.fas_abi_version() == _native.ABI_VERSION == 8
    m = re.search(r"#define FAS_ABI_VERSION (\d+)", open(HEADER).read())
    assert m and int(m.group(1)) == _native.ABI_VERSION


def test_keep_bits_size(lib):
    """FAS_VARIANT_KEEP_BITS sizes the caller's keep-bit buffer: with dropout,
    B*Hq*ceil(M/32)*N*4 bytes of key-major words, plus B*Hq*Mpad*ceil(N/32)*4
    of row blocks (256-byte-aligned parts) only when the backward cannot
    store dS (more than 16 GiB of it); 0 without dropout."""
    q = torch.empty(2, 3, 100, 64, dtype=torch.float16)
    k = torch.empty(2, 3, 70, 64, dtype=torch.float16)
    a = _native.make_args(q, k, k, q, True, 0.125, (0.1, 1, 0))
    keys = 2 * 3 * 4 * 70 * 4                   # ceil(100/32) = 4 row words per key
    al = lambda x: (x + 255) // 256 * 256
    assert lib.fas_workspace_bytes(_native.VARIANT_KEEP_BITS, ctypes.byref(a), 0) == al(keys)
    # B1 H64 S32768 causal: 64 * 524,800 dS blocks of 2 KiB (68.8 GB) exceed
    # 16 GiB, so the row blocks are included (sizes only, nothing allocated).
    big = make_args(1, 64, 64, 32768, 32768, 64)
    big.dropout_p, big.dropout_seed = 0.1, 1
    keys = 64 * 1024 * 32768 * 4
    rows = 64 * 32768 * 1024 * 4
    assert lib.fas_workspace_bytes(_native.VARIANT_KEEP_BITS, ctypes.byref(big), 0) == al(keys) + al(rows)
    b = _native.make_args(q, k, k, q, True, 0.125)
    assert lib.fas_workspace_bytes(_native.VARIANT_KEEP_BITS, ctypes.byref(b), 0) == 0


def test_exports_match_header(lib):
    declared = header_functions()
    assert declared == set(_native.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_public_api_matches_reference_names():
    """__init__.py:29-39 of the reference."""
    assert set(fas.__all__) == {
        "attention", "attention_with_scores", "attention_with_row_sum", "attention_with_col_sum",
        "attention_with_col_sum_sequential", "attention_with_softmax_col_sum",
        "attention_cross_token_qk_sum", "attention_cross_token_softmax_sum",
        "attention_cross_token_softmax_sum_buffered"}


def make_args(B=1, Hq=4, Hk=2, M=300, N=300, D=128, causal=1, dtype=0, ptr=0x10000):
    a = _native.AttnArgs()
    a.dtype, a.causal, a.sm_scale = dtype, causal, 1.0 / (D ** 0.5)
    a.batch, a.heads_q, a.heads_k, a.seqlen_q, a.seqlen_k, a.head_dim = B, Hq, Hk, M, N, D
    a.q = a.k = a.v = a.out = ptr  # never dereferenced by the rejected calls below
    for name, H, L in (("q_stride", Hq, M), ("k_stride", Hk, N), ("v_stride", Hk, N),
                       ("out_stride", Hq, M)):
        setattr(a, name, _native._I64x4(H * L * D, L * D, D, 1))
    return a


def _col_plan(B, Hq, Hk, ncols, buffered, cus=256):
    """Head split of the softmax column pass, restated: the fold's G query
    heads are dealt to nsplit workgroups per unit (a mirror pair of 256-key
    blocks, or one key block of the buffered pass); nsplit is the smallest of
    least cost, cost = rounds of concurrent workgroups x heads per workgroup.
    Returns (nsplit, units, output groups)."""
    G = Hq // Hk
    groups = B * Hk
    if buffered:
        bk = 256 if ncols % 4 == 0 else 64
        units, slots = -(-ncols // bk), 8 * cus
    else:
        units, slots = (-(-ncols // 256) + 1) // 2, cus
    cost = {ns: -(-(units * ns * groups) // slots) * -(-G // ns) for ns in range(1, G + 1)}
    best = min(cost.values())
    return min(ns for ns, c in cost.items() if c == best), units, groups


def test_col_plan_examples():
    """The plan on the BASELINE shapes: 7 splits for 4 KV heads of 7 query
    heads (224 workgroups instead of 32), none at 8 KV heads x 32 pairs (256
    workgroups), one head per workgroup for the cross-token pass at split
    12288 (768 workgroups in 3 rounds beat 192 in one round of 4 heads)."""
    assert _col_plan(1, 28, 4, 4096, False) == (7, 8, 4)
    assert _col_plan(1, 32, 8, 16384, False) == (1, 32, 8)
    assert _col_plan(1, 32, 8, 12288, False) == (4, 24, 8)
    assert _col_plan(1, 32, 32, 4096, False) == (1, 8, 32)
    assert _col_plan(1, 32, 8, 12288, True) == (4, 48, 8)


def test_workspace_sizes(lib):
    B, Hq, Hk, M, N, D, split = 2, 8, 2, 300, 300, 64, 100

    def r256(x):
        return (x + 255) // 256 * 256

    def folds(ncols, buffered):
        ns, units, groups = _col_plan(B, Hq, Hk, ncols, buffered)
        return 0 if ns == 1 else r256(groups * ns * ncols * 4) + r256(groups * units * 4)

    a = make_args(B, Hq, Hk, M, N, D)
    ws = lambda v: lib.fas_workspace_bytes(v, ctypes.byref(a), split)  # noqa: E731
    assert ws(_native.VARIANT_SCORES) == 0
    assert ws(_native.VARIANT_ROW_SUM) == 0
    nblk = (M + 63) // 64
    assert ws(_native.VARIANT_COL_SUM) == r256(B * Hk * (nblk + 1) * D * 4)
    assert ws(_native.VARIANT_COL_SUM_SEQUENTIAL) == ws(_native.VARIANT_COL_SUM)
    assert folds(N, False) > 0  # 4 query heads per KV head, 4 workgroups unsplit: split
    assert ws(_native.VARIANT_SOFTMAX_COL_SUM) == r256(B * Hq * M * 4) + folds(N, False)
    assert ws(_native.VARIANT_CROSS_QK_SUM) == r256(B * Hk * ((M - split + 63) // 64 + 1) * D * 4)
    assert ws(_native.VARIANT_CROSS_SOFTMAX_SUM) == r256(B * Hq * M * 4) + folds(split, False)
    # The buffered region: fp16 exponents, then one fp32 offset per row and
    # 64-key tile.
    assert ws(_native.VARIANT_CROSS_SOFTMAX_SUM_BUFFERED) == (
        r256(B * Hq * M * 4) + folds(split, True) + r256(B * Hq * (M - split) * split * 2)
        + r256(B * Hq * (M - split) * ((split + 63) // 64) * 4))
    # MHA needs no per-query-head partials.
    a1 = make_args(B, 4, 4, M, N, D)
    assert lib.fas_workspace_bytes(_native.VARIANT_SOFTMAX_COL_SUM, ctypes.byref(a1), 0) == \
        r256(B * 4 * M * 4)


def _ds_blocks(M, N, causal):
    """dS blocks (32 rows x 32 keys) the backward stores per head, counted one
    by one: rows padded to whole 128-row blocks, and under the causal mask
    only blocks holding a visible pair, (N - M) + i >= j for some row i and
    key j of the block."""
    mpad = (M + 127) // 128 * 128
    n32 = (N + 31) // 32
    return sum(1 for r in range(mpad // 32) for j in range(n32)
               if not causal or (N - M) + 32 * r + 31 >= 32 * j)


def test_attention_backward_workspace(lib):
    """Two (B*Hq, Mpad) fp32 row arrays, Mpad = M rounded up to 128, plus
    per-query-head fp32 dK|dV partials only when Hq > Hk and the KV-head
    grid B*Hk*ceil(N/128) is below 256 workgroups, plus 2 KiB per stored dS
    block, which a query with split != 0 leaves out."""
    def r256(x):
        return (x + 255) // 256 * 256

    def ws(a, split=0):
        return lib.fas_workspace_bytes(_native.VARIANT_ATTENTION_BACKWARD, ctypes.byref(a), split)

    B, Hq, Hk, M, N, D = 2, 8, 2, 300, 500, 64
    a = make_args(B, Hq, Hk, M, N, D)
    mpad = 384
    base = 2 * r256(B * Hq * mpad * 4) + r256(B * Hq * N * 2 * D * 4)
    assert ws(a, 1) == base
    assert ws(a) == base + r256(B * Hq * _ds_blocks(M, N, True) * 2048)
    a = make_args(64, 8, 4, 128, 128, 32)  # 64 * 4 * 1 = 256 workgroups: no partials
    assert ws(a, 1) == 2 * r256(64 * 8 * 128 * 4)
    a = make_args(1, 4, 4, 100, 100, 128)  # MHA: no partials
    assert ws(a, 1) == 2 * r256(4 * 128 * 4)
    assert ws(a) == 2 * r256(4 * 128 * 4) + r256(4 * _ds_blocks(100, 100, True) * 2048)


@pytest.mark.parametrize("M,N", [(300, 500), (500, 300), (1, 64), (130, 100), (2000, 40),
                                 (40, 2000), (4096, 4096), (777, 1025), (100, 4000)])
@pytest.mark.parametrize("causal", [1, 0])
def test_attention_backward_ds_blocks(lib, M, N, causal):
    """The library's closed-form count of stored dS blocks (per-row-block
    prefix sums of clamped visible-block counts) against the count made block
    by block, for M < N, M > N (rows with no key), ragged and tiny shapes."""
    def r256(x):
        return (x + 255) // 256 * 256

    a = make_args(1, 2, 2, M, N, 64, causal=causal)
    full = lib.fas_workspace_bytes(_native.VARIANT_ATTENTION_BACKWARD, ctypes.byref(a), 0)
    nods = lib.fas_workspace_bytes(_native.VARIANT_ATTENTION_BACKWARD, ctypes.byref(a), 1)
    assert full - nods == r256(2 * _ds_blocks(M, N, causal) * 2048)


def test_attention_entry_points_reject_bad_requests(lib):
    a = make_args()
    st3 = _native._I64x3(300, 1, 1)
    st4 = _native._I64x4(4 * 300 * 128, 300 * 128, 128, 1)
    kst = _native._I64x4(2 * 300 * 128, 300 * 128, 128, 1)
    # forward: the normalizer output is required
    assert lib.fas_attention_forward(ctypes.byref(a), None, st3, None, 0, None) == _native.FAS_ERR_INVALID
    assert "fas_attention_forward" in _err(lib) and "lse" in _err(lib)
    # backward: a NULL dout, a misaligned dk, a workspace short of the
    # minimum (the size without the stored dS)
    need = lib.fas_workspace_bytes(_native.VARIANT_ATTENTION_BACKWARD, ctypes.byref(a), 1)
    rc = lib.fas_attention_backward(ctypes.byref(a), None, st4, 0x10000, st3, 0x10000, st4,
                                    0x10000, kst, 0x10000, kst, 0x10000, need, None)
    assert rc == _native.FAS_ERR_INVALID and "dout is NULL" in _err(lib)
    rc = lib.fas_attention_backward(ctypes.byref(a), 0x10000, st4, 0x10000, st3, 0x10000, st4,
                                    0x10008, kst, 0x10000, kst, 0x10000, need, None)
    assert rc == _native.FAS_ERR_INVALID and "dk rows must be 16-byte aligned" in _err(lib)
    rc = lib.fas_attention_backward(ctypes.byref(a), 0x10000, st4, 0x10000, st3, 0x10000, st4,
                                    0x10000, kst, 0x10000, kst, 0x10000, need - 1, None)
    assert rc == _native.FAS_ERR_WORKSPACE and "fas_attention_backward" in _err(lib)
    # total attention: unsupported head dim
    bad = make_args(D=48)
    rc = lib.fas_total_attention(ctypes.byref(bad), 0x10000, st3, 0x10000, st3, None)
    assert rc == _native.FAS_ERR_UNSUPPORTED and "head_dim 48" in _err(lib)


def test_key_split_workspace(lib):
    """Short query range against long keys: B*Hq*ceil(M/256) = 4 workgroups,
    32 key tiles -> 4 splits of 8 tiles; partials (B*Hq*4*256) x (D + 3) fp32."""
    def r256(x):
        return (x + 255) // 256 * 256

    B, Hq, Hk, M, N, D = 1, 4, 2, 32, 2048, 128
    a = make_args(B, Hq, Hk, M, N, D)
    rows = B * Hq * 4 * 256
    split = r256(rows * D * 4) + 3 * r256(rows * 4)
    ws = lambda v, s=0: lib.fas_workspace_bytes(v, ctypes.byref(a), s)  # noqa: E731
    assert ws(_native.VARIANT_ROW_SUM) == split
    assert ws(_native.VARIANT_ATTENTION_FORWARD) == split
    ns, units, groups = _col_plan(B, Hq, Hk, N, False)
    assert ns == 2
    assert ws(_native.VARIANT_SOFTMAX_COL_SUM) == (
        r256(B * Hq * M * 4) + r256(groups * ns * N * 4) + r256(groups * units * 4) + split)
    assert ws(_native.VARIANT_SCORES) == split  # key-split forward + scores-only kernel
    # enough row blocks: no split
    a = make_args(1, 32, 32, 4096, 4096, 128)
    assert lib.fas_workspace_bytes(_native.VARIANT_ROW_SUM, ctypes.byref(a), 0) == 0


def test_workspace_rejects_bad_requests(lib):
    a = make_args()
    assert lib.fas_workspace_bytes(_native.VARIANT_CROSS_QK_SUM, ctypes.byref(a), 0) == SIZE_MAX
    assert lib.fas_workspace_bytes(_native.VARIANT_CROSS_QK_SUM, ctypes.byref(a), 301) == SIZE_MAX
    assert lib.fas_workspace_bytes(99, ctypes.byref(a), 1) == SIZE_MAX
    bad = make_args(D=48)
    assert lib.fas_workspace_bytes(_native.VARIANT_COL_SUM, ctypes.byref(bad), 0) == SIZE_MAX


def _err(lib):
    return _native.last_error(lib)


def test_rejects_unsupported_head_dim(lib):
    a = make_args(D=48)
    st = _native._I64x4(1, 1, 1, 1)
    rc = lib.fas_attention_with_scores(ctypes.byref(a), 0x10000, st, None, 0, None)
    assert rc == _native.FAS_ERR_UNSUPPORTED
    assert "fas_attention_with_scores" in _err(lib) and "head_dim 48" in _err(lib)


def test_rejects_bad_heads_and_dtype(lib):
    a = make_args(Hq=6, Hk=4)
    st = _native._I64x3(1, 1, 1)
    assert lib.fas_attention_with_row_sum(ctypes.byref(a), 0x10000, st, None, 0, None) == _native.FAS_ERR_INVALID
    assert "multiple" in _err(lib)
    a = make_args(dtype=7)
    assert lib.fas_attention_with_row_sum(ctypes.byref(a), 0x10000, st, None, 0, None) == \
        _native.FAS_ERR_UNSUPPORTED


def test_rejects_null_and_misaligned_tensors(lib):
    st = _native._I64x3(1, 1, 1)
    a = make_args()
    a.q = None
    assert lib.fas_attention_with_row_sum(ctypes.byref(a), 0x10000, st, None, 0, None) == _native.FAS_ERR_INVALID
    assert "q is NULL" in _err(lib)
    a = make_args()
    a.k_stride = _native._I64x4(2 * 300 * 128, 300 * 128, 130, 1)  # row stride not a multiple of 8
    assert lib.fas_attention_with_row_sum(ctypes.byref(a), 0x10000, st, None, 0, None) == _native.FAS_ERR_INVALID
    assert "k rows must be 16-byte aligned" in _err(lib)
    a = make_args()
    a.v_stride = _native._I64x4(2 * 300 * 128, 300 * 128, 128, 2)
    assert lib.fas_attention_with_row_sum(ctypes.byref(a), 0x10000, st, None, 0, None) == _native.FAS_ERR_INVALID
    assert "innermost stride" in _err(lib)


def test_rejects_split_out_of_range(lib):
    a = make_args()
    st = _native._I64x3(1, 1, 1)
    for split in (0, -3, 301):
        rc = lib.fas_attention_cross_token_softmax_sum(ctypes.byref(a), split, 0x10000, st,
                                                       0x10000, 1 << 30, None)
        assert rc == _native.FAS_ERR_INVALID, split
        assert "split" in _err(lib)


def test_rejects_short_workspace(lib):
    a = make_args()
    st = _native._I64x3(1, 1, 1)
    need = lib.fas_workspace_bytes(_native.VARIANT_SOFTMAX_COL_SUM, ctypes.byref(a), 0)
    rc = lib.fas_attention_with_softmax_col_sum(ctypes.byref(a), 0x10000, st, 0x10000, need - 1,
                                                None)
    assert rc == _native.FAS_ERR_WORKSPACE and str(need) in _err(lib)
    rc = lib.fas_attention_with_col_sum(ctypes.byref(a), 0x10000, st, None, 0, None)
    assert rc == _native.FAS_ERR_WORKSPACE


def test_error_code_maps_to_runtime_error():
    class FakeLib:
        @staticmethod
        def fas_last_error():
            return b"fas_attention_with_scores: HIP launch failed: out of memory"

    with pytest.raises(RuntimeError, match="HIP launch failed: out of memory"):
        _native.check(FakeLib(), _native.FAS_ERR_HIP, "fas_attention_with_scores")
    _native.check(FakeLib(), _native.FAS_OK, "fas_attention_with_scores")


# ------------------------------------------------------------ launchers

def _cpu_qkv(D=64, H=4, Hk=4, Hv=None, M=32, N=32, dtype=torch.float16):
    q = torch.zeros(1, H, M, D, dtype=dtype)
    k = torch.zeros(1, Hk, N, D, dtype=dtype)
    v = torch.zeros(1, Hv or Hk, N, D, dtype=dtype)
    return q, k, v


@pytest.mark.parametrize("fn", sorted(fas.__all__))
def test_launcher_keeps_reference_asserts(fn):
    f = getattr(fas, fn)
    split = ("cross" in fn,)
    args = (16,) if split[0] else ()
    q, k, v = _cpu_qkv(D=48)
    with pytest.raises(AssertionError):
        f(q, k, v, *args)
    q, k, v = _cpu_qkv(H=6, Hk=4)
    with pytest.raises(AssertionError):
        f(q, k, v, *args)
    q, k, v = _cpu_qkv(Hk=2, Hv=4)
    with pytest.raises(AssertionError):
        f(q, k, v, *args)
    if split[0]:
        q, k, v = _cpu_qkv()
        with pytest.raises(AssertionError):
            f(q, k, v, 0)
        with pytest.raises(AssertionError):
            f(q, k, v, 33)


@pytest.mark.parametrize("fn", sorted(fas.__all__))
def test_launcher_fails_loudly_without_device(fn):
    """No CPU fallback: host tensors are rejected, with or without dropout."""
    f = getattr(fas, fn)
    args = (16,) if "cross" in fn else ()
    q, k, v = _cpu_qkv()
    with pytest.raises(RuntimeError, match="HIP device"):
        f(q, k, v, *args, causal=True)
    with pytest.raises(RuntimeError, match="HIP device"):
        f(q, k, v, *args, causal=True, dropout_p=0.1)
    # fp32: accepted by the reference (TF32 products in Triton), rejected here
    with pytest.raises(AssertionError, match="float16 or bfloat16"):
        f(q.float(), k.float(), v.float(), *args)


def test_package_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "flash_attn_with_score_amd")
    for dirpath, _, files in os.walk(pkg):
        for name in files:
            if name.endswith(".py"):
                text = open(os.path.join(dirpath, name)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), name


def test_rows_aligned_helper():
    x = torch.zeros(2, 3, 5, 64, dtype=torch.float16)
    assert _common._rows_aligned(x)
    assert not _common._rows_aligned(x[..., 1:])


def test_dropout_requests(lib):
    """Dropout arguments are validated before anything is launched."""
    st3 = _native._I64x3(1, 1, 1)
    st4 = _native._I64x4(1, 1, 1, 1)
    for bad in (1.0, -0.25, float("nan")):
        a = make_args()
        a.dropout_p = bad
        rc = lib.fas_attention_with_row_sum(ctypes.byref(a), 0x10000, st3, None, 0, None)
        assert rc == _native.FAS_ERR_INVALID and "dropout_p" in _err(lib)
    # a 64-bit offset with an element index past 2^31: the reference's index
    # would depend on its block sizes
    a = make_args(B=1, Hq=4, Hk=4, M=32768, N=32768, D=64)
    a.dropout_p, a.dropout_offset = 0.1, 2**31
    rc = lib.fas_attention_with_row_sum(ctypes.byref(a), 0x10000, st3, None, 0, None)
    assert rc == _native.FAS_ERR_UNSUPPORTED and "2^31" in _err(lib)
    # the backward pass validates dropout_p like the forward
    a = make_args()
    a.dropout_p = 1.5
    rc = lib.fas_attention_backward(ctypes.byref(a), 0x10000, st4, 0x10000, st3, 0x10000, st4,
                                    0x10000, st4, 0x10000, st4, None, 0, None)
    assert rc == _native.FAS_ERR_INVALID and "dropout_p" in _err(lib)


def test_dropout_p_checked_in_python():
    import torch
    from flash_attn_with_score_amd import _common

    t = torch.zeros(1, 1, 4, 16, dtype=torch.float16)
    for bad in (1.0, -0.1):
        with pytest.raises(ValueError, match="dropout_p"):
            _common.check_device_inputs(t, t, t, bad)


def test_make_args_packs_every_field():
    """make_args fills struct fas_attn_args with one packed record: every
    field reads back as written, including strides of views, negative
    sm_scale and 64-bit dropout seed and offset."""
    q = torch.empty(2, 100, 6, 64, dtype=torch.bfloat16).transpose(1, 2)
    k = torch.empty(2, 3, 70, 64, dtype=torch.bfloat16)
    v = torch.empty(2, 3, 70, 64, dtype=torch.bfloat16)
    o = torch.empty(2, 6, 100, 64, dtype=torch.bfloat16)
    a = _native.make_args(q, k, v, o, True, -0.25, (0.1, 2**63 + 5, 2**40 + 7))
    assert (a.dtype, a.causal, a.sm_scale, a.reserved) == (1, 1, -0.25, 0)
    assert (a.batch, a.heads_q, a.heads_k, a.seqlen_q, a.seqlen_k, a.head_dim) == (
        2, 6, 3, 100, 70, 64)
    assert (a.q, a.k, a.v, a.out) == (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr())
    assert tuple(a.q_stride) == q.stride() and tuple(a.k_stride) == k.stride()
    assert tuple(a.v_stride) == v.stride() and tuple(a.out_stride) == o.stride()
    assert a.dropout_p == pytest.approx(0.1) and a.reserved2 == 0
    assert (a.dropout_seed, a.dropout_offset) == (2**63 + 5, 2**40 + 7)
    b = _native.make_args(o, k, v, o, False, 0.5)
    assert (b.dtype, b.causal, b.dropout_p, b.dropout_seed, b.dropout_offset) == (1, 0, 0.0, 0, 0)
