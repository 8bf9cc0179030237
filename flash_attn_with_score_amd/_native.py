"""ctypes binding of libfas.so, the gfx950 C ABI declared in include/fas.h.

The library is loaded lazily, after torch (so it binds to the HIP runtime
torch already mapped: both carry the soname libamdhip64.so.7).  There is no
fallback: if the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import struct
import threading
from pathlib import Path

import torch

ABI_VERSION = 8

DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1}

FAS_OK = 0
FAS_ERR_INVALID = -1
FAS_ERR_UNSUPPORTED = -2
FAS_ERR_WORKSPACE = -3
FAS_ERR_HIP = -4

# fas_variant (include/fas.h)
VARIANT_SCORES = 0
VARIANT_ROW_SUM = 1
VARIANT_COL_SUM = 2
VARIANT_COL_SUM_SEQUENTIAL = 3
VARIANT_SOFTMAX_COL_SUM = 4
VARIANT_CROSS_QK_SUM = 5
VARIANT_CROSS_SOFTMAX_SUM = 6
VARIANT_CROSS_SOFTMAX_SUM_BUFFERED = 7
VARIANT_ATTENTION_BACKWARD = 8
VARIANT_ATTENTION_FORWARD = 9
VARIANT_KEEP_BITS = 10  # size of the keep_bits buffer (fas_attn_args.keep_bits)

_I64x4 = ctypes.c_int64 * 4
_I64x3 = ctypes.c_int64 * 3


class AttnArgs(ctypes.Structure):
    """Mirror of struct fas_attn_args (include/fas.h)."""

    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("sm_scale", ctypes.c_float),
        ("reserved", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("heads_q", ctypes.c_int64),
        ("heads_k", ctypes.c_int64),
        ("seqlen_q", ctypes.c_int64),
        ("seqlen_k", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("q_stride", _I64x4),
        ("k_stride", _I64x4),
        ("v_stride", _I64x4),
        ("out_stride", _I64x4),
        ("dropout_p", ctypes.c_float),
        ("reserved2", ctypes.c_int32),
        ("dropout_seed", ctypes.c_uint64),
        ("dropout_offset", ctypes.c_uint64),
        ("keep_bits", ctypes.c_void_p),
    ]


def strides4(t: torch.Tensor):
    return _I64x4(*t.stride())


def strides3(t: torch.Tensor):
    return _I64x3(*t.stride())


# AttnArgs as one packed record (the C struct has no padding), so that a
# call fills it with a single pack instead of ~30 ctypes field writes.
_ARGS_PACK = struct.Struct("<iifi6q4Q16qfiQQQ")
assert _ARGS_PACK.size == ctypes.sizeof(AttnArgs) and AttnArgs.keep_bits.offset == 248


def make_args(q, k, v, o, causal: bool, sm_scale: float, dropout=None,
              keep_bits: int | None = 0) -> AttnArgs:
    """dropout: None, or (dropout_p, seed, offset) of the reference's stream;
    keep_bits: device address of the forward's keep-bit buffer, or 0 (None: 0)."""
    B, H, M, D = q.shape
    if dropout is None:
        dp, seed, offset = 0.0, 0, 0
    else:
        dp = float(dropout[0])
        seed = int(dropout[1]) & 0xFFFFFFFFFFFFFFFF
        offset = int(dropout[2]) & 0xFFFFFFFFFFFFFFFF
    return AttnArgs.from_buffer_copy(_ARGS_PACK.pack(
        DTYPE_CODES[q.dtype], 1 if causal else 0, float(sm_scale), 0,
        B, H, k.shape[1], M, k.shape[2], D,
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
        *q.stride(), *k.stride(), *v.stride(), *o.stride(),
        dp, 0, seed, offset, keep_bits or 0))


_P = ctypes.POINTER
_WS = [ctypes.c_void_p, ctypes.c_size_t]
_SIGNATURES = {
    "fas_abi_version": (ctypes.c_int, []),
    "fas_last_error": (ctypes.c_char_p, []),
    "fas_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, _P(AttnArgs), ctypes.c_int64]),
    "fas_attention_with_scores": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x4, *_WS, ctypes.c_void_p]),
    "fas_attention_scores": (ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x4, ctypes.c_void_p]),
    "fas_attention_with_row_sum": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x3, *_WS, ctypes.c_void_p]),
    "fas_attention_with_col_sum": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x3, *_WS, ctypes.c_void_p]),
    "fas_attention_with_col_sum_sequential": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x3, *_WS, ctypes.c_void_p]),
    "fas_attention_with_softmax_col_sum": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x3, *_WS, ctypes.c_void_p]),
    "fas_attention_with_softmax_col_sum_noalloc": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x3, ctypes.c_void_p]),
    "fas_attention_cross_token_qk_sum": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_int64, ctypes.c_void_p, _I64x3, *_WS, ctypes.c_void_p]),
    "fas_attention_cross_token_softmax_sum": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_int64, ctypes.c_void_p, _I64x3, *_WS, ctypes.c_void_p]),
    "fas_attention_cross_token_softmax_sum_buffered": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_int64, ctypes.c_void_p, _I64x3, *_WS, ctypes.c_void_p]),
    "fas_attention_forward": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x3, *_WS, ctypes.c_void_p]),
    "fas_total_attention": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x3, ctypes.c_void_p, _I64x3, ctypes.c_void_p]),
    "fas_attention_backward": (
        ctypes.c_int, [_P(AttnArgs), ctypes.c_void_p, _I64x4, ctypes.c_void_p, _I64x3,
                       ctypes.c_void_p, _I64x4, ctypes.c_void_p, _I64x4, ctypes.c_void_p, _I64x4,
                       *_WS, ctypes.c_void_p]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def library_path() -> Path:
    override = os.environ.get("FAS_LIBRARY")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / "libfas.so"


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Returns the loaded library, raising if it is missing or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"flash_attn_with_score_amd: native library {path} is not built; run "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`python flash_attn_with_score_amd/csrc/build.py`")
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.fas_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libfas.so ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def last_error(lib) -> str:
    msg = lib.fas_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(lib, rc: int, fn: str) -> None:
    """Maps a negative fas_status to RuntimeError carrying the C message."""
    if rc == FAS_OK:
        return
    msg = last_error(lib) or f"error code {rc}"
    raise RuntimeError(f"{fn}: {msg}")
