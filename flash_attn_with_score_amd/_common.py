"""Launcher plumbing shared by the drop-in entry points.

Each public function in this package follows the reference launcher's steps
(e.g. attention_with_scores.py:239-333): validate shapes with the same
asserts, default sm_scale to 1/sqrt(D), force innermost contiguity, allocate
the outputs with torch on q's device, then make exactly one call into the
gfx950 C ABI on torch's current stream.  Where the reference retries a Triton
launch on an out-of-resources error, the HIP kernels have fixed, compile-time
LDS budgets, so a failing call is reported at once as RuntimeError.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native

SUPPORTED_HEAD_DIMS = {16, 32, 64, 128}


def maybe_contiguous(x: torch.Tensor) -> torch.Tensor:
    """Innermost-contiguous view of x (flash.py:23-26)."""
    return x.contiguous() if x.stride(-1) != 1 else x


def _rows_aligned(x: torch.Tensor) -> bool:
    # The kernels move 16-byte vectors: row starts must be 16-byte aligned.
    s0, s1, s2 = x.stride()[:3]
    return not ((x.data_ptr() & 15) | (s0 & 7) | (s1 & 7) | (s2 & 7))


def as_kernel_operand(x: torch.Tensor) -> torch.Tensor:
    if x.stride(-1) == 1 and _rows_aligned(x):
        return x
    x = maybe_contiguous(x)
    return x if _rows_aligned(x) else x.contiguous()


@dataclass
class Problem:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    B: int
    H: int
    M: int
    N: int
    D: int
    Hk: int
    sm_scale: float


def check_device_inputs(q, k, v, dropout_p: float) -> None:
    """Checks this build adds after the reference's own asserts."""
    if not 0.0 <= dropout_p < 1.0:
        raise ValueError(f"flash_attn_with_score_amd: dropout_p {dropout_p} outside [0, 1)")
    assert q.dtype in _native.DTYPE_CODES, f"q.dtype must be float16 or bfloat16, got {q.dtype}"
    assert k.dtype == q.dtype and v.dtype == q.dtype, "q, k, v must share one dtype"
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("flash_attn_with_score_amd: q, k, v must be HIP device tensors")
    assert k.device == q.device and v.device == q.device, "q, k, v must be on one device"
    assert q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q, k, v must be (B, H, S, D)"
    assert k.shape[0] == q.shape[0] and v.shape[0] == q.shape[0], "batch sizes must match"
    assert v.shape[2] == k.shape[2], "k and v must have the same sequence length"


def draw_dropout(q, k, dropout_p: float):
    """(dropout_p, seed, offset) for a launcher that applies dropout, drawn as
    the reference's launchers draw it: philox_cuda_seed_offset(B*H*M*N)
    before the launch (e.g. attention_with_scores.py:264-268); None when
    dropout_p is 0."""
    if not dropout_p > 0.0:
        return None
    from .dropout import philox_cuda_seed_offset

    B, H, M, _ = q.shape
    seed, offset = philox_cuda_seed_offset(B * H * M * k.shape[2], q.device.index)
    return (dropout_p, seed, offset)


def finish_problem(q, k, v, sm_scale) -> Problem:
    B, H, M, D = q.shape
    N = k.shape[2]
    Hk = k.shape[1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    q, k, v = as_kernel_operand(q), as_kernel_operand(k), as_kernel_operand(v)
    return Problem(q, k, v, B, H, M, N, D, Hk, float(sm_scale))


def new_output(q: torch.Tensor) -> torch.Tensor:
    o = torch.empty_like(q)
    return o if _rows_aligned(o) and o.stride(-1) == 1 else torch.empty(
        q.shape, dtype=q.dtype, device=q.device)


def _raw_stream(index: int) -> int:
    return torch.cuda.current_stream(index).cuda_stream


# torch's current stream of a device as a raw handle without building a
# Stream object (the call costs ~0.3 us instead of several).
_current_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", _raw_stream)


def call(fn_name: str, q: torch.Tensor, *args) -> None:
    """Invokes one C entry point on q's device and torch's current stream."""
    lib = _native.load()
    fn = getattr(lib, fn_name)
    index = q.device.index
    if index == torch.cuda.current_device():
        rc = fn(*args, _current_raw_stream(index))
    else:
        with torch.cuda.device(index):
            rc = fn(*args, _current_raw_stream(index))
    _native.check(lib, rc, fn_name)


def workspace(variant: int, args, split: int, device,
              limit: int | None = None) -> tuple[int, int, torch.Tensor | None]:
    """Allocates the device workspace an entry point needs (torch caching
    allocator, 256-byte aligned) and returns (pointer, bytes, tensor); with
    `limit`, a workspace larger than that is not allocated (pointer 0, no
    tensor) and the caller takes its route without it."""
    import ctypes

    lib = _native.load()
    nbytes = lib.fas_workspace_bytes(variant, ctypes.byref(args), int(split))
    if nbytes == ctypes.c_size_t(-1).value:
        raise RuntimeError(f"fas_workspace_bytes: {_native.last_error(lib) or 'invalid request'}")
    if nbytes == 0 or (limit is not None and nbytes > limit):
        return 0, nbytes, None
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    ptr = buf.data_ptr()
    ptr += (-ptr) % 256
    return ptr, nbytes, buf
