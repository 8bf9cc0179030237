"""philox_cuda_seed_offset: the dropout stream's (seed, offset) pair.

Drop-in for the reference's dropout.py:5-15.  It reads the device's default
generator state, (seed, philox offset) as two int64 words, returns them, and
advances the generator's offset by the increment rounded up to a multiple of
4, so that successive launches draw disjoint ranges of the Philox stream.
The kernels key Philox with the seed and count from the offset
(flash_attn_with_score_amd/csrc/fas_device.hpp: philox6_word0).
"""
from __future__ import annotations

import torch

__all__ = ["philox_cuda_seed_offset"]


def philox_cuda_seed_offset(increment: int, device=None):
    torch.cuda.init()  # default_generators is filled when the device initialises
    if device is None:
        device = torch.cuda.current_device()
    gen = torch.cuda.default_generators[device]
    state = gen.get_state()
    words = state.view(torch.int64)
    seed, offset = int(words[0]), int(words[1])
    words[1] += (increment + 3) // 4 * 4
    gen.set_state(state)
    return seed, offset
