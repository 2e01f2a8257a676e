"""Oracle: closed forms of the three stick relayouts.

Test infrastructure only (see ``oracle/__init__.py``).

For a row-major [R, C] tensor X (C, R multiples of 64 here):
* to_sticks:       default layout [C/64, R, 64]/[64, C, 1]
                   dev[i, j, k] = X[j, 64 i + k]
                   (docs/source/user_guide/tensors_and_layouts.md:305-318 loop nest;
                   torch_spyre/csrc/spyre_tensor_impl.cpp:46-80 tiling)
* from_sticks:     the inverse.
* transpose_restick: dim_order [1, 0] layout [R/64, C, 64]/[64 C, 1, C]
                   dev[i, j, k] = X[64 i + k, j]
                   (restickify target, torch_spyre/_inductor/pass_utils.py:749-781;
                   the dim_order=[1,0] weight layout, torch_spyre/model_utils.py:111-138)

Parity pins (tests/test_oracle_layout.py): each closed form equals the
generic DMA loop-nest execution of ``oracle.layout`` for the corresponding
SpyreTensorLayout on several shapes, and the layouts themselves are pinned by
the reference's golden tables.
"""

from __future__ import annotations

import numpy as np


def to_sticks(x: np.ndarray) -> np.ndarray:
    R, C = x.shape
    return np.ascontiguousarray(x.reshape(R, C // 64, 64).transpose(1, 0, 2))


def from_sticks(dev: np.ndarray) -> np.ndarray:
    T, R, S = dev.shape
    return np.ascontiguousarray(dev.transpose(1, 0, 2).reshape(R, T * S))


def transpose_restick(x: np.ndarray) -> np.ndarray:
    R, C = x.shape
    return np.ascontiguousarray(x.reshape(R // 64, 64, C).transpose(0, 2, 1))


def random_finite_f16_bits(shape, seed: int) -> np.ndarray:
    """Random 16-bit patterns with NaN/Inf exponents (0x7C00 all set) resampled,
    as raw uint16 (bit-exact comparisons never go through float)."""
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 1 << 16, size=shape, dtype=np.uint32).astype(np.uint16)
    bad = (u & 0x7C00) == 0x7C00
    while bad.any():
        u[bad] = rng.integers(0, 1 << 16, size=int(bad.sum()), dtype=np.uint32).astype(np.uint16)
        bad = (u & 0x7C00) == 0x7C00
    return u
