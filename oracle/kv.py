"""Oracle: the overwrite (KV-cache write) semantics.

Test infrastructure only (see ``oracle/__init__.py``).

``overwrite`` restates the reference's CPU kernel of spyre::overwrite
(torch_spyre/_inductor/customops.py:298-308): narrow ``output`` along each
dims[i] at offsets[i] to input's size and copy ``input`` into it.
``append_token`` is the same operation on logical pages [P, Hkv, 64, D]:
token position p of sequence b goes to page block_table[b][p // 64], slot
p % 64 (the test_overwrite pattern, tests/inductor/test_overwrite.py:166-187,
with the offset chosen through the block table).

Parity pins (tests/test_oracle_kv.py): overwrite equals index assignment on
numpy arrays; ten sequential single-token writes into a [1, 8, 64, 128]
cache (the reference test's shape) touch exactly those slots.
"""

from __future__ import annotations

import numpy as np

PAGE = 64


def overwrite(inp: np.ndarray, out: np.ndarray, dims, offsets) -> None:
    sl = [slice(None)] * out.ndim
    for d, o in zip(dims, offsets):
        sl[d] = slice(o, o + inp.shape[d])
    out[tuple(sl)] = inp


def append_token(k_log, v_log, k_new, v_new, block_table, positions) -> None:
    """k_new/v_new [B, Hkv, D] into logical pages [P, Hkv, 64, D] in place."""
    for b, p in enumerate(positions):
        if p < 0:
            continue
        page = int(block_table[b][p // PAGE])
        overwrite(k_new[b][None, :, None, :], k_log, [0, 2], [page, p % PAGE])
        overwrite(v_new[b][None, :, None, :], v_log, [0, 2], [page, p % PAGE])
