"""CPU: pin the KV-write oracle (overwrite / append) to index assignment and
to the reference test's sequential-write pattern."""

import numpy as np
import torch

from oracle import kv as OK


def test_overwrite_equals_torch_narrow_copy():
    """torch_spyre/_inductor/customops.py:298-308: narrow along each dim, copy."""
    rng = np.random.default_rng(0)
    out = rng.standard_normal((4, 8, 64, 128)).astype(np.float32)
    inp = rng.standard_normal((1, 8, 1, 128)).astype(np.float32)
    want = torch.from_numpy(out.copy())
    sl = want.narrow(0, 2, 1).narrow(2, 17, 1)
    sl.copy_(torch.from_numpy(inp))
    OK.overwrite(inp, out, [0, 2], [2, 17])
    assert np.array_equal(out, want.numpy())


def test_ten_sequential_writes_touch_only_their_slots():
    """tests/inductor/test_overwrite.py:166-187 pattern: ten single-token writes
    into [1, 8, 64, 128] at dim 2."""
    cache = np.zeros((1, 8, 64, 128), np.float32)
    toks = [np.full((1, 8, 1, 128), i + 1, np.float32) for i in range(10)]
    for i, t in enumerate(toks):
        OK.overwrite(t, cache, [2], [i])
    for i in range(10):
        assert (cache[0, :, i] == i + 1).all()
    assert not cache[0, :, 10:].any()


def test_append_token_uses_block_table():
    k = np.zeros((5, 2, 64, 64), np.float32)
    v = np.zeros_like(k)
    table = np.array([[3, 1], [4, 0]])
    kn = np.ones((2, 2, 64), np.float32)
    vn = 2 * np.ones((2, 2, 64), np.float32)
    OK.append_token(k, v, kn, vn, table, [70, -1])
    assert (k[1, :, 6] == 1).all() and (v[1, :, 6] == 2).all()  # position 70 -> page table[0][1] = 1, slot 6
    assert np.count_nonzero(k) == 2 * 64 and np.count_nonzero(v) == 2 * 64  # sequence 1 skipped
