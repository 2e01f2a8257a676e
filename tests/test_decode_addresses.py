"""CPU: the addresses the dense decode route loads (decode_attn.hip's
load_k_dense / load_v_dense, enumerated on the host by
spyre_dense_decode_load_extent from the kernel's own address functions).

The kernel reads a 64-token run of a K / V head through a buffer resource
whose range ends with the run's last token's 2 D bytes.  These tests check,
for every lane and load, that nothing past that end is touched even if the
hardware range check covered only the per-lane offset (not the scalar
one), and that the last token's bytes are read.  No GPU is used."""

import ctypes

import pytest


@pytest.fixture(scope="module")
def L():
    from torch_spyre_amd import _lib

    return _lib.lib()


def extent(L, D, rows, k_row, v_row):
    ke, ve, n = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    rc = L.spyre_dense_decode_load_extent(D, rows, k_row, v_row, ctypes.byref(ke), ctypes.byref(ve), ctypes.byref(n))
    assert rc == 0
    return ke.value, ve.value, n.value


# Token strides in bytes: dense rows, padded rows, a [B, S, H, D] layout
# (H = 8 heads between tokens), a slice of a wider row, and 0 (one row
# expanded over the tokens).  The route takes no other stride below 2 D
# bytes (dense_decode_launch).
def row_bytes(D):
    return [2 * D, 2 * D + 16, 16 * D, 2 * D * 8 + 32, 0]


@pytest.mark.parametrize("D", [64, 128])
def test_window_loads_stay_inside_the_run(L, D):
    """A 64-token window (every steady-state run, and the last run of a
    context that is not a multiple of 64): the loads end exactly with the
    last token's 2 D bytes."""
    for k_row in row_bytes(D):
        for v_row in row_bytes(D):
            ke, ve, n = extent(L, D, 64, k_row, v_row)
            assert ke == 63 * k_row + 2 * D, (k_row, ke)
            assert ve == 63 * v_row + 2 * D, (v_row, ve)
            # every load touches memory: 64 lanes x (8 D / 64 K + 16 V) loads
            assert n == 64 * (8 * D // 64 + 16)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("rows", [1, 2, 3, 7, 8, 15, 16, 17, 31, 32, 33, 40, 47, 48, 63])
def test_short_context_reads_nothing_past_its_last_token(L, D, rows):
    """A context of fewer than 64 tokens: its one run's loads of tokens past
    the context are out of range, the others end inside the last token."""
    for k_row in row_bytes(D):
        v_row = k_row
        ke, ve, n = extent(L, D, rows, k_row, v_row)
        assert ke == (rows - 1) * k_row + 2 * D, (rows, k_row, ke)
        assert ve == (rows - 1) * v_row + 2 * D, (rows, v_row, ve)
        # only the context's tokens are loaded: each by D / 8 K loads (16
        # bytes each) and by the 16 lanes of its V lane group (with stride
        # 0 every load reads the one row, inside the range)
        assert n == (rows if k_row else 64) * (D // 8 + 16)


def test_bad_arguments(L):
    ke, ve, n = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    for D, rows in ((96, 64), (128, 0), (128, 65)):
        assert L.spyre_dense_decode_load_extent(D, rows, 256, 256, ctypes.byref(ke), ctypes.byref(ve),
                                                ctypes.byref(n)) != 0
