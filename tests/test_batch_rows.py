"""BatchFetcher row selection without a GPU: the library's host computation
(sdf_batch_rows) equals the oracle's restatement of the reference's RNG and
scaling (src/utils/batch_fetcher.cpp:63-72, src/utils/random.h:11-56), and
the restatement behaves as the mathematics says: consecutive rows wrap
modulo n, random rows are uniform on [0, n), depend only on the element's
global position, and the integer hash maps 0 to 0."""

import numpy as np
import pytest

from oracle import oracle


@pytest.mark.parametrize("b,B,n,shuffle", [
    (0, 1000, 77, False), (5, 4096, 10_000, False), (123, 1 << 16, 3, False),
    (0, 1000, 77, True), (7, 4096, 1_000_003, True), (1 << 20, 4096, 5, True),
    (3, 1 << 16, 1, True), (9, 333, 0xFFFFFFFF, True),
])
def test_library_matches_oracle(b, B, n, shuffle):
    from sdfoam_amd.fetch import batch_rows

    got = batch_rows(b, B, n, shuffle)
    want = oracle.batch_rows(b, B, n, shuffle)
    assert np.array_equal(got, want)
    assert got.max() < n


def test_consecutive_rows_wrap():
    r = oracle.batch_rows(3, 10, 7, False)
    assert r.tolist() == [(30 + j) % 7 for j in range(10)]


def test_random_rows_uniform_and_positional():
    n = 10
    rows = np.concatenate([oracle.batch_rows(b, 10_000, n, True) for b in range(10)])
    counts = np.bincount(rows, minlength=n)
    expected = rows.size / n
    chi2 = float(np.sum((counts - expected) ** 2 / expected))
    assert chi2 < 30.0  # 9 dof: p ~ 4e-4
    # element j of batch b depends only on b * B + j
    a = oracle.batch_rows(2, 100, 1000, True)  # positions 200..299
    c = oracle.batch_rows(1, 200, 1000, True)  # positions 200..399
    d = oracle.batch_rows(0, 300, 1000, True)  # positions 0..299
    assert np.array_equal(a, c[:100]) and np.array_equal(a, d[200:])
    assert not np.array_equal(a, oracle.batch_rows(3, 100, 1000, True))


def test_hash_fixed_point_and_scaling():
    assert int(oracle._mix32(np.array([0], dtype=np.uint32))[0]) == 0
    # n = 1: every draw maps to row 0
    assert np.all(oracle.batch_rows(4, 1000, 1, True) == 0)


def test_create_rejects_bad_arguments():
    import ctypes as C

    from sdfoam_amd import _lib

    L = _lib.lib()
    h = C.c_void_p()
    buf = (C.c_uint8 * 64)()
    p = C.cast(buf, C.c_void_p)
    assert L.sdf_batch_fetcher_create(None, 64, 8, 4, 1, p, 1 << 20, 0, C.byref(h)) == 1
    assert b"data must hold" in L.sdf_last_error()
    assert L.sdf_batch_fetcher_create(p, 64, 8, 0, 1, p, 1 << 20, 0, C.byref(h)) == 1
    assert L.sdf_batch_fetcher_create(p, 64, 8, 4, 1, p, 10, 0, C.byref(h)) == 1
    assert b"device_ring must hold 128 bytes" in L.sdf_last_error()
    assert L.sdf_batch_fetcher_ring_bytes(24, 1000) == 4 * 24 * 1000
    assert L.sdf_batch_fetcher_destroy(None) == 0
