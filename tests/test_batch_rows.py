"""BatchFetcher row selection without a GPU: the library's host computation
(sdf_batch_rows) equals the oracle's restatement of the reference's RNG and
scaling (src/utils/batch_fetcher.cpp:63-72, src/utils/random.h:11-56), and
the restatement behaves as the mathematics says: consecutive rows wrap
modulo n, random rows are uniform on [0, n), depend only on the element's
global position, the integer hash maps 0 to 0 and is undone by its
published inverse, and a row grows with its draw.  The seed constant
0x2815db5b (src/utils/random.h:27) is checked by reading only."""

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


# The inverse of "triple32" as C. Wellons publishes it beside the hash in
# hash-prospector's README: each xorshift undone by xorshifts at multiples of
# its shift, each multiplier by its inverse modulo 2^32, in reverse order.
# Its multipliers are not the hash's, so composing the two checks the hash's
# multipliers and shifts against a second published record of them.
_INV_STEPS = ((14, 0x32B21703), (15, 0x469E0DB1), (11, 0x79A85073))
_INV_LAST_SHIFT = 17


def _xorshift_inverse(x, s):
    y = x.copy()
    k = s
    while k < 32:
        y ^= x >> np.uint32(k)
        k += s
    return y


def _triple32_inverse(x):
    x = x.astype(np.uint32)
    with np.errstate(over="ignore"):
        for s, m in _INV_STEPS:
            x = _xorshift_inverse(x, s)
            x *= np.uint32(m)
        x = _xorshift_inverse(x, _INV_LAST_SHIFT)
    return x


def _hash_inputs():
    rng = np.random.default_rng(11)
    edge = np.array([0, 1, 2, 0x2815DB5B, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFE, 0xFFFFFFFF],
                    dtype=np.uint32)
    return np.concatenate([edge, np.arange(1 << 16, dtype=np.uint32),
                           rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)])


def test_hash_inverts_with_published_inverse():
    x = _hash_inputs()
    assert np.array_equal(_triple32_inverse(oracle._mix32(x)), x)
    assert np.array_equal(oracle._mix32(_triple32_inverse(x)), x)


def _mix_variant(x, shifts, mults):
    x = x.astype(np.uint32)
    with np.errstate(over="ignore"):
        for i, m in enumerate(mults):
            x ^= x >> np.uint32(shifts[i])
            x *= np.uint32(m)
        x ^= x >> np.uint32(shifts[3])
    return x


@pytest.mark.parametrize("n", [2, 3, 1000, 1_000_003])
def test_row_scaling_is_monotone_in_the_draw(n):
    """With the hash pinned, a row is a non-decreasing function of its draw
    mix32(seed ^ 0x2815db5b), near draw * n / 2^32 (within 1 + n^2 / 2^32:
    the divisor 0xffffffff // n is truncated), and for n = 2 exactly
    [draw >= 0x7fffffff] (0xffffffff // 2 = 0x7fffffff: draws below it give
    0, the rest 1, or 2 clamped to 1).  A scaling by remainder fails these."""
    B = 1 << 16
    rows = oracle.batch_rows(5, B, n, True).astype(np.int64)
    seed = (np.uint64(5 * B) + np.arange(B, dtype=np.uint64)).astype(np.uint32)
    draw = oracle._mix32(seed ^ np.uint32(0x2815DB5B)).astype(np.int64)
    order = np.argsort(draw, kind="stable")
    assert np.all(np.diff(rows[order]) >= 0)
    assert np.all(np.abs(rows - (draw * n >> 32)) <= 1 + int(np.ceil(1.001 * n * n / 2.0**32)))
    assert rows.max() == n - 1 or n > B
    if n == 2:
        assert np.array_equal(rows, (draw >= 0x7FFFFFFF).astype(np.int64))


@pytest.mark.parametrize("which", range(7))
def test_hash_inverse_check_catches_a_wrong_constant(which):
    """Plants one plausible slip in the hash (a shift off by one, a
    multiplier off by 2, which keeps it odd and the hash a bijection) and
    shows that the inversion check above fails for it."""
    shifts = [17, 11, 15, 14]
    mults = [0xED5AD4BB, 0xAC4C1B51, 0x31848BAB]
    x = _hash_inputs()[:1 << 16]
    assert np.array_equal(_triple32_inverse(_mix_variant(x, shifts, mults)), x)
    if which < 4:
        shifts[which] += 1
    else:
        mults[which - 4] = (mults[which - 4] + 2) & 0xFFFFFFFF
    assert not np.array_equal(_triple32_inverse(_mix_variant(x, shifts, mults)), x)


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
