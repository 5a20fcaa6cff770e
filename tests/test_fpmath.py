"""Pins of the shared fp-math contract (include/sdfoam_fpmath.h) on the host:
exp against libm in double precision, the fp16 rounding against numpy's
IEEE conversion, the decode exhaustively."""

import numpy as np


def ulp32(x):
    x = np.abs(np.asarray(x, dtype=np.float32))
    return np.spacing(x).astype(np.float64)


def test_exp_within_one_ulp(oracle_lib):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        np.linspace(-87.3, 88.7, 2_000_001),
        rng.uniform(-1, 1, 1_000_000),
        rng.normal(0, 1e-4, 100_000),
    ]).astype(np.float32)
    got = oracle_lib.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    err_ulp = np.abs(got - ref) / ulp32(ref.astype(np.float32))
    assert err_ulp.max() <= 1.0, f"max error {err_ulp.max():.3f} ulp"
    # most results are correctly rounded
    assert np.mean(got == ref.astype(np.float32)) > 0.9


def test_exp_special_values(oracle_lib):
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.8, -87.4, -200.0, 1e-30, -1e-30],
                 dtype=np.float32)
    y = oracle_lib.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert np.isposinf(y[2]) and y[3] == 0.0 and np.isnan(y[4])
    assert np.isposinf(y[5])
    assert y[6] == 0.0 and y[7] == 0.0  # below the normal range: flushed to +0
    assert y[8] == 1.0 and y[9] == 1.0
    # monotone over a fine sweep
    s = np.linspace(-87.3, 88.7, 500_001, dtype=np.float32)
    e = oracle_lib.expf(s)
    assert np.all(np.diff(e.astype(np.float64)) >= 0)


def test_sigmoid_matches_definition(oracle_lib):
    import ctypes

    lib = oracle_lib.lib()
    for v in [-50.0, -3.0, -0.5, 0.0, 0.25, 4.0, 60.0]:
        got = lib.oracle_sigmoidf(ctypes.c_float(v))
        assert abs(got - 1.0 / (1.0 + np.exp(-v))) <= 2.5e-7 * max(1e-30, got) + 1e-38
    assert lib.oracle_sigmoidf(ctypes.c_float(0.0)) == 0.5


def test_f16_rounding_matches_ieee(oracle_lib):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.uniform(-66000, 66000, 1_000_000),
        rng.uniform(-2, 2, 1_000_000),
        rng.uniform(-1e-4, 1e-4, 500_000),
        rng.uniform(-1e-7, 1e-7, 200_000),
    ]).astype(np.float32)
    # exact halfway points between neighbouring halves, normal and subnormal
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    mids = mids[np.isfinite(mids)]
    x = np.concatenate([x, mids, -mids, np.array([65504, 65519.99, 65520, 1e9, 2.0 ** -25,
                                                  2.0 ** -24, 3 * 2.0 ** -26], np.float32)])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = oracle_lib.f32_to_f16_bits(x)
    assert np.array_equal(got, ref)


def test_f16_decode_exhaustive(oracle_lib):
    import ctypes

    lib = oracle_lib.lib()
    bits = np.arange(65536, dtype=np.uint32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([lib.oracle_f16_to_f32(ctypes.c_uint16(int(b))) for b in bits], dtype=np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()
