"""Pin of the SH basis (src/tracing/sh_utils.cuh:8-62) against scipy's
complex spherical harmonics (Condon-Shortley phase): the reference's real
basis is Y_{l,m} = sqrt(2) Im Y_l^{|m|} for m < 0, Y_l^0 for m = 0 and
sqrt(2) Re Y_l^m for m > 0, ordered m = -l..l."""

import numpy as np
import pytest
import scipy.special as sp


def real_sh(l, m, theta, phi):
    """theta: polar angle from +z, phi: azimuth from +x."""
    if hasattr(sp, "sph_harm_y"):
        Y = sp.sph_harm_y(l, abs(m), theta, phi)
    else:  # older scipy: sph_harm(m, l, azimuth, polar)
        Y = sp.sph_harm(abs(m), l, phi, theta)
    if m < 0:
        return np.sqrt(2.0) * Y.imag
    if m == 0:
        return Y.real
    return np.sqrt(2.0) * Y.real


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_basis_matches_scipy(oracle_lib, degree):
    rng = np.random.default_rng(degree)
    d = rng.normal(size=(200, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    d = d.astype(np.float32)
    for v in d:
        got = oracle_lib.sh_basis(degree, v)
        x, y, z = v.astype(np.float64)
        theta = np.arccos(np.clip(z, -1, 1))
        phi = np.arctan2(y, x)
        k = 0
        for l in range(degree + 1):
            for m in range(-l, l + 1):
                ref = real_sh(l, m, theta, phi)
                assert abs(got[k] - ref) <= 2e-6 * max(1.0, abs(ref)), (l, m, got[k], ref)
                k += 1
        assert np.all(got[k:] == 0.0)


def test_axis_values(oracle_lib):
    c0, c1 = 0.28209479177387814, 0.4886025119029199
    for v, lin in [((1, 0, 0), (0, 0, -c1)), ((0, 1, 0), (-c1, 0, 0)), ((0, 0, 1), (0, c1, 0))]:
        got = oracle_lib.sh_basis(1, np.array(v, np.float32))
        assert got[0] == np.float32(c0)
        assert np.allclose(got[1:4], lin, atol=0, rtol=1e-7)
