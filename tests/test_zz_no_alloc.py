"""sdf_trace_forward_noalloc: the forward without caller scratch (its fp16
offset table in the library's static device array), through the C ABI.

Two calls in a row, the second over a smaller scene, each checked against
sdf_trace_forward on the same inputs: rgba, depth, depth indices and loop
counts bit-exact (the same kernels on the same inputs); contributions within
the summation bound (fp32 atomics in another order); the same points touched
by alpha.  The smaller scene's stale table entries beyond its own must not
matter, and the second call's results are also held against the oracle.  A
scene beyond the array's capacity is refused before any work is queued."""

import ctypes as C

import numpy as np
import pytest

from conftest import scene
from test_gpu_parity import gamma, to_dev, u32, _threads


def _args(w, dev, lib, noalloc):
    import torch

    from sdfoam_amd import _lib

    R = w.num_rays
    N = w.num_points
    Q = int(w.quantiles.shape[-1])
    t = dict(points=to_dev(w.points, dev), attrs=to_dev(w.attributes, dev),
             adj=u32(w.adjacency, dev), offs=u32(w.offsets, dev), rays=to_dev(w.rays, dev),
             start=u32(w.extra["start"], dev), q=to_dev(w.quantiles, dev),
             sharp=torch.tensor([w.inv_s], dtype=torch.float32, device=dev))
    out = dict(rgba=torch.empty((R, 4), dtype=torch.float32, device=dev),
               depth=torch.zeros((R, Q), dtype=torch.float32, device=dev),
               didx=torch.zeros((R, Q), dtype=torch.int32, device=dev),
               nis=torch.empty(R, dtype=torch.int32, device=dev),
               contrib=torch.zeros(N, dtype=torch.float32, device=dev),
               alpha=torch.zeros(N, dtype=torch.float32, device=dev))
    D = w.attributes.shape[-1]
    s = _lib.TraceSettings(1e-7, 1024, _lib.SDF_ALPHA_NEUS, D - 1, 0, _lib.SDF_ATTR_F32)
    head = (w.sh_degree, C.byref(s), N, t["points"].data_ptr(), t["attrs"].data_ptr(),
            int(w.adjacency.size), t["adj"].data_ptr(), t["offs"].data_ptr(), R,
            t["rays"].data_ptr(), t["start"].data_ptr(), Q, t["q"].data_ptr(),
            out["rgba"].data_ptr(), out["depth"].data_ptr(), out["didx"].data_ptr(),
            out["nis"].data_ptr(), out["contrib"].data_ptr(), t["sharp"].data_ptr(),
            out["alpha"].data_ptr())
    stream = torch.cuda.current_stream(dev).cuda_stream
    if noalloc:
        rc = lib.sdf_trace_forward_noalloc(*head, stream)
    else:
        nbytes = int(lib.sdf_trace_scratch_bytes(N, int(w.adjacency.size)))
        scratch = torch.empty((nbytes + 7) // 8, dtype=torch.int64, device=dev)
        rc = lib.sdf_trace_forward(*head, scratch.data_ptr(), nbytes, stream)
        torch.cuda.synchronize()
        del scratch
    _lib.check(rc)
    torch.cuda.synchronize()
    res = {k: v.cpu().numpy() for k, v in out.items()}
    del t, out
    return res


def _same(a, b, R):
    for k in ("rgba", "depth", "didx", "nis"):
        assert np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)), k
    # contributions are sums of nonnegative weights: |a - b| <= 2 gamma_R max
    ca, cb = a["contrib"].astype(np.float64), b["contrib"].astype(np.float64)
    tol = 2 * gamma(R) * np.maximum(ca, cb) + 1e-12
    assert np.all(np.abs(ca - cb) <= tol), "contribution"
    assert np.array_equal(a["alpha"] != 0, b["alpha"] != 0), "points touched by alpha"


@pytest.mark.gpu
def test_noalloc_forward_matches_forward(oracle_lib):
    import torch

    from sdfoam_amd import _lib

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dev = torch.device("cuda:0")
    lib = _lib.lib()
    big, small = scene(2), scene(1)
    assert big.adjacency.size > small.adjacency.size
    for w in (big, small):
        print(f"noalloc forward: {w.num_points} points, {w.adjacency.size} adjacency entries, "
              f"{w.num_rays} rays", flush=True)
        got = _args(w, dev, lib, noalloc=True)
        ref = _args(w, dev, lib, noalloc=False)
        _same(got, ref, w.num_rays)
    ora = oracle_lib.trace_forward(
        small.sh_degree, small.points, small.attributes, small.adjacency, small.offsets,
        small.rays, small.extra["start"], small.quantiles, alpha_mode="sdfoam",
        inv_s=small.inv_s, threads=_threads())
    R = small.num_rays
    assert np.array_equal(got["nis"].view(np.uint32).reshape(R),
                          ora.num_intersections.reshape(R))
    assert np.array_equal(got["didx"].view(np.uint32).reshape(R, -1),
                          ora.depth_indices.reshape(R, -1))
    np.testing.assert_allclose(got["rgba"], ora.rgba.reshape(R, 4), rtol=1e-4, atol=1e-5)


def test_noalloc_refuses_scenes_beyond_its_scratch():
    """The capacity check comes before any HIP call (no GPU needed)."""
    from sdfoam_amd import _lib

    lib = _lib.lib()
    cap = (128 << 20) // 8 - 32  # SDF_NOALLOC_SCRATCH_BYTES / 8 - 32
    buf = (C.c_uint64 * 64)()
    p = C.cast(buf, C.c_void_p)
    s = _lib.TraceSettings(1e-7, 1024, 1, 48, 0, 0)
    rc = lib.sdf_trace_forward_noalloc(3, C.byref(s), 10, p, p, cap + 1, p, p, 1, p, p, 0, None,
                                       p, None, None, p, None, p, p, None)
    assert rc == _lib.SDF_E_INVALID
    assert b"static scratch" in lib.sdf_last_error()
