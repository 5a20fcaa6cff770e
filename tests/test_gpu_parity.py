"""GPU parity: libsdfoam_hip.so (through its C ABI, via the sdfoam_amd host
mirror) against the scalar host oracle on the same seeded inputs.

Bars (the contract of the port):
* visit sequences (hash + step count + full sequences on C1),
  num_intersections, depth_indices, fp16 offset table, AABB tree, nn:
  bit-exact;
* rgba, depth: |d| <= 1e-5 + 1e-4 |ref|;
* gradients and contribution (fp32 atomics in any order against the
  oracle's fp64 sum): |d| <= 1e-5 + 1e-4 |ref| + gamma_{K-1} A, with
  A = sum |c_k| over the element's K contributions and
  gamma_n = n u / (1 - n u), u = 2^-24 (the order-independent bound for
  recursive summation, Higham 2002, section 4.2);
* alpha: the value some visiting step of that point wrote (the reference
  stores it racily, src/tracing/pipeline.cu:159); untouched points stay 0.
"""

import os

import numpy as np
import pytest

from conftest import scene

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def _threads():
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return 4


def gamma(k):
    k = np.maximum(np.asarray(k, dtype=np.float64) - 1.0, 0.0)
    ku = k * U
    # the bound holds for n u < 1 only; a count past that must not pass silently
    assert np.all(ku < 0.5), f"summation bound vacuous for K up to {int(k.max()) + 1}"
    return ku / (1.0 - ku)


def assert_close_model(name, got, ref, abs_sum, k):
    got = np.asarray(got, dtype=np.float64)
    tol = 1e-5 + 1e-4 * np.abs(ref) + gamma(k) * abs_sum
    err = np.abs(got - ref)
    bad = ~(err <= tol)
    if bad.any():
        i = np.argmax(np.where(bad, err / np.maximum(tol, 1e-30), 0))
        raise AssertionError(
            f"{name}: {int(bad.sum())} of {bad.size} elements out of tolerance; worst at "
            f"{np.unravel_index(i, np.shape(ref))}: got {got.ravel()[i]!r} ref {np.ravel(ref)[i]!r} "
            f"tol {tol.ravel()[i]!r}")


def assert_close(name, got, ref, rtol=1e-4, atol=1e-5):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    tol = atol + rtol * np.abs(ref)
    bad = ~(err <= tol)
    if bad.any():
        i = np.argmax(np.where(bad, err, 0))
        raise AssertionError(f"{name}: {int(bad.sum())} of {bad.size} out of tolerance; worst "
                             f"got {got.ravel()[i]!r} ref {ref.ravel()[i]!r}")


@pytest.fixture(scope="module")
def torch_dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def to_dev(a, dev, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev)


def u32(a, dev):
    import torch

    return to_dev(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32), dev).view(torch.uint32)


def np_u32(t):
    import torch

    return t.view(torch.int32).cpu().numpy().view(np.uint32)


def gpu_scene(w, dev):
    return dict(
        points=to_dev(w.points, dev),
        attributes=to_dev(w.attributes, dev),
        point_adjacency=u32(w.adjacency, dev),
        point_adjacency_offsets=u32(w.offsets, dev),
        rays=to_dev(w.rays, dev),
        start_point=u32(w.extra["start"], dev),
    )


# ---------------------------------------------------------------------------


def test_fpmath_device_bitexact(torch_dev, oracle_lib):
    import torch

    from sdfoam_amd import _lib

    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.uniform(-110, 100, 400_000),
        rng.uniform(-1, 1, 400_000),
        rng.normal(0, 1e-3, 100_000),
        np.array([0.0, -0.0, 88.72, 88.73, -87.33, -87.34, -103.0, 1e-30, -1e-30, np.inf, -np.inf]),
    ]).astype(np.float32)
    xd = to_dev(x, torch_dev)
    out = torch.empty_like(xd)
    _lib.check(_lib.lib().sdf_debug_fpmath(0, xd.data_ptr(), out.data_ptr(), x.size, None))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = oracle_lib.expf(x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "device exp differs from host"

    # fp16 rounding: wide range incl. halfway points, subnormals and overflow
    y = np.concatenate([
        rng.uniform(-70000, 70000, 200_000),
        rng.uniform(-2, 2, 400_000),
        rng.uniform(-1e-4, 1e-4, 200_000),
        (np.arange(1, 2048, dtype=np.float64) * 2.0 ** -25),
        (np.arange(1, 4096, dtype=np.float64) * 2.0 ** -12 + 0.5 * 2.0 ** -11),
    ]).astype(np.float32)
    yd = to_dev(y, torch_dev)
    h = torch.empty(y.size, dtype=torch.int16, device=torch_dev)
    _lib.check(_lib.lib().sdf_debug_fpmath(1, yd.data_ptr(), h.data_ptr(), y.size, None))
    torch.cuda.synchronize()
    got_h = h.cpu().numpy().view(np.uint16)
    assert np.array_equal(got_h, oracle_lib.f32_to_f16_bits(y))
    assert np.array_equal(got_h, y.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("cfg", [1, 2])
def test_prefetch_diff_bitexact(torch_dev, oracle_lib, cfg):
    import torch

    from sdfoam_amd import prefetch_adjacent_diff

    w = scene(cfg)
    g = gpu_scene(w, torch_dev)
    d = prefetch_adjacent_diff(g["points"], g["point_adjacency"], g["point_adjacency_offsets"])
    torch.cuda.synchronize()
    got = d.cpu().numpy().view(np.uint16)[: w.adjacency.size]
    ref = oracle_lib.prefetch_adjacent_diff(w.points, w.adjacency, w.offsets)
    assert np.array_equal(got, ref)


def with_neighbour_deltas(ref, adjacency, offsets):
    """The oracle's prefetch_adjacent_diff entries [E, 4] (fourth half 0) with
    the fourth half the table built beside the cell table carries: the
    neighbour minus the row's point as int16, 0x8000 where that does not fit."""
    offs = np.asarray(offsets, dtype=np.int64)
    rows = np.repeat(np.arange(offs.size - 1), np.diff(offs))
    d = np.asarray(adjacency, dtype=np.int64) - rows
    fourth = np.where(np.abs(d) <= 32767, d & 0xFFFF, 0x8000).astype(np.uint16)
    out = np.array(ref, dtype=np.uint16).reshape(-1, 4)
    assert not out[:, 3].any()
    out[:, 3] = fourth
    return out


def test_neighbour_delta_encoding():
    """The host restatement of the fourth half on hand cases: in-range deltas
    of both signs, the int16 limits and beyond (0x8000 = read the adjacency)."""
    # rows 0, 0, 1, 1, 2, 3, 3, then 40000, 40000 (rows 4..39999 empty)
    adj = np.array([1, 0, 32769, 40000, 5, 2, 32770, 7232, 7233], dtype=np.uint32)
    offs = np.array([0, 2, 4, 5] + [7] * 39997 + [9], dtype=np.uint32)
    got = with_neighbour_deltas(np.zeros((9, 4), np.uint16), adj, offs)[:, 3]
    # deltas 1, 0, 32768, 39999, 3, -1, 32767, -32768, -32767
    assert got.tolist() == [1, 0, 0x8000, 0x8000, 3, 0xFFFF, 32767, 0x8000, 0x8001]


@pytest.mark.parametrize("cfg,dtype", [(1, "float32"), (2, "float32"), (2, "float16")])
def test_forward_offset_table_bitexact(torch_dev, oracle_lib, cfg, dtype):
    """The forward builds its fp16 offset table in the same pass as its cell
    table; the table it keeps for the backward equals the oracle's
    prefetch_adjacent_diff bit for bit in the offset halves, carries each
    entry's neighbour delta in the fourth, and has its 32 padding entries
    zero."""
    import torch

    import sdfoam_amd

    w = scene(cfg)
    g = gpu_scene(w, torch_dev)
    if dtype == "float16":
        g["attributes"] = g["attributes"].half()
    pipe = sdfoam_amd.create_pipeline(w.sh_degree, dtype)
    fwd = pipe.trace_forward(**g, alpha_mode="sdfoam", inv_s=torch.tensor([w.inv_s], device=torch_dev),
                             record_walk=True)
    torch.cuda.synchronize()
    E = w.adjacency.size
    table = fwd["trace_plan"].table.view(torch.uint8)[:(E + 32) * 8].cpu().numpy().view(np.uint16)
    ref = oracle_lib.prefetch_adjacent_diff(w.points, w.adjacency, w.offsets)
    assert np.array_equal(table[:4 * E], with_neighbour_deltas(ref, w.adjacency, w.offsets).reshape(-1))
    assert not table[4 * E:].any()


def test_offset_table_with_empty_rows(torch_dev, oracle_lib):
    """CSR rows may be empty (a point whose row was cleared): the tables are
    built by runs of 64 rows, so an entry's row is the last one starting at or
    before it.  Every 7th point of C1 loses its row (and runs of empty rows
    occur); the forward's table, the plain table and the forward itself
    still equal the oracle's."""
    import dataclasses

    import torch

    import sdfoam_amd
    from sdfoam_amd import prefetch_adjacent_diff

    w = scene(1)
    offs = w.offsets.astype(np.int64)
    deg = np.diff(offs)
    keep_row = np.ones(w.points.shape[0], dtype=bool)
    keep_row[::7] = False
    keep_row[100:140] = False  # a run of empty rows
    deg = np.where(keep_row, deg, 0)
    rows = np.repeat(np.arange(w.points.shape[0]), np.diff(offs))
    adj = w.adjacency[keep_row[rows]]
    new_offs = np.concatenate([[0], np.cumsum(deg)]).astype(np.uint32)
    w2 = dataclasses.replace(w, adjacency=np.ascontiguousarray(adj, dtype=np.uint32),
                             offsets=new_offs)
    ref_table = oracle_lib.prefetch_adjacent_diff(w2.points, w2.adjacency, w2.offsets)
    g = gpu_scene(w2, torch_dev)
    plain = prefetch_adjacent_diff(g["points"], g["point_adjacency"], g["point_adjacency_offsets"])
    pipe = sdfoam_amd.create_pipeline(w2.sh_degree)
    fwd = pipe.trace_forward(**g, alpha_mode="sdfoam",
                             inv_s=torch.tensor([w2.inv_s], device=torch_dev), record_walk=True)
    torch.cuda.synchronize()
    E = w2.adjacency.size
    assert np.array_equal(plain.cpu().numpy().view(np.uint16)[:E].reshape(-1), ref_table.reshape(-1))
    table = fwd["trace_plan"].table.view(torch.uint8)[:(E + 32) * 8].cpu().numpy().view(np.uint16)
    assert np.array_equal(table[:4 * E],
                          with_neighbour_deltas(ref_table, w2.adjacency, w2.offsets).reshape(-1))
    out, st, ref = _forward_both(w2, torch_dev, oracle_lib, "sdfoam")
    _check_forward(out, st, ref, w2, 0)


def _forward_both(w, dev, oracle_lib, mode, record=0, inv_s=None, sort_rays=None,
                  record_walk=False):
    import torch

    import sdfoam_amd

    inv = w.inv_s if inv_s is None else inv_s
    g = gpu_scene(w, dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    q = to_dev(w.quantiles, dev)
    out = pipe.trace_forward(**g, depth_quantiles=q, return_contribution=True, alpha_mode=mode,
                             inv_s=torch.tensor([inv], device=dev), sort_rays=sort_rays,
                             record_walk=record_walk)
    st = pipe.walk_stats(**g, alpha_mode=mode, inv_s=torch.tensor([inv], device=dev),
                         record_cells=record)
    torch.cuda.synchronize()
    ref = oracle_lib.trace_forward(
        w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets, w.rays, w.extra["start"],
        w.quantiles, alpha_mode=mode, inv_s=inv, record=record, threads=_threads(),
        point_visits=True)
    return out, st, ref


def _check_forward(out, st, ref, w, record):
    R = w.num_rays
    ni = np_u32(out["num_intersections"]).reshape(R)
    assert np.array_equal(ni, ref.num_intersections.reshape(R)), "num_intersections"
    vh = st["visit_hash"].cpu().numpy().view(np.uint64)
    assert np.array_equal(vh, ref.visit_hash.reshape(R)), "visit hash"
    assert np.array_equal(st["steps"].cpu().numpy().astype(np.uint32), ref.steps.reshape(R))
    assert np.array_equal(st["faces"].cpu().numpy().astype(np.uint64), ref.faces.reshape(R))
    if record:
        cells = st["cells"].cpu().numpy().view(np.uint32)
        n = np.minimum(ref.steps.reshape(R), record)
        mask = np.arange(record)[None, :] < n[:, None]
        assert np.array_equal(np.where(mask, cells, 0), np.where(mask, ref.cells, 0)), "cells"
    assert np.array_equal(np_u32(out["depth_indices"]).reshape(R, -1),
                          ref.depth_indices.reshape(R, -1)), "depth_indices"
    rgba = out["rgba"].cpu().numpy().reshape(R, 4)
    assert_close("rgba", rgba, ref.rgba.reshape(R, 4))
    assert_close("depth", out["depth"].cpu().numpy().reshape(R, -1), ref.depth.reshape(R, -1))
    contrib = out["contribution"].cpu().numpy().reshape(-1)
    cref = ref.contribution.reshape(-1)
    # each point's sum has K = its number of cell steps over all rays of
    # fp32 weights (>= 0, the same bits on both sides); unvisited points stay 0
    k = ref.point_visits
    assert np.all(contrib[k == 0] == 0.0), "contribution of unvisited points"
    assert_close_model("contribution", contrib, cref, np.abs(cref), k)
    # alpha: some visiting step's value; unvisited points untouched
    alpha = out["alpha"].cpu().numpy().reshape(-1)
    visited = np.zeros(w.num_points, dtype=bool)
    if record:
        cells = ref.cells
        n = np.minimum(ref.steps.reshape(R), record)
        mask = np.arange(record)[None, :] < n[:, None]
        vc = cells[mask]
        va = ref.cell_alphas[mask]
        visited[vc] = True
        pairs = set(zip(vc.tolist(), va.view(np.uint32).tolist()))
        for p in np.nonzero(visited)[0]:
            assert (int(p), int(alpha[p:p + 1].view(np.uint32)[0])) in pairs, f"alpha of point {p}"
        assert np.all(alpha[~visited] == 0.0)
    return rgba


@pytest.mark.parametrize("mode", ["sdfoam", "standard"])
def test_forward_parity_c1(torch_dev, oracle_lib, mode):
    w = scene(1, mode=mode)
    out, st, ref = _forward_both(w, torch_dev, oracle_lib, mode, record=1100)
    rgba = _check_forward(out, st, ref, w, 1100)
    print(f"C1 {mode}: rgba bit-exact fraction "
          f"{np.mean(rgba.view(np.uint32) == ref.rgba.reshape(-1, 4).view(np.uint32)):.4f}")


def test_forward_parity_c2(torch_dev, oracle_lib):
    w = scene(2)
    out, st, ref = _forward_both(w, torch_dev, oracle_lib, "sdfoam", record=0)
    _check_forward(out, st, ref, w, 0)


def test_forward_parity_c2_sharp(torch_dev, oracle_lib):
    """inv_s = 50: opaque surfaces, walks end early on the weight threshold."""
    w = scene(2)
    out, st, ref = _forward_both(w, torch_dev, oracle_lib, "sdfoam", record=0, inv_s=50.0)
    _check_forward(out, st, ref, w, 0)


def _backward_both(w, dev, oracle_lib, mode, inv_s=None, ray_error=False, walk=False,
                   walk_budget=None, sort_rays=None, grad_accum=True):
    """GPU forward + backward (with walk=True: the backward replays the
    forward's walk record, `walk_budget` trips per wavefront; with
    grad_accum=False: atomics go to the output arrays, not to the per-cell
    accumulator rows) and the oracle's backward on the same inputs."""
    import torch

    import sdfoam_amd

    inv = w.inv_s if inv_s is None else inv_s
    g = gpu_scene(w, dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    q = to_dev(w.quantiles, dev)
    inv_t = torch.tensor([inv], device=dev)
    fwd = pipe.trace_forward(**g, depth_quantiles=q, alpha_mode=mode, inv_s=inv_t,
                             record_walk=walk, walk_budget=walk_budget, sort_rays=sort_rays)
    if walk and mode == "sdfoam":
        assert fwd["trace_plan"].budget == (walk_budget or 1024 + 2)
    rerr = None
    if ray_error:
        rerr_np = np.random.default_rng(11).uniform(0, 1, w.rays.shape[:-1]).astype(np.float32)
        rerr = to_dev(rerr_np, dev)
    bwd = pipe.trace_backward(**g, rgb_out=fwd["rgba"], grad_in=to_dev(w.grad_rgba, dev),
                              depth_quantiles=q, depth_indices=fwd["depth_indices"],
                              depth_grad_in=to_dev(w.depth_grad, dev), ray_error=rerr,
                              alpha_mode=mode, inv_s=inv_t,
                              trace_plan=fwd.get("trace_plan"), grad_accum=grad_accum)
    st = pipe.walk_stats(**g, backward=True, alpha_mode=mode, inv_s=inv_t)
    torch.cuda.synchronize()
    rgba = fwd["rgba"].cpu().numpy()
    didx = np_u32(fwd["depth_indices"])
    ref = oracle_lib.trace_backward(
        w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets, w.rays, w.extra["start"],
        rgba, w.grad_rgba, w.quantiles, didx, w.depth_grad,
        None if rerr is None else rerr.cpu().numpy(), alpha_mode=mode, inv_s=inv,
        threads=_threads())
    return bwd, st, ref


def record_rows(plan):
    """A walk record's trips in wavefront order, from its chunk tables and
    pool: entries {next, t1} [waves, trips, 64] (uint64), colours
    [waves, trips, 64, 4] and which trips have a chunk [waves, trips];
    trips without one read as 0."""
    from sdfoam_amd import _lib

    slots = -(-plan.budget // 16)
    waves = int(_lib.lib().sdf_walk_record_full_chunks(plan.num_rays, plan.ray_image_width,
                                                       plan.budget)) // slots
    pool = -(-plan.chunks // 8) * 8
    off = plan.record_ptr - plan.entries.data_ptr()
    raw = plan.entries[off:off + plan.nbytes].cpu().numpy()
    head = 8 * 256
    tbytes = -(-waves * slots * 4 // 256) * 256
    table = raw[head:head + waves * slots * 4].view(np.uint32).reshape(waves, slots)
    e0 = head + tbytes
    ents = raw[e0:e0 + pool * 1024 * 8].view(np.uint64).reshape(pool, 16, 64)
    cols = raw[e0 + pool * 1024 * 8:e0 + pool * 1024 * 24].view(np.float32).reshape(pool, 16, 64, 4)
    have = table != 0xFFFFFFFF
    assert (table[have] < pool).all()
    idx = np.where(have, table, 0)
    E = np.where(have[:, :, None, None], ents[idx], 0).reshape(waves, slots * 16, 64)
    Cc = np.where(have[:, :, None, None, None], cols[idx], 0).reshape(waves, slots * 16, 64, 4)
    return E, Cc, np.repeat(have, 16, axis=1)


def sum_depth(w, ref):
    """Depth of the backward's summation tree for the sharpness scalar: the
    most steps one lane takes (from the oracle backward `ref`, same walks),
    six wave-reduction levels and one atomic per wavefront of the launch
    (16x16-pixel tiles of four wavefronts for image-shaped rays, 256-ray
    blocks otherwise; the tile count is also an upper bound for the same rays
    launched flat, ceil(W H / 256) <= ceil(W / 16) ceil(H / 16))."""
    steps = int(ref.steps.max()) if w.num_rays else 0
    if w.rays.ndim >= 3:
        h, wd = w.rays.shape[-3], w.rays.shape[-2]
        waves = 4 * (-(-wd // 16)) * (-(-(w.num_rays // wd) // 16))
    else:
        waves = 4 * (-(-w.num_rays // 256))
    return steps + 6 + waves


def _check_backward(bwd, st, ref, w):
    R = w.num_rays
    vh = st["visit_hash"].cpu().numpy().view(np.uint64)
    assert np.array_equal(vh, ref.visit_hash.reshape(R)), "backward visit hash"
    assert_close_model("points_grad", bwd["points_grad"].cpu().numpy(), ref.points_grad,
                       ref.points_grad_abs, ref.points_grad_k)
    assert_close_model("attr_grad", bwd["attr_grad"].cpu().numpy(), ref.attr_grad,
                       ref.attr_grad_abs, ref.attr_grad_k)
    sg = float(bwd["sharpness_grad"].cpu().numpy().reshape(-1)[0])
    # the kernel sums a lane's steps in order, reduces the wave in 6 levels
    # and adds one value per wavefront to the scalar: no term passes through
    # more than (steps of a lane) + 6 + (wavefronts) additions, the depth of
    # that summation tree, which bounds the error as K does for a chain
    assert_close_model("sharpness_grad", np.array([sg]), np.array([ref.sharpness_grad]),
                       np.array([ref.sharpness_abs]),
                       np.array([min(ref.sharpness_k, sum_depth(w, ref))]))
    print(f"sharpness: gpu {sg!r} ref {ref.sharpness_grad!r} |d| {abs(sg - ref.sharpness_grad):.3e} "
          f"sqrt(K) u A {np.sqrt(max(ref.sharpness_k, 1)) * U * ref.sharpness_abs:.3e}")
    if "point_error" in bwd:
        assert_close_model("point_error", bwd["point_error"].cpu().numpy().reshape(-1),
                           ref.point_error.reshape(-1), np.abs(ref.point_error.reshape(-1)), R)
    assert np.all(bwd["ray_grad"].cpu().numpy() == 0)


@pytest.mark.parametrize("mode", ["sdfoam", "standard"])
def test_backward_parity_c1(torch_dev, oracle_lib, mode):
    w = scene(1, mode=mode)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, mode, ray_error=True)
    _check_backward(bwd, st, ref, w)


def test_backward_parity_c2(torch_dev, oracle_lib):
    w = scene(2)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, "sdfoam")
    _check_backward(bwd, st, ref, w)


@pytest.mark.parametrize("degree", [1, 2])
@pytest.mark.parametrize("mode", ["sdfoam", "standard"])
def test_sh_degrees_1_2(torch_dev, oracle_lib, mode, degree):
    """SH degrees 1 and 2 (the accumulator's 32-float rows; owner lanes of
    13 and 28 attribute components): forward and backward with the walk
    record against the oracle."""
    w = scene(1, mode=mode, sh_degree=degree)
    assert w.sh_degree == degree
    out, st, ref = _forward_both(w, torch_dev, oracle_lib, mode)
    _check_forward(out, st, ref, w, 0)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, mode, ray_error=True, walk=True)
    _check_backward(bwd, st, ref, w)


@pytest.mark.parametrize("mode", ["sdfoam", "standard"])
def test_backward_direct_updates_c1(torch_dev, oracle_lib, mode):
    """The backward without the gradient accumulator: atomics straight into
    points_grad, attribute_grad and point_error."""
    w = scene(1, mode=mode)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, mode, ray_error=True, walk=True,
                                  grad_accum=False)
    _check_backward(bwd, st, ref, w)


def test_backward_direct_updates_c2(torch_dev, oracle_lib):
    w = scene(2)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, "sdfoam", walk=True,
                                  grad_accum=False)
    _check_backward(bwd, st, ref, w)


@pytest.mark.parametrize("mode", ["sdfoam", "standard"])
@pytest.mark.parametrize("pool", ["one chunk per XCD", "a third"])
def test_backward_walk_record_small_pool(torch_dev, oracle_lib, mode, pool, monkeypatch):
    """Walk records whose chunk pool runs out: wavefronts that find none
    left record nothing from there on and the backward scans those trips
    (8 chunks: most wavefronts get none; a third of the chunks every trip
    needs: the pool runs out part way through the launch)."""
    from sdfoam_amd import _lib, pipeline

    w = scene(2, mode=mode)
    full = int(_lib.lib().sdf_walk_record_full_chunks(w.num_rays, w.rays.shape[-2], 1026))
    n = 8 if pool == "one chunk per XCD" else full // 3
    monkeypatch.setattr(pipeline._RecordNeed, "estimate", lambda self: n)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, mode, walk=True)
    _check_backward(bwd, st, ref, w)


def test_walk_record_sized_by_need(torch_dev):
    """The record's counters hold the chunks the walk asked for: every
    wavefront claims one chunk per 16 trips it walks (its longest lane's
    loop count, num_intersections).  The next forward's pool has, for each
    of the 8 XCDs, the most one XCD asked for plus an eighth and one."""
    import math

    import torch

    import sdfoam_amd
    from sdfoam_amd import _lib, pipeline

    w = scene(1)
    g = gpu_scene(w, torch_dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    inv_t = torch.tensor([w.inv_s], device=torch_dev)
    fwd = pipe.trace_forward(**g, alpha_mode="sdfoam", inv_s=inv_t, record_walk=True)
    torch.cuda.synchronize()
    plan = fwd["trace_plan"]
    counters = plan.record_counters().cpu().numpy()
    asked = int(counters.sum())
    H, W = w.rays.shape[:2]
    ni = np_u32(fwd["num_intersections"]).reshape(H, W).astype(np.int64)
    want = 0
    for ty in range(0, H, 8):
        for tx in range(0, W, 8):
            want += -(-min(int(ni[ty:ty + 8, tx:tx + 8].max()), plan.budget) // 16)
    assert asked == want
    _, _, have = record_rows(plan)
    assert int(have.sum()) // 16 == asked  # the first pool had room for every claim
    fwd2 = pipe.trace_forward(**g, alpha_mode="sdfoam", inv_s=inv_t, record_walk=True)
    per = math.ceil(int(counters.max()) * pipeline.RECORD_MARGIN) + 1
    full = int(_lib.lib().sdf_walk_record_full_chunks(w.num_rays, W, plan.budget))
    assert fwd2["trace_plan"].chunks == min(8 * per, full)


@pytest.mark.parametrize("budget", [None, 2, 7])
def test_backward_walk_record_c1(torch_dev, oracle_lib, budget):
    """Backward replaying the forward's walk record: full record, and budgets
    so small that every wavefront goes back to scanning mid-walk."""
    w = scene(1)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, "sdfoam", ray_error=True, walk=True,
                                  walk_budget=budget)
    _check_backward(bwd, st, ref, w)


def test_backward_walk_record_c2(torch_dev, oracle_lib):
    w = scene(2)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, "sdfoam", walk=True)
    _check_backward(bwd, st, ref, w)


def test_backward_walk_record_c2_sharp(torch_dev, oracle_lib):
    """inv_s = 50: walks end on the weight threshold, lanes of a wavefront
    stop at different trips."""
    w = scene(2)
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, "sdfoam", inv_s=50.0, walk=True)
    _check_backward(bwd, st, ref, w)


@pytest.mark.parametrize("budget", [None, 2])
def test_walk_record_standard_mode(torch_dev, oracle_lib, budget):
    """Standard mode: the forward records the steps where the density
    backward's unsafe walk takes the same exit and the backward replays them
    (budget 2: every wavefront goes back to its own unsafe scan mid-walk)."""
    w = scene(1, mode="standard")
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, "standard", ray_error=True,
                                  walk=True, walk_budget=budget)
    _check_backward(bwd, st, ref, w)


def test_walk_record_standard_mode_c2(torch_dev, oracle_lib):
    w = scene(2, mode="standard")
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, "standard", walk=True)
    _check_backward(bwd, st, ref, w)


@pytest.mark.parametrize("cfg", [1, 2])
def test_walk_record_standard_marks_differing_steps(torch_dev, cfg):
    """The standard-mode parity tests above cover the backward's re-meet
    replay only if their scenes hold steps where the unsafe walk leaves the
    forward's: count the entries the forward marks {next | 2^31, t1}.  C2 has
    them (asserted); C1's count is reported."""
    import torch

    import sdfoam_amd

    w = scene(cfg, mode="standard")
    g = gpu_scene(w, torch_dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    fwd = pipe.trace_forward(**g, alpha_mode="standard", record_walk=True)
    plan = fwd["trace_plan"]
    torch.cuda.synchronize()
    E, _, have = record_rows(plan)
    nxt = E[have] & np.uint64(0xFFFFFFFF)
    marked = int(np.count_nonzero(((nxt & np.uint64(0x80000000)) != 0)
                                  & (nxt < np.uint64(0xFFFFFFFE))))
    stepped = int(np.count_nonzero(nxt < np.uint64(w.num_points)))
    print(f"C{cfg} standard: {marked} marked of {stepped + marked} recorded steps")
    if cfg == 2:
        assert marked > 0


def test_walk_record_mismatch_raises(torch_dev):
    import torch

    import sdfoam_amd

    w = scene(1)
    g = gpu_scene(w, torch_dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    inv_t = torch.tensor([w.inv_s], device=torch_dev)
    fwd = pipe.trace_forward(**g, alpha_mode="sdfoam", inv_s=inv_t, record_walk=True)
    with pytest.raises(RuntimeError, match="trace_plan does not belong"):
        pipe.trace_backward(**g, rgb_out=fwd["rgba"], grad_in=to_dev(w.grad_rgba, torch_dev),
                            alpha_mode="sdfoam", inv_s=inv_t, max_intersections=100,
                            trace_plan=fwd["trace_plan"])


def test_backward_reuses_forward_table(torch_dev):
    """With the forward's plan the backward skips rebuilding the offset table
    while the scene tensors are unmodified, and rebuilds it after an in-place
    change of the points (version counter)."""
    import torch

    import sdfoam_amd
    from sdfoam_amd import _lib

    w = scene(2)
    g = gpu_scene(w, torch_dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    inv_t = torch.tensor([w.inv_s], device=torch_dev)
    grad = to_dev(w.grad_rgba, torch_dev)

    def backward(plan):
        _lib.set_timing(True)
        b = pipe.trace_backward(**g, rgb_out=fwd["rgba"], grad_in=grad, alpha_mode="sdfoam",
                                inv_s=inv_t, trace_plan=plan)
        torch.cuda.synchronize()
        kinds = [k for k, _ in _lib.collect_timings()]
        _lib.set_timing(False)
        return b, kinds

    fwd = pipe.trace_forward(**g, alpha_mode="sdfoam", inv_s=inv_t, record_walk=True)
    b_reuse, kinds = backward(fwd["trace_plan"])
    assert "prefetch_adjacent_diff" not in kinds and "backward" in kinds
    b_plain, kinds = backward(None)
    assert "prefetch_adjacent_diff" in kinds
    g["points"].add_(0.0)  # same values, new version: the kept table is not trusted
    b_again, kinds = backward(fwd["trace_plan"])
    assert "prefetch_adjacent_diff" in kinds
    # the runs differ only in the order of their fp32 atomics (parity with the
    # oracle is tested above); a wrong table would change the walks entirely
    for k in ("points_grad", "attr_grad", "sharpness_grad"):
        ref = b_plain[k].cpu().numpy()
        for b in (b_reuse, b_again):
            np.testing.assert_allclose(b[k].cpu().numpy(), ref, rtol=1e-4,
                                       atol=1e-5 * float(np.abs(ref).max()))


@pytest.mark.parametrize("mode,dtype", [("sdfoam", "float32"), ("standard", "float32"),
                                        ("sdfoam", "float16"), ("standard", "float16")])
def test_cell_table_same_results(torch_dev, mode, dtype, monkeypatch):
    """The forward over the cell table (the default) and over the caller's
    arrays give the same bits: rgba, depths, depth indices, loop counts and
    the walk record (steps and their colours; the records are zeroed first,
    since a wave writes only the rows it walks) are per ray and
    deterministic.  Contribution is summed by fp32 atomics in any order, so
    it is compared to the summation bound used against the oracle."""
    import torch

    import sdfoam_amd
    from sdfoam_amd import pipeline

    allocate = pipeline.TracePlan.allocate_record

    def allocate_zeroed(self, budget, chunks=0):
        allocate(self, budget, chunks)
        self.entries.zero_()

    monkeypatch.setattr(pipeline.TracePlan, "allocate_record", allocate_zeroed)

    w = scene(2, mode=mode)
    g = gpu_scene(w, torch_dev)
    tdt = torch.float16 if dtype == "float16" else torch.float32
    g["attributes"] = g["attributes"].to(tdt)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree, dtype)
    q = to_dev(w.quantiles, torch_dev)
    inv_t = torch.tensor([w.inv_s], device=torch_dev)
    outs = [pipe.trace_forward(**g, depth_quantiles=q, return_contribution=True, alpha_mode=mode,
                               inv_s=inv_t, record_walk=True, walk_budget=64, cell_table=ct)
            for ct in (False, True)]
    torch.cuda.synchronize()
    a, b = outs

    def bits(t):
        return t.contiguous().view(torch.uint8).cpu().numpy()

    for k in ("rgba", "depth", "depth_indices", "num_intersections"):
        assert np.array_equal(bits(a[k]), bits(b[k])), k
    for x, y, name in zip(record_rows(a["trace_plan"]), record_rows(b["trace_plan"]),
                          ("record entries", "record colours", "record chunks")):
        assert np.array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8)), name
    ca = a["contribution"].double().cpu().numpy().ravel()
    cb = b["contribution"].double().cpu().numpy().ravel()
    if dtype == "float32":
        # the same fp32 weights (>= 0) summed in two orders, at most one per
        # ray: each sum is within gamma_R of the exact one
        tol = 2 * gamma(w.num_rays) * np.abs(ca) + 1e-30
        assert (np.abs(ca - cb) <= tol).all(), "contribution"
    else:
        # fp16 atomics round every add: compare the totals
        assert abs(ca.sum() - cb.sum()) <= 1e-2 * abs(ca.sum()) + 1e-3, "contribution"


def flat(w):
    """The workload with its rays as a flat [R, 6] batch (no image layout)."""
    import dataclasses

    R = w.num_rays
    return dataclasses.replace(
        w, rays=w.rays.reshape(R, 6), quantiles=w.quantiles.reshape(R, -1),
        grad_rgba=w.grad_rgba.reshape(R, 4), depth_grad=w.depth_grad.reshape(R, -1),
        extra=dict(w.extra, start=w.extra["start"].reshape(R)))


@pytest.mark.parametrize("mode", ["sdfoam", "standard"])
def test_sorted_rays_c1(torch_dev, oracle_lib, mode):
    """Rays traced in the order of sdf_ray_order: same results, forward and
    backward (the backward sorts again when it gets no plan)."""
    w = flat(scene(1, mode=mode))
    out, st, ref = _forward_both(w, torch_dev, oracle_lib, mode, record=1100, sort_rays=True)
    _check_forward(out, st, ref, w, 1100)
    assert out["trace_plan"].order is not None
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, mode, ray_error=True, sort_rays=True)
    _check_backward(bwd, st, ref, w)


def test_sorted_rays_with_walk_record_c2(torch_dev, oracle_lib):
    """C2's 160000 rays as a flat batch: sorted automatically (>= 32768 rays)
    and replayed from the walk record."""
    w = flat(scene(2))
    bwd, st, ref = _backward_both(w, torch_dev, oracle_lib, "sdfoam", walk=True)
    _check_backward(bwd, st, ref, w)
    out, st, ref = _forward_both(w, torch_dev, oracle_lib, "sdfoam", record=0)
    _check_forward(out, st, ref, w, 0)
    assert out["trace_plan"].order is not None


def test_ray_order_is_a_stable_permutation(torch_dev):
    """sdf_ray_order: a permutation of the rays, grouped by start cell, the
    same on every call."""
    import torch

    import sdfoam_amd

    w = flat(scene(2))
    g = gpu_scene(w, torch_dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    o1 = pipe.trace_forward(**g, sort_rays=True)["trace_plan"].order
    o2 = pipe.trace_forward(**g, sort_rays=True)["trace_plan"].order
    torch.cuda.synchronize()
    a = o1.cpu().numpy().view(np.uint32)
    assert np.array_equal(a, o2.cpu().numpy().view(np.uint32))
    assert np.array_equal(np.sort(a), np.arange(w.num_rays, dtype=np.uint32))
    st = w.extra["start"][a]
    assert np.all(np.diff(st.astype(np.int64)) >= 0)


def test_aabb_tree_and_nn_exact(torch_dev, oracle_lib):
    import torch

    import sdfoam_amd

    w = scene(2)
    pts = to_dev(w.points, torch_dev)
    tree = sdfoam_amd.build_aabb_tree(pts)
    torch.cuda.synchronize()
    ref_tree = oracle_lib.build_aabb_tree(w.points)
    got = tree.cpu().numpy()
    n2 = got.shape[0]
    assert np.array_equal(got[: n2 - 1], ref_tree[: n2 - 1])
    rng = np.random.default_rng(5)
    queries = np.concatenate([
        rng.uniform(-1.6, 1.6, (3000, 3)),
        rng.normal(0, 3, (500, 3)),
        w.points[rng.integers(0, w.num_points, 200)],  # exact hits
        w.rays.reshape(-1, 6)[:1, :3],
    ]).astype(np.float32)
    idx = sdfoam_amd.nn(pts, tree, to_dev(queries, torch_dev))
    torch.cuda.synchronize()
    ref = oracle_lib.nn(w.points, queries, threads=_threads())
    assert np.array_equal(np_u32(idx), ref)


@pytest.mark.parametrize("n", [32, 33, 64, 65, 129, 4096, 4097, 70_000, 300_000])
def test_nn_tree_depths(torch_dev, oracle_lib, n):
    """nn over trees of every shape the search distinguishes: one group of
    points (n <= 64), the depth-6 boxes over points (n <= 4096), the depth-6
    and depth-12 boxes held in LDS over points, and boxes below depth 12 read
    from the tree (n > 262,144).  Duplicated points make ties, which go to
    the smaller index; the host's exact nearest neighbour is the reference."""
    import torch

    import sdfoam_amd

    rng = np.random.default_rng(n)
    pts = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
    pts[n // 2] = pts[n // 3]
    pts[n - 1] = pts[0]
    queries = np.concatenate([
        rng.uniform(-1.3, 1.3, (2000, 3)),
        rng.normal(0, 5, (100, 3)),
        pts[rng.integers(0, n, 100)],
        pts[[n // 2, n // 3, 0, n - 1]],
    ]).astype(np.float32)
    p = to_dev(pts, torch_dev)
    tree = sdfoam_amd.build_aabb_tree(p)
    idx = sdfoam_amd.nn(p, tree, to_dev(queries, torch_dev))
    torch.cuda.synchronize()
    ref = oracle_lib.nn(pts, queries, threads=_threads())
    assert np.array_equal(np_u32(idx), ref)
    assert ref[-4] == ref[-3] == n // 3 and ref[-2] == ref[-1] == 0


def test_get_starting_point_matches_nn(torch_dev, oracle_lib):
    import torch

    import sdfoam_amd

    w = scene(1)
    pts = to_dev(w.points, torch_dev)
    tree = sdfoam_amd.build_aabb_tree(pts)
    rays = to_dev(w.rays, torch_dev)
    sp = sdfoam_amd.get_starting_point(rays, pts, tree)
    torch.cuda.synchronize()
    assert sp.dtype == torch.uint32 and tuple(sp.shape) == w.rays.shape[:-1]
    assert np.array_equal(np_u32(sp), w.extra["start"])


@pytest.mark.parametrize("origins", [1, 64, 255, 256, 3000])
def test_start_points_batch(torch_dev, oracle_lib, origins):
    """get_starting_point on a batch of random rays from `origins` distinct
    positions (drawn with replacement, so every origin repeats), some inside
    the point cloud and some far outside it, the first one at the origin with
    x = +0 or -0 (two bit patterns, so origins + 1 keys): equal to nn over
    the distinct origins (the reference's torch.unique + nn) and to the
    host's exact nearest neighbour.  Up to 256 keys are searched by the scan
    over all points (255 origins: exactly 256), more by the tree (256)."""
    import torch

    import sdfoam_amd

    w = scene(2)
    pts = to_dev(w.points, torch_dev)
    tree = sdfoam_amd.build_aabb_tree(pts)
    rng = np.random.default_rng(origins)
    cams = rng.normal(0.0, 1.0, (origins, 3)).astype(np.float32)
    cams *= rng.choice([0.3, 4.0], size=(origins, 1)).astype(np.float32)
    cams[0] = 0.0
    R = 20000
    pick = rng.integers(0, origins, R)
    rays = np.zeros((R, 6), dtype=np.float32)
    rays[:, :3] = cams[pick]
    rays[:, 3:] = rng.normal(size=(R, 3)).astype(np.float32)
    rays[pick == 0, 0] = np.where(rng.random((pick == 0).sum()) < 0.5, 0.0, -0.0)
    rd = to_dev(rays, torch_dev)
    sp = sdfoam_amd.get_starting_point(rd, pts, tree)
    uniq, inv = torch.unique(rd[:, :3], dim=0, return_inverse=True)
    ref = sdfoam_amd.nn(pts, tree, uniq).long()[inv]
    torch.cuda.synchronize()
    got = np_u32(sp)
    assert np.array_equal(got, ref.cpu().numpy().astype(np.uint32))
    host = oracle_lib.nn(w.points, cams, threads=_threads())
    assert np.array_equal(got, host[pick])


def test_trace_rays_autograd(torch_dev):
    import torch

    import sdfoam_amd

    w = scene(1)
    g = gpu_scene(w, torch_dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    pts = g["points"].clone().requires_grad_(True)
    attrs = g["attributes"].clone().requires_grad_(True)
    inv = torch.full((w.num_points, 1), w.inv_s, device=torch_dev, requires_grad=True)
    q = to_dev(w.quantiles, torch_dev)
    rgba, depth, contrib, nis, errbox, alpha = sdfoam_amd.TraceRays.apply(
        pipe, pts, attrs, g["point_adjacency"], g["point_adjacency_offsets"], g["rays"],
        g["start_point"], q, True, True, inv, 1e-6, w.attributes.shape[-1] - 1)
    gr = to_dev(w.grad_rgba, torch_dev)
    gd = to_dev(w.depth_grad, torch_dev)
    loss = (rgba * gr).sum() + (depth * gd).sum()
    loss.backward()
    assert pts.grad is not None and attrs.grad is not None and inv.grad is not None
    assert torch.isfinite(pts.grad).all() and torch.isfinite(attrs.grad).all()
    assert inv.grad.shape == inv.shape
    # only element 0 of the sharpness gradient is written (the reference reads sharpness[0])
    assert torch.count_nonzero(inv.grad[1:]) == 0
    assert float(rgba.detach()[..., 3].max()) <= 1.0
    del contrib, nis, errbox, alpha


def test_walk_record_other_attributes(torch_dev):
    """A plan handed to a backward over other attributes than its forward's
    (the record holds the forward's colours) leaves its walk record out: the
    gradients equal those of the backward without a plan, not those the
    forward's colours would give."""
    import torch

    import sdfoam_amd

    w = scene(2)
    g = gpu_scene(w, torch_dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    inv_t = torch.tensor([w.inv_s], device=torch_dev)
    grad = to_dev(w.grad_rgba, torch_dev)
    fwd = pipe.trace_forward(**g, alpha_mode="sdfoam", inv_s=inv_t, record_walk=True)
    g2 = dict(g)
    g2["attributes"] = g["attributes"] * 1.25 + 0.05

    def backward(plan):
        return pipe.trace_backward(**g2, rgb_out=fwd["rgba"], grad_in=grad, alpha_mode="sdfoam",
                                   inv_s=inv_t, trace_plan=plan)

    b_plan, b_plain = backward(fwd["trace_plan"]), backward(None)
    b_own = pipe.trace_backward(**g, rgb_out=fwd["rgba"], grad_in=grad, alpha_mode="sdfoam",
                                inv_s=inv_t, trace_plan=fwd["trace_plan"])
    for k in ("points_grad", "attr_grad", "sharpness_grad"):
        ref = b_plain[k].cpu().numpy()
        np.testing.assert_allclose(b_plan[k].cpu().numpy(), ref, rtol=1e-4,
                                   atol=1e-5 * float(np.abs(ref).max()))
    # the other attributes change the gradients (the check above can fail)
    a, b = b_own["attr_grad"].cpu().numpy(), b_plain["attr_grad"].cpu().numpy()
    assert np.abs(a - b).max() > 1e-3 * np.abs(b).max()
