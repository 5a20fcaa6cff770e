"""GPU checks at the full sizes of configs C4 (3M points, 8 ring cameras of
1297x840) and C5 (2M points with a stale adjacency, 2^20 rays drawn from 64
cameras, two quantiles), where the oracle would take minutes on every ray:

* size-independent properties of the full batch: the start cells of
  get_starting_point equal the host nearest neighbour; the contributions of
  all cells sum to the sum of the rays' opacities (sum_k T_k alpha_k =
  1 - T per ray); loop counts and depth indices are in range; gradients are
  finite;
* oracle parity (the bars of test_gpu_parity) on a seeded subset of the
  same rays, forward and backward with the walk record, and the inference
  render of a full C4 camera bit-exact;
* at the headline config C3, the measured forward and backward against the
  oracle on every one of the 1.92M rays;
* the GPU triangulation of C3's 1M points against Qhull, every table.

Scene generation (Qhull at 2-3M points) takes one to two minutes; progress
lines are printed as each stage ends."""

import dataclasses
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def say(pytestconfig):
    capman = pytestconfig.pluginmanager.getplugin("capturemanager")
    t0 = time.time()

    def _say(msg):
        with capman.global_and_fixture_disabled():
            print(f"\n[large {time.time() - t0:6.1f}s] {msg}", flush=True)

    return _say


_CACHE = {}


def big_scene(index, say):
    if index not in _CACHE:
        from sdfoam_amd import scenes

        say(f"generating C{index}")
        w = scenes.make_config(index)
        say(f"C{index} ready: N={w.num_points} E={w.adjacency.size} R={w.num_rays}")
        _CACHE[index] = w
    return _CACHE[index]


def _u32(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev).view(torch.uint32)


def _full_batch_properties(w, dev, say, rays_np, q_np, g_np, dg_np):
    """GPU start cells, forward + backward with the walk record over the
    whole batch, and the properties that hold at any size."""
    import torch

    import sdfoam_amd
    from sdfoam_amd import scenes

    pts = torch.from_numpy(w.points).to(dev)
    attrs = torch.from_numpy(w.attributes).to(dev)
    adj, offs = _u32(w.adjacency, dev), _u32(w.offsets, dev)
    rays = torch.from_numpy(rays_np).to(dev)
    tree = sdfoam_amd.build_aabb_tree(pts)
    start = sdfoam_amd.get_starting_point(rays, pts, tree)
    torch.cuda.synchronize()
    host_start = scenes.start_points_for(w.points, rays_np)
    got_start = start.view(torch.int32).cpu().numpy().view(np.uint32)
    assert np.array_equal(got_start.reshape(-1), host_start.reshape(-1)), "start cells"
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    inv = torch.tensor([w.inv_s], device=dev)
    q = torch.from_numpy(q_np).to(dev)
    fwd = pipe.trace_forward(pts, attrs, adj, offs, rays, start, depth_quantiles=q,
                             return_contribution=True, alpha_mode="sdfoam", inv_s=inv,
                             record_walk=True)
    bwd = pipe.trace_backward(pts, attrs, adj, offs, rays, start, fwd["rgba"],
                              torch.from_numpy(g_np).to(dev), q, fwd["depth_indices"],
                              torch.from_numpy(dg_np).to(dev), alpha_mode="sdfoam", inv_s=inv,
                              trace_plan=fwd["trace_plan"])
    torch.cuda.synchronize()
    say(f"full batch traced: {rays_np.size // 6} rays")
    rgba = fwd["rgba"].cpu().numpy().reshape(-1, 4)
    contrib = fwd["contribution"].cpu().numpy().astype(np.float64)
    a_sum = float(np.sum(rgba[:, 3].astype(np.float64)))
    c_sum = float(np.sum(contrib))
    assert abs(c_sum - a_sum) <= 1e-4 * a_sum + 1e-3, (c_sum, a_sum)
    ni = fwd["num_intersections"].view(torch.int32).cpu().numpy().reshape(-1)
    assert ni.min() >= 1 and ni.max() <= 1025
    didx = fwd["depth_indices"].view(torch.int32).cpu().numpy().view(np.uint32).reshape(-1)
    assert np.all((didx < w.num_points) | (didx == 0xFFFFFFFF))
    for k in ("points_grad", "attr_grad", "sharpness_grad"):
        assert torch.isfinite(bwd[k]).all(), k
    assert float(rgba[:, 3].mean()) > 0.05  # the batch sees geometry
    return host_start


def _subset(w, rays, q, g, dg, start):
    return dataclasses.replace(w, rays=np.ascontiguousarray(rays), quantiles=np.ascontiguousarray(q),
                               grad_rgba=np.ascontiguousarray(g),
                               depth_grad=np.ascontiguousarray(dg),
                               extra={"start": np.ascontiguousarray(start)})


def test_c5_training_step(dev, oracle_lib, say):
    from test_gpu_parity import _backward_both, _check_backward, _check_forward, _forward_both

    w = big_scene(5, say)
    start = _full_batch_properties(w, dev, say, w.rays, w.quantiles, w.grad_rgba, w.depth_grad)
    sub = _subset(w, w.rays[::16], w.quantiles[::16], w.grad_rgba[::16], w.depth_grad[::16],
                  start.reshape(-1)[::16])
    out, st, ref = _forward_both(sub, dev, oracle_lib, "sdfoam", record=0)
    _check_forward(out, st, ref, sub, 0)
    say("C5 subset forward parity")
    bwd, st, ref = _backward_both(sub, dev, oracle_lib, "sdfoam", walk=True)
    _check_backward(bwd, st, ref, sub)
    say("C5 subset backward parity")


def test_c4_cameras(dev, oracle_lib, say):
    from test_gpu_parity import _backward_both, _check_backward, _check_forward, _forward_both

    w = big_scene(4, say)
    start = _full_batch_properties(w, dev, say, w.rays, w.quantiles, w.grad_rgba, w.depth_grad)
    # camera 3, every 8th row and column: an image-shaped subset (tile path)
    sl = (3, slice(None, None, 8), slice(None, None, 8))
    sub = _subset(w, w.rays[sl], w.quantiles[sl], w.grad_rgba[sl], w.depth_grad[sl], start[sl])
    out, st, ref = _forward_both(sub, dev, oracle_lib, "sdfoam", record=0)
    _check_forward(out, st, ref, sub, 0)
    say("C4 subset forward parity")
    bwd, st, ref = _backward_both(sub, dev, oracle_lib, "sdfoam", walk=True)
    _check_backward(bwd, st, ref, sub)
    say("C4 subset backward parity")


FNV_OFFSET = np.uint64(0xcbf29ce484222325)
FNV_PRIME = np.uint64(0x100000001b3)


def record_walks(plan, start, num_points):
    """Per-ray visit hash (FNV-1a over the stepped cells, as the oracle's) and
    step count of an sdfoam forward over image-shaped rays, decoded from the
    walk record that forward wrote.  Wavefront w of the record is the 8x8
    quarter w % 4 of 16x16 pixel tile w // 4 (row-major tiles); lane l is
    pixel (l % 8, l // 8) of that quarter.  Each trip's entry holds the next
    cell of the lane's step, 0xffffffff where the walk ended without a step
    and 0xfffffffe where the lane walks no more; a trip past the wavefront's
    last one has no chunk (table entry 0xffffffff).  Fails if some XCD asked
    for more chunks than its part of the pool held (trips left unrecorded)."""
    import torch

    from sdfoam_amd import _lib

    W, R = plan.ray_image_width, plan.num_rays
    H = R // W
    slots = -(-plan.budget // 16)
    waves = int(_lib.lib().sdf_walk_record_full_chunks(R, W, plan.budget)) // slots
    pool = -(-plan.chunks // 8) * 8
    asked = plan.record_counters().cpu().numpy()
    assert int(asked.max()) <= pool // 8, ("pool too small", asked, pool)
    off = plan.record_ptr - plan.entries.data_ptr()
    head = 8 * 256
    table = plan.entries[off + head:off + head + waves * slots * 4].cpu().numpy()
    table = table.view(np.uint32).reshape(waves, slots)
    e0 = off + head + -(-waves * slots * 4 // 256) * 256
    ents = plan.entries[e0:e0 + pool * 1024 * 8].view(torch.int32).cpu().numpy()
    nxt = ents.view(np.uint32)[0::2]  # {next, t1 bits} pairs: the next cells
    del ents
    tiles_x = -(-W // 16)
    w = np.arange(waves, dtype=np.int64)[:, None]
    ln = np.arange(64, dtype=np.int64)[None, :]
    t, qd = w // 4, w % 4
    x = (t % tiles_x) * 16 + (qd & 1) * 8 + (ln & 7)
    y = (t // tiles_x) * 16 + (qd >> 1) * 8 + (ln >> 3)
    valid = ((x < W) & (y < H)).reshape(-1)
    ray = (y * W + x).reshape(-1)
    cur = np.zeros(waves * 64, dtype=np.uint32)
    cur[valid] = start.reshape(-1)[ray[valid]]
    h = np.full(waves * 64, FNV_OFFSET, dtype=np.uint64)
    steps = np.zeros(waves * 64, dtype=np.uint32)
    idx = np.nonzero(valid & (cur < num_points))[0]
    for trip in range(plan.budget):
        if idx.size == 0:
            break
        c = table[idx >> 6, trip >> 4].astype(np.int64)
        e = np.full(idx.size, 0xFFFFFFFE, dtype=np.uint32)
        have = c != 0xFFFFFFFF
        e[have] = nxt[c[have] * 1024 + (trip & 15) * 64 + (idx[have] & 63)]
        stepped = e < num_points
        si = idx[stepped]
        h[si] = (h[si] ^ cur[si].astype(np.uint64)) * FNV_PRIME
        steps[si] += 1
        cur[si] = e[stepped]
        idx = si
    assert idx.size == 0, "lanes still walking at the end of the budget"
    out_h = np.zeros(R, dtype=np.uint64)
    out_s = np.zeros(R, dtype=np.uint32)
    out_h[ray[valid]] = h[valid]
    out_s[ray[valid]] = steps[valid]
    return out_h, out_s


_C3 = {}


def _c3_headline(dev, oracle_lib, say):
    """The headline step as bench.py runs it, set up once per module: C3's
    scene and start cells, a first forward that sizes the walk record, then
    the measured forward (cell table, walk record in a pool sized by the
    first forward's need), and the oracle forward on every ray."""
    if _C3:
        return _C3
    import torch

    import sdfoam_amd
    from test_gpu_parity import _threads

    w = big_scene(3, say)
    start = _full_batch_properties(w, dev, say, w.rays, w.quantiles, w.grad_rgba, w.depth_grad)
    g = dict(points=torch.from_numpy(w.points).to(dev),
             attributes=torch.from_numpy(w.attributes).to(dev),
             point_adjacency=_u32(w.adjacency, dev), point_adjacency_offsets=_u32(w.offsets, dev),
             rays=torch.from_numpy(w.rays).to(dev), start_point=_u32(start, dev))
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    inv = torch.tensor([w.inv_s], device=dev)
    q = torch.from_numpy(w.quantiles).to(dev)
    first = pipe.trace_forward(**g, depth_quantiles=q, return_contribution=True,
                               alpha_mode="sdfoam", inv_s=inv, record_walk=True)
    torch.cuda.synchronize()
    full_pool = first["trace_plan"].chunks
    del first
    fwd = pipe.trace_forward(**g, depth_quantiles=q, return_contribution=True,
                             alpha_mode="sdfoam", inv_s=inv, record_walk=True)
    torch.cuda.synchronize()
    plan = fwd["trace_plan"]
    assert plan.chunks < full_pool  # sized by the first forward's need
    say(f"C3 measured forward: record pool of {plan.chunks} chunks")
    ref = oracle_lib.trace_forward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                   w.rays, start, w.quantiles, alpha_mode="sdfoam",
                                   inv_s=w.inv_s, threads=_threads(), point_visits=True)
    say(f"oracle forward on all {w.num_rays} rays ({float(ref.steps.mean()):.1f} steps per ray)")
    _C3.update(w=w, start=start, g=g, pipe=pipe, inv=inv, q=q, fwd=fwd, ref=ref)
    return _C3


def test_c3_headline_forward(dev, oracle_lib, say):
    """The headline workload as bench.py times it (C3: 1M points near a
    superquadric, SH degree 3, sdfoam alpha, inv_s = e^0.3, 1600x1200 rays),
    checked on every one of the 1.92M rays against the oracle:

    * the visit hash and step count of each ray, decoded from the walk record
      that the measured forward launch (the cell-table kernel, with the exit
      neighbours taken from the table's int16 deltas) wrote, bit-exact;
    * that launch's num_intersections and depth indices bit-exact, rgba and
      depth within 1e-4 / 1e-5;
    * its contribution within the summation bound with K = each point's
      number of cell steps (from the oracle); unvisited points exactly 0;
    * the backward's walk of every ray (walk statistics of the backward
      kernel) equals the oracle's."""
    import torch

    from test_gpu_parity import assert_close, assert_close_model, np_u32

    c = _c3_headline(dev, oracle_lib, say)
    w, fwd, ref = c["w"], c["fwd"], c["ref"]
    R = w.num_rays
    vh, st = record_walks(fwd["trace_plan"], c["start"], w.num_points)
    assert np.array_equal(st, ref.steps.reshape(R)), "steps (walk record)"
    assert np.array_equal(vh, ref.visit_hash.reshape(R)), "visit hash (walk record)"
    say(f"C3 visit hashes of the measured forward bit-exact on all {R} rays")
    ni = np_u32(fwd["num_intersections"]).reshape(R)
    assert np.array_equal(ni, ref.num_intersections.reshape(R)), "num_intersections"
    assert np.array_equal(np_u32(fwd["depth_indices"]).reshape(R, -1),
                          ref.depth_indices.reshape(R, -1)), "depth_indices"
    assert_close("rgba", fwd["rgba"].cpu().numpy().reshape(R, 4), ref.rgba.reshape(R, 4))
    assert_close("depth", fwd["depth"].cpu().numpy().reshape(R, -1), ref.depth.reshape(R, -1))
    contrib = fwd["contribution"].cpu().numpy().reshape(-1)
    cref = ref.contribution.reshape(-1)
    k = ref.point_visits
    assert np.all(contrib[k == 0] == 0.0), "contribution of unvisited points"
    assert_close_model("contribution", contrib, cref, np.abs(cref), k)
    say(f"C3 contribution within the bound (K up to {int(k.max())})")
    bst = c["pipe"].walk_stats(**c["g"], backward=True, alpha_mode="sdfoam", inv_s=c["inv"])
    torch.cuda.synchronize()
    assert np.array_equal(bst["visit_hash"].cpu().numpy().view(np.uint64),
                          ref.visit_hash.reshape(-1)), "backward walk"


def test_c3_headline_backward(dev, oracle_lib, say):
    """The measured backward of the headline step (the full 1.92M-ray batch
    replaying the measured forward's walk record, per-cell gradient
    accumulator, as bench.py times it) against the oracle's backward on every
    ray: position, attribute and sharpness gradients within the summation
    bound (per-element K and sum |c| from the oracle's side buffers)."""
    import torch

    from test_gpu_parity import _check_backward, _threads

    c = _c3_headline(dev, oracle_lib, say)
    w, fwd = c["w"], c["fwd"]
    bwd = c["pipe"].trace_backward(**c["g"], rgb_out=fwd["rgba"],
                                   grad_in=torch.from_numpy(w.grad_rgba).to(dev),
                                   depth_quantiles=c["q"], depth_indices=fwd["depth_indices"],
                                   depth_grad_in=torch.from_numpy(w.depth_grad).to(dev),
                                   alpha_mode="sdfoam", inv_s=c["inv"],
                                   trace_plan=fwd["trace_plan"])
    bst = c["pipe"].walk_stats(**c["g"], backward=True, alpha_mode="sdfoam", inv_s=c["inv"])
    torch.cuda.synchronize()
    say("C3 measured backward done; oracle backward on every ray")
    from test_gpu_parity import np_u32

    ref = oracle_lib.trace_backward(
        w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets, w.rays, c["start"],
        fwd["rgba"].cpu().numpy(), w.grad_rgba, w.quantiles, np_u32(fwd["depth_indices"]),
        w.depth_grad, alpha_mode="sdfoam", inv_s=w.inv_s, threads=_threads())
    say("oracle backward done")
    full = dataclasses.replace(w, extra={"start": np.ascontiguousarray(c["start"])})
    _check_backward(bwd, bst, ref, full)
    say(f"C3 backward parity on all {w.num_rays} rays")
    _C3.clear()


def test_c3_subset_backwards(dev, oracle_lib, say):
    """The other backward paths at C3, on image-shaped subsets: the backward
    that replays a walk record of its own forward (every 4th row and column,
    120k rays) and the one that scans every face again (no walk record; every
    8th row and column)."""
    from test_gpu_parity import _backward_both, _check_backward

    w = big_scene(3, say)
    start = w.extra.get("start")
    if start is None:
        from sdfoam_amd import scenes

        start = scenes.start_points_for(w.points, w.rays)
    sl = (slice(None, None, 4), slice(None, None, 4))
    sub = _subset(w, w.rays[sl], w.quantiles[sl], w.grad_rgba[sl], w.depth_grad[sl], start[sl])
    bwd, st, ref = _backward_both(sub, dev, oracle_lib, "sdfoam", walk=True)
    _check_backward(bwd, st, ref, sub)
    say(f"C3 backward parity on the {sub.num_rays}-ray image subset")
    del bwd, st, ref
    sl8 = (slice(None, None, 8), slice(None, None, 8))
    sub8 = _subset(w, w.rays[sl8], w.quantiles[sl8], w.grad_rgba[sl8], w.depth_grad[sl8],
                   start[sl8])
    bwd, st, ref = _backward_both(sub8, dev, oracle_lib, "sdfoam", walk=False)
    _check_backward(bwd, st, ref, sub8)
    say(f"C3 scanning backward parity on the {sub8.num_rays}-ray image subset")


def test_c4_render_full_camera(dev, oracle_lib, say):
    from test_gpu_render import _render_both

    from sdfoam_amd import scenes

    w = big_scene(4, say)
    cam = scenes.camera_dict(w.extra["cameras"][5])
    got, ref = _render_both(w, dev, oracle_lib, cam)
    assert np.array_equal(got, ref.rgba8)
    say("C4 full-camera render bit-exact")


def test_c3_triangulation_matches_qhull(dev, say):
    """Triangulation.rebuild at C3's 1M points: every table the GPU path
    (certified cells, the open points certified again among themselves,
    exhaustively, hull cells included, merge) produces equals the tables of
    Qhull's tetrahedralisation of all points, bit for bit; no point went to
    Qhull."""
    import torch

    import sdfoam_amd
    from sdfoam_amd import scenes
    from sdfoam_amd.triangulation import host_tables, qhull_tetrahedra

    pts_np, _ = scenes._scene_c3(np.random.default_rng(0))
    pts = torch.from_numpy(pts_np).to(dev)
    t = time.time()
    tri = sdfoam_amd.Triangulation(pts)
    torch.cuda.synchronize()
    say(f"GPU triangulation of {pts_np.shape[0]} points: {time.time() - t:.2f}s, "
        f"{tri.last_stats['open']} open points")
    assert tri.last_method == "gpu"
    st = tri.last_stats
    assert st.get("open_levels") and st["open_points_qhull"] == 0, st
    assert "open_gpu_retry" not in st, st
    sorted_pts = pts[tri.permutation().to(torch.long)].cpu().numpy()
    t = time.time()
    simplices, neighbors = qhull_tetrahedra(sorted_pts)
    ref = host_tables(sorted_pts, simplices, neighbors)
    say(f"Qhull + host tables: {time.time() - t:.1f}s")
    for k, v in ref.items():
        got = getattr(tri, k)().view(torch.int32).cpu().numpy().view(np.uint32)
        assert np.array_equal(got.reshape(v.shape), v), k


def test_c3_standard_record_replays_the_unsafe_walk(dev, oracle_lib, say):
    """Standard mode at C3 (1M points, 1600x1200 rays): the backward that
    replays the forward's record, leaving it where the unsafe walk differs and
    taking it up again where the walks meet, gives the gradients of the
    backward that scans every step.  A lane replaying from a wrong place would
    follow other cells and move the sums far outside this tolerance.  Both,
    and the standard-mode forward, also meet the oracle's parity bars on an
    image-shaped subset of the same workload."""
    import torch

    import sdfoam_amd
    from sdfoam_amd import scenes

    say("generating C3 (standard)")
    w = scenes.make_config(3, mode="standard")
    pts = torch.from_numpy(w.points).to(dev)
    attrs = torch.from_numpy(w.attributes).to(dev)
    adj, offs = _u32(w.adjacency, dev), _u32(w.offsets, dev)
    rays = torch.from_numpy(w.rays).to(dev)
    tree = sdfoam_amd.build_aabb_tree(pts)
    start = sdfoam_amd.get_starting_point(rays, pts, tree)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    q = torch.from_numpy(w.quantiles).to(dev)
    grad = torch.from_numpy(w.grad_rgba).to(dev)
    dg = torch.from_numpy(w.depth_grad).to(dev)
    fwd = pipe.trace_forward(pts, attrs, adj, offs, rays, start, depth_quantiles=q,
                             alpha_mode="standard", record_walk=True)

    def backward(plan):
        return pipe.trace_backward(pts, attrs, adj, offs, rays, start, fwd["rgba"], grad, q,
                                   fwd["depth_indices"], dg, alpha_mode="standard",
                                   trace_plan=plan)

    b_rec, b_scan = backward(fwd["trace_plan"]), backward(None)
    torch.cuda.synchronize()
    say("C3 standard backward with and without the record")
    for k in ("points_grad", "attr_grad"):
        a, b = b_rec[k].cpu().numpy(), b_scan[k].cpu().numpy()
        scale = float(np.abs(b).max())
        assert scale > 0, k
        np.testing.assert_allclose(a, b, rtol=1e-3, atol=1e-5 * scale, err_msg=k)
    del b_rec, b_scan, fwd
    # and both paths against the oracle (density mode) on the image subset of
    # every 4th row and column (120k rays through the tile path)
    from test_gpu_parity import _backward_both, _check_backward, _check_forward, _forward_both

    host_start = start.view(torch.int32).cpu().numpy().view(np.uint32).reshape(w.rays.shape[:-1])
    sl = (slice(None, None, 4), slice(None, None, 4))
    sub = _subset(w, w.rays[sl], w.quantiles[sl], w.grad_rgba[sl], w.depth_grad[sl],
                  host_start[sl])
    out, st, ref = _forward_both(sub, dev, oracle_lib, "standard", record=0)
    _check_forward(out, st, ref, sub, 0)
    for walk in (True, False):
        bwd, st, ref = _backward_both(sub, dev, oracle_lib, "standard", walk=walk)
        _check_backward(bwd, st, ref, sub)
    say(f"C3 standard forward and backward (record and scan) parity on {sub.num_rays} rays")
