"""The host mirror's argument checks, without a GPU: the same messages, in
the same order, as the reference's bindings
(torch_bindings/pipeline_bindings.cpp:12-75, 176-210, 734-751;
torch_bindings/triangulation_bindings.cpp:117-181).  Checks that come
before the device checks are reachable with CPU tensors."""

import pytest
import torch

import sdfoam_amd


def scene(n=40, D=49):
    pts = torch.zeros(n, 3)
    attrs = torch.zeros(n, D)
    adj = torch.zeros(8, dtype=torch.uint32)
    offs = torch.zeros(n + 1, dtype=torch.uint32)
    rays = torch.zeros(5, 6)
    start = torch.zeros(5, dtype=torch.uint32)
    return pts, attrs, adj, offs, rays, start


def test_create_pipeline():
    p = sdfoam_amd.create_pipeline(3)
    assert p.attribute_dim() == 49 and p.attribute_type() == torch.float32
    assert sdfoam_amd.create_pipeline(0, "torch.float32").attribute_dim() == 4
    assert sdfoam_amd.create_pipeline(1, "float16").attribute_type() == torch.float16
    with pytest.raises(RuntimeError, match="Unsupported SH degree"):
        sdfoam_amd.create_pipeline(4)
    with pytest.raises(RuntimeError, match="Unsupported attribute type"):
        sdfoam_amd.create_pipeline(0, "float64")
    with pytest.raises(RuntimeError, match="unsupported dtype 'int8'"):
        sdfoam_amd.create_pipeline(0, "int8")


def test_scene_checks_in_order():
    pipe = sdfoam_amd.create_pipeline(3)
    pts, attrs, adj, offs, rays, start = scene()
    with pytest.raises(RuntimeError, match=r"points had dimension 4 along axis -1, expected 3"):
        pipe.trace_forward(torch.zeros(40, 4), attrs, adj, offs, rays, start)
    with pytest.raises(RuntimeError, match=r"points had dtype Double, expected float32"):
        pipe.trace_forward(pts.double(), attrs, adj, offs, rays, start)
    with pytest.raises(RuntimeError, match=r"unsupported dtype 'Int'"):
        pipe.trace_forward(pts.int(), attrs, adj, offs, rays, start)
    with pytest.raises(RuntimeError, match="points must be on CUDA device"):
        pipe.trace_forward(pts, attrs, adj, offs, rays, start)


def test_backward_checks():
    pipe = sdfoam_amd.create_pipeline(3)
    pts, attrs, adj, offs, rays, start = scene()
    with pytest.raises(RuntimeError, match="points must be on CUDA device"):
        pipe.trace_backward(pts, attrs, adj, offs, rays, start, torch.zeros(5, 4), torch.zeros(5, 4))


def test_spatial_checks():
    with pytest.raises(RuntimeError, match="points must have 3 as the last dimension"):
        sdfoam_amd.build_aabb_tree(torch.zeros(40, 4))
    with pytest.raises(RuntimeError, match="points must have 2 dimensions"):
        sdfoam_amd.build_aabb_tree(torch.zeros(2, 40, 3))
    with pytest.raises(RuntimeError, match="points must be on CUDA device"):
        sdfoam_amd.build_aabb_tree(torch.zeros(40, 3))
    with pytest.raises(RuntimeError, match="points and queries must have the same dtype"):
        sdfoam_amd.nn(torch.zeros(40, 3), torch.zeros(64, 2, 3), torch.zeros(5, 3).double())
    with pytest.raises(RuntimeError, match="points and tree must have the same dtype"):
        sdfoam_amd.nn(torch.zeros(40, 3), torch.zeros(64, 2, 3).double(), torch.zeros(5, 3))
    with pytest.raises(RuntimeError, match="points must be on CUDA device"):
        sdfoam_amd.nn(torch.zeros(40, 3), torch.zeros(64, 2, 3), torch.zeros(5, 3))


def test_trace_rays_signature():
    """TraceRays.forward takes the reference's arguments in the reference's
    order (sdfoam_model/render.py:12-29)."""
    import inspect

    params = list(inspect.signature(sdfoam_amd.TraceRays.forward).parameters)
    assert params == ["ctx", "pipeline", "_points", "_attributes", "_point_adjacency",
                      "_point_adjacency_offsets", "rays", "start_point", "depth_quantiles",
                      "return_contribution", "use_sdfoam", "inv_s", "eps", "sdf_channel"]


def test_trace_plan_keeps_record_for_its_own_inputs():
    """The walk record holds the forward's colours, so a plan hands it to the
    backward only for the forward's tensors (same storage, unmodified) and
    the same alpha mode and sdf channel; otherwise the backward scans."""
    from sdfoam_amd import _lib
    from sdfoam_amd.pipeline import TracePlan

    pts, attrs, adj, offs, rays, start = scene()
    s = _lib.TraceSettings(0.01, 100, 1, 48, 0, 0)
    plan = TracePlan(5, s, "cpu")
    plan.allocate_record(4)
    plan.record_key = TracePlan.record_key(s, pts, attrs, adj, offs, rays, start)
    same = plan.desc(TracePlan.record_key(s, pts, attrs, adj, offs, rays, start))
    assert same.walk_record == plan.record_ptr and same.walk_budget == 4
    assert plan.record_ptr % 256 == 0 and same.walk_record_chunks == plan.chunks > 0
    assert same.walk_record_bytes == plan.nbytes > 0
    others = [TracePlan.record_key(s, pts, attrs.clone(), adj, offs, rays, start)]
    attrs.add_(0.0)  # same values, new version
    others.append(TracePlan.record_key(s, pts, attrs, adj, offs, rays, start))
    s2 = _lib.TraceSettings(0.01, 100, 1, 47, 0, 0)
    others.append(TracePlan.record_key(s2, pts, attrs, adj, offs, rays, start))
    for key in others:
        d = plan.desc(key)
        assert not d.walk_record and d.walk_record_bytes == 0 and d.walk_budget == 0


def test_sdfoam_import_name():
    """`import sdfoam` (the reference's module name, sdfoam_model/scene.py:8)
    gives this build's objects for every name the reference's scripts use."""
    import sdfoam

    for name in ("create_pipeline", "build_aabb_tree", "nn", "Triangulation",
                 "TriangulationFailedError", "farthest_neighbor", "BatchFetcher"):
        assert getattr(sdfoam, name) is getattr(sdfoam_amd, name), name
    with pytest.raises(RuntimeError, match="viewer"):
        sdfoam.run_with_viewer(None, None)


def test_record_walk_default_follows_autograd():
    """record_walk=None records only when a backward can follow: the
    attributes or inv_s require grad, or the points do with grad mode on
    (inside an autograd Function's forward grad mode is off, so there the
    points alone do not count: the reference's scene builds its attributes
    without grad under torch.no_grad())."""
    from sdfoam_amd.pipeline import _backward_can_follow

    pts = torch.nn.Parameter(torch.zeros(4, 3))
    att = torch.nn.Parameter(torch.zeros(4, 49))
    attributes = torch.cat([att[:, :48], att[:, 48:]], dim=-1)
    assert _backward_can_follow(pts, attributes, 1.0)
    with torch.no_grad():
        frozen = torch.cat([att[:, :48], att[:, 48:]], dim=-1)
        assert not _backward_can_follow(pts, frozen, torch.ones(4, 1))
    assert _backward_can_follow(pts, frozen, 1.0)  # grad mode on: the points count
    inv = torch.ones(4, 1, requires_grad=True)
    with torch.no_grad():
        assert _backward_can_follow(pts, frozen, inv)
    assert not _backward_can_follow(pts.detach(), frozen, 50.0)


def test_release_trace_plan_drops_the_record():
    """release_trace_plan removes the plan a forward attached to its rgba
    (a kept rgba then holds no walk record); a tensor without one is left as
    it is."""
    import torch

    import sdfoam_amd
    from sdfoam_amd import pipeline

    rgba = torch.zeros(4, 4)
    setattr(rgba, pipeline._PLAN_ATTR, object())
    sdfoam_amd.release_trace_plan(rgba)
    assert not hasattr(rgba, pipeline._PLAN_ATTR)
    sdfoam_amd.release_trace_plan(rgba)
    sdfoam_amd.release_trace_plan(torch.zeros(2))

