"""The reference's calling pattern on this build, against the oracle.

``SDFoamScene.forward`` (sdfoam_model/scene.py:252-265, 272-324) builds its
trace data on every call and hands it to ``TraceRays``
(sdfoam_model/render.py:10-189):

* attributes = ``torch.cat([torch.cat([att_dc, att_sh], -1), last], -1)``
  cast to the attribute dtype, last = the SDF (sdfoam) or the softplus
  density (standard);
* inv_s = ``exp(variance)`` as ``[1, 1]``, clipped to [1e-6, 1e6], expanded
  to ``(N, 1)`` and made contiguous (an N-float copy; the tracer reads
  element 0); ``ones([1, 1])`` in standard mode;
* start points from ``torch.unique`` over the ray origins and ``sdfoam.nn``;
* ``TraceRays.apply(pipeline, points, attributes, adjacency, offsets, rays,
  start, quantiles, True, use_sdfoam, inv_s, 1e-6, D - 1 or -1)``.

Here that pattern runs through the ``sdfoam`` import name, and the leaf
gradients autograd delivers (positions, dc, SH, last channel, variance) are
compared with the oracle backward under the bars of test_gpu_parity,
including a batch whose upstream gradient holds a NaN ray (the non-finite
gradients it causes are zeroed, as the reference's TraceRays does)."""

import numpy as np
import pytest

from conftest import scene
from test_gpu_parity import U, assert_close_model, gamma, sum_depth, to_dev, u32, _threads

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _flat(w):
    R = w.num_rays
    return (w.rays.reshape(R, 6), w.quantiles.reshape(R, -1), w.grad_rgba.reshape(R, 4),
            w.depth_grad.reshape(R, -1))


def _scene_step(w, dev, mode, nan_ray=None):
    """One SDFoamScene.forward + backward on leaves built from the workload;
    returns the leaves (with .grad) and what the oracle needs."""
    import torch

    import sdfoam

    rays_np, q_np, g_np, dg_np = _flat(w)
    N = w.num_points
    D = w.attributes.shape[-1]
    C = D - 1
    pts = to_dev(w.points, dev).requires_grad_(True)
    att_dc = to_dev(w.attributes[:, :3], dev).requires_grad_(True)
    att_sh = to_dev(w.attributes[:, 3:C], dev).requires_grad_(True)
    use_sdfoam = mode == "sdfoam"
    if use_sdfoam:
        last = to_dev(w.attributes[:, C:], dev).requires_grad_(True)
        variance = torch.tensor(float(np.log(w.inv_s)), device=dev, requires_grad=True)
        inv_s = (torch.ones([1, 1], device=dev) * torch.exp(variance))[:, :1].clip(1e-6, 1e6)
        inv_s = inv_s.expand(N, 1).to(dtype=torch.float32).contiguous()
    else:
        # the reference's density channel: softplus(beta = 10) of a logit; the
        # workload's last channel is that density, so invert it for the leaf
        dens = w.attributes[:, C:].astype(np.float64)
        logit = np.log(np.expm1(np.maximum(dens, 1e-30) * 10.0)) / 10.0
        last = to_dev(logit.astype(np.float32), dev).requires_grad_(True)
        variance = None
        inv_s = torch.ones([1, 1], device=dev, dtype=torch.float32).contiguous()
    adj, offs = u32(w.adjacency, dev), u32(w.offsets, dev)
    tree = sdfoam.build_aabb_tree(pts.detach())
    pipe = sdfoam.create_pipeline(w.sh_degree, "float32")
    rays = to_dev(rays_np, dev)
    q = to_dev(q_np, dev)

    last_chan = last if use_sdfoam else torch.nn.functional.softplus(last, beta=10)
    attributes = torch.cat([torch.cat([att_dc, att_sh], dim=-1), last_chan], dim=-1)
    attributes = attributes.to(torch.float32).contiguous()
    with torch.no_grad():
        origins = rays[..., :3]
        uniq, inverse = torch.unique(origins, dim=0, return_inverse=True)
        start = sdfoam.nn(pts.detach(), tree, uniq).long()[inverse].type(torch.uint32)
    rgba, depth, contrib, nis, errbox, alpha = sdfoam.TraceRays.apply(
        pipe, pts, attributes, adj, offs, rays, start, q, True, use_sdfoam, inv_s, 1e-6,
        int(D - 1) if use_sdfoam else -1)
    plan = getattr(rgba, "_sdfoam_trace_plan", None)
    assert plan is not None and plan.entries is not None, "a training forward records its walk"
    g = to_dev(g_np, dev)
    if nan_ray is not None:
        g[nan_ray] = float("nan")
    loss = (rgba * g).sum() + (depth * to_dev(dg_np, dev)).sum()
    loss.backward()
    assert not hasattr(rgba, "_sdfoam_trace_plan"), "the backward consumes the plan"
    start_np = start.view(torch.int32).cpu().numpy().view(np.uint32)
    return dict(pts=pts, att_dc=att_dc, att_sh=att_sh, last=last, variance=variance,
                rgba=rgba.detach().cpu().numpy(), didx=depth_idx(pipe, w, dev, attributes, pts,
                                                              adj, offs, rays, start, q, inv_s,
                                                              mode),
                start=start_np, g=g.cpu().numpy(), attributes=attributes.detach().cpu().numpy())


def depth_idx(pipe, w, dev, attributes, pts, adj, offs, rays, start, q, inv_s, mode):
    """The forward's quantile point indices (the oracle's density backward
    reads them)."""
    import torch

    with torch.no_grad():
        out = pipe.trace_forward(pts.detach(), attributes.detach(), adj, offs, rays, start,
                                 depth_quantiles=q, alpha_mode=mode, inv_s=inv_s.detach())
        return out["depth_indices"].view(torch.int32).cpu().numpy().view(np.uint32)


def _check(w, st, mode, oracle_lib):
    rays_np, q_np, _, dg_np = _flat(w)
    inv = w.inv_s if mode == "sdfoam" else 1.0
    ref = oracle_lib.trace_backward(
        w.sh_degree, w.points, st["attributes"], w.adjacency, w.offsets, rays_np, st["start"],
        st["rgba"], st["g"], q_np, st["didx"], dg_np, alpha_mode=mode, inv_s=inv,
        threads=_threads())

    def fin(a, b):
        return np.where(np.isfinite(a), a, 0.0), np.where(np.isfinite(a), b, 0.0)

    pg, pga = fin(ref.points_grad, ref.points_grad_abs)
    assert_close_model("points.grad", st["pts"].grad.cpu().numpy(), pg, pga, ref.points_grad_k)
    ag, aga = fin(ref.attr_grad, ref.attr_grad_abs)
    C = ag.shape[1] - 1
    k = ref.attr_grad_k
    assert_close_model("att_dc.grad", st["att_dc"].grad.cpu().numpy(), ag[:, :3], aga[:, :3],
                       k[:, :3])
    assert_close_model("att_sh.grad", st["att_sh"].grad.cpu().numpy(), ag[:, 3:C], aga[:, 3:C],
                       k[:, 3:C])
    got_last = st["last"].grad.cpu().numpy().reshape(-1)
    if mode == "sdfoam":
        assert_close_model("sdf.grad", got_last, ag[:, C], aga[:, C], k[:, C])
        # variance -> exp -> clip -> expand(N, 1): only element 0 of the
        # tracer's sharpness gradient is nonzero
        sg = ref.sharpness_grad if np.isfinite(ref.sharpness_grad) else 0.0
        sa = ref.sharpness_abs if np.isfinite(ref.sharpness_grad) else 0.0
        expect = sg * w.inv_s
        got = float(st["variance"].grad.cpu())
        tol = 1e-5 + 1e-4 * abs(expect) + gamma(min(ref.sharpness_k, sum_depth(w, ref))) * sa * w.inv_s + 4 * U * abs(expect)
        assert abs(got - expect) <= tol, (got, expect, tol)
    else:
        # softplus_beta10'(x) = sigmoid(10 x): the tracer's density gradient times it
        x = w.attributes[:, C].astype(np.float64)
        logit = np.log(np.expm1(np.maximum(x, 1e-30) * 10.0)) / 10.0
        dsp = 1.0 / (1.0 + np.exp(-10.0 * logit))
        assert_close_model("density logit.grad", got_last, ag[:, C] * dsp, aga[:, C] * dsp,
                           k[:, C])
    return ref


@pytest.mark.parametrize("cfg,mode", [(1, "sdfoam"), (1, "standard"), (2, "sdfoam")])
def test_scene_forward_contract(torch_dev, oracle_lib, cfg, mode):
    w = scene(cfg, mode=mode)
    st = _scene_step(w, torch_dev, mode)
    ref = _check(w, st, mode, oracle_lib)
    assert np.isfinite(ref.attr_grad).all()


def test_scene_forward_nonfinite_zeroing(torch_dev, oracle_lib):
    """A NaN upstream gradient on one ray: every gradient element that ray
    touches is non-finite in the oracle and zero in what autograd delivers;
    every other element still matches."""
    w = scene(1)
    st = _scene_step(w, torch_dev, "sdfoam", nan_ray=w.num_rays // 2 + 32)
    ref = _check(w, st, "sdfoam", oracle_lib)
    bad = ~np.isfinite(ref.attr_grad)
    assert bad.any() and not bad.all()
    C = ref.attr_grad.shape[1] - 1
    assert np.all(st["att_dc"].grad.cpu().numpy()[bad[:, :3]] == 0.0)
    assert np.all(st["last"].grad.cpu().numpy().reshape(-1)[bad[:, C]] == 0.0)
    badp = ~np.isfinite(ref.points_grad)
    assert badp.any() and np.all(st["pts"].grad.cpu().numpy()[badp] == 0.0)


def test_eval_render_records_nothing(torch_dev):
    """Under torch.no_grad() the scene's attributes and inv_s do not require
    grad: the forward keeps no walk record (nor any plan for a backward)."""
    import torch

    import sdfoam

    w = scene(2)
    rays_np, q_np, _, _ = _flat(w)
    pts = torch.nn.Parameter(to_dev(w.points, torch_dev))
    att = torch.nn.Parameter(to_dev(w.attributes, torch_dev))
    adj, offs = u32(w.adjacency, torch_dev), u32(w.offsets, torch_dev)
    pipe = sdfoam.create_pipeline(w.sh_degree)
    rays = to_dev(rays_np, torch_dev)
    start = u32(w.extra["start"].reshape(-1), torch_dev)
    with torch.no_grad():
        attributes = torch.cat([att[:, :-1], att[:, -1:]], dim=-1).contiguous()
        inv_s = torch.full((w.num_points, 1), w.inv_s, device=torch_dev)
        out = sdfoam.TraceRays.apply(pipe, pts, attributes, adj, offs, rays, start, None, True,
                                     True, inv_s, 1e-6, w.attributes.shape[-1] - 1)
        plan = getattr(out[0], "_sdfoam_trace_plan", None)
        assert plan is None or plan.entries is None
