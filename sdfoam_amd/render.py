"""``TraceRays``: the autograd Function around the tracer.

Same forward/backward contract as the reference's ``TraceRays``
(sdfoam_model/render.py:10-189): forward returns
``(rgba, depth, contribution, num_intersections, ErrorBox, alpha)``; backward
calls ``trace_backward`` with the saved forward outputs, zeroes non-finite
gradients and returns gradients for ``points``, ``attributes`` and, in
sdfoam mode, ``inv_s``.  The calls to the pipeline are the reference's: the
forward's trace plan (ray order, walk record, offset table) reaches the
backward on the saved ``rgba`` tensor, as it does when the reference's own
``TraceRays`` drives this build's pipeline.  The walk is recorded only when
a backward can follow (the attributes or ``inv_s`` require grad), so an
evaluation render under ``torch.no_grad()`` records nothing.
"""

from __future__ import annotations

import torch


class ErrorBox:
    """Carrier for per-ray error in and per-point error out
    (sdfoam_model/render.py:4-7)."""

    def __init__(self):
        self.ray_error = None
        self.point_error = None


class TraceRays(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pipeline, _points, _attributes, _point_adjacency, _point_adjacency_offsets,
                rays, start_point, depth_quantiles, return_contribution, use_sdfoam=False,
                inv_s=50.0, eps=1e-6, sdf_channel=None):
        ctx.rays = rays
        ctx.start_point = start_point
        ctx.pipeline = pipeline
        ctx.points = _points
        ctx.attributes = _attributes
        ctx.point_adjacency = _point_adjacency
        ctx.point_adjacency_offsets = _point_adjacency_offsets
        ctx.depth_quantiles = depth_quantiles
        ctx.use_sdfoam = bool(use_sdfoam)
        ctx.inv_s = inv_s
        ctx.eps = float(eps)
        ctx.sdf_channel = (
            int(sdf_channel) if sdf_channel is not None
            else (_attributes.shape[-1] - 1 if use_sdfoam else -1)
        )
        results = pipeline.trace_forward(
            _points, _attributes, _point_adjacency, _point_adjacency_offsets, rays, start_point,
            depth_quantiles=depth_quantiles,
            return_contribution=return_contribution,
            alpha_mode="sdfoam" if ctx.use_sdfoam else "standard",
            inv_s=ctx.inv_s,
            eps=ctx.eps,
            sdf_channel=ctx.sdf_channel,
        )
        ctx.rgba = results["rgba"]
        ctx.depth_indices = results.get("depth_indices", None)
        errbox = ErrorBox()
        ctx.errbox = errbox
        return (
            results["rgba"],
            results.get("depth", None),
            results.get("contribution", None),
            results["num_intersections"],
            errbox,
            results["alpha"],
        )

    @staticmethod
    def backward(ctx, grad_rgba, grad_depth, grad_contribution, grad_num_intersections,
                 errbox_grad, grad_alpha):
        del grad_contribution, grad_num_intersections, errbox_grad, grad_alpha
        results = ctx.pipeline.trace_backward(
            ctx.points, ctx.attributes, ctx.point_adjacency, ctx.point_adjacency_offsets,
            ctx.rays, ctx.start_point, ctx.rgba, grad_rgba,
            ctx.depth_quantiles, ctx.depth_indices, grad_depth, ctx.errbox.ray_error,
            alpha_mode="sdfoam" if ctx.use_sdfoam else "standard",
            inv_s=ctx.inv_s,
            eps=ctx.eps,
            sdf_channel=ctx.sdf_channel,
        )
        points_grad = results["points_grad"].contiguous()
        attr_grad = results["attr_grad"].contiguous()
        sharpness_grad = results["sharpness_grad"].contiguous()
        if sharpness_grad is not None and isinstance(ctx.inv_s, torch.Tensor):
            sharpness_grad = sharpness_grad.to(ctx.inv_s.dtype).view_as(ctx.inv_s)
        ctx.errbox.point_error = results.get("point_error", None)
        points_grad[~points_grad.isfinite()] = 0
        attr_grad[~attr_grad.isfinite()] = 0
        if sharpness_grad is not None:
            sharpness_grad[~sharpness_grad.isfinite()] = 0
        del (ctx.rays, ctx.start_point, ctx.pipeline, ctx.rgba, ctx.points, ctx.attributes,
             ctx.point_adjacency, ctx.point_adjacency_offsets, ctx.depth_quantiles)
        return (
            None,
            points_grad,
            attr_grad,
            None,
            None,
            None,
            None,
            None,
            None,
            None,
            sharpness_grad if ctx.use_sdfoam else None,
            None,
            None,
        )
