"""The ``Pipeline`` operator surface of the reference's ``sdfoam`` module.

``create_pipeline`` / ``Pipeline.trace_forward`` / ``Pipeline.trace_backward``
take the same arguments, apply the same checks with the same messages, and
return the same dicts of tensors as the reference's pybind11 bindings
(torch_bindings/pipeline_bindings.cpp:12-75, 124-607, 744-837).  The work is
done by libsdfoam_hip.so through its C ABI, on torch's current stream.

Deliberate differences, all on paths where the reference's behaviour is
undefined or wasteful:
* no ``.item()`` host sync for ``inv_s`` (the kernels read the tensor);
* ``ray_grad`` is returned zeroed instead of uninitialised;
* an ``sdf_channel`` beyond the attribute row raises instead of reading out
  of bounds; start points or neighbours out of range end the walk;
* ``inv_s`` may also be a Python number.
"""

from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib
from ._lib import TraceSettings, check, ptr

# torch dtype -> c10::toString name, as printed in the reference's messages
_C10_NAMES = {
    torch.float32: "Float",
    torch.float64: "Double",
    torch.float16: "Half",
    torch.bfloat16: "BFloat16",
    torch.int64: "Long",
    torch.int32: "Int",
    torch.int16: "Short",
    torch.int8: "Char",
    torch.uint8: "Byte",
    torch.bool: "Bool",
}
for _name in ("uint16", "uint32", "uint64"):
    if hasattr(torch, _name):
        _C10_NAMES[getattr(torch, _name)] = _name.replace("uint", "UInt")

_SCALAR_NAMES = {torch.float32: "float32", torch.float64: "float64", torch.float16: "float16"}


def _c10(dtype) -> str:
    return _C10_NAMES.get(dtype, str(dtype).replace("torch.", ""))


def _scalar_type(dtype) -> str:
    """dtype_to_scalar_type (torch_bindings/bindings.h:44-54)."""
    if dtype in _SCALAR_NAMES:
        return _SCALAR_NAMES[dtype]
    raise RuntimeError(f"unsupported dtype '{_c10(dtype)}'")


def _is_cuda(t: torch.Tensor) -> bool:
    return t.device.type == "cuda"


def _dtype_string_to_scalar_type(dtype: str) -> str:
    """torch_bindings/pipeline_bindings.cpp:734-745."""
    if dtype in ("float32", "torch.float32"):
        return "float32"
    if dtype in ("float64", "torch.float64"):
        return "float64"
    if dtype in ("float16", "torch.float16"):
        return "float16"
    raise RuntimeError(f"unsupported dtype '{dtype}'")


def _parse_alpha_mode(alpha_mode) -> int:
    """torch_bindings/pipeline_bindings.cpp:221-229."""
    if alpha_mode is None:
        return _lib.SDF_ALPHA_STANDARD
    mode = str(alpha_mode).lower()
    if mode in ("sdfoam", "sdf", "alpha_neus"):
        return _lib.SDF_ALPHA_NEUS
    return _lib.SDF_ALPHA_STANDARD


def _inv_s_to_tensor(inv_s, like: torch.Tensor) -> torch.Tensor:
    """torch_bindings/pipeline_bindings.cpp:124-136."""
    if inv_s is None:
        return torch.ones(1, dtype=torch.float32, device=like.device)
    if not isinstance(inv_s, torch.Tensor):
        return torch.tensor([float(inv_s)], dtype=torch.float32, device=like.device)
    s = inv_s.contiguous()
    if s.device != like.device or s.dtype != torch.float32:
        s = s.to(like.device, torch.float32).contiguous()
    return s


# a wavefront's first pool of walk-record chunks, when no earlier forward
# over rays of this count and layout tells what the walk needs: this many
# trips per wavefront on average
RECORD_INITIAL_TRIPS = 256
# pools after that: per XCD, the chunks the last such forward asked for
# there, plus an eighth and one
RECORD_MARGIN = 1.125
RECORD_COUNTERS = 8  # uint32 at 256-byte strides at the start of a record
# rays in no particular order are traced in sorted order from this many on
AUTO_SORT_MIN_RAYS = 32768


class TracePlan:
    """What a forward hands its backward (no counterpart in the reference;
    sdf_trace_plan in the C ABI):

    * ``order``: the launch order of the rays (sdf_ray_order), for rays in no
      particular order;
    * ``entries``: the walk record, each ray's steps and their colours and
      sdf/density values (24 bytes per step, up to ``budget`` trips per
      wavefront of 64 rays), in a pool of ``chunks`` chunks of 16 trips that
      the wavefronts claim as they walk (``record_ptr``: its 256-byte
      aligned start in ``entries``);
    * ``table``: the forward's fp16 offset table of the scene, which the
      backward reuses instead of rebuilding it while the points, adjacency
      and offsets tensors are the same and unmodified (same storage and
      version counter).

    Valid for a backward over the same rays, start points, scene, attributes
    and settings; the tracer checks the ray count, image width and walk
    limit, and uses the walk record only when the backward's rays, start
    points, scene and attribute tensors are the forward's (same storage,
    unmodified) with the same alpha mode and sdf channel."""

    def __init__(self, num_rays: int, settings, device):
        self.num_rays = num_rays
        self.ray_image_width = int(settings.ray_image_width)
        self.max_intersections = int(settings.max_intersections)
        self.device = torch.device(device)
        self.order = None
        self.entries = None
        self.record_ptr = 0
        self.nbytes = 0
        self.budget = 0
        self.chunks = 0
        self.table = None
        self.table_bytes = 0
        self.table_key = None
        self.record_key = None

    @staticmethod
    def scene_key(points, adjacency, offsets) -> tuple:
        return tuple((t.data_ptr(), t._version, t.numel()) for t in (points, adjacency, offsets))

    @staticmethod
    def record_key(settings, *tensors) -> tuple:
        """What the walk record depends on: the traced tensors (storage,
        version counter, size) and the alpha mode and sdf channel (the record
        holds each step's colour and sdf/density value)."""
        return (int(settings.alpha_mode), int(settings.sdf_channel)) + tuple(
            (t.data_ptr(), t._version, t.numel()) for t in tensors)

    def keep_table(self, table: torch.Tensor, nbytes: int, key: tuple) -> None:
        self.table, self.table_bytes, self.table_key = table, nbytes, key

    def table_for(self, key: tuple):
        """The kept offset table if it belongs to this scene, else None."""
        return self.table if self.table is not None and key == self.table_key else None

    def sort_rays(self, num_points: int, rays: torch.Tensor, start: torch.Tensor) -> None:
        L = _lib.lib()
        nbytes = int(L.sdf_ray_order_scratch_bytes(num_points, self.num_rays))
        if nbytes == 0:
            raise RuntimeError("sdf_ray_order_scratch_bytes failed")
        # 256-byte alignment for the sort's scratch
        scratch = torch.empty(nbytes + 256, dtype=torch.uint8, device=self.device)
        base = scratch.data_ptr()
        aligned = (base + 255) & ~255
        self.order = torch.empty(self.num_rays, dtype=torch.int32, device=self.device)
        with torch.cuda.device(self.device):
            check(L.sdf_ray_order(num_points, self.num_rays, ptr(rays), ptr(start),
                                  ptr(self.order), aligned, nbytes,
                                  _lib.stream_handle(self.device)))
        # `scratch` may be freed now: torch reuses it only for later work on
        # this stream, which runs after the sort

    def allocate_record(self, budget, chunks: int = 0) -> None:
        """A record for up to ``budget`` trips per wavefront (default: every
        trip the walk limit allows, max_intersections + 1, plus the
        terminating row) in a pool of ``chunks`` chunks (0: the pool of
        RECORD_INITIAL_TRIPS trips per wavefront, or every trip if that is
        less)."""
        if budget is None:
            budget = self.max_intersections + 2
        budget = int(budget)
        if budget <= 0:
            raise RuntimeError("walk_budget must be positive")
        L = _lib.lib()
        full = int(L.sdf_walk_record_full_chunks(self.num_rays, self.ray_image_width, budget))
        if chunks <= 0:
            chunks = int(L.sdf_walk_record_full_chunks(self.num_rays, self.ray_image_width,
                                                       min(budget, RECORD_INITIAL_TRIPS)))
        chunks = max(1, min(int(chunks), full))
        self.nbytes = int(L.sdf_walk_record_pool_bytes(self.num_rays, self.ray_image_width,
                                                       budget, chunks))
        self.entries = torch.empty(self.nbytes + 256, dtype=torch.uint8, device=self.device)
        self.record_ptr = (self.entries.data_ptr() + 255) & ~255
        self.budget = budget
        self.chunks = chunks

    def record_counters(self) -> torch.Tensor:
        """The record's chunk counters (int32 [8], on the device): their sum
        is the number of chunks the last forward asked for."""
        off = self.record_ptr - self.entries.data_ptr()
        return self.entries[off:off + 256 * RECORD_COUNTERS].view(torch.int32)[::64]

    def desc(self, record_key=None):
        """The C descriptor; the walk record is left out when `record_key`
        (the backward's inputs) is not the one it was recorded for, so the
        backward scans for itself."""
        use_record = self.entries is not None and (record_key is None
                                                   or record_key == self.record_key)
        d = _lib.TracePlanDesc(
            self.record_ptr if use_record else None, self.nbytes if use_record else 0,
            self.budget if use_record else 0,
            None if self.order is None else self.order.data_ptr())
        d.walk_record_chunks = self.chunks if use_record else 0
        return d

    def matches(self, num_rays: int, settings, device) -> bool:
        return (num_rays == self.num_rays
                and int(settings.ray_image_width) == self.ray_image_width
                and int(settings.max_intersections) == self.max_intersections
                and self.device == torch.device(device))

    def check_matches(self, num_rays: int, settings, device) -> None:
        if not self.matches(num_rays, settings, device):
            raise RuntimeError("trace_plan does not belong to these rays and settings")


class _RecordNeed:
    """What the walk records of one ray count and layout needed: the chunk
    counters of the last forward, copied to pinned host memory behind the
    forward and read once that copy has completed (no synchronisation)."""

    def __init__(self):
        self.host = torch.zeros(RECORD_COUNTERS, dtype=torch.int32).pin_memory()
        self.event = None
        self.per_xcd = 0  # the most chunks one XCD asked for

    def observe(self, plan: "TracePlan") -> None:
        self.host.copy_(plan.record_counters(), non_blocking=True)
        self.event = torch.cuda.Event()
        self.event.record()

    def estimate(self) -> int:
        """Chunks for the next pool (0: no forward has told yet).  Each XCD
        claims from its own eighth of the pool, so the eighths are sized for
        the XCD that asked for most."""
        if self.event is not None and self.event.query():
            self.per_xcd = int(self.host.max())
            self.event = None
        if self.per_xcd <= 0:
            return 0
        return (int(math.ceil(self.per_xcd * RECORD_MARGIN)) + 1) * RECORD_COUNTERS


def _backward_can_follow(points, attributes, inv_s) -> bool:
    """Whether autograd can ask for this trace's backward: some traced input
    requires grad.  Under ``torch.no_grad()`` the reference's scene builds its
    attribute rows and sharpness without grad (sdfoam_model/scene.py:259-265,
    252-254), so evaluation renders fall outside this even though the points
    are parameters."""
    return bool(attributes.requires_grad
                or (isinstance(inv_s, torch.Tensor) and inv_s.requires_grad)
                or (points.requires_grad and torch.is_grad_enabled()))


# attribute of a forward's rgba tensor that carries its trace plan to the
# backward over it (the reference's TraceRays hands the backward that tensor)
_PLAN_ATTR = "_sdfoam_trace_plan"


def release_trace_plan(rgba: torch.Tensor) -> None:
    """Drop the trace plan (walk record, ray order, offset table) that a
    forward attached to its ``rgba``, for an ``rgba`` kept without a backward
    over it (no counterpart in the reference).  A later backward over that
    ``rgba`` scans for itself, with the same results."""
    if hasattr(rgba, _PLAN_ATTR):
        delattr(rgba, _PLAN_ATTR)


def _auto_sort(sort_rays, settings, num_rays: int) -> bool:
    if sort_rays is None:
        return int(settings.ray_image_width) == 0 and num_rays >= AUTO_SORT_MIN_RAYS
    if sort_rays and int(settings.ray_image_width) != 0:
        raise RuntimeError("sort_rays needs rays in no image layout (shape [R, 6])")
    return bool(sort_rays)


class Pipeline:
    """A tracing pipeline for one SH degree and attribute dtype
    (src/tracing/pipeline.h:79-161)."""

    def __init__(self, sh_degree: int, attr_dtype: torch.dtype):
        self._sh_degree = int(sh_degree)
        self._attr_dtype = attr_dtype
        # (rays, image width, budget, device) -> _RecordNeed
        self._record_need = {}

    # -- src/tracing/pipeline.h:158-160 -------------------------------------
    def attribute_dim(self) -> int:
        return 1 + 3 * (self._sh_degree + 1) ** 2

    def attribute_type(self) -> torch.dtype:
        return self._attr_dtype

    @property
    def sh_degree(self) -> int:
        return self._sh_degree

    # -- validation (torch_bindings/pipeline_bindings.cpp:12-75) -------------
    def _validate_scene_data(self, points, attributes, point_adjacency, point_adjacency_offsets):
        if points.size(-1) != 3:
            raise RuntimeError(f"points had dimension {points.size(-1)} along axis -1, expected 3")
        if _scalar_type(points.dtype) != "float32":
            raise RuntimeError(f"points had dtype {_c10(points.dtype)}, expected float32")
        if not _is_cuda(points):
            raise RuntimeError("points must be on CUDA device")
        num_points = points.numel() // 3
        D = self.attribute_dim()
        if attributes.size(-1) != D:
            raise RuntimeError(
                f"attributes had dimension {attributes.size(-1)} along axis -1, expected {D}")
        if attributes.numel() // D != num_points:
            raise RuntimeError("attributes must have the same number of rows as points")
        if attributes.dtype != self._attr_dtype:
            _scalar_type(attributes.dtype)
            raise RuntimeError(
                f"attributes had dtype {_c10(attributes.dtype)}, expected "
                f"{_SCALAR_NAMES[self._attr_dtype]}")
        if not _is_cuda(attributes):
            raise RuntimeError("attributes must be on CUDA device")
        if point_adjacency_offsets.dtype != torch.uint32:
            raise RuntimeError("point_adjacency_offsets must have uint32 dtype")
        if not _is_cuda(point_adjacency_offsets):
            raise RuntimeError("point_adjacency_offsets must be on CUDA device")
        if point_adjacency_offsets.numel() != num_points + 1:
            raise RuntimeError("point_adjacency_offsets must have num_points + 1 elements")
        if point_adjacency.dtype != torch.uint32:
            raise RuntimeError("point_adjacency must have uint32 dtype")
        if not _is_cuda(point_adjacency):
            raise RuntimeError("point_adjacency must be on CUDA device")

    def _validate_rays(self, rays, start_point, num_rays):
        if rays.size(-1) != 6:
            raise RuntimeError("rays must have 6 as the last dimension")
        if rays.dtype != torch.float32:
            raise RuntimeError("rays must have float32 dtype")
        if not _is_cuda(rays):
            raise RuntimeError("rays must be on CUDA device")
        if start_point.numel() != num_rays:
            raise RuntimeError("start_point must have the same batch size as rays")
        if start_point.dtype != torch.uint32:
            raise RuntimeError("start_point must have uint32 dtype")
        if not _is_cuda(start_point):
            raise RuntimeError("start_point must be on CUDA device")

    def _settings(self, weight_threshold, max_intersections, alpha_mode, sdf_channel, rays=None):
        """default_trace_settings + kwargs (src/tracing/pipeline.h:29-40;
        torch_bindings/pipeline_bindings.cpp:212-242), plus the image-width
        layout hint for rays shaped [..., H, W, 6]."""
        mode = _parse_alpha_mode(alpha_mode)
        if sdf_channel is not None:
            ch = int(sdf_channel)
        elif mode == _lib.SDF_ALPHA_NEUS:
            ch = self.attribute_dim() - 1
        else:
            ch = -1
        width = int(rays.shape[-2]) if rays is not None and rays.dim() >= 3 else 0
        return TraceSettings(
            1e-7 if weight_threshold is None else float(weight_threshold),
            1024 if max_intersections is None else int(max_intersections),
            mode,
            ch,
            width,
            _lib.SDF_ATTR_F16 if self._attr_dtype == torch.float16 else _lib.SDF_ATTR_F32,
        )

    def _zeros_attr(self, shape, device) -> torch.Tensor:
        """Zeroed buffer of the attribute type for atomic accumulation: fp16
        atomics are packed 4-byte words, so an odd element count gets one
        padding half (the result is a view of the first elements)."""
        n = 1
        for d in shape:
            n *= int(d)
        if self._attr_dtype == torch.float16 and n % 2 == 1:
            return torch.zeros(n + 1, dtype=self._attr_dtype, device=device)[:n].view(shape)
        return torch.zeros(shape, dtype=self._attr_dtype, device=device)

    @staticmethod
    def _scratch(num_points: int, num_adj: int, device) -> tuple[torch.Tensor, int]:
        nbytes = int(_lib.lib().sdf_trace_scratch_bytes(num_points, num_adj))
        buf = torch.empty((nbytes + 7) // 8, dtype=torch.int64, device=device)
        return buf, nbytes

    # -- trace_forward (torch_bindings/pipeline_bindings.cpp:138-334) -------
    def trace_forward(self, points, attributes, point_adjacency, point_adjacency_offsets, rays,
                      start_point, depth_quantiles=None, weight_threshold=None,
                      max_intersections=None, return_contribution=False, alpha_mode=None,
                      inv_s=None, eps=None, sdf_channel=None, record_walk=None,
                      walk_budget=None, sort_rays=None, cell_table=True):
        """Reference arguments and outputs, plus (no counterpart in the
        reference):

        * ``record_walk=True`` records the rays' steps so that the backward
          skips its face scans (standard mode: the steps where the density
          backward's unsafe walk takes the same exit, which is all of them
          but for degenerate ties); ``walk_budget`` bounds the recorded trips
          per wavefront (default: all the walk limit allows).  The record's
          storage is sized by need: the first forward over rays of this
          count and layout gets room for 256 trips per wavefront on
          average, later ones what the last one asked for plus an eighth;
          trips the pool has no room for are scanned again by the backward.
          ``None`` (the default) records when a backward can
          follow: the attributes or ``inv_s`` require grad (or the points do
          with grad mode on), which is how the reference's scene calls it in
          training and not under ``torch.no_grad()``;
        * ``sort_rays``: trace rays of shape [R, 6] in sorted order
          (sdf_ray_order); None sorts from 32768 rays on.  Outputs stay in
          the caller's order;
        * ``cell_table``: copy each cell's position, CSR row bounds and
          attribute row into one aligned record before walking (a temporary
          of 64-256 bytes per point, sdf_cell_table_bytes); False walks over
          the caller's arrays.  Results are the same.

        When either applies, the result holds ``"trace_plan"``, which
        ``trace_backward(trace_plan=...)`` over the same rays and settings
        takes.  The plan also rides on the returned ``rgba`` tensor, so a
        ``trace_backward`` handed that tensor as ``rgb_out`` (as the
        reference's ``TraceRays`` does) uses it without being given it."""
        points_c = points.contiguous()
        attributes_c = attributes.contiguous()
        adj_c = point_adjacency.contiguous()
        offs_c = point_adjacency_offsets.contiguous()
        rays_c = rays.contiguous()
        start_c = start_point.contiguous()
        sharpness = _inv_s_to_tensor(inv_s, rays_c)

        self._validate_scene_data(points, attributes, point_adjacency, point_adjacency_offsets)
        return_depth = depth_quantiles is not None
        num_points = points_c.size(0)
        num_adj = adj_c.size(0)
        num_rays = rays_c.numel() // 6
        self._validate_rays(rays_c, start_c, num_rays)
        num_q = 0
        dq = None
        if return_depth:
            dq = depth_quantiles.contiguous()
            num_q = dq.size(-1)
            if dq.dtype != torch.float32:
                raise RuntimeError("depth_quantiles must have float32 dtype")
            if not _is_cuda(dq):
                raise RuntimeError("depth_quantiles must be on CUDA device")
            if num_q == 0 or dq.numel() // num_q != num_rays:
                raise RuntimeError("depth_quantiles must have the same batch size as rays")
        settings = self._settings(weight_threshold, max_intersections, alpha_mode, sdf_channel, rays_c)

        dev = rays_c.device
        lead = tuple(rays_c.shape[:-1])
        rgba = torch.empty(lead + (4,), dtype=self._attr_dtype, device=dev)
        nisect = torch.empty(lead + (1,), dtype=torch.uint32, device=dev)
        contribution = self._zeros_attr((num_points, 1), dev) if return_contribution else None
        depth = didx = None
        if return_depth:
            depth = torch.zeros(lead + (num_q,), dtype=torch.float32, device=dev)
            didx = torch.zeros(lead + (num_q,), dtype=torch.uint32, device=dev)
        alpha = torch.zeros((num_points, 1), dtype=torch.float32, device=dev)
        scratch, nbytes = self._scratch(num_points, num_adj, dev)
        plan = None
        if record_walk is None:
            want_record = num_rays > 0 and _backward_can_follow(points, attributes, inv_s)
        else:
            want_record = bool(record_walk)
        want_sort = num_rays > 0 and _auto_sort(sort_rays, settings, num_rays)
        if want_record or want_sort:
            plan = TracePlan(num_rays, settings, dev)
            if want_sort:
                plan.sort_rays(num_points, rays_c, start_c)
            need = None
            if want_record:
                budget = plan.max_intersections + 2 if walk_budget is None else int(walk_budget)
                need = self._record_need.setdefault(
                    (num_rays, plan.ray_image_width, budget, str(dev)), _RecordNeed())
                plan.allocate_record(budget, need.estimate())
                plan.record_key = TracePlan.record_key(settings, points, attributes,
                                                       point_adjacency, point_adjacency_offsets,
                                                       rays, start_point)
            # keyed on the caller's tensors: a contiguous copy made above is
            # freed after this call and its storage may be handed out again
            plan.keep_table(scratch, nbytes,
                            TracePlan.scene_key(points, point_adjacency, point_adjacency_offsets))
        args = (
            self._sh_degree, C.byref(settings), num_points, ptr(points_c), ptr(attributes_c),
            num_adj, ptr(adj_c), ptr(offs_c), num_rays, ptr(rays_c), ptr(start_c), num_q,
            ptr(dq), ptr(rgba), ptr(depth), ptr(didx), ptr(nisect), ptr(contribution),
            ptr(sharpness), ptr(alpha), ptr(scratch), nbytes, _lib.stream_handle(dev))
        desc = plan.desc() if plan is not None else None
        cells = None
        if cell_table and num_rays > 0:
            cbytes = int(_lib.lib().sdf_cell_table_bytes(self._sh_degree, settings.attr_type,
                                                         num_points))
            cells = torch.empty(cbytes + 256, dtype=torch.uint8, device=dev)
            if desc is None:
                desc = _lib.TracePlanDesc()
            desc.cell_table = (cells.data_ptr() + 255) & ~255
            desc.cell_table_bytes = cbytes
        with torch.cuda.device(dev):
            if desc is None:
                check(_lib.lib().sdf_trace_forward(*args))
            else:
                check(_lib.lib().sdf_trace_forward_planned(C.byref(desc), *args))
        # `cells` may be freed now: torch reuses it only for later work on
        # this stream, which runs after the forward
        del cells
        if plan is not None and plan.entries is not None:
            with torch.cuda.device(dev):
                need.observe(plan)
        out = {"rgba": rgba}
        if return_depth:
            out["depth"] = depth
            out["depth_indices"] = didx
        if return_contribution:
            out["contribution"] = contribution
        out["num_intersections"] = nisect
        out["alpha"] = alpha
        if plan is not None:
            out["trace_plan"] = plan
            setattr(rgba, _PLAN_ATTR, plan)
        return out

    # -- trace_backward (torch_bindings/pipeline_bindings.cpp:336-607) ------
    def trace_backward(self, points, attributes, point_adjacency, point_adjacency_offsets, rays,
                       start_point, rgb_out, grad_in, depth_quantiles=None, depth_indices=None,
                       depth_grad_in=None, ray_error=None, weight_threshold=None,
                       max_intersections=None, alpha_mode=None, inv_s=None, eps=None,
                       sdf_channel=None, trace_plan=None, sort_rays=None, grad_accum=True):
        """Reference arguments and outputs, plus ``trace_plan`` (the
        forward's "trace_plan": its ray order and walk record; by default the
        plan the forward attached to ``rgb_out``, which this call detaches),
        ``sort_rays`` (as in trace_forward, when no plan is given) and
        ``grad_accum``: accumulate each cell's gradients in one aligned fp32
        row of a temporary buffer (256 bytes per cell at SH degree 3) before
        adding them to the outputs (fp16 outputs: rounded once); False
        updates the outputs directly."""
        points_c = points.contiguous()
        attributes_c = attributes.contiguous()
        adj_c = point_adjacency.contiguous()
        offs_c = point_adjacency_offsets.contiguous()
        rays_c = rays.contiguous()
        start_c = start_point.contiguous()
        sharpness = _inv_s_to_tensor(inv_s, rays_c)

        self._validate_scene_data(points, attributes, point_adjacency, point_adjacency_offsets)
        return_depth = depth_quantiles is not None
        return_error = ray_error is not None
        num_points = points_c.size(0)
        num_adj = adj_c.size(0)
        num_rays = rays_c.numel() // 6
        self._validate_rays(rays_c, start_c, num_rays)

        g = grad_in.contiguous()
        if g.size(-1) != 4:
            raise RuntimeError("rgb_grad_in must have 4 as the last dimension")
        if g.dtype != self._attr_dtype:
            _scalar_type(g.dtype)
            raise RuntimeError(
                f"rgb_grad_in had dtype {_c10(g.dtype)}, expected {_SCALAR_NAMES[self._attr_dtype]}")
        if not _is_cuda(g):
            raise RuntimeError("rgb_grad_in must be on CUDA device")
        if g.numel() // 4 != num_rays:
            raise RuntimeError("rgb_grad_in must have the same batch size as rays")

        num_q = 0
        dq = didx = dgrad = None
        if return_depth:
            dq = depth_quantiles.contiguous()
            num_q = dq.size(-1)
            if dq.dtype != torch.float32:
                raise RuntimeError("depth_quantiles must have float32 dtype")
            if not _is_cuda(dq):
                raise RuntimeError("depth_quantiles must be on CUDA device")
            if dq.numel() != num_rays * num_q:
                raise RuntimeError("depth_quantiles must have the same batch size as rays")
            if depth_grad_in is None:
                raise RuntimeError("depth_grad must be provided if depth_quantiles is provided")
            if depth_indices is None:
                raise RuntimeError("bad optional access")
            didx = depth_indices.contiguous()
            if didx.dtype != torch.uint32:
                raise RuntimeError("depth_indices must have uint32 dtype")
            if not _is_cuda(didx):
                raise RuntimeError("depth_indices must be on CUDA device")
            if didx.numel() != num_rays * num_q:
                raise RuntimeError("depth_indices must have the same batch size as rays")
            dgrad = depth_grad_in.contiguous()
            if dgrad.size(-1) != num_q:
                raise RuntimeError(
                    "depth_grad must have the same number of depth quantiles as depth_quantiles")
            if dgrad.dtype != torch.float32:
                _scalar_type(dgrad.dtype)
                raise RuntimeError(f"depth_grad had dtype {_c10(dgrad.dtype)}, expected float32")
            if not _is_cuda(dgrad):
                raise RuntimeError("depth_grad must be on CUDA device")
            if dgrad.numel() != num_rays * num_q:
                raise RuntimeError("depth_grad must have the same batch size as rays")

        rerr = None
        point_error = None
        dev = rays_c.device
        if return_error:
            rerr = ray_error.contiguous()
            if rerr.dtype != self._attr_dtype:
                _scalar_type(rerr.dtype)
                raise RuntimeError(
                    f"ray_error had dtype {_c10(rerr.dtype)}, expected {_SCALAR_NAMES[self._attr_dtype]}")
            if not _is_cuda(rerr):
                raise RuntimeError("ray_error must be on CUDA device")
            if rerr.numel() != num_rays:
                raise RuntimeError("ray_error must have the same batch size as rays")
            point_error = self._zeros_attr((num_points, 1), dev)

        settings = self._settings(weight_threshold, max_intersections, alpha_mode, sdf_channel, rays_c)
        rgba = rgb_out.contiguous()
        if rgba.dtype != self._attr_dtype or rgba.numel() != 4 * num_rays or not _is_cuda(rgba):
            raise RuntimeError("rgb_out must be the forward's rgba output")

        num_attr = attributes_c.size(0)
        attr_grad = self._zeros_attr((num_attr, self.attribute_dim()), dev)
        points_grad = torch.zeros((num_points, 3), dtype=rays_c.dtype, device=dev)
        ray_grad = torch.zeros_like(rays_c)
        sharpness_grad = torch.zeros_like(sharpness, dtype=torch.float32)
        table_ready = False
        # the plan of the forward that produced rgb_out, used by one backward
        # (detached here, so the record does not outlive it with the tensor)
        carried = getattr(rgb_out, _PLAN_ATTR, None)
        if carried is not None:
            delattr(rgb_out, _PLAN_ATTR)
            if trace_plan is None and carried.matches(num_rays, settings, dev):
                trace_plan = carried
        if trace_plan is not None:
            trace_plan.check_matches(num_rays, settings, dev)
            kept = trace_plan.table_for(
                TracePlan.scene_key(points, point_adjacency, point_adjacency_offsets))
            if kept is not None:
                scratch, nbytes, table_ready = kept, trace_plan.table_bytes, True
        if not table_ready:
            scratch, nbytes = self._scratch(num_points, num_adj, dev)
        if trace_plan is None and num_rays > 0 and _auto_sort(sort_rays, settings, num_rays):
            trace_plan = TracePlan(num_rays, settings, dev)
            trace_plan.sort_rays(num_points, rays_c, start_c)
        args = (
            self._sh_degree, C.byref(settings), num_points, ptr(points_c), ptr(attributes_c),
            num_adj, ptr(adj_c), ptr(offs_c), num_rays, ptr(rays_c), ptr(start_c), num_q,
            ptr(dq), ptr(didx), ptr(rgba), ptr(g), ptr(dgrad), ptr(rerr), ptr(points_grad),
            ptr(attr_grad), ptr(point_error), ptr(sharpness), ptr(sharpness_grad),
            ptr(scratch), nbytes, _lib.stream_handle(dev))
        desc = _lib.TracePlanDesc()
        if trace_plan is not None:
            desc = trace_plan.desc(TracePlan.record_key(settings, points, attributes,
                                                        point_adjacency, point_adjacency_offsets,
                                                        rays, start_point))
        desc.scratch_ready = 1 if table_ready else 0
        accum = None
        if grad_accum and num_rays > 0:
            accum_bytes = int(_lib.lib().sdf_grad_accum_bytes(self._sh_degree, num_points))
            accum = torch.empty(accum_bytes + 256, dtype=torch.uint8, device=dev)
            desc.grad_accum = (accum.data_ptr() + 255) & ~255
            desc.grad_accum_bytes = accum_bytes
        with torch.cuda.device(dev):
            if trace_plan is None and accum is None:
                check(_lib.lib().sdf_trace_backward(*args))
            else:
                check(_lib.lib().sdf_trace_backward_planned(C.byref(desc), *args))
        # `accum` may be freed now: torch reuses it only for later work on
        # this stream
        out = {
            "points_grad": points_grad,
            "attr_grad": attr_grad,
            "ray_grad": ray_grad,
            "sharpness_grad": sharpness_grad,
        }
        if return_error:
            out["point_error"] = point_error
        return out

    # -- trace_benchmark (torch_bindings/pipeline_bindings.cpp:609-732) -------
    def trace_benchmark(self, points, attributes, point_adjacency, point_adjacency_offsets,
                        adjacent_diff, camera, start_point, output_rgba, weight_threshold=None,
                        max_intersections=None, alpha_mode=None, inv_s=None, eps=None,
                        sdf_channel=None, *, bg_color=None, checker_bg=False):
        """Render one camera into ``output_rgba`` (uint32 RGBA8, ``height x
        width`` elements, row ``height - 1 - j`` holds pixel row j).

        ``camera`` is the reference's dict: ``position``, ``forward``,
        ``right``, ``up`` (3 floats each), ``fov`` (vertical, radians),
        ``width``, ``height``, ``model`` ("pinhole" | "fisheye").
        ``adjacent_diff`` is the fp16 offset table ``[E, 4]`` (as
        ``prefetch_adjacent_diff`` returns it, or ``(x_adj - x_self)`` cast to
        half with a zero 4th column).  ``start_point`` is one uint32 cell.
        ``bg_color`` / ``checker_bg`` (no counterpart in the reference's
        binding, which always uses the white default) set the background."""
        points_c = points.contiguous()
        attributes_c = attributes.contiguous()
        adj_c = point_adjacency.contiguous()
        offs_c = point_adjacency_offsets.contiguous()
        diff_c = adjacent_diff.contiguous()
        sharpness = _inv_s_to_tensor(inv_s, output_rgba)
        self._validate_scene_data(points, attributes, point_adjacency, point_adjacency_offsets)
        num_points = points_c.size(0)
        num_adj = adj_c.size(0)

        cam = _lib.Camera()
        for key in ("position", "forward", "up", "right"):
            v = torch.as_tensor(camera[key]).detach().to("cpu", torch.float32).reshape(-1)
            if v.numel() < 3:
                raise RuntimeError(f"camera {key} must have 3 elements")
            getattr(cam, key)[:] = [float(x) for x in v[:3]]
        cam.fov = float(camera["fov"])
        cam.width = int(camera["width"])
        cam.height = int(camera["height"])
        model = str(camera["model"])
        if model == "pinhole":
            cam.model = _lib.SDF_CAMERA_PINHOLE
        elif model == "fisheye":
            cam.model = _lib.SDF_CAMERA_FISHEYE
        else:
            raise RuntimeError("Invalid camera model")

        if start_point.numel() != 1:
            raise RuntimeError("start_point must have a single element")
        if start_point.dtype != torch.uint32:
            raise RuntimeError("start_point must have uint32 dtype")
        if not _is_cuda(start_point):
            raise RuntimeError("start_point must be on CUDA device")
        if output_rgba.numel() != cam.width * cam.height:
            raise RuntimeError("output_rgba must have width * height elements")
        if output_rgba.dtype != torch.uint32:
            raise RuntimeError("output_rgba must have uint32 dtype")
        if not _is_cuda(output_rgba):
            raise RuntimeError("output_rgba must be on CUDA device")
        if not output_rgba.is_contiguous():
            raise RuntimeError("output_rgba must be contiguous")
        if diff_c.element_size() != 2 or diff_c.numel() < 4 * num_adj or not _is_cuda(diff_c):
            raise RuntimeError("adjacent_diff must be a CUDA tensor of 4 halves per adjacency entry")

        settings = self._settings(weight_threshold, max_intersections, alpha_mode, sdf_channel)
        vis = _lib.Visualization()
        bg = [1.0, 1.0, 1.0] if bg_color is None else [float(x) for x in bg_color]
        vis.bg_color[:] = bg
        vis.checker_bg = 1 if checker_bg else 0
        dev = output_rgba.device
        with torch.cuda.device(dev):
            check(_lib.lib().sdf_trace_benchmark(
                self._sh_degree, C.byref(settings), num_points, ptr(points_c),
                ptr(attributes_c), num_adj, ptr(adj_c), ptr(offs_c), ptr(diff_c),
                diff_c.numel() // 4, C.byref(cam), C.byref(vis), ptr(start_point),
                ptr(output_rgba), ptr(sharpness), _lib.stream_handle(dev)))

    # -- walk statistics (measurement / parity hook) -------------------------
    def walk_stats(self, points, attributes, point_adjacency, point_adjacency_offsets, rays,
                   start_point, *, backward=False, alpha_mode=None, inv_s=None,
                   weight_threshold=None, max_intersections=None, sdf_channel=None,
                   record_cells: int = 0):
        """Per-ray visit hash, step count, faces scanned and faces of stepped
        cells of the forward (or backward) walk, plus the first
        ``record_cells`` visited cells of each ray."""
        points_c = points.contiguous()
        attributes_c = attributes.contiguous()
        adj_c = point_adjacency.contiguous()
        offs_c = point_adjacency_offsets.contiguous()
        rays_c = rays.contiguous()
        start_c = start_point.contiguous()
        self._validate_scene_data(points, attributes, point_adjacency, point_adjacency_offsets)
        num_rays = rays_c.numel() // 6
        self._validate_rays(rays_c, start_c, num_rays)
        sharpness = _inv_s_to_tensor(inv_s, rays_c)
        settings = self._settings(weight_threshold, max_intersections, alpha_mode, sdf_channel, rays_c)
        dev = rays_c.device
        n = points_c.size(0)
        num_adj = adj_c.size(0)
        vh = torch.zeros(num_rays, dtype=torch.int64, device=dev)
        steps = torch.zeros(num_rays, dtype=torch.int32, device=dev)
        faces = torch.zeros(num_rays, dtype=torch.int64, device=dev)
        faces_st = torch.zeros(num_rays, dtype=torch.int64, device=dev)
        cells = (torch.full((num_rays, record_cells), -1, dtype=torch.int32, device=dev)
                 if record_cells else None)
        scratch, nbytes = self._scratch(n, num_adj, dev)
        with torch.cuda.device(dev):
            check(_lib.lib().sdf_trace_walk_stats(
                self._sh_degree, C.byref(settings), 1 if backward else 0, n, ptr(points_c),
                ptr(attributes_c), num_adj, ptr(adj_c), ptr(offs_c), num_rays, ptr(rays_c),
                ptr(start_c), ptr(sharpness), ptr(vh), ptr(steps), ptr(faces), ptr(faces_st),
                ptr(cells), record_cells, ptr(scratch), nbytes, _lib.stream_handle(dev)))
        return {"visit_hash": vh, "steps": steps, "faces": faces, "faces_stepped": faces_st,
                "cells": cells}


_registry: list[Pipeline] = []


def create_pipeline(sh_degree: int, attr_dtype: str = "float32") -> Pipeline:
    """torch_bindings/pipeline_bindings.cpp:747-751 and src/tracing/pipeline.cu:1476-1506.
    Pipelines are kept in a process-wide registry, as the reference does."""
    st = _dtype_string_to_scalar_type(str(attr_dtype))
    if st == "float64":
        raise RuntimeError("Unsupported attribute type")
    if int(sh_degree) not in (0, 1, 2, 3):
        raise RuntimeError("Unsupported SH degree")
    p = Pipeline(int(sh_degree), torch.float32 if st == "float32" else torch.float16)
    _registry.append(p)
    return p


def prefetch_adjacent_diff(points, point_adjacency, point_adjacency_offsets) -> torch.Tensor:
    """fp16 neighbour offsets [E + 32, 4] (src/tracing/pipeline.cu:1202-1242)."""
    points_c = points.contiguous()
    adj_c = point_adjacency.contiguous()
    offs_c = point_adjacency_offsets.contiguous()
    n = points_c.size(0)
    e = adj_c.size(0)
    out = torch.empty((e + 32, 4), dtype=torch.float16, device=points_c.device)
    with torch.cuda.device(points_c.device):
        check(_lib.lib().sdf_prefetch_adjacent_diff(
            ptr(points_c), n, e, ptr(adj_c), ptr(offs_c), ptr(out),
            _lib.stream_handle(points_c.device)))
    return out
