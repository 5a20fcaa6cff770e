"""The C ABI without a GPU: libsdfoam_hip.so loads, exports every symbol the
headers under include/ declare, and rejects bad arguments with its own
messages before any HIP call."""

import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    with open(os.path.join(ROOT, "include", "sdfoam_hip.h")) as f:
        text = f.read()
    for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(sdf_\w+)\s*\(", text, re.M):
        names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported():
    from sdfoam_amd import _lib

    names = declared_functions()
    assert len(names) >= 12
    assert names == set(_lib.EXPORTS)
    L = C.CDLL(_lib.LIB_PATH)
    for n in names:
        assert hasattr(L, n), n


def test_pure_queries():
    from sdfoam_amd import _lib

    L = _lib.lib()
    assert L.sdf_version().startswith(b"sdfoam_hip")
    assert [L.sdf_attribute_dim(d) for d in range(4)] == [4, 13, 28, 49]
    assert L.sdf_attribute_dim(4) == -1 and L.sdf_attribute_dim(-1) == -1
    assert L.sdf_trace_scratch_bytes(10, 100) == (100 + 32) * 8


def _settings(mode=1, ch=48, width=0):
    from sdfoam_amd._lib import TraceSettings

    return TraceSettings(1e-7, 1024, mode, ch, width)


def _fwd(L, degree=3, settings=None, num_points=10, scratch=True, scratch_bytes=None, rays=1,
         width=0):
    s = settings or _settings(width=width)
    buf = (C.c_uint64 * 64)()
    p = C.cast(buf, C.c_void_p)
    nb = L.sdf_trace_scratch_bytes(num_points, 4) if scratch_bytes is None else scratch_bytes
    return L.sdf_trace_forward(degree, C.byref(s), num_points, p, p, 4, p, p, rays, p, p, 0,
                               None, p, None, None, p, None, p, p, p if scratch else None, nb,
                               None)


def test_forward_argument_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    assert _fwd(L, degree=4) == 1
    assert L.sdf_last_error() == b"Unsupported SH degree"
    assert _fwd(L, settings=_settings(mode=7)) == 1
    assert b"alpha_mode" in L.sdf_last_error()
    assert _fwd(L, settings=_settings(ch=49)) == 1
    assert b"sdf_channel 49 out of range" in L.sdf_last_error()
    assert _fwd(L, num_points=0) == 1
    assert _fwd(L, scratch=False) == 1
    assert b"scratch must hold" in L.sdf_last_error()
    assert _fwd(L, scratch_bytes=8) == 1
    assert _fwd(L, rays=10, width=3) == 1
    assert b"ray_image_width 3 does not divide" in L.sdf_last_error()


def test_walk_record_sizes_and_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    # 8 counters (256 bytes apart), the chunk tables (one uint32 per 16 trips
    # and wavefront, rounded up to 256 bytes), then the pool: chunks of 16
    # rows of 64 entries of 24 bytes (the step and its colour), a multiple of
    # 8 chunks.  Wavefronts: 4 a block, blocks padded to a multiple of 8
    chunk = 16 * 64 * 24
    assert L.sdf_walk_record_bytes(256, 0, 10) == 2048 + 256 + 32 * chunk
    assert L.sdf_walk_record_full_chunks(256, 0, 10) == 32
    assert L.sdf_walk_record_full_chunks(256, 0, 40) == 96
    assert L.sdf_walk_record_bytes(8 * 256 + 1, 0, 3) == 2048 + 256 + 64 * chunk
    # 1600 x 1200 image: 100 x 75 tiles of 16 x 16, 7504 blocks
    assert L.sdf_walk_record_bytes(1600 * 1200, 1600, 1) == 2048 + 120064 + 30016 * chunk
    assert L.sdf_walk_record_pool_bytes(256, 0, 10, 5) == 2048 + 256 + 8 * chunk
    assert L.sdf_walk_record_pool_bytes(256, 0, 10, 0) == L.sdf_walk_record_bytes(256, 0, 10)
    assert L.sdf_walk_record_pool_bytes(256, 0, 0, 5) == 0
    s = _settings()
    buf = (C.c_uint64 * 64)()
    p = C.cast(buf, C.c_void_p)
    nb = L.sdf_trace_scratch_bytes(10, 4)
    base = C.cast(buf, C.c_void_p).value
    aligned = (base + 255) & ~255
    for addr, budget, nbytes, msg in ((aligned, 0, 1 << 20, b"budget must be positive"),
                                      (aligned, 2, 100, b"walk record must hold"),
                                      (aligned + 16, 2, 1 << 20,
                                       b"walk record must be 256-byte aligned")):
        rec = _lib.TracePlanDesc(addr, nbytes, budget, None)
        rc = L.sdf_trace_forward_planned(C.byref(rec), 3, C.byref(s), 10, p, p, 4, p, p, 1, p,
                                          p, 0, None, p, None, None, p, None, p, p, p, nb, None)
        assert rc == 1 and msg in L.sdf_last_error()
        rc = L.sdf_trace_backward_planned(C.byref(rec), 3, C.byref(s), 10, p, p, 4, p, p, 1, p,
                                           p, 0, None, None, p, p, None, None, p, p, None, p,
                                           None, p, nb, None)
        assert rc == 1 and msg in L.sdf_last_error()


def test_grad_accum_sizes_and_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    # one row per cell: D + 4 floats (attributes, position, point error)
    # rounded up to 8, 32, 32, 64 floats
    assert [L.sdf_grad_accum_bytes(d, 10) for d in range(4)] == [320, 1280, 1280, 2560]
    assert L.sdf_grad_accum_bytes(4, 10) == 0
    assert L.sdf_grad_accum_bytes(3, 1 << 20) == 256 << 20
    s = _settings()
    buf = (C.c_uint64 * 512)()
    p = C.cast(buf, C.c_void_p)
    nb = L.sdf_trace_scratch_bytes(10, 4)
    base = C.cast(buf, C.c_void_p).value
    misaligned = base + 8 if (base + 8) % 256 else base + 16
    for addr, nbytes, msg in ((base, 2559, b"gradient accumulator must hold 2560 bytes"),
                              (misaligned, 2560, b"must be 256-byte aligned")):
        plan = _lib.TracePlanDesc(None, 0, 0, None, addr, nbytes)
        rc = L.sdf_trace_backward_planned(C.byref(plan), 3, C.byref(s), 10, p, p, 4, p, p, 1, p,
                                          p, 0, None, None, p, p, None, None, p, p, None, p,
                                          None, p, nb, None)
        assert rc == 1 and msg in L.sdf_last_error()


def test_cell_table_sizes_and_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    # per cell: position, CSR begin and end (20 bytes), then the attribute
    # row (D = 4, 13, 28, 49 values), rounded up to a power of two >= 64
    assert [L.sdf_cell_table_bytes(d, 0, 10) for d in range(4)] == [640, 1280, 2560, 2560]
    assert [L.sdf_cell_table_bytes(d, 1, 10) for d in range(4)] == [640, 640, 1280, 1280]
    assert L.sdf_cell_table_bytes(4, 0, 10) == 0
    assert L.sdf_cell_table_bytes(3, 2, 10) == 0
    assert L.sdf_cell_table_bytes(3, 0, 1 << 20) == 256 << 20
    s = _settings()
    buf = (C.c_uint64 * 512)()
    p = C.cast(buf, C.c_void_p)
    nb = L.sdf_trace_scratch_bytes(10, 4)
    base = C.cast(buf, C.c_void_p).value
    aligned = (base + 255) & ~255
    for addr, nbytes, msg in ((aligned, 2559, b"cell table must hold 2560 bytes"),
                              (aligned + 16, 2560, b"cell table must be 256-byte aligned")):
        plan = _lib.TracePlanDesc()
        plan.cell_table, plan.cell_table_bytes = addr, nbytes
        rc = L.sdf_trace_forward_planned(C.byref(plan), 3, C.byref(s), 10, p, p, 4, p, p, 1, p,
                                         p, 0, None, p, None, None, p, None, p, p, p, nb, None)
        assert rc == 1 and msg in L.sdf_last_error()


def test_start_points_sizes_and_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    # a counter line, the hash table and its slot numbers (4 bytes per slot,
    # a power of two >= 2 rays and >= 64), 4 + 4 + 8 bytes per ray; every
    # part 256-byte aligned
    def up(x):
        return -(-x // 256) * 256

    for rays in (1, 100, 1000):
        slots = max(64, 1 << (2 * rays - 1).bit_length())
        want = 256 + 2 * up(4 * slots) + 2 * up(4 * rays) + up(8 * rays)
        assert L.sdf_start_points_scratch_bytes(rays) == want
    buf = (C.c_uint64 * 4096)()
    p = C.cast(buf, C.c_void_p)
    base = C.cast(buf, C.c_void_p).value
    aligned = (base + 255) & ~255
    need = L.sdf_start_points_scratch_bytes(10)
    assert L.sdf_start_points(p, 10, p, 31, p, p, aligned, need, None) == 1
    assert b"at least 32" in L.sdf_last_error()
    assert L.sdf_start_points(p, 10, p, 40, p, p, aligned, need - 1, None) == 1
    assert b"scratch must hold" in L.sdf_last_error()
    assert L.sdf_start_points(p, 10, p, 40, p, p, aligned + 8, need, None) == 1
    assert b"256-byte aligned" in L.sdf_last_error()
    # the tree has pow2(N) boxes in 32 bits: more than 2^31 points is refused
    # before any work, by the start lookup, nn and the tree build alike
    big = (1 << 31) + 1
    assert L.sdf_start_points(p, 10, p, big, p, p, aligned, need, None) == 1
    assert b"at most 2147483648 points" in L.sdf_last_error()
    assert L.sdf_nn(p, p, p, big, 10, p, None) == 1
    assert b"at most 2147483648 points" in L.sdf_last_error()
    assert L.sdf_build_aabb_tree(p, big, p, None) == 1
    assert b"at most 2147483648 points" in L.sdf_last_error()


def test_triangulation_table_argument_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    assert L.sdf_delaunay_adjacency_capacity(100, 500) == 4 * 100 + 2 * 500 + 64
    buf = (C.c_uint64 * 128)()
    p = C.cast(buf, C.c_void_p)
    base = C.cast(buf, C.c_void_p).value
    aligned = (base + 255) & ~255
    rc = L.sdf_delaunay_tables(p, 100, p, p, 500, p, p, p, p, p, 10, aligned, 1 << 20, None)
    assert rc == 1 and b"point_adjacency must hold 1464 entries" in L.sdf_last_error()
    rc = L.sdf_delaunay_tables(p, 100, p, p, 500, p, p, p, p, p, 1464, aligned + 8, 1 << 20, None)
    assert rc == 1 and b"256-byte aligned" in L.sdf_last_error()
    rc = L.sdf_delaunay_tables(None, 100, p, p, 500, p, p, p, p, p, 1464, aligned, 1 << 20, None)
    assert rc == 1 and b"NULL pointer" in L.sdf_last_error()
    assert L.sdf_sort_points(p, 0, None, None, 0, None) == 0
    assert L.sdf_sort_points(p, 10, None, p, 1 << 20, None) == 1
    assert b"NULL pointer" in L.sdf_last_error()


def test_gpu_delaunay_argument_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    buf = (C.c_uint64 * 128)()
    p = C.cast(buf, C.c_void_p)
    base = C.cast(buf, C.c_void_p).value
    aligned = (base + 255) & ~255
    counts = (C.c_uint64 * 5)()
    rc = L.sdf_delaunay_certify(p, 31, p, 10, p, counts, aligned, 1 << 20, None)
    assert rc == 1 and b"less than 32 points" in L.sdf_last_error()
    rc = L.sdf_delaunay_certify(p, (1 << 26) + 1, p, 10, p, counts, aligned, 1 << 20, None)
    assert rc == 1 and b"at most 2^26 points" in L.sdf_last_error()
    rc = L.sdf_delaunay_certify(p, 100, p, 10, None, counts, aligned, 1 << 20, None)
    assert rc == 1 and b"NULL pointer" in L.sdf_last_error()
    rc = L.sdf_delaunay_certify(p, 100, p, 10, p, counts, aligned + 8, 1 << 20, None)
    assert rc == 1 and b"256-byte aligned" in L.sdf_last_error()
    rc = L.sdf_delaunay_certify_exhaustive(p, 31, p, 10, p, counts, aligned, 1 << 20, None)
    assert rc == 1 and b"less than 32 points" in L.sdf_last_error()
    rc = L.sdf_delaunay_certify_exhaustive(p, (1 << 20) + 1, p, 10, p, counts, aligned, 1 << 20,
                                           None)
    assert rc == 1 and b"at most 2^20 points" in L.sdf_last_error()
    rc = L.sdf_delaunay_certify_exhaustive(p, 100, p, 10, None, counts, aligned, 1 << 20, None)
    assert rc == 1 and b"NULL pointer" in L.sdf_last_error()
    result = (C.c_uint64 * 4)()
    rc = L.sdf_delaunay_merge(p, 100, aligned, 1 << 20, None, 5, p, 1, p, p, 10, result,
                              aligned, 1 << 20, None)
    assert rc == 1 and b"NULL pointer" in L.sdf_last_error()
    rc = L.sdf_delaunay_merge(p, 100, aligned + 16, 1 << 20, p, 5, p, 1, p, p, 10, result,
                              aligned, 1 << 20, None)
    assert rc == 1 and b"256-byte aligned" in L.sdf_last_error()
    rc = L.sdf_delaunay_merge(p, 100, aligned, 1 << 20, p, 1 << 31, p, 1 << 31, p, p, 10,
                              result, aligned, 1 << 20, None)
    assert rc == 1 and b"too many reports" in L.sdf_last_error()
    rc = L.sdf_delaunay_merge(p, 100, aligned, 1 << 20, p, 5, p, (1 << 26) + 1, p, p, 10,
                              result, aligned, 1 << 20, None)
    assert rc == 1 and b"at most 2^26 points and candidates" in L.sdf_last_error()
    # the incremental rebuild's calls
    rc = L.sdf_delaunay_check(p, 100, p, p, 10, None, p, aligned, 1 << 20, None)
    assert rc == 1 and b"NULL pointer" in L.sdf_last_error()
    rc = L.sdf_delaunay_check(p, 100, p, p, 10, p, p, aligned + 64, 1 << 20, None)
    assert rc == 1 and b"256-byte aligned" in L.sdf_last_error()
    rc = L.sdf_delaunay_check(p, 31, p, p, 10, p, p, aligned, 1 << 20, None)
    assert rc == 1 and b"less than 32 points" in L.sdf_last_error()
    rc = L.sdf_delaunay_certify_points(p, 100, None, 5, p, 10, p, counts, aligned, 1 << 20, None)
    assert rc == 1 and b"NULL pointer" in L.sdf_last_error()
    rc = L.sdf_delaunay_certify_points(p, (1 << 26) + 1, p, 5, p, 10, p, counts, aligned,
                                       1 << 20, None)
    assert rc == 1 and b"at most 2^26 points" in L.sdf_last_error()
    rc = L.sdf_delaunay_merge_verified(p, 100, aligned, 1 << 20, p, 5, p, 1, None, 3, p, p, 10,
                                       result, aligned, 1 << 20, None)
    assert rc == 1 and b"NULL pointer" in L.sdf_last_error()
    rc = L.sdf_delaunay_merge_verified(p, 100, aligned, 1 << 20, p, 1 << 31, p, 1 << 30, p,
                                       1 << 30, p, p, 10, result, aligned, 1 << 20, None)
    assert rc == 1 and b"too many reports" in L.sdf_last_error()


def test_ray_order_and_plan_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    buf = (C.c_uint64 * 64)()
    p = C.cast(buf, C.c_void_p)
    # (the scratch size comes from rocPRIM's query for the current device, so
    # it is only known on a GPU host)
    assert L.sdf_ray_order(1000, 5000, p, p, None, p, 100, None) == 1
    assert b"NULL pointer" in L.sdf_last_error()
    assert L.sdf_ray_order(1000, 0, None, None, None, None, 0, None) == 0
    # a ray order with an image layout is rejected before any launch
    s = _settings(width=1)
    plan = _lib.TracePlanDesc(None, 0, 0, p)
    nb = L.sdf_trace_scratch_bytes(10, 4)
    rc = L.sdf_trace_forward_planned(C.byref(plan), 3, C.byref(s), 10, p, p, 4, p, p, 1, p, p, 0,
                                     None, p, None, None, p, None, p, p, p, nb, None)
    assert rc == 1 and b"ray order needs ray_image_width == 0" in L.sdf_last_error()


def test_trace_benchmark_argument_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    buf = (C.c_uint64 * 64)()
    p = C.cast(buf, C.c_void_p)
    s = _settings()
    cam = _lib.Camera()
    cam.fov, cam.width, cam.height, cam.model = 1.0, 8, 8, 0

    def call(diff_entries=4, camera=cam, start=p):
        return L.sdf_trace_benchmark(3, C.byref(s), 10, p, p, 4, p, p, p, diff_entries,
                                     C.byref(camera) if camera is not None else None, None,
                                     start, p, p, None)

    assert call(diff_entries=3) == 1 and b"adjacent_diff must hold" in L.sdf_last_error()
    assert call(camera=None) == 1 and b"camera must not be NULL" in L.sdf_last_error()
    bad = _lib.Camera()
    bad.fov, bad.width, bad.height, bad.model = 1.0, 8, 8, 7
    assert call(camera=bad) == 1 and L.sdf_last_error() == b"Invalid camera model"
    big = _lib.Camera()
    big.fov, big.width, big.height, big.model = 1.0, 1 << 16, 1 << 16, 0
    assert call(camera=big) == 1 and b"width * height" in L.sdf_last_error()
    assert call(start=None) == 1 and b"start_point" in L.sdf_last_error()


def test_batch_gather_argument_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    buf = (C.c_uint64 * 16)()
    p = C.cast(buf, C.c_void_p)
    assert L.sdf_batch_gather(p, 10, 24, 0, 0, 1, p, None) == 0  # empty batch
    assert L.sdf_batch_gather(None, 10, 24, 0, 4, 1, p, None) == 1
    assert b"NULL pointer" in L.sdf_last_error()
    assert L.sdf_batch_gather(p, 0, 24, 0, 4, 1, p, None) == 1
    assert b"num_rows" in L.sdf_last_error()
    assert L.sdf_batch_gather(p, 10, 6, 0, 4, 1, p, None) == 1
    assert b"multiple of 4" in L.sdf_last_error()
    base = C.cast(buf, C.c_void_p).value
    assert L.sdf_batch_gather(base + 2, 10, 24, 0, 4, 1, p, None) == 1
    assert b"4-byte aligned" in L.sdf_last_error()


def test_nn_and_tree_argument_errors():
    from sdfoam_amd import _lib

    L = _lib.lib()
    buf = (C.c_uint64 * 8)()
    p = C.cast(buf, C.c_void_p)
    assert L.sdf_nn(p, p, p, 31, 1, p, None) == 1
    assert L.sdf_last_error() == b"number of points must be at least 32"
    assert L.sdf_build_aabb_tree(None, 10, p, None) == 1
    assert L.sdf_debug_fpmath(5, p, p, 1, None) == 1


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from sdfoam_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(_lib.LibraryError, match="not built"):
        _lib.lib()
