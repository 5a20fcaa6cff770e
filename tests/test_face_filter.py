"""The walk's face filter (walk_advance in sdfoam_amd/csrc/trace_device.h)
skips the division t = num / dp where bounds show the face cannot be taken.
The exit face must stay the one the exact rule picks: a scalar C statement
of the filter (tests/face_filter_host.c, gcc, IEEE division and fmaf) is run
on millions of random and boundary cases (num a few ulps from t1 dp or t0 dp,
subnormal products, t0 = 0, t1 infinite or negative; 0 < dp < 2^17, the range
of diff . d for fp16 diffs and a unit direction) and must never skip a face
the exact rule takes, nor misjudge "some t <= t0" of the standard-mode
scan."""

import ctypes as C
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_face_filter_never_skips_a_taken_face(tmp_path):
    so = tmp_path / "libvf.so"
    subprocess.run(["gcc", "-O2", "-shared", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
                    os.path.join(ROOT, "tests", "face_filter_host.c"), "-o", str(so), "-lm"],
                   check=True)
    L = C.CDLL(str(so))
    L.vf_check.restype = C.c_longlong
    L.vf_check.argtypes = [C.c_longlong, C.c_uint64]
    for seed in (1, 2, 3):
        assert L.vf_check(4_000_000, seed) == 0


def test_face_filter_check_catches_a_narrower_bound(tmp_path):
    """The check itself: with the bounds' 2^-21 widening dropped, boundary
    cases must show up as violations."""
    src = open(os.path.join(ROOT, "tests", "face_filter_host.c")).read()
    narrowed = src.replace("fmaf(fabsf(t1), 0x1p-21f, t1)", "t1").replace(
        "t0 * (1.0f - 0x1p-21f)", "t0")
    assert narrowed != src
    c = tmp_path / "vf_narrow.c"
    c.write_text(narrowed)
    so = tmp_path / "libvf_narrow.so"
    subprocess.run(["gcc", "-O2", "-shared", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
                    str(c), "-o", str(so), "-lm"], check=True)
    L = C.CDLL(str(so))
    L.vf_check.restype = C.c_longlong
    L.vf_check.argtypes = [C.c_longlong, C.c_uint64]
    assert L.vf_check(2_000_000, 1) > 0
