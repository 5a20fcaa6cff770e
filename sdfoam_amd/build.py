"""Build recipe for libsdfoam_hip.so (gfx950) with hipcc.

``python -m sdfoam_amd.build`` compiles the HIP sources under csrc/ into
``sdfoam_amd/libsdfoam_hip.so`` in-tree (no JIT cache), so the built library
travels with the source tree.

Floating-point flags are part of the library's numerical contract:
* ``-ffp-contract=off``: no implicit fused multiply-adds, only explicit fmaf;
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: IEEE fp32 division and sqrt;
* packed fp32 ops disabled (no v_pk_fma_f32 / v_pk_mul_f32 / v_pk_add_f32).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libsdfoam_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = os.environ.get("SDFOAM_OFFLOAD_ARCH", "gfx950")

SOURCES = ["trace_kernels.hip", "aabb_kernels.hip", "order_kernels.hip", "delaunay_tables.hip",
           "delaunay_gpu.hip", "batch_fetcher.hip", "triangulation_kernels.hip", "capi.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build libsdfoam_hip.so)")
    return path


def build(verbose: bool = False, jobs: int = 4) -> str:
    """Compile every HIP source and link the shared library; returns its path."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src in SOURCES:
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if len(procs) >= jobs:
            _wait(procs.pop(0))
    while procs:
        _wait(procs.pop(0))
    tmp = LIB_PATH + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if out.returncode != 0:
        raise RuntimeError("link failed:\n" + out.stdout.decode(errors="replace"))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def _wait(item):
    src, p = item
    out, _ = p.communicate()
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n" + out.decode(errors="replace"))
    text = out.decode(errors="replace").strip()
    # hipcc's host pass reports the device-only target feature; nothing else is expected
    lines = [l for l in text.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if lines:
        print(f"[{src}]\n" + "\n".join(lines), file=sys.stderr)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
