"""Writes tests/golden/c1.npz: the inputs of workload C1 (4104 points, Qhull
adjacency, 64x64 rays) and the scalar oracle's outputs on them, forward and
backward, in both alpha modes.

The reference ships no golden vectors and cannot run here (it needs nvcc
and an NVIDIA GPU), so these are not reference outputs: they freeze the
generated inputs (the Delaunay adjacency depends on the Qhull build) and the
oracle's results, as a regression pin for the oracle and a fixed-input case
for the GPU path.  The oracle itself is pinned by the closed-form,
invariant, brute-force and finite-difference tests.

Run from the repository root:  python tests/golden/gen_golden.py
"""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402
from sdfoam_amd import scenes  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c1.npz")


def main():
    oracle.build()
    arrays = {}
    base = scenes.make_config(1)
    start = scenes.start_points_for(base.points, base.rays)
    arrays.update(points=base.points, adjacency=base.adjacency, offsets=base.offsets,
                  rays=base.rays, start=start, quantiles=base.quantiles,
                  grad_rgba=base.grad_rgba, depth_grad=base.depth_grad,
                  inv_s=np.float32(base.inv_s))
    inv = float(np.float32(base.inv_s))
    for mode in ("sdfoam", "standard"):
        # same points, rays and upstream gradients; the last channel is the
        # SDF (sdfoam) or a softplus density (standard)
        w = scenes.make_config(1, mode=mode)
        arrays[f"{mode}_attributes"] = w.attributes
        f = oracle.trace_forward(0, base.points, w.attributes, base.adjacency, base.offsets,
                                 base.rays, start, base.quantiles, alpha_mode=mode, inv_s=inv)
        b = oracle.trace_backward(0, base.points, w.attributes, base.adjacency, base.offsets,
                                  base.rays, start, f.rgba, base.grad_rgba, base.quantiles,
                                  f.depth_indices, base.depth_grad, alpha_mode=mode, inv_s=inv)
        arrays.update({
            f"{mode}_rgba": f.rgba,
            f"{mode}_depth": f.depth,
            f"{mode}_depth_indices": f.depth_indices,
            f"{mode}_num_intersections": f.num_intersections,
            f"{mode}_visit_hash": f.visit_hash,
            f"{mode}_contribution": f.contribution.astype(np.float32),
            f"{mode}_points_grad": b.points_grad.astype(np.float32),
            f"{mode}_attr_grad": b.attr_grad.astype(np.float32),
            f"{mode}_sharpness_grad": np.float64(b.sharpness_grad),
            f"{mode}_backward_visit_hash": b.visit_hash,
        })
    np.savez_compressed(OUT, **arrays)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
