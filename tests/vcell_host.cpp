// Host build of the GPU Delaunay's cell clipping (sdfoam_amd/csrc/voronoi_cell.h)
// for the CPU tests: the same code the kernel runs, driven one cell at a time.
#include <cmath>
#include <cstdint>

#include "../sdfoam_amd/csrc/voronoi_cell.h"

using namespace sdfoam_hip::vcell;

extern "C" {

// Cell of point `center` clipped by `cand` (indices, nearest first) until the
// next candidate is beyond twice the farthest vertex.  Box [lo, hi]
// (absolute).  Writes the status and, for each cell vertex, the three
// neighbour indices (-1 for a box face); returns the vertex count.
int vc_cell(const float *points, int center, const int32_t *cand, int num_cand,
            const double *lo, const double *hi, uint32_t *status, int32_t *verts_out,
            int max_out) {
    static Cell cell; // large: keep it off the stack
    double o[3] = {points[3 * center], points[3 * center + 1], points[3 * center + 2]};
    double rlo[3], rhi[3];
    for (int k = 0; k < 3; ++k) {
        rlo[k] = lo[k] - o[k];
        rhi[k] = hi[k] - o[k];
    }
    cell_init(cell, rlo, rhi);
    double reach2 = INFINITY;
    for (int i = 0; i < num_cand; ++i) {
        const int c = cand[i];
        double q[3];
        for (int k = 0; k < 3; ++k) q[k] = (double)points[3 * c + k] - o[k];
        const double d2 = q[0] * q[0] + q[1] * q[1] + q[2] * q[2];
        if (d2 > 4.0 * max_r2(cell) * (1.0 + 1e-9)) {
            reach2 = d2;
            break;
        }
        if (!clip(cell, q, c)) break;
    }
    *status = settle(cell, reach2);
    const int n = cell.num_verts < max_out ? cell.num_verts : max_out;
    for (int i = 0; i < n; ++i)
        for (int k = 0; k < 3; ++k) verts_out[3 * i + k] = cell.planes[cell.verts[i].p[k]].point;
    return cell.num_verts;
}

// Pairing check of the dual triangles of a fresh box: number of directed
// edges whose reverse is missing (0 for a consistently oriented cell).
int vc_box_unpaired(void) {
    static Cell cell;
    const double lo[3] = {-1, -2, -3}, hi[3] = {4, 5, 6};
    cell_init(cell, lo, hi);
    int bad = 0;
    for (int i = 0; i < cell.num_verts; ++i)
        for (int k = 0; k < 3; ++k) {
            const int a = cell.verts[i].p[k], b = cell.verts[i].p[(k + 1) % 3];
            int found = 0;
            for (int j = 0; j < cell.num_verts; ++j)
                for (int m = 0; m < 3; ++m)
                    if (cell.verts[j].p[m] == b && cell.verts[j].p[(m + 1) % 3] == a) ++found;
            bad += found == 1 ? 0 : 1;
        }
    return bad;
}

int vc_insphere(const double *a, const double *b, const double *c, const double *q) {
    return in_sphere(a, b, c, q);
}
}
