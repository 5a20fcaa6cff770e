// Host build of the GPU Delaunay's per-item code (sdfoam_amd/csrc/voronoi_cell.h,
// sdfoam_amd/csrc/delaunay_grid.h) for the CPU tests: the same code the
// kernels run, driven one cell or one candidate at a time.
#include <cmath>
#include <algorithm>
#include <cstdint>
#include <utility>
#include <vector>

#include "../sdfoam_amd/csrc/delaunay_grid.h"

using namespace sdfoam_hip::vcell;
namespace dgrid = sdfoam_hip::dgrid;

namespace {
// the grids of the last vc_grid call
dgrid::GridGeom g_geom;
std::vector<dgrid::CellEntry> g_table[dgrid::kLevels];
std::vector<uint32_t> g_sorted[dgrid::kLevels];
std::vector<float> g_spts; // coordinates in the sorted order, 4 floats a point

dgrid::GridView view() {
    dgrid::GridView v{};
    v.g = g_geom;
    for (int l = 0; l < dgrid::kLevels; ++l) {
        v.table[l] = g_table[l].data();
        v.sorted[l] = g_sorted[l].data();
    }
    v.spts = g_spts.data();
    return v;
}
} // namespace

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

// The device's grids over n points (bounding box of the floats; the points
// stably sorted once by the Morton code of their finest cell, and per level
// the hash table of occupied cells over that order, filled by the same
// probing); returns the number of occupied cells of level 0 (dims: its
// dimensions), 0 if the box is degenerate.
int vc_grid(const float *points, uint32_t n, uint32_t *dims) {
    double lo[3] = {INFINITY, INFINITY, INFINITY}, hi[3] = {-INFINITY, -INFINITY, -INFINITY};
    for (uint32_t i = 0; i < n; ++i)
        for (int k = 0; k < 3; ++k) {
            lo[k] = std::fmin(lo[k], (double)points[3 * i + k]);
            hi[k] = std::fmax(hi[k], (double)points[3 * i + k]);
        }
    if (!dgrid::grid_geometry(lo, hi, n, g_geom)) return 0;
    const uint64_t slots = g_geom.table_mask + 1;
    const dgrid::GridLevel &l0 = g_geom.level[0];
    std::vector<std::pair<uint64_t, uint32_t>> keyed(n);
    for (uint32_t i = 0; i < n; ++i)
        keyed[i] = {dgrid::morton_key(
                        (uint32_t)dgrid::axis_cell(points[3 * i], g_geom.lo[0], l0.inv_h, l0.dims[0]),
                        (uint32_t)dgrid::axis_cell(points[3 * i + 1], g_geom.lo[1], l0.inv_h, l0.dims[1]),
                        (uint32_t)dgrid::axis_cell(points[3 * i + 2], g_geom.lo[2], l0.inv_h, l0.dims[2])),
                    i};
    std::stable_sort(keyed.begin(), keyed.end(),
                     [](const auto &a, const auto &b) { return a.first < b.first; });
    g_spts.assign(4ull * n, 0.0f);
    for (uint32_t t = 0; t < n; ++t)
        for (int k = 0; k < 3; ++k) g_spts[4ull * t + k] = points[3ull * keyed[t].second + k];
    int occupied0 = 0;
    std::vector<uint64_t> key(n);
    for (int l = 0; l < dgrid::kLevels; ++l) {
        g_sorted[l].resize(n);
        for (uint32_t t = 0; t < n; ++t) {
            g_sorted[l][t] = keyed[t].second;
            key[t] = dgrid::level_key(keyed[t].first, l);
        }
        std::vector<dgrid::CellEntry> &table = g_table[l];
        table.assign(slots, dgrid::CellEntry{dgrid::kEmptyKey, 0u, 0u});
        int occupied = 0;
        for (uint32_t t = 0; t < n; ++t) {
            if (t > 0 && key[t] == key[t - 1]) continue;
            uint32_t e = t + 1;
            while (e < n && key[e] == key[t]) ++e;
            uint64_t sl = dgrid::key_hash(key[t]) & g_geom.table_mask;
            while (table[sl].key != dgrid::kEmptyKey) sl = (sl + 1) & g_geom.table_mask;
            table[sl] = dgrid::CellEntry{key[t], t, e};
            ++occupied;
        }
        if (l == 0) occupied0 = occupied;
    }
    for (int k = 0; k < 3; ++k) dims[k] = g_geom.level[0].dims[k];
    return occupied0;
}

// On the last grid: points whose level-l cell (from their position, as a
// lookup computes it) differs from their finest cell's coordinates shifted
// right by l (as the single Morton order assumes), over every level, plus
// cells whose run in the Morton order is not contiguous (a key met again
// after another one).
long long vc_grid_mismatches(const float *points, uint32_t n) {
    long long bad = 0;
    const dgrid::GridLevel &l0 = g_geom.level[0];
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t f[3];
        for (int k = 0; k < 3; ++k)
            f[k] = (uint32_t)dgrid::axis_cell(points[3 * i + k], g_geom.lo[k], l0.inv_h, l0.dims[k]);
        const uint64_t m = dgrid::morton_key(f[0], f[1], f[2]);
        for (int l = 0; l < dgrid::kLevels; ++l) {
            const uint64_t want = dgrid::point_key(g_geom, l, points[3 * i], points[3 * i + 1],
                                                   points[3 * i + 2]);
            bad += dgrid::level_key(m, l) != want ? 1 : 0;
        }
    }
    for (int l = 0; l < dgrid::kLevels; ++l) {
        std::vector<uint64_t> seen;
        uint64_t prev = dgrid::kEmptyKey;
        for (uint32_t t = 0; t < n; ++t) {
            const uint32_t i = g_sorted[l][t];
            const uint64_t k = dgrid::point_key(g_geom, l, points[3 * i], points[3 * i + 1],
                                                points[3 * i + 2]);
            if (k != prev) {
                seen.push_back(k);
                prev = k;
            }
        }
        std::sort(seen.begin(), seen.end());
        bad += (long long)(seen.size() - (size_t)(std::unique(seen.begin(), seen.end()) - seen.begin()));
    }
    // the two table lookups agree, on every point's cell (found) and on the
    // cells beside it (often empty)
    const dgrid::GridView gv = view();
    for (int l = 0; l < dgrid::kLevels; ++l) {
        const dgrid::GridLevel &lv = g_geom.level[l];
        for (uint32_t i = 0; i < n; ++i) {
            int c[3];
            for (int k = 0; k < 3; ++k)
                c[k] = dgrid::axis_cell(points[3 * i + k], g_geom.lo[k], lv.inv_h, lv.dims[k]);
            for (int d = 0; d < 3; ++d) {
                const int cx = c[0] + d;
                if (cx >= (int)lv.dims[0]) continue;
                uint32_t b0, e0, b1, e1;
                dgrid::cell_range(gv, l, (uint32_t)cx, (uint32_t)c[1], (uint32_t)c[2], b0, e0);
                dgrid::cell_range_grouped(gv, l, (uint32_t)cx, (uint32_t)c[1], (uint32_t)c[2], b1,
                                          e1);
                bad += (b0 != b1 || e0 != e1) ? 1 : 0;
                if (d == 0) bad += e0 > b0 ? 0 : 1; // the point's own cell holds it
            }
        }
    }
    return bad;
}

// certify_cell for every point on the last grid: status [n], coincident
// count, and the report rows (point, a, b, c) of certified cells, up to
// capacity; returns the number of rows asked for.
long long vc_certify(const float *points, uint32_t n, uint32_t *status, uint32_t *reports,
                     long long capacity, long long *coincident) {
    static Cell cell;
    const dgrid::GridView gv = view();
    long long rows = 0;
    *coincident = 0;
    for (uint32_t i = 0; i < n; ++i) {
        bool co = false;
        status[i] = dgrid::certify_cell(points, i, gv, cell, co);
        *coincident += co ? 1 : 0;
        if (status[i] != kCertified) continue;
        for (int v = 0; v < cell.num_verts; ++v, ++rows) {
            if (rows >= capacity) continue;
            reports[4 * rows] = i;
            for (int k = 0; k < 3; ++k)
                reports[4 * rows + 1 + k] = (uint32_t)cell.planes[cell.verts[v].p[k]].point;
        }
    }
    return rows;
}

// sphere_empty for m candidates [m, 4] on the last grid (status: that of
// vc_certify).
void vc_sphere_empty(const float *points, const uint32_t *cand, long long m,
                     const uint32_t *status, uint32_t *keep) {
    const dgrid::GridView gv = view();
    for (long long t = 0; t < m; ++t)
        keep[t] = dgrid::sphere_empty(points, cand + 4 * t, gv, status);
}
}

