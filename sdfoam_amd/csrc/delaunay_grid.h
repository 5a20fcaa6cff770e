// The point grids of the GPU Delaunay and the two per-item steps that use
// them (host and device): one point's certified Voronoi cell (certify_cell:
// the one-cell statement of the decisions certify_kernel makes with a whole
// wavefront per cell, run by the host tests), and one candidate
// tetrahedron's empty-circumsphere test (sphere_empty, run by
// keep_empty_kernel and the host tests).
#pragma once

#include <cmath>
#include <cstdint>

#include "voronoi_cell.h"

namespace sdfoam_hip {
namespace dgrid {

// A hierarchy of sparse grids over the points, kLevelRatio times coarser
// per axis from each level to the next: the coarsest has cells of about
// twice the mean point spacing over the bounding box, the finest is
// kLevelRatio^(kLevels-1) times finer, so that regions a million times denser
// than the mean still have a level with a few points per cell.  Only
// occupied cells are stored: the points are sorted once by the Morton code
// of their finest-level cell, which also orders them by their cell on every
// coarser level (a level-l cell is the finest cell's coordinates shifted
// right by l, exactly, since the cell edges are the finest one's times
// powers of two), and each level is an open-addressing hash table from cell
// key to the cell's run of that one order.  A
// cell starts on the finest level where its point's own grid cell holds
// another point, is clipped ring by ring there, and moves up a level when
// the rings it would still need exceed kMaxRing.
constexpr int kLevels = 11;
constexpr double kLevelRatio = 2.0;
constexpr int kMaxRing = 6;  // rings per level
constexpr int kMinRing = 2;  // rings on a level before moving up
constexpr int kBoxRing = 3;  // from here, a cell still reaching the box on a
                             // level above its first is left open (hull points;
                             // at 2, a quarter more cells by large empty regions
                             // were left open too: C3 10.7k against 7.9k)
// Candidate points a cell may examine in all before it is left open (bounds
// the slowest cell).
constexpr uint32_t kMaxCandidates = 65536;
constexpr uint32_t kAxisCells = (1u << 21) - 1; // cells per axis at most (21-bit keys)
constexpr uint64_t kEmptyKey = ~0ull;

struct alignas(16) CellEntry {
    uint64_t key;        // cx | cy << 21 | cz << 42, kEmptyKey if the slot is free
    uint32_t start, end; // the cell's points: sorted[start : end]
};

struct GridLevel {
    double h, inv_h; // cell edge
    uint32_t dims[3];
    uint32_t pad;
};

struct GridGeom {
    double lo[3];     // grid origin (the points' bounding box)
    double slack;     // rounding allowance of a cell's bounds
    double box_lo[3]; // clipping box: the bounding box grown by its extent
    double box_hi[3];
    GridLevel level[kLevels];
    uint64_t table_mask; // hash table slots - 1 (the same for every level)
};

struct GridView {
    GridGeom g;
    const CellEntry *table[kLevels];
    const uint32_t *sorted[kLevels]; // point ids by cell (one array: the Morton order)
    // the points' coordinates in that order (x, y, z, 0 per point): a run of
    // a cell's candidates is a run of memory, not one cache line per point
    const float *spts;
};

// Hash table slots: a power of two of at least twice the points, so that
// every probe sequence meets a free slot.
inline uint64_t table_slots(uint32_t n) {
    uint64_t c = 64;
    while (c < 2ull * n + 2) c <<= 1;
    return c;
}

// The grids over the bounding box [lo, hi] of n points, and the clipping box:
// the bounding box grown by box_scale times its extent.  False if the box is
// not finite or has no extent.
inline bool grid_geometry(const double *lo, const double *hi, uint32_t n, GridGeom &g,
                          double box_scale = 1.0) {
    double ext = 0.0, mag = 0.0;
    for (int k = 0; k < 3; ++k) {
        if (!std::isfinite(lo[k]) || !std::isfinite(hi[k]) || !(hi[k] >= lo[k])) return false;
        ext = std::fmax(ext, hi[k] - lo[k]);
        mag = std::fmax(mag, std::fmax(std::fabs(lo[k]), std::fabs(hi[k])));
    }
    if (!(ext > 0.0)) return false;
    double vol = 1.0;
    int axes = 0;
    for (int k = 0; k < 3; ++k)
        if (hi[k] - lo[k] > 1e-6 * ext) {
            vol *= hi[k] - lo[k];
            ++axes;
        }
    const double top = 2.0 * std::pow(vol / std::fmax(1.0, (double)n),
                                      1.0 / (double)(axes > 0 ? axes : 1));
    double h = std::fmax(top / std::pow(kLevelRatio, kLevels - 1), ext / (double)(kAxisCells - 1));
    for (int l = 0; l < kLevels; ++l) {
        GridLevel &lv = g.level[l];
        lv.h = h;
        lv.inv_h = 1.0 / h;
        for (int k = 0; k < 3; ++k)
            lv.dims[k] = (uint32_t)std::fmax(1.0, std::fmin(std::ceil((hi[k] - lo[k]) / h),
                                                          (double)kAxisCells));
        lv.pad = 0;
        h *= kLevelRatio;
    }
    g.slack = 1e-12 * (mag + ext);
    g.table_mask = table_slots(n) - 1;
    for (int k = 0; k < 3; ++k) {
        g.lo[k] = lo[k];
        g.box_lo[k] = lo[k] - box_scale * ext;
        g.box_hi[k] = hi[k] + box_scale * ext;
    }
    return true;
}

SDF_HD int axis_cell(double x, double lo, double inv_h, uint32_t dim) {
    const double c = (x - lo) * inv_h;
    if (!(c > 0.0)) return 0;
    const uint32_t u = c < 4294967295.0 ? (uint32_t)c : 0xffffffffu;
    return (int)(u < dim ? u : dim - 1);
}

SDF_HD uint64_t cell_key(uint32_t cx, uint32_t cy, uint32_t cz) {
    return (uint64_t)cx | ((uint64_t)cy << 21) | ((uint64_t)cz << 42);
}

// Morton code of a cell (21 bits per axis, x lowest) and back.
SDF_HD uint64_t spread3(uint32_t v) {
    uint64_t x = v & 0x1fffffull;
    x = (x | x << 32) & 0x1f00000000ffffull;
    x = (x | x << 16) & 0x1f0000ff0000ffull;
    x = (x | x << 8) & 0x100f00f00f00f00full;
    x = (x | x << 4) & 0x10c30c30c30c30c3ull;
    x = (x | x << 2) & 0x1249249249249249ull;
    return x;
}
SDF_HD uint32_t compact3(uint64_t x) {
    x &= 0x1249249249249249ull;
    x = (x | x >> 2) & 0x10c30c30c30c30c3ull;
    x = (x | x >> 4) & 0x100f00f00f00f00full;
    x = (x | x >> 8) & 0x1f0000ff0000ffull;
    x = (x | x >> 16) & 0x1f00000000ffffull;
    x = (x | x >> 32) & 0x1fffffull;
    return (uint32_t)x;
}
SDF_HD uint64_t morton_key(uint32_t cx, uint32_t cy, uint32_t cz) {
    return spread3(cx) | spread3(cy) << 1 | spread3(cz) << 2;
}
// The level-l cell key of the finest cell with Morton code m.
SDF_HD uint64_t level_key(uint64_t m, int l) {
    return cell_key(compact3(m) >> l, compact3(m >> 1) >> l, compact3(m >> 2) >> l);
}

SDF_HD uint64_t point_key(const GridGeom &g, int l, double x, double y, double z) {
    const GridLevel &lv = g.level[l];
    return cell_key((uint32_t)axis_cell(x, g.lo[0], lv.inv_h, lv.dims[0]),
                    (uint32_t)axis_cell(y, g.lo[1], lv.inv_h, lv.dims[1]),
                    (uint32_t)axis_cell(z, g.lo[2], lv.inv_h, lv.dims[2]));
}

// 64-bit mixing (the splitmix64 finaliser) for the table slot.
SDF_HD uint64_t key_hash(uint64_t k) {
    k ^= k >> 30;
    k *= 0xbf58476d1ce4e5b9ull;
    k ^= k >> 27;
    k *= 0x94d049bb133111ebull;
    k ^= k >> 31;
    return k;
}

// The points of cell (cx, cy, cz) of level l: sorted[l][b : e] (empty if
// the cell holds none).
SDF_HD void cell_range(const GridView &gv, int l, uint32_t cx, uint32_t cy, uint32_t cz,
                       uint32_t &b, uint32_t &e) {
    const uint64_t key = cell_key(cx, cy, cz);
    const uint64_t mask = gv.g.table_mask;
    const CellEntry *t = gv.table[l];
    b = e = 0;
    for (uint64_t s = key_hash(key) & mask;; s = (s + 1) & mask) {
        const CellEntry en = t[s];
        if (en.key == key) {
            b = en.start;
            e = en.end;
            return;
        }
        if (en.key == kEmptyKey) return;
    }
}

// Probe of one table slot for `key`: true once the search ends there (the
// key found: its run in b, e; or an empty slot: the cell holds no point).
SDF_HD bool slot_ends(const CellEntry &en, uint64_t key, uint32_t &b, uint32_t &e) {
    if (en.key == key) {
        b = en.start;
        e = en.end;
        return true;
    }
    return en.key == kEmptyKey;
}

// cell_range probing a 64-byte group of four slots at a time: the group's
// loads go out together, so a probe sequence within it (nearly all of them)
// waits for one memory access.  For the circumsphere scans, which wait on
// their lookups (check_kernel 20.9 -> 19.7 ms at C3); the certification,
// which keeps more registers live, runs ~1% slower with it.
SDF_HD void cell_range_grouped(const GridView &gv, int l, uint32_t cx, uint32_t cy,
                               uint32_t cz, uint32_t &b, uint32_t &e) {
    const uint64_t key = cell_key(cx, cy, cz);
    const uint64_t mask = gv.g.table_mask;
    const CellEntry *t = gv.table[l];
    b = e = 0;
    for (uint64_t s = key_hash(key) & mask;;) {
        const uint64_t g0 = s & ~3ull; // the table has a power of two >= 4 slots
        const uint32_t k0 = (uint32_t)(s - g0);
        const CellEntry c0 = t[g0], c1 = t[g0 + 1], c2 = t[g0 + 2], c3 = t[g0 + 3];
        if (k0 == 0u && slot_ends(c0, key, b, e)) return;
        if (k0 <= 1u && slot_ends(c1, key, b, e)) return;
        if (k0 <= 2u && slot_ends(c2, key, b, e)) return;
        if (slot_ends(c3, key, b, e)) return;
        s = (g0 + 4) & mask;
    }
}

// The first level of point x: the finest whose grid cell around x holds
// another point (the coarsest if none does).
SDF_HD int first_level(const GridView &gv, const double *x) {
    const GridGeom &g = gv.g;
    for (int l = 0; l < kLevels - 1; ++l) {
        const GridLevel &lv = g.level[l];
        uint32_t b, e;
        cell_range(gv, l, (uint32_t)axis_cell(x[0], g.lo[0], lv.inv_h, lv.dims[0]),
                   (uint32_t)axis_cell(x[1], g.lo[1], lv.inv_h, lv.dims[1]),
                   (uint32_t)axis_cell(x[2], g.lo[2], lv.inv_h, lv.dims[2]), b, e);
        if (e - b >= 2) return l;
    }
    return kLevels - 1;
}

// Bounding box of the cell's vertices, grown by their error bounds: a
// candidate q can cut the cell only if max over the box of x.q exceeds
// |q|^2 / 2.
SDF_HD void vertex_box(const vcell::Cell &cell, double *lo, double *hi) {
    for (int k = 0; k < 3; ++k) {
        lo[k] = cell.verts[0].x[k];
        hi[k] = cell.verts[0].x[k];
    }
    double e = 0.0;
    for (int i = 0; i < cell.num_verts; ++i) {
        const vcell::Vert &v = cell.verts[i];
        for (int k = 0; k < 3; ++k) {
            lo[k] = v.x[k] < lo[k] ? v.x[k] : lo[k];
            hi[k] = v.x[k] > hi[k] ? v.x[k] : hi[k];
        }
        e = v.e > e ? v.e : e;
    }
    for (int k = 0; k < 3; ++k) {
        lo[k] -= e;
        hi[k] += e;
    }
}

SDF_HD bool touches_box(const vcell::Cell &cell) {
    for (int i = 0; i < cell.num_verts; ++i)
        for (int k = 0; k < 3; ++k)
            if (cell.planes[cell.verts[i].p[k]].point < 0) return true;
    return false;
}

// Was point x (absolute) in the part of a finer level already searched?
SDF_HD bool searched(const GridGeom &g, int l, const double *x, const int (*hc)[3],
                     const int *rings) {
    for (int m = 0; m < l; ++m) {
        if (rings[m] < 0) continue;
        const GridLevel &lv = g.level[m];
        bool in = true;
        for (int k = 0; k < 3 && in; ++k) {
            const int c = axis_cell(x[k], g.lo[k], lv.inv_h, lv.dims[k]);
            in = c - hc[m][k] <= rings[m] && hc[m][k] - c <= rings[m];
        }
        if (in) return true;
    }
    return false;
}

// The Voronoi cell of point i, clipped by the grid rings around it, nearest
// ring first, finest level first, until every point that could still cut
// it has been seen (certified), it is left open, or a sign is undecided.
// `coincident` is set when another point has the same coordinates (the cell
// is then undecided).
SDF_HD uint32_t certify_cell(const float *p, uint32_t i, const GridView &gv, vcell::Cell &cell,
                             bool &coincident) {
    const GridGeom &g = gv.g;
    coincident = false;
    const double o[3] = {(double)p[3ull * i], (double)p[3ull * i + 1], (double)p[3ull * i + 2]};
    {
        double rlo[3], rhi[3];
        for (int k = 0; k < 3; ++k) {
            rlo[k] = g.box_lo[k] - o[k];
            rhi[k] = g.box_hi[k] - o[k];
        }
        vcell::cell_init(cell, rlo, rhi);
    }
    double mr2 = vcell::max_r2(cell);
    double blo[3], bhi[3];
    vertex_box(cell, blo, bhi);
    int hc[kLevels][3];
    int rings[kLevels];
    for (int l = 0; l < kLevels; ++l) {
        rings[l] = -1;
        for (int k = 0; k < 3; ++k)
            hc[l][k] = axis_cell(o[k], g.lo[k], g.level[l].inv_h, g.level[l].dims[k]);
    }
    uint32_t examined = 0;
    const int l0 = first_level(gv, o);
    for (int l = l0; l < kLevels; ++l) {
        const GridLevel &lv = g.level[l];
        const uint32_t *sorted = gv.sorted[l];
        const int *h = hc[l];
        for (int r = 0; r <= kMaxRing; ++r) {
            for (int dz = -r; dz <= r; ++dz) {
                const int cz = h[2] + dz;
                if (cz < 0 || cz >= (int)lv.dims[2]) continue;
                for (int dy = -r; dy <= r; ++dy) {
                    const int cy = h[1] + dy;
                    if (cy < 0 || cy >= (int)lv.dims[1]) continue;
                    // inside the shell only the two end cells of a row are new
                    const bool full_row = r == 0 || dz == -r || dz == r || dy == -r || dy == r;
                    const int step = full_row ? 1 : 2 * r;
                    for (int dx = -r; dx <= r; dx += step) {
                        const int cx = h[0] + dx;
                        if (cx < 0 || cx >= (int)lv.dims[0]) continue;
                        uint32_t begin, end;
                        cell_range(gv, l, (uint32_t)cx, (uint32_t)cy, (uint32_t)cz, begin, end);
                        examined += end - begin;
                        if (examined > kMaxCandidates) return vcell::kOpen;
                        for (uint32_t k = begin; k < end; ++k) {
                            const uint32_t j = sorted[k];
                            if (j == i) continue;
                            const float *sp = gv.spts + 4ull * k;
                            const double x[3] = {(double)sp[0], (double)sp[1], (double)sp[2]};
                            const double q[3] = {x[0] - o[0], x[1] - o[1], x[2] - o[2]};
                            const double d2 = q[0] * q[0] + q[1] * q[1] + q[2] * q[2];
                            if (d2 == 0.0) {
                                coincident = true;
                                cell.status = vcell::kUncertain;
                                return cell.status;
                            }
                            if (d2 > 4.0 * mr2 * (1.0 + 1e-9)) continue; // cannot cut
                            // the bisector x.q = |q|^2 / 2 misses the vertices' box
                            // (by more than the rounding of the sums)
                            double reach_q = 0.0, mag = d2;
                            for (int m = 0; m < 3; ++m) {
                                const double b = q[m] > 0.0 ? bhi[m] : blo[m];
                                reach_q += b * q[m];
                                mag += vcell::dabs(b * q[m]);
                            }
                            if (reach_q < 0.5 * d2 - 1e-14 * mag) continue;
                            if (l > l0 && searched(g, l, x, hc, rings)) continue;
                            bool cut = false;
                            if (!vcell::clip(cell, q, (int32_t)j, &cut)) return cell.status;
                            if (cut) {
                                mr2 = vcell::max_r2(cell);
                                vertex_box(cell, blo, bhi);
                            }
                        }
                    }
                }
            }
            rings[l] = r;
            // every point not yet seen lies r cells of this level away or
            // more (or nowhere)
            const bool all = h[0] - r <= 0 && h[0] + r >= (int)lv.dims[0] - 1 && h[1] - r <= 0 &&
                             h[1] + r >= (int)lv.dims[1] - 1 && h[2] - r <= 0 &&
                             h[2] + r >= (int)lv.dims[2] - 1;
            const double reach = (double)r * lv.h - g.slack;
            const double reach2 = all ? INFINITY : (reach > 0.0 ? reach * reach : 0.0);
            if (4.0 * mr2 * (1.0 + 1e-9) < reach2) return vcell::settle(cell, reach2);
            if (r >= kBoxRing && touches_box(cell)) {
                if (l == l0) break;
                return vcell::kOpen;
            }
            // rings this level would still need if the cell shrank no more
            if (r >= kMinRing && 4.0 * mr2 * (1.0 + 1e-9) > (kMaxRing * lv.h) * (kMaxRing * lv.h))
                break;
        }
    }
    return vcell::kOpen;
}

// The circumsphere of a candidate tetrahedron v[4] (ids below n) and the
// part of a grid level to scan for points inside it: (y, z) columns of cells
// over the sphere's box, each scanned along x over the cells the sphere
// reaches in that column.
struct Sphere {
    double o[3];        // v[0]
    vcell::Plane pl[3]; // bisectors of v[0] and v[1..3] (normals: relative positions)
    double ctr[3];      // circumcentre relative to o
    double r;           // radius, grown by the circumcentre's error bound
    int l;              // grid level
    int lo_c[3], hi_c[3];
};

// False if the tetrahedron is flat (no circumcentre).  The level is the
// finest on which the sphere's box spans at most `max_cols` (y, z) columns:
// many small cells for a wavefront that scans the columns in parallel, a
// few cells of about the sphere's size for one lane that scans them all.
SDF_HD bool sphere_setup(const float *p, const uint32_t *v, const GridView &gv, Sphere &S,
                         double max_cols = 256.0) {
    const GridGeom &g = gv.g;
    for (int k = 0; k < 3; ++k) S.o[k] = (double)p[3ull * v[0] + k];
    for (int s = 0; s < 3; ++s) {
        for (int k = 0; k < 3; ++k) S.pl[s].n[k] = (double)p[3ull * v[s + 1] + k] - S.o[k];
        S.pl[s].c = 0.5 * (S.pl[s].n[0] * S.pl[s].n[0] + S.pl[s].n[1] * S.pl[s].n[1] +
                           S.pl[s].n[2] * S.pl[s].n[2]);
        S.pl[s].point = (int32_t)v[s + 1];
    }
    // the circumcentre (relative to o) is where the three bisectors meet, to
    // within err per coordinate (meet's bound); a point strictly inside the
    // true sphere lies within |ctr| + 2 sqrt(3) err of the computed centre.
    // The margin is absolute: a relative one would let the nearly flat
    // tetrahedra on a planar face of the hull (radii ~1e6 times the scene)
    // cover the whole scene.
    double err = 0.0;
    if (!vcell::meet(S.pl[0], S.pl[1], S.pl[2], S.ctr, &err)) return false;
    const double r2 = S.ctr[0] * S.ctr[0] + S.ctr[1] * S.ctr[1] + S.ctr[2] * S.ctr[2];
    S.r = sqrt(r2) * (1.0 + 1e-12) + 4.0 * err + g.slack;
    // the finest level whose cells cover the sphere's box in few columns
    for (S.l = 0;; ++S.l) {
        const GridLevel &lv = g.level[S.l];
        for (int k = 0; k < 3; ++k) {
            S.lo_c[k] = axis_cell(S.o[k] + S.ctr[k] - S.r, g.lo[k], lv.inv_h, lv.dims[k]);
            S.hi_c[k] = axis_cell(S.o[k] + S.ctr[k] + S.r, g.lo[k], lv.inv_h, lv.dims[k]);
        }
        const double cols =
            (double)(S.hi_c[1] - S.lo_c[1] + 1) * (double)(S.hi_c[2] - S.lo_c[2] + 1);
        if (cols <= max_cols || S.l == kLevels - 1) break;
    }
    return true;
}

SDF_HD uint32_t sphere_columns(const Sphere &S) {
    return (uint32_t)(S.hi_c[1] - S.lo_c[1] + 1) * (uint32_t)(S.hi_c[2] - S.lo_c[2] + 1);
}

// Status of a point an incremental rebuild neither certifies nor lists as
// open (its old tetrahedra are kept): like a certified point, its sign on a
// sphere must be decided.
constexpr uint32_t kStatusClean = 4u;

// Points of column `col` against the sphere: 0 if one lies strictly inside,
// 2 if none does but one's sign is undecided and it is certified or clean (an
// open point exactly on the sphere is passed over: the candidates' own
// triangulation of the open points already chose among such points), 1
// otherwise.
SDF_HD uint32_t sphere_scan_column(const float *p, const uint32_t *v, const GridView &gv,
                                   const uint32_t *status, const Sphere &S, uint32_t col) {
    const GridGeom &g = gv.g;
    const GridLevel &lv = g.level[S.l];
    const uint32_t ny = (uint32_t)(S.hi_c[1] - S.lo_c[1] + 1);
    const int cy = S.lo_c[1] + (int)(col % ny), cz = S.lo_c[2] + (int)(col / ny);
    // squared distance from the centre to the column's y and z extent
    double rem = S.r * S.r;
    const int cc[3] = {0, cy, cz};
    for (int k = 1; k < 3; ++k) {
        const double blo = g.lo[k] + (double)cc[k] * lv.h - S.o[k] - g.slack;
        const double bhi = blo + lv.h + 2.0 * g.slack;
        const double e =
            S.ctr[k] < blo ? blo - S.ctr[k] : (S.ctr[k] > bhi ? S.ctr[k] - bhi : 0.0);
        rem -= e * e;
    }
    if (rem < 0.0) return 1u;
    const double w = sqrt(rem);
    const int x0 = axis_cell(S.o[0] + S.ctr[0] - w - g.slack, g.lo[0], lv.inv_h, lv.dims[0]);
    const int x1 = axis_cell(S.o[0] + S.ctr[0] + w + g.slack, g.lo[0], lv.inv_h, lv.dims[0]);
    const uint32_t *sorted = gv.sorted[S.l];
    uint32_t res = 1u;
    for (int cx = x0 > S.lo_c[0] ? x0 : S.lo_c[0]; cx <= (x1 < S.hi_c[0] ? x1 : S.hi_c[0]); ++cx) {
        uint32_t begin, end;
        cell_range_grouped(gv, S.l, (uint32_t)cx, (uint32_t)cy, (uint32_t)cz, begin, end);
        for (uint32_t k = begin; k < end; ++k) {
            const uint32_t j = sorted[k];
            if (j == v[0] || j == v[1] || j == v[2] || j == v[3]) continue;
            const float *sp = gv.spts + 4ull * k;
            double q[3];
            for (int m = 0; m < 3; ++m) q[m] = (double)sp[m] - S.o[m];
            const double e0 = q[0] - S.ctr[0], e1 = q[1] - S.ctr[1], e2 = q[2] - S.ctr[2];
            if (e0 * e0 + e1 * e1 + e2 * e2 > S.r * S.r) continue; // clearly outside
            const int s = vcell::in_sphere(S.pl[0].n, S.pl[1].n, S.pl[2].n, q);
            if (s > 0) return 0u;
            if (s == 0 && (status[j] == vcell::kCertified || status[j] == kStatusClean)) res = 2u;
        }
    }
    return res;
}

// Candidate tetrahedron v[4] (ids below n): 1 if no point lies strictly
// inside its circumsphere, 0 if one does, 2 if it is flat or, with none
// inside, a certified or clean point's sign could not be decided.
SDF_HD uint32_t sphere_empty(const float *p, const uint32_t *v, const GridView &gv,
                             const uint32_t *status, double max_cols = 256.0) {
    Sphere S;
    if (!sphere_setup(p, v, gv, S, max_cols)) return 2u;
    uint32_t res = 1u;
    const uint32_t cols = sphere_columns(S);
    for (uint32_t c = 0; c < cols; ++c) {
        const uint32_t r = sphere_scan_column(p, v, gv, status, S, c);
        if (r == 0u) return 0u;
        if (r == 2u) res = 2u;
    }
    return res;
}

} // namespace dgrid
} // namespace sdfoam_hip
