// One Voronoi cell by plane clipping, for the GPU Delaunay (host and device).
//
// The cell of point o (coordinates relative to o, so o = 0) is the part of a
// box closer to o than to any other point: the box clipped by the bisector
// plane of o and each candidate q, {x : x.q < |q|^2 / 2}.  It is kept as its
// vertices, each the meeting point of three planes (box faces or bisectors),
// stored as a triangle of plane indices ("dual" form): clipping removes the
// vertices outside the new plane and closes the hole with triangles (a, b, q)
// along the boundary edges (a, b).  A vertex of three bisectors (o, a, b, c)
// is the centre of the sphere through o, a, b, c, and it lies outside
// q's halfspace exactly when q is inside that sphere: that decision is made
// by the sign of the insphere determinant, evaluated in double with an error
// bound, and an uncertain sign makes the cell uncertain (never guessed).
// Vertices on box faces use their computed positions with a margin.
//
// Completeness: a candidate q can cut vertex v only if |q| < 2 |v|, so once
// every point within 2 max|v| has been processed the cell is final.  A final
// cell without box vertices is "certified": each of its vertices (o, a, b, c)
// is a Delaunay tetrahedron of the whole point set.
#pragma once

#include <cstdint>

#ifdef __HIPCC__
#define SDF_HD __host__ __device__ __forceinline__
#else
#define SDF_HD inline
#endif

namespace sdfoam_hip {
namespace vcell {

constexpr int kMaxPlanes = 64;  // 6 box faces + bisectors
constexpr int kMaxVerts = 128; // triangles (cell vertices)
constexpr int kMaxEdges = 96;   // directed edges of the removed region

enum Status : uint32_t {
    kCertified = 0,
    kOpen = 1,       // not final yet / touches the box
    kUncertain = 2,  // a sign could not be decided
    kOverflow = 3,   // more planes or vertices than the fixed capacity
};

struct Plane {
    double n[3]; // normal: x.n < c inside
    double c;
    int32_t point; // candidate index (>= 0) or -1 for a box face
};

struct Vert {
    uint8_t p[3]; // plane indices, counter-clockwise seen from outside
    double x[3];  // position
    double e;     // bound on the error of each coordinate of x
    double r2;    // |x|^2
};

struct Cell {
    Plane planes[kMaxPlanes];
    Vert verts[kMaxVerts];
    int num_planes;
    int num_verts;
    uint32_t status;
};

SDF_HD double dabs(double x) { return x < 0.0 ? -x : x; }

// 3x3 determinant of rows a, b, c and its permanent (|terms| summed)
SDF_HD double det3(const double *a, const double *b, const double *c, double &perm) {
    const double m0 = b[1] * c[2] - b[2] * c[1];
    const double m1 = b[0] * c[2] - b[2] * c[0];
    const double m2 = b[0] * c[1] - b[1] * c[0];
    const double p0 = dabs(b[1] * c[2]) + dabs(b[2] * c[1]);
    const double p1 = dabs(b[0] * c[2]) + dabs(b[2] * c[0]);
    const double p2 = dabs(b[0] * c[1]) + dabs(b[1] * c[0]);
    perm = dabs(a[0]) * p0 + dabs(a[1]) * p1 + dabs(a[2]) * p2;
    return a[0] * m0 - a[1] * m1 + a[2] * m2;
}

// Relative error bounds: each determinant is a sum of products of exact
// inputs (coordinates relative to o are exact differences of floats) and
// the rounded lifts |x|^2; the bounds below are a few times the textbook
// ones (3x3: 7 eps, lifted 4x4: 16 eps of the permanent).
constexpr double kEps = 1.1102230246251565e-16; // 2^-53
constexpr double kOrientBound = 16.0 * kEps;
constexpr double kInsphereBound = 64.0 * kEps;

// Is q inside the sphere through o = 0, a, b, c?  +1 inside, -1 outside,
// 0 uncertain.  Inside <=> det4 * det3 < 0 with det4 = det[x, |x|^2] over
// rows a, b, c, q and det3 = det[a; b; c] (Schur complement).
SDF_HD int in_sphere(const double *a, const double *b, const double *c, const double *q) {
    double po;
    const double o3 = det3(a, b, c, po);
    if (dabs(o3) <= kOrientBound * po) return 0;
    const double la = a[0] * a[0] + a[1] * a[1] + a[2] * a[2];
    const double lb = b[0] * b[0] + b[1] * b[1] + b[2] * b[2];
    const double lc = c[0] * c[0] + c[1] * c[1] + c[2] * c[2];
    const double lq = q[0] * q[0] + q[1] * q[1] + q[2] * q[2];
    // expansion along the lift column
    double p_bcq, p_acq, p_abq, p_abc;
    const double d_bcq = det3(b, c, q, p_bcq);
    const double d_acq = det3(a, c, q, p_acq);
    const double d_abq = det3(a, b, q, p_abq);
    const double d_abc = det3(a, b, c, p_abc);
    const double det4 = -la * d_bcq + lb * d_acq - lc * d_abq + lq * d_abc;
    const double perm4 = la * p_bcq + lb * p_acq + lc * p_abq + lq * p_abc;
    if (dabs(det4) <= kInsphereBound * perm4) return 0;
    return (det4 < 0.0) == (o3 > 0.0) ? 1 : -1;
}

// Meeting point of three planes (Cramer's rule); false if they are (nearly)
// dependent.  err: a bound on the rounding error of each coordinate (a few
// times the first-order bound 9 eps sum|c| |minor| / |det| + 7 eps |x|
// perm(det) / |det| of the rounded expressions below, plus 4 eps |x| for the
// quotient: a product with the rounded reciprocal of det is within 2 eps of
// the numerator over det; one reciprocal, not three fp64 divisions).
SDF_HD bool meet(const Plane &A, const Plane &B, const Plane &C, double *x,
                 double *err = nullptr) {
    const double bc[3] = {B.n[1] * C.n[2] - B.n[2] * C.n[1], B.n[2] * C.n[0] - B.n[0] * C.n[2],
                          B.n[0] * C.n[1] - B.n[1] * C.n[0]};
    const double ca[3] = {C.n[1] * A.n[2] - C.n[2] * A.n[1], C.n[2] * A.n[0] - C.n[0] * A.n[2],
                          C.n[0] * A.n[1] - C.n[1] * A.n[0]};
    const double ab[3] = {A.n[1] * B.n[2] - A.n[2] * B.n[1], A.n[2] * B.n[0] - A.n[0] * B.n[2],
                          A.n[0] * B.n[1] - A.n[1] * B.n[0]};
    const double d = A.n[0] * bc[0] + A.n[1] * bc[1] + A.n[2] * bc[2];
    const double na = dabs(A.n[0]) + dabs(A.n[1]) + dabs(A.n[2]);
    const double nb = dabs(B.n[0]) + dabs(B.n[1]) + dabs(B.n[2]);
    const double nc = dabs(C.n[0]) + dabs(C.n[1]) + dabs(C.n[2]);
    if (!(dabs(d) > 1e-12 * na * nb * nc)) return false;
    const double inv = 1.0 / d;
    for (int k = 0; k < 3; ++k) x[k] = (A.c * bc[k] + B.c * ca[k] + C.c * ab[k]) * inv;
    if (err) {
        // permanents of the 2x2 minors
        const double pbc[3] = {dabs(B.n[1] * C.n[2]) + dabs(B.n[2] * C.n[1]),
                               dabs(B.n[2] * C.n[0]) + dabs(B.n[0] * C.n[2]),
                               dabs(B.n[0] * C.n[1]) + dabs(B.n[1] * C.n[0])};
        const double pca[3] = {dabs(C.n[1] * A.n[2]) + dabs(C.n[2] * A.n[1]),
                               dabs(C.n[2] * A.n[0]) + dabs(C.n[0] * A.n[2]),
                               dabs(C.n[0] * A.n[1]) + dabs(C.n[1] * A.n[0])};
        const double pab[3] = {dabs(A.n[1] * B.n[2]) + dabs(A.n[2] * B.n[1]),
                               dabs(A.n[2] * B.n[0]) + dabs(A.n[0] * B.n[2]),
                               dabs(A.n[0] * B.n[1]) + dabs(A.n[1] * B.n[0])};
        const double pd = dabs(A.n[0]) * pbc[0] + dabs(A.n[1]) * pbc[1] + dabs(A.n[2]) * pbc[2];
        const double inv_ad = dabs(inv);
        double e = 0.0;
        for (int k = 0; k < 3; ++k) {
            const double m = dabs(A.c) * pbc[k] + dabs(B.c) * pca[k] + dabs(C.c) * pab[k];
            const double ek =
                32.0 * kEps * (m + dabs(x[k]) * pd) * inv_ad + 4.0 * kEps * dabs(x[k]);
            e = ek > e ? ek : e;
        }
        *err = e;
    }
    return true;
}

// Is vertex v outside plane P (the bisector of o and P's point)?  +1 / -1 / 0.
SDF_HD int outside(const Cell &cell, const Vert &v, const Plane &P, const double *qpos) {
    const Plane &A = cell.planes[v.p[0]], &B = cell.planes[v.p[1]], &C = cell.planes[v.p[2]];
    if (A.point >= 0 && B.point >= 0 && C.point >= 0) {
        // the three bisector normals are the relative positions a, b, c
        return in_sphere(A.n, B.n, C.n, qpos);
    }
    const double s = v.x[0] * P.n[0] + v.x[1] * P.n[1] + v.x[2] * P.n[2] - P.c;
    const double scale = (dabs(v.x[0]) + dabs(v.x[1]) + dabs(v.x[2])) *
                             (dabs(P.n[0]) + dabs(P.n[1]) + dabs(P.n[2])) +
                         dabs(P.c);
    if (dabs(s) <= 1e-9 * scale) return 0;
    return s > 0.0 ? 1 : -1;
}

// Box [lo, hi] around o (relative coordinates; lo < 0 < hi).
SDF_HD void cell_init(Cell &cell, const double *lo, const double *hi) {
    cell.num_planes = 6;
    cell.status = kOpen;
    for (int k = 0; k < 3; ++k) {
        Plane &pl = cell.planes[2 * k];     // x_k < hi_k
        Plane &pm = cell.planes[2 * k + 1]; // -x_k < -lo_k
        for (int j = 0; j < 3; ++j) pl.n[j] = pm.n[j] = 0.0;
        pl.n[k] = 1.0;
        pl.c = hi[k];
        pm.n[k] = -1.0;
        pm.c = -lo[k];
        pl.point = pm.point = -1;
    }
    // corners: planes (x side, y side, z side), ordered counter-clockwise
    // seen from outside (flip when the number of "low" sides is odd)
    cell.num_verts = 0;
    for (int sx = 0; sx < 2; ++sx)
        for (int sy = 0; sy < 2; ++sy)
            for (int sz = 0; sz < 2; ++sz) {
                Vert &v = cell.verts[cell.num_verts++];
                const uint8_t px = (uint8_t)(0 + sx), py = (uint8_t)(2 + sy), pz = (uint8_t)(4 + sz);
                if (((sx + sy + sz) & 1) == 0) {
                    v.p[0] = px;
                    v.p[1] = py;
                    v.p[2] = pz;
                } else {
                    v.p[0] = px;
                    v.p[1] = pz;
                    v.p[2] = py;
                }
                v.x[0] = sx ? lo[0] : hi[0];
                v.x[1] = sy ? lo[1] : hi[1];
                v.x[2] = sz ? lo[2] : hi[2];
                v.e = 0.0;
                v.r2 = v.x[0] * v.x[0] + v.x[1] * v.x[1] + v.x[2] * v.x[2];
            }
}

SDF_HD double max_r2(const Cell &cell) {
    double m = 0.0;
    for (int i = 0; i < cell.num_verts; ++i) m = cell.verts[i].r2 > m ? cell.verts[i].r2 : m;
    return m;
}

// Drops the planes no vertex uses any more (cut away by later planes) and
// renumbers the vertices' plane indices; true if room was made.
SDF_HD bool compact_planes(Cell &cell) {
    bool used[kMaxPlanes];
    uint8_t map[kMaxPlanes];
    for (int i = 0; i < cell.num_planes; ++i) used[i] = false;
    for (int i = 0; i < cell.num_verts; ++i)
        for (int k = 0; k < 3; ++k) used[cell.verts[i].p[k]] = true;
    int w = 0;
    for (int i = 0; i < cell.num_planes; ++i) {
        if (!used[i]) continue;
        map[i] = (uint8_t)w;
        if (w != i) cell.planes[w] = cell.planes[i];
        ++w;
    }
    for (int i = 0; i < cell.num_verts; ++i)
        for (int k = 0; k < 3; ++k) cell.verts[i].p[k] = map[cell.verts[i].p[k]];
    cell.num_planes = w;
    return w < kMaxPlanes;
}

// Clips the cell by the bisector of o and candidate `point` at relative
// position q.  Returns false when the cell became uncertain or overflowed
// (cell.status says which); *cut (if given) says whether the plane removed
// any vertex.
SDF_HD bool clip(Cell &cell, const double *q, int32_t point, bool *cut = nullptr) {
    if (cut) *cut = false;
    if (cell.num_planes >= kMaxPlanes && !compact_planes(cell)) {
        cell.status = kOverflow;
        return false;
    }
    Plane &P = cell.planes[cell.num_planes];
    P.n[0] = q[0];
    P.n[1] = q[1];
    P.n[2] = q[2];
    P.c = 0.5 * (q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
    P.point = point;
    // conflicts: the vertex position decides where it is clear of the
    // plane by more than its error bound (and the dot product's rounding),
    // the exact test elsewhere
    bool out[kMaxVerts];
    int n_out = 0;
    const double qn = dabs(q[0]) + dabs(q[1]) + dabs(q[2]);
    for (int i = 0; i < cell.num_verts; ++i) {
        const Vert &v = cell.verts[i];
        const double sd = v.x[0] * q[0] + v.x[1] * q[1] + v.x[2] * q[2] - P.c;
        const double bound =
            v.e * qn +
            4.0 * kEps * (dabs(v.x[0] * q[0]) + dabs(v.x[1] * q[1]) + dabs(v.x[2] * q[2]) + P.c);
        if (sd < -bound || sd > bound) {
            out[i] = sd > 0.0;
            n_out += out[i] ? 1 : 0;
            continue;
        }
        const int s = outside(cell, v, P, q);
        if (s == 0) {
            cell.status = kUncertain;
            return false;
        }
        out[i] = s > 0;
        n_out += out[i] ? 1 : 0;
    }
    if (n_out == 0) return true; // the plane misses the cell
    if (cut) *cut = true;
    if (n_out == cell.num_verts) {
        cell.status = kUncertain; // o itself would be cut off: impossible
        return false;
    }
    // boundary edges: directed edges of removed triangles whose reverse is
    // not an edge of another removed triangle
    uint8_t ea[kMaxEdges], eb[kMaxEdges];
    int ne = 0;
    for (int i = 0; i < cell.num_verts; ++i) {
        if (!out[i]) continue;
        for (int k = 0; k < 3; ++k) {
            if (ne >= kMaxEdges) {
                cell.status = kOverflow;
                return false;
            }
            ea[ne] = cell.verts[i].p[k];
            eb[ne] = cell.verts[i].p[(k + 1) % 3];
            ++ne;
        }
    }
    const uint8_t np = (uint8_t)cell.num_planes;
    int kept = 0;
    // compact the surviving vertices first
    for (int i = 0; i < cell.num_verts; ++i)
        if (!out[i]) cell.verts[kept++] = cell.verts[i];
    cell.num_verts = kept;
    for (int e = 0; e < ne; ++e) {
        bool interior = false;
        for (int f = 0; f < ne; ++f) {
            if (ea[f] == eb[e] && eb[f] == ea[e]) {
                interior = true;
                break;
            }
        }
        if (interior) continue;
        if (cell.num_verts >= kMaxVerts) {
            cell.status = kOverflow;
            return false;
        }
        Vert &v = cell.verts[cell.num_verts];
        v.p[0] = ea[e];
        v.p[1] = eb[e];
        v.p[2] = np;
        if (!meet(cell.planes[v.p[0]], cell.planes[v.p[1]], P, v.x, &v.e)) {
            cell.status = kUncertain;
            return false;
        }
        v.r2 = v.x[0] * v.x[0] + v.x[1] * v.x[1] + v.x[2] * v.x[2];
        ++cell.num_verts;
    }
    ++cell.num_planes;
    return true;
}

// Final status once every point within the candidate radius r (squared:
// reach2) has been clipped: certified if 4 max|v|^2 < reach2 and no vertex
// lies on a box face.
SDF_HD uint32_t settle(Cell &cell, double reach2) {
    if (cell.status == kUncertain || cell.status == kOverflow) return cell.status;
    if (!(4.0 * max_r2(cell) * (1.0 + 1e-9) < reach2)) return kOpen;
    for (int i = 0; i < cell.num_verts; ++i)
        for (int k = 0; k < 3; ++k)
            if (cell.planes[cell.verts[i].p[k]].point < 0) return kOpen;
    cell.status = kCertified;
    return kCertified;
}

} // namespace vcell
} // namespace sdfoam_hip
