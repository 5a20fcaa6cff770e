// The Delaunay tetrahedralisation on the GPU, by certified Voronoi cells.
//
// certify: a uniform grid over the points (about two points per grid cell),
// then one lane per point clips its Voronoi cell (voronoi_cell.h) by the
// points of the grid rings around it until every point within twice the
// cell's farthest vertex has been seen.  A cell closed by bisectors alone,
// every sign decided, is certified: each of its vertices is a Delaunay
// tetrahedron, written as (point, a, b, c).  The other points (the hull, the
// layer under it, undecided signs) are listed as open.
//
// merge: the caller triangulates the open points on its own (a few percent
// of them); a candidate tetrahedron whose circumsphere holds no point at all
// is Delaunay (exactly those with four open vertices are needed).  Each
// certified tetrahedron is kept once, from its lowest certified vertex;
// neighbours come from a vertex-to-tetrahedra table, one lane per face.
//
// For points in general position this is the one Delaunay tetrahedralisation
// the reference grows by insertion on the GPU (src/delaunay/delaunay.cu:
// 271-345 with sample_initial_tets.cu, growth_iteration.cu).
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <cmath>
#include <cstring>

#include "delaunay_grid.h"
#include "trace_kernels.h"

namespace sdfoam_hip {

namespace {

size_t a256(size_t x) { return (x + 255u) & ~(size_t)255u; }
inline dim3 grid1(uint64_t n) { return dim3((unsigned)((n + 255u) / 256u)); }

using dgrid::GridGeom;
using dgrid::GridView;

struct GridScratch {
    GridGeom *geom;
    unsigned long long *counters;
    uint32_t *mm, *counts, *ids, *ids_sorted, *index, *status;
    uint32_t *start[dgrid::kLevels], *sorted[dgrid::kLevels];
    void *temp;
    size_t temp_bytes;
    size_t total;
};

GridScratch carve_grid(void *base, uint32_t n, size_t temp_bytes) {
    GridScratch s{};
    char *p = static_cast<char *>(base);
    const uint64_t cc = dgrid::level_cell_capacity(n);
    auto take = [&](size_t bytes) {
        char *q = p;
        p += a256(bytes);
        return q;
    };
    s.geom = reinterpret_cast<GridGeom *>(take(sizeof(GridGeom)));
    s.counters = reinterpret_cast<unsigned long long *>(take(8 * 8));
    s.mm = reinterpret_cast<uint32_t *>(take(6 * 4));
    for (int l = 0; l < dgrid::kLevels; ++l) {
        s.start[l] = reinterpret_cast<uint32_t *>(take(4 * (cc + 1)));
        s.sorted[l] = reinterpret_cast<uint32_t *>(take(4ull * n));
    }
    s.counts = reinterpret_cast<uint32_t *>(take(4 * (cc + 1)));
    s.ids = reinterpret_cast<uint32_t *>(take(4ull * n));
    s.ids_sorted = reinterpret_cast<uint32_t *>(take(4ull * n));
    s.index = reinterpret_cast<uint32_t *>(take(4ull * n));
    s.status = reinterpret_cast<uint32_t *>(take(4ull * n));
    s.temp = p;
    s.temp_bytes = temp_bytes;
    s.total = (size_t)(p - static_cast<char *>(base)) + a256(temp_bytes);
    return s;
}

size_t grid_temp_bytes(uint32_t n) {
    size_t a = 0, b = 0;
    const uint32_t *k = nullptr;
    uint32_t *ko = nullptr;
    if (rocprim::radix_sort_pairs(nullptr, a, k, ko, k, ko, (size_t)n, 0u, 32u) != hipSuccess)
        return 0;
    if (rocprim::exclusive_scan(nullptr, b, k, ko, 0u, (size_t)dgrid::level_cell_capacity(n) + 1,
                                rocprim::plus<uint32_t>()) != hipSuccess)
        return 0;
    return std::max(a, b);
}

__device__ __forceinline__ uint32_t ordered(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    return (u & 0x80000000u) ? ~u : (u ^ 0x80000000u);
}

float unordered(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

__global__ __launch_bounds__(64) void init_kernel(uint32_t *__restrict__ mm,
                                                  unsigned long long *__restrict__ counters) {
    if (mm != nullptr && threadIdx.x < 3) {
        mm[threadIdx.x] = 0xffffffffu;
        mm[3 + threadIdx.x] = 0u;
    }
    if (threadIdx.x < 8) counters[threadIdx.x] = 0ull;
}

__global__ __launch_bounds__(256) void bbox_kernel(const float *__restrict__ p, uint32_t n,
                                                   uint32_t *__restrict__ mm) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    uint32_t lo[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu}, hi[3] = {0u, 0u, 0u};
    if (i < n)
        for (int k = 0; k < 3; ++k) lo[k] = hi[k] = ordered(p[3ull * i + k]);
    // wave reduction, then one atomic per wave and bound
    for (int off = 32; off > 0; off >>= 1)
        for (int k = 0; k < 3; ++k) {
            lo[k] = min(lo[k], (uint32_t)__shfl_xor((int)lo[k], off));
            hi[k] = max(hi[k], (uint32_t)__shfl_xor((int)hi[k], off));
        }
    if ((threadIdx.x & 63u) == 0)
        for (int k = 0; k < 3; ++k) {
            atomicMin(mm + k, lo[k]);
            atomicMax(mm + 3 + k, hi[k]);
        }
}

__global__ __launch_bounds__(256) void cell_ids_kernel(const float *__restrict__ p, uint32_t n,
                                                       GridGeom g, int level,
                                                       uint32_t *__restrict__ ids,
                                                       uint32_t *__restrict__ index,
                                                       uint32_t *__restrict__ counts) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const uint32_t c =
        dgrid::cell_index(g, level, p[3ull * i], p[3ull * i + 1], p[3ull * i + 2]);
    ids[i] = c;
    index[i] = i;
    atomicAdd(counts + c, 1u);
}

__global__ __launch_bounds__(256) void fill_kernel(uint32_t *__restrict__ v, uint64_t n,
                                                   uint32_t value) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) v[i] = value;
}

// counters: 0 report rows asked for, 1 open points, 2 undecided cells,
// 3 cells over the fixed capacity, 4 coincident point pairs seen (twice).
__global__ __launch_bounds__(64) void certify_kernel(const float *__restrict__ p, uint32_t n,
                                                     GridView gv, uint32_t *__restrict__ reports,
                                                     uint64_t report_capacity,
                                                     unsigned long long *__restrict__ counters,
                                                     uint32_t *__restrict__ open,
                                                     uint32_t *__restrict__ status_out) {
    const uint32_t i = blockIdx.x * 64u + threadIdx.x;
    if (i >= n) return;
    vcell::Cell cell;
    bool coincident = false;
    const uint32_t st = dgrid::certify_cell(p, i, gv, cell, coincident);
    if (coincident) atomicAdd(counters + 4, 1ull);
    status_out[i] = st;
    if (st == vcell::kCertified) {
        const unsigned long long nv = (unsigned long long)cell.num_verts;
        const unsigned long long at = atomicAdd(counters, nv);
        if (at + nv <= report_capacity) {
            for (int v = 0; v < cell.num_verts; ++v) {
                const vcell::Vert &vx = cell.verts[v];
                uint32_t *row = reports + 4ull * (at + (unsigned long long)v);
                row[0] = i;
                row[1] = (uint32_t)cell.planes[vx.p[0]].point;
                row[2] = (uint32_t)cell.planes[vx.p[1]].point;
                row[3] = (uint32_t)cell.planes[vx.p[2]].point;
            }
        }
    } else {
        const unsigned long long at = atomicAdd(counters + 1, 1ull);
        open[at] = i;
        if (st == vcell::kUncertain) atomicAdd(counters + 2, 1ull);
        if (st == vcell::kOverflow) atomicAdd(counters + 3, 1ull);
    }
}

// 1 if no point lies strictly inside the circumsphere of candidate t, 0 if
// one does, 2 if the tetrahedron is invalid, flat, or a sign could not be
// decided.
__global__ __launch_bounds__(64) void keep_empty_kernel(const float *__restrict__ p, uint32_t n,
                                                        GridView gv,
                                                        const uint32_t *__restrict__ cand,
                                                        uint32_t m,
                                                        const uint32_t *__restrict__ status,
                                                        uint32_t *__restrict__ keep) {
    const uint32_t t = blockIdx.x * 64u + threadIdx.x;
    if (t >= m) return;
    uint32_t v[4];
    bool valid = true;
    for (int k = 0; k < 4; ++k) {
        v[k] = cand[4ull * t + k];
        valid = valid && v[k] < n;
    }
    if (!valid) {
        keep[t] = 2u;
        return;
    }
    keep[t] = dgrid::sphere_empty(p, v, gv, status);
}

// Row t of [reports; candidates] survives: a report (i, a, b, c) when i is
// its lowest certified vertex, a candidate when keep says so.
// errors: 0 a report index out of range, 1 an undecided candidate.
__global__ __launch_bounds__(256) void select_kernel(const uint32_t *__restrict__ reports,
                                                     uint64_t nr,
                                                     const uint32_t *__restrict__ keep,
                                                     uint64_t m,
                                                     const uint32_t *__restrict__ status,
                                                     uint32_t n, uint32_t *__restrict__ flag,
                                                     unsigned long long *__restrict__ errors) {
    const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (t >= nr + m) return;
    uint32_t f = 0;
    if (t < nr) {
        const uint32_t i = reports[4 * t];
        f = i < n ? 1u : 0u;
        for (int k = 1; k < 4 && f; ++k) {
            const uint32_t v = reports[4 * t + k];
            if (v >= n) f = 0u;
            else if (v < i && status[v] == vcell::kCertified) f = 2u;
        }
        if (f == 0u) atomicAdd(errors, 1ull);
        f = f == 1u ? 1u : 0u;
    } else {
        const uint32_t k = keep[t - nr];
        f = k == 1u ? 1u : 0u;
        if (k == 2u) atomicAdd(errors + 1, 1ull);
    }
    flag[t] = f;
}

__global__ __launch_bounds__(256) void compact_kernel(const uint32_t *__restrict__ reports,
                                                      uint64_t nr,
                                                      const uint32_t *__restrict__ cand,
                                                      uint64_t m,
                                                      const uint32_t *__restrict__ flag,
                                                      const uint32_t *__restrict__ pos,
                                                      uint32_t *__restrict__ out,
                                                      uint64_t capacity) {
    const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (t >= nr + m || !flag[t]) return;
    const uint64_t w = pos[t];
    if (w >= capacity) return;
    const uint32_t *src = t < nr ? reports + 4 * t : cand + 4 * (t - nr);
    for (int k = 0; k < 4; ++k) out[4 * w + k] = src[k];
}

__global__ __launch_bounds__(256) void vertex_count_kernel(const uint32_t *__restrict__ tets,
                                                           uint64_t T,
                                                           uint32_t *__restrict__ counts) {
    const uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (e < 4 * T) atomicAdd(counts + tets[e], 1u);
}

__global__ __launch_bounds__(256) void vertex_fill_kernel(const uint32_t *__restrict__ tets,
                                                          uint64_t T,
                                                          uint32_t *__restrict__ cursor,
                                                          uint32_t *__restrict__ entries) {
    const uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (e >= 4 * T) return;
    const uint32_t at = atomicAdd(cursor + tets[e], 1u);
    entries[at] = (uint32_t)(e >> 2);
}

// Neighbour across the face of tet t opposite vertex j: the other tet of
// the face's lowest vertex that holds all three (-1 on the hull).
// acc: 0 faces without a neighbour, 1 faces shared by three tets or more.
__global__ __launch_bounds__(256) void face_neighbor_kernel(const uint32_t *__restrict__ tets,
                                                            uint64_t T,
                                                            const uint32_t *__restrict__ offs,
                                                            const uint32_t *__restrict__ entries,
                                                            int32_t *__restrict__ nbr,
                                                            unsigned long long *__restrict__ acc) {
    const uint64_t f = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (f >= 4 * T) return;
    const uint64_t t = f >> 2;
    const uint32_t j = (uint32_t)(f & 3u);
    uint32_t a[3];
    int w = 0;
    for (uint32_t k = 0; k < 4; ++k)
        if (k != j) a[w++] = tets[4 * t + k];
    const uint32_t lowest = min(a[0], min(a[1], a[2]));
    int32_t other = -1;
    int found = 0;
    for (uint32_t e = offs[lowest]; e < offs[lowest + 1]; ++e) {
        const uint32_t s = entries[e];
        if (s == (uint32_t)t) continue;
        int hits = 0;
        for (int k = 0; k < 4; ++k) {
            const uint32_t x = tets[4ull * s + k];
            hits += (x == a[0] || x == a[1] || x == a[2]) ? 1 : 0;
        }
        if (hits == 3) {
            other = (int32_t)s;
            ++found;
        }
    }
    nbr[f] = other;
    if (found == 0) atomicAdd(acc, 1ull);
    if (found > 1) atomicAdd(acc + 1, 1ull);
}

struct MergeScratch {
    unsigned long long *acc;
    uint32_t *keep, *flag, *pos, *vcount, *voffs, *ventries;
    void *temp;
    size_t temp_bytes;
    size_t total;
};

MergeScratch carve_merge(void *base, uint32_t n, uint64_t nr, uint64_t m, uint64_t tcap,
                         size_t temp_bytes) {
    MergeScratch s{};
    char *p = static_cast<char *>(base);
    auto take = [&](size_t bytes) {
        char *q = p;
        p += a256(bytes);
        return q;
    };
    s.acc = reinterpret_cast<unsigned long long *>(take(8 * 8));
    s.keep = reinterpret_cast<uint32_t *>(take(4 * m));
    s.flag = reinterpret_cast<uint32_t *>(take(4 * (nr + m)));
    s.pos = reinterpret_cast<uint32_t *>(take(4 * (nr + m)));
    s.vcount = reinterpret_cast<uint32_t *>(take(4ull * n + 4));
    s.voffs = reinterpret_cast<uint32_t *>(take(4ull * n + 4));
    s.ventries = reinterpret_cast<uint32_t *>(take(16 * tcap));
    s.temp = p;
    s.temp_bytes = temp_bytes;
    s.total = (size_t)(p - static_cast<char *>(base)) + a256(temp_bytes);
    return s;
}

size_t merge_temp_bytes(uint32_t n, uint64_t rows) {
    size_t a = 0, b = 0;
    const uint32_t *k = nullptr;
    uint32_t *ko = nullptr;
    if (rocprim::exclusive_scan(nullptr, a, k, ko, 0u, (size_t)std::max<uint64_t>(rows, 1),
                                rocprim::plus<uint32_t>()) != hipSuccess)
        return 0;
    if (rocprim::exclusive_scan(nullptr, b, k, ko, 0u, (size_t)n + 1,
                                rocprim::plus<uint32_t>()) != hipSuccess)
        return 0;
    return std::max(a, b);
}

} // namespace

size_t delaunay_certify_scratch_bytes(uint32_t num_points) {
    if (num_points == 0) return 0;
    const size_t temp = grid_temp_bytes(num_points);
    if (temp == 0) return 0;
    return carve_grid(nullptr, num_points, temp).total;
}

hipError_t launch_delaunay_certify(const float *points, uint32_t n, uint32_t *reports,
                                   uint64_t report_capacity, uint32_t *open, uint64_t counts[5],
                                   void *scratch, size_t bytes, hipStream_t stream) {
    for (int k = 0; k < 5; ++k) counts[k] = 0;
    const size_t temp = grid_temp_bytes(n);
    GridScratch s = carve_grid(scratch, n, temp);
    if (n == 0 || temp == 0 || s.total > bytes) return hipErrorInvalidValue;
    hipLaunchKernelGGL(init_kernel, dim3(1), dim3(64), 0, stream, s.mm, s.counters);
    hipLaunchKernelGGL(bbox_kernel, grid1(n), dim3(256), 0, stream, points, n, s.mm);
    uint32_t hm[6];
    hipError_t e = hipMemcpyAsync(hm, s.mm, sizeof(hm), hipMemcpyDeviceToHost, stream);
    if (e != hipSuccess) return e;
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
    GridGeom g{};
    double lo[3], hi[3];
    for (int k = 0; k < 3; ++k) {
        lo[k] = (double)unordered(hm[k]);
        hi[k] = (double)unordered(hm[3 + k]);
    }
    if (!dgrid::grid_geometry(lo, hi, n, g)) return hipErrorInvalidValue;
    // each level: cell of every point, counts -> starts, points by cell
    for (int l = 0; l < dgrid::kLevels; ++l) {
        const uint64_t cells = g.level[l].num_cells;
        hipLaunchKernelGGL(fill_kernel, grid1(cells + 1), dim3(256), 0, stream, s.counts,
                           (uint64_t)cells + 1, 0u);
        hipLaunchKernelGGL(cell_ids_kernel, grid1(n), dim3(256), 0, stream, points, n, g, l,
                           s.ids, s.index, s.counts);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        size_t tb = s.temp_bytes;
        e = rocprim::exclusive_scan(s.temp, tb, s.counts, s.start[l], 0u, (size_t)cells + 1,
                                    rocprim::plus<uint32_t>(), stream);
        if (e != hipSuccess) return e;
        tb = s.temp_bytes;
        e = rocprim::radix_sort_pairs(s.temp, tb, s.ids, s.ids_sorted, s.index, s.sorted[l],
                                      (size_t)n, 0u, 32u, stream);
        if (e != hipSuccess) return e;
    }
    // the geometry stays in the scratch for the merge (`g` lives until the
    // synchronisation below)
    if ((e = hipMemcpyAsync(s.geom, &g, sizeof(g), hipMemcpyHostToDevice, stream)) != hipSuccess)
        return e;
    GridView gv{};
    gv.g = g;
    for (int l = 0; l < dgrid::kLevels; ++l) {
        gv.start[l] = s.start[l];
        gv.sorted[l] = s.sorted[l];
    }
    hipLaunchKernelGGL(certify_kernel, dim3((n + 63u) / 64u), dim3(64), 0, stream, points, n, gv,
                       reports, report_capacity, s.counters, open, s.status);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    unsigned long long hc[8];
    if ((e = hipMemcpyAsync(hc, s.counters, sizeof(hc), hipMemcpyDeviceToHost, stream)) !=
            hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
        return e;
    for (int k = 0; k < 5; ++k) counts[k] = hc[k];
    return hipSuccess;
}

size_t delaunay_merge_scratch_bytes(uint32_t n, uint64_t nr, uint64_t m, uint64_t tcap) {
    const size_t temp = merge_temp_bytes(n, nr + m);
    if (temp == 0) return 0;
    return carve_merge(nullptr, n, nr, m, tcap, temp).total;
}

hipError_t launch_delaunay_merge(const float *points, uint32_t n, void *grid_scratch,
                                 size_t grid_bytes, const uint32_t *reports, uint64_t nr,
                                 const uint32_t *cand, uint64_t m, uint32_t *tets, int32_t *nbr,
                                 uint64_t tcap, uint64_t result[4], void *scratch, size_t bytes,
                                 hipStream_t stream) {
    for (int k = 0; k < 4; ++k) result[k] = 0;
    const size_t gtemp = grid_temp_bytes(n);
    const GridScratch gs = carve_grid(grid_scratch, n, gtemp);
    const size_t temp = merge_temp_bytes(n, nr + m);
    const MergeScratch s = carve_merge(scratch, n, nr, m, tcap, temp);
    if (n == 0 || gtemp == 0 || gs.total > grid_bytes || temp == 0 || s.total > bytes)
        return hipErrorInvalidValue;
    if (nr + m >= 0xffffffffull) return hipErrorInvalidValue;
    GridView gv{};
    hipError_t e =
        hipMemcpyAsync(&gv.g, gs.geom, sizeof(GridGeom), hipMemcpyDeviceToHost, stream);
    if (e != hipSuccess) return e;
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
    for (int l = 0; l < dgrid::kLevels; ++l) {
        gv.start[l] = gs.start[l];
        gv.sorted[l] = gs.sorted[l];
    }
    hipLaunchKernelGGL(init_kernel, dim3(1), dim3(64), 0, stream, nullptr, s.acc);
    if (m > 0)
        hipLaunchKernelGGL(keep_empty_kernel, dim3((unsigned)((m + 63u) / 64u)), dim3(64), 0,
                           stream, points, n, gv, cand, (uint32_t)m, gs.status, s.keep);
    const uint64_t rows = nr + m;
    uint32_t last[2] = {0, 0};
    if (rows > 0) {
        hipLaunchKernelGGL(select_kernel, grid1(rows), dim3(256), 0, stream, reports, nr, s.keep,
                           m, gs.status, n, s.flag, s.acc + 2);
        size_t tb = s.temp_bytes;
        e = rocprim::exclusive_scan(s.temp, tb, s.flag, s.pos, 0u, (size_t)rows,
                                    rocprim::plus<uint32_t>(), stream);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(compact_kernel, grid1(rows), dim3(256), 0, stream, reports, nr, cand,
                           m, s.flag, s.pos, tets, tcap);
        if ((e = hipMemcpyAsync(last, s.pos + (rows - 1), 4, hipMemcpyDeviceToHost, stream)) !=
                hipSuccess ||
            (e = hipMemcpyAsync(last + 1, s.flag + (rows - 1), 4, hipMemcpyDeviceToHost,
                                stream)) != hipSuccess)
            return e;
    }
    unsigned long long acc[8];
    if ((e = hipMemcpyAsync(acc, s.acc, sizeof(acc), hipMemcpyDeviceToHost, stream)) !=
            hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
        return e;
    const uint64_t T = (uint64_t)last[0] + last[1];
    result[0] = T;
    result[2] = acc[2] + acc[3];
    if (T > tcap || result[2] != 0 || T == 0) return hipSuccess;
    // vertex -> tets table (CSR), then one lane per face
    hipLaunchKernelGGL(fill_kernel, grid1((uint64_t)n + 1), dim3(256), 0, stream, s.vcount,
                       (uint64_t)n + 1, 0u);
    hipLaunchKernelGGL(vertex_count_kernel, grid1(4 * T), dim3(256), 0, stream, tets, T,
                       s.vcount);
    size_t tb = s.temp_bytes;
    e = rocprim::exclusive_scan(s.temp, tb, s.vcount, s.voffs, 0u, (size_t)n + 1,
                                rocprim::plus<uint32_t>(), stream);
    if (e != hipSuccess) return e;
    if ((e = hipMemcpyAsync(s.vcount, s.voffs, 4ull * n, hipMemcpyDeviceToDevice, stream)) !=
        hipSuccess)
        return e;
    hipLaunchKernelGGL(vertex_fill_kernel, grid1(4 * T), dim3(256), 0, stream, tets, T, s.vcount,
                       s.ventries);
    hipLaunchKernelGGL(face_neighbor_kernel, grid1(4 * T), dim3(256), 0, stream, tets, T, s.voffs,
                       s.ventries, nbr, s.acc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = hipMemcpyAsync(acc, s.acc, 16, hipMemcpyDeviceToHost, stream)) != hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
        return e;
    result[1] = acc[0];
    result[3] = acc[1];
    return hipSuccess;
}

} // namespace sdfoam_hip
