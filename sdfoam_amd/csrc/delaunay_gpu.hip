// The Delaunay tetrahedralisation on the GPU, by certified Voronoi cells.
//
// certify: sparse grids over the points (delaunay_grid.h), then one
// wavefront per point clips its Voronoi cell by the points of the grid rings
// around it, with the decisions of vcell::clip (voronoi_cell.h), until every
// point within twice the cell's farthest vertex has been seen.  A cell closed
// by bisectors alone, every sign decided, is certified: each of its vertices
// is a Delaunay tetrahedron, written as (point, a, b, c).  The other points
// (the hull, the layer under it, undecided signs) are listed as open.
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

#include <algorithm>
#include <cmath>
#include <cstring>

#include "delaunay_grid.h"
#include "delaunay_gpu.h"
#include "trace_kernels.h"

namespace sdfoam_hip {

namespace {

size_t a256(size_t x) { return (x + 255u) & ~(size_t)255u; }
inline dim3 grid1(uint64_t n) { return dim3((unsigned)((n + 255u) / 256u)); }

using dgrid::GridGeom;
using dgrid::GridView;

struct GridScratch {
    GridGeom *geom;
    uint64_t *tag; // kGridTag and the point count, once the grid is built
    unsigned long long *counters;
    uint32_t *mm, *index, *status;
    uint64_t *keys, *keys_sorted;
    dgrid::CellEntry *table[dgrid::kLevels];
    uint32_t *sorted[dgrid::kLevels];
    float *spts; // coordinates in the sorted order, 4 floats a point
    void *temp;
    size_t temp_bytes;
    size_t total;
};

GridScratch carve_grid(void *base, uint32_t n, size_t temp_bytes) {
    GridScratch s{};
    char *p = static_cast<char *>(base);
    const uint64_t slots = dgrid::table_slots(n);
    auto take = [&](size_t bytes) {
        char *q = p;
        p += a256(bytes);
        return q;
    };
    s.geom = reinterpret_cast<GridGeom *>(take(sizeof(GridGeom)));
    s.tag = reinterpret_cast<uint64_t *>(take(2 * 8));
    s.counters = reinterpret_cast<unsigned long long *>(take(8 * 8));
    s.mm = reinterpret_cast<uint32_t *>(take(6 * 4));
    for (int l = 0; l < dgrid::kLevels; ++l)
        s.table[l] = reinterpret_cast<dgrid::CellEntry *>(take(sizeof(dgrid::CellEntry) * slots));
    // one order serves every level
    uint32_t *sorted = reinterpret_cast<uint32_t *>(take(4ull * n));
    for (int l = 0; l < dgrid::kLevels; ++l) s.sorted[l] = sorted;
    s.spts = reinterpret_cast<float *>(take(16ull * n));
    s.keys = reinterpret_cast<uint64_t *>(take(8ull * n));
    s.keys_sorted = reinterpret_cast<uint64_t *>(take(8ull * n));
    s.index = reinterpret_cast<uint32_t *>(take(4ull * n));
    s.status = reinterpret_cast<uint32_t *>(take(4ull * n));
    s.temp = p;
    s.temp_bytes = temp_bytes;
    s.total = (size_t)(p - static_cast<char *>(base)) + a256(temp_bytes);
    return s;
}

size_t grid_temp_bytes(uint32_t n) {
    size_t a = 0;
    const uint64_t *k = nullptr;
    uint64_t *ko = nullptr;
    const uint32_t *v = nullptr;
    uint32_t *vo = nullptr;
    if (rocprim::radix_sort_pairs(nullptr, a, k, ko, v, vo, (size_t)n, 0u, 63u) != hipSuccess)
        return 0;
    return a;
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

constexpr uint64_t kGridTag = 0x5344464f414d4752ull;

__global__ __launch_bounds__(64) void tag_kernel(uint64_t *__restrict__ tag, uint64_t a,
                                                 uint64_t b) {
    if (threadIdx.x == 0) {
        tag[0] = a;
        tag[1] = b;
    }
}

__global__ __launch_bounds__(64) void init_kernel(uint32_t *__restrict__ mm,
                                                  unsigned long long *__restrict__ counters) {
    if (mm != nullptr && threadIdx.x < 3) {
        mm[threadIdx.x] = 0xffffffffu;
        mm[3 + threadIdx.x] = 0u;
    }
    if (threadIdx.x < 8) counters[threadIdx.x] = 0ull;
}

// Bounds of the points as orderable bits: a grid-stride pass (kBboxBlocks
// blocks), a block reduction, then one atomic per block and bound (one per
// wavefront serialised ~15k same-address atomics: ~1 ms at 1M points).
constexpr uint32_t kBboxBlocks = 1024;

__global__ __launch_bounds__(256) void bbox_kernel(const float *__restrict__ p, uint32_t n,
                                                   uint32_t *__restrict__ mm) {
    __shared__ uint32_t red[4][6];
    uint32_t lo[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu}, hi[3] = {0u, 0u, 0u};
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u)
        for (int k = 0; k < 3; ++k) {
            const uint32_t o = ordered(p[3ull * i + k]);
            lo[k] = min(lo[k], o);
            hi[k] = max(hi[k], o);
        }
    for (int off = 32; off > 0; off >>= 1)
        for (int k = 0; k < 3; ++k) {
            lo[k] = min(lo[k], (uint32_t)__shfl_xor((int)lo[k], off));
            hi[k] = max(hi[k], (uint32_t)__shfl_xor((int)hi[k], off));
        }
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0)
        for (int k = 0; k < 3; ++k) {
            red[w][k] = lo[k];
            red[w][3 + k] = hi[k];
        }
    __syncthreads();
    if (threadIdx.x < 3) {
        const uint32_t k = threadIdx.x;
        atomicMin(mm + k, min(min(red[0][k], red[1][k]), min(red[2][k], red[3][k])));
        atomicMax(mm + 3 + k, max(max(red[0][3 + k], red[1][3 + k]), max(red[2][3 + k], red[3][3 + k])));
    }
}

// Morton code of each point's finest-level cell.
__global__ __launch_bounds__(256) void morton_keys_kernel(const float *__restrict__ p, uint32_t n,
                                                          GridGeom g, uint64_t *__restrict__ keys,
                                                          uint32_t *__restrict__ index) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const dgrid::GridLevel &lv = g.level[0];
    keys[i] = dgrid::morton_key(
        (uint32_t)dgrid::axis_cell((double)p[3ull * i], g.lo[0], lv.inv_h, lv.dims[0]),
        (uint32_t)dgrid::axis_cell((double)p[3ull * i + 1], g.lo[1], lv.inv_h, lv.dims[1]),
        (uint32_t)dgrid::axis_cell((double)p[3ull * i + 2], g.lo[2], lv.inv_h, lv.dims[2]));
    index[i] = i;
}

// The points' coordinates in the sorted order (x, y, z, 0).
__global__ __launch_bounds__(256) void gather_points_kernel(const float *__restrict__ p,
                                                            const uint32_t *__restrict__ order,
                                                            uint32_t n, float4 *__restrict__ out) {
    const uint32_t k = blockIdx.x * 256u + threadIdx.x;
    if (k >= n) return;
    const uint32_t j = order[k];
    out[k] = make_float4(p[3ull * j], p[3ull * j + 1], p[3ull * j + 2], 0.0f);
}

// Level-l cell keys of the points in Morton order.
__global__ __launch_bounds__(256) void level_keys_kernel(const uint64_t *__restrict__ morton,
                                                         uint32_t n, int level,
                                                         uint64_t *__restrict__ keys) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) keys[i] = dgrid::level_key(morton[i], level);
}

__global__ __launch_bounds__(256) void fill_kernel(uint32_t *__restrict__ v, uint64_t n,
                                                   uint32_t value) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) v[i] = value;
}

__global__ __launch_bounds__(256) void table_clear_kernel(dgrid::CellEntry *__restrict__ t,
                                                          uint64_t slots) {
    const uint64_t s = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (s < slots) t[s] = dgrid::CellEntry{dgrid::kEmptyKey, 0u, 0u};
}

// The first point of each run of equal keys claims a slot for its cell
// (linear probing from the key's hash) and records where the run starts.
__global__ __launch_bounds__(256) void table_insert_kernel(const uint64_t *__restrict__ ks,
                                                           uint32_t n,
                                                           dgrid::CellEntry *__restrict__ t,
                                                           uint64_t mask) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n || (i > 0 && ks[i] == ks[i - 1])) return;
    const uint64_t key = ks[i];
    for (uint64_t s = dgrid::key_hash(key) & mask;; s = (s + 1) & mask) {
        const unsigned long long prev = atomicCAS(
            reinterpret_cast<unsigned long long *>(&t[s].key), (unsigned long long)dgrid::kEmptyKey,
            (unsigned long long)key);
        if (prev == dgrid::kEmptyKey || prev == key) {
            t[s].start = i;
            return;
        }
    }
}

// The last point of each run records where the run ends.
__global__ __launch_bounds__(256) void table_end_kernel(const uint64_t *__restrict__ ks,
                                                        uint32_t n,
                                                        dgrid::CellEntry *__restrict__ t,
                                                        uint64_t mask) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n || (i + 1 < n && ks[i + 1] == ks[i])) return;
    const uint64_t key = ks[i];
    for (uint64_t s = dgrid::key_hash(key) & mask;; s = (s + 1) & mask) {
        const uint64_t k = t[s].key;
        if (k == key) {
            t[s].end = i + 1;
            return;
        }
        if (k == dgrid::kEmptyKey) return; // (the insert pass placed every key)
    }
}

// ---- certify: one wavefront per point ---------------------------------
//
// The cell of one point is shared by the 64 lanes of a wavefront: its
// planes (at most 64) in LDS, its vertices (at most 128) two per lane in
// registers.  Candidates are read 64 at a time (one grid cell per lane, the
// cell's points in rounds), filtered per lane, and the survivors clipped
// nearest first by the whole wavefront: each lane classifies its two
// vertices, a 64 x 64 bitmap of the removed vertices' directed edges gives
// the boundary edges (an edge is on the boundary when its reverse was not
// removed), and the new vertices go through a staging list into free slots.
// The decisions are those of dgrid::certify_cell and vcell::clip; every
// branch that ends a cell is taken by the whole wavefront together.

constexpr int kWavePlanes = 64;
constexpr int kWaveVerts = 128;
constexpr int kWaveNew = 64;    // new vertices one clip may make
constexpr uint32_t kFree = 0xffffffffu;

struct StagedVert {
    uint32_t planes;
    double x[3], e, r2;
};

// A cell vertex as the batch test reads it (position and error bound).
struct TestVert {
    double x[3], e;
};

struct WaveShared {
    double pn[kWavePlanes][3]; // plane normals
    double pc[kWavePlanes];    // plane offsets: x.n < c inside
    int32_t pp[kWavePlanes];   // candidate index, -1 for a box face
    uint32_t edges[kWavePlanes * kWavePlanes / 32];
    uint32_t used[2];
    uint8_t remap[kWavePlanes];
    uint16_t fresh[kWaveNew];   // wave_clip's boundary edges, ea | eb << 6
    uint8_t owner[64];          // a batch's lane whose cell range starts at each lane
    union {
        StagedVert stg[kWaveNew];     // wave_clip's new vertices
        TestVert tv[kWaveVerts];      // wave_may_cut's copy of the vertices
    };
    double mr2, blo[3], bhi[3]; // max |v|^2 and the vertices' box (the cell's bounds)
};

struct WaveCell {
    uint32_t vp[2]; // plane indices a | b << 8 | c << 16 of this lane's two slots (kFree if none)
    double vx[2][3], ve[2], vr2[2];
    int np;                         // planes in use (same in every lane)
};

__device__ __forceinline__ uint32_t wlane() { return threadIdx.x & 63u; }
__device__ __forceinline__ uint64_t wballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }
// set bits of m in the lanes below this one
__device__ __forceinline__ uint32_t wbelow(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
// Cross-lane moves without an LDS round trip.  A DPP move (`CTRL`:
// row_shr:k = 0x110 + k, row_bcast:15 = 0x142, row_bcast:31 = 0x143) reads a
// neighbouring lane's register in the same VALU instruction; lanes whose
// source lies outside their row of 16, or whose row `ROWS` leaves out, get
// `old`.  A read of one lane (`readlane`) gives a uniform value.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ uint32_t dpp_u(uint32_t old, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWS, 0xf, false);
}
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)b, hi = (uint32_t)(b >> 32);
    return __builtin_bit_cast(double, (uint64_t)dpp_u<CTRL, ROWS>(hi, hi) << 32 |
                                          dpp_u<CTRL, ROWS>(lo, lo));
}
__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int lane) {
    return (uint64_t)readlane_u((uint32_t)(v >> 32), lane) << 32 | readlane_u((uint32_t)v, lane);
}
__device__ __forceinline__ double readlane_d(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    return __builtin_bit_cast(double, (uint64_t)readlane_u((uint32_t)(b >> 32), lane) << 32 |
                                          readlane_u((uint32_t)b, lane));
}
// Maximum / minimum over the wave (every lane active): lane 15 of each row
// gathers its row by shifts of 1, 2, 4 and 8 (a lane without a source keeps
// its own value, which max and min ignore), rows 1 and 3 take rows 0 and 2,
// rows 2 and 3 take lane 31, and lane 63 holds the result.
__device__ __forceinline__ double wmaxd(double v) {
    v = fmax(v, dpp_d<0x111>(v));
    v = fmax(v, dpp_d<0x112>(v));
    v = fmax(v, dpp_d<0x114>(v));
    v = fmax(v, dpp_d<0x118>(v));
    v = fmax(v, dpp_d<0x142, 0xa>(v));
    v = fmax(v, dpp_d<0x143, 0xc>(v));
    return readlane_d(v, 63);
}
__device__ __forceinline__ double wmind(double v) {
    v = fmin(v, dpp_d<0x111>(v));
    v = fmin(v, dpp_d<0x112>(v));
    v = fmin(v, dpp_d<0x114>(v));
    v = fmin(v, dpp_d<0x118>(v));
    v = fmin(v, dpp_d<0x142, 0xa>(v));
    v = fmin(v, dpp_d<0x143, 0xc>(v));
    return readlane_d(v, 63);
}
// inclusive prefix maximum over the lanes (every lane active), as wscanu
__device__ __forceinline__ uint32_t wscanmaxu(uint32_t v) {
    v = max(v, dpp_u<0x111>(0u, v));
    v = max(v, dpp_u<0x112>(0u, v));
    v = max(v, dpp_u<0x114>(0u, v));
    v = max(v, dpp_u<0x118>(0u, v));
    v = max(v, dpp_u<0x142, 0xa>(0u, v));
    v = max(v, dpp_u<0x143, 0xc>(0u, v));
    return v;
}
// inclusive prefix sum over the lanes (every lane active): within rows by
// shifts of 1, 2, 4 and 8 (no source: 0), then rows 1 and 3 add the row
// before, rows 2 and 3 add lane 31
__device__ __forceinline__ uint32_t wscanu(uint32_t v) {
    v += dpp_u<0x111>(0u, v);
    v += dpp_u<0x112>(0u, v);
    v += dpp_u<0x114>(0u, v);
    v += dpp_u<0x118>(0u, v);
    v += dpp_u<0x142, 0xa>(0u, v);
    v += dpp_u<0x143, 0xc>(0u, v);
    return v;
}

__device__ __forceinline__ uint32_t plane_of(uint32_t vp, int k) { return (vp >> (8 * k)) & 0xffu; }

// max |v|^2 and the vertices' box grown by the largest error bound
// (dgrid::vertex_box).
__device__ void wave_bounds(WaveCell &c, WaveShared &sh) {
    double r2 = 0.0, e = 0.0, lo[3], hi[3];
    for (int k = 0; k < 3; ++k) {
        lo[k] = INFINITY;
        hi[k] = -INFINITY;
    }
    for (int s = 0; s < 2; ++s) {
        if (c.vp[s] == kFree) continue;
        r2 = fmax(r2, c.vr2[s]);
        e = fmax(e, c.ve[s]);
        for (int k = 0; k < 3; ++k) {
            lo[k] = fmin(lo[k], c.vx[s][k]);
            hi[k] = fmax(hi[k], c.vx[s][k]);
        }
    }
    // every lane stores the same values; the wave's own later reads see them
    sh.mr2 = wmaxd(r2);
    e = wmaxd(e);
    for (int k = 0; k < 3; ++k) {
        sh.blo[k] = wmind(lo[k]) - e;
        sh.bhi[k] = wmaxd(hi[k]) + e;
    }
}

__device__ void wave_init(WaveCell &c, WaveShared &sh, const double *rlo, const double *rhi) {
    const uint32_t l = wlane();
    if (l < 6) {
        const int k = (int)(l >> 1);
        for (int m = 0; m < 3; ++m) sh.pn[l][m] = 0.0;
        sh.pn[l][k] = (l & 1u) ? -1.0 : 1.0;
        sh.pc[l] = (l & 1u) ? -rlo[k] : rhi[k];
        sh.pp[l] = -1;
    }
    c.np = 6;
    c.vp[0] = c.vp[1] = kFree;
    if (l < 8) {
        // corners as vcell::cell_init makes them
        const uint32_t sx = (l >> 2) & 1u, sy = (l >> 1) & 1u, sz = l & 1u;
        const uint32_t px = sx, py = 2u + sy, pz = 4u + sz;
        c.vp[0] = ((sx + sy + sz) & 1u) == 0 ? (px | py << 8 | pz << 16)
                                              : (px | pz << 8 | py << 16);
        c.vx[0][0] = sx ? rlo[0] : rhi[0];
        c.vx[0][1] = sy ? rlo[1] : rhi[1];
        c.vx[0][2] = sz ? rlo[2] : rhi[2];
        c.ve[0] = 0.0;
        c.vr2[0] = c.vx[0][0] * c.vx[0][0] + c.vx[0][1] * c.vx[0][1] + c.vx[0][2] * c.vx[0][2];
    }
    wave_bounds(c, sh);
    __syncthreads();
}

// Drops planes no vertex uses (vcell::compact_planes); false if all are used.
__device__ bool wave_compact_planes(WaveCell &c, WaveShared &sh) {
    const uint32_t l = wlane();
    if (l < 2) sh.used[l] = 0u;
    __syncthreads();
    for (int s = 0; s < 2; ++s)
        if (c.vp[s] != kFree)
            for (int k = 0; k < 3; ++k) {
                const uint32_t q = plane_of(c.vp[s], k);
                atomicOr(&sh.used[q >> 5], 1u << (q & 31u));
            }
    __syncthreads();
    const uint64_t used = (uint64_t)sh.used[0] | ((uint64_t)sh.used[1] << 32);
    const bool mine = (used >> l) & 1ull;
    const uint32_t to = wbelow(used);
    double n0 = 0.0, n1 = 0.0, n2 = 0.0, pc = 0.0;
    int32_t pp = 0;
    if (mine) {
        n0 = sh.pn[l][0];
        n1 = sh.pn[l][1];
        n2 = sh.pn[l][2];
        pc = sh.pc[l];
        pp = sh.pp[l];
        sh.remap[l] = (uint8_t)to;
    }
    __syncthreads();
    if (mine) {
        sh.pn[to][0] = n0;
        sh.pn[to][1] = n1;
        sh.pn[to][2] = n2;
        sh.pc[to] = pc;
        sh.pp[to] = pp;
    }
    for (int s = 0; s < 2; ++s)
        if (c.vp[s] != kFree)
            c.vp[s] = (uint32_t)sh.remap[plane_of(c.vp[s], 0)] |
                      (uint32_t)sh.remap[plane_of(c.vp[s], 1)] << 8 |
                      (uint32_t)sh.remap[plane_of(c.vp[s], 2)] << 16;
    c.np = __popcll(used);
    __syncthreads();
    return c.np < kWavePlanes;
}

// Clips the cell by the bisector of o and `point` (relative position q,
// qc = |q|^2 / 2).  0: the plane misses the cell, 1: cut, 2: undecided,
// 3: over capacity.  The whole wavefront calls it with the same arguments.
__device__ int wave_clip(WaveCell &c, WaveShared &sh, const double *q, double qc,
                         int32_t point) {
    const uint32_t l = wlane();
    if (c.np >= kWavePlanes && !wave_compact_planes(c, sh)) return 3;
    const double qn = vcell::dabs(q[0]) + vcell::dabs(q[1]) + vcell::dabs(q[2]);
    bool out[2] = {false, false}, undecided = false;
    for (int s = 0; s < 2; ++s) {
        if (c.vp[s] == kFree) continue;
        const double *x = c.vx[s];
        const double sd = x[0] * q[0] + x[1] * q[1] + x[2] * q[2] - qc;
        const double bound =
            c.ve[s] * qn + 4.0 * vcell::kEps *
                               (vcell::dabs(x[0] * q[0]) + vcell::dabs(x[1] * q[1]) +
                                vcell::dabs(x[2] * q[2]) + qc);
        if (sd < -bound || sd > bound) {
            out[s] = sd > 0.0;
            continue;
        }
        // the exact decision (vcell::outside)
        const uint32_t a = plane_of(c.vp[s], 0), b = plane_of(c.vp[s], 1),
                       cc = plane_of(c.vp[s], 2);
        int sg;
        if (sh.pp[a] >= 0 && sh.pp[b] >= 0 && sh.pp[cc] >= 0) {
            const double A[3] = {sh.pn[a][0], sh.pn[a][1], sh.pn[a][2]};
            const double B[3] = {sh.pn[b][0], sh.pn[b][1], sh.pn[b][2]};
            const double Cn[3] = {sh.pn[cc][0], sh.pn[cc][1], sh.pn[cc][2]};
            sg = vcell::in_sphere(A, B, Cn, q);
        } else {
            const double scale =
                (vcell::dabs(x[0]) + vcell::dabs(x[1]) + vcell::dabs(x[2])) * qn +
                vcell::dabs(qc);
            sg = vcell::dabs(sd) <= 1e-9 * scale ? 0 : (sd > 0.0 ? 1 : -1);
        }
        if (sg == 0) undecided = true;
        out[s] = sg > 0;
    }
    if (wballot(undecided)) return 2;
    const uint64_t o0 = wballot(out[0]), o1 = wballot(out[1]);
    if ((o0 | o1) == 0ull) return 0;
    const uint64_t a0 = wballot(c.vp[0] != kFree), a1 = wballot(c.vp[1] != kFree);
    if (o0 == a0 && o1 == a1) return 2; // every vertex cut: o itself would go
    // the removed vertices' directed edges
    sh.edges[l] = 0u;
    sh.edges[l + 64] = 0u;
    __syncthreads();
    for (int s = 0; s < 2; ++s)
        if (out[s])
            for (int k = 0; k < 3; ++k) {
                const uint32_t ea = plane_of(c.vp[s], k), eb = plane_of(c.vp[s], (k + 1) % 3);
                const uint32_t bit = ea * kWavePlanes + eb;
                atomicOr(&sh.edges[bit >> 5], 1u << (bit & 31u));
            }
    __syncthreads();
    // boundary edges (reverse not removed): one new vertex each, listed as
    // 16-bit {ea, eb} fields of one register (no indexed array: it would
    // live in scratch memory)
    uint64_t fresh = 0;
    uint32_t fresh5 = 0, nf = 0;
    for (int s = 0; s < 2; ++s)
        if (out[s])
            for (int k = 0; k < 3; ++k) {
                const uint32_t ea = plane_of(c.vp[s], k), eb = plane_of(c.vp[s], (k + 1) % 3);
                const uint32_t rev = eb * kWavePlanes + ea;
                if (!((sh.edges[rev >> 5] >> (rev & 31u)) & 1u)) {
                    if (nf < 5)
                        fresh |= (uint64_t)(ea | eb << 6) << (12u * nf);
                    else
                        fresh5 = ea | eb << 6;
                    ++nf;
                }
            }
    const uint32_t incl = wscanu(nf);
    const uint32_t total = readlane_u(incl, 63);
    const uint32_t base = incl - nf;
    const uint32_t kept = __popcll(a0 & ~o0) + __popcll(a1 & ~o1);
    if (total > (uint32_t)kWaveNew || kept + total > (uint32_t)kWaveVerts) return 3;
    const uint32_t np = (uint32_t)c.np;
    vcell::Plane P;
    P.n[0] = q[0];
    P.n[1] = q[1];
    P.n[2] = q[2];
    P.c = qc;
    P.point = point;
    // the boundary edges go to one lane each (lane t makes new vertex t), so
    // the vertices are made side by side rather than up to six after another
    // on the lanes that found them
    for (uint32_t t = 0; t < nf; ++t)
        sh.fresh[base + t] = (uint16_t)(t < 5 ? (uint32_t)(fresh >> (12u * t)) & 0xfffu : fresh5);
    __syncthreads();
    bool bad = false;
    if (l < total) {
        const uint32_t f = sh.fresh[l];
        const uint32_t ea = f & 63u, eb = f >> 6;
        vcell::Plane A, B;
        for (int k = 0; k < 3; ++k) {
            A.n[k] = sh.pn[ea][k];
            B.n[k] = sh.pn[eb][k];
        }
        A.c = sh.pc[ea];
        B.c = sh.pc[eb];
        A.point = sh.pp[ea];
        B.point = sh.pp[eb];
        StagedVert &v = sh.stg[l];
        double x[3], e = 0.0;
        if (!vcell::meet(A, B, P, x, &e)) {
            bad = true;
        } else {
            v.planes = ea | eb << 8 | np << 16;
            v.x[0] = x[0];
            v.x[1] = x[1];
            v.x[2] = x[2];
            v.e = e;
            v.r2 = x[0] * x[0] + x[1] * x[1] + x[2] * x[2];
        }
    }
    if (wballot(bad)) {
        __syncthreads();
        return 2;
    }
    for (int s = 0; s < 2; ++s)
        if (out[s]) c.vp[s] = kFree;
    if (l == 0) {
        sh.pn[np][0] = q[0];
        sh.pn[np][1] = q[1];
        sh.pn[np][2] = q[2];
        sh.pc[np] = qc;
        sh.pp[np] = point;
    }
    c.np = (int)np + 1;
    __syncthreads();
    // free slots take the new vertices, slot 0 of every lane first
    const uint64_t f0 = ~wballot(c.vp[0] != kFree), f1 = ~wballot(c.vp[1] != kFree);
    for (int s = 0; s < 2; ++s) {
        if (c.vp[s] != kFree) continue;
        const uint32_t rank = s == 0 ? wbelow(f0) : (uint32_t)__popcll(f0) + wbelow(f1);
        if (rank >= total) continue;
        const StagedVert &v = sh.stg[rank];
        c.vp[s] = v.planes;
        c.vx[s][0] = v.x[0];
        c.vx[s][1] = v.x[1];
        c.vx[s][2] = v.x[2];
        c.ve[s] = v.e;
        c.vr2[s] = v.r2;
    }
    __syncthreads();
    return 1;
}

// The lanes whose candidate plane (relative position q, qc = |q|^2 / 2;
// `mine`: the lane holds one) may cut the cell: each lane tests its plane
// against every vertex (copied to LDS), and a plane that leaves every
// vertex inside by more than the bound wave_clip uses (the vertex's error
// bound and the dot product's rounding) misses the cell, and every cell the
// clips that follow make (they only shrink it).  One pass for a batch of
// candidates in place of a wave_clip call each, most of which find no cut
// where the cell is large.
__device__ uint64_t wave_may_cut(const WaveCell &c, WaveShared &sh, bool mine, const double *q,
                                 double qc) {
    const uint64_t a0 = wballot(c.vp[0] != kFree), a1 = wballot(c.vp[1] != kFree);
    const uint32_t n0 = (uint32_t)__popcll(a0), nv = n0 + (uint32_t)__popcll(a1);
    for (int s = 0; s < 2; ++s) {
        if (c.vp[s] == kFree) continue;
        TestVert &t = sh.tv[s == 0 ? wbelow(a0) : n0 + wbelow(a1)];
        t.x[0] = c.vx[s][0];
        t.x[1] = c.vx[s][1];
        t.x[2] = c.vx[s][2];
        t.e = c.ve[s];
    }
    __syncthreads();
    bool cut = false;
    if (mine) {
        const double qn = vcell::dabs(q[0]) + vcell::dabs(q[1]) + vcell::dabs(q[2]);
        for (uint32_t v = 0; v < nv && !cut; ++v) {
            const double *x = sh.tv[v].x;
            const double sd = x[0] * q[0] + x[1] * q[1] + x[2] * q[2] - qc;
            const double bound =
                sh.tv[v].e * qn + 4.0 * vcell::kEps *
                                      (vcell::dabs(x[0] * q[0]) + vcell::dabs(x[1] * q[1]) +
                                       vcell::dabs(x[2] * q[2]) + qc);
            cut = !(sd < -bound);
        }
    }
    const uint64_t m = wballot(cut);
    __syncthreads(); // the copy is read before wave_clip stages vertices there
    return m;
}

// The cells of the rings r = 0 .. kMaxRing around a grid cell, ring by ring
// (ring r: the (2r+1)^3 - (2r-1)^3 cells at Chebyshev distance r, entries
// (2r-1)^3 .. (2r+1)^3 - 1), each ring in z, y, x order; an entry packs
// (dx + 8) | (dy + 8) << 4 | (dz + 8) << 8.  A pass over a ring's cells then
// takes only its shell, not the whole cube around it (r = 3: 4 passes of 64
// lanes instead of 6), and no lane divides by the ring's side.
struct RingCells {
    static constexpr int kSide = 2 * dgrid::kMaxRing + 1;
    uint16_t v[kSide * kSide * kSide];
    constexpr RingCells() : v() {
        int k = 0;
        for (int r = 0; r <= dgrid::kMaxRing; ++r)
            for (int dz = -r; dz <= r; ++dz)
                for (int dy = -r; dy <= r; ++dy)
                    for (int dx = -r; dx <= r; ++dx) {
                        const int ax = dx < 0 ? -dx : dx, ay = dy < 0 ? -dy : dy,
                                  az = dz < 0 ? -dz : dz;
                        const int m = ax > ay ? (ax > az ? ax : az) : (ay > az ? ay : az);
                        if (m == r)
                            v[k++] = (uint16_t)((dx + 8) | (dy + 8) << 4 | (dz + 8) << 8);
                    }
    }
};
static_assert(dgrid::kMaxRing < 8, "ring offsets fit 4 bits");
__constant__ RingCells kRingCells = RingCells();

// The clipping box of an exhaustive certification: the bounding box grown by
// this many times its extent, so that the hull cells' Voronoi vertices
// (circumcentres of Delaunay tetrahedra on the hull, some ~1e6 extents away
// for nearly flat ones) lie inside it.
constexpr double kExhaustiveBox = 1e8;

// Candidates that survive the per-lane filters in a batch before the batch
// test pays for itself (a wave_clip call that finds no cut costs about as
// much as the test over a typical cell's vertices).
constexpr int kBatchTestMin = 3;

__device__ bool wave_touches_box(const WaveCell &c, const WaveShared &sh) {
    bool t = false;
    for (int s = 0; s < 2; ++s)
        if (c.vp[s] != kFree)
            for (int k = 0; k < 3; ++k) t = t || sh.pp[plane_of(c.vp[s], k)] < 0;
    return wballot(t) != 0ull;
}

// counters: 0 report rows asked for, 1 open points, 2 undecided cells,
// 3 cells over the fixed capacity, 4 coincident point pairs seen (twice).
// One 64-thread block per point (per entry of `query` when it is given).  Four waves per SIMD (128 VGPRs, 200 bytes
// of spills per lane) run it ~20% faster than the two its natural register
// count (203) allows; three (168 VGPRs, 40 bytes) run it ~10% slower than
// four.  What is uniform over the wave and indexed at run time (the grid
// cell and searched rings per level) or needed by every lane (the cell's
// bounds) lives in LDS, not in per-lane registers or scratch.
template <bool EXHAUSTIVE>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(4))) void certify_kernel(const float *__restrict__ p, uint32_t n,
                                                     GridView gv, uint32_t *__restrict__ reports,
                                                     uint64_t report_capacity,
                                                     unsigned long long *__restrict__ counters,
                                                     uint32_t *__restrict__ open,
                                                     uint32_t *__restrict__ status_out,
                                                     const uint32_t *__restrict__ query,
                                                     uint32_t max_candidates) {
    __shared__ WaveShared sh;
    // the point's grid cell and searched rings per level (uniform over the
    // wave; indexed by level, so kept in LDS rather than scratch memory)
    __shared__ int hc[dgrid::kLevels][3];
    __shared__ int rings[dgrid::kLevels];
    const uint32_t i = query ? query[blockIdx.x] : blockIdx.x;
    if (i >= n) return;
    const uint32_t l = wlane();
    const GridGeom &g = gv.g;
    const double o[3] = {(double)p[3ull * i], (double)p[3ull * i + 1], (double)p[3ull * i + 2]};
    WaveCell c;
    {
        double rlo[3], rhi[3];
        for (int k = 0; k < 3; ++k) {
            rlo[k] = g.box_lo[k] - o[k];
            rhi[k] = g.box_hi[k] - o[k];
        }
        wave_init(c, sh, rlo, rhi);
    }
    if (l < (uint32_t)dgrid::kLevels) {
        rings[l] = -1;
        for (int k = 0; k < 3; ++k)
            hc[l][k] = dgrid::axis_cell(o[k], g.lo[k], g.level[l].inv_h, g.level[l].dims[k]);
    }
    __syncthreads();
    uint32_t st = vcell::kOpen, examined = 0;
    bool decided = false, coincident = false;
    // dgrid::first_level with every level's lookup in flight at once: lane
    // l < kLevels - 1 looks up the point's cell of level l
    int l0 = dgrid::kLevels - 1;
    {
        uint32_t b = 0, e = 0;
        if (l < (uint32_t)dgrid::kLevels - 1u)
            dgrid::cell_range(gv, (int)l, (uint32_t)hc[l][0], (uint32_t)hc[l][1],
                              (uint32_t)hc[l][2], b, e);
        const uint64_t two = wballot(e - b >= 2u);
        if (two) l0 = __builtin_ctzll(two);
    }
    for (int lev = l0; lev < dgrid::kLevels && !decided; ++lev) {
        const dgrid::GridLevel &lv = g.level[lev];
        const uint32_t *sorted = gv.sorted[lev];
        const int *h = hc[lev];
        // ring 1 takes ring 0 (the point's own cell) in with it: after ring 0
        // alone the search always went on (no point lies beyond 0 cells yet,
        // short of a grid of one cell, where ring 1 holds no cell)
        for (int r = 1; r <= dgrid::kMaxRing && !decided; ++r) {
            const uint32_t first = r == 1 ? 0u : (uint32_t)((2 * r - 1) * (2 * r - 1) * (2 * r - 1));
            const uint32_t cells = (uint32_t)((2 * r + 1) * (2 * r + 1) * (2 * r + 1)) - first;
            for (uint32_t base = 0; base < cells && !decided; base += 64) {
                // one grid cell of the ring's shell per lane
                const uint32_t t = base + l;
                uint32_t b = 0, e = 0;
                if (t < cells) {
                    const uint32_t d = kRingCells.v[first + t];
                    const int cx = h[0] + (int)(d & 15u) - 8, cy = h[1] + (int)(d >> 4 & 15u) - 8,
                              cz = h[2] + (int)(d >> 8) - 8;
                    if (cx >= 0 && cx < (int)lv.dims[0] && cy >= 0 && cy < (int)lv.dims[1] &&
                        cz >= 0 && cz < (int)lv.dims[2])
                        dgrid::cell_range(gv, lev, (uint32_t)cx, (uint32_t)cy, (uint32_t)cz, b,
                                          e);
                }
                // the batch's points, 64 at a time in cell order: lane l
                // takes point f0 + l of the concatenated cell ranges (its
                // cell: the first lane whose inclusive prefix exceeds it)
                const uint32_t cnt = e - b;
                const uint32_t incl = wscanu(cnt);
                const uint32_t total = readlane_u(incl, 63);
                examined += total;
                if (examined > max_candidates) {
                    decided = true;
                    break;
                }
                for (uint32_t f0 = 0; f0 < total && !decided; f0 += 64) {
                    const uint32_t f = f0 + l;
                    // each cell range starting in this window marks its first
                    // lane with its own lane; a running maximum over the lanes
                    // carries it on (the ranges follow one another in lane
                    // order), from the range holding f0 (lanes whose ranges
                    // end at or before f0 are below it); lanes past `total`
                    // keep the last range
                    sh.owner[l] = 0u;
                    __syncthreads();
                    const uint32_t ex = incl - cnt;
                    if (cnt > 0u && ex > f0 && ex < f0 + 64u) sh.owner[ex - f0] = (uint8_t)l;
                    __syncthreads();
                    const uint32_t owner =
                        wscanmaxu(max((uint32_t)sh.owner[l],
                                      (uint32_t)__popcll(wballot(incl <= f0))));
                    const uint32_t ob = (uint32_t)__shfl((int)b, (int)owner, 64);
                    const uint32_t oex = (uint32_t)__shfl((int)(incl - cnt), (int)owner, 64);
                    bool surv = false, dup = false;
                    double q[3] = {0.0, 0.0, 0.0}, d2 = INFINITY;
                    uint32_t j = 0;
                    if (f < total) {
                        j = sorted[ob + (f - oex)];
                        if (j != i) {
                            const float4 sp =
                                reinterpret_cast<const float4 *>(gv.spts)[ob + (f - oex)];
                            const double x[3] = {(double)sp.x, (double)sp.y, (double)sp.z};
                            q[0] = x[0] - o[0];
                            q[1] = x[1] - o[1];
                            q[2] = x[2] - o[2];
                            d2 = q[0] * q[0] + q[1] * q[1] + q[2] * q[2];
                            if (d2 == 0.0) {
                                dup = true;
                            } else if (d2 <= 4.0 * sh.mr2 * (1.0 + 1e-9)) {
                                double reach_q = 0.0, mag = d2;
                                for (int m = 0; m < 3; ++m) {
                                    const double bb = q[m] > 0.0 ? sh.bhi[m] : sh.blo[m];
                                    reach_q += bb * q[m];
                                    mag += vcell::dabs(bb * q[m]);
                                }
                                surv = !(reach_q < 0.5 * d2 - 1e-14 * mag) &&
                                       !(lev > l0 && dgrid::searched(g, lev, x, hc, rings));
                            }
                        }
                    }
                    if (wballot(dup)) {
                        coincident = true;
                        st = vcell::kUncertain;
                        decided = true;
                        break;
                    }
                    uint64_t m = wballot(surv);
                    if (__popcll(m) >= kBatchTestMin) m = wave_may_cut(c, sh, surv, q, 0.5 * d2);
                    bool clipped = false;
                    while (m) {
                        // nearest first
                        const bool mine = (m >> l) & 1ull;
                        const double dm = wmind(mine ? d2 : INFINITY);
                        const uint64_t hit = wballot(mine && d2 == dm);
                        const int src = __builtin_ctzll(hit);
                        m &= ~(1ull << src);
                        const double qq[3] = {readlane_d(q[0], src), readlane_d(q[1], src),
                                              readlane_d(q[2], src)};
                        const double dd = readlane_d(d2, src);
                        const int32_t jj = (int32_t)readlane_u(j, src);
                        // the cell may have shrunk since the filter
                        if (dd > 4.0 * sh.mr2 * (1.0 + 1e-9)) continue;
                        double reach_q = 0.0, mag = dd;
                        for (int mm = 0; mm < 3; ++mm) {
                            const double bb = qq[mm] > 0.0 ? sh.bhi[mm] : sh.blo[mm];
                            reach_q += bb * qq[mm];
                            mag += vcell::dabs(bb * qq[mm]);
                        }
                        if (reach_q < 0.5 * dd - 1e-14 * mag) continue;
                        const int rc = wave_clip(c, sh, qq, 0.5 * dd, jj);
                        if (rc >= 2) {
                            st = rc == 2 ? vcell::kUncertain : vcell::kOverflow;
                            decided = true;
                            break;
                        }
                        clipped = clipped || rc == 1;
                    }
                    // the batch's clips leave the bounds of the cell before them, which
                    // still hold it (a clip only shrinks a cell); tightened once per batch
                    if (clipped && !decided) wave_bounds(c, sh);
                }
            }
            if (decided) break;
            if (l == 0) rings[lev] = r;
            __syncthreads();
            // every point not yet seen lies r cells of this level away or more
            const bool all = h[0] - r <= 0 && h[0] + r >= (int)lv.dims[0] - 1 && h[1] - r <= 0 &&
                             h[1] + r >= (int)lv.dims[1] - 1 && h[2] - r <= 0 &&
                             h[2] + r >= (int)lv.dims[2] - 1;
            const double reach = (double)r * lv.h - g.slack;
            const double reach2 = all ? INFINITY : (reach > 0.0 ? reach * reach : 0.0);
            const bool box = wave_touches_box(c, sh);
            if (4.0 * sh.mr2 * (1.0 + 1e-9) < reach2) {
                st = box ? vcell::kOpen : vcell::kCertified;
                decided = true;
                break;
            }
            if (r >= dgrid::kBoxRing && box) {
                if (lev == l0) break;
                decided = true;
                break;
            }
            if (r >= dgrid::kMinRing &&
                4.0 * sh.mr2 * (1.0 + 1e-9) > (dgrid::kMaxRing * lv.h) * (dgrid::kMaxRing * lv.h))
                break;
        }
    }
    // exhaustive: a cell the grid search leaves open is clipped by every point
    // of the set (the batch test drops the planes that miss it); it is then
    // exact, certified if no box face is left, else a hull cell whose
    // vertices off the box faces (circumcentres inside the box) are reported
    // as well
    bool hull_cell = false;
    if (EXHAUSTIVE && st == vcell::kOpen && !coincident) {
        bool failed = false;
        const uint32_t *order = gv.sorted[0];
        for (uint32_t base = 0; base < n && !failed; base += 64u) {
            // the points in the grid's (Morton) order
            const uint32_t k = base + l;
            const uint32_t j = k < n ? order[k] : i;
            bool surv = false, dup = false;
            double q[3] = {0.0, 0.0, 0.0}, d2 = INFINITY;
            if (j != i) {
                const float4 sp = reinterpret_cast<const float4 *>(gv.spts)[k];
                q[0] = (double)sp.x - o[0];
                q[1] = (double)sp.y - o[1];
                q[2] = (double)sp.z - o[2];
                d2 = q[0] * q[0] + q[1] * q[1] + q[2] * q[2];
                if (d2 == 0.0) {
                    dup = true;
                } else if (d2 <= 4.0 * sh.mr2 * (1.0 + 1e-9)) {
                    double reach_q = 0.0, mag = d2;
                    for (int mm = 0; mm < 3; ++mm) {
                        const double bb = q[mm] > 0.0 ? sh.bhi[mm] : sh.blo[mm];
                        reach_q += bb * q[mm];
                        mag += vcell::dabs(bb * q[mm]);
                    }
                    surv = !(reach_q < 0.5 * d2 - 1e-14 * mag);
                }
            }
            if (wballot(dup)) {
                coincident = true;
                st = vcell::kUncertain;
                failed = true;
                break;
            }
            uint64_t m = wballot(surv);
            if (__popcll(m) >= kBatchTestMin) m = wave_may_cut(c, sh, surv, q, 0.5 * d2);
            bool clipped = false;
            while (m) {
                const bool mine = (m >> l) & 1ull;
                const double dm = wmind(mine ? d2 : INFINITY);
                const uint64_t hit = wballot(mine && d2 == dm);
                const int src = __builtin_ctzll(hit);
                m &= ~(1ull << src);
                const double qq[3] = {readlane_d(q[0], src), readlane_d(q[1], src),
                                      readlane_d(q[2], src)};
                const double dd = readlane_d(d2, src);
                const int32_t jj = (int32_t)readlane_u(j, src);
                // a point the grid search clipped by already: its plane holds
                // vertices of the cell, which the exact test cannot place
                if (wballot((int)l < c.np && sh.pp[l] == jj)) continue;
                const int rc = wave_clip(c, sh, qq, 0.5 * dd, jj);
                if (rc >= 2) {
                    st = rc == 2 ? vcell::kUncertain : vcell::kOverflow;
                    failed = true;
                    break;
                }
                clipped = clipped || rc == 1;
            }
            // the batch's clips leave the bounds of the cell before them, which
            // still hold it (a clip only shrinks a cell); tightened once per batch
            if (clipped && !failed) wave_bounds(c, sh);
        }
        if (!failed) {
            hull_cell = wave_touches_box(c, sh);
            st = hull_cell ? vcell::kOpen : vcell::kCertified;
        }
    }
    if (l == 0) {
        status_out[i] = st;
        if (coincident) atomicAdd(counters + 4, 1ull);
    }
    if (hull_cell) {
        // the vertices of three bisectors: Delaunay tetrahedra of the set
        bool fin[2] = {false, false};
        for (int s = 0; s < 2; ++s)
            fin[s] = c.vp[s] != kFree && sh.pp[plane_of(c.vp[s], 0)] >= 0 &&
                     sh.pp[plane_of(c.vp[s], 1)] >= 0 && sh.pp[plane_of(c.vp[s], 2)] >= 0;
        const uint64_t a0 = wballot(fin[0]), a1 = wballot(fin[1]);
        const unsigned long long nv = (unsigned long long)(__popcll(a0) + __popcll(a1));
        unsigned long long at = 0;
        if (l == 0) at = atomicAdd(counters, nv);
        at = readlane_u64(at, 0);
        if (at + nv <= report_capacity)
            for (int s = 0; s < 2; ++s) {
                if (!fin[s]) continue;
                const uint32_t idx = s == 0 ? wbelow(a0) : (uint32_t)__popcll(a0) + wbelow(a1);
                uint32_t *row = reports + 4ull * (at + idx);
                row[0] = i;
                row[1] = (uint32_t)sh.pp[plane_of(c.vp[s], 0)];
                row[2] = (uint32_t)sh.pp[plane_of(c.vp[s], 1)];
                row[3] = (uint32_t)sh.pp[plane_of(c.vp[s], 2)];
            }
        if (l == 0) {
            const unsigned long long at2 = atomicAdd(counters + 1, 1ull);
            open[at2] = i;
        }
    } else if (st == vcell::kCertified) {
        const uint64_t a0 = wballot(c.vp[0] != kFree), a1 = wballot(c.vp[1] != kFree);
        const unsigned long long nv = (unsigned long long)(__popcll(a0) + __popcll(a1));
        unsigned long long at = 0;
        if (l == 0) at = atomicAdd(counters, nv);
        at = readlane_u64(at, 0);
        if (at + nv <= report_capacity)
            for (int s = 0; s < 2; ++s) {
                if (c.vp[s] == kFree) continue;
                const uint32_t idx = s == 0 ? wbelow(a0) : (uint32_t)__popcll(a0) + wbelow(a1);
                uint32_t *row = reports + 4ull * (at + idx);
                row[0] = i;
                row[1] = (uint32_t)sh.pp[plane_of(c.vp[s], 0)];
                row[2] = (uint32_t)sh.pp[plane_of(c.vp[s], 1)];
                row[3] = (uint32_t)sh.pp[plane_of(c.vp[s], 2)];
            }
    } else if (l == 0) {
        const unsigned long long at = atomicAdd(counters + 1, 1ull);
        open[at] = i;
        if (st == vcell::kUncertain) atomicAdd(counters + 2, 1ull);
        if (st == vcell::kOverflow) atomicAdd(counters + 3, 1ull);
    }
}

// One 64-thread block per candidate t: 1 if no point lies strictly inside
// its circumsphere, 0 if one does, 2 if the tetrahedron is invalid or flat
// or, with none inside, a certified point's sign is undecided
// (dgrid::sphere_empty).  The lanes take the sphere's cell columns in turn
// and stop together once one finds a point inside.
__global__ __launch_bounds__(64) void keep_empty_kernel(const float *__restrict__ p, uint32_t n,
                                                        GridView gv,
                                                        const uint32_t *__restrict__ cand,
                                                        uint32_t m,
                                                        const uint32_t *__restrict__ status,
                                                        uint32_t *__restrict__ keep) {
    const uint32_t t = blockIdx.x;
    if (t >= m) return;
    const uint32_t l = threadIdx.x & 63u;
    uint32_t v[4];
    bool valid = true;
    for (int k = 0; k < 4; ++k) {
        v[k] = cand[4ull * t + k];
        valid = valid && v[k] < n;
    }
    dgrid::Sphere S;
    if (!valid || !dgrid::sphere_setup(p, v, gv, S)) {
        if (l == 0) keep[t] = 2u;
        return;
    }
    const uint32_t cols = dgrid::sphere_columns(S);
    // first the 8 x 8 columns around the centre's (where a point inside is
    // likeliest), then all of them in row-major order from 32 before it (a
    // candidate that is not Delaunay is rejected in the first rounds: the
    // corner-first order made the merge of C4's incremental rebuild 67 ms
    // against 46)
    uint32_t c0 = 0;
    bool inside = false, undecided = false;
    {
        const dgrid::GridLevel &lv = gv.g.level[S.l];
        const int ny = S.hi_c[1] - S.lo_c[1] + 1, nz = S.hi_c[2] - S.lo_c[2] + 1;
        const int cy = dgrid::axis_cell(S.o[1] + S.ctr[1], gv.g.lo[1], lv.inv_h, lv.dims[1]);
        const int cz = dgrid::axis_cell(S.o[2] + S.ctr[2], gv.g.lo[2], lv.inv_h, lv.dims[2]);
        const int ry = cy < S.lo_c[1] ? 0 : (cy > S.hi_c[1] ? ny - 1 : cy - S.lo_c[1]);
        const int rz = cz < S.lo_c[2] ? 0 : (cz > S.hi_c[2] ? nz - 1 : cz - S.lo_c[2]);
        c0 = ((uint32_t)ry + (uint32_t)rz * (uint32_t)ny + cols - (32u % cols)) % cols;
        if (cols > 64u) {
            const int y = ry - 4 + (int)(l & 7u), z = rz - 4 + (int)(l >> 3);
            if (y >= 0 && y < ny && z >= 0 && z < nz) {
                const uint32_t r =
                    dgrid::sphere_scan_column(p, v, gv, status, S, (uint32_t)(y + z * ny));
                inside = r == 0u;
                undecided = r == 2u;
            }
            inside = __builtin_amdgcn_ballot_w64(inside) != 0ull;
        }
    }
    for (uint32_t base = 0; !inside && base < cols; base += 64) {
        if (base + l < cols) {
            const uint32_t r =
                dgrid::sphere_scan_column(p, v, gv, status, S, (base + l + c0) % cols);
            inside = r == 0u;
            undecided = undecided || r == 2u;
        }
        if (__builtin_amdgcn_ballot_w64(inside)) {
            inside = true;
            break;
        }
    }
    undecided = __builtin_amdgcn_ballot_w64(undecided) != 0ull;
    if (l == 0) keep[t] = inside ? 0u : (undecided ? 2u : 1u);
}

// Incremental rebuild, kCheckLanes lanes per tetrahedron t of the previous
// tetrahedralisation over the moved points: keep[t] = 1 when no point lies
// strictly inside its circumsphere and every sign is decided (status: every
// point clean), else 0.  The vertices of a tetrahedron not kept are marked
// dirty (1), the three vertices of each face without a neighbour (the old
// hull) dirty and on the hull (2).
// The sphere is scanned on the finest level where it spans at most 6 x 6
// columns (at C3's 1M points, with one lane per tetrahedron, 29.5 ms for
// 6.7M tetrahedra, against 55 ms at 3 x 3, 43 ms at 4 x 4 and 53 ms at
// 8 x 8); the group's lanes take its columns in turn (2-8 lanes a group
// ~19 ms, one lane 25 ms, 16 lanes 21 ms, 64 lanes 33 ms).  errors[0]: rows
// with a vertex out of range.
constexpr uint32_t kCheckLanes = 4;

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void check_kernel(const float *__restrict__ p, uint32_t n,
                                                    GridView gv,
                                                    const uint32_t *__restrict__ status,
                                                    const uint32_t *__restrict__ tets,
                                                    const int32_t *__restrict__ nbr, uint64_t T,
                                                    uint32_t *__restrict__ keep,
                                                    uint32_t *__restrict__ dirty,
                                                    unsigned long long *__restrict__ errors) {
    static_assert(64u % kCheckLanes == 0u, "groups within a wavefront");
    const uint64_t t = ((uint64_t)blockIdx.x * 256u + threadIdx.x) / kCheckLanes;
    const uint32_t sub = threadIdx.x % kCheckLanes;
    const bool live = t < T;
    uint32_t v[4] = {0u, 0u, 0u, 0u};
    bool valid = live;
    if (live)
        for (int k = 0; k < 4; ++k) {
            v[k] = tets[4 * t + k];
            valid = valid && v[k] < n;
        }
    // a sphere still wider than 8 x 8 columns of the coarsest level (the
    // huge spheres of flat tetrahedra at the hull) is not scanned: its
    // tetrahedron is not kept, which only adds dirty points
    dgrid::Sphere S;
    bool kept = valid && dgrid::sphere_setup(p, v, gv, S, 36.0);
    const uint32_t cols = kept ? dgrid::sphere_columns(S) : 0u;
    kept = kept && cols <= 64u;
    bool hit = false;
    for (uint32_t c = sub; kept && !hit && c < cols; c += kCheckLanes)
        hit = dgrid::sphere_scan_column(p, v, gv, status, S, c) != 1u;
    // the group's lanes are consecutive bits of the wavefront's ballot
    const uint64_t hits = __builtin_amdgcn_ballot_w64(hit);
    const uint32_t first = (threadIdx.x & 63u) & ~(kCheckLanes - 1u);
    const uint64_t group = kCheckLanes == 64u ? ~0ull : ((1ull << kCheckLanes) - 1ull) << first;
    kept = kept && (hits & group) == 0ull;
    if (!live || sub != 0u) return;
    if (!valid) {
        keep[t] = 0u;
        atomicAdd(errors, 1ull);
        return;
    }
    keep[t] = kept ? 1u : 0u;
    if (!kept)
        for (int k = 0; k < 4; ++k) atomicMax(dirty + v[k], 1u);
    for (int j = 0; j < 4; ++j) {
        if (nbr[4 * t + j] >= 0) continue;
        for (int k = 0; k < 4; ++k)
            if (k != j) atomicMax(dirty + v[k], 2u);
    }
}

// Row t of [reports; candidates; verified] survives: a report (i, a, b, c)
// when i is its lowest certified vertex, a candidate when keep says so, a
// verified tetrahedron always.
// errors: 0 a report index out of range, 1 an undecided candidate.
__global__ __launch_bounds__(256) void select_kernel(const uint32_t *__restrict__ reports,
                                                     uint64_t nr,
                                                     const uint32_t *__restrict__ keep,
                                                     uint64_t m,
                                                     const uint32_t *__restrict__ verified,
                                                     uint64_t nv,
                                                     const uint32_t *__restrict__ status,
                                                     uint32_t n, uint32_t *__restrict__ flag,
                                                     unsigned long long *__restrict__ errors) {
    const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (t >= nr + m + nv) return;
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
    } else if (t < nr + m) {
        const uint32_t k = keep[t - nr];
        f = k == 1u ? 1u : 0u;
        if (k == 2u) atomicAdd(errors + 1, 1ull);
    } else {
        f = 1u;
        for (int k = 0; k < 4; ++k)
            if (verified[4 * (t - nr - m) + k] >= n) f = 0u;
        if (f == 0u) atomicAdd(errors, 1ull);
    }
    flag[t] = f;
}

__global__ __launch_bounds__(256) void compact_kernel(const uint32_t *__restrict__ reports,
                                                      uint64_t nr,
                                                      const uint32_t *__restrict__ cand,
                                                      uint64_t m,
                                                      const uint32_t *__restrict__ verified,
                                                      uint64_t nv,
                                                      const uint32_t *__restrict__ flag,
                                                      const uint32_t *__restrict__ pos,
                                                      uint32_t *__restrict__ out,
                                                      uint64_t capacity) {
    const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (t >= nr + m + nv || !flag[t]) return;
    const uint64_t w = pos[t];
    if (w >= capacity) return;
    const uint32_t *src = t < nr       ? reports + 4 * t
                          : t < nr + m ? cand + 4 * (t - nr)
                                       : verified + 4 * (t - nr - m);
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

namespace {

// The grid levels over the points into the scratch, its geometry kept there
// for the calls that follow; `g` receives it too and must live until the
// caller's next synchronisation of the stream (the copy reads it).
hipError_t build_grid(const float *points, uint32_t n, const GridScratch &s, GridGeom &g,
                      hipStream_t stream, double box_scale = 1.0) {
    hipLaunchKernelGGL(tag_kernel, dim3(1), dim3(64), 0, stream, s.tag, 0ull, 0ull);
    hipLaunchKernelGGL(init_kernel, dim3(1), dim3(64), 0, stream, s.mm, s.counters);
    hipLaunchKernelGGL(bbox_kernel, dim3(std::min<uint32_t>(grid1(n).x, kBboxBlocks)), dim3(256), 0,
                       stream, points, n, s.mm);
    uint32_t hm[6];
    hipError_t e = hipMemcpyAsync(hm, s.mm, sizeof(hm), hipMemcpyDeviceToHost, stream);
    if (e != hipSuccess) return e;
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
    double lo[3], hi[3];
    for (int k = 0; k < 3; ++k) {
        lo[k] = (double)unordered(hm[k]);
        hi[k] = (double)unordered(hm[3 + k]);
    }
    if (!dgrid::grid_geometry(lo, hi, n, g, box_scale)) return hipErrorInvalidValue;
    // the points sorted once by the Morton code of their finest cell (one
    // radix sort in place of one per level; 11 at ~0.25 ms each at 1M
    // points), then per level the table of occupied cells over that order
    hipLaunchKernelGGL(morton_keys_kernel, grid1(n), dim3(256), 0, stream, points, n, g, s.keys,
                       s.index);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    size_t tb = s.temp_bytes;
    e = rocprim::radix_sort_pairs(s.temp, tb, s.keys, s.keys_sorted, s.index, s.sorted[0],
                                  (size_t)n, 0u, 63u, stream);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gather_points_kernel, grid1(n), dim3(256), 0, stream, points, s.sorted[0],
                       n, reinterpret_cast<float4 *>(s.spts));
    const uint64_t slots = g.table_mask + 1;
    for (int l = 0; l < dgrid::kLevels; ++l) {
        hipLaunchKernelGGL(level_keys_kernel, grid1(n), dim3(256), 0, stream, s.keys_sorted, n, l,
                           s.keys);
        hipLaunchKernelGGL(table_clear_kernel, grid1(slots), dim3(256), 0, stream, s.table[l],
                           slots);
        hipLaunchKernelGGL(table_insert_kernel, grid1(n), dim3(256), 0, stream, s.keys, n,
                           s.table[l], g.table_mask);
        hipLaunchKernelGGL(table_end_kernel, grid1(n), dim3(256), 0, stream, s.keys, n,
                           s.table[l], g.table_mask);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if ((e = hipMemcpyAsync(s.geom, &g, sizeof(g), hipMemcpyHostToDevice, stream)) != hipSuccess)
        return e;
    hipLaunchKernelGGL(tag_kernel, dim3(1), dim3(64), 0, stream, s.tag, kGridTag, (uint64_t)n);
    return hipGetLastError();
}

GridView grid_view(const GridScratch &s, const GridGeom &g) {
    GridView gv{};
    gv.g = g;
    for (int l = 0; l < dgrid::kLevels; ++l) {
        gv.table[l] = s.table[l];
        gv.sorted[l] = s.sorted[l];
    }
    gv.spts = s.spts;
    return gv;
}

// Candidates a listed point's cell (an incremental rebuild's dirty point) may
// examine before it is left open, a quarter of the whole set's cap: the few
// cells that certify only after some 50k candidates (beside large empty
// regions; 1,000-2,400 cuts and 3-6 ms each) set the length of the call, and
// left open they go to the open points' exhaustive pass, and skip the next
// rebuild's certification (C3 incremental rebuild 44.3 -> 42.0 ms; the whole
// set's cap at 16,384 would leave 11.8k points open against 7.9k and take the
// full rebuild 59.0 -> 59.8 ms).
constexpr uint32_t kMaxCandidatesDirty = 16384;

// certify_kernel over all points (query == nullptr) or the nq listed ones,
// then the counters to the host.
hipError_t run_certify(const float *points, uint32_t n, const uint32_t *query, uint32_t nq,
                       const GridView &gv, const GridScratch &s, uint32_t *reports,
                       uint64_t report_capacity, uint32_t *open, uint64_t counts[5],
                       hipStream_t stream, bool exhaustive = false) {
    hipError_t e;
    if (nq > 0) {
        const uint32_t cap = query ? kMaxCandidatesDirty : dgrid::kMaxCandidates;
        if (exhaustive)
            hipLaunchKernelGGL(certify_kernel<true>, dim3(nq), dim3(64), 0, stream, points, n, gv,
                               reports, report_capacity, s.counters, open, s.status, query, cap);
        else
            hipLaunchKernelGGL(certify_kernel<false>, dim3(nq), dim3(64), 0, stream, points, n, gv,
                               reports, report_capacity, s.counters, open, s.status, query, cap);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    unsigned long long hc[8];
    if ((e = hipMemcpyAsync(hc, s.counters, sizeof(hc), hipMemcpyDeviceToHost, stream)) !=
            hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
        return e;
    for (int k = 0; k < 5; ++k) counts[k] = hc[k];
    return hipSuccess;
}

} // namespace

namespace {

hipError_t certify_all(const float *points, uint32_t n, uint32_t *reports,
                       uint64_t report_capacity, uint32_t *open, uint64_t counts[5],
                       void *scratch, size_t bytes, hipStream_t stream, bool exhaustive) {
    for (int k = 0; k < 5; ++k) counts[k] = 0;
    const size_t temp = grid_temp_bytes(n);
    GridScratch s = carve_grid(scratch, n, temp);
    if (n == 0 || temp == 0 || s.total > bytes) return hipErrorInvalidValue;
    GridGeom g{};
    hipError_t e = build_grid(points, n, s, g, stream, exhaustive ? kExhaustiveBox : 1.0);
    if (e != hipSuccess) return e;
    return run_certify(points, n, nullptr, n, grid_view(s, g), s, reports, report_capacity, open,
                       counts, stream, exhaustive);
}

} // namespace

hipError_t launch_delaunay_certify(const float *points, uint32_t n, uint32_t *reports,
                                   uint64_t report_capacity, uint32_t *open, uint64_t counts[5],
                                   void *scratch, size_t bytes, hipStream_t stream) {
    return certify_all(points, n, reports, report_capacity, open, counts, scratch, bytes, stream,
                       false);
}

hipError_t launch_delaunay_certify_exhaustive(const float *points, uint32_t n, uint32_t *reports,
                                              uint64_t report_capacity, uint32_t *open,
                                              uint64_t counts[5], void *scratch, size_t bytes,
                                              hipStream_t stream) {
    return certify_all(points, n, reports, report_capacity, open, counts, scratch, bytes, stream,
                       true);
}

hipError_t launch_delaunay_check(const float *points, uint32_t n, const uint32_t *tets,
                                 const int32_t *nbr, uint64_t T, uint32_t *keep, uint32_t *dirty,
                                 uint64_t *errors, void *scratch, size_t bytes,
                                 hipStream_t stream) {
    *errors = 0;
    const size_t temp = grid_temp_bytes(n);
    GridScratch s = carve_grid(scratch, n, temp);
    if (n == 0 || temp == 0 || s.total > bytes) return hipErrorInvalidValue;
    GridGeom g{};
    hipError_t e = build_grid(points, n, s, g, stream);
    if (e != hipSuccess) return e;
    // every point clean until certify_points certifies or opens it
    hipLaunchKernelGGL(fill_kernel, grid1(n), dim3(256), 0, stream, s.status, (uint64_t)n,
                       dgrid::kStatusClean);
    hipLaunchKernelGGL(fill_kernel, grid1(n), dim3(256), 0, stream, dirty, (uint64_t)n, 0u);
    if (T > 0)
        hipLaunchKernelGGL(check_kernel, grid1(T * kCheckLanes), dim3(256), 0, stream, points, n,
                           grid_view(s, g), s.status, tets, nbr, T, keep, dirty, s.counters + 5);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    unsigned long long hc[8];
    if ((e = hipMemcpyAsync(hc, s.counters, sizeof(hc), hipMemcpyDeviceToHost, stream)) !=
            hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
        return e;
    *errors = hc[5];
    return hipSuccess;
}

hipError_t launch_delaunay_certify_points(const float *points, uint32_t n, const uint32_t *query,
                                          uint32_t nq, uint32_t *reports,
                                          uint64_t report_capacity, uint32_t *open,
                                          uint64_t counts[5], void *scratch, size_t bytes,
                                          hipStream_t stream) {
    for (int k = 0; k < 5; ++k) counts[k] = 0;
    const size_t temp = grid_temp_bytes(n);
    GridScratch s = carve_grid(scratch, n, temp);
    if (n == 0 || temp == 0 || s.total > bytes) return hipErrorInvalidValue;
    GridGeom g{};
    uint64_t tag[2] = {0, 0};
    hipError_t e = hipMemcpyAsync(&g, s.geom, sizeof(g), hipMemcpyDeviceToHost, stream);
    if (e != hipSuccess) return e;
    if ((e = hipMemcpyAsync(tag, s.tag, sizeof(tag), hipMemcpyDeviceToHost, stream)) != hipSuccess)
        return e;
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
    // the grid must come from a check call over these points
    if (tag[0] != kGridTag || tag[1] != (uint64_t)n) return hipErrorNotReady;
    hipLaunchKernelGGL(init_kernel, dim3(1), dim3(64), 0, stream, nullptr, s.counters);
    return run_certify(points, n, query, nq, grid_view(s, g), s, reports, report_capacity, open,
                       counts, stream);
}

size_t delaunay_merge_scratch_bytes(uint32_t n, uint64_t nr, uint64_t m, uint64_t tcap) {
    const size_t temp = merge_temp_bytes(n, nr + m);
    if (temp == 0) return 0;
    return carve_merge(nullptr, n, nr, m, tcap, temp).total;
}

hipError_t launch_delaunay_merge(const float *points, uint32_t n, void *grid_scratch,
                                 size_t grid_bytes, const uint32_t *reports, uint64_t nr,
                                 const uint32_t *cand, uint64_t m, const uint32_t *verified,
                                 uint64_t nv, uint32_t *tets, int32_t *nbr, uint64_t tcap,
                                 uint64_t result[4], void *scratch, size_t bytes,
                                 hipStream_t stream) {
    for (int k = 0; k < 4; ++k) result[k] = 0;
    const size_t gtemp = grid_temp_bytes(n);
    const GridScratch gs = carve_grid(grid_scratch, n, gtemp);
    // the scratch is sized for nr reports and m + nv candidates (keep holds
    // m + nv entries, of which the verified rows use none)
    const size_t temp = merge_temp_bytes(n, nr + m + nv);
    const MergeScratch s = carve_merge(scratch, n, nr, m + nv, tcap, temp);
    if (n == 0 || gtemp == 0 || gs.total > grid_bytes || temp == 0 || s.total > bytes)
        return hipErrorInvalidValue;
    if (nr + m + nv >= 0xffffffffull) return hipErrorInvalidValue;
    GridView gv{};
    hipError_t e =
        hipMemcpyAsync(&gv.g, gs.geom, sizeof(GridGeom), hipMemcpyDeviceToHost, stream);
    if (e != hipSuccess) return e;
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
    for (int l = 0; l < dgrid::kLevels; ++l) {
        gv.table[l] = gs.table[l];
        gv.sorted[l] = gs.sorted[l];
    }
    gv.spts = gs.spts;
    hipLaunchKernelGGL(init_kernel, dim3(1), dim3(64), 0, stream, nullptr, s.acc);
    if (m > 0)
        hipLaunchKernelGGL(keep_empty_kernel, dim3((unsigned)m), dim3(64), 0, stream, points, n,
                           gv, cand, (uint32_t)m, gs.status, s.keep);
    const uint64_t rows = nr + m + nv;
    uint32_t last[2] = {0, 0};
    if (rows > 0) {
        hipLaunchKernelGGL(select_kernel, grid1(rows), dim3(256), 0, stream, reports, nr, s.keep,
                           m, verified, nv, gs.status, n, s.flag, s.acc + 2);
        size_t tb = s.temp_bytes;
        e = rocprim::exclusive_scan(s.temp, tb, s.flag, s.pos, 0u, (size_t)rows,
                                    rocprim::plus<uint32_t>(), stream);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(compact_kernel, grid1(rows), dim3(256), 0, stream, reports, nr, cand,
                           m, verified, nv, s.flag, s.pos, tets, tcap);
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
