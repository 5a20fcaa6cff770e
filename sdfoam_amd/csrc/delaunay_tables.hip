// Device side of the adjacency producer around the Delaunay tetrahedralisation:
//
// * sort_points: the point order the reference's tree builder leaves
//   (src/aabb_tree/aabb_tree.cu:62-190): for segment sizes pow2(N), pow2(N)/2,
//   ..., 2 a stable sort by one coordinate (x, y, z, x, ...).  Segments larger
//   than 1024 sort within their segment when there are more than 1024 of
//   them, and as one whole array otherwise; segments of at most 1024 sort
//   within their 1024-point block.  Each pass here is one stable 64-bit radix
//   sort of (segment, orderable key) pairs carrying the permutation.
//
// * delaunay_tables: the tables the reference's Triangulation exposes
//   (src/delaunay/delaunay.cu:146-226; torch_bindings/triangulation_bindings.cpp
//   :11-115) from a tetrahedralisation given as vertex quadruples and
//   face neighbours (Qhull's simplices / neighbors): tets positively
//   oriented and ordered by their sorted vertex sets, tet adjacency as
//   4 k + m, the lowest tet of each point and the Delaunay edges as CSR
//   with ascending rows.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>
#include <rocprim/device/device_select.hpp>

#include "trace_kernels.h"

namespace sdfoam_hip {

namespace {

constexpr uint32_t kSortBlock = 1024; // src/aabb_tree/aabb_tree.cu:15

size_t align256(size_t x) { return (x + 255u) & ~(size_t)255u; }

uint32_t bits_for(uint64_t max_value) {
    uint32_t b = 1;
    while (b < 32 && (1ull << b) <= max_value) ++b;
    return b;
}

uint32_t pow2_round_up(uint32_t x) {
    uint32_t p = 1;
    while (p < x) p <<= 1;
    return p;
}

inline dim3 grid1(uint64_t n) { return dim3((unsigned)((n + 255u) / 256u)); }

// float bits -> unsigned keys that sort like the floats
// (src/aabb_tree/aabb_tree.cu:85-94)
__global__ __launch_bounds__(256) void orderable_keys_kernel(const float *__restrict__ points,
                                                             uint64_t n3,
                                                             uint32_t *__restrict__ keys) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= n3) return;
    const uint32_t u = __builtin_bit_cast(uint32_t, points[i]);
    keys[i] = (u & 0x80000000u) ? ~u : (u ^ 0x80000000u);
}

__global__ __launch_bounds__(256) void iota_kernel(uint32_t *__restrict__ v, uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) v[i] = i;
}

// key of sorted position i: segment << 32 | coordinate key of point perm[i]
__global__ __launch_bounds__(256) void pass_keys_kernel(const uint32_t *__restrict__ ckeys,
                                                        const uint32_t *__restrict__ perm,
                                                        uint32_t n, uint32_t dim,
                                                        uint32_t seg_shift, bool whole,
                                                        uint64_t *__restrict__ keys) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const uint64_t seg = whole ? 0ull : (uint64_t)(i >> seg_shift);
    keys[i] = (seg << 32) | ckeys[3ull * perm[i] + dim];
}

// ---- tables ----------------------------------------------------------------

// Orientation sign as the host computes it: vol = (b - a) x (c - a) . (d - a)
// in double, each product rounded, no fused operations (the build flags
// disable contraction).
__device__ __forceinline__ double orient_vol(const float *__restrict__ p, const uint32_t *s) {
    double a[3], b[3], c[3], d[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        a[k] = (double)p[3ull * s[0] + k];
        b[k] = (double)p[3ull * s[1] + k];
        c[k] = (double)p[3ull * s[2] + k];
        d[k] = (double)p[3ull * s[3] + k];
    }
    const double u0 = b[0] - a[0], u1 = b[1] - a[1], u2 = b[2] - a[2];
    const double v0 = c[0] - a[0], v1 = c[1] - a[1], v2 = c[2] - a[2];
    const double w0 = d[0] - a[0], w1 = d[1] - a[1], w2 = d[2] - a[2];
    const double x0 = u1 * v2 - u2 * v1;
    const double x1 = u2 * v0 - u0 * v2;
    const double x2 = u0 * v1 - u1 * v0;
    return (x0 * w0 + x1 * w1) + x2 * w2;
}

// Puts tet t in its canonical vertex order (ascending, the last two
// swapped when the volume is negative; neighbours follow their vertices)
// and forms its sort keys from the sorted vertex set.
__global__ __launch_bounds__(256) void orient_kernel(
    const float *__restrict__ points, uint32_t num_points, const uint32_t *__restrict__ tets_in,
    const int32_t *__restrict__ nbr_in, uint32_t num_tets, uint32_t *__restrict__ tets_o,
    int32_t *__restrict__ nbr_o, uint64_t *__restrict__ key_hi, uint64_t *__restrict__ key_lo,
    uint32_t *__restrict__ index, uint32_t *__restrict__ error, uint32_t kb) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= num_tets) return;
    uint32_t s[4];
    int32_t nb[4];
    bool ok = true;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        s[k] = tets_in[4ull * t + k];
        nb[k] = nbr_in[4ull * t + k];
        ok = ok && s[k] < num_points && (nb[k] < 0 || (uint32_t)nb[k] < num_tets);
    }
    if (!ok) {
        atomicOr(error, 1u);
        s[0] = s[1] = s[2] = s[3] = 0u;
        nb[0] = nb[1] = nb[2] = nb[3] = -1;
    }
    // canonical vertex order: ascending (each neighbour stays opposite its
    // vertex), then the last two swapped when the volume is negative
#define SDF_CSWAP2(i, j)                                                                           \
    if (s[j] < s[i]) {                                                                            \
        const uint32_t ts = s[i];                                                                 \
        s[i] = s[j];                                                                              \
        s[j] = ts;                                                                                \
        const int32_t tn = nb[i];                                                                 \
        nb[i] = nb[j];                                                                            \
        nb[j] = tn;                                                                               \
    }
    SDF_CSWAP2(0, 1) SDF_CSWAP2(2, 3) SDF_CSWAP2(0, 2) SDF_CSWAP2(1, 3) SDF_CSWAP2(1, 2)
#undef SDF_CSWAP2
    if (ok && orient_vol(points, s) < 0.0) {
        uint32_t ts = s[2];
        s[2] = s[3];
        s[3] = ts;
        int32_t tn = nb[2];
        nb[2] = nb[3];
        nb[3] = tn;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        tets_o[4ull * t + k] = s[k];
        nbr_o[4ull * t + k] = nb[k];
    }
    // sorted vertex set (4-element sorting network)
    uint32_t v[4] = {s[0], s[1], s[2], s[3]};
#define SDF_CSWAP(i, j)                                                                            \
    {                                                                                             \
        const uint32_t lo = min(v[i], v[j]), hi = max(v[i], v[j]);                                \
        v[i] = lo;                                                                                \
        v[j] = hi;                                                                                \
    }
    SDF_CSWAP(0, 1) SDF_CSWAP(2, 3) SDF_CSWAP(0, 2) SDF_CSWAP(1, 3) SDF_CSWAP(1, 2)
#undef SDF_CSWAP
    key_hi[t] = ((uint64_t)v[0] << kb) | v[1];
    key_lo[t] = ((uint64_t)v[2] << kb) | v[3];
    index[t] = t;
}

__global__ __launch_bounds__(256) void gather_u64_kernel(const uint64_t *__restrict__ src,
                                                         const uint32_t *__restrict__ idx,
                                                         uint32_t n, uint64_t *__restrict__ dst) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) dst[i] = src[idx[i]];
}

__global__ __launch_bounds__(256) void rank_kernel(const uint32_t *__restrict__ order, uint32_t n,
                                                   uint32_t *__restrict__ rank) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) rank[order[i]] = i;
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t *__restrict__ v, uint64_t n,
                                                       uint32_t value) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) v[i] = value;
}

// New tet i = old tet order[i]: vertices, adjacency (neighbour's new index
// and the position of its vertex not in tet i), lowest tet per vertex, and
// its six edges.
__global__ __launch_bounds__(256) void emit_kernel(
    const uint32_t *__restrict__ order, const uint32_t *__restrict__ rank,
    const uint32_t *__restrict__ tets_o, const int32_t *__restrict__ nbr_o, uint32_t num_tets,
    uint32_t *__restrict__ tets_out, uint32_t *__restrict__ tet_adj,
    uint32_t *__restrict__ vert_to_tet, uint64_t *__restrict__ edges, uint32_t kb) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= num_tets) return;
    const uint32_t t = order[i];
    uint32_t s[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) s[k] = tets_o[4ull * t + k];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        tets_out[4ull * i + j] = s[j];
        atomicMin(vert_to_tet + s[j], i);
        const int32_t nb = nbr_o[4ull * t + j];
        uint32_t a = kNoIndex;
        if (nb >= 0) {
            uint32_t m = 0;
            for (int q = 3; q >= 0; --q) {
                const uint32_t o = tets_o[4ull * (uint32_t)nb + q];
                if (o != s[0] && o != s[1] && o != s[2] && o != s[3]) m = (uint32_t)q;
            }
            a = 4u * rank[nb] + m;
        }
        tet_adj[4ull * i + j] = a;
    }
    int e = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
        for (int q = p + 1; q < 4; ++q) {
            const uint32_t lo = min(s[p], s[q]), hi = max(s[p], s[q]);
            edges[6ull * i + e] = ((uint64_t)lo << kb) | hi;
            ++e;
        }
    }
}

// Both directions of the U unique edges; counts per row.
__global__ __launch_bounds__(256) void both_dirs_kernel(const uint64_t *__restrict__ uniq,
                                                        const uint64_t *__restrict__ num_unique,
                                                        uint64_t capacity,
                                                        uint64_t *__restrict__ dirs,
                                                        uint32_t *__restrict__ counts,
                                                        uint32_t *__restrict__ error,
                                                        uint32_t kb) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint64_t u = *num_unique;
    if (i >= u) return;
    if (2 * u > capacity) {
        if (i == 0) atomicOr(error, 2u);
        return;
    }
    const uint64_t k = uniq[i];
    const uint32_t lo = (uint32_t)(k >> kb), hi = (uint32_t)(k & ((1ull << kb) - 1ull));
    dirs[2 * i] = k;
    dirs[2 * i + 1] = ((uint64_t)hi << kb) | lo;
    atomicAdd(counts + lo, 1u);
    atomicAdd(counts + hi, 1u);
}

__global__ __launch_bounds__(256) void low_words_kernel(const uint64_t *__restrict__ keys,
                                                        const uint64_t *__restrict__ num_unique,
                                                        uint64_t capacity,
                                                        uint32_t *__restrict__ out, uint32_t kb) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint64_t n = 2 * *num_unique;
    if (i < n && n <= capacity) out[i] = (uint32_t)(keys[i] & ((1ull << kb) - 1ull));
}

struct TablesScratch {
    uint32_t *tets_o;
    int32_t *nbr_o;
    uint64_t *key_hi, *key_lo, *key_tmp, *key_sorted;
    uint32_t *idx_a, *idx_b, *rank;
    uint64_t *edges, *edges_sorted, *uniq, *num_unique;
    uint64_t *dirs, *dirs_sorted;
    uint32_t *counts, *error;
    void *temp;
    size_t temp_bytes;
};

size_t tables_temp_bytes(uint32_t num_points, uint32_t num_tets, uint64_t capacity) {
    size_t a = 0, b = 0, c = 0, d = 0;
    const uint64_t *k = nullptr;
    uint64_t *ko = nullptr;
    const uint32_t *v = nullptr;
    uint32_t *vo = nullptr;
    const uint64_t ne = 6ull * num_tets;
    // the sorts run over 2 kb bits (launch_delaunay_tables); the size for
    // 64 bits is asked as well and the larger kept
    const uint32_t kb = num_points > 1u ? 32u - (uint32_t)__builtin_clz(num_points - 1u) : 1u;
    for (const uint32_t bits : {64u, 2u * kb}) {
        size_t a1 = 0, b1 = 0, d1 = 0;
        if (rocprim::radix_sort_pairs(nullptr, a1, k, ko, v, vo, num_tets, 0u, bits) !=
                hipSuccess ||
            rocprim::radix_sort_keys(nullptr, b1, k, ko, (size_t)ne, 0u, bits) != hipSuccess ||
            rocprim::radix_sort_keys(nullptr, d1, k, ko, (size_t)capacity, 0u, bits) !=
                hipSuccess)
            return 0;
        a = std::max(a, a1);
        b = std::max(b, b1);
        d = std::max(d, d1);
    }
    if (rocprim::unique(nullptr, c, k, ko, (uint64_t *)nullptr, (size_t)ne) != hipSuccess) return 0;
    size_t e = 0;
    if (rocprim::exclusive_scan(nullptr, e, v, vo, 0u, (size_t)num_points + 1,
                                rocprim::plus<uint32_t>()) != hipSuccess)
        return 0;
    return std::max(std::max(std::max(a, b), std::max(c, d)), e);
}

// Carves the scratch; returns false if it is too small.
bool carve(void *scratch, size_t scratch_bytes, uint32_t num_points, uint32_t num_tets,
           uint64_t capacity, TablesScratch &s) {
    char *p = static_cast<char *>(scratch);
    auto take = [&](size_t bytes) {
        char *q = p;
        p += align256(bytes);
        return q;
    };
    const uint64_t T = num_tets, ne = 6ull * num_tets;
    s.tets_o = reinterpret_cast<uint32_t *>(take(16 * T));
    s.nbr_o = reinterpret_cast<int32_t *>(take(16 * T));
    s.key_hi = reinterpret_cast<uint64_t *>(take(8 * T));
    s.key_lo = reinterpret_cast<uint64_t *>(take(8 * T));
    s.key_tmp = reinterpret_cast<uint64_t *>(take(8 * T));
    s.key_sorted = reinterpret_cast<uint64_t *>(take(8 * T));
    s.idx_a = reinterpret_cast<uint32_t *>(take(4 * T));
    s.idx_b = reinterpret_cast<uint32_t *>(take(4 * T));
    s.rank = reinterpret_cast<uint32_t *>(take(4 * T));
    s.edges = reinterpret_cast<uint64_t *>(take(8 * ne));
    s.edges_sorted = reinterpret_cast<uint64_t *>(take(8 * ne));
    s.uniq = reinterpret_cast<uint64_t *>(take(8 * ne));
    s.num_unique = reinterpret_cast<uint64_t *>(take(8));
    s.dirs = reinterpret_cast<uint64_t *>(take(8 * capacity));
    s.dirs_sorted = reinterpret_cast<uint64_t *>(take(8 * capacity));
    s.counts = reinterpret_cast<uint32_t *>(take(4ull * (num_points + 1)));
    s.error = reinterpret_cast<uint32_t *>(take(4));
    const size_t used = (size_t)(p - static_cast<char *>(scratch));
    if (used > scratch_bytes) return false;
    s.temp = p;
    s.temp_bytes = scratch_bytes - used;
    return true;
}

size_t tables_fixed_bytes(uint32_t num_points, uint32_t num_tets, uint64_t capacity) {
    const uint64_t T = num_tets, ne = 6ull * num_tets;
    return align256(16 * T) * 2 + align256(8 * T) * 4 + align256(4 * T) * 3 + align256(8 * ne) * 3 +
           align256(8) + align256(8 * capacity) * 2 + align256(4ull * (num_points + 1)) +
           align256(4);
}

} // namespace

uint64_t delaunay_edge_capacity(uint32_t num_points, uint32_t num_tets) {
    // a tetrahedralised ball: V - E + F - T = 1 with F = (4T + H) / 2 and
    // H <= 2V hull triangles, so 2E <= 4V + 2T
    return 4ull * num_points + 2ull * num_tets + 64u;
}

size_t sort_points_scratch_bytes(uint32_t num_points) {
    size_t temp = 0;
    const uint64_t *k = nullptr;
    uint64_t *ko = nullptr;
    const uint32_t *v = nullptr;
    uint32_t *vo = nullptr;
    if (rocprim::radix_sort_pairs(nullptr, temp, k, ko, v, vo, num_points, 0u, 64u) != hipSuccess)
        return 0;
    return align256(12ull * num_points) + align256(8ull * num_points) * 2 +
           align256(4ull * num_points) + align256(temp);
}

hipError_t launch_sort_points(const float *points, uint32_t num_points, uint32_t *perm,
                              void *scratch, size_t scratch_bytes, hipStream_t stream) {
    if (num_points == 0) return hipSuccess;
    char *p = static_cast<char *>(scratch);
    uint32_t *ckeys = reinterpret_cast<uint32_t *>(p);
    p += align256(12ull * num_points);
    uint64_t *keys = reinterpret_cast<uint64_t *>(p);
    p += align256(8ull * num_points);
    uint64_t *keys_sorted = reinterpret_cast<uint64_t *>(p);
    p += align256(8ull * num_points);
    uint32_t *perm_b = reinterpret_cast<uint32_t *>(p);
    p += align256(4ull * num_points);
    const size_t used = (size_t)(p - static_cast<char *>(scratch));
    if (used > scratch_bytes) return hipErrorInvalidValue;
    const size_t temp = scratch_bytes - used;
    const uint32_t n = num_points;
    hipLaunchKernelGGL(orderable_keys_kernel, grid1(3ull * n), dim3(256), 0, stream, points,
                       3ull * n, ckeys);
    hipLaunchKernelGGL(iota_kernel, grid1(n), dim3(256), 0, stream, perm, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint32_t *cur = perm, *nxt = perm_b;
    uint32_t seg = pow2_round_up(n);
    uint32_t dim = 0;
    while (seg > 1) {
        const uint64_t nseg = ((uint64_t)n + seg - 1) / seg;
        bool whole = false;
        uint32_t shift, max_seg;
        if (seg > kSortBlock) {
            whole = nseg <= 1024;
            shift = (uint32_t)__builtin_ctz(seg);
            max_seg = whole ? 0u : (uint32_t)(nseg - 1);
        } else {
            shift = 10; // 1024-point blocks
            max_seg = (n - 1) >> 10;
        }
        hipLaunchKernelGGL(pass_keys_kernel, grid1(n), dim3(256), 0, stream, ckeys, cur, n, dim,
                           shift, whole, keys);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        size_t t = temp;
        e = rocprim::radix_sort_pairs(p, t, keys, keys_sorted, cur, nxt, n, 0u,
                                      32u + bits_for(max_seg), stream);
        if (e != hipSuccess) return e;
        uint32_t *sw = cur;
        cur = nxt;
        nxt = sw;
        seg >>= 1;
        dim = (dim + 1) % 3;
    }
    if (cur != perm)
        return hipMemcpyAsync(perm, cur, 4ull * n, hipMemcpyDeviceToDevice, stream);
    return hipSuccess;
}

size_t delaunay_tables_scratch_bytes(uint32_t num_points, uint32_t num_tets) {
    const uint64_t cap = delaunay_edge_capacity(num_points, num_tets);
    const size_t temp = tables_temp_bytes(num_points, num_tets, cap);
    if (temp == 0) return 0;
    return tables_fixed_bytes(num_points, num_tets, cap) + align256(temp);
}

hipError_t launch_delaunay_tables(const float *points, uint32_t num_points,
                                  const uint32_t *tets_in, const int32_t *nbr_in,
                                  uint32_t num_tets, uint32_t *tets_out, uint32_t *tet_adj,
                                  uint32_t *vert_to_tet, uint32_t *offsets, uint32_t *adjacency,
                                  uint64_t adjacency_capacity, uint32_t &input_error,
                                  void *scratch, size_t scratch_bytes, hipStream_t stream) {
    input_error = 0;
    const uint64_t cap = delaunay_edge_capacity(num_points, num_tets);
    if (adjacency_capacity < cap) return hipErrorInvalidValue;
    TablesScratch s;
    if (!carve(scratch, scratch_bytes, num_points, num_tets, cap, s)) return hipErrorInvalidValue;
    const uint32_t T = num_tets;
    // keys pack two point ids of kb bits each, so the radix sorts run over 2 kb
    // bits (40 at 1M points) instead of 64
    const uint32_t kb = num_points > 1u ? 32u - (uint32_t)__builtin_clz(num_points - 1u) : 1u;
    hipLaunchKernelGGL(fill_u32_kernel, grid1(1), dim3(256), 0, stream, s.error, (uint64_t)1, 0u);
    hipLaunchKernelGGL(fill_u32_kernel, grid1(num_points), dim3(256), 0, stream, vert_to_tet,
                       (uint64_t)num_points, kNoIndex);
    hipLaunchKernelGGL(fill_u32_kernel, grid1((uint64_t)num_points + 1), dim3(256), 0, stream,
                       s.counts, (uint64_t)num_points + 1, 0u);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint64_t num_unique = 0;
    if (T > 0) {
        hipLaunchKernelGGL(orient_kernel, grid1(T), dim3(256), 0, stream, points, num_points,
                           tets_in, nbr_in, T, s.tets_o, s.nbr_o, s.key_hi, s.key_lo, s.idx_a,
                           s.error, kb);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // lexicographic order of (key_hi, key_lo): stable sort by key_lo, then by key_hi
        size_t t = s.temp_bytes;
        e = rocprim::radix_sort_pairs(s.temp, t, s.key_lo, s.key_sorted, s.idx_a, s.idx_b, T, 0u,
                                      2u * kb, stream);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(gather_u64_kernel, grid1(T), dim3(256), 0, stream, s.key_hi, s.idx_b,
                           T, s.key_tmp);
        t = s.temp_bytes;
        e = rocprim::radix_sort_pairs(s.temp, t, s.key_tmp, s.key_sorted, s.idx_b, s.idx_a, T, 0u,
                                      2u * kb, stream);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(rank_kernel, grid1(T), dim3(256), 0, stream, s.idx_a, T, s.rank);
        hipLaunchKernelGGL(emit_kernel, grid1(T), dim3(256), 0, stream, s.idx_a, s.rank, s.tets_o,
                           s.nbr_o, T, tets_out, tet_adj, vert_to_tet, s.edges, kb);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        const uint64_t ne = 6ull * T;
        t = s.temp_bytes;
        e = rocprim::radix_sort_keys(s.temp, t, s.edges, s.edges_sorted, (size_t)ne, 0u, 2u * kb,
                                     stream);
        if (e != hipSuccess) return e;
        t = s.temp_bytes;
        e = rocprim::unique(s.temp, t, s.edges_sorted, s.uniq, s.num_unique, (size_t)ne,
                            rocprim::equal_to<uint64_t>(), stream);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(both_dirs_kernel, grid1(ne), dim3(256), 0, stream, s.uniq,
                           s.num_unique, cap, s.dirs, s.counts, s.error, kb);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // the edge count decides the size of the last sort: read it (and the
        // input checks) on the host
        uint32_t err = 0;
        if ((e = hipMemcpyAsync(&num_unique, s.num_unique, 8, hipMemcpyDeviceToHost, stream)) !=
                hipSuccess ||
            (e = hipMemcpyAsync(&err, s.error, 4, hipMemcpyDeviceToHost, stream)) != hipSuccess ||
            (e = hipStreamSynchronize(stream)) != hipSuccess)
            return e;
        input_error = err;
        if (err != 0) return hipSuccess;
        if (2 * num_unique > cap) {
            input_error = 2u;
            return hipSuccess;
        }
        const uint64_t n2 = 2 * num_unique;
        t = s.temp_bytes;
        e = rocprim::radix_sort_keys(s.temp, t, s.dirs, s.dirs_sorted, (size_t)n2, 0u, 2u * kb,
                                     stream);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(low_words_kernel, grid1(n2), dim3(256), 0, stream, s.dirs_sorted,
                           s.num_unique, cap, adjacency, kb);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    size_t t = s.temp_bytes;
    return rocprim::exclusive_scan(s.temp, t, s.counts, offsets, 0u, (size_t)num_points + 1,
                                   rocprim::plus<uint32_t>(), stream);
}

} // namespace sdfoam_hip
