// Start-cell lookup: implicit AABB tree over point pairs and an exact
// nearest-neighbour search, for gfx950.
//
// Tree layout (src/aabb_tree/aabb_tree.cuh:35-43): with td = log2(pow2(N)),
// the node (depth d, index i) is box number 2^td - 2^(d+1) + i of a
// [pow2(N), 2, 3] array (min xyz, max xyz); the leaves (depth td-1) bound
// consecutive point pairs, the last point repeated as padding.
//
// The search gives one wave64 to a query.  The wave tests a group of up to
// 64 sibling nodes per step (one per lane), six tree levels apart (depths 6,
// 12, 18, ...), and descends depth first: at each level the children are
// taken in the order of their lower bounds, so the first leaf visit already
// gives a tight bound, and every node whose lower bound exceeds the best
// distance is skipped.  The top two group levels (depth 6: 64 boxes, depth 12:
// 4,096 boxes) are copied into LDS once per block, so a search reads global
// memory only below depth 12.  The fp32 box distance is a lower bound of the
// fp32 point distance (rounding is monotone), so the result is the exact fp32
// nearest neighbour; ties go to the smallest index.
#include "trace_kernels.h"

#include <algorithm>

namespace sdfoam_hip {

__device__ __forceinline__ uint32_t ilog2_u32(uint32_t x) { return x ? 31u - __clz(x) : 0u; }

__device__ __host__ inline uint32_t pow2_up(uint32_t x) {
    if (x <= 1) return 1;
    uint32_t r = 1;
    while (r < x) r <<= 1;
    return r;
}

// leaves (src/aabb_tree/aabb_tree.cu:192-221)
__global__ __launch_bounds__(kBlock) void build_leaves_kernel(const float *__restrict__ points,
                                                              uint32_t num_points, uint32_t leaves,
                                                              float *__restrict__ tree) {
    const uint32_t l = blockIdx.x * kBlock + threadIdx.x;
    if (l == 0) {
        // the unused last entry of the [pow2(N), 2, 3] array
        float *z = tree + 6ull * (2ull * leaves - 1);
#pragma unroll
        for (int c = 0; c < 6; ++c) z[c] = 0.0f;
    }
    if (l >= leaves) return;
    const uint32_t pi = 2 * l;
    const float *a = points + 3ull * (pi < num_points ? pi : num_points - 1);
    const float *b = (pi + 1 < num_points) ? points + 3ull * (pi + 1) : a;
    float *node = tree + 6ull * l;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float av = a[c], bv = b[c];
        node[c] = fminf(av, bv);
        node[3 + c] = fmaxf(av, bv);
    }
}

// one level above `child_start` (src/aabb_tree/aabb_tree.cu:254-292)
__global__ __launch_bounds__(kBlock) void build_level_kernel(float *__restrict__ tree,
                                                             uint64_t child_start, uint32_t width) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= width) return;
    const float *c0 = tree + 6ull * (child_start + 2ull * i);
    const float *c1 = c0 + 6;
    float *node = tree + 6ull * (child_start + 2ull * width + i);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        node[c] = fminf(c0[c], c1[c]);
        node[3 + c] = fmaxf(c0[c + 3], c1[c + 3]);
    }
}

hipError_t launch_build_aabb_tree(const float *points, uint32_t num_points, float *tree,
                                  hipStream_t stream) {
    const uint32_t n2 = pow2_up(num_points);
    const uint32_t leaves = n2 / 2;
    if (leaves == 0) return hipSuccess;
    hipLaunchKernelGGL(build_leaves_kernel, dim3((leaves + kBlock - 1) / kBlock), dim3(kBlock), 0,
                       stream, points, num_points, leaves, tree);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint64_t start = 0;
    for (uint32_t width = leaves / 2; width >= 1; width /= 2) {
        hipLaunchKernelGGL(build_level_kernel, dim3((width + kBlock - 1) / kBlock), dim3(kBlock), 0,
                           stream, tree, start, width);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        start += 2ull * width;
    }
    return hipSuccess;
}

// ---------------------------------------------------------------------------

// Blocks of 16 waves share one copy of the top levels (1 block per CU).
constexpr int kNNBlock = 1024;
constexpr int kNNWaves = kNNBlock / 64;
constexpr uint32_t kNNTopA = 64;           // boxes at depth 6
constexpr uint32_t kNNTopB = 4096;         // boxes at depth 12
constexpr uint32_t kNNTop = kNNTopA + kNNTopB;
// Group levels of a descent: depths 6, 12, ..., 30 below the root (tree
// depth <= 32); the points are tested without a level of their own.
constexpr int kNNLevels = 6;
constexpr uint32_t kNNMaxBlocks = 256;

struct NNShared {
    float top[6][kNNTop];              // min x, y, z, max x, y, z (SoA: no bank conflicts)
    float lb[kNNWaves][kNNLevels][64]; // lower bounds of each level's pending nodes
};

__device__ __forceinline__ float point_dist(const float *__restrict__ p, float qx, float qy,
                                            float qz) {
    const float dx = p[0] - qx, dy = p[1] - qy, dz = p[2] - qz;
    return sqrtf(sdf_dot3(dx, dy, dz, dx, dy, dz));
}

// distance from q to the box (0 inside): (min - q).max(0).max(q - max).norm()
// (src/aabb_tree/aabb_tree.cuh:272-275)
__device__ __forceinline__ float box_dist(const float *__restrict__ b, float qx, float qy,
                                          float qz) {
    const float dx = fmaxf(fmaxf(b[0] - qx, 0.0f), qx - b[3]);
    const float dy = fmaxf(fmaxf(b[1] - qy, 0.0f), qy - b[4]);
    const float dz = fmaxf(fmaxf(b[2] - qz, 0.0f), qz - b[5]);
    return sqrtf(sdf_dot3(dx, dy, dz, dx, dy, dz));
}

// wave-wide lexicographic minimum of (value, index)
__device__ __forceinline__ void wave_argmin(float &v, uint32_t &idx) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const uint32_t oi = __shfl_xor(idx, off, 64);
        if (ov < v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
}

__device__ __forceinline__ float box_dist_top(const NNShared &sh, uint32_t b, float qx, float qy,
                                             float qz) {
    const float dx = fmaxf(fmaxf(sh.top[0][b] - qx, 0.0f), qx - sh.top[3][b]);
    const float dy = fmaxf(fmaxf(sh.top[1][b] - qy, 0.0f), qy - sh.top[4][b]);
    const float dz = fmaxf(fmaxf(sh.top[2][b] - qz, 0.0f), qz - sh.top[5][b]);
    return sqrtf(sdf_dot3(dx, dy, dz, dx, dy, dz));
}

// Copies the boxes of depths 6 and 12 (those above the points) into LDS.
// Every thread of the block calls it; it ends with a block barrier.
__device__ void nn_load_top(const float *__restrict__ tree, uint32_t td, NNShared &sh) {
    const uint64_t n2 = 1ull << td;
    for (uint32_t t = threadIdx.x; t < kNNTop; t += kNNBlock) {
        const uint32_t d = t < kNNTopA ? 6u : 12u;
        const uint32_t i = t < kNNTopA ? t : t - kNNTopA;
        if (d >= td) continue; // no boxes at that depth: never read
        const float *b = tree + 6ull * ((n2 - (2ull << d)) + i);
#pragma unroll
        for (int c = 0; c < 6; ++c) sh.top[c][t] = b[c];
    }
    __syncthreads();
}

// Nearest point to q for the whole wavefront (the result is uniform), over
// the tree of depth td (points padded to 2^td).  NaN lower bounds mark nodes
// that are taken, outside the group or not comparable (NaN query): a node is
// pending while lb <= best.  0 when no point has a distance (NaN query).
__device__ uint32_t nn_wave(const float *__restrict__ points, const float *__restrict__ tree,
                            uint32_t num_points, uint32_t td, float qx, float qy, float qz,
                            NNShared &sh, uint32_t wave) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t n2 = 1ull << td;
    const float kInf = __builtin_bit_cast(float, 0x7f800000u);
    const float kNaN = __builtin_bit_cast(float, 0x7fc00000u);
    float best = kInf;
    uint32_t best_idx = kNoIndex;

    // the points of a group: one per lane
    auto test_points = [&](uint32_t first, uint32_t size) {
        const uint32_t p = first + lane;
        const bool ok = lane < size && p < num_points;
        float dist = ok ? point_dist(points + 3ull * p, qx, qy, qz) : kInf;
        uint32_t idx = ok ? p : kNoIndex;
        wave_argmin(dist, idx);
        if (dist < best || (dist == best && idx < best_idx)) {
            best = dist;
            best_idx = idx;
        }
    };
    // lower bound of node `first + lane` of depth d (NaN outside the group)
    auto bound = [&](uint32_t d, uint32_t first, uint32_t size) {
        const uint32_t node = first + lane;
        if (lane >= size) return kNaN;
        if (d == 6) return box_dist_top(sh, node, qx, qy, qz);
        if (d == 12) return box_dist_top(sh, kNNTopA + node, qx, qy, qz);
        return box_dist(tree + 6ull * ((n2 - (2ull << d)) + node), qx, qy, qz);
    };

    if (td <= 6) { // a single group of points
        test_points(0, 1u << td);
        const uint32_t r = (uint32_t)__builtin_amdgcn_readfirstlane((int)best_idx);
        return r == kNoIndex ? 0u : r;
    }
    float(*lbs)[64] = sh.lb[wave];
    // lane k holds the first node of level k's group (level k at depth
    // min(6 (k + 1), td), all of it below the points' depth)
    uint32_t first_of = 0;
    lbs[0][lane] = bound(6, 0, 64);
    int k = 0;
    while (k >= 0) {
        __builtin_amdgcn_wave_barrier();
        const float lb = lbs[k][lane];
        const bool pending = lb <= best;
        float bl = pending ? lb : kInf;
        uint32_t bi = pending ? lane : 64u;
        wave_argmin(bl, bi);
        if (bi >= 64u) { // level done
            --k;
            continue;
        }
        if (lane == bi) lbs[k][lane] = kNaN; // taken
        const uint32_t d = 6u * (uint32_t)(k + 1);
        const uint32_t node = (uint32_t)__builtin_amdgcn_readlane((int)first_of, k) + bi;
        const uint32_t dc = d + 6 < td ? d + 6 : td;
        const uint32_t cfirst = node << (dc - d);
        const uint32_t csize = 1u << (dc - d);
        if (dc == td) {
            test_points(cfirst, csize);
            continue;
        }
        ++k; // k + 1 < kNNLevels: dc < td <= 32 makes dc <= 30
        if (lane == (uint32_t)k) first_of = cfirst;
        lbs[k][lane] = bound(dc, cfirst, csize);
    }
    const uint32_t r = (uint32_t)__builtin_amdgcn_readfirstlane((int)best_idx);
    return r == kNoIndex ? 0u : r;
}

__global__ __launch_bounds__(kNNBlock) void nn_kernel(const float *__restrict__ points,
                                                      const float *__restrict__ tree,
                                                      const float *__restrict__ queries,
                                                      uint32_t num_points, uint32_t num_queries,
                                                      uint32_t *__restrict__ indices) {
    __shared__ NNShared sh;
    const uint32_t td = ilog2_u32(pow2_up(num_points));
    nn_load_top(tree, td, sh);
    const uint32_t wave = threadIdx.x >> 6;
    for (uint32_t qi = blockIdx.x * kNNWaves + wave; qi < num_queries; qi += gridDim.x * kNNWaves) {
        const uint32_t r = nn_wave(points, tree, num_points, td, queries[3ull * qi],
                                   queries[3ull * qi + 1], queries[3ull * qi + 2], sh, wave);
        if ((threadIdx.x & 63u) == 0) indices[qi] = r;
    }
}

hipError_t launch_nn(const float *points, const float *tree, const float *queries,
                     uint32_t num_points, uint32_t num_queries, uint32_t *indices,
                     hipStream_t stream) {
    if (num_queries == 0) return hipSuccess;
    const uint32_t blocks = std::min<uint32_t>((num_queries + kNNWaves - 1) / kNNWaves, kNNMaxBlocks);
    hipLaunchKernelGGL(nn_kernel, dim3(blocks), dim3(kNNBlock), 0, stream, points, tree, queries,
                       num_points, num_queries, indices);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Start cells of a ray batch (get_starting_point, sdfoam_model/scene.py:
// 272-282): the nearest point to each ray's origin.  A batch's rays come from
// few camera positions, so the origins are deduplicated on the GPU in an
// open-addressing hash table keyed on their bits (the reference sorts them
// with torch.unique, which synchronises with the host), each distinct
// origin's nearest point is found once, and every ray takes its origin's.
// With at most kStartBrute distinct origins the search is a scan over all
// points (one pass over the points for all of them: the same fp32 distances
// as nn_wave, ties to the smallest index), else nn_wave per origin.  Equal
// results to nn over the distinct origins for finite points and origins.

constexpr uint32_t kStartBrute = 256;
constexpr uint32_t kStartPts = 8;          // points per thread in the scan

__host__ StartLayout start_layout(uint32_t num_rays) {
    StartLayout l;
    uint64_t t = 64;
    while (t < 2ull * num_rays) t *= 2;
    l.table_slots = t;
    auto up = [](uint64_t x) { return (x + 255u) / 256u * 256u; };
    l.table = 256;
    l.uid = l.table + up(4 * t);
    l.ray_slot = l.uid + up(4 * t);
    l.uq_ray = l.ray_slot + up(4ull * num_rays);
    l.best = l.uq_ray + up(4ull * num_rays);
    l.bytes = l.best + up(8ull * num_rays);
    return l;
}

__device__ __forceinline__ uint32_t origin_hash(uint32_t x, uint32_t y, uint32_t z) {
    uint32_t h = x * 0x9e3779b1u ^ (y + 0x7f4a7c15u) * 0x85ebca77u ^ (z + 0x165667b1u) * 0xc2b2ae3du;
    h ^= h >> 15;
    h *= 0x2c1b3c6du;
    h ^= h >> 12;
    return h;
}

__device__ __forceinline__ bool same_origin(const float *__restrict__ rays, uint32_t a, uint32_t b) {
    const uint32_t *ra = reinterpret_cast<const uint32_t *>(rays + 6ull * a);
    const uint32_t *rb = reinterpret_cast<const uint32_t *>(rays + 6ull * b);
    return ra[0] == rb[0] && ra[1] == rb[1] && ra[2] == rb[2];
}

__global__ __launch_bounds__(kBlock) void start_init_kernel(uint32_t *__restrict__ counter,
                                                            uint32_t *__restrict__ table,
                                                            uint64_t slots) {
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < slots;
         i += (uint64_t)gridDim.x * kBlock)
        table[i] = kNoIndex;
    if (blockIdx.x == 0 && threadIdx.x == 0) *counter = 0u;
}

// Each ray claims the first free slot of its probe sequence or finds the
// slot of an equal origin there.  The table has at least twice as many slots
// as rays, so every probe sequence reaches a free slot or its origin's.
// Rays of one wavefront with the bits of its first ray's origin take that
// ray's slot without probing: a batch from one camera then makes one probe
// per wavefront instead of every ray contending for the same slot.
__global__ __launch_bounds__(kBlock) void start_hash_kernel(const float *__restrict__ rays,
                                                            uint32_t num_rays,
                                                            uint32_t *__restrict__ table,
                                                            uint64_t slots,
                                                            uint32_t *__restrict__ ray_slot) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= num_rays) return;
    const uint32_t *o = reinterpret_cast<const uint32_t *>(rays + 6ull * i);
    const uint32_t ox = o[0], oy = o[1], oz = o[2];
    // the first active lane's id and origin, read by every lane (before any
    // branch: a cross-lane read in a branch sees only the lanes in it)
    const uint32_t lead = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x & 63u));
    const uint32_t lx = (uint32_t)__builtin_amdgcn_readfirstlane((int)ox);
    const uint32_t ly = (uint32_t)__builtin_amdgcn_readfirstlane((int)oy);
    const uint32_t lz = (uint32_t)__builtin_amdgcn_readfirstlane((int)oz);
    const bool follower = ((threadIdx.x & 63u) != lead) & (ox == lx) & (oy == ly) & (oz == lz);
    uint64_t h = origin_hash(ox, oy, oz) & (slots - 1);
    if (!follower) {
        for (uint64_t probe = 0; probe < slots; ++probe) {
            uint32_t s = table[h];
            if (s == kNoIndex) {
                s = atomicCAS(table + h, kNoIndex, i);
                if (s == kNoIndex) break; // claimed
            }
            if (same_origin(rays, s, i)) break;
            h = (h + 1) & (slots - 1);
        }
    }
    // the first ray's slot (its probe has ended: the loop above is done)
    const uint32_t lead_slot = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)h);
    ray_slot[i] = follower ? lead_slot : (uint32_t)h;
}

// Numbers the claimed slots (the distinct origins) and resets their results.
__global__ __launch_bounds__(kBlock) void start_unique_kernel(const uint32_t *__restrict__ table,
                                                              uint64_t slots,
                                                              uint32_t *__restrict__ counter,
                                                              uint32_t *__restrict__ uid,
                                                              uint32_t *__restrict__ uq_ray,
                                                              uint64_t *__restrict__ best) {
    for (uint64_t h = (uint64_t)blockIdx.x * kBlock + threadIdx.x; h < slots;
         h += (uint64_t)gridDim.x * kBlock) {
        const uint32_t r = table[h];
        if (r == kNoIndex) continue;
        const uint32_t u = atomicAdd(counter, 1u);
        uid[h] = u;
        uq_ray[u] = r;
        best[u] = ~0ull;
    }
}

// At most kStartBrute distinct origins: every block scans kBlock * kStartPts
// points for all of them; per origin the smallest (distance bits, index)
// of the block goes into `best` with one atomic.
__global__ __launch_bounds__(kBlock) void start_brute_kernel(const float *__restrict__ points,
                                                             uint32_t num_points,
                                                             const float *__restrict__ rays,
                                                             const uint32_t *__restrict__ counter,
                                                             const uint32_t *__restrict__ uq_ray,
                                                             uint64_t *__restrict__ best) {
    __shared__ float q[kStartBrute][3];
    __shared__ unsigned long long slot[kStartBrute];
    const uint32_t count = *counter;
    if (count == 0 || count > kStartBrute) return; // the whole grid
    for (uint32_t u = threadIdx.x; u < count; u += kBlock) {
        const float *o = rays + 6ull * uq_ray[u];
        q[u][0] = o[0];
        q[u][1] = o[1];
        q[u][2] = o[2];
        slot[u] = ~0ull;
    }
    __syncthreads();
    const uint64_t p0 = (uint64_t)blockIdx.x * kBlock * kStartPts;
    float px[kStartPts], py[kStartPts], pz[kStartPts];
#pragma unroll
    for (uint32_t k = 0; k < kStartPts; ++k) {
        const uint64_t j = p0 + (uint64_t)k * kBlock + threadIdx.x;
        const bool ok = j < num_points;
        px[k] = ok ? points[3 * j] : 0.0f;
        py[k] = ok ? points[3 * j + 1] : 0.0f;
        pz[k] = ok ? points[3 * j + 2] : 0.0f;
    }
    for (uint32_t u = 0; u < count; ++u) {
        const float qx = q[u][0], qy = q[u][1], qz = q[u][2];
        unsigned long long key = ~0ull;
#pragma unroll
        for (uint32_t k = 0; k < kStartPts; ++k) {
            const uint64_t j = p0 + (uint64_t)k * kBlock + threadIdx.x;
            const float dx = px[k] - qx, dy = py[k] - qy, dz = pz[k] - qz;
            const float d = sqrtf(sdf_dot3(dx, dy, dz, dx, dy, dz));
            const unsigned long long c =
                ((unsigned long long)__builtin_bit_cast(uint32_t, d) << 32) | (uint32_t)j;
            if (j < num_points && d == d && c < key) key = c; // NaN: no candidate
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned long long o = __shfl_xor(key, off, 64);
            key = o < key ? o : key;
        }
        if ((threadIdx.x & 63u) == 0 && key != ~0ull) atomicMin(slot + u, key);
    }
    __syncthreads();
    for (uint32_t u = threadIdx.x; u < count; u += kBlock)
        if (slot[u] != ~0ull) atomicMin(reinterpret_cast<unsigned long long *>(best) + u, slot[u]);
}

// More distinct origins: one tree search per origin, the waves of the grid
// taking the origins in turn.
__global__ __launch_bounds__(kNNBlock) void start_tree_kernel(const float *__restrict__ points,
                                                              uint32_t num_points,
                                                              const float *__restrict__ tree,
                                                              const float *__restrict__ rays,
                                                              const uint32_t *__restrict__ counter,
                                                              const uint32_t *__restrict__ uq_ray,
                                                              uint64_t *__restrict__ best) {
    __shared__ NNShared sh;
    const uint32_t count = *counter;
    if (count <= kStartBrute) return; // the whole grid
    const uint32_t td = ilog2_u32(pow2_up(num_points));
    nn_load_top(tree, td, sh);
    const uint32_t wave = threadIdx.x >> 6;
    for (uint32_t u = blockIdx.x * kNNWaves + wave; u < count; u += gridDim.x * kNNWaves) {
        const float *o = rays + 6ull * uq_ray[u];
        const uint32_t r = nn_wave(points, tree, num_points, td, o[0], o[1], o[2], sh, wave);
        if ((threadIdx.x & 63u) == 0) best[u] = r;
    }
}

__global__ __launch_bounds__(kBlock) void start_scatter_kernel(uint32_t num_rays,
                                                               const uint32_t *__restrict__ ray_slot,
                                                               const uint32_t *__restrict__ uid,
                                                               const uint64_t *__restrict__ best,
                                                               uint32_t *__restrict__ start) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= num_rays) return;
    const uint64_t b = best[uid[ray_slot[i]]];
    start[i] = b == ~0ull ? 0u : (uint32_t)b;
}

hipError_t launch_start_points(const float *rays, uint32_t num_rays, const float *points,
                               uint32_t num_points, const float *tree, uint32_t *start,
                               void *scratch, hipStream_t stream) {
    if (num_rays == 0) return hipSuccess;
    const StartLayout l = start_layout(num_rays);
    char *base = static_cast<char *>(scratch);
    uint32_t *counter = reinterpret_cast<uint32_t *>(base);
    uint32_t *table = reinterpret_cast<uint32_t *>(base + l.table);
    uint32_t *uid = reinterpret_cast<uint32_t *>(base + l.uid);
    uint32_t *ray_slot = reinterpret_cast<uint32_t *>(base + l.ray_slot);
    uint32_t *uq_ray = reinterpret_cast<uint32_t *>(base + l.uq_ray);
    uint64_t *best = reinterpret_cast<uint64_t *>(base + l.best);
    const uint32_t slot_blocks = (uint32_t)std::min<uint64_t>((l.table_slots + kBlock - 1) / kBlock, 4096);
    const uint32_t ray_blocks = (num_rays + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(start_init_kernel, dim3(slot_blocks), dim3(kBlock), 0, stream, counter, table,
                       l.table_slots);
    hipLaunchKernelGGL(start_hash_kernel, dim3(ray_blocks), dim3(kBlock), 0, stream, rays, num_rays,
                       table, l.table_slots, ray_slot);
    hipLaunchKernelGGL(start_unique_kernel, dim3(slot_blocks), dim3(kBlock), 0, stream, table,
                       l.table_slots, counter, uid, uq_ray, best);
    const uint32_t point_blocks = (uint32_t)(((uint64_t)num_points + kBlock * kStartPts - 1) /
                                             (kBlock * kStartPts));
    hipLaunchKernelGGL(start_brute_kernel, dim3(point_blocks), dim3(kBlock), 0, stream, points,
                       num_points, rays, counter, uq_ray, best);
    hipLaunchKernelGGL(start_tree_kernel, dim3(kNNMaxBlocks), dim3(kNNBlock), 0, stream, points,
                       num_points, tree, rays, counter, uq_ray, best);
    hipLaunchKernelGGL(start_scatter_kernel, dim3(ray_blocks), dim3(kBlock), 0, stream, num_rays,
                       ray_slot, uid, best, start);
    return hipGetLastError();
}

} // namespace sdfoam_hip
