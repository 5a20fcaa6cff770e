// Start-cell lookup: implicit AABB tree over point pairs and an exact
// nearest-neighbour search, for gfx950.
//
// Tree layout (src/aabb_tree/aabb_tree.cuh:35-43): with td = log2(pow2(N)),
// the node (depth d, index i) is box number 2^td - 2^(d+1) + i of a
// [pow2(N), 2, 3] array (min xyz, max xyz); the leaves (depth td-1) bound
// consecutive point pairs, the last point repeated as padding.
//
// The search gives one wave64 to a query.  The wave tests a group of up to
// 64 sibling nodes per step (one per lane), six tree levels apart, and keeps a
// depth-first stack of node groups in LDS: the group under the best lane is
// visited first, so the first leaf visit already gives a tight bound, and
// every group whose lower bound exceeds the best distance is skipped.  The fp32
// box distance is a lower bound of the fp32 point distance (rounding is
// monotone), so the result is the exact fp32 nearest neighbour; ties go to
// the smallest index.
#include "trace_kernels.h"

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

constexpr int kNNWaves = kBlock / 64;
// The stack holds, per tree depth visited (at most ceil(32 / 6) of them), the
// <= 63 pending sibling groups of the group being expanded, plus one.
constexpr int kNNStack = 512;

struct NNItem {
    uint32_t depth_size; // depth | (group size << 8)
    uint32_t first;      // first node of the group
    float lb;            // lower bound of the parent node
    uint32_t pad;
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

__global__ __launch_bounds__(kBlock) void nn_kernel(const float *__restrict__ points,
                                                    const float *__restrict__ tree,
                                                    const float *__restrict__ queries,
                                                    uint32_t num_points, uint32_t num_queries,
                                                    uint32_t *__restrict__ indices) {
    __shared__ NNItem stack_all[kNNWaves][kNNStack];
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t qi = blockIdx.x * kNNWaves + wave;
    if (qi >= num_queries) return; // uniform per wave
    NNItem *st = stack_all[wave];
    const float qx = queries[3ull * qi], qy = queries[3ull * qi + 1], qz = queries[3ull * qi + 2];
    const uint32_t td = ilog2_u32(pow2_up(num_points));
    const uint64_t n2 = 1ull << td;
    const float kInf = __builtin_bit_cast(float, 0x7f800000u);

    float best = kInf;
    uint32_t best_idx = kNoIndex;
    int sp = 0;
    {
        const uint32_t d0 = td < 6 ? td : 6;
        if (lane == 0) st[0] = NNItem{d0 | ((1u << d0) << 8), 0u, 0.0f, 0u};
        sp = 1;
    }
    __builtin_amdgcn_wave_barrier();
    while (sp > 0) {
        --sp;
        const NNItem it = st[sp];
        __builtin_amdgcn_wave_barrier();
        if (it.lb > best) continue;
        const uint32_t d = it.depth_size & 0xffu;
        const uint32_t size = it.depth_size >> 8;
        const uint32_t node = it.first + lane;
        bool valid = lane < size;
        if (d == td) {
            valid = valid && node < num_points;
            float dist = valid ? point_dist(points + 3ull * node, qx, qy, qz) : kInf;
            uint32_t idx = valid ? node : kNoIndex;
            wave_argmin(dist, idx);
            if (dist < best || (dist == best && idx < best_idx)) {
                best = dist;
                best_idx = idx;
            }
            continue;
        }
        const float *box = tree + 6ull * ((n2 - (2ull << d)) + node);
        const float lb = valid ? box_dist(box, qx, qy, qz) : kInf;
        const bool keep = valid && !(lb > best);
        float bl = keep ? lb : kInf;
        uint32_t bi = keep ? lane : 64u;
        wave_argmin(bl, bi);
        const uint32_t dc = (d + 6 < td) ? d + 6 : td;
        const uint32_t csize = 1u << (dc - d);
        const uint32_t cfirst = node << (dc - d);
        const bool push = keep && lane != bi;
        const uint64_t pm = __ballot(push);
        const uint64_t below = (lane == 0) ? 0ull : (pm & (~0ull >> (64 - lane)));
        const int pos = sp + (int)__popcll(below);
        const int npush = (int)__popcll(pm) + (bi < 64u ? 1 : 0);
        if (sp + npush > kNNStack) break; // unreachable: the stack bound is kNNStack
        if (push) st[pos] = NNItem{dc | (csize << 8), cfirst, lb, 0u};
        if (bi < 64u && lane == bi) st[sp + npush - 1] = NNItem{dc | (csize << 8), cfirst, lb, 0u};
        sp += npush;
        __builtin_amdgcn_wave_barrier();
    }
    if (lane == 0) indices[qi] = best_idx == kNoIndex ? 0u : best_idx;
}

hipError_t launch_nn(const float *points, const float *tree, const float *queries,
                     uint32_t num_points, uint32_t num_queries, uint32_t *indices,
                     hipStream_t stream) {
    if (num_queries == 0) return hipSuccess;
    hipLaunchKernelGGL(nn_kernel, dim3((num_queries + kNNWaves - 1) / kNNWaves), dim3(kBlock), 0,
                       stream, points, tree, queries, num_points, num_queries, indices);
    return hipGetLastError();
}

} // namespace sdfoam_hip
