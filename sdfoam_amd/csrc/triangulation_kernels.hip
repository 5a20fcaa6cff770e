// Kernels that serve the triangulation side of the foam: per-point farthest
// Delaunay neighbour and mean half-edge length (the densification step's
// inputs, src/delaunay/triangulation_ops.cu:8-44).
#include "trace_kernels.h"

namespace sdfoam_hip {

namespace {

// One lane per point over its CSR row.  The reference accumulates
// `sum += 0.5 * distance` with a double constant, i.e. in double rounded
// back to float at every step; that is kept.  Neighbours out of range are
// skipped (the reference reads them).
__global__ __launch_bounds__(256) void farthest_neighbor_kernel(
    const float *__restrict__ points, uint32_t num_points, const uint32_t *__restrict__ adj,
    const uint32_t *__restrict__ offs, uint32_t num_adj, uint32_t *__restrict__ indices,
    float *__restrict__ cell_radius) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= num_points) return;
    const float px = points[3ull * i], py = points[3ull * i + 1], pz = points[3ull * i + 2];
    uint32_t beg = offs[i], end = offs[i + 1];
    if (end > num_adj) end = num_adj;
    if (beg > end) beg = end;
    const uint32_t nf = offs[i + 1] - offs[i];
    uint32_t far_idx = kNoIndex;
    float sum = 0.0f, max_d = 0.0f;
    for (uint32_t k = beg; k < end; ++k) {
        const uint32_t q = adj[k];
        if (q >= num_points) continue;
        const float dx = points[3ull * q] - px;
        const float dy = points[3ull * q + 1] - py;
        const float dz = points[3ull * q + 2] - pz;
        const float d = sqrtf(sdf_dot3(dx, dy, dz, dx, dy, dz));
        sum = (float)((double)sum + 0.5 * (double)d);
        if (d > max_d) {
            max_d = d;
            far_idx = q;
        }
    }
    indices[i] = far_idx;
    cell_radius[i] = sum / (float)nf;
}

} // namespace

hipError_t launch_farthest_neighbor(const float *points, uint32_t num_points, const uint32_t *adj,
                                    const uint32_t *offs, uint32_t num_adj, uint32_t *indices,
                                    float *cell_radius, hipStream_t stream) {
    if (num_points == 0) return hipSuccess;
    hipLaunchKernelGGL(farthest_neighbor_kernel, dim3((num_points + 255u) / 256u), dim3(256), 0,
                       stream, points, num_points, adj, offs, num_adj, indices, cell_radius);
    return hipGetLastError();
}

} // namespace sdfoam_hip
