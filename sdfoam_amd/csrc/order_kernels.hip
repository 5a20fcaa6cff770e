// Launch order for rays given in no particular order (training batches of
// rays drawn at random over many cameras).  The tracer's wavefront-level
// coherence (shared gathers, grouped gradient updates, equal walk lengths)
// needs neighbouring lanes to trace neighbouring rays; sorting by start cell,
// then by direction along a Z-order curve, restores it.  The permutation is
// stable (radix sort) and the same for the forward and its backward.
#include <rocprim/device/device_radix_sort.hpp>

#include "trace_kernels.h"

namespace sdfoam_hip {

namespace {

__device__ __forceinline__ uint32_t spread_bits16(uint32_t x) {
    x &= 0xffffu;
    x = (x | (x << 8)) & 0x00ff00ffu;
    x = (x | (x << 4)) & 0x0f0f0f0fu;
    x = (x | (x << 2)) & 0x33333333u;
    x = (x | (x << 1)) & 0x55555555u;
    return x;
}

__device__ __forceinline__ uint32_t quantize16(float a) {
    // a in [-1, 1] -> [0, 65535]; NaN -> 0
    const float q = fminf(fmaxf(fmaf(a, 32767.5f, 32767.5f), 0.0f), 65535.0f);
    return (uint32_t)q;
}

// key = start cell << 32 | Morton(octahedral direction, 16 + 16 bits)
__global__ __launch_bounds__(256) void ray_key_kernel(const float *__restrict__ rays,
                                                      const uint32_t *__restrict__ start,
                                                      uint32_t n, uint64_t *__restrict__ keys,
                                                      uint32_t *__restrict__ index) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const float dx = rays[6ull * i + 3], dy = rays[6ull * i + 4], dz = rays[6ull * i + 5];
    const float l1 = fabsf(dx) + fabsf(dy) + fabsf(dz);
    float u = 0.0f, v = 0.0f;
    if (l1 > 0.0f && l1 < 3.0e38f) {
        u = dx / l1;
        v = dy / l1;
        if (dz < 0.0f) {
            const float fu = (1.0f - fabsf(v)) * (u >= 0.0f ? 1.0f : -1.0f);
            const float fv = (1.0f - fabsf(u)) * (v >= 0.0f ? 1.0f : -1.0f);
            u = fu;
            v = fv;
        }
    }
    const uint32_t morton = spread_bits16(quantize16(u)) | (spread_bits16(quantize16(v)) << 1);
    keys[i] = ((uint64_t)start[i] << 32) | morton;
    index[i] = i;
}

uint32_t key_end_bit(uint32_t num_points) {
    uint32_t bits = 1;
    // start cells are < num_points, or num_points and above for invalid ones
    // (they sort last); cover values up to 2 * num_points
    while (bits < 32 && (1ull << bits) <= 2ull * num_points) ++bits;
    return 32u + bits;
}

size_t align256(size_t x) { return (x + 255u) & ~(size_t)255u; }

} // namespace

size_t ray_order_scratch_bytes(uint32_t num_points, uint32_t num_rays) {
    size_t temp = 0;
    const uint64_t *k = nullptr;
    uint64_t *ko = nullptr;
    const uint32_t *v = nullptr;
    uint32_t *vo = nullptr;
    if (rocprim::radix_sort_pairs(nullptr, temp, k, ko, v, vo, num_rays, 0u,
                                  key_end_bit(num_points)) != hipSuccess)
        return 0;
    return align256(8ull * num_rays) * 2 + align256(4ull * num_rays) + align256(temp);
}

hipError_t launch_ray_order(uint32_t num_points, uint32_t num_rays, const float *rays,
                            const uint32_t *start, uint32_t *order, void *scratch,
                            size_t scratch_bytes, hipStream_t stream) {
    if (num_rays == 0) return hipSuccess;
    char *p = static_cast<char *>(scratch);
    uint64_t *keys = reinterpret_cast<uint64_t *>(p);
    p += align256(8ull * num_rays);
    uint64_t *keys_sorted = reinterpret_cast<uint64_t *>(p);
    p += align256(8ull * num_rays);
    uint32_t *index = reinterpret_cast<uint32_t *>(p);
    p += align256(4ull * num_rays);
    const size_t used = (size_t)(p - static_cast<char *>(scratch));
    if (used > scratch_bytes) return hipErrorInvalidValue;
    size_t temp = scratch_bytes - used;
    const uint32_t grid = (num_rays + 255u) / 256u;
    hipLaunchKernelGGL(ray_key_kernel, dim3(grid), dim3(256), 0, stream, rays, start, num_rays,
                       keys, index);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return rocprim::radix_sort_pairs(p, temp, keys, keys_sorted, index, order, num_rays, 0u,
                                     key_end_bit(num_points), stream);
}

} // namespace sdfoam_hip
