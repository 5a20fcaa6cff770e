// Host entry of delaunay_gpu.hip beside the ones trace_kernels.h declares:
// the certification of a small point set with every open cell clipped by
// every point (the open points' own tetrahedra, hull cells included).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace sdfoam_hip {

// launch_delaunay_certify with the clipping box grown to 1e8 extents and a
// cell the grid search leaves open clipped by every point; a hull cell's
// vertices off the box are reported too (the point is still listed as open).
hipError_t launch_delaunay_certify_exhaustive(const float *points, uint32_t num_points,
                                              uint32_t *reports, uint64_t report_capacity,
                                              uint32_t *open, uint64_t counts[5], void *scratch,
                                              size_t scratch_bytes, hipStream_t stream);

} // namespace sdfoam_hip
