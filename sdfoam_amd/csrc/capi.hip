// extern "C" entry points of libsdfoam_hip.so (declared in
// include/sdfoam_hip.h).  Argument checks, stream plumbing, optional kernel
// timing; no device allocation.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "delaunay_gpu.h"
#include "trace_kernels.h"

using namespace sdfoam_hip;

namespace {
thread_local char g_err[512] = "";
} // namespace

namespace sdfoam_hip {

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char *where) {
    return fail(SDF_E_HIP, "%s: %s", where, hipGetErrorString(e));
}

} // namespace sdfoam_hip

namespace {

// ---- optional kernel timing ----------------------------------------------
// When enabled, every kernel launch is bracketed by two HIP events recorded
// on its stream, kept in a ring until sdf_timing_collect reads them.
constexpr int kRing = 512;
struct TimedLaunch {
    hipEvent_t begin;
    hipEvent_t end;
    int kind;
};
bool g_timing = false;
TimedLaunch g_ring[kRing] = {};
int g_ring_n = 0;
int g_open = -1;

void tbegin(int kind, hipStream_t s) {
    g_open = -1;
    if (!g_timing || g_ring_n >= kRing) return;
    TimedLaunch &t = g_ring[g_ring_n];
    if (!t.begin && hipEventCreate(&t.begin) != hipSuccess) return;
    if (!t.end && hipEventCreate(&t.end) != hipSuccess) return;
    t.kind = kind;
    if (hipEventRecord(t.begin, s) != hipSuccess) return;
    g_open = g_ring_n;
}

void tend(hipStream_t s) {
    if (g_open < 0) return;
    if (hipEventRecord(g_ring[g_open].end, s) == hipSuccess) g_ring_n = g_open + 1;
    g_open = -1;
}

int check_scene(int sh_degree, const sdf_trace_settings *settings, uint32_t num_points,
                const float *points, const float *attributes, uint32_t adjacency_size,
                const uint32_t *adj, const uint32_t *offs, uint32_t num_rays, const float *rays,
                const uint32_t *start, const float *sharpness, void *scratch,
                size_t scratch_bytes) {
    if (sh_degree < 0 || sh_degree > 3) return fail(SDF_E_INVALID, "Unsupported SH degree");
    if (!settings) return fail(SDF_E_INVALID, "settings must not be NULL");
    if (settings->alpha_mode != SDF_ALPHA_STANDARD && settings->alpha_mode != SDF_ALPHA_NEUS)
        return fail(SDF_E_INVALID, "alpha_mode must be 0 (standard) or 1 (sdfoam)");
    if (settings->attr_type != SDF_ATTR_F32 && settings->attr_type != SDF_ATTR_F16)
        return fail(SDF_E_INVALID, "attr_type must be 0 (float32) or 1 (float16)");
    const int D = 1 + 3 * (sh_degree + 1) * (sh_degree + 1);
    if (settings->sdf_channel >= D)
        return fail(SDF_E_INVALID, "sdf_channel %d out of range for attribute dim %d",
                    settings->sdf_channel, D);
    if (settings->ray_image_width != 0 && num_rays % settings->ray_image_width != 0)
        return fail(SDF_E_INVALID, "ray_image_width %u does not divide the %u rays",
                    settings->ray_image_width, num_rays);
    if (num_points == 0) return fail(SDF_E_INVALID, "num_points must be positive");
    if (!points || !attributes || !offs || (!adj && adjacency_size > 0))
        return fail(SDF_E_INVALID, "scene pointers must not be NULL");
    if (num_rays > 0 && (!rays || !start))
        return fail(SDF_E_INVALID, "rays and start_point_index must not be NULL");
    if (!sharpness) return fail(SDF_E_INVALID, "sharpness must not be NULL");
    const size_t need = sdf_trace_scratch_bytes(num_points, adjacency_size);
    if (!scratch || scratch_bytes < need)
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    if ((reinterpret_cast<uintptr_t>(scratch) & 7u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 8-byte aligned");
    return SDF_OK;
}

SceneView make_scene(uint32_t num_points, const float *points, const float *attributes,
                     uint32_t adjacency_size, const uint32_t *adj, const uint32_t *offs,
                     void *scratch) {
    SceneView sc;
    sc.points = points;
    sc.attrs = attributes;
    sc.adj = adj;
    sc.offs = offs;
    sc.diff = static_cast<const uint2 *>(scratch);
    sc.cells = nullptr;
    sc.num_points = num_points;
    sc.num_adj = adjacency_size;
    return sc;
}

// plan == NULL: neither aid.  A walk record must hold
// sdf_walk_record_pool_bytes(num_rays, ray_image_width, walk_budget,
// walk_record_chunks) bytes; a ray order needs ray_image_width == 0.
int check_plan(const sdf_trace_plan *plan, uint32_t num_rays, uint32_t ray_image_width,
               WalkRecordArgs &rec, const uint32_t *&order) {
    rec = WalkRecordArgs{};
    order = nullptr;
    if (!plan) return SDF_OK;
    if (plan->ray_order) {
        if (ray_image_width != 0)
            return fail(SDF_E_INVALID, "a ray order needs ray_image_width == 0");
        order = plan->ray_order;
    }
    if (!plan->walk_record) return SDF_OK;
    if (plan->walk_budget == 0) return fail(SDF_E_INVALID, "walk record budget must be positive");
    const uint32_t tiles = num_ray_tiles(num_rays, ray_image_width);
    const uint64_t pool = record_pool_chunks(tiles, plan->walk_budget, plan->walk_record_chunks);
    if (pool >= kNoIndex) return fail(SDF_E_INVALID, "walk record pool too large");
    const uint64_t need = walk_record_bytes_for(tiles, plan->walk_budget, pool);
    if (plan->walk_record_bytes < need)
        return fail(SDF_E_INVALID, "walk record must hold %llu bytes (got %zu)",
                    (unsigned long long)need, plan->walk_record_bytes);
    if ((reinterpret_cast<uintptr_t>(plan->walk_record) & 255u) != 0)
        return fail(SDF_E_INVALID, "walk record must be 256-byte aligned");
    char *base = static_cast<char *>(plan->walk_record);
    rec.counters = reinterpret_cast<uint32_t *>(base);
    rec.chunks = reinterpret_cast<uint32_t *>(base + kRecordHeadBytes);
    rec.entries =
        reinterpret_cast<uint2 *>(base + kRecordHeadBytes + walk_record_table_bytes(tiles, plan->walk_budget));
    // the pool is a multiple of 8 chunks of 8 KB, so the colours stay aligned
    rec.colors = reinterpret_cast<float4 *>(rec.entries + pool * kChunkEntries);
    rec.budget = plan->walk_budget;
    rec.pool = (uint32_t)pool;
    return SDF_OK;
}

int trace_forward_impl(const sdf_trace_plan *plan, int sh_degree,
                       const sdf_trace_settings *settings, uint32_t num_points,
                       const float *points, const float *attributes, uint32_t adjacency_size,
                       const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets,
                       uint32_t num_rays, const float *rays, const uint32_t *start_point_index,
                       uint32_t num_depth_quantiles, const float *depth_quantiles,
                       float *ray_rgba, float *quantile_depths,
                       uint32_t *quantile_point_indices, uint32_t *num_intersections,
                       float *point_contribution, const float *sharpness, float *alpha_output,
                       void *scratch, size_t scratch_bytes, void *stream) {
    int rc = check_scene(sh_degree, settings, num_points, points, attributes, adjacency_size,
                         point_adjacency, point_adjacency_offsets, num_rays, rays,
                         start_point_index, sharpness, scratch, scratch_bytes);
    if (rc != SDF_OK) return rc;
    if (num_rays > 0 && !ray_rgba) return fail(SDF_E_INVALID, "ray_rgba must not be NULL");
    if (num_depth_quantiles > 0 && (!depth_quantiles || !quantile_depths || !quantile_point_indices))
        return fail(SDF_E_INVALID, "depth buffers must not be NULL when num_depth_quantiles > 0");
    const bool half = settings->attr_type == SDF_ATTR_F16;
    if ((reinterpret_cast<uintptr_t>(ray_rgba) & (half ? 7u : 15u)) != 0)
        return fail(SDF_E_INVALID, "ray_rgba must be %d-byte aligned", half ? 8 : 16);
    if (half && (reinterpret_cast<uintptr_t>(point_contribution) & 3u) != 0)
        return fail(SDF_E_INVALID, "fp16 point_contribution must be 4-byte aligned");
    WalkRecordArgs rec = {};
    const uint32_t *order = nullptr;
    rc = check_plan(plan, num_rays, settings->ray_image_width, rec, order);
    if (rc != SDF_OK) return rc;
    uint32_t *cells = nullptr;
    if (plan && plan->cell_table) {
        const size_t need = sdf_cell_table_bytes(sh_degree, settings->attr_type, num_points);
        if (plan->cell_table_bytes < need)
            return fail(SDF_E_INVALID, "cell table must hold %zu bytes (got %zu)", need,
                        plan->cell_table_bytes);
        if ((reinterpret_cast<uintptr_t>(plan->cell_table) & 255u) != 0)
            return fail(SDF_E_INVALID, "cell table must be 256-byte aligned");
        cells = static_cast<uint32_t *>(plan->cell_table);
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    FwdArgs a = {};
    a.scene = make_scene(num_points, points, attributes, adjacency_size, point_adjacency,
                         point_adjacency_offsets, scratch);
    hipError_t e;
    if (cells) {
        // the offset table and the cell table in one pass
        tbegin(SDF_KERNEL_SCENE_PREP, s);
        e = launch_scene_prep(sh_degree, half, a.scene, cells, static_cast<uint2 *>(scratch), s);
        tend(s);
        if (e != hipSuccess) return hip_fail(e, "scene preparation");
        a.scene.cells = cells;
    } else {
        tbegin(SDF_KERNEL_PREFETCH, s);
        e = launch_prefetch_diff(points, num_points, adjacency_size, point_adjacency,
                                 point_adjacency_offsets, static_cast<uint2 *>(scratch), s);
        tend(s);
        if (e != hipSuccess) return hip_fail(e, "prefetch_adjacent_diff");
    }
    if (num_rays == 0) return SDF_OK;
    a.record = rec;
    a.order = order;
    if (rec.entries) {
        const uint64_t words =
            walk_record_waves(num_ray_tiles(num_rays, settings->ray_image_width)) * chunk_slots(rec.budget);
        e = launch_record_reset(rec, words, s);
        if (e != hipSuccess) return hip_fail(e, "walk record reset");
    }
    a.settings = *settings;
    a.rays = rays;
    a.num_rays = num_rays;
    a.num_tiles = num_ray_tiles(num_rays, settings->ray_image_width);
    a.start = start_point_index;
    a.num_quantiles = num_depth_quantiles;
    a.quantiles = num_depth_quantiles ? depth_quantiles : nullptr;
    a.sharpness = sharpness;
    a.rgba = ray_rgba;
    a.depth = quantile_depths;
    a.depth_indices = quantile_point_indices;
    a.num_intersections = num_intersections;
    a.contribution = point_contribution;
    a.alpha_out = alpha_output;
    tbegin(SDF_KERNEL_FORWARD, s);
    e = launch_forward(sh_degree, a, settings->alpha_mode == SDF_ALPHA_NEUS, false, half, s);
    tend(s);
    if (e != hipSuccess) return hip_fail(e, "forward");
    return SDF_OK;
}

int trace_backward_impl(const sdf_trace_plan *plan, int sh_degree,
                        const sdf_trace_settings *settings, uint32_t num_points,
                        const float *points, const float *attributes, uint32_t adjacency_size,
                        const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets,
                        uint32_t num_rays, const float *rays, const uint32_t *start_point_index,
                        uint32_t num_depth_quantiles, const float *depth_quantiles,
                        const uint32_t *quantile_point_indices, const float *ray_rgba,
                        const float *ray_rgba_grad, const float *depth_grad,
                        const float *ray_error, float *points_grad, float *attribute_grad,
                        float *point_error, const float *sharpness, float *sharpness_grad,
                        void *scratch, size_t scratch_bytes, void *stream) {
    int rc = check_scene(sh_degree, settings, num_points, points, attributes, adjacency_size,
                         point_adjacency, point_adjacency_offsets, num_rays, rays,
                         start_point_index, sharpness, scratch, scratch_bytes);
    if (rc != SDF_OK) return rc;
    const bool neus = settings->alpha_mode == SDF_ALPHA_NEUS;
    if (!points_grad || !attribute_grad)
        return fail(SDF_E_INVALID, "points_grad and attribute_grad must not be NULL");
    if (num_rays > 0 && (!ray_rgba || !ray_rgba_grad))
        return fail(SDF_E_INVALID, "ray_rgba and ray_rgba_grad must not be NULL");
    if (num_depth_quantiles > 0 && (!depth_quantiles || !depth_grad))
        return fail(SDF_E_INVALID, "depth_grad must be provided if depth_quantiles is provided");
    if (!neus && num_depth_quantiles > 0 && !quantile_point_indices)
        return fail(SDF_E_INVALID, "depth_indices must be provided in standard mode");
    const bool half = settings->attr_type == SDF_ATTR_F16;
    if (((reinterpret_cast<uintptr_t>(ray_rgba) | reinterpret_cast<uintptr_t>(ray_rgba_grad)) &
         (half ? 7u : 15u)) != 0)
        return fail(SDF_E_INVALID, "ray_rgba and ray_rgba_grad must be %d-byte aligned",
                    half ? 8 : 16);
    if (half && ((reinterpret_cast<uintptr_t>(attribute_grad) |
                  reinterpret_cast<uintptr_t>(point_error)) & 3u) != 0)
        return fail(SDF_E_INVALID, "fp16 attribute_grad and point_error must be 4-byte aligned");
    WalkRecordArgs rec = {};
    const uint32_t *order = nullptr;
    rc = check_plan(plan, num_rays, settings->ray_image_width, rec, order);
    if (rc != SDF_OK) return rc;
    float *accum = nullptr;
    if (plan && plan->grad_accum) {
        const size_t need = sdf_grad_accum_bytes(sh_degree, num_points);
        if (plan->grad_accum_bytes < need)
            return fail(SDF_E_INVALID, "gradient accumulator must hold %zu bytes (got %zu)", need,
                        plan->grad_accum_bytes);
        if ((reinterpret_cast<uintptr_t>(plan->grad_accum) & 255u) != 0)
            return fail(SDF_E_INVALID, "gradient accumulator must be 256-byte aligned");
        accum = static_cast<float *>(plan->grad_accum);
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    if (!(plan && plan->scratch_ready)) {
        tbegin(SDF_KERNEL_PREFETCH, s);
        e = launch_prefetch_diff(points, num_points, adjacency_size, point_adjacency,
                                 point_adjacency_offsets, static_cast<uint2 *>(scratch), s);
        tend(s);
        if (e != hipSuccess) return hip_fail(e, "prefetch_adjacent_diff");
    }
    if (num_rays == 0) return SDF_OK;
    if (accum) {
        tbegin(SDF_KERNEL_GRAD_CLEAR, s);
        e = launch_grad_clear(sh_degree, accum, num_points, s);
        tend(s);
        if (e != hipSuccess) return hip_fail(e, "gradient accumulator clear");
    }
    BwdArgs a = {};
    a.record = rec;
    a.order = order;
    a.scene = make_scene(num_points, points, attributes, adjacency_size, point_adjacency,
                         point_adjacency_offsets, scratch);
    a.settings = *settings;
    a.rays = rays;
    a.num_rays = num_rays;
    a.num_tiles = num_ray_tiles(num_rays, settings->ray_image_width);
    a.start = start_point_index;
    a.num_quantiles = num_depth_quantiles;
    a.quantiles = num_depth_quantiles ? depth_quantiles : nullptr;
    a.depth_indices = quantile_point_indices;
    a.rgba = ray_rgba;
    a.rgba_grad = ray_rgba_grad;
    a.depth_grad = num_depth_quantiles ? depth_grad : nullptr;
    a.ray_error = point_error ? ray_error : nullptr;
    a.sharpness = sharpness;
    a.points_grad = points_grad;
    a.attr_grad = attribute_grad;
    a.point_error = ray_error ? point_error : nullptr;
    a.sharpness_grad = sharpness_grad;
    a.accum = accum;
    tbegin(SDF_KERNEL_BACKWARD, s);
    e = launch_backward(sh_degree, a, neus, false, half, s);
    tend(s);
    if (e != hipSuccess) return hip_fail(e, "backward");
    if (accum) {
        tbegin(SDF_KERNEL_GRAD_FINALIZE, s);
        e = launch_grad_finalize(sh_degree, accum, num_points, attribute_grad, points_grad,
                                 a.point_error, half, s);
        tend(s);
        if (e != hipSuccess) return hip_fail(e, "gradient accumulator finalize");
    }
    return SDF_OK;
}

} // namespace

// ---- the forward for callers that cannot allocate -------------------------
// sdf_trace_forward_noalloc keeps the fp16 offset table in this file-scope
// device array instead of caller scratch: every GPU the library runs on holds
// its own copy until the process ends.  In host code the array's name is only
// a host-side stand-in; kernels get the device address hipGetSymbolAddress
// gives for the current device, looked up on the entry point's first call on
// that device and kept per device.  The prefetch pass rewrites every entry
// the walk reads (the padding included) on each call, so nothing has to start
// at zero.
static __device__ __align__(256) uint8_t noalloc_scratch[SDF_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void *g_noalloc_ptr[kMaxDevices] = {};

// Device address of noalloc_scratch on the current device.
int noalloc_scratch_ptr(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return fail(SDF_E_INVALID, "device %d: the library keeps scratch for devices 0..%d", dev,
                    kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(noalloc_scratch)");
        if (!p) return fail(SDF_E_HIP, "hipGetSymbolAddress(noalloc_scratch) gave NULL");
        g_noalloc_ptr[dev] = p;
    }
    *out = g_noalloc_ptr[dev];
    return SDF_OK;
}

} // namespace

extern "C" {

const char *sdf_version(void) { return "sdfoam_hip 0.1 (gfx950)"; }

const char *sdf_last_error(void) { return g_err; }

int sdf_attribute_dim(int sh_degree) {
    if (sh_degree < 0 || sh_degree > 3) return -1;
    return 1 + 3 * (sh_degree + 1) * (sh_degree + 1);
}

size_t sdf_cell_table_bytes(int sh_degree, int attr_type, uint32_t num_points) {
    if (sh_degree < 0 || sh_degree > 3) return 0;
    if (attr_type != SDF_ATTR_F32 && attr_type != SDF_ATTR_F16) return 0;
    return (size_t)num_points * cell_record_bytes(sh_degree, attr_type == SDF_ATTR_F16 ? 2 : 4);
}

size_t sdf_grad_accum_bytes(int sh_degree, uint32_t num_points) {
    if (sh_degree < 0 || sh_degree > 3) return 0;
    return (size_t)num_points * accum_stride(sh_degree) * sizeof(float);
}

size_t sdf_trace_scratch_bytes(uint32_t num_points, uint32_t adjacency_size) {
    (void)num_points;
    return ((size_t)adjacency_size + kDiffPad) * 8u;
}

int sdf_prefetch_adjacent_diff(const float *points, uint32_t num_points, uint32_t adjacency_size,
                               const uint32_t *point_adjacency,
                               const uint32_t *point_adjacency_offsets, uint16_t *adjacent_diff,
                               void *stream) {
    if (!points || !point_adjacency_offsets || !adjacent_diff ||
        (!point_adjacency && adjacency_size > 0))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    if (num_points == 0) return fail(SDF_E_INVALID, "num_points must be positive");
    if ((reinterpret_cast<uintptr_t>(adjacent_diff) & 7u) != 0)
        return fail(SDF_E_INVALID, "adjacent_diff must be 8-byte aligned");
    hipError_t e = launch_prefetch_diff(points, num_points, adjacency_size, point_adjacency,
                                        point_adjacency_offsets,
                                        reinterpret_cast<uint2 *>(adjacent_diff),
                                        static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "prefetch_adjacent_diff");
    return SDF_OK;
}

int sdf_trace_forward(int sh_degree, const sdf_trace_settings *settings, uint32_t num_points,
                      const float *points, const float *attributes, uint32_t adjacency_size,
                      const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets,
                      uint32_t num_rays, const float *rays, const uint32_t *start_point_index,
                      uint32_t num_depth_quantiles, const float *depth_quantiles, float *ray_rgba,
                      float *quantile_depths, uint32_t *quantile_point_indices,
                      uint32_t *num_intersections, float *point_contribution,
                      const float *sharpness, float *alpha_output, void *scratch,
                      size_t scratch_bytes, void *stream) {
    return trace_forward_impl(nullptr, sh_degree, settings, num_points, points, attributes,
                              adjacency_size, point_adjacency, point_adjacency_offsets, num_rays,
                              rays, start_point_index, num_depth_quantiles, depth_quantiles,
                              ray_rgba, quantile_depths, quantile_point_indices,
                              num_intersections, point_contribution, sharpness, alpha_output,
                              scratch, scratch_bytes, stream);
}

int sdf_trace_forward_noalloc(int sh_degree, const sdf_trace_settings *settings,
                              uint32_t num_points, const float *points, const float *attributes,
                              uint32_t adjacency_size, const uint32_t *point_adjacency,
                              const uint32_t *point_adjacency_offsets, uint32_t num_rays,
                              const float *rays, const uint32_t *start_point_index,
                              uint32_t num_depth_quantiles, const float *depth_quantiles,
                              float *ray_rgba, float *quantile_depths,
                              uint32_t *quantile_point_indices, uint32_t *num_intersections,
                              float *point_contribution, const float *sharpness,
                              float *alpha_output, void *stream) {
    const size_t need = sdf_trace_scratch_bytes(num_points, adjacency_size);
    if (need > SDF_NOALLOC_SCRATCH_BYTES)
        return fail(SDF_E_INVALID,
                    "sdf_trace_forward_noalloc: %u adjacency entries need %zu bytes of offset "
                    "table, more than its %zu-byte static scratch (at most %zu entries); use "
                    "sdf_trace_forward with caller scratch",
                    adjacency_size, need, (size_t)SDF_NOALLOC_SCRATCH_BYTES,
                    (size_t)SDF_NOALLOC_SCRATCH_BYTES / 8 - kDiffPad);
    void *table = nullptr;
    const int rc = noalloc_scratch_ptr(&table);
    if (rc != SDF_OK) return rc;
    return trace_forward_impl(nullptr, sh_degree, settings, num_points, points, attributes,
                              adjacency_size, point_adjacency, point_adjacency_offsets, num_rays,
                              rays, start_point_index, num_depth_quantiles, depth_quantiles,
                              ray_rgba, quantile_depths, quantile_point_indices,
                              num_intersections, point_contribution, sharpness, alpha_output,
                              table, SDF_NOALLOC_SCRATCH_BYTES, stream);
}

int sdf_trace_backward(int sh_degree, const sdf_trace_settings *settings, uint32_t num_points,
                       const float *points, const float *attributes, uint32_t adjacency_size,
                       const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets,
                       uint32_t num_rays, const float *rays, const uint32_t *start_point_index,
                       uint32_t num_depth_quantiles, const float *depth_quantiles,
                       const uint32_t *quantile_point_indices, const float *ray_rgba,
                       const float *ray_rgba_grad, const float *depth_grad,
                       const float *ray_error, float *points_grad, float *attribute_grad,
                       float *point_error, const float *sharpness, float *sharpness_grad,
                       void *scratch, size_t scratch_bytes, void *stream) {
    return trace_backward_impl(nullptr, sh_degree, settings, num_points, points, attributes,
                               adjacency_size, point_adjacency, point_adjacency_offsets,
                               num_rays, rays, start_point_index, num_depth_quantiles,
                               depth_quantiles, quantile_point_indices, ray_rgba, ray_rgba_grad,
                               depth_grad, ray_error, points_grad, attribute_grad, point_error,
                               sharpness, sharpness_grad, scratch, scratch_bytes, stream);
}

int sdf_trace_benchmark(int sh_degree, const sdf_trace_settings *settings, uint32_t num_points,
                        const float *points, const float *attributes, uint32_t adjacency_size,
                        const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets,
                        const uint16_t *adjacent_diff, size_t adjacent_diff_entries,
                        const sdf_camera *camera, const sdf_visualization *vis,
                        const uint32_t *start_point_index, uint32_t *output_rgba,
                        const float *sharpness, void *stream) {
    if (sh_degree < 0 || sh_degree > 3) return fail(SDF_E_INVALID, "Unsupported SH degree");
    if (!settings) return fail(SDF_E_INVALID, "settings must not be NULL");
    if (settings->alpha_mode != SDF_ALPHA_STANDARD && settings->alpha_mode != SDF_ALPHA_NEUS)
        return fail(SDF_E_INVALID, "alpha_mode must be 0 (standard) or 1 (sdfoam)");
    if (settings->attr_type != SDF_ATTR_F32 && settings->attr_type != SDF_ATTR_F16)
        return fail(SDF_E_INVALID, "attr_type must be 0 (float32) or 1 (float16)");
    const int D = 1 + 3 * (sh_degree + 1) * (sh_degree + 1);
    if (settings->sdf_channel >= D)
        return fail(SDF_E_INVALID, "sdf_channel %d out of range for attribute dim %d",
                    settings->sdf_channel, D);
    if (num_points == 0) return fail(SDF_E_INVALID, "num_points must be positive");
    if (!points || !attributes || !point_adjacency_offsets ||
        (!point_adjacency && adjacency_size > 0))
        return fail(SDF_E_INVALID, "scene pointers must not be NULL");
    if (!adjacent_diff || adjacent_diff_entries < adjacency_size)
        return fail(SDF_E_INVALID, "adjacent_diff must hold one row of 4 halves per adjacency "
                                   "entry (%u rows, got %zu)",
                    adjacency_size, adjacent_diff_entries);
    if ((reinterpret_cast<uintptr_t>(adjacent_diff) & 7u) != 0)
        return fail(SDF_E_INVALID, "adjacent_diff must be 8-byte aligned");
    if (!camera) return fail(SDF_E_INVALID, "camera must not be NULL");
    if (camera->model != SDF_CAMERA_PINHOLE && camera->model != SDF_CAMERA_FISHEYE)
        return fail(SDF_E_INVALID, "Invalid camera model");
    if (camera->width == 0 || camera->height == 0 ||
        (uint64_t)camera->width * camera->height > 0xffffffffull)
        return fail(SDF_E_INVALID, "camera width and height must be positive and "
                                   "width * height < 2^32");
    if (!start_point_index) return fail(SDF_E_INVALID, "start_point must not be NULL");
    if (!output_rgba) return fail(SDF_E_INVALID, "output_rgba must not be NULL");
    if (!sharpness) return fail(SDF_E_INVALID, "sharpness must not be NULL");

    RenderArgs a = {};
    a.scene = make_scene(num_points, points, attributes, adjacency_size, point_adjacency,
                         point_adjacency_offsets, const_cast<uint16_t *>(adjacent_diff));
    a.settings = *settings;
    for (int k = 0; k < 3; ++k) {
        a.position[k] = camera->position[k];
        a.forward[k] = camera->forward[k];
        a.right[k] = camera->right[k];
        a.up[k] = camera->up[k];
        // default_visualization_settings: white background
        a.bg[k] = vis ? vis->bg_color[k] : 1.0f;
    }
    a.checker_bg = vis ? vis->checker_bg : 0;
    a.fov = camera->fov;
    // pinhole focal factor, once per launch (cast_ray evaluates it per ray)
    a.focal = 1.0f / tanf(camera->fov * 0.5f);
    a.width = camera->width;
    a.height = camera->height;
    a.model = camera->model;
    a.num_tiles = num_ray_tiles(camera->width * camera->height, camera->width);
    a.start = start_point_index;
    a.sharpness = sharpness;
    a.out = output_rgba;
    hipStream_t s = static_cast<hipStream_t>(stream);
    tbegin(SDF_KERNEL_RENDER, s);
    hipError_t e = launch_render(sh_degree, a, settings->alpha_mode == SDF_ALPHA_NEUS,
                                 settings->attr_type == SDF_ATTR_F16, s);
    tend(s);
    if (e != hipSuccess) return hip_fail(e, "trace_benchmark");
    return SDF_OK;
}

size_t sdf_ray_order_scratch_bytes(uint32_t num_points, uint32_t num_rays) {
    return ray_order_scratch_bytes(num_points, num_rays);
}

int sdf_ray_order(uint32_t num_points, uint32_t num_rays, const float *rays,
                  const uint32_t *start_point_index, uint32_t *order, void *scratch,
                  size_t scratch_bytes, void *stream) {
    if (num_rays == 0) return SDF_OK;
    if (!rays || !start_point_index || !order || !scratch)
        return fail(SDF_E_INVALID, "NULL pointer argument");
    const size_t need = ray_order_scratch_bytes(num_points, num_rays);
    if (need == 0) return fail(SDF_E_HIP, "ray order: scratch size query failed");
    if (scratch_bytes < need)
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 256-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    tbegin(SDF_KERNEL_RAY_ORDER, s);
    hipError_t e = launch_ray_order(num_points, num_rays, rays, start_point_index, order, scratch,
                                    scratch_bytes, s);
    tend(s);
    if (e != hipSuccess) return hip_fail(e, "ray_order");
    return SDF_OK;
}

size_t sdf_walk_record_bytes(uint32_t num_rays, uint32_t ray_image_width, uint32_t budget) {
    return sdf_walk_record_pool_bytes(num_rays, ray_image_width, budget, 0);
}

size_t sdf_walk_record_pool_bytes(uint32_t num_rays, uint32_t ray_image_width, uint32_t budget,
                                  uint32_t chunks) {
    if (budget == 0) return 0;
    const uint32_t tiles = num_ray_tiles(num_rays, ray_image_width);
    return (size_t)walk_record_bytes_for(tiles, budget, record_pool_chunks(tiles, budget, chunks));
}

uint32_t sdf_walk_record_full_chunks(uint32_t num_rays, uint32_t ray_image_width,
                                     uint32_t budget) {
    const uint64_t c = walk_record_full_chunks(num_ray_tiles(num_rays, ray_image_width), budget);
    return c >= kNoIndex ? kNoIndex : (uint32_t)c;
}

int sdf_trace_forward_planned(
    const sdf_trace_plan *plan, int sh_degree, const sdf_trace_settings *settings,
    uint32_t num_points, const float *points, const float *attributes, uint32_t adjacency_size,
    const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets, uint32_t num_rays,
    const float *rays, const uint32_t *start_point_index, uint32_t num_depth_quantiles,
    const float *depth_quantiles, float *ray_rgba, float *quantile_depths,
    uint32_t *quantile_point_indices, uint32_t *num_intersections, float *point_contribution,
    const float *sharpness, float *alpha_output, void *scratch, size_t scratch_bytes,
    void *stream) {
    return trace_forward_impl(plan, sh_degree, settings, num_points, points, attributes,
                              adjacency_size, point_adjacency, point_adjacency_offsets, num_rays,
                              rays, start_point_index, num_depth_quantiles, depth_quantiles,
                              ray_rgba, quantile_depths, quantile_point_indices,
                              num_intersections, point_contribution, sharpness, alpha_output,
                              scratch, scratch_bytes, stream);
}

int sdf_trace_backward_planned(
    const sdf_trace_plan *plan, int sh_degree, const sdf_trace_settings *settings,
    uint32_t num_points, const float *points, const float *attributes, uint32_t adjacency_size,
    const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets, uint32_t num_rays,
    const float *rays, const uint32_t *start_point_index, uint32_t num_depth_quantiles,
    const float *depth_quantiles, const uint32_t *quantile_point_indices, const float *ray_rgba,
    const float *ray_rgba_grad, const float *depth_grad, const float *ray_error,
    float *points_grad, float *attribute_grad, float *point_error, const float *sharpness,
    float *sharpness_grad, void *scratch, size_t scratch_bytes, void *stream) {
    return trace_backward_impl(plan, sh_degree, settings, num_points, points, attributes,
                               adjacency_size, point_adjacency, point_adjacency_offsets,
                               num_rays, rays, start_point_index, num_depth_quantiles,
                               depth_quantiles, quantile_point_indices, ray_rgba, ray_rgba_grad,
                               depth_grad, ray_error, points_grad, attribute_grad, point_error,
                               sharpness, sharpness_grad, scratch, scratch_bytes, stream);
}

// The tree has pow2(N) boxes (N rounded up to a power of two in 32 bits).
constexpr uint32_t kMaxTreePoints = 1u << 31;

int sdf_build_aabb_tree(const float *points, uint32_t num_points, float *aabb_tree,
                        void *stream) {
    if (!points || !aabb_tree) return fail(SDF_E_INVALID, "NULL pointer argument");
    if (num_points == 0) return fail(SDF_E_INVALID, "num_points must be positive");
    if (num_points > kMaxTreePoints)
        return fail(SDF_E_INVALID, "at most %u points (got %u)", kMaxTreePoints, num_points);
    hipStream_t s = static_cast<hipStream_t>(stream);
    tbegin(SDF_KERNEL_AABB_TREE, s);
    hipError_t e = launch_build_aabb_tree(points, num_points, aabb_tree, s);
    tend(s);
    if (e != hipSuccess) return hip_fail(e, "build_aabb_tree");
    return SDF_OK;
}

int sdf_farthest_neighbor(const float *points, uint32_t num_points, uint32_t adjacency_size,
                          const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets,
                          uint32_t *indices, float *cell_radius, void *stream) {
    if (num_points == 0) return SDF_OK;
    if (!points || !point_adjacency_offsets || !indices || !cell_radius ||
        (!point_adjacency && adjacency_size > 0))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = launch_farthest_neighbor(points, num_points, point_adjacency,
                                            point_adjacency_offsets, adjacency_size, indices,
                                            cell_radius, s);
    if (e != hipSuccess) return hip_fail(e, "farthest_neighbor");
    return SDF_OK;
}

size_t sdf_sort_points_scratch_bytes(uint32_t num_points) {
    return sort_points_scratch_bytes(num_points);
}

int sdf_sort_points(const float *points, uint32_t num_points, uint32_t *perm, void *scratch,
                    size_t scratch_bytes, void *stream) {
    if (num_points == 0) return SDF_OK;
    if (!points || !perm || !scratch) return fail(SDF_E_INVALID, "NULL pointer argument");
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 256-byte aligned");
    const size_t need = sort_points_scratch_bytes(num_points);
    if (need == 0) return fail(SDF_E_HIP, "sort_points: no device to size the sort for");
    if (scratch_bytes < need)
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    hipError_t e = launch_sort_points(points, num_points, perm, scratch, scratch_bytes,
                                      static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "sort_points");
    return SDF_OK;
}

uint64_t sdf_delaunay_adjacency_capacity(uint32_t num_points, uint32_t num_tets) {
    return delaunay_edge_capacity(num_points, num_tets);
}

size_t sdf_delaunay_tables_scratch_bytes(uint32_t num_points, uint32_t num_tets) {
    return delaunay_tables_scratch_bytes(num_points, num_tets);
}

int sdf_delaunay_tables(const float *points, uint32_t num_points, const uint32_t *tets,
                        const int32_t *neighbors, uint32_t num_tets, uint32_t *tets_out,
                        uint32_t *tet_adjacency, uint32_t *vert_to_tet,
                        uint32_t *point_adjacency_offsets, uint32_t *point_adjacency,
                        uint64_t point_adjacency_capacity, void *scratch, size_t scratch_bytes,
                        void *stream) {
    if (!points || !vert_to_tet || !point_adjacency_offsets || !scratch ||
        (num_tets > 0 && (!tets || !neighbors || !tets_out || !tet_adjacency || !point_adjacency)))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 256-byte aligned");
    if (num_points == 0 && num_tets > 0)
        return fail(SDF_E_INVALID, "tets need points");
    const uint64_t cap = delaunay_edge_capacity(num_points, num_tets);
    if (point_adjacency_capacity < cap)
        return fail(SDF_E_INVALID, "point_adjacency must hold %llu entries (got %llu)",
                    (unsigned long long)cap, (unsigned long long)point_adjacency_capacity);
    const size_t need = delaunay_tables_scratch_bytes(num_points, num_tets);
    if (need == 0) return fail(SDF_E_HIP, "delaunay_tables: no device to size the sorts for");
    if (scratch_bytes < need)
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    uint32_t input_error = 0;
    hipError_t e = launch_delaunay_tables(points, num_points, tets, neighbors, num_tets, tets_out,
                                          tet_adjacency, vert_to_tet, point_adjacency_offsets,
                                          point_adjacency, point_adjacency_capacity, input_error,
                                          scratch, scratch_bytes,
                                          static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "delaunay_tables");
    if (input_error & 1u)
        return fail(SDF_E_INVALID, "tets or neighbors hold an index out of range");
    if (input_error & 2u)
        return fail(SDF_E_INVALID, "more edges than a tetrahedralised ball can have");
    return SDF_OK;
}

size_t sdf_delaunay_certify_scratch_bytes(uint32_t num_points) {
    return delaunay_certify_scratch_bytes(num_points);
}

int sdf_delaunay_certify(const float *points, uint32_t num_points, uint32_t *reports,
                         uint64_t report_capacity, uint32_t *open_points, uint64_t *counts,
                         void *scratch, size_t scratch_bytes, void *stream) {
    if (!points || !open_points || !counts || !scratch || (report_capacity > 0 && !reports))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 256-byte aligned");
    if (num_points < 32)
        return fail(SDF_E_INVALID, "Delaunay triangulation does not support less than 32 points");
    if (num_points > (1u << 26))
        return fail(SDF_E_INVALID, "sdf_delaunay_certify takes at most 2^26 points");
    const size_t need = delaunay_certify_scratch_bytes(num_points);
    if (need == 0) return fail(SDF_E_HIP, "delaunay_certify: no device to size the sorts for");
    if (scratch_bytes < need)
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    hipError_t e = launch_delaunay_certify(points, num_points, reports, report_capacity,
                                           open_points, counts, scratch, scratch_bytes,
                                           static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue)
        return fail(SDF_E_INVALID, "points must be finite and span a volume");
    if (e != hipSuccess) return hip_fail(e, "delaunay_certify");
    return SDF_OK;
}

int sdf_delaunay_certify_exhaustive(const float *points, uint32_t num_points, uint32_t *reports,
                                    uint64_t report_capacity, uint32_t *open_points,
                                    uint64_t *counts, void *scratch, size_t scratch_bytes,
                                    void *stream) {
    if (!points || !open_points || !counts || !scratch || (report_capacity > 0 && !reports))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 256-byte aligned");
    if (num_points < 32)
        return fail(SDF_E_INVALID, "Delaunay triangulation does not support less than 32 points");
    if (num_points > (1u << 20))
        return fail(SDF_E_INVALID, "sdf_delaunay_certify_exhaustive takes at most 2^20 points");
    const size_t need = delaunay_certify_scratch_bytes(num_points);
    if (need == 0) return fail(SDF_E_HIP, "delaunay_certify: no device to size the sorts for");
    if (scratch_bytes < need)
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    hipError_t e = launch_delaunay_certify_exhaustive(points, num_points, reports,
                                                      report_capacity, open_points, counts,
                                                      scratch, scratch_bytes,
                                                      static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue)
        return fail(SDF_E_INVALID, "points must be finite and span a volume");
    if (e != hipSuccess) return hip_fail(e, "delaunay_certify_exhaustive");
    return SDF_OK;
}

size_t sdf_delaunay_merge_scratch_bytes(uint32_t num_points, uint64_t num_reports,
                                        uint64_t num_candidates, uint64_t tet_capacity) {
    return delaunay_merge_scratch_bytes(num_points, num_reports, num_candidates, tet_capacity);
}

static int delaunay_merge_common(const char *name, const float *points, uint32_t num_points,
                                 void *certify_scratch, size_t certify_scratch_bytes,
                                 const uint32_t *reports, uint64_t num_reports,
                                 const uint32_t *candidates, uint64_t num_candidates,
                                 const uint32_t *verified, uint64_t num_verified, uint32_t *tets,
                                 int32_t *neighbors, uint64_t tet_capacity, uint64_t *result,
                                 void *scratch, size_t scratch_bytes, void *stream) {
    if (!points || !certify_scratch || !result || !scratch || (num_reports > 0 && !reports) ||
        (num_candidates > 0 && !candidates) || (num_verified > 0 && !verified) ||
        (tet_capacity > 0 && (!tets || !neighbors)))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0 ||
        (reinterpret_cast<uintptr_t>(certify_scratch) & 255u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 256-byte aligned");
    if (num_points < 32)
        return fail(SDF_E_INVALID, "Delaunay triangulation does not support less than 32 points");
    if (num_reports + num_candidates + num_verified >= 0xffffffffull)
        return fail(SDF_E_INVALID, "too many reports and candidates");
    if (num_points > (1u << 26) || num_candidates > (1ull << 26))
        return fail(SDF_E_INVALID, "%s takes at most 2^26 points and candidates", name);
    const size_t gneed = delaunay_certify_scratch_bytes(num_points);
    const size_t need = delaunay_merge_scratch_bytes(num_points, num_reports,
                                                     num_candidates + num_verified, tet_capacity);
    if (gneed == 0 || need == 0) return fail(SDF_E_HIP, "%s: no device to size the scans for", name);
    if (certify_scratch_bytes < gneed)
        return fail(SDF_E_INVALID, "certify_scratch must hold %zu bytes (got %zu)", gneed,
                    certify_scratch_bytes);
    if (scratch_bytes < need)
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    hipError_t e = launch_delaunay_merge(points, num_points, certify_scratch,
                                         certify_scratch_bytes, reports, num_reports, candidates,
                                         num_candidates, verified, num_verified, tets, neighbors,
                                         tet_capacity, result, scratch, scratch_bytes,
                                         static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, name);
    if (result[2] != 0)
        return fail(SDF_E_INVALID, "%llu reports or candidates were invalid or undecided",
                    (unsigned long long)result[2]);
    if (result[0] > tet_capacity)
        return fail(SDF_E_INVALID, "tets must hold %llu rows (got %llu)",
                    (unsigned long long)result[0], (unsigned long long)tet_capacity);
    if (result[3] != 0)
        return fail(SDF_E_INVALID, "%llu faces are shared by more than two tets",
                    (unsigned long long)result[3]);
    return SDF_OK;
}

int sdf_delaunay_merge(const float *points, uint32_t num_points, void *certify_scratch,
                       size_t certify_scratch_bytes, const uint32_t *reports,
                       uint64_t num_reports, const uint32_t *candidates, uint64_t num_candidates,
                       uint32_t *tets, int32_t *neighbors, uint64_t tet_capacity,
                       uint64_t *result, void *scratch, size_t scratch_bytes, void *stream) {
    return delaunay_merge_common("delaunay_merge", points, num_points, certify_scratch,
                                 certify_scratch_bytes, reports, num_reports, candidates,
                                 num_candidates, nullptr, 0, tets, neighbors, tet_capacity, result,
                                 scratch, scratch_bytes, stream);
}

int sdf_delaunay_merge_verified(const float *points, uint32_t num_points, void *certify_scratch,
                                size_t certify_scratch_bytes, const uint32_t *reports,
                                uint64_t num_reports, const uint32_t *candidates,
                                uint64_t num_candidates, const uint32_t *verified,
                                uint64_t num_verified, uint32_t *tets, int32_t *neighbors,
                                uint64_t tet_capacity, uint64_t *result, void *scratch,
                                size_t scratch_bytes, void *stream) {
    return delaunay_merge_common("delaunay_merge_verified", points, num_points, certify_scratch,
                                 certify_scratch_bytes, reports, num_reports, candidates,
                                 num_candidates, verified, num_verified, tets, neighbors,
                                 tet_capacity, result, scratch, scratch_bytes, stream);
}

static int delaunay_scratch_ok(const char *name, uint32_t num_points, const void *scratch,
                               size_t scratch_bytes) {
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 256-byte aligned");
    if (num_points < 32)
        return fail(SDF_E_INVALID, "Delaunay triangulation does not support less than 32 points");
    if (num_points > (1u << 26)) return fail(SDF_E_INVALID, "%s takes at most 2^26 points", name);
    const size_t need = delaunay_certify_scratch_bytes(num_points);
    if (need == 0) return fail(SDF_E_HIP, "%s: no device to size the sorts for", name);
    if (scratch_bytes < need)
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    return SDF_OK;
}

int sdf_delaunay_check(const float *points, uint32_t num_points, const uint32_t *tets,
                       const int32_t *neighbors, uint64_t num_tets, uint32_t *keep,
                       uint32_t *dirty, void *certify_scratch, size_t certify_scratch_bytes,
                       void *stream) {
    if (!points || !dirty || !certify_scratch || (num_tets > 0 && (!tets || !neighbors || !keep)))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    const int rc = delaunay_scratch_ok("sdf_delaunay_check", num_points, certify_scratch,
                                       certify_scratch_bytes);
    if (rc != SDF_OK) return rc;
    uint64_t errors = 0;
    hipError_t e = launch_delaunay_check(points, num_points, tets, neighbors, num_tets, keep,
                                         dirty, &errors, certify_scratch, certify_scratch_bytes,
                                         static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue)
        return fail(SDF_E_INVALID, "points must be finite and span a volume");
    if (e != hipSuccess) return hip_fail(e, "delaunay_check");
    if (errors != 0)
        return fail(SDF_E_INVALID, "%llu tets have a vertex id >= num_points",
                    (unsigned long long)errors);
    return SDF_OK;
}

int sdf_delaunay_certify_points(const float *points, uint32_t num_points, const uint32_t *query,
                                uint32_t num_query, uint32_t *reports, uint64_t report_capacity,
                                uint32_t *open_points, uint64_t *counts, void *certify_scratch,
                                size_t certify_scratch_bytes, void *stream) {
    if (!points || !open_points || !counts || !certify_scratch || (num_query > 0 && !query) ||
        (report_capacity > 0 && !reports))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    const int rc = delaunay_scratch_ok("sdf_delaunay_certify_points", num_points,
                                       certify_scratch, certify_scratch_bytes);
    if (rc != SDF_OK) return rc;
    if (num_query > num_points)
        return fail(SDF_E_INVALID, "at most num_points query points (got %u)", num_query);
    hipError_t e = launch_delaunay_certify_points(points, num_points, query, num_query, reports,
                                                  report_capacity, open_points, counts,
                                                  certify_scratch, certify_scratch_bytes,
                                                  static_cast<hipStream_t>(stream));
    if (e == hipErrorNotReady)
        return fail(SDF_E_INVALID, "certify_scratch holds no grid of these points "
                                   "(call sdf_delaunay_check first)");
    if (e != hipSuccess) return hip_fail(e, "delaunay_certify_points");
    return SDF_OK;
}

int sdf_nn(const float *points, const float *aabb_tree, const float *queries, uint32_t num_points,
           uint32_t num_queries, uint32_t *indices, void *stream) {
    if (num_points < 32) return fail(SDF_E_INVALID, "number of points must be at least 32");
    if (num_points > kMaxTreePoints)
        return fail(SDF_E_INVALID, "at most %u points (got %u)", kMaxTreePoints, num_points);
    if (!points || !aabb_tree || (num_queries > 0 && (!queries || !indices)))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    tbegin(SDF_KERNEL_NN, s);
    hipError_t e = launch_nn(points, aabb_tree, queries, num_points, num_queries, indices, s);
    tend(s);
    if (e != hipSuccess) return hip_fail(e, "nn");
    return SDF_OK;
}

size_t sdf_start_points_scratch_bytes(uint32_t num_rays) {
    return start_layout(num_rays).bytes;
}

int sdf_start_points(const float *rays, uint32_t num_rays, const float *points,
                     uint32_t num_points, const float *aabb_tree, uint32_t *start, void *scratch,
                     size_t scratch_bytes, void *stream) {
    if (num_points < 32) return fail(SDF_E_INVALID, "number of points must be at least 32");
    if (num_points > kMaxTreePoints)
        return fail(SDF_E_INVALID, "at most %u points (got %u)", kMaxTreePoints, num_points);
    if (!points || !aabb_tree || (num_rays > 0 && (!rays || !start)))
        return fail(SDF_E_INVALID, "NULL pointer argument");
    const size_t need = sdf_start_points_scratch_bytes(num_rays);
    if (num_rays > 0 && (!scratch || scratch_bytes < need))
        return fail(SDF_E_INVALID, "scratch must hold %zu bytes (got %zu)", need, scratch_bytes);
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0)
        return fail(SDF_E_INVALID, "scratch must be 256-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    tbegin(SDF_KERNEL_NN, s);
    hipError_t e = launch_start_points(rays, num_rays, points, num_points, aabb_tree, start,
                                       scratch, s);
    tend(s);
    if (e != hipSuccess) return hip_fail(e, "start points");
    return SDF_OK;
}

int sdf_trace_walk_stats(int sh_degree, const sdf_trace_settings *settings, int backward,
                         uint32_t num_points, const float *points, const float *attributes,
                         uint32_t adjacency_size, const uint32_t *point_adjacency,
                         const uint32_t *point_adjacency_offsets, uint32_t num_rays,
                         const float *rays, const uint32_t *start_point_index,
                         const float *sharpness, uint64_t *visit_hash, uint32_t *steps,
                         uint64_t *faces, uint64_t *faces_stepped, uint32_t *cells,
                         uint32_t cells_stride, void *scratch, size_t scratch_bytes,
                         void *stream) {
    int rc = check_scene(sh_degree, settings, num_points, points, attributes, adjacency_size,
                         point_adjacency, point_adjacency_offsets, num_rays, rays,
                         start_point_index, sharpness, scratch, scratch_bytes);
    if (rc != SDF_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = launch_prefetch_diff(points, num_points, adjacency_size, point_adjacency,
                                        point_adjacency_offsets, static_cast<uint2 *>(scratch), s);
    if (e != hipSuccess) return hip_fail(e, "prefetch_adjacent_diff");
    if (num_rays == 0) return SDF_OK;
    const bool neus = settings->alpha_mode == SDF_ALPHA_NEUS;
    const SceneView sc = make_scene(num_points, points, attributes, adjacency_size,
                                    point_adjacency, point_adjacency_offsets, scratch);
    if (!backward) {
        FwdArgs a = {};
        a.scene = sc;
        a.settings = *settings;
        a.rays = rays;
        a.num_rays = num_rays;
        a.num_tiles = num_ray_tiles(num_rays, settings->ray_image_width);
        a.start = start_point_index;
        a.sharpness = sharpness;
        a.visit_hash = visit_hash;
        a.steps = steps;
        a.faces = faces;
        a.faces_stepped = faces_stepped;
        a.cells = cells;
        a.cells_stride = cells ? cells_stride : 0;
        e = launch_forward(sh_degree, a, neus, true, settings->attr_type == SDF_ATTR_F16, s);
    } else {
        BwdArgs a = {};
        a.scene = sc;
        a.settings = *settings;
        a.rays = rays;
        a.num_rays = num_rays;
        a.num_tiles = num_ray_tiles(num_rays, settings->ray_image_width);
        a.start = start_point_index;
        a.sharpness = sharpness;
        a.visit_hash = visit_hash;
        a.steps = steps;
        a.faces = faces;
        a.faces_stepped = faces_stepped;
        a.cells = cells;
        a.cells_stride = cells ? cells_stride : 0;
        e = launch_backward(sh_degree, a, neus, true, settings->attr_type == SDF_ATTR_F16, s);
    }
    if (e != hipSuccess) return hip_fail(e, "walk_stats");
    return SDF_OK;
}

int sdf_debug_fpmath(int op, const float *in, void *out, uint64_t n, void *stream) {
    if (op < 0 || op > 2) return fail(SDF_E_INVALID, "op must be 0, 1 or 2");
    if (n == 0) return SDF_OK;
    if (!in || !out) return fail(SDF_E_INVALID, "NULL pointer argument");
    hipError_t e = launch_fpmath(op, in, out, n, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "fpmath");
    return SDF_OK;
}

int sdf_set_timing(int enable) {
    g_timing = enable != 0;
    g_ring_n = 0;
    g_open = -1;
    return SDF_OK;
}

int sdf_timing_collect(int *kinds, float *ms, int max_n, int *n_out) {
    if (!n_out) return fail(SDF_E_INVALID, "n_out must not be NULL");
    const int n = g_ring_n < max_n ? g_ring_n : max_n;
    for (int i = 0; i < n; ++i) {
        hipError_t e = hipEventSynchronize(g_ring[i].end);
        if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
        float t = 0.0f;
        e = hipEventElapsedTime(&t, g_ring[i].begin, g_ring[i].end);
        if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
        if (kinds) kinds[i] = g_ring[i].kind;
        if (ms) ms[i] = t;
    }
    *n_out = n;
    g_ring_n = 0;
    return SDF_OK;
}

} // extern "C"
