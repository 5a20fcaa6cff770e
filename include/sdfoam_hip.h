/*
 * sdfoam_hip.h -- C ABI of libsdfoam_hip.so, the MI355X (gfx950) build of
 * SDFoam's Voronoi-foam tracer.
 *
 * Plain pointers and sizes only.  Every pointer argument named as device
 * memory must point to memory the calling process allocated on the current
 * HIP device; `stream` is a hipStream_t passed as void* (NULL = the legacy
 * default stream).  Calls are asynchronous on `stream` unless stated.  Every
 * call returns 0 on success or a nonzero SDF_E_* code; sdf_last_error()
 * returns the calling thread's last message.
 *
 * The library allocates no device memory: callers pass the scratch the
 * tracer needs (size from sdf_trace_scratch_bytes).
 *
 * Each entry point names the reference interface it replaces
 * (paths are into mmlab-cv/SDFoam).
 */
#ifndef SDFOAM_HIP_H
#define SDFOAM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SDF_OK 0
#define SDF_E_INVALID 1 /* bad argument (size, degree, null pointer) */
#define SDF_E_HIP 2     /* a HIP runtime call failed */

/* alpha_mode values (src/tracing/pipeline.h:10) */
#define SDF_ALPHA_STANDARD 0u
#define SDF_ALPHA_NEUS 1u

/* The TraceSettings fields the forward/backward kernels read
 * (src/tracing/pipeline.h:12-27; defaults src/tracing/pipeline.h:29-40:
 * weight_threshold 1e-7, max_intersections 1024, alpha_mode standard,
 * sdf_channel -1).  inv_s, eps and the viewer fields are not read by the
 * reference's kernels and are not part of this struct.
 * ray_image_width is a layout hint with no counterpart in the reference: 0
 * for rays in any order, or W when the rays are image rows of W pixels
 * ([..., H, W, 6]); the kernels then give each wavefront an 8x8 pixel tile.
 * Results do not depend on it.
 * attr_type is the pipeline's attribute type (the reference's
 * CUDATracingPipeline<float | __half, L>, src/tracing/pipeline.cu:1482-1502):
 * with SDF_ATTR_F16, attributes, ray_rgba, ray_rgba_grad, ray_error,
 * point_contribution, attribute_grad and point_error are fp16; positions,
 * rays, depths, quantiles, alpha, points_grad and sharpness stay fp32.  The
 * fp16 buffers that are accumulated atomically (point_contribution,
 * attribute_grad, point_error) must be 4-byte aligned and hold one padding
 * half past an odd element count. */
#define SDF_ATTR_F32 0u
#define SDF_ATTR_F16 1u
typedef struct sdf_trace_settings {
    float weight_threshold;
    uint32_t max_intersections;
    uint32_t alpha_mode;
    int32_t sdf_channel;
    uint32_t ray_image_width;
    uint32_t attr_type;
} sdf_trace_settings;

/* Library version string. */
const char *sdf_version(void);

/* Thread-local description of the last failure. */
const char *sdf_last_error(void);

/* 1 + 3 (L+1)^2, or -1 for an unsupported degree.
 * Replaces Pipeline::attribute_dim (src/tracing/pipeline.h:158,
 * src/tracing/pipeline.cu:1467-1469). */
int sdf_attribute_dim(int sh_degree);

/* Bytes of scratch sdf_trace_forward / sdf_trace_backward need for a scene
 * with `adjacency_size` CSR entries (the fp16 neighbour-offset table,
 * (E + 32) x 8 bytes, as src/tracing/pipeline.cu:1270, 1328). */
size_t sdf_trace_scratch_bytes(uint32_t num_points, uint32_t adjacency_size);

/* adjacent_diff[k] = fp16(points[adjacency[k]] - points[i]) for every CSR
 * entry k of row i, 4 halves per entry (w = 0); rows with out-of-range
 * neighbours get NaN planes.  `adjacent_diff` holds (E + 32) x 4 halves.
 * Offsets are expected non-decreasing (a CSR row array, as the reference's
 * triangulation writes them).  With others the entries are unspecified, as
 * in the reference (its one-thread-per-row kernel writes overlapping rows
 * racily and leaves entries outside every row unwritten); every read and
 * write stays within the table.
 * Replaces prefetch_adjacent_diff (src/tracing/pipeline.h:70-77,
 * src/tracing/pipeline.cu:1202-1242). */
int sdf_prefetch_adjacent_diff(const float *points, uint32_t num_points,
                               uint32_t adjacency_size,
                               const uint32_t *point_adjacency,
                               const uint32_t *point_adjacency_offsets,
                               uint16_t *adjacent_diff, void *stream);

/* Forward trace: per ray rgba [R,4], depth [R,Q] and depth_indices [R,Q]
 * (both NULL when Q = 0), num_intersections [R]; per point contribution
 * [N] (+= weights; NULL to skip) and alpha [N] (a visiting ray's alpha).
 * Attributes are fp32 AoS [N, D], D = sdf_attribute_dim(sh_degree); rays are
 * [R, 6] (origin, direction); sharpness is read at element 0.
 * Outputs contribution and alpha must be zeroed by the caller.
 * Replaces Pipeline::trace_forward (src/tracing/pipeline.h:83-101,
 * src/tracing/pipeline.cu:1251-1303). */
int sdf_trace_forward(int sh_degree, const sdf_trace_settings *settings,
                      uint32_t num_points, const float *points,
                      const float *attributes, uint32_t adjacency_size,
                      const uint32_t *point_adjacency,
                      const uint32_t *point_adjacency_offsets,
                      uint32_t num_rays, const float *rays,
                      const uint32_t *start_point_index,
                      uint32_t num_depth_quantiles,
                      const float *depth_quantiles, float *ray_rgba,
                      float *quantile_depths, uint32_t *quantile_point_indices,
                      uint32_t *num_intersections, float *point_contribution,
                      const float *sharpness, float *alpha_output,
                      void *scratch, size_t scratch_bytes, void *stream);

/* Backward trace: accumulates points_grad [N,3], attribute_grad [N,D],
 * sharpness_grad [1] (NULL to skip) and point_error [N] (NULL to skip; then
 * ray_error is ignored).  Gradient buffers must be zeroed by the caller.
 * alpha_mode NEUS runs backward_sdf, STANDARD runs the density backward.
 * ray_rgba is the forward's rgba; quantile_point_indices is read in
 * standard mode only.
 * Replaces Pipeline::trace_backward (src/tracing/pipeline.h:104-126,
 * src/tracing/pipeline.cu:1305-1391). */
int sdf_trace_backward(int sh_degree, const sdf_trace_settings *settings,
                       uint32_t num_points, const float *points,
                       const float *attributes, uint32_t adjacency_size,
                       const uint32_t *point_adjacency,
                       const uint32_t *point_adjacency_offsets,
                       uint32_t num_rays, const float *rays,
                       const uint32_t *start_point_index,
                       uint32_t num_depth_quantiles,
                       const float *depth_quantiles,
                       const uint32_t *quantile_point_indices,
                       const float *ray_rgba, const float *ray_rgba_grad,
                       const float *depth_grad, const float *ray_error,
                       float *points_grad, float *attribute_grad,
                       float *point_error, const float *sharpness,
                       float *sharpness_grad, void *scratch,
                       size_t scratch_bytes, void *stream);

/* sdf_trace_forward without caller scratch.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * call allocates nothing: the fp16 offset table lives in a static device
 * array of SDF_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it
 * runs on until the process ends (its first call on a device looks up the
 * array's address there).  Scenes are limited to
 * SDF_NOALLOC_SCRATCH_BYTES / 8 - 32 = 16,777,184 adjacency entries (about
 * one million Delaunay points); larger ones fail with SDF_E_INVALID before
 * any work is queued.  All calls on one GPU share the array, so calls that
 * overlap on one GPU (on other streams or threads) race: the caller must
 * serialise them.  Arguments and results are sdf_trace_forward's. */
#define SDF_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
int sdf_trace_forward_noalloc(int sh_degree, const sdf_trace_settings *settings,
                              uint32_t num_points, const float *points,
                              const float *attributes, uint32_t adjacency_size,
                              const uint32_t *point_adjacency,
                              const uint32_t *point_adjacency_offsets,
                              uint32_t num_rays, const float *rays,
                              const uint32_t *start_point_index,
                              uint32_t num_depth_quantiles,
                              const float *depth_quantiles, float *ray_rgba,
                              float *quantile_depths,
                              uint32_t *quantile_point_indices,
                              uint32_t *num_intersections,
                              float *point_contribution, const float *sharpness,
                              float *alpha_output, void *stream);

/* Camera of the inference render (src/tracing/camera.h:17-27). */
#define SDF_CAMERA_PINHOLE 0
#define SDF_CAMERA_FISHEYE 1
typedef struct sdf_camera {
    float position[3];
    float forward[3];
    float right[3];
    float up[3];
    float fov; /* vertical, radians */
    uint32_t width;
    uint32_t height;
    uint32_t model; /* SDF_CAMERA_* */
} sdf_camera;

/* Background of the inference render (the fields of VisualizationSettings
 * the render reads, src/tracing/pipeline.h:50-68). */
typedef struct sdf_visualization {
    float bg_color[3];
    int32_t checker_bg;
} sdf_visualization;

/* Inference render: one ray per pixel cast in the kernel, all starting in
 * cell *start_point_index (device pointer, one element), composited as the
 * forward and packed as RGBA8 (colour + T * background, alpha 255) into
 * output_rgba[(height - 1 - j) * width + i].  adjacent_diff is the caller's
 * fp16 offset table, adjacent_diff_entries >= adjacency_size rows of 4
 * halves (as prefetch_adjacent_diff writes them).  vis NULL: white, no
 * checker (default_visualization_settings).  settings->ray_image_width is
 * ignored.
 * Replaces Pipeline::trace_benchmark (src/tracing/pipeline.h:144-156,
 * src/tracing/pipeline.cu:1067-1199, 1432-1466). */
int sdf_trace_benchmark(int sh_degree, const sdf_trace_settings *settings,
                        uint32_t num_points, const float *points,
                        const float *attributes, uint32_t adjacency_size,
                        const uint32_t *point_adjacency,
                        const uint32_t *point_adjacency_offsets,
                        const uint16_t *adjacent_diff,
                        size_t adjacent_diff_entries, const sdf_camera *camera,
                        const sdf_visualization *vis,
                        const uint32_t *start_point_index,
                        uint32_t *output_rgba, const float *sharpness,
                        void *stream);

/* ---- trace plan (no counterpart in the reference) ---------------------- *
 * Two optional aids for a forward and the backward over the same rays, start
 * points, scene and settings.  Results are identical with and without them.
 *
 * Walk record: the forward records each ray's steps (next cell and exit
 * distance, and the step's colour and sdf/density value: 24 bytes a step,
 * up to `walk_budget` trips per wavefront of 64 rays); the backward then reads
 * the steps instead of scanning the cell faces again, and a recorded step's
 * colour instead of the cell's attribute row, so the record is valid only
 * for a backward over the attributes the forward traced.  In standard mode
 * the density backward walks in the unsafe mode: where it would take another
 * exit the forward marks its step, and the backward scans from there until its
 * walk meets the recorded one again.  Rays past `walk_budget` trips, or that
 * walk further in the backward, scan as usual.
 * walk_record == NULL: no record.
 * Storage is sized by need: a wavefront takes chunks of 16 trips from a
 * pool of `walk_record_chunks` as its walk gets there, and records nothing
 * more once the pool (split in 8 parts, one per XCD) has none left for it.
 * The record starts with 8 counters, 256 bytes apart (uint32 at byte offsets
 * 0, 256, ..., 1792): after the forward their sum is the number of chunks
 * the walk asked for, pool or not, i.e. the pool a forward over the same
 * rays needs to record every trip up to `walk_budget`.
 *
 * Ray order: a permutation of [0, num_rays) from sdf_ray_order; the kernels
 * trace rays in that order (outputs stay in the caller's order).  For rays
 * in no particular order (random training batches) it makes the rays of a
 * wavefront start in the same cell and point the same way.  Requires
 * settings->ray_image_width == 0.  ray_order == NULL: the caller's order.
 *
 * Gradient accumulator (backward): one 256-byte-aligned fp32 row per cell
 * holding that cell's attribute, position and point-error gradients side by
 * side.  The backward clears it, adds every ray's contributions into it,
 * then adds each row into attribute_grad, points_grad and point_error (fp16
 * outputs of an fp16 pipeline get the fp32 sums rounded once).  A wavefront's atomic update
 * of a cell then touches fewer 64-byte memory segments than updates of the
 * three output arrays do.  grad_accum == NULL: updates go to the outputs.
 *
 * Cell table (forward): the forward first copies, per cell, its position,
 * CSR row bounds and attribute row into one aligned record (64-256 bytes,
 * sdf_cell_table_bytes), in the same pass that fills the offset table, then
 * walks over the records, so a step reads one or two whole cache lines of the
 * cell instead of parts of three arrays.  cell_table == NULL: the forward
 * reads the arrays. */
typedef struct sdf_trace_plan {
    void *walk_record;        /* device memory, 256-byte aligned, or NULL */
    size_t walk_record_bytes; /* >= sdf_walk_record_pool_bytes(num_rays, ray_image_width,
                                 walk_budget, walk_record_chunks) */
    uint32_t walk_budget;     /* trips recorded per wavefront at most */
    const uint32_t *ray_order; /* device memory [num_rays], or NULL */
    void *grad_accum;          /* device memory, 256-byte aligned, or NULL */
    size_t grad_accum_bytes;   /* >= sdf_grad_accum_bytes(sh_degree, num_points) */
    uint32_t scratch_ready;    /* backward: nonzero if `scratch` already holds this
                                  scene's offset table (the forward over the same
                                  scene filled it); the backward then skips
                                  rebuilding it */
    void *cell_table;          /* forward: device memory, 256-byte aligned, or NULL */
    size_t cell_table_bytes;   /* >= sdf_cell_table_bytes(sh_degree, attr_type, num_points) */
    uint32_t walk_record_chunks; /* chunks of 16 trips in the record's pool, rounded up to
                                    a multiple of 8; 0: every wavefront's `walk_budget`
                                    trips (sdf_walk_record_full_chunks) */
} sdf_trace_plan;

/* Bytes of a walk record for every wavefront's `budget` trips (a pool that
 * never runs out), and for a pool of `chunks` chunks (0: the same). */
size_t sdf_walk_record_bytes(uint32_t num_rays, uint32_t ray_image_width,
                             uint32_t budget);
size_t sdf_walk_record_pool_bytes(uint32_t num_rays, uint32_t ray_image_width,
                                  uint32_t budget, uint32_t chunks);
uint32_t sdf_walk_record_full_chunks(uint32_t num_rays, uint32_t ray_image_width,
                                     uint32_t budget);

/* Bytes of the forward's cell table (0 for an invalid degree or type). */
size_t sdf_cell_table_bytes(int sh_degree, int attr_type, uint32_t num_points);

/* Bytes of the backward's gradient accumulator (0 for an invalid degree). */
size_t sdf_grad_accum_bytes(int sh_degree, uint32_t num_points);

/* Scratch bytes of sdf_ray_order. */
size_t sdf_ray_order_scratch_bytes(uint32_t num_points, uint32_t num_rays);

/* order[num_rays]: rays sorted by (start cell, Z-order of the octahedral
 * direction); stable, so the same inputs give the same order.  scratch must
 * be 256-byte aligned. */
int sdf_ray_order(uint32_t num_points, uint32_t num_rays, const float *rays,
                  const uint32_t *start_point_index, uint32_t *order,
                  void *scratch, size_t scratch_bytes, void *stream);

/* sdf_trace_forward with a plan (writes the walk record if given). */
int sdf_trace_forward_planned(
    const sdf_trace_plan *plan, int sh_degree,
    const sdf_trace_settings *settings, uint32_t num_points,
    const float *points, const float *attributes, uint32_t adjacency_size,
    const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets,
    uint32_t num_rays, const float *rays, const uint32_t *start_point_index,
    uint32_t num_depth_quantiles, const float *depth_quantiles,
    float *ray_rgba, float *quantile_depths, uint32_t *quantile_point_indices,
    uint32_t *num_intersections, float *point_contribution,
    const float *sharpness, float *alpha_output, void *scratch,
    size_t scratch_bytes, void *stream);

/* sdf_trace_backward with a plan (replays the forward's walk record). */
int sdf_trace_backward_planned(
    const sdf_trace_plan *plan, int sh_degree,
    const sdf_trace_settings *settings, uint32_t num_points,
    const float *points, const float *attributes, uint32_t adjacency_size,
    const uint32_t *point_adjacency, const uint32_t *point_adjacency_offsets,
    uint32_t num_rays, const float *rays, const uint32_t *start_point_index,
    uint32_t num_depth_quantiles, const float *depth_quantiles,
    const uint32_t *quantile_point_indices, const float *ray_rgba,
    const float *ray_rgba_grad, const float *depth_grad,
    const float *ray_error, float *points_grad, float *attribute_grad,
    float *point_error, const float *sharpness, float *sharpness_grad,
    void *scratch, size_t scratch_bytes, void *stream);

/* ---- batch prefetcher ---------------------------------------------------
 * Replaces BatchFetcher (src/utils/batch_fetcher.h:7-21,
 * src/utils/batch_fetcher.cpp:29-157; torch_bindings/torch_bindings.cpp:
 * 32-63).  A worker thread gathers batches of `batch_size` rows (`stride`
 * bytes each) of the host array `data` -- random rows seeded per element as
 * the reference seeds them (shuffle), or consecutive rows wrapping around --
 * into pinned staging buffers, and uploads them into a ring of 4 slots of
 * caller-allocated device memory on its own stream.  Each
 * sdf_batch_fetcher_next copies the next batch, in order, into `dst` on the
 * caller's stream (the stream first waits for the batch's upload; the call
 * blocks only until the worker has queued it).  `data` and `device_ring` must
 * stay valid until sdf_batch_fetcher_destroy returns. */
typedef struct sdf_batch_fetcher sdf_batch_fetcher;

/* Device bytes of the ring: 4 * stride * batch_size. */
size_t sdf_batch_fetcher_ring_bytes(size_t stride, size_t batch_size);

/* num_threads: gather threads (0 = 8). */
int sdf_batch_fetcher_create(const void *data, size_t num_bytes, size_t stride,
                             size_t batch_size, int shuffle, void *device_ring,
                             size_t device_ring_bytes, uint32_t num_threads,
                             sdf_batch_fetcher **out);
int sdf_batch_fetcher_next(sdf_batch_fetcher *fetcher, void *dst, void *stream);
int sdf_batch_fetcher_destroy(sdf_batch_fetcher *fetcher);

/* The rows batch `batch_index` takes (host computation, for tests). */
void sdf_batch_rows(uint32_t batch_index, size_t batch_size, size_t num_rows,
                    int shuffle, uint32_t *rows);

/* Batch `batch_index` of a device-resident array `data` [num_rows] of
 * `stride`-byte rows (a multiple of 4; 4-byte aligned) into `dst`
 * [batch_size] on `stream`: the rows sdf_batch_rows selects (the
 * reference's per-element seeding, src/utils/batch_fetcher.cpp:63-72),
 * gathered by the GPU.  No counterpart in the reference, which keeps the
 * array on the host (src/utils/batch_fetcher.cpp:29-157): for arrays that
 * fit in HBM it replaces the host gather and upload of BatchFetcher::next. */
int sdf_batch_gather(const void *data, size_t num_rows, size_t stride,
                     uint32_t batch_index, size_t batch_size, int shuffle,
                     void *dst, void *stream);

/* Implicit AABB tree over consecutive point pairs, tree [pow2(N), 2, 3]
 * (node (d, i) at 2^td - 2^(d+1) + i; the last entry is zeroed);
 * 1 <= N <= 2^31 (here and for sdf_nn and sdf_start_points).
 * Replaces build_aabb_tree (src/aabb_tree/aabb_tree.h:10-13,
 * src/aabb_tree/aabb_tree.cu:294-341). */
int sdf_build_aabb_tree(const float *points, uint32_t num_points,
                        float *aabb_tree, void *stream);

/* Exact nearest point of each query by fp32 distance (ties: smallest
 * index); num_points >= 32 as in the reference.
 * Replaces nn (src/aabb_tree/aabb_tree.h:16-23,
 * src/aabb_tree/aabb_tree.cu:343-415). */
int sdf_nn(const float *points, const float *aabb_tree, const float *queries,
           uint32_t num_points, uint32_t num_queries, uint32_t *indices,
           void *stream);

/* Start cell of each ray: the nearest point to its origin (rays [num_rays, 6],
 * origin first), as sdf_nn over the distinct origins gives it for finite
 * points and origins (ties: smallest index), without a host synchronisation:
 * the origins are deduplicated on the GPU by their bits, and each distinct
 * one is searched once (a scan over all points when there are at most 256,
 * else the tree).  scratch: sdf_start_points_scratch_bytes(num_rays),
 * 256-byte aligned; num_points >= 32.
 * Replaces get_starting_point (sdfoam_model/scene.py:272-282: torch.unique
 * over the origins, then nn). */
size_t sdf_start_points_scratch_bytes(uint32_t num_rays);
int sdf_start_points(const float *rays, uint32_t num_rays, const float *points,
                     uint32_t num_points, const float *aabb_tree, uint32_t *start,
                     void *scratch, size_t scratch_bytes, void *stream);

/* Per point: the farthest CSR neighbour (UINT32_MAX if none is farther
 * than 0) and cell_radius = sum of half the neighbour distances / row length.
 * Neighbours out of range are skipped.
 * Replaces farthest_neighbor (src/delaunay/triangulation_ops.h:8-16,
 * src/delaunay/triangulation_ops.cu:8-44;
 * torch_bindings/triangulation_bindings.cpp:183-214). */
int sdf_farthest_neighbor(const float *points, uint32_t num_points,
                          uint32_t adjacency_size,
                          const uint32_t *point_adjacency,
                          const uint32_t *point_adjacency_offsets,
                          uint32_t *indices, float *cell_radius, void *stream);

/* Scratch bytes of sdf_sort_points (0 where no GPU is present). */
size_t sdf_sort_points_scratch_bytes(uint32_t num_points);

/* perm[num_points]: the point order the reference's tree builder leaves
 * (sorted points = points[perm]); scratch 256-byte aligned.
 * Replaces sort_points (src/aabb_tree/aabb_tree.h:10-14,
 * src/aabb_tree/aabb_tree.cu:62-190). */
int sdf_sort_points(const float *points, uint32_t num_points, uint32_t *perm,
                    void *scratch, size_t scratch_bytes, void *stream);

/* point_adjacency entries sdf_delaunay_tables needs room for: 4 N + 2 T + 64
 * (2 E <= 4 N + 2 T for a tetrahedralised ball). */
uint64_t sdf_delaunay_adjacency_capacity(uint32_t num_points, uint32_t num_tets);

/* Scratch bytes of sdf_delaunay_tables (0 where no GPU is present). */
size_t sdf_delaunay_tables_scratch_bytes(uint32_t num_points, uint32_t num_tets);

/* Tables of a Delaunay tetrahedralisation given as tets [T,4] (vertex ids,
 * either orientation, any order) and neighbors [T,4] (the tet across the
 * face opposite vertex j, or -1 on the hull), as Qhull returns them:
 * tets_out [T,4] with vertices ascending except the last two, swapped
 * where that makes the tet positively oriented (det[b-a, c-a, d-a] > 0 in
 * double), ordered by their sorted vertex sets; tet_adjacency [T,4] = 4 k + m for
 * neighbour k and its face m, UINT32_MAX on the hull; vert_to_tet [N] the
 * lowest tet holding each point (UINT32_MAX if none);
 * point_adjacency_offsets [N+1] and point_adjacency (the Delaunay edges, CSR
 * with ascending rows; offsets[N] entries are written).  Synchronizes the
 * stream once.  scratch 256-byte aligned.
 * Replaces the tables of Triangulation (src/delaunay/delaunay.h:14-44,
 * src/delaunay/delaunay.cu:146-226;
 * torch_bindings/triangulation_bindings.cpp:11-115). */
int sdf_delaunay_tables(const float *points, uint32_t num_points,
                        const uint32_t *tets, const int32_t *neighbors,
                        uint32_t num_tets, uint32_t *tets_out,
                        uint32_t *tet_adjacency, uint32_t *vert_to_tet,
                        uint32_t *point_adjacency_offsets,
                        uint32_t *point_adjacency,
                        uint64_t point_adjacency_capacity, void *scratch,
                        size_t scratch_bytes, void *stream);

/* The Delaunay tetrahedralisation on the GPU, in two calls around a host
 * triangulation of the few points the GPU leaves open.  Together they
 * replace the tetrahedra of Triangulation::rebuild
 * (src/delaunay/delaunay.cu:271-345: sample_initial_tets, growth_iteration,
 * delete_delaunay_violations).
 *
 * sdf_delaunay_certify: a Voronoi cell per point, clipped by its
 * neighbours on a uniform grid; a cell closed by bisectors with every sign
 * decided certifies its tetrahedra, written to reports [capacity, 4] as
 * (point, a, b, c).  The other points go to open_points [N].  counts[5]
 * (host): report rows asked for (more than report_capacity: nothing is
 * lost but the rows past it; call again with room for counts[0]), open
 * points, undecided cells, cells over the fixed capacity, coincident
 * points seen (nonzero: duplicate points).  scratch 256-byte aligned, kept
 * for sdf_delaunay_merge.  32 to 2^26 points.  Synchronizes the stream. */
size_t sdf_delaunay_certify_scratch_bytes(uint32_t num_points);
int sdf_delaunay_certify(const float *points, uint32_t num_points,
                         uint32_t *reports, uint64_t report_capacity,
                         uint32_t *open_points, uint64_t *counts, void *scratch,
                         size_t scratch_bytes, void *stream);

/* sdf_delaunay_certify_exhaustive: sdf_delaunay_certify for a small set
 * (the points the full certification leaves open, certified among
 * themselves), with a clipping box 1e8 extents wide and every cell the grid
 * search leaves open clipped by every point of the set.  A cell then closed
 * certifies as above; a cell still reaching the box (a hull point of the
 * set) is listed in open_points and its vertices off the box faces are
 * reported as well: with the certified ones, every Delaunay tetrahedron of
 * the set whose circumcentre lies within the box.  counts as for
 * sdf_delaunay_certify.  32 to 2^20 points (its time grows as the square
 * of the number the grid search leaves open).  Synchronizes the stream.
 * No counterpart in the reference: it replaces the host triangulation of
 * the open points between the two calls above. */
int sdf_delaunay_certify_exhaustive(const float *points, uint32_t num_points,
                                    uint32_t *reports, uint64_t report_capacity,
                                    uint32_t *open_points, uint64_t *counts,
                                    void *scratch, size_t scratch_bytes, void *stream);

/* sdf_delaunay_merge: candidates [M, 4] (the Delaunay tetrahedra of the open
 * points, as global point ids) are kept where their circumsphere holds no
 * point; each certified tetrahedron is kept once.  Writes tets [T, 4] (any
 * orientation, any order) and neighbors [T, 4] (across the face opposite
 * vertex j, -1 on the hull), the form sdf_delaunay_tables takes.  result[4]
 * (host): T, hull faces, invalid or undecided rows, faces of three tets.
 * certify_scratch: the scratch of the sdf_delaunay_certify call that made
 * the reports.  Fails when a candidate's sign cannot be decided or
 * T > tet_capacity (result[0] then holds T).  At most 2^26 candidates.
 * Synchronizes the stream. */
size_t sdf_delaunay_merge_scratch_bytes(uint32_t num_points, uint64_t num_reports,
                                        uint64_t num_candidates, uint64_t tet_capacity);
int sdf_delaunay_merge(const float *points, uint32_t num_points,
                       void *certify_scratch, size_t certify_scratch_bytes,
                       const uint32_t *reports, uint64_t num_reports,
                       const uint32_t *candidates, uint64_t num_candidates,
                       uint32_t *tets, int32_t *neighbors, uint64_t tet_capacity,
                       uint64_t *result, void *scratch, size_t scratch_bytes,
                       void *stream);

/* Incremental rebuild over moved points, the same tetrahedra count
 * (replaces delete_delaunay_violations, src/delaunay/delete_violations.cu:
 * 7-178, and the regrowth from its frontier, src/delaunay/delaunay.cu:
 * 288-345).
 *
 * sdf_delaunay_check: the grid over the moved points into certify_scratch
 * (sdf_delaunay_certify_scratch_bytes), then each old tetrahedron [T, 4]
 * (neighbors [T, 4], -1 on the hull, as sdf_delaunay_merge writes them):
 * keep[t] = 1 when no point lies strictly inside its circumsphere (every
 * sign decided), else 0.  dirty[N]: 2 for the vertices of hull faces, 1 for
 * the other vertices of tetrahedra not kept, else 0 (the hull's vertices
 * need not be certified: their cells are unbounded, they go straight to the
 * open points).  A tetrahedron with a clean vertex is a
 * Delaunay tetrahedron of the moved points exactly when it is one of the
 * kept old ones; the others all have four dirty vertices.  Fails on a
 * vertex id >= N.  Synchronizes the stream. */
int sdf_delaunay_check(const float *points, uint32_t num_points,
                       const uint32_t *tets, const int32_t *neighbors,
                       uint64_t num_tets, uint32_t *keep, uint32_t *dirty,
                       void *certify_scratch, size_t certify_scratch_bytes,
                       void *stream);

/* sdf_delaunay_certify_points: sdf_delaunay_certify for the listed points
 * only (query [Q], ids below N; reports, open_points and counts as there),
 * on the grid an sdf_delaunay_check call over the same points left in the
 * scratch; the other points count as clean.  Then sdf_delaunay_merge_verified
 * merges its reports, the open points' candidates and the kept old
 * tetrahedra that have a clean vertex and no certified one.
 * Synchronizes the stream. */
int sdf_delaunay_certify_points(const float *points, uint32_t num_points,
                                const uint32_t *query, uint32_t num_query,
                                uint32_t *reports, uint64_t report_capacity,
                                uint32_t *open_points, uint64_t *counts,
                                void *certify_scratch, size_t certify_scratch_bytes,
                                void *stream);

/* sdf_delaunay_merge with verified rows [V, 4] kept as they are (their
 * circumspheres already checked).  scratch:
 * sdf_delaunay_merge_scratch_bytes(N, num_reports, num_candidates + V,
 * tet_capacity). */
int sdf_delaunay_merge_verified(const float *points, uint32_t num_points,
                                void *certify_scratch, size_t certify_scratch_bytes,
                                const uint32_t *reports, uint64_t num_reports,
                                const uint32_t *candidates, uint64_t num_candidates,
                                const uint32_t *verified, uint64_t num_verified,
                                uint32_t *tets, int32_t *neighbors, uint64_t tet_capacity,
                                uint64_t *result, void *scratch, size_t scratch_bytes,
                                void *stream);

/* ---- measurement and test hooks (no counterpart in the reference) ----- */

/* Per-ray walk statistics of the forward (backward = 0) or backward
 * (backward = 1) walk with the same settings: FNV-1a-64 hash of the cell
 * sequence of the steps, number of steps, faces scanned in all loop
 * iterations and faces of the stepped cells.  Any output may be NULL.
 * Used by the parity tests (visit sequences) and the bench (byte model). */
int sdf_trace_walk_stats(int sh_degree, const sdf_trace_settings *settings,
                         int backward, uint32_t num_points, const float *points,
                         const float *attributes, uint32_t adjacency_size,
                         const uint32_t *point_adjacency,
                         const uint32_t *point_adjacency_offsets,
                         uint32_t num_rays, const float *rays,
                         const uint32_t *start_point_index,
                         const float *sharpness, uint64_t *visit_hash,
                         uint32_t *steps, uint64_t *faces,
                         uint64_t *faces_stepped, uint32_t *cells,
                         uint32_t cells_stride, void *scratch,
                         size_t scratch_bytes, void *stream);

/* Evaluate the fp-math contract on the device, n elements:
 * op 0: out_f32 = sdf_expf(in); op 1: out_u16 = fp16 bits of in (RNE);
 * op 2: out_f32 = sdf_sigmoidf(in). */
int sdf_debug_fpmath(int op, const float *in, void *out, uint64_t n,
                     void *stream);

/* Kernel timing.  While enabled, every kernel launch of the entry points
 * above is bracketed by two HIP events recorded on its stream (up to 512
 * launches are kept).  sdf_timing_collect waits for them, writes each
 * launch's kind (SDF_KERNEL_*) and duration in milliseconds, in launch
 * order, sets *n_out, and empties the record.  sdf_set_timing also empties
 * it.  Not for use under stream capture. */
#define SDF_KERNEL_PREFETCH 0
#define SDF_KERNEL_FORWARD 1
#define SDF_KERNEL_BACKWARD 2
#define SDF_KERNEL_AABB_TREE 3
#define SDF_KERNEL_NN 4
#define SDF_KERNEL_RENDER 5
#define SDF_KERNEL_RAY_ORDER 6
#define SDF_KERNEL_GRAD_CLEAR 7
#define SDF_KERNEL_GRAD_FINALIZE 8
#define SDF_KERNEL_SCENE_PREP 9 /* offset table + cell table, one pass */
int sdf_set_timing(int enable);
int sdf_timing_collect(int *kinds, float *ms, int max_n, int *n_out);

#ifdef __cplusplus
}
#endif

#endif /* SDFOAM_HIP_H */
