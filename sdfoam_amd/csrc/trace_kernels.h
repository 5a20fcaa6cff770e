// Kernel argument blocks and launchers shared by the C ABI (capi.hip) and
// the kernels (trace_kernels.hip, aabb_kernels.hip).
#pragma once

#include "trace_device.h"

namespace sdfoam_hip {

// Set the calling thread's sdf_last_error() message and return `code`
// (capi.hip).
int fail(int code, const char *fmt, ...);
int hip_fail(hipError_t e, const char *where);

// Walk record: for every wavefront, up to `budget` trips of 64 entries (one
// per lane) of {next cell, bits of t1}, with next = kNoIndex where the
// lane's walk ended on that trip and kWalkUnrecorded where the lane was not
// walking.  Written by the forward of the sdfoam (safe) walk, replayed by
// its backward, which then skips the face scans; a lane scans again from
// its first unrecorded trip (past `budget`, past the wavefront's last
// recorded chunk, or where it outlives the forward's walk).  Beside every
// entry, in a second array of the same shape, the forward keeps the step's
// colour and density channel {r, g, b, row[channel]} (channel: sdf_channel
// in sdfoam mode, D - 1 in standard mode), so the backward of a recorded
// step reads 16 bytes instead of the cell's attribute row and skips the SH
// sum.
//
// Storage is sized by need: trips are stored in chunks of kChunkTrips rows
// that a wavefront claims from a shared pool as it walks (a counter per
// XCD, each with its own eighth of the pool, so the claims of one XCD stay
// in its L2); its chunk table lists them in trip order.  A wavefront whose
// claim finds its sub-pool empty records nothing from there on.  The
// counters keep counting past their sub-pools, so after the forward their
// sum is the number of chunks the walk asked for.
constexpr uint32_t kWalkUnrecorded = 0xfffffffeu;
// Standard mode: where the density backward's unsafe walk would leave the
// forward's safe one, the forward keeps its own step as {next | kWalkDiffers,
// t1} (num_points < 2^31 - 1, so the mark leaves both sentinels free); the
// backward scans from there and takes up the record again once its walk
// stands where the forward stood after one of the next kSeekWindow steps.
constexpr uint32_t kWalkDiffers = 0x80000000u;
constexpr uint32_t kSeekWindow = 8;
constexpr uint32_t kWalkRecordEntryBytes = 8u + 16u;
constexpr uint32_t kChunkTrips = 16;
constexpr uint32_t kChunkEntries = kChunkTrips * 64;
// record layout: kXcds counters (one 256-byte line each), the chunk tables
// (rounded up to 256 bytes), the pool's entries, then their colours
constexpr uint32_t kRecordHeadBytes = kXcds * 256;

struct WalkRecordArgs {
    uint2 *entries;     // NULL: no record; chunk k is entries [k, k + 1) * kChunkEntries
    float4 *colors;     // entries' colours, same indexing
    uint32_t *chunks;   // per wavefront, chunk_slots(budget) chunk numbers (kNoIndex: none)
    uint32_t *counters; // chunks asked for, per XCD (64 words apart)
    uint32_t budget;    // trips recorded per wavefront at most
    uint32_t pool;      // chunks in the pool (a multiple of kXcds)
};

__host__ __device__ inline uint32_t chunk_slots(uint32_t budget) {
    return (budget + kChunkTrips - 1) / kChunkTrips;
}

// Stores into the walk record.  It is written once by the forward and read
// once by the backward, so the stores are non-temporal: they do not displace
// the scene's cell data from L2 while the forward walks.
__device__ inline void record_store(uint2 *p, uint2 v) {
    __builtin_nontemporal_store(((uint64_t)v.y << 32) | v.x, reinterpret_cast<uint64_t *>(p));
}
__device__ inline void record_store(float4 *p, float4 v) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<f4v *>(p));
}

// Loads from the walk record (the backward reads each entry once): also
// non-temporal, so the stream of record rows does not displace the cells'
// points and gradient rows from L2.
__device__ inline uint2 record_load(const uint2 *p) {
    const uint64_t v = __builtin_nontemporal_load(reinterpret_cast<const uint64_t *>(p));
    return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}
__device__ inline float4 record_load(const float4 *p) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v w = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p));
    return make_float4(w.x, w.y, w.z, w.w);
}

// wavefronts of the launch grid, the padding blocks included (they write
// their "unrecorded" row)
__host__ inline uint64_t walk_record_waves(uint32_t num_tiles) {
    return (uint64_t)grid_blocks_for_tiles(num_tiles) * (kBlock / 64);
}

// chunks for `budget` trips of every wavefront (what a pool that can never
// run out holds), a multiple of kXcds
__host__ inline uint64_t walk_record_full_chunks(uint32_t num_tiles, uint32_t budget) {
    const uint64_t c = walk_record_waves(num_tiles) * chunk_slots(budget);
    return (c + kXcds - 1) / kXcds * kXcds;
}

// the pool of a plan asking for `chunks` (0: the full pool), rounded up to
// a multiple of kXcds
__host__ inline uint64_t record_pool_chunks(uint32_t num_tiles, uint32_t budget, uint32_t chunks) {
    if (chunks == 0) return walk_record_full_chunks(num_tiles, budget);
    return ((uint64_t)chunks + kXcds - 1) / kXcds * kXcds;
}

__host__ inline uint64_t walk_record_table_bytes(uint32_t num_tiles, uint32_t budget) {
    return (walk_record_waves(num_tiles) * chunk_slots(budget) * 4 + 255) / 256 * 256;
}

__host__ inline uint64_t walk_record_bytes_for(uint32_t num_tiles, uint32_t budget,
                                               uint64_t chunks) {
    return kRecordHeadBytes + walk_record_table_bytes(num_tiles, budget) +
           chunks * kChunkEntries * kWalkRecordEntryBytes;
}

// this wavefront's chunk table.  Tables belong to tiles, not blocks, so
// kernels with different tile runs share them.
template <uint32_t CHUNK>
__device__ inline uint32_t *walk_record_table(const WalkRecordArgs &r) {
    const uint64_t wave = (uint64_t)block_tile<CHUNK>() * (kBlock / 64) + (threadIdx.x >> 6);
    return r.chunks + wave * chunk_slots(r.budget);
}

// This lane's entry of trip `trip` (< budget) of the wavefront with chunk
// table `tab`, or NULL where that trip has no chunk.
__device__ inline uint64_t record_slot(const WalkRecordArgs &r, const uint32_t *tab,
                                       uint32_t trip, uint32_t lane) {
    const uint32_t c = tab[trip / kChunkTrips];
    return c == kNoIndex ? ~0ull
                         : (uint64_t)c * kChunkEntries + (trip % kChunkTrips) * 64u + lane;
}

struct FwdArgs {
    WalkRecordArgs record;
    const uint32_t *order; // NULL, or the launch order of the rays (num_tiles from num_rays)
    SceneView scene;
    sdf_trace_settings settings;
    const float *rays;
    uint32_t num_rays;
    uint32_t num_tiles; // num_ray_tiles(num_rays, settings.ray_image_width)
    const uint32_t *start;
    uint32_t num_quantiles;
    const float *quantiles;
    const float *sharpness;
    void *rgba; // [R, 4] of the attribute type
    float *depth;
    uint32_t *depth_indices;
    uint32_t *num_intersections;
    void *contribution; // [N] of the attribute type
    float *alpha_out;
    // walk statistics (STATS instantiation only)
    uint64_t *visit_hash;
    uint32_t *steps;
    uint64_t *faces;
    uint64_t *faces_stepped;
    uint32_t *cells;
    uint32_t cells_stride;
};

struct BwdArgs {
    WalkRecordArgs record;
    const uint32_t *order;
    SceneView scene;
    sdf_trace_settings settings;
    const float *rays;
    uint32_t num_rays;
    uint32_t num_tiles; // num_ray_tiles(num_rays, settings.ray_image_width)
    const uint32_t *start;
    uint32_t num_quantiles;
    const float *quantiles;
    const uint32_t *depth_indices;
    const void *rgba;      // attribute type
    const void *rgba_grad; // attribute type
    const float *depth_grad;
    const void *ray_error; // attribute type
    const float *sharpness;
    float *points_grad;
    void *attr_grad;   // attribute type
    void *point_error; // attribute type
    float *sharpness_grad;
    // per-cell fp32 gradient rows (accum_stride(L) floats: attribute row,
    // position x/y/z, point error), added into the outputs by
    // launch_grad_finalize; nullptr: atomics go to the outputs directly
    float *accum;
    // walk statistics (STATS instantiation only)
    uint64_t *visit_hash;
    uint32_t *steps;
    uint64_t *faces;
    uint64_t *faces_stepped;
    uint32_t *cells;
    uint32_t cells_stride;
};

// Inference render (Pipeline::trace_benchmark): rays cast per pixel.
struct RenderArgs {
    SceneView scene; // diff: the caller's table, no padding
    sdf_trace_settings settings;
    float position[3], forward[3], right[3], up[3];
    float fov, focal; // focal = 1 / tan(fov / 2)
    uint32_t width, height, model;
    uint32_t num_tiles; // num_ray_tiles(width * height, width)
    float bg[3];
    int32_t checker_bg;
    const uint32_t *start; // one element
    const float *sharpness;
    uint32_t *out;
};

hipError_t launch_render(int L, const RenderArgs &a, bool neus, bool half, hipStream_t stream);

// Ray launch order for rays in no particular order: sort by (start cell,
// Morton code of the octahedral direction) so a wavefront's rays start
// together and point the same way.
size_t ray_order_scratch_bytes(uint32_t num_points, uint32_t num_rays);
hipError_t launch_ray_order(uint32_t num_points, uint32_t num_rays, const float *rays,
                            const uint32_t *start, uint32_t *order, void *scratch,
                            size_t scratch_bytes, hipStream_t stream);

hipError_t launch_prefetch_diff(const float *points, uint32_t num_points, uint32_t num_adj,
                                const uint32_t *adj, const uint32_t *offs, uint2 *diff,
                                hipStream_t stream);
// Before a forward that records: the counters to 0 and every chunk table
// entry to kNoIndex.
hipError_t launch_record_reset(const WalkRecordArgs &r, uint64_t table_words, hipStream_t stream);
// half: fp16 attributes (settings.attr_type == SDF_ATTR_F16).  With
// a.scene.cells set, the forward (not its statistics instantiation) walks
// over that cell table, which launch_cell_table filled.
hipError_t launch_forward(int L, const FwdArgs &a, bool neus, bool stats, bool half,
                          hipStream_t stream);
// Fills the fp16 offset table `diff` (as launch_prefetch_diff) and the cell
// table (cell_record_bytes(L, attribute size) per cell) from sc's points,
// adjacency, offsets and attributes, in one pass.
hipError_t launch_scene_prep(int L, bool half, const SceneView &sc, uint32_t *cells, uint2 *diff,
                             hipStream_t stream);
// Floats per cell row of the backward's gradient accumulator: the next
// power of two >= D + 4 (attribute row, position, point error), at least 8,
// so that a row spans the fewest 64-byte segments.
constexpr uint32_t accum_stride(int L) {
    return L <= 0 ? 8u : L <= 2 ? 32u : 64u;
}

// Clears num_points rows of the accumulator.
hipError_t launch_grad_clear(int L, float *accum, uint32_t num_points, hipStream_t stream);

// attribute_grad [N, D] += rows[:, :D]; points_grad [N, 3] += rows[:, D:D+3];
// point_error [N] += rows[:, D+3] (point_error may be nullptr).  attr_grad and
// point_error are fp16 when `half` (the sum is rounded once), else fp32.
hipError_t launch_grad_finalize(int L, const float *accum, uint32_t num_points, void *attr_grad,
                                float *points_grad, void *point_error, bool half,
                                hipStream_t stream);

hipError_t launch_backward(int L, const BwdArgs &a, bool neus, bool stats, bool half,
                           hipStream_t stream);
hipError_t launch_fpmath(int op, const float *in, void *out, uint64_t n, hipStream_t stream);

hipError_t launch_farthest_neighbor(const float *points, uint32_t num_points, const uint32_t *adj,
                                    const uint32_t *offs, uint32_t num_adj, uint32_t *indices,
                                    float *cell_radius, hipStream_t stream);

// delaunay_tables.hip
size_t sort_points_scratch_bytes(uint32_t num_points);
hipError_t launch_sort_points(const float *points, uint32_t num_points, uint32_t *perm,
                              void *scratch, size_t scratch_bytes, hipStream_t stream);
uint64_t delaunay_edge_capacity(uint32_t num_points, uint32_t num_tets);
size_t delaunay_tables_scratch_bytes(uint32_t num_points, uint32_t num_tets);
// Synchronizes `stream` once (the edge count sizes the last sort).
// input_error: 1 = a vertex or neighbour index out of range, 2 = more edges
// than a tetrahedralised ball can have.
hipError_t launch_delaunay_tables(const float *points, uint32_t num_points,
                                  const uint32_t *tets_in, const int32_t *nbr_in,
                                  uint32_t num_tets, uint32_t *tets_out, uint32_t *tet_adj,
                                  uint32_t *vert_to_tet, uint32_t *offsets, uint32_t *adjacency,
                                  uint64_t adjacency_capacity, uint32_t &input_error,
                                  void *scratch, size_t scratch_bytes, hipStream_t stream);

// delaunay_gpu.hip
size_t delaunay_certify_scratch_bytes(uint32_t num_points);
// counts: report rows asked for, open points, undecided cells, cells over
// capacity, coincident point pairs.  Synchronizes `stream` twice.
hipError_t launch_delaunay_certify(const float *points, uint32_t num_points, uint32_t *reports,
                                   uint64_t report_capacity, uint32_t *open, uint64_t counts[5],
                                   void *scratch, size_t scratch_bytes, hipStream_t stream);
size_t delaunay_merge_scratch_bytes(uint32_t num_points, uint64_t num_reports,
                                    uint64_t num_candidates, uint64_t tet_capacity);
// result: tets, hull faces, invalid or undecided rows, faces of three tets.
// The verified rows (num_verified of them) are kept as they are; the scratch
// is sized for num_candidates + num_verified candidates.
hipError_t launch_delaunay_merge(const float *points, uint32_t num_points, void *grid_scratch,
                                 size_t grid_bytes, const uint32_t *reports, uint64_t num_reports,
                                 const uint32_t *candidates, uint64_t num_candidates,
                                 const uint32_t *verified, uint64_t num_verified,
                                 uint32_t *tets, int32_t *neighbors, uint64_t tet_capacity,
                                 uint64_t result[4], void *scratch, size_t scratch_bytes,
                                 hipStream_t stream);
// Incremental rebuild: the grid over the moved points into the certify
// scratch, every point clean, then one lane per old tetrahedron (keep, dirty
// marks).  errors: rows with a vertex out of range.  Synchronizes `stream`.
hipError_t launch_delaunay_check(const float *points, uint32_t num_points, const uint32_t *tets,
                                 const int32_t *neighbors, uint64_t num_tets, uint32_t *keep,
                                 uint32_t *dirty, uint64_t *errors, void *scratch,
                                 size_t scratch_bytes, hipStream_t stream);
// certify_kernel over the listed points on the grid a launch_delaunay_check
// call over the same points left in the scratch (hipErrorNotReady if none).
hipError_t launch_delaunay_certify_points(const float *points, uint32_t num_points,
                                          const uint32_t *query, uint32_t num_query,
                                          uint32_t *reports, uint64_t report_capacity,
                                          uint32_t *open, uint64_t counts[5], void *scratch,
                                          size_t scratch_bytes, hipStream_t stream);

hipError_t launch_build_aabb_tree(const float *points, uint32_t num_points, float *tree,
                                  hipStream_t stream);
// Scratch of launch_start_points: a counter, the origin hash table (uid
// beside it), each ray's slot, the distinct origins' rays and results.
struct StartLayout {
    uint64_t table_slots;
    size_t table, uid, ray_slot, uq_ray, best, bytes;
};
StartLayout start_layout(uint32_t num_rays);
// start[i] = the nearest point to ray i's origin (as nn over the distinct
// origins), without a host synchronisation.
hipError_t launch_start_points(const float *rays, uint32_t num_rays, const float *points,
                               uint32_t num_points, const float *tree, uint32_t *start,
                               void *scratch, hipStream_t stream);
hipError_t launch_nn(const float *points, const float *tree, const float *queries,
                     uint32_t num_points, uint32_t num_queries, uint32_t *indices,
                     hipStream_t stream);

} // namespace sdfoam_hip
