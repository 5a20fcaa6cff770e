// Forward / backward kernels of the Voronoi-foam tracer for gfx950, and the
// fp16 neighbour-offset prepass.
//
// One lane per ray, wave64, 256 lanes per block.  The walk is wave
// synchronous: every trip of the kernel's loop advances each live lane by one
// cell (the divergent part: face scan and the step's arithmetic), then the
// whole wave reconverges and applies the step's scattered updates grouped by
// cell.  Coherent rays of a wave sit in the same few cells at a time, so the
// lanes of a wave that stepped into one cell are summed first (ballot +
// readlane), and the sum goes out as one coalesced atomic instruction: lane i
// of the wave owns component i of the cell's gradient row.  The reference
// issues ~52 single-word atomics per step per ray instead
// (src/tracing/pipeline.cu:500-533).
//
// Each per-element contribution is the same fp32 product the reference
// forms; only the order of the sums differs (fp32 atomics have no order).
#include "trace_kernels.h"

#include <algorithm>

namespace sdfoam_hip {

// ---------------------------------------------------------------------------
// prefetch_adjacent_diff (src/tracing/pipeline.cu:1202-1242) by one lane per
// CSR entry, the row of entry k found by a binary search of the offsets.  Used
// for scenes without points only (every entry is then a NaN plane); otherwise
// scene_prep_kernel builds the table by rows.

__global__ __launch_bounds__(kBlock) void prefetch_diff_kernel(
    const float *__restrict__ points, uint32_t num_points, uint32_t num_adj,
    const uint32_t *__restrict__ adj, const uint32_t *__restrict__ offs,
    uint2 *__restrict__ diff) {
    const uint32_t k = blockIdx.x * kBlock + threadIdx.x;
    if (k >= num_adj + kDiffPad) return;
    if (k >= num_adj) {
        diff[k] = make_uint2(0u, 0u);
        return;
    }
    // last row i with offs[i] <= k
    uint32_t lo = 0, hi = num_points; // invariant: offs[lo] <= k, answer < hi
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (offs[mid] <= k) {
            lo = mid;
        } else {
            hi = mid;
        }
    }
    const uint32_t a = adj[k];
    if (a >= num_points) {
        diff[k] = make_uint2(0x7e007e00u, 0x7e00u); // NaN plane
        return;
    }
    const float px = points[3ull * lo], py = points[3ull * lo + 1], pz = points[3ull * lo + 2];
    const float qx = points[3ull * a], qy = points[3ull * a + 1], qz = points[3ull * a + 2];
    const uint32_t hx = f32_to_f16(qx - px);
    const uint32_t hy = f32_to_f16(qy - py);
    const uint32_t hz = f32_to_f16(qz - pz);
    diff[k] = make_uint2(hx | (hy << 16), hz);
}

// ---------------------------------------------------------------------------
// wave helpers

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}

__device__ __forceinline__ int first_lane(uint64_t mask) { return __builtin_ctzll(mask); }

// Lane mask of a per-lane predicate, taking the bool as the compare mask it
// already is (no widening to a 0/1 integer first).
__device__ __forceinline__ uint64_t lane_mask(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// The forward's claim of chunk `slot` of its wavefront's walk record: the
// first active lane takes the next chunk of its XCD's sub-pool (none once
// that is used up; the counter still counts the claim) and enters it in the
// chunk table.  The result is uniform over the wave.
__device__ inline uint32_t record_claim(const WalkRecordArgs &r, uint32_t *tab, uint32_t slot) {
    const uint32_t x = blockIdx.x % kXcds;
    const uint32_t per = r.pool / kXcds;
    uint32_t got = kNoIndex;
    if (lane_id() == (uint32_t)first_lane(__ballot(1))) {
        const uint32_t k = atomicAdd(r.counters + 64u * x, 1u);
        got = k < per ? x * per + k : kNoIndex;
        tab[slot] = got;
    }
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)got);
}

// The forward's per-cell updates, `contribution[cell] += w` per step and
// `alpha[cell] = a visiting step's alpha` (src/tracing/pipeline.cu:159-163;
// the reference's alpha store is a last-writer race), go through a per-wave
// hash table in LDS: a stepped lane claims its cell's slot by a
// compare-and-swap of the slot's tag (equal cells share it, others probe
// on), adds its weight there and stores its alpha, and every kContribTrips
// trips each lane flushes kContribSlots / 64 slots: one contribution atomic
// and one alpha store per distinct cell of those trips.  A flush follows at
// most 64 * kContribTrips = kContribSlots claims, so a probe always ends at
// its cell's slot or a free one.  The lanes' claims run side by side (a
// serial round per distinct cell costs more), and one global atomic per step
// costs far more (same-address adds serialise in L2).
constexpr uint32_t kContribTrips = 8;
constexpr uint32_t kContribSlots = 64 * kContribTrips;
constexpr uint32_t kContribFree = 0xffffffffu;

struct ContribTable {
    uint32_t tag[kContribSlots];
    float w[kContribSlots];
    float alpha[kContribSlots];
};

__device__ __forceinline__ void contrib_clear(ContribTable &ct) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (uint32_t k = 0; k < kContribSlots / 64; ++k) {
        ct.tag[lane + 64u * k] = kContribFree;
        ct.w[lane + 64u * k] = 0.0f;
    }
    __builtin_amdgcn_wave_barrier();
}

// One lane's step (any subset of the wave's lanes).
template <typename AT>
__device__ __forceinline__ void contrib_add(ContribTable &ct, uint32_t cell, float w, float alpha,
                                            void *contribution) {
    static_assert((kContribSlots & (kContribSlots - 1u)) == 0u, "a power of two");
    constexpr uint32_t kBits = __builtin_ctz(kContribSlots);
    uint32_t h = (cell * 0x9e3779b1u) >> (32u - kBits);
    for (uint32_t probe = 0; probe < kContribSlots; ++probe) {
        const uint32_t old = atomicCAS(&ct.tag[h], kContribFree, cell);
        if (old == kContribFree || old == cell) {
            atomicAdd(&ct.w[h], w);
            ct.alpha[h] = alpha;
            return;
        }
        h = (h + 1u) & (kContribSlots - 1u);
    }
    // not reached: the table has room for every claim between flushes
    if (contribution) atomic_add_elem<AT>(contribution, cell, w);
}

// The wave's pending sums (all 64 lanes).  Lane l holds slots l + 64 k; it
// flushes its occupied ones one per round, so the wave issues as many
// atomic and store instructions as its busiest lane has occupied slots
// (a few at C3) rather than one per slot position.
template <typename AT>
__device__ __forceinline__ void contrib_flush(ContribTable &ct, void *contribution, float *alpha_out) {
    static_assert(kContribSlots / 64 <= 32, "one bit per slot of a lane");
    __builtin_amdgcn_wave_barrier();
    const uint32_t lane = lane_id();
    uint32_t occ = 0u;
#pragma unroll
    for (uint32_t k = 0; k < kContribSlots / 64; ++k)
        occ |= (ct.tag[lane + 64u * k] != kContribFree ? 1u : 0u) << k;
    while (__ballot(occ != 0u)) {
        if (occ) {
            const uint32_t k = (uint32_t)__builtin_ctz(occ);
            occ &= occ - 1u;
            const uint32_t s = lane + 64u * k;
            const uint32_t c = ct.tag[s];
            const float v = ct.w[s];
            ct.tag[s] = kContribFree;
            ct.w[s] = 0.0f;
            if (contribution) atomic_add_elem<AT>(contribution, c, v);
            if (alpha_out) alpha_out[c] = ct.alpha[s];
        }
    }
    __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------------------
// forward (src/tracing/pipeline.cu:36-264)

// Waves per SIMD asked of the forward over the cell table for image rays
// (the compiler then keeps it to 512 / kForwardWaves VGPRs).
constexpr int kForwardWaves = 6;

// CT: walk over the cell table (a.scene.cells) and read attribute rows from it.
// HALF: the face scan's half-batch loads (walk_advance), for rays in an
// explicit launch order (incoherent batches such as random training pixels).
template <int L, bool NEUS, bool STATS, typename AT, bool CT = false, bool HALF = false>
__global__ __launch_bounds__(kBlock)
__attribute__((amdgpu_waves_per_eu(CT && !HALF && !STATS ? kForwardWaves : 1))) void
forward_kernel(FwdArgs a) {
    constexpr uint32_t RB = CT ? cell_record_bytes(L, sizeof(AT)) : 0u;
    constexpr int nsh = (L + 1) * (L + 1);
    constexpr int D = 1 + 3 * nsh;
    __shared__ ContribTable contrib_tables[STATS ? 1 : kBlock / 64];
    ContribTable &ct = contrib_tables[STATS ? 0 : threadIdx.x >> 6];
    if constexpr (!STATS) contrib_clear(ct);
    bool valid;
    const uint32_t ray_idx =
        ray_for_lane<kForwardChunk>(a.num_rays, a.settings.ray_image_width, a.num_tiles, valid,
                                    a.order);
    const uint32_t lane = lane_id();

    RayF ray = {};
    if (valid) ray = load_ray(a.rays, ray_idx);
    // SH basis of the lane's ray, in registers (the kernel's LDS goes to the
    // contribution table; in LDS the basis cost 16 reads per step and
    // limited the blocks per CU)
    float sh[nsh];
    sh_basis<L>(ray.dx, ray.dy, ray.dz, sh);
    const float sha = a.sharpness[0];
    const int32_t sdf_ch = a.settings.sdf_channel;
    const bool neus_alpha = NEUS && sdf_ch >= 0;
    const float thr = a.settings.weight_threshold;
    const uint32_t Q = a.num_quantiles;
    const float *rq = (valid && a.quantiles) ? a.quantiles + (uint64_t)ray_idx * Q : nullptr;
    const uint32_t max_steps = a.settings.max_intersections;

    float T = 1.0f;
    float C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
    uint32_t qi = 0;
    float q = (rq && Q > 0) ? rq[0] : 0.0f;
    uint64_t hash = kFnvOffset;
    uint32_t rec = 0;

    WalkState ws;
    walk_init<RB>(a.scene, valid ? a.start[ray_idx] : kNoIndex, ws);
    WalkCounters wc = {0u, 0u, 0ull, 0ull};
    // walk record of this wavefront: one row of 64 entries per trip, in
    // chunks of kChunkTrips rows claimed as the walk gets there; wslot is
    // this lane's entry in the current chunk's first row (~0: no chunk)
    uint32_t *wtab = nullptr;
    uint64_t wslot = ~0ull;
    if (!STATS && a.record.entries) wtab = walk_record_table<kForwardChunk>(a.record);
    uint32_t trip = 0;

    while (__ballot(ws.alive) != 0ull) {
        StepInfo si;
        si.stepped = false;
        si.found = false;
        uint2 entry = make_uint2(kWalkUnrecorded, 0u);
        if (ws.alive) {
            if constexpr (NEUS || STATS) {
                walk_advance<true, STATS, false, false, RB, HALF>(a.scene, ray, max_steps, ws, si, wc);
                entry = make_uint2(si.found ? si.next : kNoIndex,
                                   __builtin_bit_cast(uint32_t, si.t1));
            } else {
                // the density backward walks in the unsafe mode: a step is
                // recorded while that walk takes the same exit; from the first
                // step where it would not, the backward scans for itself
                walk_advance<true, false, false, true, RB, HALF>(a.scene, ray, max_steps, ws, si, wc);
                if (si.agrees)
                    entry = make_uint2(si.found ? si.next : kNoIndex,
                                       __builtin_bit_cast(uint32_t, si.t1));
                else if (si.found && a.scene.num_points < kWalkDiffers - 1u)
                    entry = make_uint2(si.next | kWalkDiffers,
                                       __builtin_bit_cast(uint32_t, si.t1));
            }
        }
        // where this trip's colour goes (the step's, if the lane steps)
        float4 *col = nullptr;
        if (wtab && trip < a.record.budget) {
            if (trip % kChunkTrips == 0) {
                const uint32_t c = record_claim(a.record, wtab, trip / kChunkTrips);
                wslot = c == kNoIndex ? ~0ull : (uint64_t)c * kChunkEntries + lane;
            }
            if (wslot != ~0ull) {
                const uint64_t i = wslot + (trip % kChunkTrips) * 64u;
                record_store(a.record.entries + i, entry);
                col = a.record.colors + i;
            }
        }
        ++trip;

        float alpha = 0.0f, w = 0.0f;
        bool keep = true;
        if (si.stepped) {
            const uint32_t cell = ws.cell;
            const float t0 = ws.t0, t1 = si.t1;
            const AT *__restrict__ row =
                CT ? reinterpret_cast<const AT *>(reinterpret_cast<const char *>(a.scene.cells) +
                                                  (uint64_t)cell * RB + kCellAttrByte)
                   : static_cast<const AT *>(a.scene.attrs) + (uint64_t)cell * D;
            float s = (float)row[D - 1];
            float chan = s; // the channel the backward reads (sdf value or density)
            const float dt = fmaxf(t1 - t0, 0.0f);
            if (neus_alpha) {
                const float d = (float)row[sdf_ch];
                chan = d;
                const float phi = sdf_sigmoidf(-sha * d);
                s = sha * phi * (1.0f - phi);
            }
            alpha = 1.0f - sdf_expf(-s * dt);
            w = T * alpha;
            const float Tn = T * (1.0f - alpha);
            if constexpr (!STATS) {
                float r, g, b;
                if (NEUS || (float)row[D - 1] > 1e-6f) {
                    sh_rgb_regs<L>(sh, row, r, g, b);
                } else {
                    r = g = b = 0.0f;
                }
                C0 = fmaf(w, r, C0);
                C1 = fmaf(w, g, C1);
                C2 = fmaf(w, b, C2);
                if (col) record_store(col, make_float4(r, g, b, chan));
                const uint64_t qbase = (uint64_t)ray_idx * Q;
                if (NEUS) {
                    const float drop = T - Tn;
                    if (drop > 1e-12f) {
                        while (qi < Q && Tn < q) {
                            float frac = (T - q) / drop;
                            frac = fminf(1.0f, fmaxf(0.0f, frac));
                            a.depth[qbase + qi] = fmaf(frac, t1 - t0, t0);
                            a.depth_indices[qbase + qi] = cell;
                            ++qi;
                            if (qi < Q) q = rq[qi];
                        }
                    }
                } else {
                    while (qi < Q && Tn < q) {
                        a.depth[qbase + qi] = t0 + logf(T / q) / s;
                        a.depth_indices[qbase + qi] = cell;
                        ++qi;
                        if (qi < Q) q = rq[qi];
                    }
                }
            } else {
                hash = fnv_step(hash, cell);
                if (a.cells && rec < a.cells_stride) a.cells[(uint64_t)ray_idx * a.cells_stride + rec] = cell;
                ++rec;
            }
            T = Tn;
            keep = T > thr;
        }

        if constexpr (!STATS) {
            // per cell: contribution += the weights, alpha = a visiting
            // step's alpha, through the wave's table
            if (si.stepped && (a.contribution || a.alpha_out))
                contrib_add<AT>(ct, ws.cell, w, alpha, a.contribution);
            if ((a.contribution || a.alpha_out) && trip % kContribTrips == 0u)
                contrib_flush<AT>(ct, a.contribution, a.alpha_out);
        }
        if (si.stepped && !keep) ws.alive = false;
        if (ws.alive && si.found) walk_move(ws, si);
    }
    // a backward lane that outlives this wave's walk reads "unrecorded": this
    // row, or (when the next trip would open a chunk) the chunk table's
    // kNoIndex, which the table starts out with
    if (wtab && trip < a.record.budget && trip % kChunkTrips != 0 && wslot != ~0ull)
        record_store(a.record.entries + wslot + (trip % kChunkTrips) * 64u,
                     make_uint2(kWalkUnrecorded, 0u));
    if constexpr (!STATS) {
        if (a.contribution || a.alpha_out) contrib_flush<AT>(ct, a.contribution, a.alpha_out);
    }

    if (!valid) return;
    if constexpr (STATS) {
        if (a.visit_hash) a.visit_hash[ray_idx] = hash;
        if (a.steps) a.steps[ray_idx] = wc.steps;
        if (a.faces) a.faces[ray_idx] = wc.faces;
        if (a.faces_stepped) a.faces_stepped[ray_idx] = wc.faces_stepped;
        return;
    }
    for (uint32_t k = qi; k < Q; ++k) {
        a.depth[(uint64_t)ray_idx * Q + k] = -1.0f;
        a.depth_indices[(uint64_t)ray_idx * Q + k] = kNoIndex;
    }
    store_attr4<AT>(a.rgba, ray_idx, make_float4(C0, C1, C2, 1.0f - T));
    if (a.num_intersections) a.num_intersections[ray_idx] = ws.n;
}

// ---------------------------------------------------------------------------
// backward, shared pieces

// Position-gradient bookkeeping of src/tracing/pipeline.cu:452-474 and
// :731-760: the gradient of a cell is flushed one step late, the first cell
// gets a face against the world origin (prev = 0) and the last two pending
// gradients are never flushed -- all as the reference does.  Returns whether
// a flush of (flush_idx, flush_g) is due.
//
// A step takes the face gradients of two faces: (prev, cur) as dprev and
// dt0_cur, and (cur, next) as dt1_cur and dt1_next.  The second face of a
// step is the first face of the next stepped step whenever that step's cell
// is this step's next (the usual case: t1 > t0 at every step), so its two
// gradients are kept (face_to, face_pq, face_qp) and the next step takes
// them instead of forming them again: the same inputs, so the same bits.
struct GeomState {
    uint32_t prev_idx;
    float prev_pt[3];
    float prev_g[3], cur_g[3], next_g[3];
    uint32_t face_to;   // cell the kept face leads to (kNoIndex: none kept)
    float face_pq[3];   // cell_isect_grad(prev_pt, x of face_to)
    float face_qp[3];   // cell_isect_grad(x of face_to, prev_pt)
};

__device__ __forceinline__ void geom_init(GeomState &gs) {
    gs.prev_idx = kNoIndex;
    gs.face_to = kNoIndex;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        gs.prev_pt[i] = 0.0f;
        gs.prev_g[i] = gs.cur_g[i] = gs.next_g[i] = 0.0f;
        gs.face_pq[i] = gs.face_qp[i] = 0.0f;
    }
}

__device__ __forceinline__ bool geom_step(GeomState &gs, uint32_t cell, const float *xc,
                                          uint32_t next, const float *xn, float dL_dt0,
                                          float dL_dt1, const RayF &ray, uint32_t &flush_idx,
                                          float *flush_g) {
    float dprev[3] = {0.0f, 0.0f, 0.0f};
    float dt1_cur[3], dt0_cur[3], dt1_next[3];
    if (gs.prev_idx != kNoIndex && cell == gs.face_to) {
        // the previous step's (cur, next) face: prev_pt and xc are its points
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            dprev[i] = gs.face_pq[i];
            dt0_cur[i] = gs.face_qp[i];
        }
    } else {
        if (gs.prev_idx != kNoIndex) cell_isect_grad(gs.prev_pt, xc, ray, dprev);
        cell_isect_grad(xc, gs.prev_pt, ray, dt0_cur);
    }
    cell_isect_grad_pair(xc, xn, ray, dt1_cur, dt1_next);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        gs.prev_g[i] = fmaf(dL_dt0, dprev[i], gs.prev_g[i]);
        gs.cur_g[i] = gs.cur_g[i] + (dL_dt0 * dt0_cur[i] + dL_dt1 * dt1_cur[i]);
        gs.next_g[i] = fmaf(dL_dt1, dt1_next[i], gs.next_g[i]);
    }
    const bool flush = gs.prev_idx != kNoIndex;
    flush_idx = gs.prev_idx;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        flush_g[i] = gs.prev_g[i];
        gs.prev_pt[i] = xc[i];
        gs.prev_g[i] = gs.cur_g[i];
        gs.cur_g[i] = gs.next_g[i];
        gs.next_g[i] = 0.0f;
        gs.face_pq[i] = dt1_cur[i];
        gs.face_qp[i] = dt1_next[i];
    }
    gs.prev_idx = cell;
    gs.face_to = next;
    return flush;
}

// Per-wave LDS tables of the backward's grouped updates.  Row 64 of `rec`
// is zero: it pads a batch of members, so padded slots add exact zeros.
// Tables are component-major with a pitch of 65 floats (lane 64 = the zero
// padding member): a lane reading its own values and the owner lanes reading
// one member's components both hit distinct LDS banks.
constexpr int kPitch = 65;

// Trips per grouping pass.  A lane's steps wait in kWindow LDS entry slots
// and are applied together every kWindow trips: rays of a wavefront enter
// the cells that others of it have just left, so a pass over several trips'
// steps meets fewer distinct cells than that many passes do (from oracle
// walks of C3 tiles: 64% of the groups over two trips, 49% over three).
// Three trips keep four blocks of 256 lanes per CU within its 160 KB of LDS
// (L = 3 without point error: 39.5 KB per block).
constexpr int kWindow = 3;

// PE: entries carry a point error (the caller asked for point_error).
template <int L, bool PE>
struct WaveTables {
    static constexpr int nsh = (L + 1) * (L + 1);
    static constexpr int kOnes = kPitch * nsh;      // offset of the row of ones
    static constexpr int kRec = kOnes + kPitch;     // offset of rec
    static constexpr int kComp = PE ? 8 : 7;        // components per entry
    static constexpr int kSlot = kPitch * kComp;    // floats per entry slot
    static constexpr int kEnd = kRec + kSlot * kWindow;
    // y [0, kOnes): SH basis function k of lane l at k * kPitch + l;
    // ones: the multiplier of the non-SH components;
    // rec [kRec, kEnd): kWindow entry slots; in slot s, component c of
    //   lane l's entry at s * kSlot + c * kPitch + l: dL/d(r, g, b, last
    //   channel), flushed position gradient (x, y, z), point error (PE)
    float buf[kEnd];
    __device__ float *y() { return buf; }
    __device__ float *rec() { return buf + kRec; }
};

// Next member of a lane mask (64 = padding once the mask is empty).  Three
// scalar instructions: s_ff1 and s_min (s_ff1 gives -1 for an empty mask)
// and s_bitset0, which takes bit m mod 64 (bit 0 of an already empty mask
// for the padding member).
__device__ __forceinline__ uint32_t pop_member(uint64_t &mm) {
    const uint32_t m = mm ? (uint32_t)__builtin_ctzll(mm) : 64u;
    asm("s_bitset0_b64 %0, %1" : "+s"(mm) : "s"(m));
    return m;
}

// What owner lane i of the wave accumulates for a member m: the product
// y[m * y_stride + y_base] * rec[m * g_stride + g_base]:
//   i < 3 nsh (SH):      Y_{i/3}(m) * dL/drgb_{i%3}(m)   (sh_utils.cuh:85-92)
//   i == last_ch:        1 * dL/dlast(m)
//   i == 60, 61, 62:     1 * flushed position gradient x, y, z (m)
//   i == 63 (PE):        1 * point error(m)
//   others:              a live component whose sum the lane never writes
struct OwnerLane {
    int y_base, g_base; // member m of slot 0: y = buf[y_base + m], g = buf[g_base + m]
    int g_slot;         // g of slot s is s * g_slot further
    bool also_last;     // last_ch is an SH component too: add dL/dlast as well
    // gradient accumulator row: this lane's float in a cell's row, and whether
    // the lane adds to it (attribute and position components; the point
    // error when it is asked for)
    uint32_t row_off;
    bool row_active;
};

template <int L, bool PE>
__device__ __forceinline__ OwnerLane owner_lane(int last_ch) {
    using T = WaveTables<L, PE>;
    constexpr int nsh = (L + 1) * (L + 1);
    const int lane = (int)lane_id();
    constexpr int D = 1 + 3 * nsh;
    OwnerLane o;
    o.also_last = false;
    o.row_off = lane < D ? (uint32_t)lane : lane >= 60 ? (uint32_t)(D + lane - 60) : 0u;
    o.row_active = lane < D || (lane >= 60 && lane < 63) || (lane == 63 && PE);
    if (lane < 3 * nsh) {
        o.y_base = (lane / 3) * kPitch;
        o.g_base = T::kRec + (lane % 3) * kPitch;
        o.also_last = lane == last_ch;
    } else {
        o.y_base = T::kOnes;
        if (lane == last_ch) {
            o.g_base = T::kRec + 3 * kPitch;
        } else if (lane >= 60 && lane < 63) {
            o.g_base = T::kRec + (4 + (lane - 60)) * kPitch;
        } else if (lane == 63 && PE) {
            o.g_base = T::kRec + 7 * kPitch;
        } else {
            o.g_base = T::kRec; // read, summed, never written (row_active is false)
        }
    }
    o.g_slot = T::kSlot;
    return o;
}

// Sum over the members in `mm` (entries in slot `slot`) of
// buf[y_base + m] * buf[g_base + slot * g_slot + m] (+ the last channel on
// the also_last lane), two members at a time.
template <bool ALSO_LAST>
__device__ __forceinline__ float sum_members(uint64_t mm, const float *__restrict__ buf,
                                             const OwnerLane &ow, int slot, const float *last) {
    const float *yb = buf + ow.y_base;
    const float *gb = buf + ow.g_base + slot * ow.g_slot;
    float acc = 0.0f;
    while (mm) {
        uint32_t m[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) m[u] = pop_member(mm);
        float y[2], g[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            y[u] = yb[m[u]];
            g[u] = gb[m[u]];
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) acc = acc + y[u] * g[u];
        if constexpr (ALSO_LAST) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                if (ow.also_last) acc = acc + last[m[u]];
            }
        }
    }
    return acc;
}

// A lane's steps between grouping passes.  Entry n (the lane's n-th step)
// sits in slot n % kWindow; it is complete once the position gradient that
// the lane's next step flushes for the same cell is attached
// (src/tracing/pipeline.cu:495-506 flushes a cell's position gradient one
// step late), or once the walk has ended.  A lane holds at most kWindow
// unapplied entries: up to kWindow - 1 complete ones and one pending.
struct StepEntries {
    uint32_t key[kWindow]; // cell of the complete entry in slot s
    uint32_t ready;        // bit s: slot s holds a complete entry not yet applied
    uint32_t flushed;      // bit s: that entry carries a flushed position gradient
    uint32_t next_slot;    // slot of the next entry published (entries go round)
    uint32_t pend_slot;    // slot of the pending entry
    uint32_t pend_cell;    // its cell
    bool pend;             // an entry waits for its position flush
};

__device__ __forceinline__ void entries_init(StepEntries &e) {
#pragma unroll
    for (int s = 0; s < kWindow; ++s) e.key[s] = 0u;
    e.ready = 0u;
    e.flushed = 0u;
    e.next_slot = 0u;
    e.pend_slot = 0u;
    e.pend_cell = 0u;
    e.pend = false;
}

// Attaches the flushed position gradient (flush) or zeros to the pending
// entry and marks it complete.
template <int L, bool PE>
__device__ __forceinline__ void complete_entry(StepEntries &e, bool flush, const float *flush_g,
                                               WaveTables<L, PE> &tb) {
    float *r = tb.rec() + e.pend_slot * WaveTables<L, PE>::kSlot + lane_id();
    r[4 * kPitch] = flush ? flush_g[0] : 0.0f;
    r[5 * kPitch] = flush ? flush_g[1] : 0.0f;
    r[6 * kPitch] = flush ? flush_g[2] : 0.0f;
#pragma unroll
    for (int s = 0; s < kWindow; ++s) {
        if (e.pend_slot == (uint32_t)s) e.key[s] = e.pend_cell;
    }
    e.ready |= 1u << e.pend_slot;
    if (flush) e.flushed |= 1u << e.pend_slot;
    e.pend = false;
}

// Publishes a lane's step (components 0..3, and 7 with PE, of its entry) as
// the pending entry.
template <int L, bool PE>
__device__ __forceinline__ void publish_step(WaveTables<L, PE> &tb, StepEntries &e, uint32_t cell,
                                             float gr, float gg, float gb, float g_last,
                                             float perr) {
    const uint32_t slot = e.next_slot;
    float *r = tb.rec() + slot * WaveTables<L, PE>::kSlot + lane_id();
    r[0] = gr;
    r[kPitch] = gg;
    r[2 * kPitch] = gb;
    r[3 * kPitch] = g_last;
    if constexpr (PE) r[7 * kPitch] = perr;
    e.pend_slot = slot;
    e.pend_cell = cell;
    e.pend = true;
    e.next_slot = slot + 1u == (uint32_t)kWindow ? 0u : slot + 1u;
}

// Grouped gradient updates of the wave's complete entries (all 64 lanes
// active).  For every distinct cell among them, owner lane i < D adds the
// sum of its component over the cell's entries to the cell's attribute row
// (one coalesced atomic instruction per cell), lanes 60..62 add the summed
// flushed position gradient and lane 63 the point error.  The owner lanes
// read the entries two at a time, two LDS reads and one product per entry.
//
// ACC: the sums go to the cell's row of the fp32 accumulator (for either
// attribute type), one row of accum_stride(L) floats per cell: an atomic add
// costs about one memory transaction per 64-byte segment it touches, and the
// row spans ceil((D + 4) / 16) of them where the three output arrays span up
// to ceil(D / 16) + 3.  The position lanes add their sums whether or not an
// entry flushed a position (then they add zeros, which leave a row as it is
// for the finalize pass: it skips zero elements), and `row` is this lane's
// element of cell 0's row, so a group costs one address add.
// !ACC: straight into attr_grad, points_grad (only when an entry of the
// group flushed a position) and point_error.
// ALSO_LAST: the last channel is an SH component too (sdf_channel < 3 nsh).
template <int L, bool PE, typename AT, bool ACC, bool ALSO_LAST>
__device__ __forceinline__ void grouped_pass_impl(StepEntries &e, const OwnerLane &ow,
                                                  WaveTables<L, PE> &tb, void *__restrict__ attr_grad,
                                                  void *__restrict__ point_error,
                                                  float *__restrict__ points_grad,
                                                  float *__restrict__ row) {
    constexpr int D = 1 + 3 * (L + 1) * (L + 1);
    const uint32_t lane = lane_id();
    const float *last = tb.rec() + 3 * kPitch;
    uint64_t todo[kWindow], flushing[kWindow];
#pragma unroll
    for (int s = 0; s < kWindow; ++s) {
        todo[s] = __ballot((e.ready >> s) & 1u);
        flushing[s] = ACC ? 0ull : __ballot((e.flushed >> s) & 1u);
    }
    while (true) {
        // leader: the first entry left, in slot order (selects, no branches)
        uint64_t lead = todo[kWindow - 1];
        uint32_t lead_key = e.key[kWindow - 1];
#pragma unroll
        for (int s = kWindow - 2; s >= 0; --s) {
            lead_key = todo[s] ? e.key[s] : lead_key;
            lead = todo[s] ? todo[s] : lead;
        }
        if (!lead) break;
        const uint32_t c = readlane_u(lead_key, first_lane(lead));
        // every ready entry of cell c is still in todo[s]
        uint64_t grp[kWindow];
        uint64_t flush_any = 0ull;
#pragma unroll
        for (int s = 0; s < kWindow; ++s) {
            grp[s] = todo[s] & lane_mask(e.key[s] == c);
            todo[s] &= ~grp[s];
            if constexpr (!ACC) flush_any |= grp[s] & flushing[s];
        }
        // an empty group half sums to +0 in no iterations, as the product
        // sums of the nonempty ones are added to 0 in slot order
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < kWindow; ++s) {
            const float *ls = last + s * WaveTables<L, PE>::kSlot;
            acc = acc + sum_members<ALSO_LAST>(grp[s], tb.buf, ow, s, ls);
        }
        if constexpr (ACC) {
            if (ow.row_active) atomicAdd(row + (uint64_t)c * accum_stride(L), acc);
        } else {
            const bool pos = flush_any != 0ull;
            if constexpr (sizeof(AT) == 4) {
                // one atomic instruction: the row, the position and the point error
                float *dst = nullptr;
                if (lane < (uint32_t)D) {
                    dst = static_cast<float *>(attr_grad) + (uint64_t)c * D + lane;
                } else if (lane >= 60u && lane < 63u) {
                    if (pos) dst = points_grad + 3ull * c + (lane - 60u);
                } else if (PE && lane == 63u) {
                    dst = static_cast<float *>(point_error) + c;
                }
                if (dst) atomicAdd(dst, acc);
            } else {
                atomic_add_row<AT>(attr_grad, c, lane, (uint32_t)D, acc);
                if (PE && lane == 63u) atomic_add_elem<AT>(point_error, c, acc);
                if (pos && lane >= 60u && lane < 63u)
                    atomicAdd(points_grad + 3ull * c + (lane - 60u), acc);
            }
        }
    }
    e.ready = 0u;
    e.flushed = 0u;
}

// Where a wave's grouped passes send their sums (decided once per kernel).
struct PassTarget {
    void *attr_grad;
    void *point_error;
    float *points_grad;
    float *row;         // accumulator: this lane's element of cell 0's row, or nullptr
    bool also_last;     // some owner lane adds the last channel to an SH component
};

template <int L, bool PE, typename AT>
__device__ __forceinline__ void grouped_pass(StepEntries &e, const OwnerLane &ow,
                                             WaveTables<L, PE> &tb, const PassTarget &t) {
    __builtin_amdgcn_wave_barrier();
    if (t.row) {
        if (t.also_last)
            grouped_pass_impl<L, PE, AT, true, true>(e, ow, tb, t.attr_grad, t.point_error,
                                                     t.points_grad, t.row);
        else
            grouped_pass_impl<L, PE, AT, true, false>(e, ow, tb, t.attr_grad, t.point_error,
                                                      t.points_grad, t.row);
    } else {
        if (t.also_last)
            grouped_pass_impl<L, PE, AT, false, true>(e, ow, tb, t.attr_grad, t.point_error,
                                                      t.points_grad, t.row);
        else
            grouped_pass_impl<L, PE, AT, false, false>(e, ow, tb, t.attr_grad, t.point_error,
                                                       t.points_grad, t.row);
    }
    __builtin_amdgcn_wave_barrier();
}

template <int L>
__device__ __forceinline__ PassTarget pass_target(const BwdArgs &a, const OwnerLane &ow) {
    PassTarget t;
    t.attr_grad = a.attr_grad;
    t.point_error = a.point_error;
    t.points_grad = a.points_grad;
    t.row = a.accum ? a.accum + ow.row_off : nullptr;
    t.also_last = __ballot(ow.also_last) != 0ull;
    return t;
}

template <int L, bool PE>
__device__ __forceinline__ void tables_init(WaveTables<L, PE> &tb, const float *sh) {
    using T = WaveTables<L, PE>;
    constexpr int nsh = (L + 1) * (L + 1);
    static_assert(T::kComp * kWindow <= 64, "one lane per padding row");
    const uint32_t lane = lane_id();
#pragma unroll
    for (int k = 0; k < nsh; ++k) tb.y()[k * kPitch + lane] = sh[k];
    // the padding member (lane 64): zero basis and zero record
    if (lane < (uint32_t)nsh) tb.y()[lane * kPitch + 64] = 0.0f;
    if (lane < (uint32_t)(T::kComp * kWindow)) tb.rec()[lane * kPitch + 64] = 0.0f;
    tb.buf[T::kOnes + lane] = 1.0f;
    if (lane == 0) tb.buf[T::kOnes + 64] = 1.0f;
    __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------------------
// backward_sdf (src/tracing/pipeline.cu:267-550)

template <int L, bool STATS, typename AT, bool PE = false>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4, 8))) void
backward_sdf_kernel(BwdArgs a) {
    constexpr int nsh = (L + 1) * (L + 1);
    constexpr int D = 1 + 3 * nsh;
    __shared__ WaveTables<L, PE> tables[kBlock / 64];
    bool valid;
    const uint32_t ray_idx =
        ray_for_lane<kBackwardChunk>(a.num_rays, a.settings.ray_image_width, a.num_tiles, valid,
                                     a.order);
    const uint32_t lane = lane_id();
    WaveTables<L, PE> &tb = tables[threadIdx.x >> 6];

    RayF ray = {};
    if (valid) ray = load_ray(a.rays, ray_idx);
    {
        float sh0[nsh];
        sh_basis<L>(ray.dx, ray.dy, ray.dz, sh0);
        tables_init<L, PE>(tb, sh0);
    }
    const float *sh = tb.y() + lane; // this ray's SH basis, in LDS (stride kPitch)

    const float sha = a.sharpness[0];
    const int32_t sdf_ch = a.settings.sdf_channel >= 0 ? a.settings.sdf_channel : D - 1;
    const bool write_sdf = a.settings.sdf_channel >= 0;
    const OwnerLane owner = owner_lane<L, PE>(write_sdf ? sdf_ch : -1);
    const PassTarget target = pass_target<L>(a, owner);
    const float thr = a.settings.weight_threshold;
    const uint32_t Q = a.num_quantiles;
    const float *rq = (valid && a.quantiles) ? a.quantiles + (uint64_t)ray_idx * Q : nullptr;
    const float *rdg = (valid && a.depth_grad) ? a.depth_grad + (uint64_t)ray_idx * Q : nullptr;
    // the statistics instantiation gets no rgba / gradient buffers
    float4 g4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 c4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (!STATS && valid) {
        g4 = load_attr4<AT>(a.rgba_grad, ray_idx);
        c4 = load_attr4<AT>(a.rgba, ray_idx);
    }
    const float err =
        (valid && a.ray_error) ? (float)static_cast<const AT *>(a.ray_error)[ray_idx] : 0.0f;

    float T = 1.0f;
    float C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
    uint32_t qi = 0;
    float q = (rq && Q > 0) ? rq[0] : 0.0f;
    float g_logT = 0.0f;
    float sharp_acc = 0.0f;
    GeomState gs;
    geom_init(gs);
    uint64_t hash = kFnvOffset;
    uint32_t rec = 0;

    WalkState ws;
    walk_init(a.scene, valid ? a.start[ray_idx] : kNoIndex, ws);
    WalkCounters wc = {0u, 0u, 0ull, 0ull};
    // replay of the forward's walk record: while this lane's entries are
    // recorded, the step is read instead of scanned; from the first
    // unrecorded (or out-of-range) entry on, the lane scans.  wslot: this
    // lane's entry in the first row of the trip's chunk (~0: no chunk).
    const uint32_t *wtab = nullptr;
    uint64_t wslot = ~0ull;
    bool replaying = false;
    if (!STATS && a.record.entries) {
        wtab = walk_record_table<kBackwardChunk>(a.record);
        replaying = true;
    }
    uint32_t trip = 0;
    StepEntries ents; // steps whose updates are not applied yet
    entries_init(ents);

    while (__ballot(ws.alive) != 0ull) {
        StepInfo si;
        si.stepped = false;
        si.found = false;
        // the recorded step's {r, g, b, channel}, valid when `replayed`
        float4 rc4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        bool replayed = false;
        if (wtab && trip < a.record.budget && trip % kChunkTrips == 0) {
            const uint32_t c = wtab[trip / kChunkTrips];
            wslot = c == kNoIndex ? ~0ull : (uint64_t)c * kChunkEntries + lane;
        }
        if (ws.alive) {
            uint2 e = make_uint2(kWalkUnrecorded, 0u);
            if (replaying && trip < a.record.budget && wslot != ~0ull) {
                const uint64_t i = wslot + (trip % kChunkTrips) * 64u;
                e = record_load(a.record.entries + i);
                rc4 = record_load(a.record.colors + i);
            }
            if (e.x == kNoIndex) {
                ++ws.n;
                ws.alive = false;
            } else if (e.x < a.scene.num_points) {
                ++ws.n;
                si.found = true;
                si.next = e.x;
                si.t1 = __builtin_bit_cast(float, e.y);
                si.xn[0] = a.scene.points[3ull * e.x];
                si.xn[1] = a.scene.points[3ull * e.x + 1];
                si.xn[2] = a.scene.points[3ull * e.x + 2];
                si.stepped = si.t1 > ws.t0;
                replayed = true;
            } else {
                replaying = false;
                walk_advance<true, STATS>(a.scene, ray, a.settings.max_intersections, ws, si, wc);
            }
        }
        ++trip;

        bool keep = true;
        float dr = 0.0f, dg = 0.0f, db = 0.0f, dsdf = 0.0f, pe = 0.0f;
        bool flush = false;
        uint32_t flush_idx = kNoIndex;
        float flush_g[3] = {0.0f, 0.0f, 0.0f};
        if (si.stepped) {
            const uint32_t cell = ws.cell;
            const float t0 = ws.t0, t1 = si.t1;
            if constexpr (STATS) {
                hash = fnv_step(hash, cell);
                if (a.cells && rec < a.cells_stride) a.cells[(uint64_t)ray_idx * a.cells_stride + rec] = cell;
                ++rec;
            }
            const AT *__restrict__ row = static_cast<const AT *>(a.scene.attrs) + (uint64_t)cell * D;
            const float dt = fmaxf(t1 - t0, 0.0f);
            const float d = replayed ? rc4.w : (float)row[sdf_ch];
            const float phi = sdf_sigmoidf(-sha * d);
            const float s = sha * phi * (1.0f - phi);
            const float alpha = 1.0f - sdf_expf(-s * dt);
            const float Tn = T * (1.0f - alpha);
            if constexpr (!STATS) {
                float r, g, b;
                if (replayed) {
                    r = rc4.x;
                    g = rc4.y;
                    b = rc4.z;
                } else {
                    sh_rgb<L>(sh, kPitch, row, r, g, b);
                }
                const float w = T * alpha;
                C0 = fmaf(w, r, C0);
                C1 = fmaf(w, g, C1);
                C2 = fmaf(w, b, C2);
                pe = w * err;
                dr = g4.x * w;
                dg = g4.y * w;
                db = g4.z * w;
                const float den = T * (1.0f - alpha) + 1e-6f;
                const float rest0 = (c4.x - C0) / den;
                const float rest1 = (c4.y - C1) / den;
                const float rest2 = (c4.z - C2) / den;
                float dL_dalpha = T * sdf_dot3(r - rest0, g - rest1, b - rest2, g4.x, g4.y, g4.z);
                dL_dalpha = dL_dalpha + (1.0f - c4.w) * g4.w / (1.0f - alpha + 1e-6f);
                dL_dalpha = dL_dalpha + -g_logT / fmaxf(1.0f - alpha, 1e-12f);
                const float oma = 1.0f - alpha;
                const float dL_ds = dL_dalpha * (dt * oma);
                float dL_ddelta = dL_dalpha * (s * oma);
                float units = 0.0f;
                if (rq && Q > 0) {
                    const float T0 = T;
                    const float drop = T0 - Tn;
                    if (drop > 1e-12f) {
                        while (qi < Q && Tn < q) {
                            const float gq = rdg[qi];
                            float frac = (T0 - q) / drop;
                            frac = fminf(1.0f, fmaxf(0.0f, frac));
                            units = units + gq;
                            dL_ddelta = fmaf(gq, frac, dL_ddelta);
                            if (alpha > 1e-12f && T0 > 1e-20f) {
                                g_logT = fmaf(gq, dt * q / (alpha * T0), g_logT);
                            }
                            ++qi;
                            if (qi < Q) q = rq[qi];
                        }
                    }
                }
                flush = geom_step(gs, cell, ws.xc, si.next, si.xn, units - dL_ddelta, dL_ddelta, ray,
                                  flush_idx, flush_g);
                const float dphi_dd = -sha * phi * (1.0f - phi);
                const float ds_dd = sha * (1.0f - 2.0f * phi) * dphi_dd;
                const float ds_dsha = phi * (1.0f - phi) * (1.0f - sha * d * (1.0f - 2.0f * phi));
                dsdf = dL_ds * ds_dd;
                sharp_acc += dL_ds * ds_dsha;
                if (r == 0.0f) dr = 0.0f;
                if (g == 0.0f) dg = 0.0f;
                if (b == 0.0f) db = 0.0f;
            }
            T = Tn;
            keep = T > thr;
        }
        if (si.stepped && !keep) ws.alive = false;
        if constexpr (!STATS) {
            // the pending step is complete when the lane steps again (with
            // the flush of the same cell) or when its walk ends; complete
            // steps go out every kWindow trips
            if (ents.pend && (si.stepped || !ws.alive))
                complete_entry<L, PE>(ents, si.stepped && flush, flush_g, tb);
            if (trip % kWindow == 0) grouped_pass<L, PE, AT>(ents, owner, tb, target);
            if (si.stepped) publish_step<L, PE>(tb, ents, ws.cell, dr, dg, db, dsdf, pe);
        }
        if (ws.alive && si.found) walk_move(ws, si);
    }
    if constexpr (!STATS) {
        // steps not applied when the walks ended
        const float zero3[3] = {0.0f, 0.0f, 0.0f};
        if (ents.pend) complete_entry<L, PE>(ents, false, zero3, tb);
        grouped_pass<L, PE, AT>(ents, owner, tb, target);
    }

    if constexpr (STATS) {
        if (valid) {
            if (a.visit_hash) a.visit_hash[ray_idx] = hash;
            if (a.steps) a.steps[ray_idx] = wc.steps;
            if (a.faces) a.faces[ray_idx] = wc.faces;
            if (a.faces_stepped) a.faces_stepped[ray_idx] = wc.faces_stepped;
        }
    } else {
        if (a.sharpness_grad) {
            const float v = wave_sum(sharp_acc);
            if (lane == 0 && v != 0.0f) atomicAdd(a.sharpness_grad, v);
        }
    }
}

// backward, density mode (src/tracing/pipeline.cu:553-791); the walk runs in
// the reference's unsafe mode (no t > t0 test, :782-790).
template <int L, bool STATS, typename AT, bool PE = false>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4, 8))) void
backward_density_kernel(BwdArgs a) {
    constexpr int nsh = (L + 1) * (L + 1);
    constexpr int D = 1 + 3 * nsh;
    __shared__ WaveTables<L, PE> tables[kBlock / 64];
    bool valid;
    const uint32_t ray_idx =
        ray_for_lane<kBackwardChunk>(a.num_rays, a.settings.ray_image_width, a.num_tiles, valid,
                                     a.order);
    const uint32_t lane = lane_id();
    WaveTables<L, PE> &tb = tables[threadIdx.x >> 6];

    RayF ray = {};
    if (valid) ray = load_ray(a.rays, ray_idx);
    {
        float sh0[nsh];
        sh_basis<L>(ray.dx, ray.dy, ray.dz, sh0);
        tables_init<L, PE>(tb, sh0);
    }
    const float *sh = tb.y() + lane; // this ray's SH basis, in LDS (stride kPitch)

    const OwnerLane owner = owner_lane<L, PE>(D - 1);
    const PassTarget target = pass_target<L>(a, owner);
    const float thr = a.settings.weight_threshold;
    const uint32_t Q = a.num_quantiles;
    const float *rq = (valid && a.quantiles) ? a.quantiles + (uint64_t)ray_idx * Q : nullptr;
    const float *rdg = (valid && a.depth_grad) ? a.depth_grad + (uint64_t)ray_idx * Q : nullptr;
    float4 g4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 c4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float cur_dg = 0.0f; // src/tracing/pipeline.cu:620-629
    if (!STATS && valid) {
        g4 = load_attr4<AT>(a.rgba_grad, ray_idx);
        c4 = load_attr4<AT>(a.rgba, ray_idx);
        for (uint32_t k = 0; k < Q; ++k) {
            const uint32_t pi = a.depth_indices[(uint64_t)ray_idx * Q + k];
            if (pi != kNoIndex && pi < a.scene.num_points) {
                cur_dg = cur_dg +
                         rdg[k] / (float)static_cast<const AT *>(a.scene.attrs)[(uint64_t)pi * D + D - 1];
            }
        }
    }
    const float err =
        (valid && a.ray_error) ? (float)static_cast<const AT *>(a.ray_error)[ray_idx] : 0.0f;

    float T = 1.0f;
    float C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
    uint32_t qi = 0;
    float q = (rq && Q > 0) ? rq[0] : 0.0f;
    GeomState gs;
    geom_init(gs);
    uint64_t hash = kFnvOffset;
    uint32_t rec = 0;

    WalkState ws;
    walk_init(a.scene, valid ? a.start[ray_idx] : kNoIndex, ws);
    WalkCounters wc = {0u, 0u, 0ull, 0ull};
    StepEntries ents;
    entries_init(ents);
    // replay of the forward's walk record as in backward_sdf; the forward
    // records a step only where the unsafe walk takes the same exit
    const uint32_t *wtab = nullptr;
    bool replaying = false;
    if (!STATS && a.record.entries) {
        wtab = walk_record_table<kBackwardChunk>(a.record);
        replaying = true;
    }
    uint32_t trip = 0;
    // ridx: the forward trip whose entry the lane reads next.  After an entry
    // marked kWalkDiffers the lane scans (`seeking`) until its walk stands
    // where the forward stood after one of that entry's first kSeekWindow
    // steps, then replays from the step after it.  From equal (cell, t0) the
    // two walks take the same steps wherever the forward recorded agreement,
    // so the replayed walk is the unsafe one; the step limit counts the
    // lane's own steps.
    uint32_t ridx = 0;
    bool seeking = false;

    while (__ballot(ws.alive) != 0ull) {
        StepInfo si;
        si.stepped = false;
        si.found = false;
        // the recorded step's {r, g, b, channel}, valid when `replayed`
        float4 rc4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        bool replayed = false;
        if (ws.alive) {
            uint2 e = make_uint2(kWalkUnrecorded, 0u);
            if (replaying && !seeking && ridx < a.record.budget) {
                const uint64_t i = record_slot(a.record, wtab, ridx, lane);
                if (i != ~0ull) {
                    e = record_load(a.record.entries + i);
                    rc4 = record_load(a.record.colors + i);
                }
                ++ridx;
            }
            if (e.x == kNoIndex) {
                ++ws.n;
                ws.alive = false;
            } else if (e.x < a.scene.num_points) {
                ++ws.n;
                if (ws.n > a.settings.max_intersections) {
                    ws.alive = false; // the step limit, as walk_advance applies it
                } else {
                    si.found = true;
                    si.next = e.x;
                    si.t1 = __builtin_bit_cast(float, e.y);
                    si.xn[0] = a.scene.points[3ull * e.x];
                    si.xn[1] = a.scene.points[3ull * e.x + 1];
                    si.xn[2] = a.scene.points[3ull * e.x + 2];
                    si.stepped = si.t1 > ws.t0;
                    replayed = true;
                }
            } else {
                if (e.x != kWalkUnrecorded && (e.x & ~kWalkDiffers) < a.scene.num_points) {
                    seeking = true; // entry ridx - 1: the forward's differing step
                } else if (!seeking) {
                    replaying = false;
                }
                walk_advance<false, STATS>(a.scene, ray, a.settings.max_intersections, ws, si,
                                           wc);
            }
        }
        ++trip;

        bool keep = true;
        float dr = 0.0f, dg = 0.0f, db = 0.0f, dds = 0.0f, pe = 0.0f;
        bool flush = false;
        uint32_t flush_idx = kNoIndex;
        float flush_g[3] = {0.0f, 0.0f, 0.0f};
        if (si.stepped) {
            const uint32_t cell = ws.cell;
            const float t0 = ws.t0, t1 = si.t1;
            if constexpr (STATS) {
                hash = fnv_step(hash, cell);
                if (a.cells && rec < a.cells_stride) a.cells[(uint64_t)ray_idx * a.cells_stride + rec] = cell;
                ++rec;
            }
            const AT *__restrict__ row = static_cast<const AT *>(a.scene.attrs) + (uint64_t)cell * D;
            const float s = replayed ? rc4.w : (float)row[D - 1];
            const float dt = fmaxf(t1 - t0, 0.0f);
            const float alpha = 1.0f - sdf_expf(-s * dt);
            const float Tn = T * (1.0f - alpha);
            if constexpr (!STATS) {
                float r, g, b;
                if (replayed) {
                    // the forward's colour (zero where it found no density)
                    r = rc4.x;
                    g = rc4.y;
                    b = rc4.z;
                } else if (s > 1e-6f) {
                    sh_rgb<L>(sh, kPitch, row, r, g, b);
                } else {
                    r = g = b = 0.0f;
                }
                const float w = T * alpha;
                const float dalpha_ds = dt * (1.0f - alpha);
                float dalpha_ddt = 0.0f;
                if (dt > 0.0f) dalpha_ddt = s * (1.0f - alpha);
                C0 = fmaf(w, r, C0);
                C1 = fmaf(w, g, C1);
                C2 = fmaf(w, b, C2);
                pe = w * err;
                dr = g4.x * w;
                dg = g4.y * w;
                db = g4.z * w;
                const float den = T * (1.0f - alpha + 1e-6f);
                const float rest0 = (c4.x - C0) / den;
                const float rest1 = (c4.y - C1) / den;
                const float rest2 = (c4.z - C2) / den;
                float dL_dalpha = T * sdf_dot3(r - rest0, g - rest1, b - rest2, g4.x, g4.y, g4.z);
                dL_dalpha = dL_dalpha + (1.0f - c4.w) * g4.w / (1.0f - alpha + 1e-6f);
                float dL_ds = dL_dalpha * dalpha_ds;
                float dL_ddt = dL_dalpha * dalpha_ddt;
                float dL_dt0 = 0.0f;
                while (qi < Q && Tn < q) {
                    const float dgi = rdg[qi] / s;
                    dL_dt0 = dL_dt0 + dgi;
                    dL_ds = dL_ds + -dgi * logf(T / q) / s;
                    cur_dg = cur_dg - dgi;
                    ++qi;
                    if (qi < Q) q = rq[qi];
                }
                if (qi < Q) {
                    dL_ds = fmaf(-dt, cur_dg, dL_ds);
                    dL_ddt = fmaf(-s, cur_dg, dL_ddt);
                }
                dL_dt0 = dL_dt0 + -dL_ddt;
                flush = geom_step(gs, cell, ws.xc, si.next, si.xn, dL_dt0, dL_ddt, ray, flush_idx,
                                  flush_g);
                dds = dL_ds;
                if (r == 0.0f) dr = 0.0f;
                if (g == 0.0f) dg = 0.0f;
                if (b == 0.0f) db = 0.0f;
            }
            T = Tn;
            keep = T > thr;
        }
        if (si.stepped && !keep) ws.alive = false;
        if constexpr (!STATS) {
            if (ents.pend && (si.stepped || !ws.alive))
                complete_entry<L, PE>(ents, si.stepped && flush, flush_g, tb);
            if (trip % kWindow == 0) grouped_pass<L, PE, AT>(ents, owner, tb, target);
            if (si.stepped) publish_step<L, PE>(tb, ents, ws.cell, dr, dg, db, dds, pe);
        }
        if (ws.alive && si.found) walk_move(ws, si);
        if (seeking && ws.alive) {
            // the forward's states after its steps ridx - 1, ridx, ...: back on
            // its path where one equals this lane's (cell, t0)
#pragma unroll
            for (uint32_t k = 0; k < kSeekWindow; ++k) {
                const uint32_t f = ridx - 1u + k;
                if (f >= a.record.budget) break;
                const uint64_t i = record_slot(a.record, wtab, f, lane);
                if (i == ~0ull) break;
                const uint2 fe = record_load(a.record.entries + i);
                if (fe.x == kNoIndex || fe.x == kWalkUnrecorded) break;
                if ((fe.x & ~kWalkDiffers) == ws.cell &&
                    fe.y == __builtin_bit_cast(uint32_t, ws.t0)) {
                    seeking = false;
                    ridx = f + 1u;
                    break;
                }
            }
        }
    }
    if constexpr (!STATS) {
        const float zero3[3] = {0.0f, 0.0f, 0.0f};
        if (ents.pend) complete_entry<L, PE>(ents, false, zero3, tb);
        grouped_pass<L, PE, AT>(ents, owner, tb, target);
    }

    if constexpr (STATS) {
        if (valid) {
            if (a.visit_hash) a.visit_hash[ray_idx] = hash;
            if (a.steps) a.steps[ray_idx] = wc.steps;
            if (a.faces) a.faces[ray_idx] = wc.faces;
            if (a.faces_stepped) a.faces_stepped[ray_idx] = wc.faces_stepped;
        }
    }
}

// ---------------------------------------------------------------------------
// launchers

static inline dim3 grid_for(uint64_t n) { return dim3((unsigned)((n + kBlock - 1) / kBlock)); }


template <int L, typename AT>
static hipError_t launch_forward_L(const FwdArgs &a, bool neus, bool stats, hipStream_t stream) {
    const dim3 grid(grid_blocks_for_tiles(a.num_tiles));
    const bool ct = a.scene.cells != nullptr;
    // rays in an explicit order are an incoherent batch: half-batch face loads
    const bool half = a.order != nullptr;
    if (neus) {
        if (stats) {
            hipLaunchKernelGGL((forward_kernel<L, true, true, AT>), grid, dim3(kBlock), 0, stream, a);
        } else if (ct && half) {
            hipLaunchKernelGGL((forward_kernel<L, true, false, AT, true, true>), grid, dim3(kBlock),
                               0, stream, a);
        } else if (ct) {
            hipLaunchKernelGGL((forward_kernel<L, true, false, AT, true>), grid, dim3(kBlock), 0,
                               stream, a);
        } else {
            hipLaunchKernelGGL((forward_kernel<L, true, false, AT>), grid, dim3(kBlock), 0, stream, a);
        }
    } else {
        if (stats) {
            hipLaunchKernelGGL((forward_kernel<L, false, true, AT>), grid, dim3(kBlock), 0, stream, a);
        } else if (ct && half) {
            hipLaunchKernelGGL((forward_kernel<L, false, false, AT, true, true>), grid,
                               dim3(kBlock), 0, stream, a);
        } else if (ct) {
            hipLaunchKernelGGL((forward_kernel<L, false, false, AT, true>), grid, dim3(kBlock), 0,
                               stream, a);
        } else {
            hipLaunchKernelGGL((forward_kernel<L, false, false, AT>), grid, dim3(kBlock), 0, stream, a);
        }
    }
    return hipGetLastError();
}

__global__ __launch_bounds__(kBlock) void record_reset_kernel(WalkRecordArgs r,
                                                              uint64_t table_words) {
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < table_words;
         i += (uint64_t)gridDim.x * kBlock)
        r.chunks[i] = kNoIndex;
    if (blockIdx.x == 0 && threadIdx.x < kXcds) r.counters[64u * threadIdx.x] = 0u;
}

hipError_t launch_record_reset(const WalkRecordArgs &r, uint64_t table_words, hipStream_t stream) {
    const uint32_t blocks =
        (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>((table_words + kBlock - 1) / kBlock, 4096));
    hipLaunchKernelGGL(record_reset_kernel, dim3(blocks), dim3(kBlock), 0, stream, r, table_words);
    return hipGetLastError();
}

// The forward's scene preparation in one pass: the fp16 offset table (the
// values prefetch_diff_kernel writes) and the cell table (layout at
// cell_record_bytes).  One wavefront per 64 consecutive cells: their CSR rows
// are one contiguous run of entries, so the row of an entry is found among
// the 64 row starts the wavefront holds (six cross-lane reads) instead of by a
// search of the whole offsets array.  The first wavefront also takes entries
// before offs[0], the last one those from offs[N] up to num_adj and the
// table's zero padding, as prefetch_diff_kernel does.  Record words past the
// attribute row are left unwritten (nothing reads them).  The offset table
// built with the cell table carries each entry's neighbour in its fourth
// half (`neighbour_delta`), so the walk over the cell table reads the exit
// face's neighbour from the entry it already holds.  CELLS = false: the
// offset table alone, as prefetch_adjacent_diff gives it (fourth half 0).
template <int L, typename AT, bool CELLS = true>
__global__ __launch_bounds__(kBlock) void scene_prep_kernel(const SceneView sc, uint32_t *cells,
                                                            uint2 *diff) {
    constexpr uint32_t D = 1 + 3 * (L + 1) * (L + 1);
    constexpr uint32_t RW = cell_record_bytes(L, sizeof(AT)) / 4;
    constexpr uint32_t A = kCellAttrByte / 4;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c0 = (blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6)) * 64u;
    if (c0 >= sc.num_points) return; // the whole wavefront
    const uint32_t n = min(64u, sc.num_points - c0);
    const bool last = c0 + n == sc.num_points;
    // lanes past the last cell hold a row start no entry reaches
    uint32_t beg = 0xffffffffu, end = 0u;
    float x = 0.0f, y = 0.0f, z = 0.0f;
    if (lane < n) {
        const uint32_t c = c0 + lane;
        beg = sc.offs[c];
        end = sc.offs[c + 1];
        x = sc.points[3ull * c];
        y = sc.points[3ull * c + 1];
        z = sc.points[3ull * c + 2];
        if constexpr (CELLS) {
            uint32_t *r = cells + (uint64_t)c * RW;
            *reinterpret_cast<uint4 *>(r) = make_uint4(__builtin_bit_cast(uint32_t, x),
                                                       __builtin_bit_cast(uint32_t, y),
                                                       __builtin_bit_cast(uint32_t, z), beg);
            r[4] = end;
        }
    }
    // attribute rows c0 .. c0 + n - 1: contiguous in the caller's array
    if constexpr (!CELLS) {
    } else if constexpr (sizeof(AT) == 4) {
        const uint32_t *src = static_cast<const uint32_t *>(sc.attrs) + (uint64_t)c0 * D;
        for (uint32_t j = lane; j < n * D; j += 64u) {
            const uint32_t cc = j / D;
            cells[(uint64_t)(c0 + cc) * RW + A + (j - cc * D)] = src[j];
        }
    } else {
        const uint16_t *src = static_cast<const uint16_t *>(sc.attrs) + (uint64_t)c0 * D;
        uint16_t *dst = reinterpret_cast<uint16_t *>(cells);
        for (uint32_t j = lane; j < n * D; j += 64u) {
            const uint32_t cc = j / D;
            dst[((uint64_t)(c0 + cc) * RW + A) * 2u + (j - cc * D)] = src[j];
        }
    }
    // the offset table entries of these rows
    const uint32_t first = (uint32_t)__shfl((int)beg, 0);
    const uint32_t e0 = c0 == 0 ? 0u : min(first, sc.num_adj);
    const uint32_t e1 = last ? sc.num_adj : min((uint32_t)__shfl((int)end, (int)n - 1), sc.num_adj);
    for (uint32_t k0 = e0; k0 < e1; k0 += 64u) {
        const uint32_t k = k0 + lane;
        // the last row i < n with beg_i <= k (row 0 if none)
        uint32_t row = 0;
#pragma unroll
        for (uint32_t step = 32; step > 0; step >>= 1) {
            const uint32_t probe = row + step;
            const uint32_t b = (uint32_t)__shfl((int)beg, (int)min(probe, 63u));
            if (probe < n && b <= k) row = probe;
        }
        const float px = __shfl(x, (int)row), py = __shfl(y, (int)row), pz = __shfl(z, (int)row);
        if (k < e1) {
            const uint32_t a = sc.adj[k];
            // with the cell table, the entry's fourth half (0 in the plain
            // table) holds the neighbour relative to the row's cell
            const uint32_t w = CELLS ? neighbour_delta(c0 + row, a) : 0u;
            if (a >= sc.num_points) {
                diff[k] = make_uint2(0x7e007e00u, 0x7e00u | (w << 16)); // NaN plane
            } else {
                const float qx = sc.points[3ull * a], qy = sc.points[3ull * a + 1],
                            qz = sc.points[3ull * a + 2];
                diff[k] = make_uint2(f32_to_f16(qx - px) | (f32_to_f16(qy - py) << 16),
                                     f32_to_f16(qz - pz) | (w << 16));
            }
        }
    }
    if (last && lane < kDiffPad) diff[sc.num_adj + lane] = make_uint2(0u, 0u);
}

hipError_t launch_prefetch_diff(const float *points, uint32_t num_points, uint32_t num_adj,
                                const uint32_t *adj, const uint32_t *offs, uint2 *diff,
                                hipStream_t stream) {
    if (num_points == 0) {
        hipLaunchKernelGGL(prefetch_diff_kernel, grid_for((uint64_t)num_adj + kDiffPad), dim3(kBlock),
                           0, stream, points, num_points, num_adj, adj, offs, diff);
        return hipGetLastError();
    }
    SceneView sc = {};
    sc.points = points;
    sc.adj = adj;
    sc.offs = offs;
    sc.num_points = num_points;
    sc.num_adj = num_adj;
    const uint32_t waves = (num_points + 63u) / 64u;
    hipLaunchKernelGGL((scene_prep_kernel<0, float, false>), dim3((waves + kBlock / 64 - 1) / (kBlock / 64)),
                       dim3(kBlock), 0, stream, sc, nullptr, diff);
    return hipGetLastError();
}

template <typename AT>
static hipError_t launch_scene_prep_T(int L, const SceneView &sc, uint32_t *cells, uint2 *diff,
                                      hipStream_t stream) {
    const uint32_t waves = (sc.num_points + 63u) / 64u;
    const dim3 grid((waves + kBlock / 64 - 1) / (kBlock / 64));
    switch (L) {
    case 0: hipLaunchKernelGGL((scene_prep_kernel<0, AT>), grid, dim3(kBlock), 0, stream, sc, cells, diff); break;
    case 1: hipLaunchKernelGGL((scene_prep_kernel<1, AT>), grid, dim3(kBlock), 0, stream, sc, cells, diff); break;
    case 2: hipLaunchKernelGGL((scene_prep_kernel<2, AT>), grid, dim3(kBlock), 0, stream, sc, cells, diff); break;
    case 3: hipLaunchKernelGGL((scene_prep_kernel<3, AT>), grid, dim3(kBlock), 0, stream, sc, cells, diff); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_scene_prep(int L, bool half, const SceneView &sc, uint32_t *cells, uint2 *diff,
                             hipStream_t stream) {
    if (sc.num_points == 0) return hipSuccess;
    return half ? launch_scene_prep_T<_Float16>(L, sc, cells, diff, stream)
                : launch_scene_prep_T<float>(L, sc, cells, diff, stream);
}

template <typename AT>
static hipError_t launch_forward_T(int L, const FwdArgs &a, bool neus, bool stats,
                                   hipStream_t stream) {
    switch (L) {
    case 0: return launch_forward_L<0, AT>(a, neus, stats, stream);
    case 1: return launch_forward_L<1, AT>(a, neus, stats, stream);
    case 2: return launch_forward_L<2, AT>(a, neus, stats, stream);
    case 3: return launch_forward_L<3, AT>(a, neus, stats, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_forward(int L, const FwdArgs &a, bool neus, bool stats, bool half,
                          hipStream_t stream) {
    return half ? launch_forward_T<_Float16>(L, a, neus, stats, stream)
                : launch_forward_T<float>(L, a, neus, stats, stream);
}

template <int L, typename AT>
static hipError_t launch_backward_L(const BwdArgs &a, bool neus, bool stats, hipStream_t stream) {
    const dim3 grid(grid_blocks_for_tiles(a.num_tiles));
    // PE: entries carry the point error (a larger LDS table per wave)
    const bool pe = !stats && a.point_error != nullptr;
    if (neus) {
        if (stats) {
            hipLaunchKernelGGL((backward_sdf_kernel<L, true, AT>), grid, dim3(kBlock), 0, stream, a);
        } else if (pe) {
            hipLaunchKernelGGL((backward_sdf_kernel<L, false, AT, true>), grid, dim3(kBlock), 0,
                               stream, a);
        } else {
            hipLaunchKernelGGL((backward_sdf_kernel<L, false, AT>), grid, dim3(kBlock), 0, stream, a);
        }
    } else {
        if (stats) {
            hipLaunchKernelGGL((backward_density_kernel<L, true, AT>), grid, dim3(kBlock), 0, stream,
                               a);
        } else if (pe) {
            hipLaunchKernelGGL((backward_density_kernel<L, false, AT, true>), grid, dim3(kBlock), 0,
                               stream, a);
        } else {
            hipLaunchKernelGGL((backward_density_kernel<L, false, AT>), grid, dim3(kBlock), 0,
                               stream, a);
        }
    }
    return hipGetLastError();
}

template <typename AT>
static hipError_t launch_backward_T(int L, const BwdArgs &a, bool neus, bool stats,
                                    hipStream_t stream) {
    switch (L) {
    case 0: return launch_backward_L<0, AT>(a, neus, stats, stream);
    case 1: return launch_backward_L<1, AT>(a, neus, stats, stream);
    case 2: return launch_backward_L<2, AT>(a, neus, stats, stream);
    case 3: return launch_backward_L<3, AT>(a, neus, stats, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_backward(int L, const BwdArgs &a, bool neus, bool stats, bool half,
                           hipStream_t stream) {
    return half ? launch_backward_T<_Float16>(L, a, neus, stats, stream)
                : launch_backward_T<float>(L, a, neus, stats, stream);
}

// ---------------------------------------------------------------------------
// backward gradient accumulator: clear, then add the rows into the outputs

constexpr uint32_t kAccumBlocks = 16384; // grid-stride cap of the two passes

__global__ __launch_bounds__(kBlock) void grad_clear_kernel(float4 *__restrict__ rows,
                                                            uint64_t n4) {
    const uint64_t step = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += step)
        rows[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// One thread per 16 bytes of a row (the row's padding past D + 4 floats
// skipped); an element that is exactly zero (a cell no ray reached) leaves
// its output untouched.  fp16 outputs (attribute gradients, point error) get
// the fp32 sum added and rounded once.
template <int L, typename AT>
__global__ __launch_bounds__(kBlock) void grad_finalize_kernel(
    const float4 *__restrict__ rows, uint32_t num_points, AT *__restrict__ attr_grad,
    float *__restrict__ points_grad, AT *__restrict__ point_error) {
    constexpr uint32_t S4 = accum_stride(L) / 4;
    constexpr uint32_t D = 1 + 3 * (L + 1) * (L + 1);
    constexpr uint32_t Q = (D + 4 + 3) / 4; // quads of a row that hold data
    const uint64_t total = (uint64_t)num_points * S4;
    const uint64_t step = (uint64_t)gridDim.x * kBlock;
    for (uint64_t t = (uint64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += step) {
        const uint32_t q = (uint32_t)(t % S4);
        if (q >= Q) continue;
        const float4 v4 = rows[t];
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        const uint64_t c = t / S4;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) {
            const uint32_t j = 4u * q + k;
            if (v[k] == 0.0f) continue;
            if (j < D) {
                AT &o = attr_grad[c * D + j];
                o = (AT)((float)o + v[k]);
            } else if (j < D + 3) {
                points_grad[c * 3 + (j - D)] += v[k];
            } else if (j == D + 3 && point_error) {
                AT &o = point_error[c];
                o = (AT)((float)o + v[k]);
            }
        }
    }
}

static inline dim3 accum_grid(uint64_t threads) {
    const uint64_t b = (threads + kBlock - 1) / kBlock;
    return dim3((unsigned)(b < kAccumBlocks ? (b ? b : 1) : kAccumBlocks));
}

hipError_t launch_grad_clear(int L, float *accum, uint32_t num_points, hipStream_t stream) {
    if (L < 0 || L > 3) return hipErrorInvalidValue;
    const uint64_t n4 = (uint64_t)num_points * accum_stride(L) / 4;
    hipLaunchKernelGGL(grad_clear_kernel, accum_grid(n4), dim3(kBlock), 0, stream,
                       reinterpret_cast<float4 *>(accum), n4);
    return hipGetLastError();
}

template <typename AT>
static hipError_t launch_grad_finalize_T(int L, const float *accum, uint32_t num_points,
                                        void *attr_grad, float *points_grad, void *point_error,
                                        hipStream_t stream) {
    const dim3 grid = accum_grid((uint64_t)num_points * accum_stride(L) / 4);
    const float4 *rows = reinterpret_cast<const float4 *>(accum);
    AT *ag = static_cast<AT *>(attr_grad);
    AT *pe = static_cast<AT *>(point_error);
    switch (L) {
    case 0:
        hipLaunchKernelGGL((grad_finalize_kernel<0, AT>), grid, dim3(kBlock), 0, stream, rows,
                           num_points, ag, points_grad, pe);
        break;
    case 1:
        hipLaunchKernelGGL((grad_finalize_kernel<1, AT>), grid, dim3(kBlock), 0, stream, rows,
                           num_points, ag, points_grad, pe);
        break;
    case 2:
        hipLaunchKernelGGL((grad_finalize_kernel<2, AT>), grid, dim3(kBlock), 0, stream, rows,
                           num_points, ag, points_grad, pe);
        break;
    case 3:
        hipLaunchKernelGGL((grad_finalize_kernel<3, AT>), grid, dim3(kBlock), 0, stream, rows,
                           num_points, ag, points_grad, pe);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_grad_finalize(int L, const float *accum, uint32_t num_points, void *attr_grad,
                                float *points_grad, void *point_error, bool half,
                                hipStream_t stream) {
    return half ? launch_grad_finalize_T<_Float16>(L, accum, num_points, attr_grad, points_grad,
                                                   point_error, stream)
                : launch_grad_finalize_T<float>(L, accum, num_points, attr_grad, points_grad,
                                                point_error, stream);
}

// ---------------------------------------------------------------------------
// inference render (the reference's `benchmark` kernel,
// src/tracing/pipeline.cu:1067-1199)

// One lane per pixel, 16x16 pixel tiles per block as the traced kernels.  The
// step is the forward's compositing without its per-point outputs; the walk
// reads the caller's unpadded offset table with guarded loads.
template <int L, bool NEUS, typename AT>
__global__ __launch_bounds__(kBlock) void render_kernel(RenderArgs a) {
    constexpr int nsh = (L + 1) * (L + 1);
    constexpr int D = 1 + 3 * nsh;
    __shared__ float sh_all[kBlock * nsh];
    bool valid;
    const uint32_t px = ray_for_lane<kForwardChunk>(a.width * a.height, a.width, a.num_tiles, valid);
    const uint32_t pi = valid ? px % a.width : 0u, pj = valid ? px / a.width : 0u;

    RayF ray = {};
    bool masked = false;
    if (valid) {
        float dir[3];
        sdf_cast_ray(a.forward, a.right, a.up, a.fov, a.focal, a.width, a.height, a.model, pi,
                     pj, dir);
        const float n = sqrtf(sdf_dot3(dir[0], dir[1], dir[2], dir[0], dir[1], dir[2]));
        masked = n < 0.1f;
        ray.ox = a.position[0];
        ray.oy = a.position[1];
        ray.oz = a.position[2];
        if (!masked) {
            // ray.direction /= ray.direction.norm()
            ray.dx = dir[0] / n;
            ray.dy = dir[1] / n;
            ray.dz = dir[2] / n;
        }
    }
    float *sh = sh_all + threadIdx.x; // basis function k at sh[k * kBlock]
    {
        float sh0[nsh];
        sh_basis<L>(ray.dx, ray.dy, ray.dz, sh0);
#pragma unroll
        for (int k = 0; k < nsh; ++k) sh[k * kBlock] = sh0[k];
    }
    const float sha = a.sharpness[0];
    const int32_t sdf_ch = a.settings.sdf_channel;
    const bool neus_alpha = NEUS && sdf_ch >= 0;
    const float thr = a.settings.weight_threshold;

    float T = 1.0f;
    float C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
    WalkState ws;
    walk_init(a.scene, (valid && !masked) ? a.start[0] : kNoIndex, ws);
    WalkCounters wc = {0u, 0u, 0ull, 0ull};

    while (__ballot(ws.alive) != 0ull) {
        StepInfo si;
        si.stepped = false;
        si.found = false;
        if (ws.alive)
            walk_advance<true, false, true>(a.scene, ray, a.settings.max_intersections, ws, si,
                                            wc);
        bool keep = true;
        if (si.stepped) {
            const AT *__restrict__ row = static_cast<const AT *>(a.scene.attrs) + (uint64_t)ws.cell * D;
            float s = (float)row[D - 1];
            const float dt = fmaxf(si.t1 - ws.t0, 0.0f);
            if (neus_alpha) {
                const float d = (float)row[sdf_ch];
                const float phi = sdf_sigmoidf(-sha * d);
                s = sha * phi * (1.0f - phi);
            }
            const float alpha = 1.0f - sdf_expf(-s * dt);
            const float w = T * alpha;
            float r, g, b;
            if (NEUS || (float)row[D - 1] > 1e-6f) {
                sh_rgb<L>(sh, kBlock, row, r, g, b);
            } else {
                r = g = b = 0.0f;
            }
            C0 = fmaf(w, r, C0);
            C1 = fmaf(w, g, C1);
            C2 = fmaf(w, b, C2);
            T = T * (1.0f - alpha);
            keep = T > thr;
        }
        if (si.stepped && !keep) ws.alive = false;
        if (ws.alive && si.found) walk_move(ws, si);
    }

    if (!valid) return;
    const uint64_t out_idx = (uint64_t)(a.height - 1u - pj) * a.width + pi;
    if (masked) {
        a.out[out_idx] = sdf_make_rgba8(a.bg[0], a.bg[1], a.bg[2], 1.0f);
        return;
    }
    float bg0 = a.bg[0], bg1 = a.bg[1], bg2 = a.bg[2];
    if (a.checker_bg) {
        const int is = 2 * (int)((pi / 20u) % 2u) - 1;
        const int js = 2 * (int)((pj / 20u) % 2u) - 1;
        bg0 = bg1 = bg2 = (is * js > 0) ? 0.3f : 0.5f;
    }
    a.out[out_idx] = sdf_make_rgba8(fmaf(T, bg0, C0), fmaf(T, bg1, C1), fmaf(T, bg2, C2), 1.0f);
}

template <int L, typename AT>
static hipError_t launch_render_L(const RenderArgs &a, bool neus, hipStream_t stream) {
    const dim3 grid(grid_blocks_for_tiles(a.num_tiles));
    if (neus) {
        hipLaunchKernelGGL((render_kernel<L, true, AT>), grid, dim3(kBlock), 0, stream, a);
    } else {
        hipLaunchKernelGGL((render_kernel<L, false, AT>), grid, dim3(kBlock), 0, stream, a);
    }
    return hipGetLastError();
}

template <typename AT>
static hipError_t launch_render_T(int L, const RenderArgs &a, bool neus, hipStream_t stream) {
    switch (L) {
    case 0: return launch_render_L<0, AT>(a, neus, stream);
    case 1: return launch_render_L<1, AT>(a, neus, stream);
    case 2: return launch_render_L<2, AT>(a, neus, stream);
    case 3: return launch_render_L<3, AT>(a, neus, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_render(int L, const RenderArgs &a, bool neus, bool half, hipStream_t stream) {
    return half ? launch_render_T<_Float16>(L, a, neus, stream)
                : launch_render_T<float>(L, a, neus, stream);
}

// ---------------------------------------------------------------------------
// fp-math contract on the device (test hook)

__global__ __launch_bounds__(kBlock) void fpmath_kernel(int op, const float *__restrict__ in,
                                                        void *__restrict__ out, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const float x = in[i];
    if (op == 0) {
        static_cast<float *>(out)[i] = sdf_expf(x);
    } else if (op == 1) {
        static_cast<uint16_t *>(out)[i] = (uint16_t)f32_to_f16(x);
    } else {
        static_cast<float *>(out)[i] = sdf_sigmoidf(x);
    }
}

hipError_t launch_fpmath(int op, const float *in, void *out, uint64_t n, hipStream_t stream) {
    hipLaunchKernelGGL(fpmath_kernel, grid_for(n), dim3(kBlock), 0, stream, op, in, out, n);
    return hipGetLastError();
}

} // namespace sdfoam_hip
