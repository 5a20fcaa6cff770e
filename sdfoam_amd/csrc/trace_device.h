// Device-side building blocks of the Voronoi-foam walk for gfx950.
//
// Floating-point contract: this code is compiled with -ffp-contract=off; the
// only fused multiply-adds are the explicit fmaf calls, placed where the
// reference accumulates `a += b * c`, plus the dot of include/sdfoam_fpmath.h.
// exp / sigmoid / fp16 rounding come from that header, so the per-step
// alpha, the transmittance and therefore the visit sequence are bit-identical
// to the host oracle's.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sdfoam_fpmath.h"
#include "../../include/sdfoam_hip.h"

namespace sdfoam_hip {

constexpr uint32_t kNoIndex = 0xffffffffu;
constexpr int kBlock = 256;
// entries past E in the fp16 offset table, so a face batch can over-read
constexpr uint32_t kDiffPad = 32;

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
}

__device__ __forceinline__ uint32_t f32_to_f16(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// ---- attribute types -------------------------------------------------------
// Pipelines trace fp32 or fp16 attributes (CUDATracingPipeline<float | __half,
// L>, src/tracing/pipeline.cu:1482-1502).  Attributes, rgba, its gradient,
// ray error, contribution, attribute gradients and point error have the
// attribute type; arithmetic is fp32 throughout.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

template <typename AT>
__device__ __forceinline__ float4 load_attr4(const void *base, uint64_t i) {
    if constexpr (sizeof(AT) == 4) {
        return reinterpret_cast<const float4 *>(base)[i];
    } else {
        const uint2 raw = reinterpret_cast<const uint2 *>(base)[i];
        return make_float4(f16_to_f32(raw.x), f16_to_f32(raw.x >> 16), f16_to_f32(raw.y),
                           f16_to_f32(raw.y >> 16));
    }
}

template <typename AT>
__device__ __forceinline__ void store_attr4(void *base, uint64_t i, float4 v) {
    if constexpr (sizeof(AT) == 4) {
        reinterpret_cast<float4 *>(base)[i] = v;
    } else {
        reinterpret_cast<uint2 *>(base)[i] =
            make_uint2(f32_to_f16(v.x) | (f32_to_f16(v.y) << 16), f32_to_f16(v.z) | (f32_to_f16(v.w) << 16));
    }
}

// fp16 atomics are packed pairs (global_atomic_pk_add_f16 on the 4-byte word
// holding the element); the other half of the word gets + 0.  Buffers must
// be 4-byte aligned and hold one padding half past an odd element count.
__device__ __forceinline__ void pk_add_f16(_Float16 *word_lo, _Float16 lo, _Float16 hi) {
    half2_t v = {lo, hi};
    __builtin_amdgcn_global_atomic_fadd_v2f16(
        (__attribute__((address_space(1))) half2_t *)word_lo, v);
}

template <typename AT>
__device__ __forceinline__ void atomic_add_elem(void *base, uint64_t i, float v) {
    if constexpr (sizeof(AT) == 4) {
        atomicAdd(reinterpret_cast<float *>(base) + i, v);
    } else {
        _Float16 *p = reinterpret_cast<_Float16 *>(base) + i;
        if ((reinterpret_cast<uintptr_t>(p) & 3u) == 0) {
            pk_add_f16(p, (_Float16)v, (_Float16)0.0f);
        } else {
            pk_add_f16(p - 1, (_Float16)0.0f, (_Float16)v);
        }
    }
}

// Lanes 0..n-1 of the wave add v to elements row[0..n-1] of row `row` of an
// [*, n] buffer.  Called by all 64 lanes (fp16 pairs neighbouring lanes'
// values into one packed atomic).
template <typename AT>
__device__ __forceinline__ void atomic_add_row(void *base, uint64_t row, uint32_t lane,
                                               uint32_t n, float v) {
    if constexpr (sizeof(AT) == 4) {
        if (lane < n) atomicAdd(reinterpret_cast<float *>(base) + row * n + lane, v);
    } else {
        const float vn = __shfl_down(v, 1, 64);
        _Float16 *p = reinterpret_cast<_Float16 *>(base) + row * n + lane;
        if (lane < n) {
            if ((reinterpret_cast<uintptr_t>(p) & 3u) == 0) {
                pk_add_f16(p, (_Float16)v, lane + 1 < n ? (_Float16)vn : (_Float16)0.0f);
            } else if (lane == 0) {
                pk_add_f16(p - 1, (_Float16)0.0f, (_Float16)v);
            }
        }
    }
}

struct RayF {
    float ox, oy, oz;
    float dx, dy, dz;
};

// Work decomposition.  A block is one tile of rays: 16x16 pixels (an 8x8
// tile per wavefront) when the rays are image rows of `width` pixels, else
// 256 consecutive rays.  Blocks are dealt round-robin to the 8 XCDs, each
// with its own L2, so block b is given tile (b % 8) * per + b / 8: every XCD
// walks a contiguous band of tiles whose rays cross the same cells.  The
// grid has 8 * per blocks, per = ceil(num_tiles / 8); surplus blocks idle.
constexpr uint32_t kXcds = 8;
constexpr uint32_t kTile = 16;

__host__ __device__ inline uint32_t num_ray_tiles(uint32_t num_rays, uint32_t width) {
    if (width == 0) return (num_rays + kBlock - 1) / kBlock;
    const uint32_t height = num_rays / width;
    return ((width + kTile - 1) / kTile) * ((height + kTile - 1) / kTile);
}

__host__ inline uint32_t grid_blocks_for_tiles(uint32_t num_tiles) {
    return kXcds * ((num_tiles + kXcds - 1) / kXcds);
}

// The tile of this block.  Blocks go to the XCDs round robin (block b runs
// on XCD b % 8).  CHUNK == 0: XCD x takes one contiguous run of the tiles;
// otherwise the XCDs take turns on runs of CHUNK tiles, so each XCD's work
// is spread over the whole image (the cost of a tile varies a lot across an
// image) while neighbouring tiles still share an XCD's L2.  Both are
// permutations of [0, gridDim.x).
template <uint32_t CHUNK>
__device__ __forceinline__ uint32_t block_tile() {
    const uint32_t per = gridDim.x / kXcds;
    const uint32_t k = blockIdx.x / kXcds, x = blockIdx.x % kXcds;
    if constexpr (CHUNK == 0) {
        return x * per + k;
    } else {
        const uint32_t full = (per / CHUNK) * CHUNK;
        return k < full ? ((k / CHUNK) * kXcds + x) * CHUNK + k % CHUNK
                        : kXcds * full + (k - full) * kXcds + x;
    }
}

// Tile runs of the forward and the inference render (measured on a
// 1600x1200 camera: the forward is about 13% faster than with one run per
// XCD, the backward about 2% slower, so it keeps one run per XCD).
constexpr uint32_t kForwardChunk = 128;
constexpr uint32_t kBackwardChunk = 0;

// The ray this lane traces: with `order` (a permutation of the rays, see
// order_kernels.hip) lane i of the launch takes ray order[i]; entries out of
// range leave the lane idle.  Otherwise rays in their own order, or 16x16
// pixel tiles of an image `width` pixels wide.
template <uint32_t CHUNK>
__device__ __forceinline__ uint32_t ray_for_lane(uint32_t num_rays, uint32_t width,
                                                 uint32_t num_tiles, bool &valid,
                                                 const uint32_t *__restrict__ order = nullptr) {
    const uint32_t t = block_tile<CHUNK>();
    if (t >= num_tiles) {
        valid = false;
        return 0;
    }
    if (order) {
        const uint32_t i = t * kBlock + threadIdx.x;
        const uint32_t r = i < num_rays ? order[i] : num_rays;
        valid = r < num_rays;
        return valid ? r : 0u;
    }
    if (width == 0) {
        const uint32_t i = t * kBlock + threadIdx.x;
        valid = i < num_rays;
        return i;
    }
    const uint32_t height = num_rays / width;
    const uint32_t tiles_x = (width + kTile - 1) / kTile;
    const uint32_t w = threadIdx.x >> 6, l = threadIdx.x & 63u;
    const uint32_t x = (t % tiles_x) * kTile + (w & 1u) * 8u + (l & 7u);
    const uint32_t y = (t / tiles_x) * kTile + (w >> 1) * 8u + (l >> 3);
    valid = x < width && y < height;
    return valid ? y * width + x : 0u;
}

// ray.direction /= ray.direction.norm()  (src/tracing/pipeline.cu:76-77)
__device__ __forceinline__ RayF load_ray(const float *__restrict__ rays, uint32_t i) {
    const float *r = rays + 6ull * i;
    RayF ray;
    ray.ox = r[0];
    ray.oy = r[1];
    ray.oz = r[2];
    const float x = r[3], y = r[4], z = r[5];
    const float n = sqrtf(sdf_dot3(x, y, z, x, y, z));
    ray.dx = x / n;
    ray.dy = y / n;
    ray.dz = z / n;
    return ray;
}

// Real SH basis up to degree L, 3DGS sign convention
// (src/tracing/sh_utils.cuh:8-62).
template <int L>
__device__ __forceinline__ void sh_basis(float x, float y, float z, float *sh) {
    constexpr float C0 = 0.28209479177387814f;
    constexpr float C1 = 0.4886025119029199f;
    sh[0] = C0;
    if constexpr (L > 0) {
        sh[1] = -C1 * y;
        sh[2] = C1 * z;
        sh[3] = -C1 * x;
    }
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, yz = y * z, xz = x * z;
    if constexpr (L > 1) {
        sh[4] = 1.0925484305920792f * xy;
        sh[5] = -1.0925484305920792f * yz;
        sh[6] = 0.31539156525252005f * (2.0f * zz - xx - yy);
        sh[7] = -1.0925484305920792f * xz;
        sh[8] = 0.5462742152960396f * (xx - yy);
    }
    if constexpr (L > 2) {
        sh[9] = -0.5900435899266435f * y * (3.0f * xx - yy);
        sh[10] = 2.890611442640554f * xy * z;
        sh[11] = -0.4570457994644658f * y * (4.0f * zz - xx - yy);
        sh[12] = 0.3731763325901154f * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
        sh[13] = -0.4570457994644658f * x * (4.0f * zz - xx - yy);
        sh[14] = 1.445305721320277f * z * (xx - yy);
        sh[15] = -0.5900435899266435f * x * (xx - 3.0f * yy);
    }
}

// rgb = max(0, 0.5 + sum_j Y_j * row[3j + c])  (src/tracing/sh_utils.cuh:64-75);
// fp16 rows are widened exactly (sh_utils.cuh:79, `(float)sh_rgb_vals[i]`).
// `sh` holds the ray's basis at a stride of `sh_stride` floats (the LDS
// tables keep one basis function per row, so lanes hit distinct banks).
template <int L, typename AT>
__device__ __forceinline__ void sh_rgb(const float *sh, int sh_stride, const AT *__restrict__ row,
                                       float &r, float &g, float &b) {
    constexpr int nsh = (L + 1) * (L + 1);
    float a0 = 0.5f, a1 = 0.5f, a2 = 0.5f;
    // partial unroll: 12 row values in flight at a time instead of 48 keeps
    // the kernels' register count low (same FMA order per channel)
#pragma unroll 4
    for (int j = 0; j < nsh; ++j) {
        const float y = sh[j * sh_stride];
        a0 = fmaf(y, (float)row[3 * j + 0], a0);
        a1 = fmaf(y, (float)row[3 * j + 1], a1);
        a2 = fmaf(y, (float)row[3 * j + 2], a2);
    }
    r = fmaxf(a0, 0.0f);
    g = fmaxf(a1, 0.0f);
    b = fmaxf(a2, 0.0f);
}

// sh_rgb with the basis in registers (sh[j], fully unrolled): the same fused
// products in the same order per channel, so the same bits.
template <int L, typename AT>
__device__ __forceinline__ void sh_rgb_regs(const float *sh, const AT *__restrict__ row, float &r,
                                            float &g, float &b) {
    constexpr int nsh = (L + 1) * (L + 1);
    float a0 = 0.5f, a1 = 0.5f, a2 = 0.5f;
#pragma unroll
    for (int j = 0; j < nsh; ++j) {
        a0 = fmaf(sh[j], (float)row[3 * j + 0], a0);
        a1 = fmaf(sh[j], (float)row[3 * j + 1], a1);
        a2 = fmaf(sh[j], (float)row[3 * j + 2], a2);
    }
    r = fmaxf(a0, 0.0f);
    g = fmaxf(a1, 0.0f);
    b = fmaxf(a2, 0.0f);
}

// Cell table (optional; the forward builds it from the caller's arrays before
// it walks): one record per cell holding what a step of the forward reads of
// that cell: words 0-2 the position (fp32 bits), word 3 the CSR row begin,
// word 4 its end, then from byte 20 the cell's attribute row in the
// pipeline's attribute type, zero-padded to a power of two of at least 64
// bytes.  A step then touches the record's one or two whole cache lines
// instead of the lines of three arrays (position, offsets, a 196-byte row at
// any 4-byte alignment).
constexpr uint32_t kCellAttrByte = 20;
__host__ __device__ constexpr uint32_t cell_record_bytes(int L, uint32_t attr_size) {
    const uint32_t need = kCellAttrByte + (1u + 3u * (L + 1) * (L + 1)) * attr_size;
    uint32_t b = 64;
    while (b < need) b *= 2;
    return b;
}

// Fourth half of an offset-table entry built with the cell table: the
// neighbour a of the row's cell i as a - i in int16, or kDeltaNone when it
// does not fit (the walk then reads the adjacency).  Every delta but
// kDeltaNone decodes to a exactly.
constexpr uint32_t kDeltaNone = 0x8000u;
__host__ __device__ inline uint32_t neighbour_delta(uint32_t i, uint32_t a) {
    const int64_t d = (int64_t)a - (int64_t)i;
    return (d >= -32767 && d <= 32767) ? (uint32_t)(uint16_t)(int16_t)d : kDeltaNone;
}

struct SceneView {
    const float *__restrict__ points;
    const void *__restrict__ attrs; // [N, D] of the pipeline's attribute type
    const uint32_t *__restrict__ adj;
    const uint32_t *__restrict__ offs;
    const uint2 *__restrict__ diff; // fp16 x, y | z, 0 per CSR entry
    const uint32_t *__restrict__ cells; // cell table or NULL
    uint32_t num_points;
    uint32_t num_adj;
};

struct WalkCounters {
    uint32_t n;             // loop iterations (the reference's return value)
    uint32_t steps;         // step-functor calls
    uint64_t faces;         // faces scanned
    uint64_t faces_stepped; // faces of the cells that got a step
};

// Per-lane state of the walk of src/tracing/tracing_utils.cuh:15-109.
struct WalkState {
    uint32_t cell;
    float xc[3];   // position of `cell`
    float t0;      // entry distance into `cell`
    uint32_t n;    // loop iterations so far (the reference's return value)
    uint32_t beg, end; // CSR row of `cell` (walks over a cell table)
    bool alive;
};

// Outcome of one loop iteration of the walk.
struct StepInfo {
    bool found;    // an exit face was found: the walk moves to `next`
    bool stepped;  // ... and t1 > t0: the step functor runs for `cell`
    bool agrees;   // (DUAL scans) an unsafe-mode walk takes the same exit
    uint32_t next;
    float t1;
    float xn[3];
    uint32_t beg, end; // CSR row of `next` (walks over a cell table)
};

// Position and CSR row of cell i: from the cell table when RB (its record
// bytes) is nonzero, else from the points and offsets arrays.
template <uint32_t RB>
__device__ __forceinline__ void load_cell(const SceneView &sc, uint32_t i, float *x, uint32_t &beg,
                                          uint32_t &end) {
    if constexpr (RB != 0) {
        const uint32_t *r = sc.cells + (uint64_t)i * (RB / 4);
        const uint4 h = *reinterpret_cast<const uint4 *>(r);
        x[0] = __builtin_bit_cast(float, h.x);
        x[1] = __builtin_bit_cast(float, h.y);
        x[2] = __builtin_bit_cast(float, h.z);
        beg = h.w;
        end = r[4];
    } else {
        x[0] = sc.points[3ull * i];
        x[1] = sc.points[3ull * i + 1];
        x[2] = sc.points[3ull * i + 2];
        beg = end = 0;
    }
}

template <uint32_t RB = 0>
__device__ __forceinline__ void walk_init(const SceneView &sc, uint32_t start, WalkState &ws) {
    ws.cell = start;
    ws.t0 = 0.0f;
    ws.n = 0;
    ws.alive = start < sc.num_points;
    ws.xc[0] = ws.xc[1] = ws.xc[2] = 0.0f;
    ws.beg = ws.end = 0;
    if (ws.alive) load_cell<RB>(sc, start, ws.xc, ws.beg, ws.end);
}

// One iteration of the walk: exit face = the first minimum t over the cell's
// CSR row with dp > 0 (and t > t0 in safe mode).  The reference passes
// UINT32_MAX for the index bounds; the real bounds are used here, which is
// the same walk for a well-formed scene and ends it instead of reading out
// of bounds otherwise.  Clears ws.alive when the walk ends.
// GUARD: the offset table has no padding past E (a caller's table), so the
// last batch of a row re-reads the row's last entry instead of over-reading.
// DUAL (safe scans): also tell whether the unsafe mode's exit (the first
// minimum t over dp > 0 alone) is the same face: it is unless the smallest
// such t is <= t0 (then it lies outside the safe set, or the safe set is
// empty while the unsafe one is not); sets si.agrees.
// RB: walk over a cell table of RB-byte records (0: the scene's arrays).
// HALF: a batch's second pair of entries is loaded only by the lanes whose
// row reaches it (fewer bytes for memory-bound walks of incoherent rays; one
// more branch per batch, which costs more than it saves where a wavefront's
// rays share their cells).
template <bool SAFE, bool COUNT, bool GUARD = false, bool DUAL = false, uint32_t RB = 0,
          bool HALF = false>
__device__ __forceinline__ void walk_advance(const SceneView &sc, const RayF &ray,
                                             uint32_t max_steps, WalkState &ws, StepInfo &si,
                                             WalkCounters &wc) {
    static_assert(SAFE || !DUAL, "DUAL compares a safe scan with the unsafe one");
    si.found = false;
    si.agrees = true;
    si.stepped = false;
    ++ws.n;
    if (ws.n > max_steps) {
        ws.alive = false;
        return;
    }
    const uint32_t beg = RB ? ws.beg : sc.offs[ws.cell];
    const uint32_t end = RB ? ws.end : sc.offs[ws.cell + 1];
    if (beg > end || end > sc.num_adj) {
        ws.alive = false;
        return;
    }
    const uint32_t nf = end - beg;
    const float t0 = ws.t0;
    float t1 = __builtin_bit_cast(float, 0x7f800000u);
    float tmin_u = t1; // DUAL: smallest computed t over dp > 0 (NaN never taken)
    bool below = false; // DUAL: a face with dp > 0 and t < t0 for certain
    uint32_t best = kNoIndex;
    // t = num / dp (correctly rounded) is formed only for faces that could be
    // taken.  Rounding is monotone and t0, t1 are floats, so t < t1 needs
    // num < t1 dp and t > t0 needs num > t0 dp (dp > 0).  The bounds below
    // are those products widened by 2^-21 of their size (more than the
    // roundings of the widened factor and of the fused product, 2^-24 each)
    // and by 2^-126 (for subnormal products and, as dp = diff . d < 2^17 for
    // fp16 diffs and a unit direction, quotients that round to 0), so no face
    // that the exact test takes is skipped and the exit face is the same bit
    // for bit.  t0 >= 0; t1 may be negative in unsafe scans.
    uint32_t bw = kDeltaNone; // RB: the exit entry's neighbour delta
    float t1m = t1;                             // t1 + |t1| 2^-21
    const float t0m = t0 * (1.0f - 0x1p-21f);   // t0 (1 - 2^-21)
    const float t0p = t0 * (1.0f + 0x1p-21f);   // t0 (1 + 2^-21), DUAL
    const uint2 *__restrict__ row = sc.diff + beg;
    // batches of 4: the table is padded, so the last batch may over-read
    for (uint32_t k0 = 0; k0 < nf; k0 += 4) {
        uint2 h[4];
        if constexpr (HALF && !GUARD) {
            h[0] = row[k0];
            h[1] = row[k0 + 1];
            if (k0 + 2 < nf) {
                h[2] = row[k0 + 2];
                h[3] = row[k0 + 3];
            } else {
                h[2] = h[3] = make_uint2(0u, 0u); // past the row: dropped by k < nf
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) h[u] = row[GUARD ? min(k0 + u, nf - 1) : k0 + u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t k = k0 + u;
            const float dx = f16_to_f32(h[u].x);
            const float dy = f16_to_f32(h[u].x >> 16);
            const float dz = f16_to_f32(h[u].y);
            // xc + d * 0.5 (src/tracing/tracing_utils.cuh:73): d * 0.5 is
            // exact for a widened half, so one fused op gives the same bits
            const float fx = fmaf(dx, 0.5f, ws.xc[0]);
            const float fy = fmaf(dy, 0.5f, ws.xc[1]);
            const float fz = fmaf(dz, 0.5f, ws.xc[2]);
            const float dp = sdf_dot3(dx, dy, dz, ray.dx, ray.dy, ray.dz);
            const float num = sdf_dot3(fx - ray.ox, fy - ray.oy, fz - ray.oz, dx, dy, dz);
            const bool pos = dp > 0.0f && k < nf;
            const float lo = fmaf(t0m, dp, -0x1p-126f); // < t0 dp
            bool maybe = pos && num < fmaf(t1m, dp, 0x1p-126f) && (!SAFE || num > lo);
            if constexpr (DUAL) {
                // the unsafe exit differs when some t <= t0: certain below
                // lo, certainly not above t0 (1 + 2^-21) dp, formed between
                below = below || (pos && num < lo);
                maybe = maybe || (pos && num >= lo && num <= fmaf(t0p, dp, 0x1p-126f));
            }
            if (maybe) {
                const float t = num / dp;
                if (SAFE ? (t > t0 && t < t1) : t < t1) {
                    t1 = t;
                    t1m = fmaf(fabsf(t), 0x1p-21f, t);
                    best = k;
                    if constexpr (RB != 0) bw = h[u].y >> 16;
                }
                if constexpr (DUAL) tmin_u = fminf(tmin_u, t);
            }
        }
    }
    if constexpr (COUNT) wc.faces += nf;
    if constexpr (DUAL) si.agrees = !(below || tmin_u <= t0);
    if (best == kNoIndex) {
        ws.alive = false;
        return;
    }
    // over the cell table the entry names the neighbour (but for the rare
    // deltas beyond int16); the adjacency array otherwise
    const uint32_t next = (RB != 0 && bw != kDeltaNone)
                              ? (uint32_t)((int32_t)ws.cell + (int32_t)(int16_t)(uint16_t)bw)
                              : sc.adj[beg + best];
    if (next >= sc.num_points) {
        ws.alive = false;
        return;
    }
    si.found = true;
    si.next = next;
    si.t1 = t1;
    load_cell<RB>(sc, next, si.xn, si.beg, si.end);
    si.stepped = t1 > t0;
    if constexpr (COUNT) {
        if (si.stepped) {
            wc.steps++;
            wc.faces_stepped += nf;
        }
    }
}

__device__ __forceinline__ void walk_move(WalkState &ws, const StepInfo &si) {
    ws.t0 = fmaxf(ws.t0, si.t1);
    ws.cell = si.next;
    ws.xc[0] = si.xn[0];
    ws.xc[1] = si.xn[1];
    ws.xc[2] = si.xn[2];
    ws.beg = si.beg;
    ws.end = si.end;
}

// cell_intersection_grad (src/tracing/tracing_utils.cuh:112-124):
// d t / d p for t = ((p + q) / 2 - o) . (q - p) / ((q - p) . d)
__device__ __forceinline__ void cell_isect_grad(const float *p, const float *q, const RayF &ray,
                                                float *g) {
    const float fo0 = (p[0] + q[0]) / 2.0f, fo1 = (p[1] + q[1]) / 2.0f, fo2 = (p[2] + q[2]) / 2.0f;
    const float fn0 = q[0] - p[0], fn1 = q[1] - p[1], fn2 = q[2] - p[2];
    const float num = sdf_dot3(fo0 - ray.ox, fo1 - ray.oy, fo2 - ray.oz, fn0, fn1, fn2);
    const float dp = sdf_dot3(fn0, fn1, fn2, ray.dx, ray.dy, ray.dz);
    const float dp2 = dp * dp;
    g[0] = (num * ray.dx + dp * (ray.ox - p[0])) / dp2;
    g[1] = (num * ray.dy + dp * (ray.oy - p[1])) / dp2;
    g[2] = (num * ray.dz + dp * (ray.oz - p[2])) / dp2;
}

// cell_isect_grad(p, q) and cell_isect_grad(q, p) together.  Swapping p and
// q negates the face normal q - p exactly, and with it num and dp (every
// product and fused sum of the dots changes sign only), while (p + q) / 2
// and dp^2 stay the same; so both come from one set of them, bit for bit
// what the two separate calls give.
__device__ __forceinline__ void cell_isect_grad_pair(const float *p, const float *q,
                                                     const RayF &ray, float *g_pq, float *g_qp) {
    const float fo0 = (p[0] + q[0]) / 2.0f, fo1 = (p[1] + q[1]) / 2.0f, fo2 = (p[2] + q[2]) / 2.0f;
    const float fn0 = q[0] - p[0], fn1 = q[1] - p[1], fn2 = q[2] - p[2];
    const float num = sdf_dot3(fo0 - ray.ox, fo1 - ray.oy, fo2 - ray.oz, fn0, fn1, fn2);
    const float dp = sdf_dot3(fn0, fn1, fn2, ray.dx, ray.dy, ray.dz);
    const float dp2 = dp * dp;
    g_pq[0] = (num * ray.dx + dp * (ray.ox - p[0])) / dp2;
    g_pq[1] = (num * ray.dy + dp * (ray.oy - p[1])) / dp2;
    g_pq[2] = (num * ray.dz + dp * (ray.oz - p[2])) / dp2;
    const float nnum = -num, ndp = -dp;
    g_qp[0] = (nnum * ray.dx + ndp * (ray.ox - q[0])) / dp2;
    g_qp[1] = (nnum * ray.dy + ndp * (ray.oy - q[1])) / dp2;
    g_qp[2] = (nnum * ray.dz + ndp * (ray.oz - q[2])) / dp2;
}

__device__ __forceinline__ uint64_t fnv_step(uint64_t h, uint32_t cell) {
    return (h ^ (uint64_t)cell) * 0x100000001b3ull;
}

constexpr uint64_t kFnvOffset = 0xcbf29ce484222325ull;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

} // namespace sdfoam_hip
