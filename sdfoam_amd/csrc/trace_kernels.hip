// Forward / backward kernels of the Voronoi-foam tracer for gfx950, and the
// fp16 neighbour-offset prepass.
//
// One lane per ray (wave64), 256 lanes per block.  Each lane walks its ray
// through the cells of the foam (trace_device.h), compositing in registers.
// The backward pass replays the same walk and accumulates per-point
// gradients with fp32 atomics; the sharpness gradient, a single address in
// the reference, is summed per lane and reduced per wave before one atomic.
#include "trace_kernels.h"

namespace sdfoam_hip {

// ---------------------------------------------------------------------------
// prefetch_adjacent_diff (src/tracing/pipeline.cu:1202-1242): one lane per
// CSR entry (coalesced over the adjacency array) instead of one per row; the
// row of entry k is found by a binary search of the offsets.

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
// forward (src/tracing/pipeline.cu:36-264)

template <int L, bool NEUS, bool STATS>
__global__ __launch_bounds__(kBlock) void forward_kernel(FwdArgs a) {
    const uint32_t ray_idx = blockIdx.x * kBlock + threadIdx.x;
    if (ray_idx >= a.num_rays) return;
    constexpr int nsh = (L + 1) * (L + 1);
    constexpr int D = 1 + 3 * nsh;

    const RayF ray = load_ray(a.rays, ray_idx);
    float sh[nsh];
    sh_basis<L>(ray.dx, ray.dy, ray.dz, sh);
    const float sha = a.sharpness[0];
    const int32_t sdf_ch = a.settings.sdf_channel;
    const bool neus_alpha = NEUS && sdf_ch >= 0;
    const float thr = a.settings.weight_threshold;
    const uint32_t Q = a.num_quantiles;
    const float *rq = a.quantiles ? a.quantiles + (uint64_t)ray_idx * Q : nullptr;

    float T = 1.0f;
    float C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
    uint32_t qi = 0;
    float q = (rq && Q > 0) ? rq[0] : 0.0f;
    uint64_t hash = kFnvOffset;
    uint32_t rec = 0;

    auto step = [&](uint32_t cell, uint32_t next, float t0, float t1, const float *xc,
                    const float *xn) -> bool {
        const float *__restrict__ row = a.scene.attrs + (uint64_t)cell * D;
        float s = row[D - 1];
        float r, g, b;
        if (NEUS || s > 1e-6f) {
            sh_rgb<L>(sh, row, r, g, b);
        } else {
            r = g = b = 0.0f;
        }
        float alpha;
        const float dt = fmaxf(t1 - t0, 0.0f);
        if (neus_alpha) {
            const float d = row[sdf_ch];
            const float phi = sdf_sigmoidf(-sha * d);
            s = sha * phi * (1.0f - phi);
            alpha = 1.0f - sdf_expf(-s * dt);
        } else {
            alpha = 1.0f - sdf_expf(-s * dt);
        }
        const float w = T * alpha;
        if (a.alpha_out) a.alpha_out[cell] = alpha; // racy last writer, as the reference
        if (a.contribution) atomicAdd(a.contribution + cell, w);
        C0 = fmaf(w, r, C0);
        C1 = fmaf(w, g, C1);
        C2 = fmaf(w, b, C2);
        const float Tn = T * (1.0f - alpha);
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
        if constexpr (STATS) {
            hash = fnv_step(hash, cell);
            if (a.cells && rec < a.cells_stride) a.cells[(uint64_t)ray_idx * a.cells_stride + rec] = cell;
            ++rec;
        }
        T = Tn;
        return T > thr;
    };

    WalkCounters wc;
    walk<true, STATS>(a.scene, ray, a.start[ray_idx], a.settings.max_intersections, step, wc);

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
    float4 out = make_float4(C0, C1, C2, 1.0f - T);
    *reinterpret_cast<float4 *>(a.rgba + 4ull * ray_idx) = out;
    if (a.num_intersections) a.num_intersections[ray_idx] = wc.n;
}

// ---------------------------------------------------------------------------
// backward, shared geometry bookkeeping (src/tracing/pipeline.cu:452-474 and
// :731-760): the position gradient of a cell is flushed one step late, the
// first cell gets a face against the world origin (prev = 0) and the last
// two pending gradients are never flushed -- all as the reference does.

struct GeomState {
    uint32_t prev_idx;
    float prev_pt[3];
    float prev_g[3], cur_g[3], next_g[3];
};

__device__ __forceinline__ void geom_step(GeomState &gs, uint32_t cell, const float *xc,
                                          const float *xn, float dL_dt0, float dL_dt1,
                                          const RayF &ray, float *__restrict__ points_grad) {
    float dprev[3] = {0.0f, 0.0f, 0.0f};
    if (gs.prev_idx != kNoIndex) cell_isect_grad(gs.prev_pt, xc, ray, dprev);
    float dt1_cur[3], dt0_cur[3], dt1_next[3];
    cell_isect_grad(xc, xn, ray, dt1_cur);
    cell_isect_grad(xc, gs.prev_pt, ray, dt0_cur);
    cell_isect_grad(xn, xc, ray, dt1_next);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        gs.prev_g[i] = fmaf(dL_dt0, dprev[i], gs.prev_g[i]);
        gs.cur_g[i] = gs.cur_g[i] + (dL_dt0 * dt0_cur[i] + dL_dt1 * dt1_cur[i]);
        gs.next_g[i] = fmaf(dL_dt1, dt1_next[i], gs.next_g[i]);
    }
    if (gs.prev_idx != kNoIndex) {
        float *dst = points_grad + 3ull * gs.prev_idx;
        atomicAdd(dst + 0, gs.prev_g[0]);
        atomicAdd(dst + 1, gs.prev_g[1]);
        atomicAdd(dst + 2, gs.prev_g[2]);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        gs.prev_pt[i] = xc[i];
        gs.prev_g[i] = gs.cur_g[i];
        gs.cur_g[i] = gs.next_g[i];
        gs.next_g[i] = 0.0f;
    }
    gs.prev_idx = cell;
}

// SH colour gradients, zeroed where the colour clamped to 0
// (src/tracing/pipeline.cu:528-533, src/tracing/sh_utils.cuh:85-92)
template <int L>
__device__ __forceinline__ void sh_grad(const float *sh, float r, float g, float b, float gr,
                                        float gg, float gb, float *__restrict__ grow) {
    constexpr int nsh = (L + 1) * (L + 1);
    if (r == 0.0f) gr = 0.0f;
    if (g == 0.0f) gg = 0.0f;
    if (b == 0.0f) gb = 0.0f;
#pragma unroll
    for (int j = 0; j < nsh; ++j) {
        atomicAdd(grow + 3 * j + 0, sh[j] * gr);
        atomicAdd(grow + 3 * j + 1, sh[j] * gg);
        atomicAdd(grow + 3 * j + 2, sh[j] * gb);
    }
}

// backward_sdf (src/tracing/pipeline.cu:267-550)
template <int L, bool STATS>
__global__ __launch_bounds__(kBlock) void backward_sdf_kernel(BwdArgs a) {
    const uint32_t ray_idx = blockIdx.x * kBlock + threadIdx.x;
    constexpr int nsh = (L + 1) * (L + 1);
    constexpr int D = 1 + 3 * nsh;
    float sharp_acc = 0.0f;
    if (ray_idx < a.num_rays) {
        const RayF ray = load_ray(a.rays, ray_idx);
        float sh[nsh];
        sh_basis<L>(ray.dx, ray.dy, ray.dz, sh);
        const float sha = a.sharpness[0];
        const int32_t sdf_ch = a.settings.sdf_channel >= 0 ? a.settings.sdf_channel : D - 1;
        const bool write_sdf = a.settings.sdf_channel >= 0;
        const float thr = a.settings.weight_threshold;
        const uint32_t Q = a.num_quantiles;
        const float *rq = a.quantiles ? a.quantiles + (uint64_t)ray_idx * Q : nullptr;
        const float *rdg = a.depth_grad ? a.depth_grad + (uint64_t)ray_idx * Q : nullptr;
        // the statistics instantiation gets no rgba / gradient buffers
        const float4 g4 = STATS ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                : *reinterpret_cast<const float4 *>(a.rgba_grad + 4ull * ray_idx);
        const float4 c4 = STATS ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                : *reinterpret_cast<const float4 *>(a.rgba + 4ull * ray_idx);
        const float err = a.ray_error ? a.ray_error[ray_idx] : 0.0f;

        float T = 1.0f;
        float C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
        uint32_t qi = 0;
        float q = (rq && Q > 0) ? rq[0] : 0.0f;
        float g_logT = 0.0f;
        GeomState gs;
        gs.prev_idx = kNoIndex;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            gs.prev_pt[i] = 0.0f;
            gs.prev_g[i] = gs.cur_g[i] = gs.next_g[i] = 0.0f;
        }
        uint64_t hash = kFnvOffset;
        uint32_t rec = 0;

        auto step = [&](uint32_t cell, uint32_t next, float t0, float t1, const float *xc,
                        const float *xn) -> bool {
            if constexpr (STATS) {
                hash = fnv_step(hash, cell);
                if (a.cells && rec < a.cells_stride) a.cells[(uint64_t)ray_idx * a.cells_stride + rec] = cell;
                ++rec;
            }
            const float *__restrict__ row = a.scene.attrs + (uint64_t)cell * D;
            float r, g, b;
            sh_rgb<L>(sh, row, r, g, b);
            const float dt = fmaxf(t1 - t0, 0.0f);
            const float d = row[sdf_ch];
            const float phi = sdf_sigmoidf(-sha * d);
            const float s = sha * phi * (1.0f - phi);
            const float alpha = 1.0f - sdf_expf(-s * dt);
            const float w = T * alpha;
            C0 = fmaf(w, r, C0);
            C1 = fmaf(w, g, C1);
            C2 = fmaf(w, b, C2);
            if (STATS) {
                const float Tn = T * (1.0f - alpha);
                T = Tn;
                return T > thr;
            }
            if (a.point_error) atomicAdd(a.point_error + cell, w * err);

            const float dr = g4.x * w, dg = g4.y * w, db = g4.z * w;
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
            const float Tn = T * (1.0f - alpha);
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
            geom_step(gs, cell, xc, xn, units - dL_ddelta, dL_ddelta, ray, a.points_grad);

            const float dphi_dd = -sha * phi * (1.0f - phi);
            const float ds_dd = sha * (1.0f - 2.0f * phi) * dphi_dd;
            const float ds_dsha = phi * (1.0f - phi) * (1.0f - sha * d * (1.0f - 2.0f * phi));
            float *__restrict__ grow = a.attr_grad + (uint64_t)cell * D;
            if (write_sdf) atomicAdd(grow + sdf_ch, dL_ds * ds_dd);
            sharp_acc += dL_ds * ds_dsha;
            sh_grad<L>(sh, r, g, b, dr, dg, db, grow);
            T = Tn;
            return T > thr;
        };

        WalkCounters wc;
        walk<true, STATS>(a.scene, ray, a.start[ray_idx], a.settings.max_intersections, step, wc);
        if constexpr (STATS) {
            if (a.visit_hash) a.visit_hash[ray_idx] = hash;
            if (a.steps) a.steps[ray_idx] = wc.steps;
            if (a.faces) a.faces[ray_idx] = wc.faces;
            if (a.faces_stepped) a.faces_stepped[ray_idx] = wc.faces_stepped;
        }
    }
    if constexpr (!STATS) {
        if (a.sharpness_grad) {
            const float v = wave_sum(sharp_acc);
            if ((threadIdx.x & 63) == 0 && v != 0.0f) atomicAdd(a.sharpness_grad, v);
        }
    }
}

// backward, density mode (src/tracing/pipeline.cu:553-791); the walk runs in
// the reference's unsafe mode (no t > t0 test, :782-790).
template <int L, bool STATS>
__global__ __launch_bounds__(kBlock) void backward_density_kernel(BwdArgs a) {
    const uint32_t ray_idx = blockIdx.x * kBlock + threadIdx.x;
    if (ray_idx >= a.num_rays) return;
    constexpr int nsh = (L + 1) * (L + 1);
    constexpr int D = 1 + 3 * nsh;
    const RayF ray = load_ray(a.rays, ray_idx);
    float sh[nsh];
    sh_basis<L>(ray.dx, ray.dy, ray.dz, sh);
    const float thr = a.settings.weight_threshold;
    const uint32_t Q = a.num_quantiles;
    const float *rq = a.quantiles ? a.quantiles + (uint64_t)ray_idx * Q : nullptr;
    const float *rdg = a.depth_grad ? a.depth_grad + (uint64_t)ray_idx * Q : nullptr;
    // the statistics instantiation gets no rgba / gradient / depth buffers
    const float4 g4 = STATS ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                            : *reinterpret_cast<const float4 *>(a.rgba_grad + 4ull * ray_idx);
    const float4 c4 = STATS ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                            : *reinterpret_cast<const float4 *>(a.rgba + 4ull * ray_idx);
    const float err = a.ray_error ? a.ray_error[ray_idx] : 0.0f;

    float cur_dg = 0.0f; // src/tracing/pipeline.cu:620-629
    for (uint32_t k = 0; k < (STATS ? 0u : Q); ++k) {
        const uint32_t pi = a.depth_indices[(uint64_t)ray_idx * Q + k];
        if (pi != kNoIndex && pi < a.scene.num_points) {
            cur_dg = cur_dg + rdg[k] / a.scene.attrs[(uint64_t)pi * D + D - 1];
        }
    }
    float T = 1.0f;
    float C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
    uint32_t qi = 0;
    float q = (rq && Q > 0) ? rq[0] : 0.0f;
    GeomState gs;
    gs.prev_idx = kNoIndex;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        gs.prev_pt[i] = 0.0f;
        gs.prev_g[i] = gs.cur_g[i] = gs.next_g[i] = 0.0f;
    }
    uint64_t hash = kFnvOffset;
    uint32_t rec = 0;

    auto step = [&](uint32_t cell, uint32_t next, float t0, float t1, const float *xc,
                    const float *xn) -> bool {
        if constexpr (STATS) {
            hash = fnv_step(hash, cell);
            if (a.cells && rec < a.cells_stride) a.cells[(uint64_t)ray_idx * a.cells_stride + rec] = cell;
            ++rec;
        }
        const float *__restrict__ row = a.scene.attrs + (uint64_t)cell * D;
        const float s = row[D - 1];
        float r, g, b;
        if (s > 1e-6f) {
            sh_rgb<L>(sh, row, r, g, b);
        } else {
            r = g = b = 0.0f;
        }
        const float dt = fmaxf(t1 - t0, 0.0f);
        const float alpha = 1.0f - sdf_expf(-s * dt);
        const float w = T * alpha;
        const float dalpha_ds = dt * (1.0f - alpha);
        float dalpha_ddt = 0.0f;
        if (dt > 0.0f) dalpha_ddt = s * (1.0f - alpha);
        C0 = fmaf(w, r, C0);
        C1 = fmaf(w, g, C1);
        C2 = fmaf(w, b, C2);
        if (STATS) {
            T = T * (1.0f - alpha);
            return T > thr;
        }
        if (a.point_error) atomicAdd(a.point_error + cell, w * err);
        const float dr = g4.x * w, dg = g4.y * w, db = g4.z * w;
        const float den = T * (1.0f - alpha + 1e-6f);
        const float rest0 = (c4.x - C0) / den;
        const float rest1 = (c4.y - C1) / den;
        const float rest2 = (c4.z - C2) / den;
        float dL_dalpha = T * sdf_dot3(r - rest0, g - rest1, b - rest2, g4.x, g4.y, g4.z);
        dL_dalpha = dL_dalpha + (1.0f - c4.w) * g4.w / (1.0f - alpha + 1e-6f);
        float dL_ds = dL_dalpha * dalpha_ds;
        float dL_ddt = dL_dalpha * dalpha_ddt;
        float dL_dt0 = 0.0f;
        const float Tn = T * (1.0f - alpha);
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
        geom_step(gs, cell, xc, xn, dL_dt0, dL_ddt, ray, a.points_grad);
        T = Tn;
        float *__restrict__ grow = a.attr_grad + (uint64_t)cell * D;
        sh_grad<L>(sh, r, g, b, dr, dg, db, grow);
        atomicAdd(grow + (D - 1), dL_ds);
        return T > thr;
    };

    WalkCounters wc;
    walk<false, STATS>(a.scene, ray, a.start[ray_idx], a.settings.max_intersections, step, wc);
    if constexpr (STATS) {
        if (a.visit_hash) a.visit_hash[ray_idx] = hash;
        if (a.steps) a.steps[ray_idx] = wc.steps;
        if (a.faces) a.faces[ray_idx] = wc.faces;
        if (a.faces_stepped) a.faces_stepped[ray_idx] = wc.faces_stepped;
    }
}

// ---------------------------------------------------------------------------
// launchers

static inline dim3 grid_for(uint64_t n) { return dim3((unsigned)((n + kBlock - 1) / kBlock)); }

hipError_t launch_prefetch_diff(const float *points, uint32_t num_points, uint32_t num_adj,
                                const uint32_t *adj, const uint32_t *offs, uint2 *diff,
                                hipStream_t stream) {
    hipLaunchKernelGGL(prefetch_diff_kernel, grid_for((uint64_t)num_adj + kDiffPad), dim3(kBlock), 0,
                       stream, points, num_points, num_adj, adj, offs, diff);
    return hipGetLastError();
}

template <int L>
static hipError_t launch_forward_L(const FwdArgs &a, bool neus, bool stats, hipStream_t stream) {
    const dim3 grid = grid_for(a.num_rays);
    if (neus) {
        if (stats) {
            hipLaunchKernelGGL((forward_kernel<L, true, true>), grid, dim3(kBlock), 0, stream, a);
        } else {
            hipLaunchKernelGGL((forward_kernel<L, true, false>), grid, dim3(kBlock), 0, stream, a);
        }
    } else {
        if (stats) {
            hipLaunchKernelGGL((forward_kernel<L, false, true>), grid, dim3(kBlock), 0, stream, a);
        } else {
            hipLaunchKernelGGL((forward_kernel<L, false, false>), grid, dim3(kBlock), 0, stream, a);
        }
    }
    return hipGetLastError();
}

hipError_t launch_forward(int L, const FwdArgs &a, bool neus, bool stats, hipStream_t stream) {
    switch (L) {
    case 0: return launch_forward_L<0>(a, neus, stats, stream);
    case 1: return launch_forward_L<1>(a, neus, stats, stream);
    case 2: return launch_forward_L<2>(a, neus, stats, stream);
    case 3: return launch_forward_L<3>(a, neus, stats, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int L>
static hipError_t launch_backward_L(const BwdArgs &a, bool neus, bool stats, hipStream_t stream) {
    const dim3 grid = grid_for(a.num_rays);
    if (neus) {
        if (stats) {
            hipLaunchKernelGGL((backward_sdf_kernel<L, true>), grid, dim3(kBlock), 0, stream, a);
        } else {
            hipLaunchKernelGGL((backward_sdf_kernel<L, false>), grid, dim3(kBlock), 0, stream, a);
        }
    } else {
        if (stats) {
            hipLaunchKernelGGL((backward_density_kernel<L, true>), grid, dim3(kBlock), 0, stream, a);
        } else {
            hipLaunchKernelGGL((backward_density_kernel<L, false>), grid, dim3(kBlock), 0, stream, a);
        }
    }
    return hipGetLastError();
}

hipError_t launch_backward(int L, const BwdArgs &a, bool neus, bool stats, hipStream_t stream) {
    switch (L) {
    case 0: return launch_backward_L<0>(a, neus, stats, stream);
    case 1: return launch_backward_L<1>(a, neus, stats, stream);
    case 2: return launch_backward_L<2>(a, neus, stats, stream);
    case 3: return launch_backward_L<3>(a, neus, stats, stream);
    default: return hipErrorInvalidValue;
    }
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
