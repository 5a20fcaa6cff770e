/*
 * TEST INFRASTRUCTURE -- NOT PART OF THE PRODUCT.  See sdf_oracle.h.
 *
 * Scalar C restatement of the reference's Voronoi-foam tracer
 * (src/tracing/tracing_utils.cuh, src/tracing/pipeline.cu,
 * src/tracing/sh_utils.cuh) and of its AABB tree (src/aabb_tree/).
 * Built with -O2 -ffp-contract=off, no fast-math (oracle/Makefile).
 */
#include "sdf_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "../include/sdfoam_fpmath.h"

const char *oracle_version(void) { return "sdfoam-oracle 1"; }

/* ------------------------------------------------------------------------ */
/* fpmath exports                                                            */

float oracle_expf(float x) { return sdf_expf(x); }
float oracle_sigmoidf(float x) { return sdf_sigmoidf(x); }
uint16_t oracle_f32_to_f16(float x) { return sdf_f32_to_f16_bits(x); }
float oracle_f16_to_f32(uint16_t h) { return sdf_f16_bits_to_f32(h); }

void oracle_expf_n(const float *x, float *y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = sdf_expf(x[i]);
}

void oracle_f32_to_f16_n(const float *x, uint16_t *y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = sdf_f32_to_f16_bits(x[i]);
}

/* ------------------------------------------------------------------------ */
/* accumulation helpers                                                      */

static void add_f64(double *dst, double v, int shared) {
    if (!shared) {
        *dst += v;
        return;
    }
    uint64_t *p = (uint64_t *)dst;
    uint64_t old = __atomic_load_n(p, __ATOMIC_RELAXED);
    uint64_t nw;
    do {
        double d;
        memcpy(&d, &old, 8);
        d += v;
        memcpy(&nw, &d, 8);
    } while (!__atomic_compare_exchange_n(p, &old, nw, 1, __ATOMIC_RELAXED,
                                          __ATOMIC_RELAXED));
}

static void add_u32(uint32_t *dst, int shared) {
    if (shared) {
        __atomic_fetch_add(dst, 1u, __ATOMIC_RELAXED);
    } else {
        *dst += 1u;
    }
}

static void add_u64(uint64_t *dst, int shared) {
    if (shared) {
        __atomic_fetch_add(dst, 1u, __ATOMIC_RELAXED);
    } else {
        *dst += 1u;
    }
}

/* one fp32 contribution c to gradient element i, with |c| and count */
static void grad_add(double *g, double *a, uint32_t *k, uint64_t i, float c,
                     int shared) {
    add_f64(&g[i], (double)c, shared);
    if (a) add_f64(&a[i], fabs((double)c), shared);
    if (k) add_u32(&k[i], shared);
}

/* ------------------------------------------------------------------------ */
/* SH (src/tracing/sh_utils.cuh:8-92)                                        */

static const float SH_C0 = 0.28209479177387814f;
static const float SH_C1 = 0.4886025119029199f;
static const float SH_C2[5] = {1.0925484305920792f, -1.0925484305920792f,
                               0.31539156525252005f, -1.0925484305920792f,
                               0.5462742152960396f};
static const float SH_C3[7] = {-0.5900435899266435f, 2.890611442640554f,
                               -0.4570457994644658f, 0.3731763325901154f,
                               -0.4570457994644658f, 1.445305721320277f,
                               -0.5900435899266435f};

/* sh_coefficients<degree> (src/tracing/sh_utils.cuh:25-62); unused slots 0 */
void oracle_sh_basis(uint32_t degree, float x, float y, float z,
                     float *sh) {
    for (int i = 0; i < 16; ++i) sh[i] = 0.0f;
    sh[0] = SH_C0;
    if (degree > 0) {
        sh[1] = -SH_C1 * y;
        sh[2] = SH_C1 * z;
        sh[3] = -SH_C1 * x;
    }
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, yz = y * z, xz = x * z;
    if (degree > 1) {
        sh[4] = SH_C2[0] * xy;
        sh[5] = SH_C2[1] * yz;
        sh[6] = SH_C2[2] * (2.0f * zz - xx - yy);
        sh[7] = SH_C2[3] * xz;
        sh[8] = SH_C2[4] * (xx - yy);
    }
    if (degree > 2) {
        sh[9] = SH_C3[0] * y * (3.0f * xx - yy);
        sh[10] = SH_C3[1] * xy * z;
        sh[11] = SH_C3[2] * y * (4.0f * zz - xx - yy);
        sh[12] = SH_C3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
        sh[13] = SH_C3[4] * x * (4.0f * zz - xx - yy);
        sh[14] = SH_C3[5] * z * (xx - yy);
        sh[15] = SH_C3[6] * x * (xx - 3.0f * yy);
    }
}

/* load_sh_as_rgb (src/tracing/sh_utils.cuh:64-75):
 * rgb = max(0, 0.5 + sum_i Y[i/3] * v[i]) in channel i % 3 */
static void sh_rgb(const float *sh, const float *v, uint32_t nsh, float *rgb) {
    float r[3] = {0.5f, 0.5f, 0.5f};
    for (uint32_t i = 0; i < 3 * nsh; ++i) {
        r[i % 3] = fmaf(sh[i / 3], v[i], r[i % 3]);
    }
    for (int c = 0; c < 3; ++c) rgb[c] = fmaxf(r[c], 0.0f);
}

/* ------------------------------------------------------------------------ */
/* prefetch_adjacent_diff (src/tracing/pipeline.cu:1202-1242)                */

void oracle_prefetch_adjacent_diff(const float *points, uint32_t num_points,
                                   uint32_t adjacency_size,
                                   const uint32_t *adjacency,
                                   const uint32_t *offsets, uint16_t *diff) {
    for (uint32_t i = 0; i < num_points; ++i) {
        const float *p = points + 3ull * i;
        const uint32_t beg = offsets[i], end = offsets[i + 1];
        for (uint32_t j = beg; j < end && j < adjacency_size; ++j) {
            const uint32_t a = adjacency[j];
            uint16_t *o = diff + 4ull * j;
            if (a >= num_points) {
                /* out-of-range neighbour: a NaN plane never qualifies */
                o[0] = o[1] = o[2] = 0x7e00u;
                o[3] = 0;
                continue;
            }
            const float *q = points + 3ull * a;
            o[0] = sdf_f32_to_f16_bits(q[0] - p[0]);
            o[1] = sdf_f32_to_f16_bits(q[1] - p[1]);
            o[2] = sdf_f32_to_f16_bits(q[2] - p[2]);
            o[3] = 0;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* the walk (src/tracing/tracing_utils.cuh:15-109)                           */

typedef struct {
    float o[3]; /* origin */
    float d[3]; /* unit direction */
} ray_t;

/* ray.direction /= ray.direction.norm()  (src/tracing/pipeline.cu:76-77) */
static ray_t load_ray(const float *r) {
    ray_t ray;
    for (int i = 0; i < 3; ++i) ray.o[i] = r[i];
    const float n = sqrtf(sdf_dot3(r[3], r[4], r[5], r[3], r[4], r[5]));
    for (int i = 0; i < 3; ++i) ray.d[i] = r[3 + i] / n;
    return ray;
}

typedef struct {
    const float *points;
    const uint32_t *adjacency;
    const uint32_t *offsets;
    const uint16_t *diff;
    uint32_t num_points;
    uint32_t adjacency_size;
} scene_t;

/* one cell step: returns nonzero to keep walking */
typedef int (*step_fn)(void *ctx, uint32_t cell, uint32_t next, float t0,
                       float t1, const float *x_cell, const float *x_next);

typedef struct {
    uint32_t n;             /* loop iterations (num_intersections) */
    uint32_t steps;         /* functor calls */
    uint64_t faces;         /* faces scanned */
    uint64_t faces_stepped; /* faces of stepped cells */
} walk_stats;

/* The reference passes num_points = point_adjacency_size = UINT32_MAX to the
 * walk (src/tracing/pipeline.cu:241-249); here the real sizes are passed so a
 * malformed scene ends the walk instead of reading out of bounds.  For a
 * well-formed scene the two are the same walk. */
static walk_stats walk(const scene_t *sc, const ray_t *ray, uint32_t start,
                       uint32_t max_steps, int safe_mode, step_fn fn,
                       void *ctx) {
    walk_stats st = {0, 0, 0, 0};
    float t0 = 0.0f;
    uint32_t cell = start;
    if (cell >= sc->num_points) return st;
    float xc[3] = {sc->points[3ull * cell], sc->points[3ull * cell + 1],
                   sc->points[3ull * cell + 2]};
    for (;;) {
        ++st.n;
        if (st.n > max_steps) break;
        const uint32_t beg = sc->offsets[cell];
        const uint32_t end = sc->offsets[cell + 1];
        if (beg > end || end > sc->adjacency_size) break;
        const uint32_t nf = end - beg;
        st.faces += nf;
        float t1 = sdf_bits_f32(0x7f800000u);
        uint32_t best = UINT32_MAX;
        for (uint32_t k = 0; k < nf; ++k) {
            const uint16_t *h = sc->diff + 4ull * (beg + k);
            const float dx = sdf_f16_bits_to_f32(h[0]);
            const float dy = sdf_f16_bits_to_f32(h[1]);
            const float dz = sdf_f16_bits_to_f32(h[2]);
            const float fx = xc[0] + dx * 0.5f;
            const float fy = xc[1] + dy * 0.5f;
            const float fz = xc[2] + dz * 0.5f;
            const float dp = sdf_dot3(dx, dy, dz, ray->d[0], ray->d[1], ray->d[2]);
            const float t = sdf_dot3(fx - ray->o[0], fy - ray->o[1],
                                     fz - ray->o[2], dx, dy, dz) / dp;
            if (safe_mode) {
                if (dp > 0.0f && t > t0 && t < t1) {
                    t1 = t;
                    best = k;
                }
            } else {
                if (dp > 0.0f && t < t1) {
                    t1 = t;
                    best = k;
                }
            }
        }
        if (best == UINT32_MAX) break;
        const uint32_t next = sc->adjacency[beg + best];
        if (next >= sc->num_points) break;
        const float xn[3] = {sc->points[3ull * next], sc->points[3ull * next + 1],
                             sc->points[3ull * next + 2]};
        if (t1 > t0) {
            ++st.steps;
            st.faces_stepped += nf;
            if (!fn(ctx, cell, next, t0, t1, xc, xn)) break;
        }
        t0 = fmaxf(t0, t1);
        cell = next;
        xc[0] = xn[0];
        xc[1] = xn[1];
        xc[2] = xn[2];
    }
    return st;
}

/* visit recording shared by forward and backward */
typedef struct {
    oracle_visits *v;
    uint64_t ray;
    uint64_t hash;
    uint32_t count;
} visit_rec;

static void visit_push(visit_rec *vr, uint32_t cell, float alpha, float t1) {
    vr->hash ^= (uint64_t)cell;
    vr->hash *= 0x100000001b3ull;
    if (vr->v && vr->v->point_visits)
        __atomic_fetch_add(&vr->v->point_visits[cell], 1u, __ATOMIC_RELAXED);
    if (vr->v && vr->count < vr->v->stride) {
        if (vr->v->cells) vr->v->cells[vr->ray * vr->v->stride + vr->count] = cell;
        if (vr->v->alphas) vr->v->alphas[vr->ray * vr->v->stride + vr->count] = alpha;
        if (vr->v->t_exit) vr->v->t_exit[vr->ray * vr->v->stride + vr->count] = t1;
    }
    vr->count++;
}

static void visit_finish(visit_rec *vr, const walk_stats *st) {
    if (!vr->v) return;
    if (vr->v->hash) vr->v->hash[vr->ray] = vr->hash;
    if (vr->v->steps) vr->v->steps[vr->ray] = st->steps;
    if (vr->v->faces) vr->v->faces[vr->ray] = st->faces;
    if (vr->v->faces_stepped) vr->v->faces_stepped[vr->ray] = st->faces_stepped;
}

#define FNV_OFFSET 0xcbf29ce484222325ull

/* ------------------------------------------------------------------------ */
/* threading                                                                 */

typedef void (*ray_range_fn)(void *job, uint32_t lo, uint32_t hi);

typedef struct {
    ray_range_fn fn;
    void *job;
    uint32_t lo, hi;
} thread_arg;

static void *thread_main(void *p) {
    thread_arg *a = (thread_arg *)p;
    a->fn(a->job, a->lo, a->hi);
    return NULL;
}

static void run_rays(ray_range_fn fn, void *job, uint32_t num_rays,
                     int num_threads) {
    if (num_threads <= 1 || num_rays < 64) {
        fn(job, 0, num_rays);
        return;
    }
    if (num_threads > 256) num_threads = 256;
    pthread_t th[256];
    thread_arg args[256];
    /* interleaved blocks of 256 rays keep the per-thread work balanced */
    const uint32_t chunk = (num_rays + (uint32_t)num_threads - 1) / (uint32_t)num_threads;
    int started = 0;
    for (int t = 0; t < num_threads; ++t) {
        uint32_t lo = (uint32_t)t * chunk;
        uint32_t hi = lo + chunk > num_rays ? num_rays : lo + chunk;
        if (lo >= hi) break;
        args[t].fn = fn;
        args[t].job = job;
        args[t].lo = lo;
        args[t].hi = hi;
        if (pthread_create(&th[t], NULL, thread_main, &args[t]) != 0) {
            fn(job, lo, hi);
            args[t].fn = NULL;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t) {
        if (args[t].fn) pthread_join(th[t], NULL);
    }
}

/* ------------------------------------------------------------------------ */
/* forward (src/tracing/pipeline.cu:36-264)                                  */

typedef struct {
    const oracle_settings *st;
    uint32_t sh_degree, nsh, D;
    scene_t sc;
    const float *attributes;
    const float *rays;
    const uint32_t *start;
    uint32_t Q;
    const float *quantiles;
    float sharp;
    float *rgba, *depth;
    uint32_t *depth_indices, *num_isect;
    double *contribution;
    float *alpha_out;
    oracle_visits *visits;
    int shared;
} fwd_job;

typedef struct {
    const fwd_job *job;
    uint32_t ray;
    float sh[16];
    float T;
    float C[3];
    uint32_t qi;
    float q;
    const float *rq;
    visit_rec vr;
} fwd_ray;

static int fwd_step(void *ctx, uint32_t cell, uint32_t next, float t0,
                    float t1, const float *xc, const float *xn) {
    (void)next;
    (void)xc;
    (void)xn;
    fwd_ray *r = (fwd_ray *)ctx;
    const fwd_job *j = r->job;
    const float *a = j->attributes + (uint64_t)cell * j->D;
    const int neus = j->st->alpha_mode == ORACLE_ALPHA_NEUS;
    /* load_attributes (pipeline.cu:86-101): colour gated on the last scalar
     * only in standard mode */
    float s = a[j->D - 1];
    float rgb[3];
    if (neus || s > 1e-6f) {
        sh_rgb(r->sh, a, j->nsh, rgb);
    } else {
        rgb[0] = rgb[1] = rgb[2] = 0.0f;
    }
    float alpha;
    if (neus && j->st->sdf_channel >= 0) {
        /* pipeline.cu:129-152 */
        const float d = a[j->st->sdf_channel];
        const float sha = j->sharp;
        const float phi = sdf_sigmoidf(-sha * d);
        s = sha * phi * (1.0f - phi);
        const float dt = fmaxf(t1 - t0, 0.0f);
        alpha = 1.0f - sdf_expf(-s * dt);
    } else {
        const float dt = fmaxf(t1 - t0, 0.0f);
        alpha = 1.0f - sdf_expf(-s * dt);
    }
    const float w = r->T * alpha;
    if (j->alpha_out) {
        /* racy last-writer store in the reference (pipeline.cu:159) */
        uint32_t bits = sdf_f32_bits(alpha);
        __atomic_store_n((uint32_t *)&j->alpha_out[cell], bits, __ATOMIC_RELAXED);
    }
    if (j->contribution) add_f64(&j->contribution[cell], (double)w, j->shared);
    for (int c = 0; c < 3; ++c) r->C[c] = fmaf(w, rgb[c], r->C[c]);
    const float Tn = r->T * (1.0f - alpha);
    const uint64_t qbase = (uint64_t)r->ray * j->Q;
    if (neus) {
        /* linearised-T crossing (pipeline.cu:189-216) */
        const float drop = r->T - Tn;
        if (drop > 1e-12f) {
            while (r->qi < j->Q && Tn < r->q) {
                float frac = (r->T - r->q) / drop;
                frac = fminf(1.0f, fmaxf(0.0f, frac));
                const float tq = fmaf(frac, t1 - t0, t0);
                j->depth[qbase + r->qi] = tq;
                j->depth_indices[qbase + r->qi] = cell;
                ++r->qi;
                if (r->qi < j->Q) r->q = r->rq[r->qi];
            }
        }
    } else {
        /* analytic crossing (pipeline.cu:217-230) */
        while (r->qi < j->Q && Tn < r->q) {
            j->depth[qbase + r->qi] = t0 + logf(r->T / r->q) / s;
            j->depth_indices[qbase + r->qi] = cell;
            ++r->qi;
            if (r->qi < j->Q) r->q = r->rq[r->qi];
        }
    }
    visit_push(&r->vr, cell, alpha, t1);
    r->T = Tn;
    return r->T > j->st->weight_threshold;
}

static void fwd_range(void *p, uint32_t lo, uint32_t hi) {
    const fwd_job *j = (const fwd_job *)p;
    for (uint32_t i = lo; i < hi; ++i) {
        fwd_ray r;
        memset(&r, 0, sizeof(r));
        r.job = j;
        r.ray = i;
        const ray_t ray = load_ray(j->rays + 6ull * i);
        oracle_sh_basis(j->sh_degree, ray.d[0], ray.d[1], ray.d[2], r.sh);
        r.T = 1.0f;
        r.rq = j->quantiles ? j->quantiles + (uint64_t)i * j->Q : NULL;
        r.q = (r.rq && j->Q > 0) ? r.rq[0] : 0.0f;
        r.vr.v = j->visits;
        r.vr.ray = i;
        r.vr.hash = FNV_OFFSET;
        const walk_stats st = walk(&j->sc, &ray, j->start[i],
                                   j->st->max_intersections, 1, fwd_step, &r);
        for (uint32_t q = r.qi; q < j->Q; ++q) {
            j->depth[(uint64_t)i * j->Q + q] = -1.0f;
            j->depth_indices[(uint64_t)i * j->Q + q] = UINT32_MAX;
        }
        for (int c = 0; c < 3; ++c) j->rgba[4ull * i + c] = r.C[c];
        j->rgba[4ull * i + 3] = 1.0f - r.T;
        if (j->num_isect) j->num_isect[i] = st.n;
        visit_finish(&r.vr, &st);
    }
}

static uint16_t *make_diff(const float *points, uint32_t num_points,
                           uint32_t adjacency_size, const uint32_t *adjacency,
                           const uint32_t *offsets) {
    uint16_t *diff = (uint16_t *)calloc((size_t)adjacency_size + 1, 8);
    if (!diff) return NULL;
    oracle_prefetch_adjacent_diff(points, num_points, adjacency_size, adjacency,
                                  offsets, diff);
    return diff;
}

int oracle_trace_forward(const oracle_settings *settings, uint32_t sh_degree,
                         uint32_t num_points, const float *points,
                         const float *attributes, uint32_t adjacency_size,
                         const uint32_t *adjacency, const uint32_t *offsets,
                         uint32_t num_rays, const float *rays,
                         const uint32_t *start_point, uint32_t num_quantiles,
                         const float *quantiles, const float *sharpness,
                         float *rgba, float *depth, uint32_t *depth_indices,
                         uint32_t *num_intersections, double *contribution,
                         float *alpha_out, oracle_visits *visits,
                         int num_threads) {
    if (sh_degree > 3 || !settings) return -1;
    if (num_quantiles > 0 && (!quantiles || !depth || !depth_indices)) return -1;
    fwd_job j;
    memset(&j, 0, sizeof(j));
    j.st = settings;
    j.sh_degree = sh_degree;
    j.nsh = (sh_degree + 1) * (sh_degree + 1);
    j.D = 1 + 3 * j.nsh;
    j.sc.points = points;
    j.sc.adjacency = adjacency;
    j.sc.offsets = offsets;
    j.sc.num_points = num_points;
    j.sc.adjacency_size = adjacency_size;
    j.sc.diff = make_diff(points, num_points, adjacency_size, adjacency, offsets);
    if (!j.sc.diff) return -1;
    j.attributes = attributes;
    j.rays = rays;
    j.start = start_point;
    j.Q = num_quantiles;
    j.quantiles = quantiles;
    j.sharp = sharpness ? sharpness[0] : 1.0f;
    j.rgba = rgba;
    j.depth = depth;
    j.depth_indices = depth_indices;
    j.num_isect = num_intersections;
    j.contribution = contribution;
    j.alpha_out = alpha_out;
    j.visits = visits;
    j.shared = num_threads > 1;
    run_rays(fwd_range, &j, num_rays, num_threads);
    free((void *)j.sc.diff);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* inference render (src/tracing/pipeline.cu:1067-1199, the `benchmark`      */
/* kernel behind Pipeline::trace_benchmark)                                  */

typedef struct {
    fwd_job fj;
    const oracle_camera *cam;
    float focal;
    float bg[3];
    int checker_bg;
    uint32_t *out;
    float *rgbt;  /* optional [H*W, 4]: C, T per pixel, in pixel order j * W + i */
    uint32_t *num_isect_px; /* optional [H*W] */
} bench_job;

static void bench_range(void *p, uint32_t lo, uint32_t hi) {
    const bench_job *b = (const bench_job *)p;
    const oracle_camera *cam = b->cam;
    for (uint32_t px = lo; px < hi; ++px) {
        const uint32_t i = px % cam->width, jj = px / cam->width;
        const uint32_t out_idx = (cam->height - 1 - jj) * cam->width + i;
        float dir[3];
        sdf_cast_ray(cam->forward, cam->right, cam->up, cam->fov, b->focal, cam->width,
                     cam->height, cam->model, i, jj, dir);
        const float n = sqrtf(sdf_dot3(dir[0], dir[1], dir[2], dir[0], dir[1], dir[2]));
        if (n < 0.1f) {
            /* masked fisheye pixel: the settings' background colour */
            b->out[out_idx] = sdf_make_rgba8(b->bg[0], b->bg[1], b->bg[2], 1.0f);
            if (b->rgbt) for (int c = 0; c < 4; ++c) b->rgbt[4ull * px + c] = -1.0f;
            if (b->num_isect_px) b->num_isect_px[px] = 0;
            continue;
        }
        const float r6[6] = {cam->position[0], cam->position[1], cam->position[2],
                             dir[0], dir[1], dir[2]};
        const ray_t ray = load_ray(r6); /* ray.direction /= ray.direction.norm() */
        fwd_ray r;
        memset(&r, 0, sizeof(r));
        r.job = &b->fj;
        r.ray = px;
        oracle_sh_basis(b->fj.sh_degree, ray.d[0], ray.d[1], ray.d[2], r.sh);
        r.T = 1.0f;
        /* the benchmark functor is the forward's step without its outputs
         * (no alpha / contribution / quantiles: those pointers are NULL) */
        const walk_stats st = walk(&b->fj.sc, &ray, b->fj.start[0],
                                   b->fj.st->max_intersections, 1, fwd_step, &r);
        float bg[3] = {b->bg[0], b->bg[1], b->bg[2]};
        if (b->checker_bg) {
            const int is = 2 * (int)((i / 20) % 2) - 1;
            const int js = 2 * (int)((jj / 20) % 2) - 1;
            const float g = (is * js > 0) ? 0.3f : 0.5f;
            bg[0] = bg[1] = bg[2] = g;
        }
        float col[3];
        for (int c = 0; c < 3; ++c) col[c] = fmaf(r.T, bg[c], r.C[c]);
        b->out[out_idx] = sdf_make_rgba8(col[0], col[1], col[2], 1.0f);
        if (b->rgbt) {
            for (int c = 0; c < 3; ++c) b->rgbt[4ull * px + c] = r.C[c];
            b->rgbt[4ull * px + 3] = r.T;
        }
        if (b->num_isect_px) b->num_isect_px[px] = st.n;
    }
}

float oracle_camera_focal(float fov) { return 1.0f / tanf(fov * 0.5f); }

void oracle_cast_ray(const oracle_camera *cam, uint32_t i, uint32_t j, float *dir) {
    sdf_cast_ray(cam->forward, cam->right, cam->up, cam->fov, oracle_camera_focal(cam->fov),
                 cam->width, cam->height, cam->model, i, j, dir);
}

void oracle_sincosf_n(const float *x, float *s, float *c, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) sdf_sincosf(x[i], &s[i], &c[i]);
}

void oracle_atan2f_n(const float *y, const float *x, float *out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = sdf_atan2f(y[i], x[i]);
}

uint32_t oracle_make_rgba8(float r, float g, float b, float a) {
    return sdf_make_rgba8(r, g, b, a);
}

int oracle_trace_benchmark(const oracle_settings *settings, uint32_t sh_degree,
                           uint32_t num_points, const float *points,
                           const float *attributes, uint32_t adjacency_size,
                           const uint32_t *adjacency, const uint32_t *offsets,
                           const uint16_t *adjacent_diff, const oracle_camera *camera,
                           uint32_t start_point, const float *sharpness,
                           const float *bg_color, int checker_bg, uint32_t *output_rgba,
                           float *rgbt, uint32_t *num_intersections, int num_threads) {
    if (sh_degree > 3 || !settings || !camera || !output_rgba || !adjacent_diff) return -1;
    if (camera->width == 0 || camera->height == 0) return -1;
    bench_job b;
    memset(&b, 0, sizeof(b));
    fwd_job *j = &b.fj;
    j->st = settings;
    j->sh_degree = sh_degree;
    j->nsh = (sh_degree + 1) * (sh_degree + 1);
    j->D = 1 + 3 * j->nsh;
    j->sc.points = points;
    j->sc.adjacency = adjacency;
    j->sc.offsets = offsets;
    j->sc.num_points = num_points;
    j->sc.adjacency_size = adjacency_size;
    j->sc.diff = adjacent_diff;
    j->attributes = attributes;
    j->start = &start_point;
    j->sharp = sharpness ? sharpness[0] : 1.0f;
    b.cam = camera;
    b.focal = oracle_camera_focal(camera->fov);
    /* default_visualization_settings (src/tracing/pipeline.h:59-68): white */
    for (int c = 0; c < 3; ++c) b.bg[c] = bg_color ? bg_color[c] : 1.0f;
    b.checker_bg = checker_bg;
    b.out = output_rgba;
    b.rgbt = rgbt;
    b.num_isect_px = num_intersections;
    run_rays(bench_range, &b, camera->width * camera->height, num_threads);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* backward                                                                  */

/* cell_intersection_grad (src/tracing/tracing_utils.cuh:112-124):
 * d t / d p for the bisector plane between p and q, fp32 positions */
static void cell_isect_grad(const float *p, const float *q, const ray_t *ray,
                            float *g) {
    const float fo[3] = {(p[0] + q[0]) / 2.0f, (p[1] + q[1]) / 2.0f,
                         (p[2] + q[2]) / 2.0f};
    const float fn[3] = {q[0] - p[0], q[1] - p[1], q[2] - p[2]};
    const float num = sdf_dot3(fo[0] - ray->o[0], fo[1] - ray->o[1],
                               fo[2] - ray->o[2], fn[0], fn[1], fn[2]);
    const float dp = sdf_dot3(fn[0], fn[1], fn[2], ray->d[0], ray->d[1], ray->d[2]);
    const float dp2 = dp * dp;
    for (int i = 0; i < 3; ++i) {
        const float v = num * ray->d[i] + dp * (ray->o[i] - p[i]);
        g[i] = v / dp2;
    }
}

/* exported for the tests: origin o, unit direction d */
void oracle_cell_intersection_grad(const float *p, const float *q, const float *o,
                                   const float *d, float *g) {
    ray_t ray;
    for (int i = 0; i < 3; ++i) {
        ray.o[i] = o[i];
        ray.d[i] = d[i];
    }
    cell_isect_grad(p, q, &ray, g);
}

typedef struct {
    const oracle_settings *st;
    uint32_t sh_degree, nsh, D;
    scene_t sc;
    const float *attributes;
    const float *rays;
    const uint32_t *start;
    uint32_t Q;
    const float *quantiles;
    const uint32_t *depth_indices;
    const float *rgba, *grad_rgba, *depth_grad, *ray_error;
    float sharp;
    int has_sharpness_grad;
    oracle_grads *g;
    oracle_visits *visits;
    int shared;
} bwd_job;

typedef struct {
    const bwd_job *job;
    uint32_t ray;
    ray_t r;
    float sh[16];
    float g4[4], rgba4[4];
    float err;
    float T;
    float C[3];
    uint32_t qi;
    float q;
    const float *rq, *rdg;
    float g_logT;           /* sdf mode */
    float cur_depth_grad;   /* density mode */
    uint32_t prev_idx;
    float prev_pt[3];
    float prev_grad[3], cur_grad[3], next_grad[3];
    visit_rec vr;
} bwd_ray;

/* geometry bookkeeping shared by both modes
 * (pipeline.cu:452-474 sdf, :731-760 density), quirks A-1 and A-2 included */
static void bwd_geometry(bwd_ray *r, uint32_t cell, const float *xc,
                         const float *xn, float dL_dt0, float dL_dt1) {
    const bwd_job *j = r->job;
    float dprev[3] = {0.0f, 0.0f, 0.0f};
    if (r->prev_idx != UINT32_MAX) cell_isect_grad(r->prev_pt, xc, &r->r, dprev);
    float dt1_cur[3], dt0_cur[3], dt1_next[3];
    cell_isect_grad(xc, xn, &r->r, dt1_cur);
    cell_isect_grad(xc, r->prev_pt, &r->r, dt0_cur); /* prev_pt = 0 at first (A-1) */
    cell_isect_grad(xn, xc, &r->r, dt1_next);
    for (int i = 0; i < 3; ++i) {
        r->prev_grad[i] = fmaf(dL_dt0, dprev[i], r->prev_grad[i]);
        r->cur_grad[i] = r->cur_grad[i] + (dL_dt0 * dt0_cur[i] + dL_dt1 * dt1_cur[i]);
        r->next_grad[i] = fmaf(dL_dt1, dt1_next[i], r->next_grad[i]);
    }
    if (r->prev_idx != UINT32_MAX) {
        for (int i = 0; i < 3; ++i) {
            grad_add(j->g->points_grad, j->g->points_grad_abs, j->g->points_grad_k,
                     3ull * r->prev_idx + i, r->prev_grad[i], j->shared);
        }
    }
    for (int i = 0; i < 3; ++i) {
        r->prev_pt[i] = xc[i];
        r->prev_grad[i] = r->cur_grad[i];
        r->cur_grad[i] = r->next_grad[i];
        r->next_grad[i] = 0.0f;
    }
    r->prev_idx = cell;
}

/* SH colour grads, zeroed where the colour clamped to 0
 * (pipeline.cu:528-533 / :763-772; sh_utils.cuh:85-92) */
static void bwd_sh(bwd_ray *r, uint32_t cell, const float *rgb, float *dL_drgb) {
    const bwd_job *j = r->job;
    for (int c = 0; c < 3; ++c) {
        if (rgb[c] == 0.0f) dL_drgb[c] = 0.0f;
    }
    const uint64_t base = (uint64_t)cell * j->D;
    for (uint32_t i = 0; i < 3 * j->nsh; ++i) {
        grad_add(j->g->attr_grad, j->g->attr_grad_abs, j->g->attr_grad_k, base + i,
                 r->sh[i / 3] * dL_drgb[i % 3], j->shared);
    }
}

/* backward_sdf functor (src/tracing/pipeline.cu:363-537) */
static int bwd_step_sdf(void *ctx, uint32_t cell, uint32_t next, float t0,
                        float t1, const float *xc, const float *xn) {
    (void)next;
    bwd_ray *r = (bwd_ray *)ctx;
    const bwd_job *j = r->job;
    const float *a = j->attributes + (uint64_t)cell * j->D;
    float rgb[3];
    sh_rgb(r->sh, a, j->nsh, rgb);
    const float dt = fmaxf(t1 - t0, 0.0f);
    const int sdf_ch = j->st->sdf_channel >= 0 ? j->st->sdf_channel : (int)j->D - 1;
    const float d = a[sdf_ch];
    const float sha = j->sharp;
    const float phi = sdf_sigmoidf(-sha * d);
    const float s = sha * phi * (1.0f - phi);
    const float alpha = 1.0f - sdf_expf(-s * dt);
    const float w = r->T * alpha;
    for (int c = 0; c < 3; ++c) r->C[c] = fmaf(w, rgb[c], r->C[c]);
    if (j->g->point_error) add_f64(&j->g->point_error[cell], (double)(w * r->err), j->shared);

    float dL_drgb[3] = {r->g4[0] * w, r->g4[1] * w, r->g4[2] * w};
    const float den = r->T * (1.0f - alpha) + 1e-6f;
    float rest[3];
    for (int c = 0; c < 3; ++c) rest[c] = (r->rgba4[c] - r->C[c]) / den;
    /* 0 + T * dot is T * dot */
    float dL_dalpha = r->T * sdf_dot3(rgb[0] - rest[0], rgb[1] - rest[1],
                                      rgb[2] - rest[2], r->g4[0], r->g4[1], r->g4[2]);
    dL_dalpha = dL_dalpha + (1.0f - r->rgba4[3]) * r->g4[3] / (1.0f - alpha + 1e-6f);
    dL_dalpha = dL_dalpha + -r->g_logT / fmaxf(1.0f - alpha, 1e-12f);

    const float oma = 1.0f - alpha;
    const float dalpha_ds = dt * oma;
    const float dalpha_ddelta = s * oma;
    const float dL_ds = dL_dalpha * dalpha_ds;
    float dL_ddelta = dL_dalpha * dalpha_ddelta;
    const float Tn = r->T * (1.0f - alpha);

    float dL_dt0_units = 0.0f;
    if (r->rq && j->Q > 0) {
        const float T0 = r->T;
        const float drop = T0 - Tn;
        if (drop > 1e-12f) {
            while (r->qi < j->Q && Tn < r->q) {
                const float q = r->q;
                const float gq = r->rdg[r->qi];
                float frac = (T0 - q) / drop;
                frac = fminf(1.0f, fmaxf(0.0f, frac));
                dL_dt0_units = dL_dt0_units + gq;
                dL_ddelta = fmaf(gq, frac, dL_ddelta);
                /* dL_dalpha update here is a dead store (A-13) */
                if (alpha > 1e-12f && T0 > 1e-20f) {
                    r->g_logT = fmaf(gq, dt * q / (alpha * T0), r->g_logT);
                }
                ++r->qi;
                if (r->qi < j->Q) r->q = r->rq[r->qi];
            }
        }
    }
    const float dL_dt0 = dL_dt0_units - dL_ddelta;
    const float dL_dt1 = dL_ddelta;
    bwd_geometry(r, cell, xc, xn, dL_dt0, dL_dt1);

    const float dphi_dd = -sha * phi * (1.0f - phi);
    const float ds_dd = sha * (1.0f - 2.0f * phi) * dphi_dd;
    const float ds_dsha = phi * (1.0f - phi) * (1.0f - sha * d * (1.0f - 2.0f * phi));
    const float dL_dd = dL_ds * ds_dd;
    if (j->st->sdf_channel >= 0) {
        grad_add(j->g->attr_grad, j->g->attr_grad_abs, j->g->attr_grad_k,
                 (uint64_t)cell * j->D + sdf_ch, dL_dd, j->shared);
    }
    if (j->has_sharpness_grad) {
        grad_add(j->g->sharpness_grad, j->g->sharpness_abs, NULL, 0, dL_ds * ds_dsha,
                 j->shared);
        if (j->g->sharpness_k) add_u64(j->g->sharpness_k, j->shared);
    }
    bwd_sh(r, cell, rgb, dL_drgb);
    visit_push(&r->vr, cell, alpha, t1);
    r->T = Tn;
    return r->T > j->st->weight_threshold;
}

/* backward (density) functor (src/tracing/pipeline.cu:646-778) */
static int bwd_step_density(void *ctx, uint32_t cell, uint32_t next, float t0,
                            float t1, const float *xc, const float *xn) {
    (void)next;
    bwd_ray *r = (bwd_ray *)ctx;
    const bwd_job *j = r->job;
    const float *a = j->attributes + (uint64_t)cell * j->D;
    const float s = a[j->D - 1];
    float rgb[3];
    if (s > 1e-6f) {
        sh_rgb(r->sh, a, j->nsh, rgb);
    } else {
        rgb[0] = rgb[1] = rgb[2] = 0.0f;
    }
    const float dt = fmaxf(t1 - t0, 0.0f);
    const float alpha = 1.0f - sdf_expf(-s * dt);
    const float w = r->T * alpha;
    const float dalpha_ds = dt * (1.0f - alpha);
    float dalpha_ddt = 0.0f;
    if (dt > 0.0f) dalpha_ddt = s * (1.0f - alpha);
    for (int c = 0; c < 3; ++c) r->C[c] = fmaf(w, rgb[c], r->C[c]);
    if (j->g->point_error) add_f64(&j->g->point_error[cell], (double)(w * r->err), j->shared);

    float dL_drgb[3] = {r->g4[0] * w, r->g4[1] * w, r->g4[2] * w};
    const float den = r->T * (1.0f - alpha + 1e-6f); /* A-12 */
    float rest[3];
    for (int c = 0; c < 3; ++c) rest[c] = (r->rgba4[c] - r->C[c]) / den;
    float dL_dalpha = r->T * sdf_dot3(rgb[0] - rest[0], rgb[1] - rest[1],
                                      rgb[2] - rest[2], r->g4[0], r->g4[1], r->g4[2]);
    dL_dalpha = dL_dalpha + (1.0f - r->rgba4[3]) * r->g4[3] / (1.0f - alpha + 1e-6f);
    float dL_ds = dL_dalpha * dalpha_ds;
    float dL_ddt = dL_dalpha * dalpha_ddt;
    float dL_dt0 = 0.0f;
    const float Tn = r->T * (1.0f - alpha);
    while (r->qi < j->Q && Tn < r->q) {
        const float dgi = r->rdg[r->qi] / s;
        dL_dt0 = dL_dt0 + dgi;
        dL_ds = dL_ds + -dgi * logf(r->T / r->q) / s;
        r->cur_depth_grad = r->cur_depth_grad - dgi;
        ++r->qi;
        if (r->qi < j->Q) r->q = r->rq[r->qi];
    }
    if (r->qi < j->Q) {
        dL_ds = fmaf(-dt, r->cur_depth_grad, dL_ds);
        dL_ddt = fmaf(-s, r->cur_depth_grad, dL_ddt);
    }
    dL_dt0 = dL_dt0 + -dL_ddt;
    const float dL_dt1 = dL_ddt;
    bwd_geometry(r, cell, xc, xn, dL_dt0, dL_dt1);
    visit_push(&r->vr, cell, alpha, t1);
    r->T = Tn;
    bwd_sh(r, cell, rgb, dL_drgb);
    grad_add(j->g->attr_grad, j->g->attr_grad_abs, j->g->attr_grad_k,
             (uint64_t)cell * j->D + (j->D - 1), dL_ds, j->shared);
    return r->T > j->st->weight_threshold;
}

static void bwd_range(void *p, uint32_t lo, uint32_t hi) {
    const bwd_job *j = (const bwd_job *)p;
    const int neus = j->st->alpha_mode == ORACLE_ALPHA_NEUS;
    for (uint32_t i = lo; i < hi; ++i) {
        bwd_ray r;
        memset(&r, 0, sizeof(r));
        r.job = j;
        r.ray = i;
        r.r = load_ray(j->rays + 6ull * i);
        oracle_sh_basis(j->sh_degree, r.r.d[0], r.r.d[1], r.r.d[2], r.sh);
        for (int c = 0; c < 4; ++c) {
            r.g4[c] = j->grad_rgba[4ull * i + c];
            r.rgba4[c] = j->rgba[4ull * i + c];
        }
        r.err = j->ray_error ? j->ray_error[i] : 0.0f;
        r.T = 1.0f;
        r.rq = j->quantiles ? j->quantiles + (uint64_t)i * j->Q : NULL;
        r.rdg = j->depth_grad ? j->depth_grad + (uint64_t)i * j->Q : NULL;
        r.q = (r.rq && j->Q > 0) ? r.rq[0] : 0.0f;
        r.prev_idx = UINT32_MAX;
        r.vr.v = j->visits;
        r.vr.ray = i;
        r.vr.hash = FNV_OFFSET;
        if (!neus) {
            /* pipeline.cu:620-629 */
            for (uint32_t q = 0; q < j->Q; ++q) {
                const uint32_t pi = j->depth_indices[(uint64_t)i * j->Q + q];
                if (pi != UINT32_MAX) {
                    const float sd = j->attributes[(uint64_t)pi * j->D + j->D - 1];
                    r.cur_depth_grad = r.cur_depth_grad + r.rdg[q] / sd;
                }
            }
        }
        const walk_stats st =
            walk(&j->sc, &r.r, j->start[i], j->st->max_intersections, neus ? 1 : 0,
                 neus ? bwd_step_sdf : bwd_step_density, &r);
        visit_finish(&r.vr, &st);
    }
}

int oracle_trace_backward(const oracle_settings *settings, uint32_t sh_degree,
                          uint32_t num_points, const float *points,
                          const float *attributes, uint32_t adjacency_size,
                          const uint32_t *adjacency, const uint32_t *offsets,
                          uint32_t num_rays, const float *rays,
                          const uint32_t *start_point, uint32_t num_quantiles,
                          const float *quantiles,
                          const uint32_t *depth_indices, const float *rgba,
                          const float *grad_rgba, const float *depth_grad,
                          const float *ray_error, const float *sharpness,
                          oracle_grads *grads, oracle_visits *visits,
                          int num_threads) {
    if (sh_degree > 3 || !settings || !grads || !grads->points_grad ||
        !grads->attr_grad)
        return -1;
    if (num_quantiles > 0 && (!quantiles || !depth_grad)) return -1;
    if (settings->alpha_mode != ORACLE_ALPHA_NEUS && num_quantiles > 0 &&
        !depth_indices)
        return -1;
    bwd_job j;
    memset(&j, 0, sizeof(j));
    j.st = settings;
    j.sh_degree = sh_degree;
    j.nsh = (sh_degree + 1) * (sh_degree + 1);
    j.D = 1 + 3 * j.nsh;
    j.sc.points = points;
    j.sc.adjacency = adjacency;
    j.sc.offsets = offsets;
    j.sc.num_points = num_points;
    j.sc.adjacency_size = adjacency_size;
    j.sc.diff = make_diff(points, num_points, adjacency_size, adjacency, offsets);
    if (!j.sc.diff) return -1;
    j.attributes = attributes;
    j.rays = rays;
    j.start = start_point;
    j.Q = num_quantiles;
    j.quantiles = quantiles;
    j.depth_indices = depth_indices;
    j.rgba = rgba;
    j.grad_rgba = grad_rgba;
    j.depth_grad = depth_grad;
    j.ray_error = ray_error;
    j.sharp = sharpness ? sharpness[0] : 1.0f;
    j.has_sharpness_grad = grads->sharpness_grad != NULL;
    j.g = grads;
    j.visits = visits;
    j.shared = num_threads > 1;
    run_rays(bwd_range, &j, num_rays, num_threads);
    free((void *)j.sc.diff);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* AABB tree (src/aabb_tree/aabb_tree.cu:192-341)                            */

static uint32_t ilog2(uint32_t x) {
    uint32_t r = 0;
    while (x >>= 1) ++r;
    return r;
}

static uint32_t pow2_round_up(uint32_t x) {
    return (x > 1) ? 1u << (ilog2(x - 1) + 1) : 1u;
}

/* Node (depth d, i) lives at (2^td - 2^(d+1)) + i, td = log2(pow2_round_up N);
 * the leaves (depth td-1) hold consecutive point pairs, the last point padded
 * (aabb_tree.cu:200-221).  Entry pow2(N)-1 is never written by the reference;
 * here it is zeroed. */
void oracle_build_aabb_tree(const float *points, uint32_t num_points,
                            float *tree) {
    const uint32_t n2 = pow2_round_up(num_points);
    const uint32_t leaves = n2 / 2;
    memset(tree, 0, (size_t)n2 * 6 * sizeof(float));
    for (uint32_t l = 0; l < leaves; ++l) {
        const uint32_t pi = 2 * l;
        const float *a = points + 3ull * (pi < num_points ? pi : num_points - 1);
        const float *b = (pi + 1 < num_points) ? points + 3ull * (pi + 1) : a;
        float *node = tree + 6ull * l;
        for (int c = 0; c < 3; ++c) {
            node[c] = fminf(a[c], b[c]);
            node[3 + c] = fmaxf(a[c], b[c]);
        }
    }
    uint64_t prev = 0, width = leaves;
    while (width > 1) {
        const uint64_t next = prev + width;
        for (uint64_t i = 0; i < width / 2; ++i) {
            const float *c0 = tree + 6 * (prev + 2 * i);
            const float *c1 = tree + 6 * (prev + 2 * i + 1);
            float *node = tree + 6 * (next + i);
            for (int c = 0; c < 3; ++c) {
                node[c] = fminf(c0[c], c1[c]);
                node[3 + c] = fmaxf(c0[3 + c], c1[3 + c]);
            }
        }
        prev = next;
        width /= 2;
    }
}

/* ------------------------------------------------------------------------ */
/* nearest neighbour                                                         */

typedef struct {
    const float *points;
    uint32_t num_points;
    const float *queries;
    uint32_t *indices;
} nn_job;

/* dist = (point - query).norm() (aabb_tree.cuh:202) */
static void nn_range(void *p, uint32_t lo, uint32_t hi) {
    const nn_job *j = (const nn_job *)p;
    for (uint32_t qi = lo; qi < hi; ++qi) {
        const float *q = j->queries + 3ull * qi;
        float best = FLT_MAX;
        uint32_t bi = 0;
        for (uint32_t i = 0; i < j->num_points; ++i) {
            const float *pt = j->points + 3ull * i;
            const float dx = pt[0] - q[0], dy = pt[1] - q[1], dz = pt[2] - q[2];
            const float d = sqrtf(sdf_dot3(dx, dy, dz, dx, dy, dz));
            if (d < best) {
                best = d;
                bi = i;
            }
        }
        j->indices[qi] = bi;
    }
}

void oracle_nn(const float *points, uint32_t num_points, const float *queries,
               uint32_t num_queries, uint32_t *indices, int num_threads) {
    nn_job j = {points, num_points, queries, indices};
    run_rays(nn_range, &j, num_queries, num_threads);
}

/* ------------------------------------------------------------------------ */
/* farthest_neighbor (src/delaunay/triangulation_ops.cu:8-44): the farthest  */
/* CSR neighbour and sum(0.5 * distance) / row length, the sum kept in       */
/* double and rounded to float at every step as `float += 0.5 * float` does. */

void oracle_farthest_neighbor(const float *points, uint32_t num_points,
                              const uint32_t *adjacency, const uint32_t *offsets,
                              uint32_t *indices, float *cell_radius) {
    for (uint32_t i = 0; i < num_points; ++i) {
        const float *p = points + 3ull * i;
        const uint32_t beg = offsets[i], end = offsets[i + 1];
        uint32_t far = UINT32_MAX;
        float sum = 0.0f, max_d = 0.0f;
        for (uint32_t k = beg; k < end; ++k) {
            const uint32_t q = adjacency[k];
            if (q >= num_points) continue;
            const float dx = points[3ull * q] - p[0];
            const float dy = points[3ull * q + 1] - p[1];
            const float dz = points[3ull * q + 2] - p[2];
            const float d = sqrtf(sdf_dot3(dx, dy, dz, dx, dy, dz));
            sum = (float)((double)sum + 0.5 * (double)d);
            if (d > max_d) {
                max_d = d;
                far = q;
            }
        }
        indices[i] = far;
        cell_radius[i] = sum / (float)(end - beg);
    }
}
