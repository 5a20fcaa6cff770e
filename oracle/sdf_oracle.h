/*
 * TEST INFRASTRUCTURE -- NOT PART OF THE PRODUCT.
 *
 * Scalar host oracle for the SDFoam Voronoi-foam tracer.  Only tests/,
 * __graft_entry__.smoke() and bench.py's CPU-baseline leg load it, and only
 * as the checker.  The product library (sdfoam_amd/csrc) never includes,
 * links or calls anything under oracle/.
 *
 * Every function restates one piece of the reference (file:line given at
 * each definition in sdf_oracle.c).  Arithmetic follows the shared contract
 * in include/sdfoam_fpmath.h; every other floating-point expression is
 * written out operation by operation in the reference's order, with a fused
 * multiply-add exactly where an accumulation `a += b * c` appears in the
 * reference (nothing else is contracted: built with -ffp-contract=off).
 *
 * Gradients are accumulated in double.  Alongside each gradient element the
 * oracle keeps A = sum |c_k| over its contributions and K = their count, for
 * the order-independent summation bound |fl(sum) - sum| <= gamma_{K-1} * A
 * used by the tests (Higham, Accuracy and Stability of Numerical Algorithms,
 * 2nd ed., section 4.2).
 *
 * Pinning status of each function is listed in oracle/README.md.
 */
#ifndef SDF_ORACLE_H
#define SDF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* alpha_mode values (src/tracing/pipeline.h:10) */
#define ORACLE_ALPHA_STANDARD 0u
#define ORACLE_ALPHA_NEUS 1u

typedef struct {
    float weight_threshold;     /* src/tracing/pipeline.h:13, default 1e-7 */
    uint32_t max_intersections; /* src/tracing/pipeline.h:14, default 1024 */
    uint32_t alpha_mode;        /* src/tracing/pipeline.h:17 */
    int32_t sdf_channel;        /* src/tracing/pipeline.h:20, -1 = unset */
} oracle_settings;

/* Per-ray visit recording (test aid; any pointer may be NULL).
 * hash: FNV-1a 64 over the cell index of every cell step (functor call);
 * cells/alphas: the first `stride` steps of each ray, row-major [R, stride];
 * steps: number of cell steps of each ray;
 * faces: number of faces scanned by each ray (all loop iterations);
 * point_visits: per point, the number of cell steps into it (the count K of
 * terms in its contribution sum). */
typedef struct {
    uint64_t *hash;
    uint32_t *cells;
    float *alphas;
    uint32_t stride;
    uint32_t *steps;
    uint64_t *faces;
    uint64_t *faces_stepped; /* faces of the cells that got a functor call */
    float *t_exit;           /* [R, stride]: t1 of each recorded step */
    uint32_t *point_visits;  /* [N]: cell steps into each point over all rays */
} oracle_visits;

const char *oracle_version(void);

/* fpmath contract, exported so tests can pin it */
float oracle_expf(float x);
float oracle_sigmoidf(float x);
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
void oracle_expf_n(const float *x, float *y, uint64_t n);
void oracle_f32_to_f16_n(const float *x, uint16_t *y, uint64_t n);

/* SH basis of degree <= 3 at a unit direction (src/tracing/sh_utils.cuh:25-62) */
void oracle_sh_basis(uint32_t degree, float x, float y, float z, float *out16);

/* fp16 neighbour offsets, 4 halves per CSR entry (w = 0)
 * (src/tracing/pipeline.cu:1202-1242) */
void oracle_prefetch_adjacent_diff(const float *points, uint32_t num_points,
                                   uint32_t adjacency_size,
                                   const uint32_t *adjacency,
                                   const uint32_t *offsets, uint16_t *diff);

/* Forward pass (src/tracing/pipeline.cu:36-264 with the walk of
 * src/tracing/tracing_utils.cuh:15-109).  contribution is accumulated in
 * double.  Returns 0, or -1 on bad arguments. */
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
                         int num_threads);

/* Camera of Pipeline::trace_benchmark (src/tracing/camera.h:17-27); model
 * 0 = pinhole, 1 = fisheye. */
typedef struct {
    float position[3];
    float forward[3];
    float right[3];
    float up[3];
    float fov;
    uint32_t width;
    uint32_t height;
    uint32_t model;
} oracle_camera;

/* Inference render (src/tracing/pipeline.cu:1067-1199): one ray per pixel
 * cast in-kernel (src/tracing/camera.h:56-85), one start cell for all,
 * the forward's compositing, colour + T * background packed as RGBA8 into
 * row (height - 1 - j).  adjacent_diff is the caller's fp16 offset table
 * [E, 4].  bg_color NULL = white.  rgbt (optional, [H*W, 4], pixel order
 * j * W + i) receives C and T; num_intersections (optional) the loop count. */
int oracle_trace_benchmark(const oracle_settings *settings, uint32_t sh_degree,
                           uint32_t num_points, const float *points,
                           const float *attributes, uint32_t adjacency_size,
                           const uint32_t *adjacency, const uint32_t *offsets,
                           const uint16_t *adjacent_diff, const oracle_camera *camera,
                           uint32_t start_point, const float *sharpness,
                           const float *bg_color, int checker_bg, uint32_t *output_rgba,
                           float *rgbt, uint32_t *num_intersections, int num_threads);
float oracle_camera_focal(float fov);
void oracle_cast_ray(const oracle_camera *cam, uint32_t i, uint32_t j, float *dir);
void oracle_sincosf_n(const float *x, float *s, float *c, uint64_t n);
void oracle_atan2f_n(const float *y, const float *x, float *out, uint64_t n);
uint32_t oracle_make_rgba8(float r, float g, float b, float a);

/* Gradient buffers of the backward pass.  Any of the *_abs / *_k buffers may
 * be NULL. */
typedef struct {
    double *points_grad;     /* [N, 3] */
    double *attr_grad;       /* [N, D] */
    double *sharpness_grad;  /* [1] */
    double *point_error;     /* [N] or NULL */
    double *points_grad_abs; /* [N, 3] */
    double *attr_grad_abs;   /* [N, D] */
    double *sharpness_abs;   /* [1] */
    uint32_t *points_grad_k; /* [N, 3] */
    uint32_t *attr_grad_k;   /* [N, D] */
    uint64_t *sharpness_k;   /* [1] */
} oracle_grads;

/* Backward pass.  alpha_mode NEUS follows backward_sdf
 * (src/tracing/pipeline.cu:267-550), STANDARD follows backward
 * (src/tracing/pipeline.cu:553-791); dispatch as
 * src/tracing/pipeline.cu:1338-1391. */
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
                          int num_threads);

/* d t / d p of the bisector-plane crossing between p and q for the ray
 * (o, unit d)  (src/tracing/tracing_utils.cuh:112-124). */
void oracle_cell_intersection_grad(const float *p, const float *q, const float *o,
                                   const float *d, float *g);

/* AABB tree over consecutive point pairs, layout [pow2(N), 2, 3]
 * (src/aabb_tree/aabb_tree.cu:192-341, src/aabb_tree/aabb_tree.cuh:35-43). */
void oracle_build_aabb_tree(const float *points, uint32_t num_points,
                            float *tree);

/* Exact nearest neighbour by the fp32 distance of
 * src/aabb_tree/aabb_tree.cuh:197-203 (ties: smallest index). */
void oracle_nn(const float *points, uint32_t num_points, const float *queries,
               uint32_t num_queries, uint32_t *indices, int num_threads);

/* Farthest CSR neighbour and mean half edge length per point
 * (src/delaunay/triangulation_ops.cu:8-44). */
void oracle_farthest_neighbor(const float *points, uint32_t num_points,
                              const uint32_t *adjacency, const uint32_t *offsets,
                              uint32_t *indices, float *cell_radius);

#ifdef __cplusplus
}
#endif

#endif
