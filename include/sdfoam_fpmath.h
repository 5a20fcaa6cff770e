/*
 * sdfoam_fpmath.h -- the floating-point contract shared by the HIP kernels
 * and the scalar host oracle.
 *
 * The Voronoi walk stops when the transmittance T falls to the weight
 * threshold, and T is a product of terms 1 - exp(-s * dt).  A visit sequence
 * can therefore only be bit-exact between two implementations if both compute
 * exp, the sigmoid and the fp16 rounding of the neighbour offsets to the same
 * bits.  Everything here is built from IEEE-754 operations that are correctly
 * rounded on both the x86 host and gfx950 (add, mul, fma, rint, ldexp and
 * integer bit manipulation), so the same source gives the same bits on both
 * sides as long as the translation unit is compiled with -ffp-contract=off
 * (every fused multiply-add below is written out as fmaf).
 *
 * The reference computes these with CUDA intrinsics
 * (src/tracing/pipeline.cu:18-20, 56-58, 151 `__expf`; the fp16 offsets of
 * src/tracing/pipeline.cu:1221-1222 use Eigen's `__half(float)` conversion).
 * Those intrinsics are not reproduced; exp is written from the textbook method
 * (Cody & Waite additive range reduction, then a Taylor polynomial of degree 7
 * evaluated by Horner's rule; J.-M. Muller, "Elementary Functions", ch. 11),
 * and the fp16 conversion from the IEEE-754 binary16 definition with
 * round-to-nearest-even.
 *
 * Valid as C99 (gcc) and as HIP C++ (hipcc); under HIP every function is
 * __host__ __device__.
 */
#ifndef SDFOAM_FPMATH_H
#define SDFOAM_FPMATH_H

#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define SDF_FPMATH_FN static __host__ __device__ __attribute__((always_inline)) inline
#else
#define SDF_FPMATH_FN static inline
#endif

/* ---- bit casts ---------------------------------------------------------- */

SDF_FPMATH_FN uint32_t sdf_f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof(u));
    return u;
}

SDF_FPMATH_FN float sdf_bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

/* ---- exp ---------------------------------------------------------------- */

/* Largest x with exp(x) finite in fp32, and the x below which exp(x) would be
 * subnormal.  Below the latter the function returns +0: the true value is
 * under 2^-126 and every caller (alpha = 1 - exp(-s dt), the sigmoid) adds it
 * to 1 or subtracts it from 1, where it vanishes in fp32 either way.  Keeping
 * subnormals out of the result also keeps the bits independent of the
 * hardware's subnormal mode. */
#define SDF_EXP_HI 88.72283935546875f
#define SDF_EXP_LO (-87.33654022216797f)

/* ln 2 split for Cody-Waite: LN2_HI has 16 significant bits, so k * LN2_HI is
 * exact for |k| <= 256 and x - k * LN2_HI is exact (the fma below adds a
 * single rounding on top of an exact value). */
#define SDF_LN2_HI 0.693145751953125f
#define SDF_LN2_LO 1.428606765330187e-06f
#define SDF_LOG2E 1.44269504088896341f

SDF_FPMATH_FN float sdf_expf(float x) {
    if (x != x) {
        return x; /* NaN propagates */
    }
    if (x > SDF_EXP_HI) {
        return sdf_bits_f32(0x7f800000u); /* +inf */
    }
    if (x < SDF_EXP_LO) {
        return 0.0f;
    }
    /* k = nearest integer to x / ln2;  r = x - k ln2,  |r| <= ~0.347 */
    const float k = rintf(x * SDF_LOG2E);
    float r = fmaf(k, -SDF_LN2_HI, x);
    r = fmaf(k, -SDF_LN2_LO, r);
    /* exp(r) = sum_{n=0..7} r^n / n!  (truncation error < 0.17 ulp on |r| <= 0.36) */
    float p = 1.98412698412698413e-04f;           /* 1/5040 */
    p = fmaf(p, r, 1.38888888888888889e-03f);     /* 1/720  */
    p = fmaf(p, r, 8.33333333333333333e-03f);     /* 1/120  */
    p = fmaf(p, r, 4.16666666666666667e-02f);     /* 1/24   */
    p = fmaf(p, r, 1.66666666666666667e-01f);     /* 1/6    */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

/* The reference's sigmoid, 1 / (1 + exp(-v))  (src/tracing/pipeline.cu:18-20). */
SDF_FPMATH_FN float sdf_sigmoidf(float v) {
    return 1.0f / (1.0f + sdf_expf(-v));
}

/* ---- 3-vector dot product ----------------------------------------------- */

/* a0*b0 + (a1*b1 + a2*b2): the reduction order Eigen uses for a fixed-size
 * 3-vector dot (an unrolled pairwise split 1 + 2), with the products fused
 * the way a contracting compiler fuses this expression.  Used for every dot
 * and squared norm on the path so host and device agree bit for bit. */
SDF_FPMATH_FN float sdf_dot3(float a0, float a1, float a2,
                             float b0, float b1, float b2) {
    return fmaf(a0, b0, fmaf(a1, b1, a2 * b2));
}

/* ---- binary16 ----------------------------------------------------------- */

/* fp32 -> fp16 bits, IEEE round-to-nearest-even, subnormals kept, overflow to
 * +-inf, NaN kept quiet. */
SDF_FPMATH_FN uint16_t sdf_f32_to_f16_bits(float f) {
    const uint32_t x = sdf_f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    }
    if (ax >= 0x477ff000u) {
        return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    }
    if (ax <= 0x33000000u) {
        return (uint16_t)sign; /* <= 2^-25: ties-to-even gives zero */
    }
    const int e = (int)(ax >> 23) - 127;
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t h;
    if (e >= -14) {
        h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
            h += 1u; /* a carry into the exponent is the correct result */
        }
    } else {
        const uint32_t m = mant | 0x800000u;
        const int s = 13 + (-14 - e); /* 14 .. 24 */
        h = m >> s;
        const uint32_t rem = m & ((1u << s) - 1u);
        const uint32_t half = 1u << (s - 1);
        if (rem > half || (rem == half && (h & 1u))) {
            h += 1u;
        }
    }
    return (uint16_t)(sign | h);
}

/* fp16 bits -> fp32, exact. */
SDF_FPMATH_FN float sdf_f16_bits_to_f32(uint16_t hb) {
    const uint32_t sign = ((uint32_t)hb & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)hb >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)hb & 0x3ffu;
    if (e == 0x1fu) {
        return sdf_bits_f32(sign | 0x7f800000u | (m << 13));
    }
    if (e == 0u) {
        /* subnormal (or zero): m * 2^-24, exact in fp32 */
        const float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return sdf_bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* ---- sin, cos, atan2 (camera rays) --------------------------------------- */

/* Only the fisheye camera needs these (src/tracing/camera.h:69-79, where the
 * reference calls CUDA's sinf / cosf / atan2f).  Written from the textbook
 * methods so host and device agree bit for bit: Cody-Waite reduction by pi/2
 * (three-part constant, exact products for |k| < 2^12) and Taylor
 * polynomials on |r| <= pi/4 (Muller, "Elementary Functions", ch. 11); atan
 * through atan(a) = pi/4 + atan((a - 1) / (a + 1)) and its Taylor series on
 * |t| <= tan(pi/8).  Accuracy: a few ulp for |x| < 2^12, pinned against
 * float64 in the tests.  Not for general use beyond that range. */
#define SDF_PIO2_1 1.5703125f
#define SDF_PIO2_2 4.838705062866211e-04f
#define SDF_PIO2_3 (-4.371138828673793e-08f)
#define SDF_TWO_OVER_PI 0.6366197466850281f
#define SDF_PIO2_HI 1.5707963705062866f
#define SDF_PIO2_LO (-4.371139000186243e-08f)
#define SDF_PIO4_HI 0.7853981852531433f
#define SDF_PIO4_LO (-2.1855695000931214e-08f)
#define SDF_PI_HI 3.1415927410125732f
#define SDF_PI_LO (-8.742278000372485e-08f)

SDF_FPMATH_FN void sdf_sincosf(float x, float *s_out, float *c_out) {
    const float k = rintf(x * SDF_TWO_OVER_PI);
    float r = fmaf(k, -SDF_PIO2_1, x);
    r = fmaf(k, -SDF_PIO2_2, r);
    r = fmaf(k, -SDF_PIO2_3, r);
    const float r2 = r * r;
    /* sin r = r + r^3 (-1/3! + r^2 (1/5! + r^2 (-1/7! + r^2 / 9!))) */
    float ps = 2.75573192239858907e-06f;
    ps = fmaf(ps, r2, -1.98412698412698413e-04f);
    ps = fmaf(ps, r2, 8.33333333333333333e-03f);
    ps = fmaf(ps, r2, -1.66666666666666667e-01f);
    const float s = fmaf(ps * r2, r, r);
    /* cos r = 1 + r^2 (-1/2! + r^2 (1/4! + r^2 (-1/6! + r^2 (1/8! - r^2 / 10!)))) */
    float pc = -2.75573192239858907e-07f;
    pc = fmaf(pc, r2, 2.48015873015873016e-05f);
    pc = fmaf(pc, r2, -1.38888888888888889e-03f);
    pc = fmaf(pc, r2, 4.16666666666666667e-02f);
    pc = fmaf(pc, r2, -0.5f);
    const float c = fmaf(pc, r2, 1.0f);
    const int q = ((int)k) & 3;
    if (q == 0) {
        *s_out = s;
        *c_out = c;
    } else if (q == 1) {
        *s_out = c;
        *c_out = -s;
    } else if (q == 2) {
        *s_out = -s;
        *c_out = -c;
    } else {
        *s_out = -c;
        *c_out = s;
    }
}

/* atan of a in [0, 1] */
SDF_FPMATH_FN float sdf_atan01f(float a) {
    float t = a, hi = 0.0f, lo = 0.0f;
    if (a > 0.41421356237309503f) { /* tan(pi/8) */
        t = (a - 1.0f) / (a + 1.0f);
        hi = SDF_PIO4_HI;
        lo = SDF_PIO4_LO;
    }
    const float t2 = t * t;
    /* atan t = t + t^3 sum_{n=1..9} (-1)^n t^(2n-2) / (2n+1) */
    float p = -1.0f / 19.0f;
    p = fmaf(p, t2, 1.0f / 17.0f);
    p = fmaf(p, t2, -1.0f / 15.0f);
    p = fmaf(p, t2, 1.0f / 13.0f);
    p = fmaf(p, t2, -1.0f / 11.0f);
    p = fmaf(p, t2, 1.0f / 9.0f);
    p = fmaf(p, t2, -1.0f / 7.0f);
    p = fmaf(p, t2, 1.0f / 5.0f);
    p = fmaf(p, t2, -1.0f / 3.0f);
    const float at = fmaf(p * t2, t, t);
    return hi + (at + lo);
}

/* atan2(y, x) for finite arguments; atan2(+-0, +0) = +-0, atan2(+-0, -0) = +-pi. */
SDF_FPMATH_FN float sdf_atan2f(float y, float x) {
    if (x != x || y != y) return x + y;
    const float ax = fabsf(x), ay = fabsf(y);
    float res;
    if (ax == 0.0f && ay == 0.0f) {
        res = 0.0f;
    } else if (ay <= ax) {
        res = sdf_atan01f(ay / ax);
    } else {
        res = (SDF_PIO2_HI - sdf_atan01f(ax / ay)) + SDF_PIO2_LO;
    }
    if (sdf_f32_bits(x) >> 31) res = (SDF_PI_HI - res) + SDF_PI_LO;
    return (sdf_f32_bits(y) >> 31) ? -res : res;
}

/* ---- camera rays and 8-bit colour ----------------------------------------- */

#define SDF_CAM_PINHOLE 0u
#define SDF_CAM_FISHEYE 1u

/* cast_ray (src/tracing/camera.h:56-85): the ray through pixel (i, j) at
 * (i / width, j / height), no half-pixel offset, vertical fov.  `focal` is
 * 1 / tan(fov / 2) (pinhole), computed once by the caller.  The sums of
 * scaled basis vectors are fused as a contracting compiler fuses
 * `a * f + b * r + c * u` (parity of those bits with the reference is
 * unpinned).  The direction is unit length, or zero where the fisheye
 * mask is 0. */
SDF_FPMATH_FN void sdf_cast_ray(const float *fwd, const float *right, const float *up,
                                float fov, float focal, uint32_t width, uint32_t height,
                                uint32_t model, uint32_t i, uint32_t j, float *dir) {
    const float aspect = (float)width / (float)height;
    const float x = (float)i / (float)width;
    const float y = (float)j / (float)height;
    const float u = (2.0f * x - 1.0f) * aspect;
    const float v = 1.0f - 2.0f * y;
    float mask = 1.0f;
    if (model == SDF_CAM_FISHEYE) {
        const float theta = sdf_atan2f(v, u);
        float phi = fov * sqrtf(fmaf(u, u, v * v));
        if (phi >= 3.14159265358979323846f) {
            phi = 3.14159265358979323846f - 1e-6f;
            mask = 0.0f;
        }
        float sp, cp, st, ct;
        sdf_sincosf(phi, &sp, &cp);
        sdf_sincosf(theta, &st, &ct);
        const float a = sp * ct, b = sp * st;
        for (int k = 0; k < 3; ++k) dir[k] = fmaf(cp, fwd[k], fmaf(b, up[k], a * right[k]));
    } else {
        for (int k = 0; k < 3; ++k) dir[k] = fmaf(v, up[k], fmaf(u, right[k], focal * fwd[k]));
    }
    const float n2 = sdf_dot3(dir[0], dir[1], dir[2], dir[0], dir[1], dir[2]);
    if (n2 > 0.0f) {
        const float n = sqrtf(n2);
        for (int k = 0; k < 3; ++k) dir[k] = dir[k] / n;
    }
    for (int k = 0; k < 3; ++k) dir[k] = dir[k] * mask;
}

/* make_rgba8 (src/tracing/tracing_utils.cuh:126-136): clamp to [0, 1],
 * truncate x * 255, pack r | g << 8 | b << 16 | a << 24. */
SDF_FPMATH_FN uint32_t sdf_make_rgba8(float r, float g, float b, float a) {
    r = fmaxf(0.0f, fminf(1.0f, r));
    g = fmaxf(0.0f, fminf(1.0f, g));
    b = fmaxf(0.0f, fminf(1.0f, b));
    a = fmaxf(0.0f, fminf(1.0f, a));
    const uint32_t ri = (uint32_t)(int)(r * 255.0f);
    const uint32_t gi = (uint32_t)(int)(g * 255.0f);
    const uint32_t bi = (uint32_t)(int)(b * 255.0f);
    const uint32_t ai = (uint32_t)(int)(a * 255.0f);
    return (ai << 24) | (bi << 16) | (gi << 8) | ri;
}

#endif /* SDFOAM_FPMATH_H */
