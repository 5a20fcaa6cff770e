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

#endif /* SDFOAM_FPMATH_H */
