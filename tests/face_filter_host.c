/* Host statement of the walk's face filter (sdfoam_amd/csrc/trace_device.h,
 * walk_advance): t = num / dp is formed only where the bounds say the face
 * could be taken.  vf_check runs random and boundary cases and counts those
 * where the filter would skip a face that the exact rule (correctly rounded
 * t, then t > t0 && t < t1, or t < t1 unsafe) takes, or where the DUAL
 * "some t <= t0" decision differs from the exact one. */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint64_t rng_state;
static uint64_t next_u64(void) {
    rng_state += 0x9e3779b97f4a7c15ull;
    uint64_t z = rng_state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static float as_float(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
/* a random positive float over many binades, subnormals included */
static float rand_pos(void) {
    const uint64_t r = next_u64();
    const uint32_t exp = (uint32_t)(r % 160u);            /* 0 .. 159: up to ~2^32 */
    const uint32_t man = (uint32_t)(r >> 32) & 0x7fffffu;
    return as_float((exp << 23) | man);
}
static float step_ulps(float x, int k) {
    while (k > 0) { x = nextafterf(x, INFINITY); --k; }
    while (k < 0) { x = nextafterf(x, -INFINITY); ++k; }
    return x;
}

/* returns violations */
long long vf_check(long long cases, uint64_t seed) {
    rng_state = seed;
    long long bad = 0;
    for (long long c = 0; c < cases; ++c) {
        /* dp = diff . d with fp16 diffs (|diff| <= 65504 sqrt 3) and a unit
         * direction: 0 < dp < 2^17 */
        float dp = rand_pos();
        while (!(dp < 0x1p17f)) dp = rand_pos();
        const float t0 = (next_u64() & 7u) == 0 ? 0.0f : rand_pos();
        /* t1: above t0 (safe scans), infinite, or negative (unsafe scans) */
        const uint64_t sel = next_u64() % 8u;
        float t1 = sel == 0 ? INFINITY : (sel == 1 ? -rand_pos() : t0 + rand_pos());
        /* num near t1 dp or t0 dp, a few ulps either way, or random */
        const uint64_t pick = next_u64() % 4u;
        const int k = (int)(next_u64() % 9u) - 4;
        float num;
        if (pick == 0) num = step_ulps(t1 * dp, k);
        else if (pick == 1) num = step_ulps(t0 * dp, k);
        else if (pick == 2) num = (next_u64() & 1u) ? rand_pos() : -rand_pos();
        else num = step_ulps(t1 * dp * 0.5f + t0 * dp * 0.5f, k);
        if (!isfinite(num)) continue;
        const float t = num / dp;
        const float t1m = isinf(t1) ? t1 : fmaf(fabsf(t1), 0x1p-21f, t1);
        const float t0m = t0 * (1.0f - 0x1p-21f);
        const float t0p = t0 * (1.0f + 0x1p-21f);
        const float lo = fmaf(t0m, dp, -0x1p-126f);
        const int cand = num < fmaf(t1m, dp, 0x1p-126f);
        /* safe scans take t > t0 && t < t1; unsafe ones t < t1 */
        if (t > t0 && t < t1 && !(cand && num > lo)) ++bad;
        if (t < t1 && !cand) ++bad;
        /* DUAL: "t <= t0" is certain below lo, impossible above the upper
         * bound, and formed between */
        const int certain_below = num < lo;
        const int formed = num >= lo && num <= fmaf(t0p, dp, 0x1p-126f);
        const int says = certain_below || (formed && t <= t0);
        if (says != (t <= t0)) ++bad;
    }
    return bad;
}
