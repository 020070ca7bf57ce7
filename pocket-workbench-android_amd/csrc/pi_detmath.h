// Deterministic exp / log / sin / cos / pow for host and device.
//
// The reference calls the platform libm (f32::exp, cos, sin, powf in
// model.rs:416,455-456,1042,1113), whose last-bit results are not pinned by
// the reference.  The backend fixes one definition that the host and the GPU
// evaluate identically: IEEE double arithmetic with plain + - * / (this file
// is built with -ffp-contract=off), rounded once to float.  The double result
// is within a few 1e-16 relative of the true value, so the float result is the
// correctly rounded one except for inputs within ~1e-16 of a rounding
// midpoint.  Range reduction follows Cody and Waite (split ln2 and pi/2 so the
// first products are exact); the kernels are Taylor series.
#pragma once

#include <cmath>

#if defined(__HIPCC__)
#define PI_DM __host__ __device__ inline
#else
#define PI_DM inline
#endif

// exp(x) for finite x in [-745, 709].
PI_DM double pi_exp_d(double x) {
    const double INVLN2 = 1.4426950408889634074;
    const double LN2_HI = 6.93147180369123816490e-01;
    const double LN2_LO = 1.90821492927058770002e-10;
    const double SHIFT = 6755399441055744.0;  // 1.5 * 2^52: round to nearest even
    double t = x * INVLN2;
    double kd = t + SHIFT;
    kd = kd - SHIFT;
    double r = x - kd * LN2_HI;
    r = r - kd * LN2_LO;
    double p = 1.0 / 6227020800.0;
    p = p * r + 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    return ldexp(p, (int)kd);
}

PI_DM float pi_expf(float x) {
    if (x != x) return x;
    if (x > 100.0f) return INFINITY;
    if (x < -110.0f) return 0.0f;
    return (float)pi_exp_d((double)x);
}

// log(x) for finite x > 0.
PI_DM double pi_log_d(double x) {
    const double LN2_HI = 6.93147180369123816490e-01, LN2_LO = 1.90821492927058770002e-10;
    int e = 0;
    double m = frexp(x, &e);
    if (m < 0.70710678118654752440) { m = m * 2.0; e = e - 1; }
    double t = (m - 1.0) / (m + 1.0), t2 = t * t;
    double s = 1.0 / 31.0;
    for (int i = 29; i >= 1; i -= 2) s = s * t2 + 1.0 / (double)i;
    double l = 2.0 * t * s;
    return ((double)e * LN2_LO + l) + (double)e * LN2_HI;
}

// sin and cos for |x| < 2^20.
PI_DM void pi_sincos_d(double x, double *s, double *c) {
    const double TWO_OVER_PI = 6.36619772367581382433e-01;
    const double PIO2_1 = 1.57079632673412561417e+00;
    const double PIO2_2 = 6.07710050630396597660e-11;
    const double PIO2_3 = 2.02226624879595063154e-21;
    const double SHIFT = 6755399441055744.0;
    double kd = x * TWO_OVER_PI + SHIFT;
    kd = kd - SHIFT;
    double r = x - kd * PIO2_1;
    r = r - kd * PIO2_2;
    r = r - kd * PIO2_3;
    double r2 = r * r;
    double ps = -1.0 / 51090942171709440000.0;
    ps = ps * r2 + 1.0 / 121645100408832000.0;
    ps = ps * r2 - 1.0 / 355687428096000.0;
    ps = ps * r2 + 1.0 / 1307674368000.0;
    ps = ps * r2 - 1.0 / 6227020800.0;
    ps = ps * r2 + 1.0 / 39916800.0;
    ps = ps * r2 - 1.0 / 362880.0;
    ps = ps * r2 + 1.0 / 5040.0;
    ps = ps * r2 - 1.0 / 120.0;
    ps = ps * r2 + 1.0 / 6.0;
    ps = ps * r2;
    double sr = r - r * ps;
    double pc = 1.0 / 2432902008176640000.0;
    pc = pc * r2 - 1.0 / 6402373705728000.0;
    pc = pc * r2 + 1.0 / 20922789888000.0;
    pc = pc * r2 - 1.0 / 87178291200.0;
    pc = pc * r2 + 1.0 / 479001600.0;
    pc = pc * r2 - 1.0 / 3628800.0;
    pc = pc * r2 + 1.0 / 40320.0;
    pc = pc * r2 - 1.0 / 720.0;
    pc = pc * r2 + 1.0 / 24.0;
    pc = pc * r2 - 0.5;
    pc = pc * r2;
    double cr = 1.0 + pc;
    long k = (long)kd;
    switch (k & 3) {
    case 0: *s = sr; *c = cr; break;
    case 1: *s = cr; *c = -sr; break;
    case 2: *s = -sr; *c = -cr; break;
    default: *s = -cr; *c = sr; break;
    }
}

// Seeded N(0,1) pair for element (layer*n_kv + head, position, dim) of the
// K and V caches (long-context setup): SplitMix64 finalizer hashing of the
// key, Box-Muller in IEEE double with the functions above, so the host and
// the device produce the same bits.  Independent of how many positions are
// filled.
PI_DM uint64_t pi_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
PI_DM void pi_kv_normal(uint64_t seed, uint32_t lh, uint32_t p, uint32_t d, float *k, float *v) {
    const uint64_t key = ((uint64_t)lh << 32) | ((uint64_t)p << 8) | (uint64_t)d;
    const uint64_t z1 = pi_mix64(seed ^ pi_mix64(key)), z2 = pi_mix64(z1);
    const double u1 = ((double)(z1 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(z2 >> 11) * (1.0 / 9007199254740992.0);
    const double rad = pi_exp_d(0.5 * pi_log_d(-2.0 * pi_log_d(u1)));   // sqrt(-2 ln u1)
    double sn, cs;
    pi_sincos_d(6.28318530717958647692 * u2, &sn, &cs);
    *k = (float)(rad * cs);
    *v = (float)(rad * sn);
}

inline float pi_cosf(float x) { double s, c; pi_sincos_d((double)x, &s, &c); return (float)c; }
inline float pi_sinf(float x) { double s, c; pi_sincos_d((double)x, &s, &c); return (float)s; }
inline float pi_powf(float x, float y) { return (float)pi_exp_d((double)y * pi_log_d((double)x)); }
