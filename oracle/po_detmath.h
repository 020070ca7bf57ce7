/*
 * po_detmath.h -- the oracle's exp / log / sin / cos / pow.
 *
 * TEST INFRASTRUCTURE (part of the CPU oracle).
 *
 * The reference calls the platform libm (f32::exp, cos, sin, powf in
 * model.rs:416,455-456,1042,1113 and sampler.rs:46), whose last-bit results
 * differ between libms and are not pinned by anything the reference ships.
 * The oracle therefore fixes one definition: each function is evaluated in
 * IEEE double with plain + - * / (no FMA, no libm transcendental) and rounded
 * once to float, so any IEEE machine, CPU or GPU, reproduces it bit for bit.
 * Accuracy: the double result is within a few 1e-16 relative of the true
 * value, so the float result is the correctly rounded one except for inputs
 * within ~1e-16 of a rounding midpoint.
 */
#ifndef PO_DETMATH_H
#define PO_DETMATH_H

#include <math.h>

/* exp(x) for finite x in [-745, 709]: x = k ln2 + r, |r| <= ln2/2, with ln2
 * split so k*LN2_HI is exact; exp(r) by its Taylor series to r^13. */
static inline double po_exp_d(double x) {
    const double INVLN2 = 1.4426950408889634074;
    const double LN2_HI = 6.93147180369123816490e-01; /* 0x3FE62E42FEE00000 */
    const double LN2_LO = 1.90821492927058770002e-10; /* 0x3DEA39EF35793C76 */
    const double SHIFT = 6755399441055744.0;           /* 1.5 * 2^52: round to nearest even */
    double t = x * INVLN2;
    double kd = t + SHIFT;
    kd = kd - SHIFT;
    double r = x - kd * LN2_HI;
    r = r - kd * LN2_LO;
    double p = 1.0 / 6227020800.0;           /* 1/13! */
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

static inline float po_expf(float x) {
    if (x != x) return x;
    if (x > 100.0f) return INFINITY;
    if (x < -110.0f) return 0.0f;
    return (float)po_exp_d((double)x);
}

/* log(x) for finite x > 0: x = m 2^e, m in [sqrt(1/2), sqrt(2)),
 * log m = 2 atanh((m-1)/(m+1)) by its series to t^31. */
static inline double po_log_d(double x) {
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

/* sin and cos for |x| < 2^20: reduction by pi/2 with a three-part split
 * (k*PIO2_1 and k*PIO2_2 exact for k < 2^20), then Taylor series on
 * |r| <= pi/4. */
static inline void po_sincos_d(double x, double *s, double *c) {
    const double TWO_OVER_PI = 6.36619772367581382433e-01;
    const double PIO2_1 = 1.57079632673412561417e+00;  /* 0x3FF921FB54400000 */
    const double PIO2_2 = 6.07710050630396597660e-11;  /* 0x3DD0B4611A600000 */
    const double PIO2_3 = 2.02226624879595063154e-21;  /* 0x3BA3198A2E037073 */
    const double SHIFT = 6755399441055744.0;
    double kd = x * TWO_OVER_PI + SHIFT;
    kd = kd - SHIFT;
    double r = x - kd * PIO2_1;
    r = r - kd * PIO2_2;
    r = r - kd * PIO2_3;
    double r2 = r * r;
    /* sin r = r (1 - r^2/3! + ...), cos r = 1 - r^2/2! + ... to r^21 / r^20 */
    double ps = -1.0 / 51090942171709440000.0;          /* -1/21! */
    ps = ps * r2 + 1.0 / 121645100408832000.0;          /* 1/19! */
    ps = ps * r2 - 1.0 / 355687428096000.0;             /* 1/17! */
    ps = ps * r2 + 1.0 / 1307674368000.0;               /* 1/15! */
    ps = ps * r2 - 1.0 / 6227020800.0;                  /* 1/13! */
    ps = ps * r2 + 1.0 / 39916800.0;                    /* 1/11! */
    ps = ps * r2 - 1.0 / 362880.0;                      /* 1/9! */
    ps = ps * r2 + 1.0 / 5040.0;                        /* 1/7! */
    ps = ps * r2 - 1.0 / 120.0;
    ps = ps * r2 + 1.0 / 6.0;
    ps = ps * r2;
    double sr = r - r * ps;
    double pc = 1.0 / 2432902008176640000.0;            /* 1/20! */
    pc = pc * r2 - 1.0 / 6402373705728000.0;            /* 1/18! */
    pc = pc * r2 + 1.0 / 20922789888000.0;              /* 1/16! */
    pc = pc * r2 - 1.0 / 87178291200.0;                 /* 1/14! */
    pc = pc * r2 + 1.0 / 479001600.0;                   /* 1/12! */
    pc = pc * r2 - 1.0 / 3628800.0;                     /* 1/10! */
    pc = pc * r2 + 1.0 / 40320.0;                       /* 1/8! */
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

static inline float po_cosf(float x) { double s, c; po_sincos_d((double)x, &s, &c); return (float)c; }
static inline float po_sinf(float x) { double s, c; po_sincos_d((double)x, &s, &c); return (float)s; }

/* x^y for x > 0 finite (the RoPE base): exp(y log x) in double. */
static inline float po_powf(float x, float y) { return (float)po_exp_d((double)y * po_log_d((double)x)); }

#endif
