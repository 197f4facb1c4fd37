/*
 * TEST INFRASTRUCTURE ONLY. This oracle is the CPU checker for the HIP
 * kernels in blitzgs_amd/csrc; nothing in the product may include, link or
 * call it.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg use it.
 *
 * Scalar fp32 helpers shared by every oracle file.  Every operation here is
 * written out explicitly (no compiler contraction: the oracle is built with
 * -ffp-contract=off, fmaf is used only where written) so that the device code
 * in blitzgs_amd/csrc/gs_device.h, which spells out the same operation
 * sequence, produces the same bits.
 *
 * o_expf / o_logf are restatements from the mathematics, not copies of any
 * vendor library:
 *   exp: Cody-Waite reduction x = k*ln2 + r with ln2 split into a 16-bit
 *        high part (0x3f317200) and a low part (0x35bfbe8e), then the Taylor
 *        polynomial sum_{n<=7} r^n/n! in Horner form, scaled by 2^k.
 *   log: x = m*2^e with m in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
 *        log(m) = 2*atanh(s) = 2s*(1 + s^2/3 + s^4/5 + ... + s^10/11).
 * Their accuracy against libm's double-precision exp/log is pinned in
 * tests/test_oracle_math.py.
 */
#ifndef O_MATH_H
#define O_MATH_H

#include <math.h>
#include <stdint.h>
#include <string.h>
#include <limits.h>

static inline uint32_t o_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float o_u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* exp(x) for fp32 x.  Results below FLT_MIN are returned as 0 so that no
 * denormal handling difference between host and device can matter. */
static inline float o_expf(float x)
{
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.5f) return INFINITY;
    const float k = rintf(x * 1.44269502e+00f);          /* 1/ln2 rounded   */
    float r = fmaf(-k, o_u2f(0x3f317200u), x);             /* ln2 high part   */
    r = fmaf(-k, o_u2f(0x35bfbe8eu), r);                   /* ln2 low part    */
    float p = 1.98412701e-04f;                             /* 1/7!            */
    p = fmaf(p, r, 1.38888892e-03f);                       /* 1/6!            */
    p = fmaf(p, r, 8.33333377e-03f);                       /* 1/5!            */
    p = fmaf(p, r, 4.16666679e-02f);                       /* 1/4!            */
    p = fmaf(p, r, 1.66666672e-01f);                       /* 1/3!            */
    p = fmaf(p, r, 5.00000000e-01f);                       /* 1/2!            */
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

/* natural log of fp32 x. */
static inline float o_logf(float x)
{
    if (x != x) return x;
    if (x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (x == INFINITY) return x;
    int e;
    float m = frexpf(x, &e);                 /* m in [0.5, 1)        */
    if (m < 0.707106769f) { m = m + m; e = e - 1; }
    const float f = m - 1.0f;                /* exact (Sterbenz)     */
    const float s = f / (2.0f + f);
    const float z = s * s;
    float p = 9.09090936e-02f;               /* 1/11 */
    p = fmaf(p, z, 1.11111112e-01f);         /* 1/9  */
    p = fmaf(p, z, 1.42857149e-01f);         /* 1/7  */
    p = fmaf(p, z, 2.00000003e-01f);         /* 1/5  */
    p = fmaf(p, z, 3.33333343e-01f);         /* 1/3  */
    const float s2 = s + s;
    const float lm = fmaf(s2 * z, p, s2);
    const float ef = (float)e;
    return fmaf(ef, o_u2f(0x3f317200u), fmaf(ef, o_u2f(0x35bfbe8eu), lm));
}

/* float -> int32 with truncation toward zero, saturating, NaN -> 0
 * (the semantics of the reference's device-side (int) casts). */
static inline int o_f2i_sat(float x)
{
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT_MAX;
    if (x <= -2147483648.0f) return INT_MIN;
    return (int)x;
}

static inline float o_fminf(float a, float b) { return fminf(a, b); }
static inline float o_fmaxf(float a, float b) { return fmaxf(a, b); }

#endif
