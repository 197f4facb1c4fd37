// Device-side scalar helpers shared by the rasterizer kernels (gfx950).
//
// The library is compiled with -ffp-contract=off: a*b+c is never fused
// implicitly, every fused multiply-add is an explicit __builtin_fmaf, and fp32
// division and sqrt are correctly rounded (HIP's default).  Together with the
// fixed operation order below this makes the per-Gaussian preprocess, the tile
// keys and the forward blend bit-reproducible on a CPU.
//
// gs_expf / gs_logf are written from the mathematics:
//   exp: Cody-Waite reduction x = k*ln2 + r, ln2 split into a 16-bit high part
//        (0x3f317200) and a low part (0x35bfbe8e), Taylor polynomial
//        sum_{n<=7} r^n/n! in Horner form, scaled by 2^k; results below
//        FLT_MIN are returned as 0.
//   log: x = m*2^e, m in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
//        log(m) = 2*atanh(s) = 2s*(1 + s^2/3 + ... + s^10/11).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define GS_TILE 16
#define GS_WAVE 64

namespace gs {

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// exp of the core range, x finite in [-87, 88.5]
__device__ __forceinline__ float expf_core(float x)
{
    const float k = __builtin_rintf(x * 1.44269502e+00f);
    float r = __builtin_fmaf(-k, u2f(0x3f317200u), x);
    r = __builtin_fmaf(-k, u2f(0x35bfbe8eu), r);
    float p = 1.98412701e-04f;
    p = __builtin_fmaf(p, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 5.00000000e-01f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

__device__ __forceinline__ float expf_full(float x)
{
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.5f) return __builtin_inff();
    return expf_core(x);
}

// exp for x <= 0 or NaN (the blend's Gaussian falloff); identical to
// expf_full there, branch-free
__device__ __forceinline__ float expf_nonpos(float x)
{
    float e = expf_core(__builtin_fmaxf(x, -87.0f));   // fmax(NaN, -87) = -87
    e = (x < -87.0f) ? 0.0f : e;
    return (x != x) ? x : e;
}

__device__ __forceinline__ float logf_full(float x)
{
    if (x != x) return x;
    if (x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    int e;
    float m = __builtin_frexpf(x, &e);
    if (m < 0.707106769f) { m = m + m; e = e - 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    float p = 9.09090936e-02f;
    p = __builtin_fmaf(p, z, 1.11111112e-01f);
    p = __builtin_fmaf(p, z, 1.42857149e-01f);
    p = __builtin_fmaf(p, z, 2.00000003e-01f);
    p = __builtin_fmaf(p, z, 3.33333343e-01f);
    const float s2 = s + s;
    const float lm = __builtin_fmaf(s2 * z, p, s2);
    const float ef = (float)e;
    return __builtin_fmaf(ef, u2f(0x3f317200u), __builtin_fmaf(ef, u2f(0x35bfbe8eu), lm));
}

// (int) cast with the reference's device semantics: truncate, saturate, NaN -> 0
__device__ __forceinline__ int f2i_sat(float x)
{
    if (x != x) return 0;
    if (x >= 2147483648.0f) return 0x7fffffff;
    if (x <= -2147483648.0f) return (int)0x80000000;
    return (int)x;
}

__device__ __forceinline__ unsigned clamp_tile(int v, unsigned g)
{
    v = v < 0 ? 0 : v;
    return (unsigned)v > g ? g : (unsigned)v;
}

// Square tile rect of an integer radius (the binning rule): float arithmetic
// left to right, truncation toward zero, clamped to [0, grid].
__device__ __forceinline__ void rect_int(float px, float py, int r, unsigned gx, unsigned gy,
                                         unsigned& x0, unsigned& y0, unsigned& x1, unsigned& y1)
{
    const float rf = (float)r;
    x0 = clamp_tile(f2i_sat((px - rf) / 16.0f), gx);
    y0 = clamp_tile(f2i_sat((py - rf) / 16.0f), gy);
    x1 = clamp_tile(f2i_sat(((px + rf) + 16.0f - 1.0f) / 16.0f), gx);
    y1 = clamp_tile(f2i_sat(((py + rf) + 16.0f - 1.0f) / 16.0f), gy);
}

// Gaussian falloff exponent in the fixed FMA order; ha = -0.5*a, hc = -0.5*c, nb = -b
__device__ __forceinline__ float power_of(float ha, float nb, float hc, float dx, float dy)
{
    return __builtin_fmaf(ha * dx, dx, __builtin_fmaf(hc * dy, dy, (nb * dx) * dy));
}

// ---- wave64 helpers -------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, true));
}

// Sum over the 64 lanes; the result is valid in lane 63 (row_shr scan inside
// each 16-lane row, then row_bcast:15 / row_bcast:31 across rows).
__device__ __forceinline__ float wave_sum_to_lane63(float v)
{
    v = v + dpp_f<0x111>(v);          // row_shr:1
    v = v + dpp_f<0x112>(v);          // row_shr:2
    v = v + dpp_f<0x114>(v);          // row_shr:4
    v = v + dpp_f<0x118>(v);          // row_shr:8
    v = v + dpp_f<0x142, 0xa>(v);     // row_bcast:15 into rows 1 and 3
    v = v + dpp_f<0x143, 0xc>(v);     // row_bcast:31 into rows 2 and 3
    return v;
}

__device__ __forceinline__ float bcast63(float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63)); }

// Sum over the 64 lanes, returned (uniform) in every lane.  Must be called
// with all 64 lanes active.
__device__ __forceinline__ float wave_sum(float v) { return bcast63(wave_sum_to_lane63(v)); }

__device__ __forceinline__ int wave_sum_i(int v)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ int wave_max_i(int v)
{
    for (int off = 32; off > 0; off >>= 1) {
        const int o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

}  // namespace gs
