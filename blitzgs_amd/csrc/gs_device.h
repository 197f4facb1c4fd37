// Device-side scalar helpers shared by the rasterizer kernels (gfx950).
//
// The library is compiled with -ffp-contract=off: a*b+c is never fused
// implicitly, every fused multiply-add is an explicit __builtin_fmaf, and fp32
// division and sqrt are correctly rounded (HIP's default).  Together with the
// fixed operation order below this makes the per-Gaussian preprocess and the
// tile keys bit-reproducible on a CPU; the blend's falloff uses the hardware
// exp2 (expf_fast), with the exact exp around each Gaussian's alpha cut-off.
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

// Streaming (non-temporal) stores for large write-once outputs: the hint keeps
// the written lines from displacing cached lines that later kernels re-read.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st_stream(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void st_stream(int* p, int v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void st_stream(float2* p, float2 v)
{
    __builtin_nontemporal_store(f32x2_t{v.x, v.y}, reinterpret_cast<f32x2_t*>(p));
}
__device__ __forceinline__ void st_stream(float4* p, float4 v)
{
    __builtin_nontemporal_store(f32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4_t*>(p));
}

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

// The blend's Gaussian falloff G = exp(power), power <= 0 or NaN: the
// hardware exp2 (v_exp_f32) of power * log2(e).  Relative to the exact
// expf_nonpos it is off by at most ~1e-5 for power >= -87 (the rounding of
// the product, ~|power| * 6e-8, plus about one ulp); below that both are far
// under 1/255.  NaN stays NaN.
__device__ __forceinline__ float expf_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504f); }

// The power at which opacity * exp(power) = 1/255, -log(255 * opacity), is
// each Gaussian's alpha cut-off (computed once per Gaussian with logf_full,
// below).  ALPHA_GUARD is the half-width of the window around it in which
// blend_alpha evaluates G exactly: 3e-5 in power, i.e. a relative window of
// 3e-5 in opacity * G, far above the fast exp's error there (power >= -6 for
// opacity >= 1/255: <= ~5e-7) plus the cut-off's own rounding (~1e-6).
constexpr float ALPHA_GUARD = 3e-5f;

// alpha = min(0.99, opacity * G) of one (pixel, Gaussian) evaluation with the
// fast exp; where power lies within ALPHA_GUARD of the Gaussian's cut-off
// power (any lane of the wave), G is the exact expf_nonpos instead, so the
// decision alpha >= 1/255 is the one the exact evaluation makes.  The window
// test needs only power, not the exp, so the exp's latency overlaps it.  G is
// returned too.
__device__ __forceinline__ float blend_alpha(float opacity, float power, float cut_power, float& G)
{
    const bool near = __builtin_fabsf(power - cut_power) <= ALPHA_GUARD;
    G = expf_fast(power);
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(near) != 0, 0)) {
        if (near) G = expf_nonpos(power);
    }
    return __builtin_fminf(0.99f, opacity * G);
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
// the power at which opacity * exp(power) reaches 1/255 (blend_alpha's
// window centre): NaN for a NaN opacity, +inf for opacity 0
__device__ __forceinline__ float alpha_cut_power(float opacity) { return -logf_full(255.0f * opacity); }

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

// Conservative test: can a Gaussian (mean mx,my; conic a,b,c; opacity o)
// reach alpha >= 1/255 at any pixel centre of the rectangle [x0,x1]x[y0,y1]?
// The maximum of the concave falloff exponent over the rectangle is found in
// double precision (the convex quadratic form's minimum lies at the clamped
// stationary point of one of the four edges when the mean is outside); the
// test keeps a margin of 1e-3 + 1e-6 * M, where M bounds the magnitude of the
// fp32 terms of the per-pixel exponent, far above the fp32 rounding of that
// exponent (a few ulp of M) and of exp, and far above the double rounding of
// the stationary point (which moves the edge minimum only quadratically).  A
// false answer therefore implies that the exact per-pixel fp32 evaluation
// skips the Gaussian at every pixel of the rectangle, so culling with it
// leaves the blend's results unchanged.  Non-finite inputs and
// non-positive-definite conics are always kept.
//
// The per-Gaussian part is computed once per Gaussian by cull_prepare, in
// fp32: the threshold -log(255 o) (relative error ~1e-7 of a value <= 5.6,
// far inside the margin) and the edge slopes -b/c, -b/a (an error in the
// stationary point moves the edge minimum only quadratically).  A NaN
// threshold means "always keep", +inf "never" (opacity below 1/255).
// may_touch_prepared is the per-rectangle part.
struct CullPrep {
    float thresh, nbc, nba;
};

__device__ __forceinline__ CullPrep cull_prepare(float mx, float my, float ca, float cb, float cc, float o)
{
    const float qnan = __builtin_nanf("");
    CullPrep r{qnan, 0.f, 0.f};
    if (o != o) return r;
    if (o < 1.0f / 255.0f) { r.thresh = __builtin_huge_valf(); return r; }   // alpha <= o with G <= 1
    if (!(__builtin_isfinite(mx) && __builtin_isfinite(my) && __builtin_isfinite(o))) return r;
    const double a = ca, b = cb, c = cc;
    if (!(a > 0.0 && c > 0.0 && a * c - b * b > 0.0)) return r;
    r.thresh = -logf_full(255.0f * o);
    r.nbc = -cb * __builtin_amdgcn_rcpf(cc);
    r.nba = -cb * __builtin_amdgcn_rcpf(ca);
    return r;
}

__device__ __forceinline__ bool may_touch_prepared(float thresh, float nbc, float nba, float mx, float my, float ca,
                                                   float cb, float cc, float x0, float y0, float x1, float y1)
{
    if (thresh != thresh) return true;
    if (thresh == __builtin_huge_valf()) return false;
    const double a = ca, b = cb, c = cc;
    const double dxl = (double)mx - (double)x1, dxh = (double)mx - (double)x0;
    const double dyl = (double)my - (double)y1, dyh = (double)my - (double)y0;
    if (dxl <= 0.0 && dxh >= 0.0 && dyl <= 0.0 && dyh >= 0.0) return true;
    double best = __builtin_huge_val();
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const double dx = e ? dxh : dxl;
        const double dy = __builtin_fmin(__builtin_fmax((double)nbc * dx, dyl), dyh);
        best = __builtin_fmin(best, a * dx * dx + 2.0 * b * dx * dy + c * dy * dy);
    }
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const double dy = e ? dyh : dyl;
        const double dx = __builtin_fmin(__builtin_fmax((double)nba * dy, dxl), dxh);
        best = __builtin_fmin(best, a * dx * dx + 2.0 * b * dx * dy + c * dy * dy);
    }
    const double DX = __builtin_fmax(__builtin_fabs(dxl), __builtin_fabs(dxh));
    const double DY = __builtin_fmax(__builtin_fabs(dyl), __builtin_fabs(dyh));
    const double M = 0.5 * (a * DX * DX + c * DY * DY) + __builtin_fabs(b) * DX * DY;
    const double margin = 1e-3 + 1e-6 * M;
    return -0.5 * best + margin >= (double)thresh;
}

// Tile test of the full-image path's duplicateWithKeys (reference
// diff-gaussian-rasterization_f/cuda_rasterizer/rasterizer_impl.cu:56-95,
// 144-167, max_contrib_power_rect_gaussian_float<15,15>): the falloff exponent
// 0.5 (a dx^2 + c dy^2) + b dx dy at the point of the tile's pixel rect
// [16 tx, 16 tx + 15] x [16 ty, 16 ty + 15] the reference picks (the mean if
// inside; else along the nearest edge), kept when <= thr = log(opacity * 255).
// Left-to-right fp32, no contraction; 1/(225 a) a correctly rounded division;
// saturate maps NaN to 0.
__device__ __forceinline__ float sat01(float v) { return v > 0.0f ? (v < 1.0f ? v : 1.0f) : 0.0f; }

__device__ __forceinline__ bool full_tile_keep(float mx, float my, float a, float b, float c, float thr, unsigned tx,
                                               unsigned ty)
{
    const float rminx = (float)(tx * 16u), rminy = (float)(ty * 16u);
    const float rmaxx = (float)((tx + 1u) * 16u - 1u), rmaxy = (float)((ty + 1u) * 16u - 1u);
    const float x_min_diff = rminx - mx;
    const float x_left = x_min_diff > 0.0f ? 1.0f : 0.0f;
    const float not_in_x = x_left + (mx > rmaxx ? 1.0f : 0.0f);
    const float y_min_diff = rminy - my;
    const float y_above = y_min_diff > 0.0f ? 1.0f : 0.0f;
    const float not_in_y = y_above + (my > rmaxy ? 1.0f : 0.0f);
    float power = 0.0f;
    if ((not_in_y + not_in_x) > 0.0f) {
        const float px = x_left * rminx + (1.0f - x_left) * rmaxx;
        const float py = y_above * rminy + (1.0f - y_above) * rmaxy;
        const float dx = __builtin_copysignf(15.0f, x_min_diff);
        const float dy = __builtin_copysignf(15.0f, y_min_diff);
        const float diffx = mx - px, diffy = my - py;
        const float rcp_x = 1.0f / (225.0f * a);
        const float rcp_y = 1.0f / (225.0f * c);
        const float tx_ = not_in_y * sat01((dx * a * diffx + dx * b * diffy) * rcp_x);
        const float ty_ = not_in_x * sat01((dy * b * diffx + dy * c * diffy) * rcp_y);
        const float qx = px + tx_ * dx, qy = py + ty_ * dy;
        const float ex = mx - qx, ey = my - qy;
        power = 0.5f * (a * ex * ex + c * ey * ey) + b * ex * ey;
    }
    return power <= thr;
}

// Float-extent tile rect of the full-image path (getRect(float2, float2),
// reference auxiliary.h:63-73): floor / ceil of (mean -+ extent) / 16, clamped.
__device__ __forceinline__ void rect_float(float px, float py, float ex, float ey, unsigned gx, unsigned gy,
                                           unsigned& x0, unsigned& y0, unsigned& x1, unsigned& y1)
{
    x0 = clamp_tile(f2i_sat(__builtin_floorf((px - ex) / 16.0f)), gx);
    y0 = clamp_tile(f2i_sat(__builtin_floorf((py - ey) / 16.0f)), gy);
    x1 = clamp_tile(f2i_sat(__builtin_ceilf((px + ex) / 16.0f)), gx);
    y1 = clamp_tile(f2i_sat(__builtin_ceilf((py + ey) / 16.0f)), gy);
}

// ---- wave64 helpers -------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// the writelane intrinsic (v_writelane_b32), which this compiler has no
// builtin for: (value, lane, old)
__device__ int gs_llvm_writelane(int x, int lane, int old) __asm("llvm.amdgcn.writelane.i32");

// v with lane `lane` (wave-uniform) replaced by the wave-uniform value x
__device__ __forceinline__ uint32_t write_lane(uint32_t v, uint32_t x, int lane)
{
    return (uint32_t)gs_llvm_writelane((int)x, lane, (int)v);
}

// number of set bits of m below this lane
__device__ __forceinline__ int rank_below(uint64_t m)
{
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Exclusive scan of one value per thread over a 1024-thread block; returns
// the prefix and writes the block total to *total (all threads).
__device__ __forceinline__ uint32_t block_excl_scan_1024(uint32_t v, uint32_t* s_wave, uint32_t* total)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) s_wave[wid] = x;
    __syncthreads();
    if (wid == 0) {
        uint32_t w = lane < 16 ? s_wave[lane] : 0;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const uint32_t y = __shfl_up(w, off, 64);
            if (lane >= off) w += y;
        }
        if (lane < 16) s_wave[16 + lane] = w;
    }
    __syncthreads();
    const uint32_t wbase = wid == 0 ? 0 : s_wave[16 + wid - 1];
    *total = s_wave[31];
    __syncthreads();
    return wbase + x - v;
}

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

// Twelve per-lane values summed over the wave at once (gfx950 lane swaps),
// each level a transpose-add: two registers exchange halves of their lanes so
// that one register carries the pairwise sums of both:
//   level 1  v_permlane32_swap pairs (v0,v1),...: one register holds 32-lane
//            partials of v[2i] in lanes 0-31 and of v[2i+1] in lanes 32-63;
//   level 2  v_permlane16_swap pairs of those: each 16-lane row of register
//            t[j] holds 16 partials of value 4j + m(row), m = 0,2,1,3;
//   level 3  DPP row_ror:8 (lane c of a row <-> c ^ 8): t0 and t1 share a
//            register, t0's values in lanes 0-7 of each row and t1's in lanes
//            8-15 (8 partials); t2 is folded onto itself;
//   level 4  DPP row_half_mirror (c <-> 7 - c inside each 8-lane half): that
//            register and t2's share one, t2's values in lanes 4-7 of each
//            half (4 partials);
//   level 5, 6  DPP quad_perm xor 2, xor 1: every lane of an aligned group of
//            four holds its value's total.
// 27 VALU operations instead of 12 separate full-wave reductions.  Lane L
// returns the total of value wave_sum12_index(L) (-1: a duplicate or
// nothing).  All lanes must be active.  ABS23: values 2 and 3 are summed as
// absolute values (the first level adds |a| + |b|, which costs nothing:
// source modifiers).
template <bool ABS23 = false>
__device__ __forceinline__ float wave_sum12(const float (&v)[12])
{
    float s[6];
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[2 * i]), __float_as_uint(v[2 * i + 1]),
                                                        false, false);
        const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
        s[i] = (ABS23 && i == 1) ? __builtin_fabsf(a) + __builtin_fabsf(b) : a + b;
    }
    float t[3];
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(s[2 * j]), __float_as_uint(s[2 * j + 1]),
                                                        false, false);
        t[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const int c = lane_id() & 15;
    // level 3: lanes c < 8 keep t0, c >= 8 t1; the partner c ^ 8 brings the other half
    const bool lo8 = c < 8;
    const float z = (lo8 ? t[0] : t[1]) + dpp_f<0x128>(lo8 ? t[1] : t[0]);   // row_ror:8
    const float t2 = t[2] + dpp_f<0x128>(t[2]);
    // level 4: lanes c % 8 < 4 keep z, the others t2; the partner 7 - c brings the rest
    const bool lo4 = (c & 7) < 4;
    float w = (lo4 ? z : t2) + dpp_f<0x141>(lo4 ? t2 : z);                    // row_half_mirror
    w = w + dpp_f<0x4e>(w);                                                   // quad_perm [2,3,0,1]
    w = w + dpp_f<0xb1>(w);                                                   // quad_perm [1,0,3,2]
    return w;
}

// the value whose total lane `lane` holds after wave_sum12: lane 16 r + c
// with c = 0 (t0), 4 (t2) or 8 (t1) of row r; -1 for the other lanes
__device__ __forceinline__ int wave_sum12_index(int lane)
{
    const int r = lane >> 4, c = lane & 15;
    const int m = r == 0 ? 0 : (r == 1 ? 2 : (r == 2 ? 1 : 3));
    return c == 0 ? m : (c == 4 ? 8 + m : (c == 8 ? 4 + m : -1));
}

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
