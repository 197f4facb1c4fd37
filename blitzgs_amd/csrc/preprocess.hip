// Per-Gaussian preprocess, forward and backward, for gfx950.
//
// Forward  (reference: BlitzGS submodule/diff-gaussian-rasterization_f,
//           cuda_rasterizer/forward.cu:28-284, auxiliary.h:41-184, host side
//           rasterizer_impl.cu:982-1067 and rasterize_points.cu:834-923):
//   near cull, EWA projection with the 0.3 low-pass, conic, opacity-aware
//   radius and float tile rect, SH (degree <= 3) colour with clamp flags.
// Backward (reference: same package, cuda_rasterizer/backward.cu:20-400,
//           rasterizer_impl.cu:1069-1129, rasterize_points.cu:926-1029):
//   the reference's two kernels (computeCov2DCUDA, preprocessCUDA) fused into
//   one pass that reads dL/dconic_opacity and dL/dmeans2D directly (no
//   (P,2,2) repack, no (P,3) padding, no dc/rest split and no dL/dcov3D
//   round trip through memory) and writes dL/dsh as (P,K,3) in place.
//
// The full-image path (GaussianRasterizer.forward / render_simp; reference
// forward.cu:165-284 and backward.cu:759-827 with the arguments
// rasterizer_impl.cu:396-424 and 931-954 pass) runs the same kernels with
// FULL = true: a culling mask, precomputed colours or 3D covariances, the SH
// DC term and the remaining coefficients in separate arrays, the float tile
// rect extents and tile counts as extra outputs, and dL/dcov3D, dL/ddc,
// dL/drest as separate gradients.
//
// One thread per Gaussian.  Every output element is written (zeros for culled
// Gaussians), so callers need not clear the outputs.  The forward arithmetic
// is the fixed-order fp32 sequence that oracle/o_preprocess.c restates on the
// CPU; with -ffp-contract=off the two agree bit for bit.
#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {

constexpr float SH_C0 = 0.28209479177387814f;
constexpr float SH_C1 = 0.4886025119029199f;
constexpr float SH_C2_0 = 1.0925484305920792f, SH_C2_1 = -1.0925484305920792f,
                SH_C2_2 = 0.31539156525252005f, SH_C2_3 = -1.0925484305920792f,
                SH_C2_4 = 0.5462742152960396f;
constexpr float SH_C3_0 = -0.5900435899266435f, SH_C3_1 = 2.890611442640554f,
                SH_C3_2 = -0.4570457994644658f, SH_C3_3 = 0.3731763325901154f,
                SH_C3_4 = -0.4570457994644658f, SH_C3_5 = 1.445305721320277f,
                SH_C3_6 = -0.5900435899266435f;

struct Cam {
    float v[16];
    float p[16];
    float c[3];
};

__device__ __forceinline__ void load_cam(Cam& cam, const float* __restrict__ view, const float* __restrict__ proj,
                                         const float* __restrict__ campos)
{
#pragma unroll
    for (int i = 0; i < 16; i++) { cam.v[i] = view[i]; cam.p[i] = proj[i]; }
    cam.c[0] = campos[0]; cam.c[1] = campos[1]; cam.c[2] = campos[2];
}

__device__ __forceinline__ void xform3(const float* m, float x, float y, float z, float* o)
{
    o[0] = m[0] * x + m[4] * y + m[8] * z + m[12];
    o[1] = m[1] * x + m[5] * y + m[9] * z + m[13];
    o[2] = m[2] * x + m[6] * y + m[10] * z + m[14];
}

__device__ __forceinline__ float xform_w(const float* m, float x, float y, float z)
{
    return m[3] * x + m[7] * y + m[11] * z + m[15];
}

__device__ __forceinline__ float ndc2pix(float v, int S)
{
    return (float)((((double)v + 1.0) * (double)S - 1.0) * 0.5);
}

// Rm: glm rotation matrix of the reference read row-wise (un-normalised quat)
__device__ __forceinline__ void quat_rows(float r, float x, float y, float z, float Rm[3][3])
{
    Rm[0][0] = 1.f - 2.f * (y * y + z * z); Rm[0][1] = 2.f * (x * y + r * z); Rm[0][2] = 2.f * (x * z - r * y);
    Rm[1][0] = 2.f * (x * y - r * z); Rm[1][1] = 1.f - 2.f * (x * x + z * z); Rm[1][2] = 2.f * (y * z + r * x);
    Rm[2][0] = 2.f * (x * z + r * y); Rm[2][1] = 2.f * (y * z - r * x); Rm[2][2] = 1.f - 2.f * (x * x + y * y);
}

struct Ewa {
    float t0, t1, t2;
    float u[3], w[3];
    float xmask, ymask;
};

__device__ __forceinline__ void ewa_setup(const float* V, float mx, float my, float mz, float fx, float fy,
                                          float tanfovx, float tanfovy, Ewa& e)
{
    float t[3];
    xform3(V, mx, my, mz, t);
    const float limx = 1.3f * tanfovx;
    const float limy = 1.3f * tanfovy;
    const float txtz = t[0] / t[2];
    const float tytz = t[1] / t[2];
    t[0] = __builtin_fminf(limx, __builtin_fmaxf(-limx, txtz)) * t[2];
    t[1] = __builtin_fminf(limy, __builtin_fmaxf(-limy, tytz)) * t[2];
    e.xmask = (txtz < -limx || txtz > limx) ? 0.f : 1.f;
    e.ymask = (tytz < -limy || tytz > limy) ? 0.f : 1.f;
    e.t0 = t[0]; e.t1 = t[1]; e.t2 = t[2];
    const float tz2 = t[2] * t[2];
    const float J00 = fx / t[2];
    const float J11 = fy / t[2];
    const float J20 = -(fx * t[0]) / tz2;
    const float J21 = -(fy * t[1]) / tz2;
#pragma unroll
    for (int r = 0; r < 3; r++) {
        e.u[r] = V[r * 4 + 0] * J00 + V[r * 4 + 2] * J20;
        e.w[r] = V[r * 4 + 1] * J11 + V[r * 4 + 2] * J21;
    }
}

__device__ __forceinline__ void symv(const float* c6, const float* v, float* o)
{
    o[0] = c6[0] * v[0] + c6[1] * v[1] + c6[2] * v[2];
    o[1] = c6[1] * v[0] + c6[3] * v[1] + c6[4] * v[2];
    o[2] = c6[2] * v[0] + c6[4] * v[1] + c6[5] * v[2];
}

// Load the first NC (= (DEG+1)^2) coefficients of one Gaussian's SH block.
template <int NC>
__device__ __forceinline__ void load_sh(const float* __restrict__ base, bool vec16, float* s)
{
    if (vec16) {
        const float4* b4 = reinterpret_cast<const float4*>(base);
#pragma unroll
        for (int i = 0; i < (3 * NC + 3) / 4; i++) {
            const float4 v = b4[i];
            if (4 * i + 0 < 3 * NC) s[4 * i + 0] = v.x;
            if (4 * i + 1 < 3 * NC) s[4 * i + 1] = v.y;
            if (4 * i + 2 < 3 * NC) s[4 * i + 2] = v.z;
            if (4 * i + 3 < 3 * NC) s[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 3 * NC; i++) s[i] = base[i];
    }
}

template <int DEG>
__device__ __forceinline__ void sh_color(float x, float y, float z, const float* s, float* out, bool* clamped)
{
#pragma unroll
    for (int c = 0; c < 3; c++) {
        float r = SH_C0 * s[c];
        if (DEG > 0) {
            r = r - (SH_C1 * y) * s[3 + c] + (SH_C1 * z) * s[6 + c] - (SH_C1 * x) * s[9 + c];
            if (DEG > 1) {
                const float xx = x * x, yy = y * y, zz = z * z;
                const float xy = x * y, yz = y * z, xz = x * z;
                r = r + (SH_C2_0 * xy) * s[12 + c] + (SH_C2_1 * yz) * s[15 + c] +
                    (SH_C2_2 * (2.0f * zz - xx - yy)) * s[18 + c] +
                    (SH_C2_3 * xz) * s[21 + c] + (SH_C2_4 * (xx - yy)) * s[24 + c];
                if (DEG > 2) {
                    r = r + ((SH_C3_0 * y) * (3.0f * xx - yy)) * s[27 + c] +
                        ((SH_C3_1 * xy) * z) * s[30 + c] +
                        ((SH_C3_2 * y) * (4.0f * zz - xx - yy)) * s[33 + c] +
                        ((SH_C3_3 * z) * (2.0f * zz - 3.0f * xx - 3.0f * yy)) * s[36 + c] +
                        ((SH_C3_4 * x) * (4.0f * zz - xx - yy)) * s[39 + c] +
                        ((SH_C3_5 * z) * (xx - yy)) * s[42 + c] +
                        ((SH_C3_6 * x) * (xx - 3.0f * yy)) * s[45 + c];
                }
            }
        }
        r = r + 0.5f;
        clamped[c] = r < 0.0f;
        out[c] = __builtin_fmaxf(r, 0.0f);
    }
}

// Extra inputs and outputs of the full-image path's preprocess.
struct FullPre {
    const uint8_t* culling;          // P, nonzero = skip
    const float* colors_precomp;     // P x 3 or null (null: SH colour)
    const float* cov3D_precomp;      // P x 6 or null (null: from scale and rotation)
    const float* dc;                 // P x 3
    const float* rest;               // P x M x 3
    int M;
    float* rects;                    // P x 2 float tile-rect extents
    uint32_t* tiles_touched;         // P
};

// SH coefficients of one Gaussian from the DC array and the rest array.
template <int NC>
__device__ __forceinline__ void load_sh_split(const float* __restrict__ dc, const float* __restrict__ rest, float* s)
{
    s[0] = dc[0]; s[1] = dc[1]; s[2] = dc[2];
#pragma unroll
    for (int i = 0; i < 3 * (NC - 1); i++) s[3 + i] = rest[i];
}

// 3D covariance (upper triangle) from a Gaussian's scale s (before the
// modifier) and rotation quaternion q: Sigma = M^T M with
// M = diag(mod * scale) R (reference forward.cu:118-150).  The backward
// recomputes it with this same function when the forward's copy was not kept.
__device__ __forceinline__ void cov3d_from(const float* s_raw, float4 q, float mod, float* c6)
{
    float Rm[3][3];
    quat_rows(q.x, q.y, q.z, q.w, Rm);
    const float s[3] = {mod * s_raw[0], mod * s_raw[1], mod * s_raw[2]};
    float M[3][3];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) M[i][j] = s[i] * Rm[i][j];
    c6[0] = M[0][0] * M[0][0] + M[1][0] * M[1][0] + M[2][0] * M[2][0];
    c6[1] = M[0][0] * M[0][1] + M[1][0] * M[1][1] + M[2][0] * M[2][1];
    c6[2] = M[0][0] * M[0][2] + M[1][0] * M[1][2] + M[2][0] * M[2][2];
    c6[3] = M[0][1] * M[0][1] + M[1][1] * M[1][1] + M[2][1] * M[2][1];
    c6[4] = M[0][1] * M[0][2] + M[1][1] * M[1][2] + M[2][1] * M[2][2];
    c6[5] = M[0][2] * M[0][2] + M[1][2] * M[1][2] + M[2][2] * M[2][2];
}

// The preprocess backward's per-Gaussian record (gs_preprocess_forward_rec):
// the inputs the backward reads for a visible Gaussian, packed by the forward
// into 48 bytes so that the backward reads them as three 16-byte loads from a
// dense run instead of gathering 12-, 12-, 16- and 3-byte rows of the input
// arrays (a wave's visible Gaussians, about one in five at the benchmark's
// scene, touch nearly every cache line of those arrays).  Per wave of 64
// Gaussians [64w, 64w+64): mask[w] = the ballot of the visible ones, and
// records 64w .. 64w + popcount(mask[w]) - 1 hold them in index order.
//   r0 = (mean x, y, z, scale 0), r1 = (scale 1, scale 2, clamp bits, index),
//   r2 = rotation quaternion as given (not normalised).
struct BwdRec {
    float4* rec;
    uint64_t* mask;
};

inline size_t bwdrec_mask_bytes(int P) { return (((size_t)gs_div_up((size_t)P, 64) * 8 + 255) / 256) * 256; }
inline size_t bwdrec_bytes(int P) { return bwdrec_mask_bytes(P) + (size_t)gs_div_up((size_t)P, 64) * 64 * 48; }

template <int DEG, bool FULL>
__global__ __launch_bounds__(256) void preprocess_fwd_kernel(
    int P, int K, int W, int H, float tanfovx, float tanfovy, float fx, float fy, float mod,
    const float* __restrict__ view, const float* __restrict__ proj, const float* __restrict__ campos,
    const float* __restrict__ means3D, const float* __restrict__ scales, const float* __restrict__ rotations,
    const float* __restrict__ sh, int sh_vec16, const float* __restrict__ opacities,
    float* __restrict__ means2D, float* __restrict__ depths, int* __restrict__ radii, float* __restrict__ cov3D,
    float* __restrict__ conic_opacity, float* __restrict__ rgb, uint8_t* __restrict__ clamped, FullPre F,
    BwdRec rec)
{
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= P) return;
    Cam cam;
    load_cam(cam, view, proj, campos);
    const unsigned gx = (unsigned)((W + 15) / 16), gy = (unsigned)((H + 15) / 16);

    const float mx = means3D[3 * idx], my = means3D[3 * idx + 1], mz = means3D[3 * idx + 2];
    float o_m2d[2] = {0.f, 0.f}, o_depth = 0.f, o_con[4] = {0.f, 0.f, 0.f, 0.f}, o_rgb[3] = {0.f, 0.f, 0.f};
    float c6[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float s_raw[3] = {0.f, 0.f, 0.f};
    float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
    int o_radius = 0;
    bool o_clamp[3] = {false, false, false};
    float o_ex = 0.f, o_ey = 0.f;
    uint32_t o_tiles = 0;

    do {
        if (FULL && F.culling[idx]) break;
        float pv[3];
        xform3(cam.v, mx, my, mz, pv);
        if (pv[2] <= 0.2f) break;
        float ph[3];
        xform3(cam.p, mx, my, mz, ph);
        const float pw = 1.0f / (xform_w(cam.p, mx, my, mz) + 0.0000001f);
        const float pp0 = ph[0] * pw, pp1 = ph[1] * pw;

        if (FULL && F.cov3D_precomp != nullptr) {
#pragma unroll
            for (int k = 0; k < 6; k++) c6[k] = F.cov3D_precomp[6 * (size_t)idx + k];
        } else {
            q = reinterpret_cast<const float4*>(rotations)[idx];
            s_raw[0] = scales[3 * idx]; s_raw[1] = scales[3 * idx + 1]; s_raw[2] = scales[3 * idx + 2];
            cov3d_from(s_raw, q, mod, c6);
        }

        Ewa e;
        ewa_setup(cam.v, mx, my, mz, fx, fy, tanfovx, tanfovy, e);
        float Su[3], Sw[3];
        symv(c6, e.u, Su);
        symv(c6, e.w, Sw);
        float ca = e.u[0] * Su[0] + e.u[1] * Su[1] + e.u[2] * Su[2];
        const float cb = e.u[0] * Sw[0] + e.u[1] * Sw[1] + e.u[2] * Sw[2];
        float cc = e.w[0] * Sw[0] + e.w[1] * Sw[1] + e.w[2] * Sw[2];
        ca = ca + 0.3f;
        cc = cc + 0.3f;

        const float det = ca * cc - cb * cb;
        if (det == 0.0f) break;
        const float det_inv = 1.f / det;

        const float opacity = opacities[idx];
        const float opt = gs::logf_full(opacity / (1.0f / 255.0f));
        const float sq = __builtin_sqrtf(2.0f * opt);
        const float extent = (sq != sq || (double)sq >= 3.33) ? (float)3.33 : sq;
        const float mid = 0.5f * (ca + cc);
        const float lambda = mid + __builtin_sqrtf(__builtin_fmaxf(0.01f, mid * mid - det));
        const float my_radius = extent * __builtin_sqrtf(lambda);
        if (my_radius <= 0.0f) break;

        const float pix0 = ndc2pix(pp0, W), pix1 = ndc2pix(pp1, H);
        const float ex = __builtin_fminf(extent * __builtin_sqrtf(ca), my_radius);
        const float ey = __builtin_fminf(extent * __builtin_sqrtf(cc), my_radius);
        const unsigned rminx = gs::clamp_tile(gs::f2i_sat(__builtin_floorf((pix0 - ex) / 16.0f)), gx);
        const unsigned rminy = gs::clamp_tile(gs::f2i_sat(__builtin_floorf((pix1 - ey) / 16.0f)), gy);
        const unsigned rmaxx = gs::clamp_tile(gs::f2i_sat(__builtin_ceilf((pix0 + ex) / 16.0f)), gx);
        const unsigned rmaxy = gs::clamp_tile(gs::f2i_sat(__builtin_ceilf((pix1 + ey) / 16.0f)), gy);
        const uint32_t tiles = (rmaxx - rminx) * (rmaxy - rminy);
        if (tiles == 0) break;

        // SH -> RGB (only Gaussians that survive every cull read their SH block)
        if (!FULL || F.colors_precomp == nullptr) {
            constexpr int NC = (DEG + 1) * (DEG + 1);
            float s[3 * NC];
            if (FULL)
                load_sh_split<NC>(F.dc + 3 * (size_t)idx, F.rest + (size_t)idx * F.M * 3, s);
            else
                load_sh<NC>(sh + (size_t)idx * K * 3, sh_vec16 != 0, s);
            float dir0 = mx - cam.c[0], dir1 = my - cam.c[1], dir2 = mz - cam.c[2];
            const float len = __builtin_sqrtf(dir0 * dir0 + dir1 * dir1 + dir2 * dir2);
            dir0 = dir0 / len; dir1 = dir1 / len; dir2 = dir2 / len;
            sh_color<DEG>(dir0, dir1, dir2, s, o_rgb, o_clamp);
        }

        o_depth = pv[2];
        o_radius = gs::f2i_sat(__builtin_ceilf(my_radius));
        o_m2d[0] = pix0; o_m2d[1] = pix1;
        o_con[0] = cc * det_inv;
        o_con[1] = -cb * det_inv;
        o_con[2] = ca * det_inv;
        o_con[3] = opacity;
        o_ex = ex;
        o_ey = ey;
        o_tiles = tiles;
    } while (0);

    if (FULL) {
        reinterpret_cast<float2*>(F.rects)[idx] = make_float2(o_ex, o_ey);
        F.tiles_touched[idx] = o_tiles;
    }

    reinterpret_cast<float2*>(means2D)[idx] = make_float2(o_m2d[0], o_m2d[1]);
    depths[idx] = o_depth;
    radii[idx] = o_radius;
    if (cov3D != nullptr) {   // (null: the caller keeps no copy; the backward recomputes it)
        float2* c2 = reinterpret_cast<float2*>(cov3D + 6 * (size_t)idx);
        c2[0] = make_float2(c6[0], c6[1]);
        c2[1] = make_float2(c6[2], c6[3]);
        c2[2] = make_float2(c6[4], c6[5]);
    }
    reinterpret_cast<float4*>(conic_opacity)[idx] = make_float4(o_con[0], o_con[1], o_con[2], o_con[3]);
    rgb[3 * idx + 0] = o_rgb[0];
    rgb[3 * idx + 1] = o_rgb[1];
    rgb[3 * idx + 2] = o_rgb[2];
    if (clamped != nullptr) {   // (null: the records hold the flags for the backward)
        clamped[3 * idx + 0] = o_clamp[0];
        clamped[3 * idx + 1] = o_clamp[1];
        clamped[3 * idx + 2] = o_clamp[2];
    }

    if (rec.rec != nullptr) {   // (split path only)
        const bool vis = o_radius > 0;
        const uint64_t m = __ballot(vis);
        const int lane = threadIdx.x & 63;
        if (vis) {
            const int rank = __popcll(m & ((1ull << lane) - 1ull));
            float4* r = rec.rec + 3 * (size_t)((idx & ~63) + rank);
            const uint32_t cbits = (o_clamp[0] ? 1u : 0u) | (o_clamp[1] ? 2u : 0u) | (o_clamp[2] ? 4u : 0u);
            r[0] = make_float4(mx, my, mz, s_raw[0]);
            r[1] = make_float4(s_raw[1], s_raw[2], __uint_as_float(cbits), __int_as_float(idx));
            r[2] = q;
        }
        if (lane == 0) rec.mask[idx >> 6] = m;   // lane 0 is the wave's lowest index, always < P here
    }
}

// dnormvdv (reference auxiliary.h:126-136)
__device__ __forceinline__ void dnormvdv3(const float* v, const float* dv, float* o)
{
    const float sum2 = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
    const float invsum32 = 1.0f / __builtin_sqrtf(sum2 * sum2 * sum2);
    o[0] = ((sum2 - v[0] * v[0]) * dv[0] - v[1] * v[0] * dv[1] - v[2] * v[0] * dv[2]) * invsum32;
    o[1] = (-v[0] * v[1] * dv[0] + (sum2 - v[1] * v[1]) * dv[1] - v[2] * v[1] * dv[2]) * invsum32;
    o[2] = (-v[0] * v[2] * dv[0] - v[1] * v[2] * dv[1] + (sum2 - v[2] * v[2]) * dv[2]) * invsum32;
}

template <int DEG>
__device__ __forceinline__ void sh_backward(float x, float y, float z, const float* s, const float* g,
                                            float* gsh, float* dx, float* dy, float* dz)
{
#pragma unroll
    for (int c = 0; c < 3; c++) { gsh[c] = SH_C0 * g[c]; dx[c] = 0.f; dy[c] = 0.f; dz[c] = 0.f; }
    if (DEG > 0) {
        const float b1 = -SH_C1 * y, b2 = SH_C1 * z, b3 = -SH_C1 * x;
#pragma unroll
        for (int c = 0; c < 3; c++) {
            gsh[3 + c] = b1 * g[c]; gsh[6 + c] = b2 * g[c]; gsh[9 + c] = b3 * g[c];
            dx[c] = -SH_C1 * s[9 + c];
            dy[c] = -SH_C1 * s[3 + c];
            dz[c] = SH_C1 * s[6 + c];
        }
        if (DEG > 1) {
            const float xx = x * x, yy = y * y, zz = z * z;
            const float xy = x * y, yz = y * z, xz = x * z;
            const float b4 = SH_C2_0 * xy, b5 = SH_C2_1 * yz, b6 = SH_C2_2 * (2.f * zz - xx - yy);
            const float b7 = SH_C2_3 * xz, b8 = SH_C2_4 * (xx - yy);
#pragma unroll
            for (int c = 0; c < 3; c++) {
                gsh[12 + c] = b4 * g[c]; gsh[15 + c] = b5 * g[c]; gsh[18 + c] = b6 * g[c];
                gsh[21 + c] = b7 * g[c]; gsh[24 + c] = b8 * g[c];
                dx[c] += SH_C2_0 * y * s[12 + c] + SH_C2_2 * 2.f * -x * s[18 + c] + SH_C2_3 * z * s[21 + c] + SH_C2_4 * 2.f * x * s[24 + c];
                dy[c] += SH_C2_0 * x * s[12 + c] + SH_C2_1 * z * s[15 + c] + SH_C2_2 * 2.f * -y * s[18 + c] + SH_C2_4 * 2.f * -y * s[24 + c];
                dz[c] += SH_C2_1 * y * s[15 + c] + SH_C2_2 * 2.f * 2.f * z * s[18 + c] + SH_C2_3 * x * s[21 + c];
            }
            if (DEG > 2) {
                const float b9 = SH_C3_0 * y * (3.f * xx - yy);
                const float b10 = SH_C3_1 * xy * z;
                const float b11 = SH_C3_2 * y * (4.f * zz - xx - yy);
                const float b12 = SH_C3_3 * z * (2.f * zz - 3.f * xx - 3.f * yy);
                const float b13 = SH_C3_4 * x * (4.f * zz - xx - yy);
                const float b14 = SH_C3_5 * z * (xx - yy);
                const float b15 = SH_C3_6 * x * (xx - 3.f * yy);
#pragma unroll
                for (int c = 0; c < 3; c++) {
                    gsh[27 + c] = b9 * g[c]; gsh[30 + c] = b10 * g[c]; gsh[33 + c] = b11 * g[c];
                    gsh[36 + c] = b12 * g[c]; gsh[39 + c] = b13 * g[c]; gsh[42 + c] = b14 * g[c];
                    gsh[45 + c] = b15 * g[c];
                    dx[c] += (SH_C3_0 * s[27 + c] * 3.f * 2.f * xy + SH_C3_1 * s[30 + c] * yz +
                              SH_C3_2 * s[33 + c] * -2.f * xy + SH_C3_3 * s[36 + c] * -3.f * 2.f * xz +
                              SH_C3_4 * s[39 + c] * (-3.f * xx + 4.f * zz - yy) +
                              SH_C3_5 * s[42 + c] * 2.f * xz + SH_C3_6 * s[45 + c] * 3.f * (xx - yy));
                    dy[c] += (SH_C3_0 * s[27 + c] * 3.f * (xx - yy) + SH_C3_1 * s[30 + c] * xz +
                              SH_C3_2 * s[33 + c] * (-3.f * yy + 4.f * zz - xx) +
                              SH_C3_3 * s[36 + c] * -3.f * 2.f * yz + SH_C3_4 * s[39 + c] * -2.f * xy +
                              SH_C3_5 * s[42 + c] * -2.f * yz + SH_C3_6 * s[45 + c] * -3.f * 2.f * xy);
                    dz[c] += (SH_C3_1 * s[30 + c] * xy + SH_C3_2 * s[33 + c] * 4.f * 2.f * yz +
                              SH_C3_3 * s[36 + c] * 3.f * (2.f * zz - xx - yy) +
                              SH_C3_4 * s[39 + c] * 4.f * 2.f * xz + SH_C3_5 * s[42 + c] * (xx - yy));
                }
            }
        }
    }
}

// Extra inputs and outputs of the full-image path's preprocess backward.
struct FullPreBwd {
    const float* cov3D_precomp;      // null: covariance from scale and rotation (and their gradients)
    int colors_precomp;              // nonzero: colours were given, no SH gradients
    const float* dc;                 // P x 3
    const float* rest;               // P x M x 3, null when M == 0 (then no SH gradients, as the reference)
    int M;
    float* dL_ddc;                   // P x 3
    float* dL_drest;                 // P x M x 3
    float* dL_dcov3D;                // P x 6
};

// Where preprocess_bwd_one reads a Gaussian's mean, scale (before the
// modifier), rotation and clamp flags: the input arrays, row idx ...
struct ArraySrc {
    const float* __restrict__ means3D;
    const float* __restrict__ scales;
    const float* __restrict__ rotations;
    const uint8_t* __restrict__ clamped;
    __device__ float3 mean(int idx) const
    {
        return make_float3(means3D[3 * idx], means3D[3 * idx + 1], means3D[3 * idx + 2]);
    }
    __device__ void scale(int idx, float* s) const
    {
        s[0] = scales[3 * idx]; s[1] = scales[3 * idx + 1]; s[2] = scales[3 * idx + 2];
    }
    __device__ float4 rot(int idx) const { return reinterpret_cast<const float4*>(rotations)[idx]; }
    __device__ bool clamp(int idx, int ch) const { return clamped[3 * idx + ch] != 0; }
};

// ... or the forward's record of it (BwdRec)
struct RecSrc {
    float4 r0, r1, r2;
    __device__ float3 mean(int) const { return make_float3(r0.x, r0.y, r0.z); }
    __device__ void scale(int, float* s) const { s[0] = r0.w; s[1] = r1.x; s[2] = r1.y; }
    __device__ float4 rot(int) const { return r2; }
    __device__ bool clamp(int, int ch) const { return ((__float_as_uint(r1.z) >> ch) & 1u) != 0; }
};

// Where preprocess_bwd_one reads a Gaussian's incoming gradients: the dense
// (P, k) arrays the render backward returned (dL/dmeans2D with a row stride,
// dL/dconic_opacity, dL/drgb) ...
struct DenseGrads {
    const float* __restrict__ m2d;
    int m2d_stride;
    const float* __restrict__ conic_op;
    const float* __restrict__ rgb_;
    __device__ float4 conic(int idx) const { return reinterpret_cast<const float4*>(conic_op)[idx]; }
    __device__ float mean2d(int idx, int c) const { return m2d[(size_t)idx * m2d_stride + c]; }
    __device__ float rgb(int idx, int ch) const { return rgb_[3 * idx + ch]; }
};

// ... or values the caller already holds (the render backward's accumulator
// row of the Gaussian, turned into those gradients)
struct HeldGrads {
    float4 co;
    float m[2], c[3];
    __device__ float4 conic(int) const { return co; }
    __device__ float mean2d(int, int k) const { return m[k]; }
    __device__ float rgb(int, int ch) const { return c[ch]; }
};

template <int DEG, bool STAGED, bool FULL, class Src, class Grads>
__device__ __forceinline__ void preprocess_bwd_one(
    int idx, int K, float tanfovx, float tanfovy, float fx, float fy, float mod,
    const float* __restrict__ view, const float* __restrict__ proj, const float* __restrict__ campos,
    const Src& src, const float* __restrict__ sh, int sh_vec16, const float* __restrict__ cov3D,
    const Grads& gr, float* __restrict__ m3_row, float* __restrict__ sc_row, float4* __restrict__ rot_row,
    float* __restrict__ dL_dsh, float* __restrict__ op_row, float* s_row, const FullPreBwd& F)
{
    // m3_row / sc_row / rot_row / op_row: where this Gaussian's dL/dmeans3D,
    // dL/dscales, dL/drotations and dL/dopacity go
    constexpr int NC = (DEG + 1) * (DEG + 1);
    const float4 gco = gr.conic(idx);
    *op_row = gco.w;
    float* gsh_out = FULL ? nullptr : dL_dsh + (size_t)idx * K * 3;
    const bool vec16 = sh_vec16 != 0;
    Cam cam;
    load_cam(cam, view, proj, campos);
    const float3 mean = src.mean(idx);
    const float mx = mean.x, my = mean.y, mz = mean.z;
    const float* V = cam.v;
    const float* PM = cam.p;

    // ---- SH backward first (the full path: only with SH colours and a rest
    // array): its 48 coefficients and gradients are dead before the
    // covariance backward starts; the mean term dm joins gm below, in the
    // same order as before
    const bool sh_grads = !FULL || (!F.colors_precomp && F.rest != nullptr);
    float dm[3] = {0.f, 0.f, 0.f};
    if (sh_grads) {
        float s[3 * NC];
        if (FULL)
            load_sh_split<NC>(F.dc + 3 * (size_t)idx, F.rest + (size_t)idx * F.M * 3, s);
        else
            load_sh<NC>(sh + (size_t)idx * K * 3, vec16, s);
        const float dir_orig[3] = {mx - cam.c[0], my - cam.c[1], mz - cam.c[2]};
        const float len = __builtin_sqrtf(dir_orig[0] * dir_orig[0] + dir_orig[1] * dir_orig[1] + dir_orig[2] * dir_orig[2]);
        const float x = dir_orig[0] / len, y = dir_orig[1] / len, z = dir_orig[2] / len;
        float g[3];
#pragma unroll
        for (int ch = 0; ch < 3; ch++) g[ch] = src.clamp(idx, ch) ? 0.0f : gr.rgb(idx, ch);
        float gsh[3 * NC], dx[3], dy[3], dz[3];
        sh_backward<DEG>(x, y, z, s, g, gsh, dx, dy, dz);
        const float dL_ddir[3] = {dx[0] * g[0] + dx[1] * g[1] + dx[2] * g[2],
                                  dy[0] * g[0] + dy[1] * g[1] + dy[2] * g[2],
                                  dz[0] * g[0] + dz[1] * g[1] + dz[2] * g[2]};
        dnormvdv3(dir_orig, dL_ddir, dm);
        // dL/dsh: the first NC coefficients, zeros after
        if (FULL && !STAGED) {
            F.dL_ddc[3 * (size_t)idx + 0] = gsh[0];
            F.dL_ddc[3 * (size_t)idx + 1] = gsh[1];
            F.dL_ddc[3 * (size_t)idx + 2] = gsh[2];
            float* o = F.dL_drest + (size_t)idx * F.M * 3;
#pragma unroll
            for (int i = 0; i < 3 * (NC - 1); i++) o[i] = gsh[3 + i];
            for (int i = 3 * (NC - 1); i < 3 * F.M; i++) o[i] = 0.f;
        } else if (STAGED) {
#pragma unroll
            for (int i = 0; i < 48; i++) s_row[i] = i < 3 * NC ? gsh[i] : 0.f;
        } else if (vec16) {
            float4* o4 = reinterpret_cast<float4*>(gsh_out);
#pragma unroll
            for (int i = 0; i < (3 * NC + 3) / 4; i++) {
                float v[4];
#pragma unroll
                for (int k = 0; k < 4; k++) v[k] = (4 * i + k < 3 * NC) ? gsh[4 * i + k] : 0.f;
                o4[i] = make_float4(v[0], v[1], v[2], v[3]);
            }
            for (int i = (3 * NC + 3) / 4; i < 3 * K / 4; i++) o4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
#pragma unroll
            for (int i = 0; i < 3 * NC; i++) gsh_out[i] = gsh[i];
            for (int i = 3 * NC; i < 3 * K; i++) gsh_out[i] = 0.f;
        }
    }

    float c6[6];
    if (FULL && F.cov3D_precomp != nullptr) {
#pragma unroll
        for (int k = 0; k < 6; k++) c6[k] = F.cov3D_precomp[6 * (size_t)idx + k];
    } else if (cov3D != nullptr) {
        const float2* c2 = reinterpret_cast<const float2*>(cov3D + 6 * (size_t)idx);
        const float2 a = c2[0], b = c2[1], c = c2[2];
        c6[0] = a.x; c6[1] = a.y; c6[2] = b.x; c6[3] = b.y; c6[4] = c.x; c6[5] = c.y;
    } else {
        float sr[3];
        src.scale(idx, sr);
        cov3d_from(sr, src.rot(idx), mod, c6);   // the forward's value, recomputed
    }

    // ---- conic -> 2D covariance -> 3D covariance and mean (cov2D backward)
    Ewa e;
    ewa_setup(V, mx, my, mz, fx, fy, tanfovx, tanfovy, e);
    float Su[3], Sw[3];
    symv(c6, e.u, Su);
    symv(c6, e.w, Sw);
    float a = e.u[0] * Su[0] + e.u[1] * Su[1] + e.u[2] * Su[2];
    const float b = e.u[0] * Sw[0] + e.u[1] * Sw[1] + e.u[2] * Sw[2];
    float c = e.w[0] * Sw[0] + e.w[1] * Sw[1] + e.w[2] * Sw[2];
    a = a + 0.3f;
    c = c + 0.3f;
    const float g0 = gco.x, g1 = gco.y, g2 = gco.z;
    const float denom = a * c - b * b;
    const float denom2inv = 1.0f / ((denom * denom) + 0.0000001f);
    float dL_da = 0, dL_db = 0, dL_dc = 0;
    float dcov[6] = {0, 0, 0, 0, 0, 0};
    if (denom2inv != 0) {
        dL_da = denom2inv * (-c * c * g0 + 2 * b * c * g1 + (denom - a * c) * g2);
        dL_dc = denom2inv * (-a * a * g2 + 2 * a * b * g1 + (denom - a * c) * g0);
        dL_db = denom2inv * 2 * (b * c * g0 - (denom + 2 * b * b) * g1 + a * b * g2);
        const float* u = e.u;
        const float* w = e.w;
        dcov[0] = u[0] * u[0] * dL_da + u[0] * w[0] * dL_db + w[0] * w[0] * dL_dc;
        dcov[3] = u[1] * u[1] * dL_da + u[1] * w[1] * dL_db + w[1] * w[1] * dL_dc;
        dcov[5] = u[2] * u[2] * dL_da + u[2] * w[2] * dL_db + w[2] * w[2] * dL_dc;
        dcov[1] = 2 * u[0] * u[1] * dL_da + (u[0] * w[1] + u[1] * w[0]) * dL_db + 2 * w[0] * w[1] * dL_dc;
        dcov[2] = 2 * u[0] * u[2] * dL_da + (u[0] * w[2] + u[2] * w[0]) * dL_db + 2 * w[0] * w[2] * dL_dc;
        dcov[4] = 2 * u[2] * u[1] * dL_da + (u[1] * w[2] + u[2] * w[1]) * dL_db + 2 * w[1] * w[2] * dL_dc;
    }
    if (FULL) {
        float2* o2 = reinterpret_cast<float2*>(F.dL_dcov3D + 6 * (size_t)idx);
        o2[0] = make_float2(dcov[0], dcov[1]);
        o2[1] = make_float2(dcov[2], dcov[3]);
        o2[2] = make_float2(dcov[4], dcov[5]);
    }
    float du[3], dw[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        du[k] = 2 * Su[k] * dL_da + Sw[k] * dL_db;
        dw[k] = 2 * Sw[k] * dL_dc + Su[k] * dL_db;
    }
    const float dJ00 = V[0] * du[0] + V[4] * du[1] + V[8] * du[2];
    const float dJ20 = V[2] * du[0] + V[6] * du[1] + V[10] * du[2];
    const float dJ11 = V[1] * dw[0] + V[5] * dw[1] + V[9] * dw[2];
    const float dJ21 = V[2] * dw[0] + V[6] * dw[1] + V[10] * dw[2];
    const float tz = 1.f / e.t2;
    const float tz2 = tz * tz;
    const float tz3 = tz2 * tz;
    const float dtx = e.xmask * -fx * tz2 * dJ20;
    const float dty = e.ymask * -fy * tz2 * dJ21;
    const float dtz = -fx * tz2 * dJ00 - fy * tz2 * dJ11 + (2 * fx * e.t0) * tz3 * dJ20 + (2 * fy * e.t1) * tz3 * dJ21;
    float gm[3];
    gm[0] = V[0] * dtx + V[1] * dty + V[2] * dtz;
    gm[1] = V[4] * dtx + V[5] * dty + V[6] * dtz;
    gm[2] = V[8] * dtx + V[9] * dty + V[10] * dtz;

    // ---- screen-space mean -> 3D mean
    {
        const float m_w = 1.0f / (xform_w(PM, mx, my, mz) + 0.0000001f);
        const float mul1 = (PM[0] * mx + PM[4] * my + PM[8] * mz + PM[12]) * m_w * m_w;
        const float mul2 = (PM[1] * mx + PM[5] * my + PM[9] * mz + PM[13]) * m_w * m_w;
        const float gx = gr.mean2d(idx, 0);
        const float gy = gr.mean2d(idx, 1);
        gm[0] += (PM[0] * m_w - PM[3] * mul1) * gx + (PM[1] * m_w - PM[3] * mul2) * gy;
        gm[1] += (PM[4] * m_w - PM[7] * mul1) * gx + (PM[5] * m_w - PM[7] * mul2) * gy;
        gm[2] += (PM[8] * m_w - PM[11] * mul1) * gx + (PM[9] * m_w - PM[11] * mul2) * gy;
    }

    if (sh_grads) {
        gm[0] += dm[0];
        gm[1] += dm[1];
        gm[2] += dm[2];
    }
    m3_row[0] = gm[0];
    m3_row[1] = gm[1];
    m3_row[2] = gm[2];

    // ---- 3D covariance -> scale and (un-normalised) quaternion
    if (FULL && F.cov3D_precomp != nullptr) {
        sc_row[0] = 0.f;
        sc_row[1] = 0.f;
        sc_row[2] = 0.f;
        *rot_row = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
        const float4 q = src.rot(idx);
        const float r = q.x, x = q.y, y = q.z, z = q.w;
        float Rm[3][3];
        quat_rows(r, x, y, z, Rm);
        float sr[3];
        src.scale(idx, sr);
        const float s[3] = {mod * sr[0], mod * sr[1], mod * sr[2]};
        float M[3][3];
#pragma unroll
        for (int i = 0; i < 3; i++)
#pragma unroll
            for (int j = 0; j < 3; j++) M[i][j] = s[i] * Rm[i][j];
        const float D[3][3] = {{dcov[0], 0.5f * dcov[1], 0.5f * dcov[2]},
                               {0.5f * dcov[1], dcov[3], 0.5f * dcov[4]},
                               {0.5f * dcov[2], 0.5f * dcov[4], dcov[5]}};
        float G[3][3];
#pragma unroll
        for (int i = 0; i < 3; i++)
#pragma unroll
            for (int j = 0; j < 3; j++)
                G[i][j] = (2.0f * M[i][0]) * D[0][j] + (2.0f * M[i][1]) * D[1][j] + (2.0f * M[i][2]) * D[2][j];
#pragma unroll
        for (int i = 0; i < 3; i++)
            sc_row[i] = Rm[i][0] * G[i][0] + Rm[i][1] * G[i][1] + Rm[i][2] * G[i][2];
#pragma unroll
        for (int i = 0; i < 3; i++)
#pragma unroll
            for (int j = 0; j < 3; j++) G[i][j] = G[i][j] * s[i];
        const float q0 = 2 * z * (G[0][1] - G[1][0]) + 2 * y * (G[2][0] - G[0][2]) + 2 * x * (G[1][2] - G[2][1]);
        const float q1 = 2 * y * (G[1][0] + G[0][1]) + 2 * z * (G[2][0] + G[0][2]) + 2 * r * (G[1][2] - G[2][1]) - 4 * x * (G[2][2] + G[1][1]);
        const float q2 = 2 * x * (G[1][0] + G[0][1]) + 2 * r * (G[2][0] - G[0][2]) + 2 * z * (G[1][2] + G[2][1]) - 4 * y * (G[2][2] + G[0][0]);
        const float q3 = 2 * r * (G[0][1] - G[1][0]) + 2 * x * (G[2][0] + G[0][2]) + 2 * y * (G[1][2] + G[2][1]) - 4 * z * (G[1][1] + G[0][0]);
        *rot_row = make_float4(q0, q1, q2, q3);
    }
}

// Rows of dL/dsh are staged in LDS (pitch 49 floats: conflict-free column
// writes) and copied out with fully coalesced streaming stores: as (P,16,3)
// rows of 16 bytes in the split path (K == 16), as the (P,1,3) DC and (P,M,3)
// rest arrays in the full path (M <= 15).  (Streaming stores pay off only for
// such whole-line writes: the 12-byte per-Gaussian rows are stored normally.)
constexpr int SH_PITCH = 49;

// REC: the visible Gaussians' inputs come from the forward's records (BwdRec;
// lane l of a wave takes the wave's l-th record) and visibility from their
// masks; radii, means3D, scales, rotations and clamped are not read.
template <int DEG, bool STAGED, bool FULL, bool REC = false>
__global__ __launch_bounds__(256) void preprocess_bwd_kernel(
    int P, int K, int W, int H, float tanfovx, float tanfovy, float fx, float fy, float mod,
    const float* __restrict__ view, const float* __restrict__ proj, const float* __restrict__ campos,
    const float* __restrict__ means3D, const float* __restrict__ scales, const float* __restrict__ rotations,
    const float* __restrict__ sh, int sh_vec16, const int* __restrict__ radii, const float* __restrict__ cov3D,
    const uint8_t* __restrict__ clamped, const float* __restrict__ dL_dmeans2D, int m2d_stride,
    const float* __restrict__ dL_dconic_opacity, const float* __restrict__ dL_drgb,
    float* __restrict__ dL_dmeans3D, float* __restrict__ dL_dscales, float* __restrict__ dL_drotations,
    float* __restrict__ dL_dsh, float* __restrict__ dL_dopacity, FullPreBwd F, const float4* __restrict__ rec,
    const uint64_t* __restrict__ rec_mask, int zeroed)
{
    __shared__ float s_sh[STAGED ? 256 * SH_PITCH : 1];
    __shared__ uint8_t s_vis[256];
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int lane = threadIdx.x & 63, wbase = idx & ~63;
    const bool in = idx < P;
    uint64_t vmask = 0;
    if (REC && wbase < P) vmask = rec_mask[wbase >> 6];
    const bool vis = REC ? ((vmask >> lane) & 1ull) != 0 : (in && radii[idx] > 0);
    // this Gaussian's dL/dmeans3D and dL/dscales rows
    float* m3_row = dL_dmeans3D + 3 * (size_t)idx;
    float* sc_row = dL_dscales + 3 * (size_t)idx;
    // staged rows hold SH gradients (the full path has none with precomputed
    // colours or without a rest array)
    const bool sh_rows = !FULL || (!F.colors_precomp && F.rest != nullptr);
    if (STAGED) s_vis[threadIdx.x] = (vis && sh_rows) ? 1 : 0;
    if (in && !vis) {
        if (!REC) {   // (REC: written with the visible rows below)
            dL_dopacity[idx] = reinterpret_cast<const float4*>(dL_dconic_opacity)[idx].w;
            m3_row[0] = 0.f;
            m3_row[1] = 0.f;
            m3_row[2] = 0.f;
            sc_row[0] = 0.f;
            sc_row[1] = 0.f;
            sc_row[2] = 0.f;
            reinterpret_cast<float4*>(dL_drotations)[idx] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (FULL) {
            for (int k = 0; k < 6; k++) F.dL_dcov3D[6 * (size_t)idx + k] = 0.f;
        } else if (!STAGED && !zeroed) {
            float* gsh_out = dL_dsh + (size_t)idx * K * 3;
            if (sh_vec16) {
                float4* o4 = reinterpret_cast<float4*>(gsh_out);
                for (int i = 0; i < 3 * K / 4; i++) o4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                for (int i = 0; i < 3 * K; i++) gsh_out[i] = 0.f;
            }
        }
    }
    if (FULL && !STAGED && in) {
        // SH gradients are zero unless written below (culled, precomputed colours, no rest array)
        F.dL_ddc[3 * (size_t)idx + 0] = 0.f;
        F.dL_ddc[3 * (size_t)idx + 1] = 0.f;
        F.dL_ddc[3 * (size_t)idx + 2] = 0.f;
        float* o = F.dL_drest + (size_t)idx * F.M * 3;
        for (int i = 0; i < 3 * F.M; i++) o[i] = 0.f;
    }
    if (REC) {
        // lane l computes the wave's l-th visible Gaussian; its dL/dmeans3D,
        // dL/dscales and dL/drotations come back to that Gaussian's own lane
        // (ds_bpermute), which writes them with the zero rows of the invisible
        // ones: every row of the wave's run leaves in the same few store
        // instructions, so no cache line is written back half-filled
        float m3[3] = {0.f, 0.f, 0.f}, sc[3] = {0.f, 0.f, 0.f}, op = 0.f;
        float4 rot = make_float4(0.f, 0.f, 0.f, 0.f);
        if (lane < __popcll(vmask)) {
            const float4* r = rec + 3 * (size_t)(wbase + lane);
            const RecSrc src{r[0], r[1], r[2]};
            const int id = __float_as_int(src.r1.w);
            // a record names a Gaussian of its own wave (a buffer from another
            // call could name any index: such records are skipped)
            if ((unsigned)(id - wbase) < 64u && id < P)
                preprocess_bwd_one<DEG, STAGED, FULL>(id, K, tanfovx, tanfovy, fx, fy, mod, view, proj, campos, src,
                                                      sh, sh_vec16, cov3D,
                                                      DenseGrads{dL_dmeans2D, m2d_stride, dL_dconic_opacity, dL_drgb},
                                                      m3, sc, &rot, dL_dsh, &op,
                                                      s_sh + (id - (int)blockIdx.x * 256) * SH_PITCH, F);
        }
        const int from = 4 * __popcll(vmask & ((1ull << lane) - 1ull));   // this row's computing lane, x4
        const auto take = [&](float v) {
            const float x = __int_as_float(__builtin_amdgcn_ds_bpermute(from, __float_as_int(v)));
            return vis ? x : 0.f;
        };
        const float o_m0 = take(m3[0]), o_m1 = take(m3[1]), o_m2 = take(m3[2]);
        const float o_s0 = take(sc[0]), o_s1 = take(sc[1]), o_s2 = take(sc[2]);
        const float4 o_r = make_float4(take(rot.x), take(rot.y), take(rot.z), take(rot.w));
        if (in) {
            // dL/dopacity is dL/dconic_opacity.w for every Gaussian
            dL_dopacity[idx] = reinterpret_cast<const float4*>(dL_dconic_opacity)[idx].w;
            m3_row[0] = o_m0;
            m3_row[1] = o_m1;
            m3_row[2] = o_m2;
            sc_row[0] = o_s0;
            sc_row[1] = o_s1;
            sc_row[2] = o_s2;
            reinterpret_cast<float4*>(dL_drotations)[idx] = o_r;
        }
    } else if (vis) {
        preprocess_bwd_one<DEG, STAGED, FULL>(idx, K, tanfovx, tanfovy, fx, fy, mod, view, proj, campos,
                                              ArraySrc{means3D, scales, rotations, clamped}, sh, sh_vec16, cov3D,
                                              DenseGrads{dL_dmeans2D, m2d_stride, dL_dconic_opacity, dL_drgb},
                                              m3_row, sc_row,
                                              reinterpret_cast<float4*>(dL_drotations) + idx, dL_dsh,
                                              dL_dopacity + idx, s_sh + threadIdx.x * SH_PITCH, F);
    }
    if (STAGED && FULL) {
        // coalesced copy-out of this block's rows [blockIdx*256, +nrows): 3 DC floats, then 3M rest floats
        __syncthreads();
        const int row0 = blockIdx.x * 256;
        const int nrows = min(256, P - row0);
        float* ddc = F.dL_ddc + (size_t)row0 * 3;
        for (int c = threadIdx.x; c < nrows * 3; c += 256) {
            const int r = c / 3;
            gs::st_stream(&ddc[c], s_vis[r] ? s_sh[r * SH_PITCH + (c - 3 * r)] : 0.f);
        }
        const int rw = 3 * F.M;
        float* drest = F.dL_drest + (size_t)row0 * rw;
        for (int c = threadIdx.x; c < nrows * rw; c += 256) {
            const int r = c / rw;
            gs::st_stream(&drest[c], s_vis[r] ? s_sh[r * SH_PITCH + 3 + (c - rw * r)] : 0.f);
        }
    } else if (STAGED) {
        // coalesced copy-out of this block's rows [blockIdx*256, +nrows) x 48 floats
        __syncthreads();
        const int row0 = blockIdx.x * 256;
        const int nrows = min(256, P - row0);
        float4* dst = reinterpret_cast<float4*>(dL_dsh + (size_t)row0 * 48);
        for (int c = threadIdx.x; c < nrows * 12; c += 256) {
            const int r = c / 12, col = (c - r * 12) * 4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (s_vis[r]) {
                const float* src = s_sh + r * SH_PITCH + col;
                v = make_float4(src[0], src[1], src[2], src[3]);
            } else if (zeroed) {
                continue;   // (the row already holds zeros)
            }
            gs::st_stream(&dst[c], v);
        }
    }
}

// The record path when dL/dsh arrives cleared (outputs_zeroed) and its rows
// are 16-byte vectors: a one-wave block takes PACK_RUNS consecutive
// 64-Gaussian runs and packs their visible Gaussians onto its lanes (item i
// of the runs' concatenated records on lane i mod 64, round i / 64), so the
// per-Gaussian arithmetic runs on nearly full waves instead of on the one
// lane in five that a run's visible Gaussians occupy at the benchmark's
// scene.  A round's dL/dsh rows are staged in LDS (pitch SH_PITCH) and leave
// as streaming 16-byte stores, twelve lanes to a 192-byte row (whole 64-byte
// segments); the Gaussians' dL/dmeans3D, dL/dscales and dL/drotations go to
// LDS slots at their rows, from which each run's 64 rows (zeros for the
// invisible ones) leave in the same coalesced stores as in
// preprocess_bwd_kernel.  Bit-identical to preprocess_bwd_kernel's record
// path: the same preprocess_bwd_one per Gaussian.  Two runs per block: with
// four (expected 49 items per round at one Gaussian in five visible) the
// larger LDS slots leave fewer blocks per CU and scenes where half the
// Gaussians are visible take two rounds per block; two is as fast at the
// first and keeps the second at the unpacked kernel's speed.
constexpr int PACK_RUNS = 2;

// The render backward's per-Gaussian accumulators (the listed Gaussians'
// 64-byte rows, cidx_of: a Gaussian's row or -1; cidx_of null: no row) and
// the factors its unpack applies (dmean/dpixel sx = W/2, sy = H/2; -1/2 on
// the conic terms): the incoming gradients of the preprocess backward when
// they are exactly that render backward's outputs.
struct AccIn {
    const float4* __restrict__ gacc;
    const int* __restrict__ cidx_of;
    float sx, sy;
    // unpack_grads_kernel's expressions, so the values are those it wrote
    __device__ HeldGrads of(int id) const
    {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a, c = a;
        const int cx = cidx_of != nullptr ? cidx_of[id] : -1;
        if (cx >= 0) {
            const float4* g = gacc + 4 * (size_t)cx;
            a = g[0];
            b = g[1];
            c = g[2];
            a = make_float4(a.x * sx, a.y * sy, a.z * sx, a.w * sy);
            b = make_float4(-0.5f * b.x, -0.5f * b.y, -0.5f * b.z, b.w);
        }
        return HeldGrads{b, {a.x, a.y}, {c.x, c.y, c.z}};
    }
};

// ACC: the incoming gradients from the render backward's accumulators (acc)
// instead of the dense arrays; an invisible Gaussian's dL/dopacity is then
// zero (the render listed it nowhere), so dL/dconic_opacity is not read.
template <int DEG, bool ACC>
__global__ __launch_bounds__(64) void preprocess_bwd_packed_kernel(
    int P, int K, float tanfovx, float tanfovy, float fx, float fy, float mod, const float* __restrict__ view,
    const float* __restrict__ proj, const float* __restrict__ campos, const float* __restrict__ sh,
    const float* __restrict__ cov3D, const float* __restrict__ dL_dmeans2D, int m2d_stride,
    const float* __restrict__ dL_dconic_opacity, const float* __restrict__ dL_drgb, AccIn acc,
    float* __restrict__ dL_dmeans3D, float* __restrict__ dL_dscales, float* __restrict__ dL_drotations,
    float* __restrict__ dL_dsh, float* __restrict__ dL_dopacity, const float4* __restrict__ rec,
    const uint64_t* __restrict__ rec_mask)
{
    constexpr int NC = (DEG + 1) * (DEG + 1);
    constexpr int CH = (3 * NC + 3) / 4;             // 16-byte chunks of a row that can be nonzero
    __shared__ float s_sh[64 * SH_PITCH];            // one round's dL/dsh rows
    __shared__ int s_id[64];                         // their Gaussians (-1: none)
    __shared__ float4 s_rot[PACK_RUNS * 64];         // per row of the runs: dL/drotations,
    __shared__ float s_ms[PACK_RUNS * 64 * 6];       // dL/dmeans3D and dL/dscales
    __shared__ float s_op[ACC ? PACK_RUNS * 64 : 1]; // (ACC) and dL/dopacity
    const int lane = threadIdx.x;
    const int run0 = (int)blockIdx.x * PACK_RUNS;    // first 64-run of this block
    const int nruns = (P + 63) >> 6;
    uint64_t m[PACK_RUNS];
    int pre[PACK_RUNS + 1];
    pre[0] = 0;
#pragma unroll
    for (int j = 0; j < PACK_RUNS; j++) {
        m[j] = run0 + j < nruns ? rec_mask[run0 + j] : 0ull;
        pre[j + 1] = pre[j] + __popcll(m[j]);
    }
    const int n = pre[PACK_RUNS];
    const size_t row_floats = 3 * (size_t)K;
    for (int i = lane; i < ((n + 63) & ~63); i += 64) {
        int id = -1;
        if (i < n) {
            int j = 0, pj = 0;   // the run of item i and the items before it (selects, no indexed registers)
#pragma unroll
            for (int t = 1; t < PACK_RUNS; t++) {
                const bool past = i >= pre[t];
                j = past ? t : j;
                pj = past ? pre[t] : pj;
            }
            const int wbase = (run0 + j) * 64;
            const float4* r = rec + 3 * (size_t)(wbase + i - pj);
            const RecSrc src{r[0], r[1], r[2]};
            const int g = __float_as_int(src.r1.w);
            // a record names a Gaussian of its own run (a buffer from another
            // call could name any index: such records are skipped)
            if ((unsigned)(g - wbase) < 64u && g < P) {
                id = g;
                const int row = j * 64 + (g - wbase);
                float* ms = s_ms + row * 6;
                float op;
                if constexpr (ACC) {
                    preprocess_bwd_one<DEG, true, false>(g, K, tanfovx, tanfovy, fx, fy, mod, view, proj, campos,
                                                         src, sh, 1, cov3D, acc.of(g), ms, ms + 3, &s_rot[row],
                                                         dL_dsh, &op, s_sh + lane * SH_PITCH, FullPreBwd{});
                    s_op[row] = op;
                } else {
                    preprocess_bwd_one<DEG, true, false>(
                        g, K, tanfovx, tanfovy, fx, fy, mod, view, proj, campos, src, sh, 1, cov3D,
                        DenseGrads{dL_dmeans2D, m2d_stride, dL_dconic_opacity, dL_drgb}, ms, ms + 3, &s_rot[row],
                        dL_dsh, &op, s_sh + lane * SH_PITCH, FullPreBwd{});
                }
            }
        }
        s_id[lane] = id;
        __syncthreads();
        // the round's rows: lane c takes chunk c % CH of row c / CH
        for (int c = lane; c < 64 * CH; c += 64) {
            const int r = c / CH, col = (c - r * CH) * 4;
            const int g = s_id[r];
            if (g < 0) continue;
            const float* src = s_sh + r * SH_PITCH + col;
            gs::st_stream(reinterpret_cast<float4*>(dL_dsh + (size_t)g * row_floats + col),
                          make_float4(src[0], src[1], src[2], src[3]));
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < PACK_RUNS; j++) {
        const int idx = (run0 + j) * 64 + lane;
        if (idx >= P) break;
        const bool vis = ((m[j] >> lane) & 1ull) != 0;
        float a[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float4 c = make_float4(0.f, 0.f, 0.f, 0.f);
        if (vis) {
            const float* ms = s_ms + (j * 64 + lane) * 6;
#pragma unroll
            for (int k = 0; k < 6; k++) a[k] = ms[k];
            c = s_rot[j * 64 + lane];
        }
        if constexpr (ACC)
            dL_dopacity[idx] = vis ? s_op[j * 64 + lane] : 0.f;
        else
            dL_dopacity[idx] = reinterpret_cast<const float4*>(dL_dconic_opacity)[idx].w;
        float* m3 = dL_dmeans3D + 3 * (size_t)idx;
        float* sc = dL_dscales + 3 * (size_t)idx;
        m3[0] = a[0];
        m3[1] = a[1];
        m3[2] = a[2];
        sc[0] = a[3];
        sc[1] = a[4];
        sc[2] = a[5];
        reinterpret_cast<float4*>(dL_drotations)[idx] = c;
    }
}

}  // namespace

static int preprocess_forward_impl(
    int P, int D, int K, const float* means3D, const float* scales, const float* rotations,
    const float* sh, const float* opacities, float scale_modifier, const float* viewmatrix,
    const float* projmatrix, const float* campos, float tanfovx, float tanfovy, int image_height,
    int image_width, float* means2D, float* depths, int* radii, float* cov3D, float* conic_opacity,
    float* rgb, uint8_t* clamped, void* bwd_records, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0, "P must be >= 0 (got %d)", P);
    if (P == 0) return GS_OK;
    GS_REQUIRE(D >= 0 && D <= 3, "sh_degree must be in [0, 3] (got %d)", D);
    GS_REQUIRE(K >= (D + 1) * (D + 1), "sh must have at least (D+1)^2 = %d coefficients (got %d)",
               (D + 1) * (D + 1), K);
    GS_REQUIRE(image_width > 0 && image_height > 0, "image size must be positive");
    GS_REQUIRE(((uintptr_t)rotations & 15) == 0 && ((uintptr_t)conic_opacity & 15) == 0,
               "rotations and conic_opacity must be 16-byte aligned");
    GS_REQUIRE(((uintptr_t)bwd_records & 255) == 0, "bwd_records must be 256-byte aligned");
    const int sh_vec16 = ((K & 3) == 0 && ((uintptr_t)sh & 15) == 0) ? 1 : 0;
    BwdRec rec{};
    if (bwd_records != nullptr) {
        rec.mask = static_cast<uint64_t*>(bwd_records);
        rec.rec = reinterpret_cast<float4*>(static_cast<char*>(bwd_records) + bwdrec_mask_bytes(P));
    }
    const float fy = (float)image_height / (2.0f * tanfovy);
    const float fx = (float)image_width / (2.0f * tanfovx);
    const dim3 grid(gs_div_up((size_t)P, 256)), block(256);
#define GS_PRE_FWD(DEG)                                                                             \
    GS_TIMED("preprocess_fwd_kernel", stream, hipLaunchKernelGGL((preprocess_fwd_kernel<DEG, false>), grid, block, 0, stream, P, K, image_width,        \
                       image_height, tanfovx, tanfovy, fx, fy, scale_modifier, viewmatrix, projmatrix, \
                       campos, means3D, scales, rotations, sh, sh_vec16, opacities, means2D, depths, radii, \
                       cov3D, conic_opacity, rgb, clamped, FullPre{}, rec))
    switch (D) {
        case 0: GS_PRE_FWD(0); break;
        case 1: GS_PRE_FWD(1); break;
        case 2: GS_PRE_FWD(2); break;
        default: GS_PRE_FWD(3); break;
    }
#undef GS_PRE_FWD
    GS_LAUNCH_CHECK("preprocess_fwd_kernel");
    return GS_OK;
}

extern "C" int gs_preprocess_forward(
    int P, int D, int K, const float* means3D, const float* scales, const float* rotations,
    const float* sh, const float* opacities, float scale_modifier, const float* viewmatrix,
    const float* projmatrix, const float* campos, float tanfovx, float tanfovy, int image_height,
    int image_width, float* means2D, float* depths, int* radii, float* cov3D, float* conic_opacity,
    float* rgb, uint8_t* clamped, hipStream_t stream)
{
    return preprocess_forward_impl(P, D, K, means3D, scales, rotations, sh, opacities, scale_modifier, viewmatrix,
                                   projmatrix, campos, tanfovx, tanfovy, image_height, image_width, means2D, depths,
                                   radii, cov3D, conic_opacity, rgb, clamped, nullptr, stream);
}

extern "C" int64_t gs_preprocess_record_bytes(int P) { return P <= 0 ? 0 : (int64_t)bwdrec_bytes(P); }

extern "C" int gs_preprocess_forward_rec(
    int P, int D, int K, const float* means3D, const float* scales, const float* rotations,
    const float* sh, const float* opacities, float scale_modifier, const float* viewmatrix,
    const float* projmatrix, const float* campos, float tanfovx, float tanfovy, int image_height,
    int image_width, float* means2D, float* depths, int* radii, float* cov3D, float* conic_opacity,
    float* rgb, uint8_t* clamped, void* bwd_records, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P <= 0 || bwd_records != nullptr, "bwd_records must hold gs_preprocess_record_bytes(P) bytes");
    GS_REQUIRE(P <= 0 || (means2D && depths && radii && conic_opacity && rgb), "null output");
    return preprocess_forward_impl(P, D, K, means3D, scales, rotations, sh, opacities, scale_modifier, viewmatrix,
                                   projmatrix, campos, tanfovx, tanfovy, image_height, image_width, means2D, depths,
                                   radii, cov3D, conic_opacity, rgb, clamped, bwd_records, stream);
}

static int preprocess_backward_impl(
    int P, int D, int K, const float* means3D, const float* scales, const float* rotations,
    const float* sh, float scale_modifier, const float* viewmatrix, const float* projmatrix,
    const float* campos, float tanfovx, float tanfovy, int image_height, int image_width,
    const int* radii, const float* cov3D, const uint8_t* clamped, const float* dL_dmeans2D,
    int dL_dmeans2D_stride, const float* dL_dconic_opacity, const float* dL_drgb, float* dL_dmeans3D,
    float* dL_dscales, float* dL_drotations, float* dL_dsh, float* dL_dopacity, const void* bwd_records,
    hipStream_t stream, int zeroed = 0, const AccIn* acc = nullptr)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0, "P must be >= 0 (got %d)", P);
    if (P == 0) return GS_OK;
    GS_REQUIRE(D >= 0 && D <= 3, "sh_degree must be in [0, 3] (got %d)", D);
    GS_REQUIRE(K >= (D + 1) * (D + 1), "sh must have at least (D+1)^2 = %d coefficients (got %d)",
               (D + 1) * (D + 1), K);
    GS_REQUIRE(dL_dmeans2D_stride >= 2, "dL_dmeans2D row stride must be >= 2");
    GS_REQUIRE(((uintptr_t)rotations & 15) == 0 && ((uintptr_t)dL_dconic_opacity & 15) == 0 &&
               ((uintptr_t)dL_drotations & 15) == 0,
               "rotations, dL_dconic_opacity and dL_drotations must be 16-byte aligned");
    const int sh_vec16 = ((K & 3) == 0 && ((uintptr_t)sh & 15) == 0 && ((uintptr_t)dL_dsh & 15) == 0) ? 1 : 0;
    const bool staged = K == 16 && ((uintptr_t)dL_dsh & 15) == 0;
    GS_REQUIRE(((uintptr_t)bwd_records & 255) == 0, "bwd_records must be 256-byte aligned");
    const uint64_t* rmask = static_cast<const uint64_t*>(bwd_records);
    const float4* rrec = bwd_records == nullptr ? nullptr
        : reinterpret_cast<const float4*>(static_cast<const char*>(bwd_records) + bwdrec_mask_bytes(P));
    const float fy = (float)image_height / (2.0f * tanfovy);
    const float fx = (float)image_width / (2.0f * tanfovx);
    const dim3 grid(gs_div_up((size_t)P, 256)), block(256);
    GS_REQUIRE(acc == nullptr || (rrec != nullptr && zeroed && sh_vec16),
               "the accumulator inputs need the records, cleared dL_dsh and 16-byte SH rows");
    if (rrec != nullptr && zeroed && sh_vec16) {
        const dim3 pgrid(gs_div_up((size_t)P, 64 * PACK_RUNS)), pblock(64);
        const AccIn ai = acc != nullptr ? *acc : AccIn{};
#define GS_PRE_BWD_P(DEG, ACC)                                                                               \
    GS_TIMED("preprocess_bwd_packed_kernel", stream,                                                         \
             hipLaunchKernelGGL((preprocess_bwd_packed_kernel<DEG, ACC>), pgrid, pblock, 0, stream, P, K,     \
                                tanfovx, tanfovy, fx, fy, scale_modifier, viewmatrix, projmatrix, campos, sh, \
                                cov3D, dL_dmeans2D, dL_dmeans2D_stride, dL_dconic_opacity, dL_drgb, ai,       \
                                dL_dmeans3D, dL_dscales, dL_drotations, dL_dsh, dL_dopacity, rrec, rmask))
#define GS_PRE_BWD_PA(DEG) \
    if (acc != nullptr) GS_PRE_BWD_P(DEG, true); else GS_PRE_BWD_P(DEG, false);
        switch (D) {
            case 0: GS_PRE_BWD_PA(0); break;
            case 1: GS_PRE_BWD_PA(1); break;
            case 2: GS_PRE_BWD_PA(2); break;
            default: GS_PRE_BWD_PA(3); break;
        }
#undef GS_PRE_BWD_PA
#undef GS_PRE_BWD_P
        GS_LAUNCH_CHECK("preprocess_bwd_packed_kernel");
        return GS_OK;
    }
#define GS_PRE_BWD_K(DEG, ST, RC)                                                                      \
    GS_TIMED("preprocess_bwd_kernel", stream,                                                            \
             hipLaunchKernelGGL((preprocess_bwd_kernel<DEG, ST, false, RC>), grid, block, 0, stream, P, K,   \
                                image_width, image_height, tanfovx, tanfovy, fx, fy, scale_modifier,      \
                                viewmatrix, projmatrix, campos, means3D, scales, rotations, sh, sh_vec16, \
                                radii, cov3D, clamped, dL_dmeans2D, dL_dmeans2D_stride,                   \
                                dL_dconic_opacity, dL_drgb, dL_dmeans3D, dL_dscales, dL_drotations,       \
                                dL_dsh, dL_dopacity, FullPreBwd{}, rrec, rmask, zeroed))
#define GS_PRE_BWD(DEG)                                                                                  \
    if (rrec != nullptr) {                                                                               \
        if (staged) GS_PRE_BWD_K(DEG, true, true); else GS_PRE_BWD_K(DEG, false, true);                  \
    } else {                                                                                             \
        if (staged) GS_PRE_BWD_K(DEG, true, false); else GS_PRE_BWD_K(DEG, false, false);                \
    }
    switch (D) {
        case 0: GS_PRE_BWD(0); break;
        case 1: GS_PRE_BWD(1); break;
        case 2: GS_PRE_BWD(2); break;
        default: GS_PRE_BWD(3); break;
    }
#undef GS_PRE_BWD
#undef GS_PRE_BWD_K
    GS_LAUNCH_CHECK("preprocess_bwd_kernel");
    return GS_OK;
}

extern "C" int gs_preprocess_backward(
    int P, int D, int K, const float* means3D, const float* scales, const float* rotations,
    const float* sh, float scale_modifier, const float* viewmatrix, const float* projmatrix,
    const float* campos, float tanfovx, float tanfovy, int image_height, int image_width,
    const int* radii, const float* cov3D, const uint8_t* clamped, const float* dL_dmeans2D,
    int dL_dmeans2D_stride, const float* dL_dconic_opacity, const float* dL_drgb, float* dL_dmeans3D,
    float* dL_dscales, float* dL_drotations, float* dL_dsh, float* dL_dopacity, hipStream_t stream)
{
    return preprocess_backward_impl(P, D, K, means3D, scales, rotations, sh, scale_modifier, viewmatrix, projmatrix,
                                    campos, tanfovx, tanfovy, image_height, image_width, radii, cov3D, clamped,
                                    dL_dmeans2D, dL_dmeans2D_stride, dL_dconic_opacity, dL_drgb, dL_dmeans3D,
                                    dL_dscales, dL_drotations, dL_dsh, dL_dopacity, nullptr, stream);
}

extern "C" int gs_preprocess_backward_rec(
    int P, int D, int K, const void* bwd_records, const float* sh, float scale_modifier,
    const float* viewmatrix, const float* projmatrix, const float* campos, float tanfovx, float tanfovy,
    int image_height, int image_width, const float* cov3D, const float* dL_dmeans2D, int dL_dmeans2D_stride,
    const float* dL_dconic_opacity, const float* dL_drgb, float* dL_dmeans3D, float* dL_dscales,
    float* dL_drotations, float* dL_dsh, float* dL_dopacity, int outputs_zeroed, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P <= 0 || bwd_records != nullptr, "bwd_records must be the records gs_preprocess_forward_rec wrote");
    return preprocess_backward_impl(P, D, K, nullptr, nullptr, nullptr, sh, scale_modifier, viewmatrix, projmatrix,
                                    campos, tanfovx, tanfovy, image_height, image_width, nullptr, cov3D, nullptr,
                                    dL_dmeans2D, dL_dmeans2D_stride, dL_dconic_opacity, dL_drgb, dL_dmeans3D,
                                    dL_dscales, dL_drotations, dL_dsh, dL_dopacity, bwd_records, stream,
                                    outputs_zeroed != 0 ? 1 : 0);
}

extern "C" int gs_preprocess_backward_rec_acc(
    int P, int D, int K, const void* bwd_records, const float* sh, float scale_modifier,
    const float* viewmatrix, const float* projmatrix, const float* campos, float tanfovx, float tanfovy,
    int image_height, int image_width, const float* cov3D, const void* render_acc, const int* render_cidx_of,
    float* dL_dmeans3D, float* dL_dscales, float* dL_drotations, float* dL_dsh, float* dL_dopacity,
    hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P <= 0 || bwd_records != nullptr, "bwd_records must be the records gs_preprocess_forward_rec wrote");
    GS_REQUIRE(P <= 0 || (render_acc != nullptr && ((uintptr_t)render_acc & 15) == 0),
               "render_acc must be the render's accumulators (gs_render_accumulators)");
    const AccIn acc{static_cast<const float4*>(render_acc), render_cidx_of, 0.5f * (float)image_width,
                    0.5f * (float)image_height};
    return preprocess_backward_impl(P, D, K, nullptr, nullptr, nullptr, sh, scale_modifier, viewmatrix, projmatrix,
                                    campos, tanfovx, tanfovy, image_height, image_width, nullptr, cov3D, nullptr,
                                    nullptr, 2, nullptr, nullptr, dL_dmeans3D, dL_dscales, dL_drotations, dL_dsh,
                                    dL_dopacity, bwd_records, stream, 1, &acc);
}

extern "C" int gs_preprocess_forward_full(
    int P, int D, int M, const float* means3D, const float* scales, const float* rotations, const float* dc,
    const float* rest, const float* opacities, const float* colors_precomp, const float* cov3D_precomp,
    const uint8_t* culling, float scale_modifier, const float* viewmatrix, const float* projmatrix,
    const float* campos, float tanfovx, float tanfovy, int image_height, int image_width, float* means2D,
    float* depths, int* radii, float* cov3D, float* conic_opacity, float* rgb, uint8_t* clamped, float* rects,
    uint32_t* tiles_touched, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0, "P must be >= 0 (got %d)", P);
    if (P == 0) return GS_OK;
    GS_REQUIRE(D >= 0 && D <= 3, "sh_degree must be in [0, 3] (got %d)", D);
    GS_REQUIRE(M >= 0, "M must be >= 0");
    GS_REQUIRE(colors_precomp != nullptr || (dc != nullptr && (D == 0 || (rest != nullptr && M >= (D + 1) * (D + 1) - 1))),
               "SH colours need dc and at least (D+1)^2 - 1 = %d further coefficients (got %d)",
               (D + 1) * (D + 1) - 1, M);
    GS_REQUIRE(cov3D_precomp != nullptr || (scales != nullptr && rotations != nullptr),
               "either cov3D_precomp or scales and rotations are needed");
    GS_REQUIRE(culling && means3D && opacities, "null input");
    GS_REQUIRE(image_width > 0 && image_height > 0, "image size must be positive");
    GS_REQUIRE(((uintptr_t)rotations & 15) == 0 && ((uintptr_t)conic_opacity & 15) == 0,
               "rotations and conic_opacity must be 16-byte aligned");
    GS_REQUIRE(((uintptr_t)rects & 7) == 0 && ((uintptr_t)cov3D & 7) == 0, "rects and cov3D must be 8-byte aligned");
    const FullPre F{culling, colors_precomp, cov3D_precomp, dc, rest, M, rects, tiles_touched};
    const float fy = (float)image_height / (2.0f * tanfovy);
    const float fx = (float)image_width / (2.0f * tanfovx);
    const dim3 grid(gs_div_up((size_t)P, 256)), block(256);
#define GS_PRE_FWD_FULL(DEG)                                                                                   \
    GS_TIMED("preprocess_fwd_full_kernel", stream,                                                             \
             hipLaunchKernelGGL((preprocess_fwd_kernel<DEG, true>), grid, block, 0, stream, P, 0, image_width, \
                                image_height, tanfovx, tanfovy, fx, fy, scale_modifier, viewmatrix, projmatrix, \
                                campos, means3D, scales, rotations, nullptr, 0, opacities, means2D, depths,     \
                                radii, cov3D, conic_opacity, rgb, clamped, F, BwdRec{}))
    switch (D) {
        case 0: GS_PRE_FWD_FULL(0); break;
        case 1: GS_PRE_FWD_FULL(1); break;
        case 2: GS_PRE_FWD_FULL(2); break;
        default: GS_PRE_FWD_FULL(3); break;
    }
#undef GS_PRE_FWD_FULL
    GS_LAUNCH_CHECK("preprocess_fwd_full_kernel");
    return GS_OK;
}

extern "C" int gs_preprocess_backward_full(
    int P, int D, int M, const float* means3D, const float* scales, const float* rotations, const float* dc,
    const float* rest, const float* colors_precomp, const float* cov3D_precomp, float scale_modifier,
    const float* viewmatrix, const float* projmatrix, const float* campos, float tanfovx, float tanfovy,
    int image_height, int image_width, const int* radii, const float* cov3D, const uint8_t* clamped,
    const float* dL_dmeans2D, const float* dL_dconic_opacity, const float* dL_dcolors, float* dL_dmeans3D,
    float* dL_dcov3D, float* dL_ddc, float* dL_drest, float* dL_dscales, float* dL_drotations,
    float* dL_dopacity, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0, "P must be >= 0 (got %d)", P);
    if (P == 0) return GS_OK;
    GS_REQUIRE(D >= 0 && D <= 3, "sh_degree must be in [0, 3] (got %d)", D);
    GS_REQUIRE(M >= 0, "M must be >= 0");
    const bool sh_grads = colors_precomp == nullptr && rest != nullptr && M > 0;
    GS_REQUIRE(!sh_grads || (dc != nullptr && M >= (D + 1) * (D + 1) - 1),
               "SH gradients need dc and at least (D+1)^2 - 1 = %d further coefficients (got %d)",
               (D + 1) * (D + 1) - 1, M);
    GS_REQUIRE(cov3D_precomp != nullptr || (scales != nullptr && rotations != nullptr),
               "either cov3D_precomp or scales and rotations are needed");
    GS_REQUIRE(((uintptr_t)rotations & 15) == 0 && ((uintptr_t)dL_dconic_opacity & 15) == 0 &&
               ((uintptr_t)dL_drotations & 15) == 0,
               "rotations, dL_dconic_opacity and dL_drotations must be 16-byte aligned");
    GS_REQUIRE(((uintptr_t)dL_dcov3D & 7) == 0 && ((uintptr_t)cov3D & 7) == 0,
               "dL_dcov3D and cov3D must be 8-byte aligned");
    const FullPreBwd F{cov3D_precomp, colors_precomp != nullptr, dc, sh_grads ? rest : nullptr, M, dL_ddc,
                       dL_drest, dL_dcov3D};
    const bool staged = M <= 15;
    const float fy = (float)image_height / (2.0f * tanfovy);
    const float fx = (float)image_width / (2.0f * tanfovx);
    const dim3 grid(gs_div_up((size_t)P, 256)), block(256);
#define GS_PRE_BWD_FULL(DEG)                                                                                     \
    if (staged)                                                                                                  \
        GS_TIMED("preprocess_bwd_full_kernel", stream,                                                           \
                 hipLaunchKernelGGL((preprocess_bwd_kernel<DEG, true, true>), grid, block, 0, stream, P, 0,        \
                                    image_width, image_height, tanfovx, tanfovy, fx, fy, scale_modifier,          \
                                    viewmatrix, projmatrix, campos, means3D, scales, rotations, nullptr, 0, radii, \
                                    cov3D, clamped, dL_dmeans2D, 3, dL_dconic_opacity, dL_dcolors, dL_dmeans3D,    \
                                    dL_dscales, dL_drotations, nullptr, dL_dopacity, F, nullptr, nullptr, 0));                         \
    else                                                                                                         \
        GS_TIMED("preprocess_bwd_full_kernel", stream,                                                           \
                 hipLaunchKernelGGL((preprocess_bwd_kernel<DEG, false, true>), grid, block, 0, stream, P, 0,       \
                                    image_width, image_height, tanfovx, tanfovy, fx, fy, scale_modifier,          \
                                    viewmatrix, projmatrix, campos, means3D, scales, rotations, nullptr, 0, radii, \
                                    cov3D, clamped, dL_dmeans2D, 3, dL_dconic_opacity, dL_dcolors, dL_dmeans3D,    \
                                    dL_dscales, dL_drotations, nullptr, dL_dopacity, F, nullptr, nullptr, 0))
    switch (D) {
        case 0: GS_PRE_BWD_FULL(0); break;
        case 1: GS_PRE_BWD_FULL(1); break;
        case 2: GS_PRE_BWD_FULL(2); break;
        default: GS_PRE_BWD_FULL(3); break;
    }
#undef GS_PRE_BWD_FULL
    GS_LAUNCH_CHECK("preprocess_bwd_full_kernel");
    return GS_OK;
}

namespace {

// checkFrustum (reference rasterizer_impl.cu:103-116 with in_frustum,
// auxiliary.h:158-184, prefiltered = false): visible = view-space z > 0.2.
__global__ __launch_bounds__(256) void mark_visible_kernel(int P, const float* __restrict__ means3D,
                                                           const float* __restrict__ view,
                                                           uint8_t* __restrict__ present)
{
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= P) return;
    const float x = means3D[3 * idx], y = means3D[3 * idx + 1], z = means3D[3 * idx + 2];
    const float vz = view[2] * x + view[6] * y + view[10] * z + view[14];
    present[idx] = vz <= 0.2f ? 0 : 1;
}

}  // namespace

extern "C" int gs_mark_visible(int P, const float* means3D, const float* viewmatrix, const float* projmatrix,
                               uint8_t* present, hipStream_t stream)
{
    gs::clear_error();
    (void)projmatrix;
    GS_REQUIRE(P >= 0, "P must be >= 0 (got %d)", P);
    if (P == 0) return GS_OK;
    GS_REQUIRE(means3D && viewmatrix && present, "null argument");
    GS_TIMED("mark_visible_kernel", stream,
             hipLaunchKernelGGL(mark_visible_kernel, dim3(gs_div_up((size_t)P, 256)), dim3(256), 0, stream, P,
                                means3D, viewmatrix, present));
    GS_LAUNCH_CHECK("mark_visible_kernel");
    return GS_OK;
}
