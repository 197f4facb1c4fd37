/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, never linked into the product.
 *
 * fp32 restatement of the per-Gaussian preprocess of BlitzGS's training path:
 *   forward : _f/cuda_rasterizer/forward.cu:28-284 (computeColorFromSH,
 *             computeCov2D, computeCov3D, preprocessCUDA) and
 *             _f/cuda_rasterizer/auxiliary.h:41-44,63-84,158-184
 *             (ndc2Pix, getRect(float2), transformPoint*, in_frustum);
 *             host side _f/cuda_rasterizer/rasterizer_impl.cu:982-1067.
 *   backward: _f/cuda_rasterizer/backward.cu:20-141 (SH), 146-276
 *             (computeCov2DCUDA), 280-343 (computeCov3D), 348-400
 *             (preprocessCUDA), auxiliary.h:126-136 (dnormvdv);
 *             host side _f/rasterize_points.cu:926-1029.
 * (All reference paths are under /root/reference/submodule/diff-gaussian-rasterization_f.)
 *
 * The reference writes its matrices with glm (column-major); here every
 * product is expanded into scalars.  Notation: Wm[r][c] = view[r*4+c] (the
 * rotation part of the world-to-view transform, transposed), the Jacobian
 * has non-zeros J00=fx/tz, J11=fy/tz, J20=-fx*tx/tz^2, J21=-fy*ty/tz^2, and
 * the 3x2 product T = Wm*J is stored as its two columns u (T[.][0]) and
 * w (T[.][1]).  The 2D covariance is (u^T S u, u^T S w, w^T S w) + 0.3 I.
 * Floating-point operation order is fixed (no contraction) and is spelled out
 * identically in the device code.
 */
#include "gs_oracle.h"
#include "o_math.h"

static const float SH_C0 = 0.28209479177387814f;
static const float SH_C1 = 0.4886025119029199f;
static const float SH_C2_0 = 1.0925484305920792f, SH_C2_1 = -1.0925484305920792f,
                   SH_C2_2 = 0.31539156525252005f, SH_C2_3 = -1.0925484305920792f,
                   SH_C2_4 = 0.5462742152960396f;
static const float SH_C3_0 = -0.5900435899266435f, SH_C3_1 = 2.890611442640554f,
                   SH_C3_2 = -0.4570457994644658f, SH_C3_3 = 0.3731763325901154f,
                   SH_C3_4 = -0.4570457994644658f, SH_C3_5 = 1.445305721320277f,
                   SH_C3_6 = -0.5900435899266435f;

/* _f auxiliary.h:76-96: row r of the 4x4 transform is m[r], m[4+r], m[8+r], m[12+r]. */
static inline void xform3(const float* m, float x, float y, float z, float* o)
{
    o[0] = m[0] * x + m[4] * y + m[8] * z + m[12];
    o[1] = m[1] * x + m[5] * y + m[9] * z + m[13];
    o[2] = m[2] * x + m[6] * y + m[10] * z + m[14];
}
static inline float xform_w(const float* m, float x, float y, float z)
{
    return m[3] * x + m[7] * y + m[11] * z + m[15];
}

/* _f auxiliary.h:41-44 -- evaluated in double precision. */
static inline float ndc2pix(float v, int S)
{
    return (float)((((double)v + 1.0) * (double)S - 1.0) * 0.5);
}

/* computeCov3D (_f forward.cu:127-161): Sigma = (S R)^T (S R), quaternion
 * (r,x,y,z) used without normalisation. Mm[r][c] = s_r * Rm[r][c] where Rm is
 * glm's R read row-wise. */
static void cov3d_fwd(const float* scale, float mod, const float* q, float* out6)
{
    const float r = q[0], x = q[1], y = q[2], z = q[3];
    float Rm[3][3];
    Rm[0][0] = 1.f - 2.f * (y * y + z * z); Rm[0][1] = 2.f * (x * y + r * z); Rm[0][2] = 2.f * (x * z - r * y);
    Rm[1][0] = 2.f * (x * y - r * z); Rm[1][1] = 1.f - 2.f * (x * x + z * z); Rm[1][2] = 2.f * (y * z + r * x);
    Rm[2][0] = 2.f * (x * z + r * y); Rm[2][1] = 2.f * (y * z - r * x); Rm[2][2] = 1.f - 2.f * (x * x + y * y);
    const float s[3] = { mod * scale[0], mod * scale[1], mod * scale[2] };
    float M[3][3];
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) M[i][j] = s[i] * Rm[i][j];
    /* Sigma[i][j] = sum_k M[k][i] M[k][j] */
    out6[0] = M[0][0] * M[0][0] + M[1][0] * M[1][0] + M[2][0] * M[2][0];
    out6[1] = M[0][0] * M[0][1] + M[1][0] * M[1][1] + M[2][0] * M[2][1];
    out6[2] = M[0][0] * M[0][2] + M[1][0] * M[1][2] + M[2][0] * M[2][2];
    out6[3] = M[0][1] * M[0][1] + M[1][1] * M[1][1] + M[2][1] * M[2][1];
    out6[4] = M[0][1] * M[0][2] + M[1][1] * M[1][2] + M[2][1] * M[2][2];
    out6[5] = M[0][2] * M[0][2] + M[1][2] * M[1][2] + M[2][2] * M[2][2];
}

/* Shared by cov2d forward and backward: clamped view-space mean t, the
 * columns u,w of T = Wm*J, and the clamp masks. (_f forward.cu:83-108,
 * backward.cu:166-194) */
typedef struct {
    float t[3];       /* t with x,y clamped */
    float u[3], w[3];
    float J00, J11, J20, J21;
    float xmask, ymask;
} o_ewa;

static void ewa_setup(const float* mean, float fx, float fy, float tanfovx, float tanfovy,
                      const float* view, o_ewa* e)
{
    float t[3];
    xform3(view, mean[0], mean[1], mean[2], t);
    const float limx = 1.3f * tanfovx;
    const float limy = 1.3f * tanfovy;
    const float txtz = t[0] / t[2];
    const float tytz = t[1] / t[2];
    t[0] = o_fminf(limx, o_fmaxf(-limx, txtz)) * t[2];
    t[1] = o_fminf(limy, o_fmaxf(-limy, tytz)) * t[2];
    e->xmask = (txtz < -limx || txtz > limx) ? 0.f : 1.f;
    e->ymask = (tytz < -limy || tytz > limy) ? 0.f : 1.f;
    e->t[0] = t[0]; e->t[1] = t[1]; e->t[2] = t[2];
    const float tz2 = t[2] * t[2];
    e->J00 = fx / t[2];
    e->J11 = fy / t[2];
    e->J20 = -(fx * t[0]) / tz2;
    e->J21 = -(fy * t[1]) / tz2;
    for (int r = 0; r < 3; r++) {
        e->u[r] = view[r * 4 + 0] * e->J00 + view[r * 4 + 2] * e->J20;
        e->w[r] = view[r * 4 + 1] * e->J11 + view[r * 4 + 2] * e->J21;
    }
}

/* Sigma * v for the packed symmetric 3x3 */
static inline void symv(const float* c6, const float* v, float* o)
{
    o[0] = c6[0] * v[0] + c6[1] * v[1] + c6[2] * v[2];
    o[1] = c6[1] * v[0] + c6[3] * v[1] + c6[4] * v[2];
    o[2] = c6[2] * v[0] + c6[4] * v[1] + c6[5] * v[2];
}

/* computeColorFromSH forward (_f forward.cu:28-80). sh points at the
 * Gaussian's (K,3) block; coefficient 0 is the DC term. */
static void sh_fwd(int deg, const float* pos, const float* campos, const float* sh,
                   float* out, uint8_t* clamped)
{
    float dir[3] = { pos[0] - campos[0], pos[1] - campos[1], pos[2] - campos[2] };
    const float len = sqrtf(dir[0] * dir[0] + dir[1] * dir[1] + dir[2] * dir[2]);
    dir[0] = dir[0] / len; dir[1] = dir[1] / len; dir[2] = dir[2] / len;
    const float x = dir[0], y = dir[1], z = dir[2];
    const float* s = sh;  /* s + 3*k = coefficient k */
    for (int c = 0; c < 3; c++) {
        float r = SH_C0 * s[c];
        if (deg > 0) {
            r = r - (SH_C1 * y) * s[3 + c] + (SH_C1 * z) * s[6 + c] - (SH_C1 * x) * s[9 + c];
            if (deg > 1) {
                const float xx = x * x, yy = y * y, zz = z * z;
                const float xy = x * y, yz = y * z, xz = x * z;
                r = r + (SH_C2_0 * xy) * s[12 + c] + (SH_C2_1 * yz) * s[15 + c] +
                    (SH_C2_2 * (2.0f * zz - xx - yy)) * s[18 + c] +
                    (SH_C2_3 * xz) * s[21 + c] + (SH_C2_4 * (xx - yy)) * s[24 + c];
                if (deg > 2) {
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
        clamped[c] = (r < 0.0f) ? 1 : 0;
        out[c] = o_fmaxf(r, 0.0f);
    }
}

/* Options of the full-image path's preprocess (forward.cu:165-284 with the
 * arguments rasterizer_impl.cu:396-424 passes): a culling mask, precomputed
 * colours or 3D covariances, the SH DC term and the rest in separate arrays,
 * and the float tile rect + tile count outputs.  The split path uses none. */
typedef struct {
    const uint8_t* culling;          /* P, nonzero = skip              */
    const float* colors_precomp;     /* P x 3 or NULL                  */
    const float* cov3D_precomp;      /* P x 6 or NULL                  */
    const float* dc;                 /* P x 3 (with rest) or NULL      */
    const float* rest;               /* P x M x 3                      */
    int M;
    float* rects;                    /* P x 2 or NULL                  */
    uint32_t* tiles_touched;         /* P or NULL                      */
} pre_opts;

static void pre_fwd(int P, int K, const o_camera* cam,
                    const float* means3D, const float* scales, const float* rotations,
                    const float* sh, const float* opacities, const pre_opts* o,
                    float* means2D, float* depths, int* radii, float* cov3D,
                    float* conic_opacity, float* rgb, uint8_t* clamped)
{
    const int W = cam->W, H = cam->H;
    const float fy = (float)H / (2.0f * cam->tanfovy);   /* rasterizer_impl.cu:1008-1009 */
    const float fx = (float)W / (2.0f * cam->tanfovx);
    const unsigned gx = (unsigned)((W + 15) / 16), gy = (unsigned)((H + 15) / 16);
    const float* V = cam->view;
    const float* PM = cam->proj;

#pragma omp parallel for schedule(static)
    for (int idx = 0; idx < P; idx++) {
        means2D[2 * idx] = 0.f; means2D[2 * idx + 1] = 0.f;
        depths[idx] = 0.f; radii[idx] = 0;
        for (int k = 0; k < 6; k++) cov3D[6 * idx + k] = 0.f;
        for (int k = 0; k < 4; k++) conic_opacity[4 * idx + k] = 0.f;
        for (int k = 0; k < 3; k++) { rgb[3 * idx + k] = 0.f; clamped[3 * idx + k] = 0; }
        if (o->rects) { o->rects[2 * idx] = 0.f; o->rects[2 * idx + 1] = 0.f; }
        if (o->tiles_touched) o->tiles_touched[idx] = 0;
        if (o->culling && o->culling[idx]) continue;    /* forward.cu:199-200 */

        const float* m = means3D + 3 * idx;
        /* in_frustum (auxiliary.h:158-184): near cull on view-space z */
        float pv[3];
        xform3(V, m[0], m[1], m[2], pv);
        if (pv[2] <= 0.2f) continue;
        /* projection (forward.cu:212-215) */
        float ph[3];
        xform3(PM, m[0], m[1], m[2], ph);
        const float pw = 1.0f / (xform_w(PM, m[0], m[1], m[2]) + 0.0000001f);
        const float pp0 = ph[0] * pw, pp1 = ph[1] * pw;

        float c6[6];
        if (o->cov3D_precomp) {
            for (int k = 0; k < 6; k++) c6[k] = o->cov3D_precomp[6 * idx + k];
        } else {
            cov3d_fwd(scales + 3 * idx, cam->scale_modifier, rotations + 4 * idx, c6);
            for (int k = 0; k < 6; k++) cov3D[6 * idx + k] = c6[k];
        }

        o_ewa e;
        ewa_setup(m, fx, fy, cam->tanfovx, cam->tanfovy, V, &e);
        float Su[3], Sw[3];
        symv(c6, e.u, Su);
        symv(c6, e.w, Sw);
        float ca = e.u[0] * Su[0] + e.u[1] * Su[1] + e.u[2] * Su[2];
        const float cb = e.u[0] * Sw[0] + e.u[1] * Sw[1] + e.u[2] * Sw[2];
        float cc = e.w[0] * Sw[0] + e.w[1] * Sw[1] + e.w[2] * Sw[2];
        ca = ca + 0.3f;
        cc = cc + 0.3f;

        /* forward.cu:234-238 */
        const float det = ca * cc - cb * cb;
        if (det == 0.0f) continue;
        const float det_inv = 1.f / det;
        const float con0 = cc * det_inv, con1 = -cb * det_inv, con2 = ca * det_inv;

        /* forward.cu:244-253: opacity-aware extent; min(3.33 (double), NaN) -> 3.33 */
        const float opacity = opacities[idx];
        const float opt = o_logf(opacity / (1.0f / 255.0f));
        const float sq = sqrtf(2.0f * opt);
        float extent;
        if (sq != sq || (double)sq >= 3.33) extent = (float)3.33;
        else extent = sq;
        const float mid = 0.5f * (ca + cc);
        const float lambda = mid + sqrtf(o_fmaxf(0.01f, mid * mid - det));
        const float my_radius = extent * sqrtf(lambda);
        if (my_radius <= 0.0f) continue;

        /* forward.cu:255-264 + auxiliary.h:63-73 */
        const float pix0 = ndc2pix(pp0, W), pix1 = ndc2pix(pp1, H);
        const float ex = o_fminf(extent * sqrtf(ca), my_radius);
        const float ey = o_fminf(extent * sqrtf(cc), my_radius);
        int v;
        v = o_f2i_sat(floorf((pix0 - ex) / 16.0f)); unsigned rminx = (unsigned)(v < 0 ? 0 : v); if (rminx > gx) rminx = gx;
        v = o_f2i_sat(floorf((pix1 - ey) / 16.0f)); unsigned rminy = (unsigned)(v < 0 ? 0 : v); if (rminy > gy) rminy = gy;
        v = o_f2i_sat(ceilf((pix0 + ex) / 16.0f));  unsigned rmaxx = (unsigned)(v < 0 ? 0 : v); if (rmaxx > gx) rmaxx = gx;
        v = o_f2i_sat(ceilf((pix1 + ey) / 16.0f));  unsigned rmaxy = (unsigned)(v < 0 ? 0 : v); if (rmaxy > gy) rmaxy = gy;
        const unsigned tiles = (rmaxx - rminx) * (rmaxy - rminy);
        if (tiles == 0) continue;

        /* forward.cu:268-275: SH colour unless colours are precomputed */
        if (!o->colors_precomp) {
            float col[3];
            if (o->dc) {
                float s48[48];
                for (int c = 0; c < 3; c++) s48[c] = o->dc[3 * idx + c];
                const int need = (cam->sh_degree + 1) * (cam->sh_degree + 1) - 1;
                for (int k = 0; k < 3 * need; k++) s48[3 + k] = o->rest[(size_t)idx * o->M * 3 + k];
                sh_fwd(cam->sh_degree, m, cam->campos, s48, col, clamped + 3 * idx);
            } else {
                sh_fwd(cam->sh_degree, m, cam->campos, sh + (size_t)idx * K * 3, col, clamped + 3 * idx);
            }
            rgb[3 * idx] = col[0]; rgb[3 * idx + 1] = col[1]; rgb[3 * idx + 2] = col[2];
        }

        depths[idx] = pv[2];
        radii[idx] = o_f2i_sat(ceilf(my_radius));
        means2D[2 * idx] = pix0; means2D[2 * idx + 1] = pix1;
        conic_opacity[4 * idx + 0] = con0;
        conic_opacity[4 * idx + 1] = con1;
        conic_opacity[4 * idx + 2] = con2;
        conic_opacity[4 * idx + 3] = opacity;
        if (o->rects) { o->rects[2 * idx] = ex; o->rects[2 * idx + 1] = ey; }
        if (o->tiles_touched) o->tiles_touched[idx] = tiles;
    }
}

void o_preprocess_fwd(int P, int K, const o_camera* cam,
                      const float* means3D, const float* scales, const float* rotations,
                      const float* sh, const float* opacities,
                      float* means2D, float* depths, int* radii, float* cov3D,
                      float* conic_opacity, float* rgb, uint8_t* clamped)
{
    const pre_opts o = { 0 };
    pre_fwd(P, K, cam, means3D, scales, rotations, sh, opacities, &o, means2D, depths, radii, cov3D,
            conic_opacity, rgb, clamped);
}

void o_preprocess_fwd_full(int P, int M, const o_camera* cam,
                           const float* means3D, const float* scales, const float* rotations,
                           const float* dc, const float* rest, const float* opacities,
                           const float* colors_precomp, const float* cov3D_precomp, const uint8_t* culling,
                           float* means2D, float* depths, int* radii, float* cov3D,
                           float* conic_opacity, float* rgb, uint8_t* clamped,
                           float* rects, uint32_t* tiles_touched)
{
    const pre_opts o = { culling, colors_precomp, cov3D_precomp, dc, rest, M, rects, tiles_touched };
    pre_fwd(P, 0, cam, means3D, scales, rotations, NULL, opacities, &o, means2D, depths, radii, cov3D,
            conic_opacity, rgb, clamped);
}

/* dnormvdv (auxiliary.h:126-136) */
static void dnormvdv3(const float* v, const float* dv, float* o)
{
    const float sum2 = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
    const float invsum32 = 1.0f / sqrtf(sum2 * sum2 * sum2);
    o[0] = ((sum2 - v[0] * v[0]) * dv[0] - v[1] * v[0] * dv[1] - v[2] * v[0] * dv[2]) * invsum32;
    o[1] = (-v[0] * v[1] * dv[0] + (sum2 - v[1] * v[1]) * dv[1] - v[2] * v[1] * dv[2]) * invsum32;
    o[2] = (-v[0] * v[2] * dv[0] - v[1] * v[2] * dv[1] + (sum2 - v[2] * v[2]) * dv[2]) * invsum32;
}

/* computeColorFromSH backward (backward.cu:20-141).  Writes dL/dsh (K,3) for
 * coefficients up to the degree and adds the view-direction term to dmean. */
static void sh_bwd(int deg, const float* pos, const float* campos, const float* sh,
                   const uint8_t* clamped, const float* dL_dcolor, float* dL_dsh, float* dmean)
{
    const float dir_orig[3] = { pos[0] - campos[0], pos[1] - campos[1], pos[2] - campos[2] };
    const float len = sqrtf(dir_orig[0] * dir_orig[0] + dir_orig[1] * dir_orig[1] + dir_orig[2] * dir_orig[2]);
    const float x = dir_orig[0] / len, y = dir_orig[1] / len, z = dir_orig[2] / len;
    float g[3];
    for (int c = 0; c < 3; c++) g[c] = clamped[c] ? 0.0f : dL_dcolor[c];
    float dx[3] = { 0, 0, 0 }, dy[3] = { 0, 0, 0 }, dz[3] = { 0, 0, 0 };
    const float* s = sh;
    for (int c = 0; c < 3; c++) dL_dsh[c] = SH_C0 * g[c];
    if (deg > 0) {
        const float b1 = -SH_C1 * y, b2 = SH_C1 * z, b3 = -SH_C1 * x;
        for (int c = 0; c < 3; c++) {
            dL_dsh[3 + c] = b1 * g[c]; dL_dsh[6 + c] = b2 * g[c]; dL_dsh[9 + c] = b3 * g[c];
            dx[c] = -SH_C1 * s[9 + c];
            dy[c] = -SH_C1 * s[3 + c];
            dz[c] = SH_C1 * s[6 + c];
        }
        if (deg > 1) {
            const float xx = x * x, yy = y * y, zz = z * z;
            const float xy = x * y, yz = y * z, xz = x * z;
            const float b4 = SH_C2_0 * xy, b5 = SH_C2_1 * yz, b6 = SH_C2_2 * (2.f * zz - xx - yy);
            const float b7 = SH_C2_3 * xz, b8 = SH_C2_4 * (xx - yy);
            for (int c = 0; c < 3; c++) {
                dL_dsh[12 + c] = b4 * g[c]; dL_dsh[15 + c] = b5 * g[c]; dL_dsh[18 + c] = b6 * g[c];
                dL_dsh[21 + c] = b7 * g[c]; dL_dsh[24 + c] = b8 * g[c];
                dx[c] += SH_C2_0 * y * s[12 + c] + SH_C2_2 * 2.f * -x * s[18 + c] + SH_C2_3 * z * s[21 + c] + SH_C2_4 * 2.f * x * s[24 + c];
                dy[c] += SH_C2_0 * x * s[12 + c] + SH_C2_1 * z * s[15 + c] + SH_C2_2 * 2.f * -y * s[18 + c] + SH_C2_4 * 2.f * -y * s[24 + c];
                dz[c] += SH_C2_1 * y * s[15 + c] + SH_C2_2 * 2.f * 2.f * z * s[18 + c] + SH_C2_3 * x * s[21 + c];
            }
            if (deg > 2) {
                const float b9 = SH_C3_0 * y * (3.f * xx - yy);
                const float b10 = SH_C3_1 * xy * z;
                const float b11 = SH_C3_2 * y * (4.f * zz - xx - yy);
                const float b12 = SH_C3_3 * z * (2.f * zz - 3.f * xx - 3.f * yy);
                const float b13 = SH_C3_4 * x * (4.f * zz - xx - yy);
                const float b14 = SH_C3_5 * z * (xx - yy);
                const float b15 = SH_C3_6 * x * (xx - 3.f * yy);
                for (int c = 0; c < 3; c++) {
                    dL_dsh[27 + c] = b9 * g[c]; dL_dsh[30 + c] = b10 * g[c]; dL_dsh[33 + c] = b11 * g[c];
                    dL_dsh[36 + c] = b12 * g[c]; dL_dsh[39 + c] = b13 * g[c]; dL_dsh[42 + c] = b14 * g[c];
                    dL_dsh[45 + c] = b15 * g[c];
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
    const float dL_ddir[3] = {
        dx[0] * g[0] + dx[1] * g[1] + dx[2] * g[2],
        dy[0] * g[0] + dy[1] * g[1] + dy[2] * g[2],
        dz[0] * g[0] + dz[1] * g[1] + dz[2] * g[2] };
    float dm[3];
    dnormvdv3(dir_orig, dL_ddir, dm);
    dmean[0] += dm[0]; dmean[1] += dm[1]; dmean[2] += dm[2];
}

/* computeCov3D backward (backward.cu:280-343): gradients w.r.t. the scale
 * (as multiplied by the modifier) and the un-normalised quaternion. */
static void cov3d_bwd(const float* scale, float mod, const float* q, const float* dc,
                      float* dL_dscale, float* dL_drot)
{
    const float r = q[0], x = q[1], y = q[2], z = q[3];
    float Rm[3][3];
    Rm[0][0] = 1.f - 2.f * (y * y + z * z); Rm[0][1] = 2.f * (x * y + r * z); Rm[0][2] = 2.f * (x * z - r * y);
    Rm[1][0] = 2.f * (x * y - r * z); Rm[1][1] = 1.f - 2.f * (x * x + z * z); Rm[1][2] = 2.f * (y * z + r * x);
    Rm[2][0] = 2.f * (x * z + r * y); Rm[2][1] = 2.f * (y * z - r * x); Rm[2][2] = 1.f - 2.f * (x * x + y * y);
    const float s[3] = { mod * scale[0], mod * scale[1], mod * scale[2] };
    float M[3][3];
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) M[i][j] = s[i] * Rm[i][j];
    const float D[3][3] = {
        { dc[0], 0.5f * dc[1], 0.5f * dc[2] },
        { 0.5f * dc[1], dc[3], 0.5f * dc[4] },
        { 0.5f * dc[2], 0.5f * dc[4], dc[5] } };
    /* dL/dM = 2 M D */
    float G[3][3];
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++)
            G[i][j] = (2.0f * M[i][0]) * D[0][j] + (2.0f * M[i][1]) * D[1][j] + (2.0f * M[i][2]) * D[2][j];
    for (int i = 0; i < 3; i++)
        dL_dscale[i] = Rm[i][0] * G[i][0] + Rm[i][1] * G[i][1] + Rm[i][2] * G[i][2];
    /* G[i][.] *= s_i  ->  dL/dRm */
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) G[i][j] = G[i][j] * s[i];
    dL_drot[0] = 2 * z * (G[0][1] - G[1][0]) + 2 * y * (G[2][0] - G[0][2]) + 2 * x * (G[1][2] - G[2][1]);
    dL_drot[1] = 2 * y * (G[1][0] + G[0][1]) + 2 * z * (G[2][0] + G[0][2]) + 2 * r * (G[1][2] - G[2][1]) - 4 * x * (G[2][2] + G[1][1]);
    dL_drot[2] = 2 * x * (G[1][0] + G[0][1]) + 2 * r * (G[2][0] - G[0][2]) + 2 * z * (G[1][2] + G[2][1]) - 4 * y * (G[2][2] + G[0][0]);
    dL_drot[3] = 2 * r * (G[0][1] - G[1][0]) + 2 * x * (G[2][0] + G[0][2]) + 2 * y * (G[1][2] + G[2][1]) - 4 * z * (G[1][1] + G[0][0]);
}

/* Options of the full-image path's backward (backward.cu:759-827 with the
 * arguments rasterizer_impl.cu:931-954 passes). */
typedef struct {
    int c11_slot;                    /* float4 slot of dL/dconic c11: 2 (split path) or 3 (full path) */
    const float* cov3D_precomp;      /* P x 6 or NULL: no scale/rotation gradients */
    int colors_precomp;              /* nonzero: no SH gradients */
    const float* dc;                 /* split SH: DC term, rest (P x M x 3) */
    const float* rest;
    int M;
    float* dL_ddc;                   /* P x 3 */
    float* dL_drest;                 /* P x M x 3 */
    float* dL_dcov3D;                /* P x 6 or NULL */
} pre_bwd_opts;

static void pre_bwd(int P, int K, const o_camera* cam,
                    const float* means3D, const float* scales, const float* rotations,
                    const float* sh, const int* radii, const float* cov3D,
                    const uint8_t* clamped,
                    const float* dL_dmeans2D, int m2d_stride,
                    const float* dL_dconic_opacity, const float* dL_drgb, const pre_bwd_opts* o,
                    float* dL_dmeans3D, float* dL_dscales, float* dL_drotations,
                    float* dL_dsh, float* dL_dopacity)
{
    const int W = cam->W, H = cam->H;
    const float fy = (float)H / (2.0f * cam->tanfovy);   /* rasterizer_impl.cu:1102-1103 */
    const float fx = (float)W / (2.0f * cam->tanfovx);
    const float* V = cam->view;
    const float* PM = cam->proj;
    const int full = o->dL_ddc != NULL || o->colors_precomp;

#pragma omp parallel for schedule(static)
    for (int idx = 0; idx < P; idx++) {
        /* rasterize_points.cu:977-982: opacity gradient is column 3 for every Gaussian */
        if (dL_dopacity) dL_dopacity[idx] = dL_dconic_opacity[4 * idx + 3];
        float* gm = dL_dmeans3D + 3 * idx;
        gm[0] = gm[1] = gm[2] = 0.f;
        for (int k = 0; k < 3; k++) dL_dscales[3 * idx + k] = 0.f;
        for (int k = 0; k < 4; k++) dL_drotations[4 * idx + k] = 0.f;
        if (dL_dsh) for (int k = 0; k < 3 * K; k++) dL_dsh[(size_t)idx * K * 3 + k] = 0.f;
        if (o->dL_ddc) for (int k = 0; k < 3; k++) o->dL_ddc[3 * idx + k] = 0.f;
        if (o->dL_drest) for (int k = 0; k < 3 * o->M; k++) o->dL_drest[(size_t)idx * o->M * 3 + k] = 0.f;
        if (o->dL_dcov3D) for (int k = 0; k < 6; k++) o->dL_dcov3D[6 * idx + k] = 0.f;
        if (!(radii[idx] > 0)) continue;

        const float* m = means3D + 3 * idx;
        const float* c6 = o->cov3D_precomp ? o->cov3D_precomp + 6 * idx : cov3D + 6 * idx;
        /* ---- computeCov2DCUDA (backward.cu:146-276) ---- */
        o_ewa e;
        ewa_setup(m, fx, fy, cam->tanfovx, cam->tanfovy, V, &e);
        float Su[3], Sw[3];
        symv(c6, e.u, Su);
        symv(c6, e.w, Sw);
        float a = e.u[0] * Su[0] + e.u[1] * Su[1] + e.u[2] * Su[2];
        const float b = e.u[0] * Sw[0] + e.u[1] * Sw[1] + e.u[2] * Sw[2];
        float c = e.w[0] * Sw[0] + e.w[1] * Sw[1] + e.w[2] * Sw[2];
        a = a + 0.3f;
        c = c + 0.3f;
        const float g0 = dL_dconic_opacity[4 * idx + 0];
        const float g1 = dL_dconic_opacity[4 * idx + 1];
        const float g2 = dL_dconic_opacity[4 * idx + o->c11_slot];
        const float denom = a * c - b * b;
        const float denom2inv = 1.0f / ((denom * denom) + 0.0000001f);
        float dL_da = 0, dL_db = 0, dL_dc = 0;
        float dcov[6] = { 0, 0, 0, 0, 0, 0 };
        if (denom2inv != 0) {
            dL_da = denom2inv * (-c * c * g0 + 2 * b * c * g1 + (denom - a * c) * g2);
            dL_dc = denom2inv * (-a * a * g2 + 2 * a * b * g1 + (denom - a * c) * g0);
            dL_db = denom2inv * 2 * (b * c * g0 - (denom + 2 * b * b) * g1 + a * b * g2);
            const float* u = e.u; const float* w = e.w;
            dcov[0] = u[0] * u[0] * dL_da + u[0] * w[0] * dL_db + w[0] * w[0] * dL_dc;
            dcov[3] = u[1] * u[1] * dL_da + u[1] * w[1] * dL_db + w[1] * w[1] * dL_dc;
            dcov[5] = u[2] * u[2] * dL_da + u[2] * w[2] * dL_db + w[2] * w[2] * dL_dc;
            dcov[1] = 2 * u[0] * u[1] * dL_da + (u[0] * w[1] + u[1] * w[0]) * dL_db + 2 * w[0] * w[1] * dL_dc;
            dcov[2] = 2 * u[0] * u[2] * dL_da + (u[0] * w[2] + u[2] * w[0]) * dL_db + 2 * w[0] * w[2] * dL_dc;
            dcov[4] = 2 * u[2] * u[1] * dL_da + (u[1] * w[2] + u[2] * w[1]) * dL_db + 2 * w[1] * w[2] * dL_dc;
        }
        if (o->dL_dcov3D) for (int k = 0; k < 6; k++) o->dL_dcov3D[6 * idx + k] = dcov[k];
        /* dL/du = 2 S u dL_da + S w dL_db ; dL/dw = 2 S w dL_dc + S u dL_db */
        float du[3], dw[3];
        for (int k = 0; k < 3; k++) {
            du[k] = 2 * Su[k] * dL_da + Sw[k] * dL_db;
            dw[k] = 2 * Sw[k] * dL_dc + Su[k] * dL_db;
        }
        const float dJ00 = V[0] * du[0] + V[4] * du[1] + V[8] * du[2];
        const float dJ20 = V[2] * du[0] + V[6] * du[1] + V[10] * du[2];
        const float dJ11 = V[1] * dw[0] + V[5] * dw[1] + V[9] * dw[2];
        const float dJ21 = V[2] * dw[0] + V[6] * dw[1] + V[10] * dw[2];
        const float tz = 1.f / e.t[2];
        const float tz2 = tz * tz;
        const float tz3 = tz2 * tz;
        const float dtx = e.xmask * -fx * tz2 * dJ20;
        const float dty = e.ymask * -fy * tz2 * dJ21;
        const float dtz = -fx * tz2 * dJ00 - fy * tz2 * dJ11 + (2 * fx * e.t[0]) * tz3 * dJ20 + (2 * fy * e.t[1]) * tz3 * dJ21;
        /* transformVec4x3Transpose (auxiliary.h:108-116) -- assigned */
        gm[0] = V[0] * dtx + V[1] * dty + V[2] * dtz;
        gm[1] = V[4] * dtx + V[5] * dty + V[6] * dtz;
        gm[2] = V[8] * dtx + V[9] * dty + V[10] * dtz;

        /* ---- preprocessCUDA backward (backward.cu:374-391) ---- */
        float mh[3];
        xform3(PM, m[0], m[1], m[2], mh);
        const float m_w = 1.0f / (xform_w(PM, m[0], m[1], m[2]) + 0.0000001f);
        const float mul1 = (PM[0] * m[0] + PM[4] * m[1] + PM[8] * m[2] + PM[12]) * m_w * m_w;
        const float mul2 = (PM[1] * m[0] + PM[5] * m[1] + PM[9] * m[2] + PM[13]) * m_w * m_w;
        const float gx = dL_dmeans2D[(size_t)idx * m2d_stride + 0];
        const float gy = dL_dmeans2D[(size_t)idx * m2d_stride + 1];
        gm[0] += (PM[0] * m_w - PM[3] * mul1) * gx + (PM[1] * m_w - PM[3] * mul2) * gy;
        gm[1] += (PM[4] * m_w - PM[7] * mul1) * gx + (PM[5] * m_w - PM[7] * mul2) * gy;
        gm[2] += (PM[8] * m_w - PM[11] * mul1) * gx + (PM[9] * m_w - PM[11] * mul2) * gy;

        if (!full) {
            sh_bwd(cam->sh_degree, m, cam->campos, sh + (size_t)idx * K * 3, clamped + 3 * idx,
                   dL_drgb + 3 * idx, dL_dsh + (size_t)idx * K * 3, gm);
        } else if (!o->colors_precomp && o->rest && o->M > 0) {
            /* backward.cu:392-393: SH gradients only when the rest array exists */
            const int need = (cam->sh_degree + 1) * (cam->sh_degree + 1);
            float s48[48], g48[48];
            for (int k = 0; k < 48; k++) { s48[k] = 0.f; g48[k] = 0.f; }
            for (int ch = 0; ch < 3; ch++) s48[ch] = o->dc[3 * idx + ch];
            for (int k = 0; k < 3 * (need - 1); k++) s48[3 + k] = o->rest[(size_t)idx * o->M * 3 + k];
            sh_bwd(cam->sh_degree, m, cam->campos, s48, clamped + 3 * idx, dL_drgb + 3 * idx, g48, gm);
            for (int ch = 0; ch < 3; ch++) o->dL_ddc[3 * idx + ch] = g48[ch];
            for (int k = 0; k < 3 * (need - 1); k++) o->dL_drest[(size_t)idx * o->M * 3 + k] = g48[3 + k];
        }
        if (!o->cov3D_precomp)
            cov3d_bwd(scales + 3 * idx, cam->scale_modifier, rotations + 4 * idx, dcov,
                      dL_dscales + 3 * idx, dL_drotations + 4 * idx);
    }
}

void o_preprocess_bwd(int P, int K, const o_camera* cam,
                      const float* means3D, const float* scales, const float* rotations,
                      const float* sh, const int* radii, const float* cov3D,
                      const uint8_t* clamped,
                      const float* dL_dmeans2D, int m2d_stride,
                      const float* dL_dconic_opacity, const float* dL_drgb,
                      float* dL_dmeans3D, float* dL_dscales, float* dL_drotations,
                      float* dL_dsh, float* dL_dopacity)
{
    pre_bwd_opts o = { 0 };
    o.c11_slot = 2;
    pre_bwd(P, K, cam, means3D, scales, rotations, sh, radii, cov3D, clamped, dL_dmeans2D, m2d_stride,
            dL_dconic_opacity, dL_drgb, &o, dL_dmeans3D, dL_dscales, dL_drotations, dL_dsh, dL_dopacity);
}

void o_preprocess_bwd_full(int P, int M, const o_camera* cam,
                           const float* means3D, const float* scales, const float* rotations,
                           const float* dc, const float* rest, const float* colors_precomp,
                           const float* cov3D_precomp, const int* radii, const float* cov3D,
                           const uint8_t* clamped, const float* dL_dmeans2D, const float* dL_dconic,
                           const float* dL_dcolors,
                           float* dL_dmeans3D, float* dL_dcov3D, float* dL_ddc, float* dL_drest,
                           float* dL_dscales, float* dL_drotations)
{
    pre_bwd_opts o;
    o.c11_slot = 3;
    o.cov3D_precomp = cov3D_precomp;
    o.colors_precomp = colors_precomp != NULL;
    o.dc = dc;
    o.rest = rest;
    o.M = M;
    o.dL_ddc = dL_ddc;
    o.dL_drest = dL_drest;
    o.dL_dcov3D = dL_dcov3D;
    pre_bwd(P, 0, cam, means3D, scales, rotations, NULL, radii, cov3D, clamped, dL_dmeans2D, 3, dL_dconic,
            dL_dcolors, &o, dL_dmeans3D, dL_dscales, dL_drotations, NULL, NULL);
}
