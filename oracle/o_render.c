/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, never linked into the product.
 *
 * fp32 restatement of the reference's binning and tile rendering
 * (/root/reference/submodule/diff-gaussian-rasterization_r):
 *   getHigherMsb              cuda_rasterizer/rasterizer_impl.cu:39-54
 *   duplicateWithKeys         cuda_rasterizer/rasterizer_impl.cu:74-111
 *   identifyTileRanges        cuda_rasterizer/rasterizer_impl.cu:116-138
 *   get_n_render / reduce_data_per_block  rasterizer_impl.cu:213-256
 *   updateTileTouched         cuda_rasterizer/rasterizer_impl.cu:258-282
 *   renderForward sequence    cuda_rasterizer/rasterizer_impl.cu:556-723
 *   getRect(float2,int)       cuda_rasterizer/auxiliary.h:66-76
 *   renderCUDA (forward)      cuda_rasterizer/forward.cu:263-413
 *   renderCUDA (backward)     cuda_rasterizer/backward.cu:324-530
 *   render_geo maps (fwd)     cuda_rasterizer/forward.cu:381-384,407-412
 *   render_geo maps (bwd)     cuda_rasterizer/backward.cu:393-405,427-432,476-490
 * The reference sorts with a stable LSD radix sort on bits [0, 32+msb); here a
 * stable merge sort on the full 64-bit key gives the same order (tile ids are
 * below 2^msb, checked in the tests, and depth bits are the low word).
 *
 * Per-pixel arithmetic is written in the fixed order the device code uses:
 *   d = mean - pixel;  power = fma(-0.5a*dx, dx, fma(-0.5c*dy, dy, (-b*dx)*dy))
 *   G = o_expf(power); alpha = min(0.99, o*G);  C = fma(rgb, alpha*T, C)
 * which is the reference's expression with its products grouped for FMA.
 */
#include "gs_oracle.h"
#include "o_math.h"
#include <stdlib.h>

#define OT 16  /* BLOCK_X = BLOCK_Y = 16 (config.h) */

uint32_t o_higher_msb(uint32_t n)
{
    uint32_t msb = sizeof(n) * 4;
    uint32_t step = msb;
    while (step > 1) {
        step /= 2;
        if (n >> msb) msb += step;
        else msb -= step;
    }
    if (n >> msb) msb++;
    return msb;
}

/* getRect with an integer radius: float arithmetic left to right, (int)
 * truncation toward zero, clamped to [0, grid]. */
static inline void rect_int(const float* p, int r, unsigned gx, unsigned gy,
                            unsigned* x0, unsigned* y0, unsigned* x1, unsigned* y1)
{
    const float rf = (float)r;
    int v;
    v = o_f2i_sat((p[0] - rf) / 16.0f); v = v < 0 ? 0 : v; *x0 = (unsigned)v > gx ? gx : (unsigned)v;
    v = o_f2i_sat((p[1] - rf) / 16.0f); v = v < 0 ? 0 : v; *y0 = (unsigned)v > gy ? gy : (unsigned)v;
    v = o_f2i_sat(((p[0] + rf) + 16.0f - 1.0f) / 16.0f); v = v < 0 ? 0 : v; *x1 = (unsigned)v > gx ? gx : (unsigned)v;
    v = o_f2i_sat(((p[1] + rf) + 16.0f - 1.0f) / 16.0f); v = v < 0 ? 0 : v; *y1 = (unsigned)v > gy ? gy : (unsigned)v;
}

int64_t o_binning_count(int P, int W, int H, const float* means2D, const int* radii,
                        const uint8_t* compute_locally, uint32_t* tiles_touched)
{
    const unsigned gx = (unsigned)((W + OT - 1) / OT), gy = (unsigned)((H + OT - 1) / OT);
    int64_t total = 0;
#pragma omp parallel for schedule(static) reduction(+ : total)
    for (int i = 0; i < P; i++) {
        uint32_t cnt = 0;
        if (radii[i] > 0) {
            unsigned x0, y0, x1, y1;
            rect_int(means2D + 2 * i, radii[i], gx, gy, &x0, &y0, &x1, &y1);
            for (unsigned y = y0; y < y1; y++)
                for (unsigned x = x0; x < x1; x++)
                    if (compute_locally[y * gx + x]) cnt++;
        }
        tiles_touched[i] = cnt;
        total += cnt;
    }
    return total;
}

void o_binning(int P, int W, int H, const float* means2D, const float* depths,
               const int* radii, const uint8_t* compute_locally,
               const uint32_t* tiles_touched, int64_t R,
               uint64_t* keys, uint32_t* values, uint32_t* ranges)
{
    const unsigned gx = (unsigned)((W + OT - 1) / OT), gy = (unsigned)((H + OT - 1) / OT);
    const unsigned T = gx * gy;
    int64_t* off = (int64_t*)malloc(sizeof(int64_t) * (size_t)(P > 0 ? P : 1));
    int64_t acc = 0;
    for (int i = 0; i < P; i++) { off[i] = acc; acc += tiles_touched[i]; }

    /* duplicateWithKeys: Gaussian order, then rows, then columns */
#pragma omp parallel for schedule(static)
    for (int i = 0; i < P; i++) {
        if (!(radii[i] > 0)) continue;
        int64_t o = off[i];
        unsigned x0, y0, x1, y1;
        rect_int(means2D + 2 * i, radii[i], gx, gy, &x0, &y0, &x1, &y1);
        const uint32_t dbits = o_f2u(depths[i]);
        for (unsigned y = y0; y < y1; y++)
            for (unsigned x = x0; x < x1; x++)
                if (compute_locally[y * gx + x]) {
                    keys[o] = ((uint64_t)(y * gx + x) << 32) | dbits;
                    values[o] = (uint32_t)i;
                    o++;
                }
    }
    free(off);

    /* stable sort by key */
    if (R > 1) {
        uint64_t* tk = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)R);
        uint32_t* tv = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)R);
        uint64_t* a = keys; uint32_t* av = values;
        uint64_t* b = tk; uint32_t* bv = tv;
        for (int64_t width = 1; width < R; width *= 2) {
#pragma omp parallel for schedule(dynamic, 1)
            for (int64_t lo = 0; lo < R; lo += 2 * width) {
                int64_t mid = lo + width < R ? lo + width : R;
                int64_t hi = lo + 2 * width < R ? lo + 2 * width : R;
                int64_t i = lo, j = mid, o = lo;
                while (i < mid && j < hi) {
                    if (a[j] < a[i]) { b[o] = a[j]; bv[o] = av[j]; j++; }
                    else { b[o] = a[i]; bv[o] = av[i]; i++; }
                    o++;
                }
                while (i < mid) { b[o] = a[i]; bv[o] = av[i]; i++; o++; }
                while (j < hi) { b[o] = a[j]; bv[o] = av[j]; j++; o++; }
            }
            uint64_t* s = a; a = b; b = s;
            uint32_t* sv = av; av = bv; bv = sv;
        }
        if (a != keys) {
            memcpy(keys, a, sizeof(uint64_t) * (size_t)R);
            memcpy(values, av, sizeof(uint32_t) * (size_t)R);
        }
        free(tk); free(tv);
    }

    /* identifyTileRanges (after the memset of rasterizer_impl.cu:655) */
    memset(ranges, 0, sizeof(uint32_t) * 2 * (size_t)T);
    for (int64_t idx = 0; idx < R; idx++) {
        const uint32_t cur = (uint32_t)(keys[idx] >> 32);
        if (idx == 0) ranges[2 * cur] = 0;
        else {
            const uint32_t prev = (uint32_t)(keys[idx - 1] >> 32);
            if (cur != prev) { ranges[2 * prev + 1] = (uint32_t)idx; ranges[2 * cur] = (uint32_t)idx; }
        }
        if (idx == R - 1) ranges[2 * cur + 1] = (uint32_t)R;
    }
}

/* the per-(pixel, Gaussian) Gaussian falloff exponent, in the device order */
static inline float o_power(const float* xy, const float* co, float px, float py)
{
    const float dx = xy[0] - px, dy = xy[1] - py;
    const float ha = -0.5f * co[0], hc = -0.5f * co[2], nb = -co[1];
    return fmaf(ha * dx, dx, fmaf(hc * dy, dy, (nb * dx) * dy));
}

/* Margin model of o_render_fwd's decision bounds (test hook): exp_delta != 0
 * multiplies each evaluated exp by 1 +- exp_delta (sign from a hash of the
 * Gaussian and the pixel), to emulate a blend whose exp differs slightly;
 * bound_rel is the relative exp error the margins assume (O_EXP_REL). */
static float g_exp_delta = 0.0f, g_bound_rel = O_EXP_REL;

void o_set_blend_margin_model(float exp_delta, float bound_rel)
{
    g_exp_delta = exp_delta;
    g_bound_rel = bound_rel;
}

static inline float perturb_sign(uint32_t id, size_t pid)
{
    uint32_t h = id * 0x9E3779B1u ^ (uint32_t)pid * 0x85EBCA77u;
    h ^= h >> 15; h *= 0x2C1B3C6Du; h ^= h >> 12;
    return (h & 1u) ? 1.0f : -1.0f;
}

void o_render_fwd(int P, int W, int H, const float* bg,
                  const float* means2D, const float* conic_opacity, const float* rgb,
                  const uint8_t* compute_locally,
                  const uint32_t* ranges, const uint32_t* point_list,
                  float* out_color, float* final_T, uint32_t* n_contrib,
                  uint32_t* n_contrib2loss, int32_t* out_observe,
                  int32_t* n_render, int32_t* n_consider, int32_t* n_contrib_tile,
                  int32_t* obs_near, uint8_t* stop_near)
{
    (void)P;
    const int gx = (W + OT - 1) / OT, gy = (H + OT - 1) / OT;
    const int T = gx * gy;
    const float alpha_min = 1.0f / 255.0f;
#pragma omp parallel for schedule(dynamic, 1)
    for (int t = 0; t < T; t++) {
        const int tx = t % gx, ty = t / gx;
        n_render[t] = (int32_t)(ranges[2 * t + 1] - ranges[2 * t]);
        n_consider[t] = 0; n_contrib_tile[t] = 0;
        const int x0 = tx * OT, y0 = ty * OT;
        const int x1 = x0 + OT < W ? x0 + OT : W, y1 = y0 + OT < H ? y0 + OT : H;
        if (!compute_locally[t]) {
            for (int y = y0; y < y1; y++)
                for (int x = x0; x < x1; x++) {
                    const size_t pid = (size_t)y * W + x;
                    for (int c = 0; c < 3; c++) out_color[(size_t)c * H * W + pid] = 0.f;
                    final_T[pid] = 0.f; n_contrib[pid] = 0; n_contrib2loss[pid] = 0;
                    if (stop_near) stop_near[pid] = 0;
                }
            continue;
        }
        const uint32_t rs = ranges[2 * t], re = ranges[2 * t + 1];
        int64_t s_consider = 0, s_contrib = 0;
        for (int y = y0; y < y1; y++)
            for (int x = x0; x < x1; x++) {
                const float px = (float)x, py = (float)y;
                const size_t pid = (size_t)y * W + x;
                float T_ = 1.0f, C[3] = { 0.f, 0.f, 0.f };
                uint32_t contributor = 0, last = 0, n2l = 0;
                double bound = 0.0;  /* relative error bound of T_ (decision margins only) */
                int snear = 0;
                for (uint32_t k = rs; k < re; k++) {
                    contributor++;
                    const uint32_t id = point_list[k];
                    const float* co = conic_opacity + 4 * (size_t)id;
                    const float power = o_power(means2D + 2 * (size_t)id, co, px, py);
                    if (power > 0.0f) continue;
                    const float G = o_expf(power);
                    float alpha = o_fminf(0.99f, co[3] * G);
                    if (alpha < alpha_min) continue;
                    /* test hook: the blend (not the exact alpha >= 1/255 cut) with a perturbed exp */
                    if (g_exp_delta != 0.0f)
                        alpha = o_fminf(0.99f, co[3] * (G * (1.0f + g_exp_delta * perturb_sign(id, pid))));
                    const float test_T = T_ * (1.0f - alpha);
                    const double bound_next = bound + (double)g_bound_rel * alpha / (1.0 - alpha) + 2.4e-7;
                    if (fabs((double)test_T - 1e-4) <= 1e-4 * bound_next) snear = 1;
                    if (test_T < 0.0001f) break;
                    n2l++;
                    const float wgt = alpha * T_;
                    for (int c = 0; c < 3; c++) C[c] = fmaf(rgb[3 * (size_t)id + c], wgt, C[c]);
                    if (T_ > 0.5f) {
#pragma omp atomic
                        out_observe[id]++;
                    }
                    if (obs_near && fabs((double)T_ - 0.5) <= 0.5 * bound) {
#pragma omp atomic
                        obs_near[id]++;
                    }
                    T_ = test_T;
                    bound = bound_next;
                    last = contributor;
                }
                if (stop_near) stop_near[pid] = (uint8_t)snear;
                final_T[pid] = T_;
                n_contrib[pid] = last;
                n_contrib2loss[pid] = n2l;
                for (int c = 0; c < 3; c++) out_color[(size_t)c * H * W + pid] = fmaf(T_, bg[c], C[c]);
                s_consider += last;
                s_contrib += n2l;
            }
        n_consider[t] = (int32_t)s_consider;
        n_contrib_tile[t] = (int32_t)s_contrib;
    }
}

/* plane depth of one pixel (_r forward.cu:411): all_map[4] / -(n . ray + 1e-8)
 * with n = all_map[0..2], ray = (rx, ry, 1); the dot product in float
 * (fma(n0, rx, n1 ry) + n2), the 1e-8 (a double literal), the negation and
 * the division in double, stored as float */
static inline float plane_depth(const float* M, float rx, float ry)
{
    const float s = fmaf(M[0], rx, M[1] * ry) + M[2];
    return (float)((double)M[4] / -((double)s + 1.0e-8));
}

void o_render_geo_fwd(int W, int H, float focal_x, float focal_y, float cx, float cy,
                      const float* means2D, const float* conic_opacity, const float* all_map,
                      const uint8_t* compute_locally, const uint32_t* ranges, const uint32_t* point_list,
                      float* out_all_map, float* out_plane_depth)
{
    const int gx = (W + OT - 1) / OT, gy = (H + OT - 1) / OT;
    const int T = gx * gy;
    const size_t HW = (size_t)H * W;
    const float alpha_min = 1.0f / 255.0f;
#pragma omp parallel for schedule(dynamic, 1)
    for (int t = 0; t < T; t++) {
        const int tx = t % gx, ty = t / gx;
        const int x0 = tx * OT, y0 = ty * OT;
        const int x1 = x0 + OT < W ? x0 + OT : W, y1 = y0 + OT < H ? y0 + OT : H;
        const int local = compute_locally[t] != 0;
        const uint32_t rs = ranges[2 * t], re = ranges[2 * t + 1];
        for (int y = y0; y < y1; y++)
            for (int x = x0; x < x1; x++) {
                const size_t pid = (size_t)y * W + x;
                float M[O_NUM_MAPS] = { 0.f, 0.f, 0.f, 0.f, 0.f };
                if (!local) {
                    for (int c = 0; c < O_NUM_MAPS; c++) out_all_map[c * HW + pid] = 0.f;
                    out_plane_depth[pid] = 0.f;
                    continue;
                }
                const float px = (float)x, py = (float)y;
                float T_ = 1.0f;
                for (uint32_t k = rs; k < re; k++) {
                    const uint32_t id = point_list[k];
                    const float* co = conic_opacity + 4 * (size_t)id;
                    const float power = o_power(means2D + 2 * (size_t)id, co, px, py);
                    if (power > 0.0f) continue;
                    const float alpha = o_fminf(0.99f, co[3] * o_expf(power));
                    if (alpha < alpha_min) continue;
                    const float test_T = T_ * (1.0f - alpha);
                    if (test_T < 0.0001f) break;
                    const float wgt = alpha * T_;
                    for (int c = 0; c < O_NUM_MAPS; c++) M[c] = fmaf(all_map[O_NUM_MAPS * (size_t)id + c], wgt, M[c]);
                    T_ = test_T;
                }
                for (int c = 0; c < O_NUM_MAPS; c++) out_all_map[c * HW + pid] = M[c];
                out_plane_depth[pid] = plane_depth(M, (px - cx) / focal_x, (py - cy) / focal_y);
            }
    }
}

static inline void atomic_addf(float* p, float v)
{
#pragma omp atomic
    *p += v;
}

/* full != 0: the full-image path's rule (_f backward.cu:560-566): no
 * |dL/dmean2D| output, and no conic / opacity gradient where the alpha clamp
 * at 0.99 is active (opacity * G > 0.99). */
static void render_bwd_impl(int full, int W, int H, const float* bg,
                            const float* means2D, const float* conic_opacity, const float* rgb,
                            const uint8_t* compute_locally,
                            const uint32_t* ranges, const uint32_t* point_list,
                            const float* final_T, const uint32_t* n_contrib,
                            const float* dL_dpixels,
                            float* dL_dmean2D, float* dL_dmean2D_abs, float* dL_dconic,
                            float* dL_dopacity, float* dL_dcolors, const OGeoBwd* geo)
{
    const int gx = (W + OT - 1) / OT, gy = (H + OT - 1) / OT;
    const size_t HW = (size_t)H * W;
    const int T = gx * gy;
    const float alpha_min = 1.0f / 255.0f;
    const float ddelx_dx = 0.5f * (float)W, ddely_dy = 0.5f * (float)H;
#pragma omp parallel for schedule(dynamic, 1)
    for (int t = 0; t < T; t++) {
        if (compute_locally && !compute_locally[t]) continue;
        const int tx = t % gx, ty = t / gx;
        const int x0 = tx * OT, y0 = ty * OT;
        const int x1 = x0 + OT < W ? x0 + OT : W, y1 = y0 + OT < H ? y0 + OT : H;
        const uint32_t rs = ranges[2 * t], re = ranges[2 * t + 1];
        for (int y = y0; y < y1; y++)
            for (int x = x0; x < x1; x++) {
                const size_t pid = (size_t)y * W + x;
                const float px = (float)x, py = (float)y;
                const float T_final = final_T[pid];
                float T_ = T_final;
                const uint32_t last = n_contrib[pid];
                float dpix[3], accum[3] = { 0, 0, 0 }, last_color[3] = { 0, 0, 0 };
                for (int c = 0; c < 3; c++) dpix[c] = dL_dpixels[(size_t)c * H * W + pid];
                float last_alpha = 0.f;
                /* render_geo (_r backward.cu:393-405): the maps' pixel
                 * gradients, plus the plane depth's through n and distance */
                float dmap[O_NUM_MAPS], accm[O_NUM_MAPS] = { 0, 0, 0, 0, 0 }, lastm[O_NUM_MAPS] = { 0, 0, 0, 0, 0 };
                if (geo) {
                    const float rx = (float)(((double)px - W * 0.5) / geo->fx);
                    const float ry = (float)(((double)py - H * 0.5) / geo->fy);
                    for (int c = 0; c < O_NUM_MAPS; c++) dmap[c] = geo->dL_dmaps[c * HW + pid];
                    const float* mp = geo->all_map_pixels;
                    const float n0 = mp[pid], n1 = mp[HW + pid], n2 = mp[2 * HW + pid];
                    const float distance = mp[4 * HW + pid];
                    const float tmp = (float)((double)(n0 * rx + n1 * ry + n2) + 1.0e-8);
                    const float g = geo->dL_dplane[pid];
                    dmap[O_NUM_MAPS - 1] += -g / tmp;
                    dmap[0] += g * (distance / (tmp * tmp) * rx);
                    dmap[1] += g * (distance / (tmp * tmp) * ry);
                    dmap[2] += g * (distance / (tmp * tmp));
                }
                float bg_dot = 0.f;
                for (int c = 0; c < 3; c++) bg_dot += bg[c] * dpix[c];
                /* contributor index k-rs+1 runs from the back; skip >= last */
                for (int64_t k = (int64_t)re - 1; k >= (int64_t)rs; k--) {
                    const uint32_t contributor = (uint32_t)(k - rs);  /* after the decrement */
                    if (contributor >= last) continue;
                    const uint32_t id = point_list[k];
                    const float* xy = means2D + 2 * (size_t)id;
                    const float* co = conic_opacity + 4 * (size_t)id;
                    const float dx = xy[0] - px, dy = xy[1] - py;
                    const float power = o_power(xy, co, px, py);
                    if (power > 0.0f) continue;
                    const float G = o_expf(power);
                    const float alpha = o_fminf(0.99f, co[3] * G);
                    if (alpha < alpha_min) continue;
                    T_ = T_ / (1.f - alpha);
                    const float dchannel_dcolor = alpha * T_;
                    float dL_dalpha = 0.0f;
                    for (int c = 0; c < 3; c++) {
                        const float col = rgb[3 * (size_t)id + c];
                        accum[c] = last_alpha * last_color[c] + (1.f - last_alpha) * accum[c];
                        last_color[c] = col;
                        dL_dalpha += (col - accum[c]) * dpix[c];
                        atomic_addf(&dL_dcolors[3 * (size_t)id + c], dchannel_dcolor * dpix[c]);
                    }
                    if (geo) {
                        for (int c = 0; c < O_NUM_MAPS; c++) {
                            const float m = geo->all_maps[O_NUM_MAPS * (size_t)id + c];
                            accm[c] = last_alpha * lastm[c] + (1.f - last_alpha) * accm[c];
                            lastm[c] = m;
                            dL_dalpha += (m - accm[c]) * dmap[c];
                            atomic_addf(&geo->dL_dall_map[O_NUM_MAPS * (size_t)id + c], dchannel_dcolor * dmap[c]);
                        }
                    }
                    dL_dalpha *= T_;
                    last_alpha = alpha;
                    dL_dalpha += (-T_final / (1.f - alpha)) * bg_dot;
                    const float dL_dG = co[3] * dL_dalpha;
                    const float gdx = G * dx, gdy = G * dy;
                    const float dG_ddelx = -gdx * co[0] - gdy * co[1];
                    const float dG_ddely = -gdy * co[2] - gdx * co[1];
                    const float gmx = dL_dG * dG_ddelx * ddelx_dx;
                    const float gmy = dL_dG * dG_ddely * ddely_dy;
                    atomic_addf(&dL_dmean2D[3 * (size_t)id + 0], gmx);
                    atomic_addf(&dL_dmean2D[3 * (size_t)id + 1], gmy);
                    if (!full) {
                        atomic_addf(&dL_dmean2D_abs[3 * (size_t)id + 0], fabsf(gmx));
                        atomic_addf(&dL_dmean2D_abs[3 * (size_t)id + 1], fabsf(gmy));
                    } else if (co[3] * G > 0.99f) {
                        continue;
                    }
                    atomic_addf(&dL_dconic[4 * (size_t)id + 0], -0.5f * gdx * dx * dL_dG);
                    atomic_addf(&dL_dconic[4 * (size_t)id + 1], -0.5f * gdx * dy * dL_dG);
                    atomic_addf(&dL_dconic[4 * (size_t)id + 3], -0.5f * gdy * dy * dL_dG);
                    atomic_addf(&dL_dopacity[id], G * dL_dalpha);
                }
            }
    }
}

void o_render_bwd(int P, int W, int H, const float* bg,
                  const float* means2D, const float* conic_opacity, const float* rgb,
                  const uint8_t* compute_locally,
                  const uint32_t* ranges, const uint32_t* point_list,
                  const float* final_T, const uint32_t* n_contrib,
                  const float* dL_dpixels,
                  float* dL_dmean2D, float* dL_dmean2D_abs, float* dL_dconic,
                  float* dL_dopacity, float* dL_dcolors)
{
    (void)P;
    render_bwd_impl(0, W, H, bg, means2D, conic_opacity, rgb, compute_locally, ranges, point_list, final_T,
                    n_contrib, dL_dpixels, dL_dmean2D, dL_dmean2D_abs, dL_dconic, dL_dopacity, dL_dcolors, NULL);
}

void o_render_bwd_geo(int P, int W, int H, const float* bg,
                      const float* means2D, const float* conic_opacity, const float* rgb,
                      const uint8_t* compute_locally,
                      const uint32_t* ranges, const uint32_t* point_list,
                      const float* final_T, const uint32_t* n_contrib,
                      const float* dL_dpixels,
                      float* dL_dmean2D, float* dL_dmean2D_abs, float* dL_dconic,
                      float* dL_dopacity, float* dL_dcolors, const OGeoBwd* geo)
{
    (void)P;
    render_bwd_impl(0, W, H, bg, means2D, conic_opacity, rgb, compute_locally, ranges, point_list, final_T,
                    n_contrib, dL_dpixels, dL_dmean2D, dL_dmean2D_abs, dL_dconic, dL_dopacity, dL_dcolors, geo);
}

void o_render_bwd_full(int P, int W, int H, const float* bg,
                       const float* means2D, const float* conic_opacity, const float* colors,
                       const uint32_t* ranges, const uint32_t* point_list,
                       const float* final_T, const uint32_t* n_contrib,
                       const float* dL_dpixels,
                       float* dL_dmean2D, float* dL_dconic, float* dL_dopacity, float* dL_dcolors)
{
    (void)P;
    render_bwd_impl(1, W, H, bg, means2D, conic_opacity, colors, NULL, ranges, point_list, final_T, n_contrib,
                    dL_dpixels, dL_dmean2D, NULL, dL_dconic, dL_dopacity, dL_dcolors, NULL);
}

/* ---------------------------------------------------------------- full-image path
 * (_f/cuda_rasterizer/rasterizer_impl.cu:52-210,336-486, forward.cu:291-614) */

/* max_contrib_power_rect_gaussian_float<15,15> + the keep test of
 * duplicateWithKeys (rasterizer_impl.cu:56-95,144-167): the smallest value of
 * the falloff exponent 0.5 (a dx^2 + c dy^2) + b dx dy over the tile's pixel
 * rect [16x, 16x+15] x [16y, 16y+15] (evaluated at the closest point along the
 * rect edge nearest the mean), against log(opacity * 255).  Operations are
 * left to right, no contraction; 1/(225 a) is a correctly rounded division
 * (__frcp_rn); saturate maps NaN to 0. */
static inline float sat01(float v) { return v > 0.0f ? (v < 1.0f ? v : 1.0f) : 0.0f; }

int o_full_tile_keep(const float* xy, const float* co, unsigned tx, unsigned ty)
{
    const float rminx = (float)(tx * 16u), rminy = (float)(ty * 16u);
    const float rmaxx = (float)((tx + 1u) * 16u - 1u), rmaxy = (float)((ty + 1u) * 16u - 1u);
    const float mx = xy[0], my = xy[1];
    const float a = co[0], b = co[1], c = co[2], o = co[3];
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
        const float dx = copysignf(15.0f, x_min_diff);
        const float dy = copysignf(15.0f, y_min_diff);
        const float diffx = mx - px, diffy = my - py;
        const float rcp_x = 1.0f / (225.0f * a);
        const float rcp_y = 1.0f / (225.0f * c);
        const float tx_ = not_in_y * sat01((dx * a * diffx + dx * b * diffy) * rcp_x);
        const float ty_ = not_in_x * sat01((dy * b * diffx + dy * c * diffy) * rcp_y);
        const float qx = px + tx_ * dx, qy = py + ty_ * dy;
        const float ex = mx - qx, ey = my - qy;
        power = 0.5f * (a * ex * ex + c * ey * ey) + b * ex * ey;
    }
    const float thr = o_logf(o / (1.0f / 255.0f));
    return power <= thr;
}

/* Binning of the full-image path: every Gaussian with radius > 0 reserves
 * tiles_touched slots (the area of its float-extent rect, getRect(float2,
 * float2), auxiliary.h:63-73), fills them with the kept tiles in row-major
 * order and pads the rest with the invalid key (tile 0xFFFFFFFF, depth
 * FLT_MAX) and value 0xFFFFFFFF; stable sort; ranges of the valid tiles.
 * Returns the number of valid instances; *num_buckets = sum over tiles of
 * ceil(len / 32) (perTileBucketCount, rasterizer_impl.cu:244-253). */
int64_t o_binning_full(int P, int W, int H, const float* means2D, const float* depths, const int* radii,
                       const float* rects, const float* conic_opacity, const uint32_t* tiles_touched,
                       int64_t R, uint64_t* keys, uint32_t* values, uint32_t* ranges, int64_t* num_buckets)
{
    const unsigned gx = (unsigned)((W + OT - 1) / OT), gy = (unsigned)((H + OT - 1) / OT);
    const unsigned T = gx * gy;
    int64_t* off = (int64_t*)malloc(sizeof(int64_t) * (size_t)(P > 0 ? P : 1));
    int64_t acc = 0;
    for (int i = 0; i < P; i++) { off[i] = acc; acc += tiles_touched[i]; }
    const uint32_t flt_max_bits = 0x7f7fffffu;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < P; i++) {
        if (!(radii[i] > 0)) continue;
        int64_t o = off[i];
        const int64_t end = o + tiles_touched[i];
        const float* p = means2D + 2 * (size_t)i;
        const float* ex = rects + 2 * (size_t)i;
        int v;
        v = o_f2i_sat(floorf((p[0] - ex[0]) / 16.0f)); unsigned x0 = (unsigned)(v < 0 ? 0 : v); if (x0 > gx) x0 = gx;
        v = o_f2i_sat(floorf((p[1] - ex[1]) / 16.0f)); unsigned y0 = (unsigned)(v < 0 ? 0 : v); if (y0 > gy) y0 = gy;
        v = o_f2i_sat(ceilf((p[0] + ex[0]) / 16.0f));  unsigned x1 = (unsigned)(v < 0 ? 0 : v); if (x1 > gx) x1 = gx;
        v = o_f2i_sat(ceilf((p[1] + ex[1]) / 16.0f));  unsigned y1 = (unsigned)(v < 0 ? 0 : v); if (y1 > gy) y1 = gy;
        const uint32_t dbits = o_f2u(depths[i]);
        const float* co = conic_opacity + 4 * (size_t)i;
        for (unsigned y = y0; y < y1; y++)
            for (unsigned x = x0; x < x1; x++)
                if (o_full_tile_keep(p, co, x, y)) {
                    keys[o] = ((uint64_t)(y * gx + x) << 32) | dbits;
                    values[o] = (uint32_t)i;
                    o++;
                }
        for (; o < end; o++) {
            keys[o] = ((uint64_t)0xffffffffu << 32) | flt_max_bits;
            values[o] = 0xffffffffu;
        }
    }
    free(off);
    if (R > 1) {
        uint64_t* tk = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)R);
        uint32_t* tv = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)R);
        uint64_t* a = keys; uint32_t* av = values;
        uint64_t* b = tk; uint32_t* bv = tv;
        for (int64_t width = 1; width < R; width *= 2) {
#pragma omp parallel for schedule(dynamic, 1)
            for (int64_t lo = 0; lo < R; lo += 2 * width) {
                int64_t mid = lo + width < R ? lo + width : R;
                int64_t hi = lo + 2 * width < R ? lo + 2 * width : R;
                int64_t i = lo, j = mid, o = lo;
                while (i < mid && j < hi) {
                    if (a[j] < a[i]) { b[o] = a[j]; bv[o] = av[j]; j++; }
                    else { b[o] = a[i]; bv[o] = av[i]; i++; }
                    o++;
                }
                while (i < mid) { b[o] = a[i]; bv[o] = av[i]; i++; o++; }
                while (j < hi) { b[o] = a[j]; bv[o] = av[j]; j++; o++; }
            }
            uint64_t* sw = a; a = b; b = sw;
            uint32_t* sv = av; av = bv; bv = sv;
        }
        if (a != keys) {
            memcpy(keys, a, sizeof(uint64_t) * (size_t)R);
            memcpy(values, av, sizeof(uint32_t) * (size_t)R);
        }
        free(tk); free(tv);
    }
    /* identifyTileRanges with the invalid tile skipped (rasterizer_impl.cu:194-219) */
    memset(ranges, 0, sizeof(uint32_t) * 2 * (size_t)T);
    int64_t valid = 0;
    for (int64_t idx = 0; idx < R; idx++) {
        const uint32_t cur = (uint32_t)(keys[idx] >> 32);
        const int ok = cur != 0xffffffffu;
        if (ok) valid++;
        if (idx == 0) { if (ok) ranges[2 * cur] = 0; }
        else {
            const uint32_t prev = (uint32_t)(keys[idx - 1] >> 32);
            if (cur != prev) {
                if (prev != 0xffffffffu) ranges[2 * prev + 1] = (uint32_t)idx;
                if (ok) ranges[2 * cur] = (uint32_t)idx;
            }
        }
        if (idx == R - 1 && ok) ranges[2 * cur + 1] = (uint32_t)R;
    }
    int64_t nb = 0;
    for (unsigned t = 0; t < T; t++) nb += (ranges[2 * t + 1] - ranges[2 * t] + 31) / 32;
    *num_buckets = nb;
    return valid;
}

/* renderCUDA / render_simpCUDA of the full-image path (forward.cu:291-465,
 * 466-607): the blend of the split path plus, per pixel, the Gaussian of the
 * largest blend weight alpha * T (first one on ties), which gets one count in
 * accum_max_count (when flag_max_count; render_simp always), and for
 * render_simp every contribution's alpha * T added to accum_weights and 1 to
 * accum_weights_count.  max_contrib[t] = the tile's largest last contributor.
 * The accumulations run in tile, row, column, list order. */
void o_render_fwd_full(int P, int W, int H, const float* bg, const float* means2D, const float* conic_opacity,
                       const float* colors, const uint32_t* ranges, const uint32_t* point_list, int flag_max_count,
                       float* out_color, float* final_T, uint32_t* n_contrib, uint32_t* max_contrib,
                       float* accum_max_count, float* accum_weights, int32_t* accum_weights_count)
{
    (void)P;
    const int gx = (W + OT - 1) / OT, gy = (H + OT - 1) / OT;
    const int T = gx * gy;
    const float alpha_min = 1.0f / 255.0f;
    for (int t = 0; t < T; t++) {
        const int tx = t % gx, ty = t / gx;
        const int x0 = tx * OT, y0 = ty * OT;
        const int x1 = x0 + OT < W ? x0 + OT : W, y1 = y0 + OT < H ? y0 + OT : H;
        const uint32_t rs = ranges[2 * t], re = ranges[2 * t + 1];
        uint32_t mc = 0;
        for (int y = y0; y < y1; y++)
            for (int x = x0; x < x1; x++) {
                const float px = (float)x, py = (float)y;
                float T_ = 1.0f, C[3] = { 0.f, 0.f, 0.f };
                uint32_t contributor = 0, last = 0;
                float wmax = 0.0f;
                uint32_t imax = 0;
                int upd = 0;
                for (uint32_t k = rs; k < re; k++) {
                    contributor++;
                    const uint32_t id = point_list[k];
                    const float* co = conic_opacity + 4 * (size_t)id;
                    const float power = o_power(means2D + 2 * (size_t)id, co, px, py);
                    if (power > 0.0f) continue;
                    const float alpha = o_fminf(0.99f, co[3] * o_expf(power));
                    if (alpha < alpha_min) continue;
                    const float test_T = T_ * (1.0f - alpha);
                    if (test_T < 0.0001f) break;
                    const float wgt = alpha * T_;
                    for (int c = 0; c < 3; c++) C[c] = fmaf(colors[3 * (size_t)id + c], wgt, C[c]);
                    if (wmax < wgt) { wmax = wgt; imax = id; upd = 1; }
                    if (accum_weights) {
                        accum_weights[id] += wgt;
                        accum_weights_count[id] += 1;
                    }
                    T_ = test_T;
                    last = contributor;
                }
                if (upd && (flag_max_count || accum_weights)) accum_max_count[imax] += 1.0f;
                const size_t pid = (size_t)y * W + x;
                final_T[pid] = T_;
                n_contrib[pid] = last;
                for (int c = 0; c < 3; c++) out_color[(size_t)c * H * W + pid] = fmaf(T_, bg[c], C[c]);
                if (last > mc) mc = last;
            }
        if (max_contrib) max_contrib[t] = mc;
    }
}

/* Inverse of the 4x4 matrix whose element (r, c) is m[4c + r] (the layout
 * glm::make_mat4x4 reads), by the expansion in complementary 2x2 minors, in
 * double, rounded to float in the same layout.  Stands for glm::inverse in
 * _f/cuda_rasterizer/forward.cu:686-688 (which inverts in float). */
void o_inv4_colmajor(const float* mf, float* out)
{
    double a[4][4], b[4][4];
    for (int c = 0; c < 4; c++)
        for (int r = 0; r < 4; r++) a[r][c] = (double)mf[4 * c + r];
    const double s0 = a[0][0] * a[1][1] - a[1][0] * a[0][1];
    const double s1 = a[0][0] * a[1][2] - a[1][0] * a[0][2];
    const double s2 = a[0][0] * a[1][3] - a[1][0] * a[0][3];
    const double s3 = a[0][1] * a[1][2] - a[1][1] * a[0][2];
    const double s4 = a[0][1] * a[1][3] - a[1][1] * a[0][3];
    const double s5 = a[0][2] * a[1][3] - a[1][2] * a[0][3];
    const double c5 = a[2][2] * a[3][3] - a[3][2] * a[2][3];
    const double c4 = a[2][1] * a[3][3] - a[3][1] * a[2][3];
    const double c3 = a[2][1] * a[3][2] - a[3][1] * a[2][2];
    const double c2 = a[2][0] * a[3][3] - a[3][0] * a[2][3];
    const double c1 = a[2][0] * a[3][2] - a[3][0] * a[2][2];
    const double c0 = a[2][0] * a[3][1] - a[3][0] * a[2][1];
    const double det = s0 * c5 - s1 * c4 + s2 * c3 + s3 * c2 - s4 * c1 + s5 * c0;
    const double id = 1.0 / det;
    b[0][0] = (a[1][1] * c5 - a[1][2] * c4 + a[1][3] * c3) * id;
    b[0][1] = (-a[0][1] * c5 + a[0][2] * c4 - a[0][3] * c3) * id;
    b[0][2] = (a[3][1] * s5 - a[3][2] * s4 + a[3][3] * s3) * id;
    b[0][3] = (-a[2][1] * s5 + a[2][2] * s4 - a[2][3] * s3) * id;
    b[1][0] = (-a[1][0] * c5 + a[1][2] * c2 - a[1][3] * c1) * id;
    b[1][1] = (a[0][0] * c5 - a[0][2] * c2 + a[0][3] * c1) * id;
    b[1][2] = (-a[3][0] * s5 + a[3][2] * s2 - a[3][3] * s1) * id;
    b[1][3] = (a[2][0] * s5 - a[2][2] * s2 + a[2][3] * s1) * id;
    b[2][0] = (a[1][0] * c4 - a[1][1] * c2 + a[1][3] * c0) * id;
    b[2][1] = (-a[0][0] * c4 + a[0][1] * c2 - a[0][3] * c0) * id;
    b[2][2] = (a[3][0] * s4 - a[3][1] * s2 + a[3][3] * s0) * id;
    b[2][3] = (-a[2][0] * s4 + a[2][1] * s2 - a[2][3] * s0) * id;
    b[3][0] = (-a[1][0] * c3 + a[1][1] * c1 - a[1][2] * c0) * id;
    b[3][1] = (a[0][0] * c3 - a[0][1] * c1 + a[0][2] * c0) * id;
    b[3][2] = (-a[3][0] * s3 + a[3][1] * s1 - a[3][2] * s0) * id;
    b[3][3] = (a[2][0] * s3 - a[2][1] * s1 + a[2][2] * s0) * id;
    for (int c = 0; c < 4; c++)
        for (int r = 0; r < 4; r++) out[4 * c + r] = (float)b[r][c];
}

/* render_depthCUDA (_f/cuda_rasterizer/forward.cu:616-835): the full-image
 * blend of the tile-culled list plus, per pixel, the camera ray's
 * intersection with every blended Gaussian's 3-sigma ellipsoid.
 *   ray: Pix2ndc (auxiliary.h:46-49), x / y times 1.0000001 in double, z =
 *        (100 - 100*0.01) / (100 - 0.01); inv(projmatrix) applied as
 *        transformPoint4x4 (no division by w); direction = that point - campos,
 *        normalised as glm::normalize (v * (1 / sqrt(dot))) (:686-719)
 *   per Gaussian: glm::mat3 of the unnormalised quaternion (columns m0..m2,
 *        m3..m5, m6..m8); ray origin and direction in its frame; s = 3 scale;
 *        a, b, c of the quadric, discriminant b*b - 4*a*c, t = -b/2/a,
 *        depth = t / |direction| (:764-801)
 *   rules: colour is added before the depth test; depth < 0 skips the rest
 *        (T unchanged); the largest alpha * T picks depth, discriminant, id
 *        and hit point campos + t * direction; n_contrib stays 0 (:767-823).
 * Operation order: plain float operations left to right, except the colour
 * sum fmaf(f * alpha, T, C) and the final colour fmaf(T, bg, C). */
void o_render_depth_full(int W, int H, const float* bg, const float* means2D, const float* conic_opacity,
                         const float* colors, const uint32_t* ranges, const uint32_t* point_list,
                         const float* means3D, const float* scales, const float* rotations, const float* projmatrix,
                         const float* campos, float* out_color, float* out_pts, float* out_depth, float* accum_alpha,
                         int32_t* gidx, float* discriminants)
{
    const int gx = (W + OT - 1) / OT, gy = (H + OT - 1) / OT;
    const int T = gx * gy;
    const float alpha_min = 1.0f / 255.0f;
    const size_t HW = (size_t)H * W;
    float inv[16];
    o_inv4_colmajor(projmatrix, inv);
    const float cx = campos[0], cy = campos[1], cz = campos[2];
    const float hz = (float)((100.0 - 100.0 * 0.01) / (100.0 - 0.01));
#pragma omp parallel for schedule(dynamic, 4)
    for (int t = 0; t < T; t++) {
        const int tx = t % gx, ty = t / gx;
        const int x0 = tx * OT, y0 = ty * OT;
        const int x1 = x0 + OT < W ? x0 + OT : W, y1 = y0 + OT < H ? y0 + OT : H;
        const uint32_t rs = ranges[2 * t], re = ranges[2 * t + 1];
        for (int y = y0; y < y1; y++)
            for (int x = x0; x < x1; x++) {
                const float px = (float)x, py = (float)y;
                const float ndx = (2.0f * px + 1.0f) / (float)W - 1.0f;
                const float ndy = (2.0f * py + 1.0f) / (float)H - 1.0f;
                const float hx = (float)((double)ndx * 1.0000001), hy = (float)((double)ndy * 1.0000001);
                const float ox = inv[0] * hx + inv[4] * hy + inv[8] * hz + inv[12];
                const float oy = inv[1] * hx + inv[5] * hy + inv[9] * hz + inv[13];
                const float oz = inv[2] * hx + inv[6] * hy + inv[10] * hz + inv[14];
                const float rdx = ox - cx, rdy = oy - cy, rdz = oz - cz;
                const float len = sqrtf(rdx * rdx + rdy * rdy + rdz * rdz);
                const float il = 1.0f / len;
                const float nx = rdx * il, ny = rdy * il, nz = rdz * il;
                float T_ = 1.0f, C[3] = { 0.f, 0.f, 0.f };
                float wmax = 0.f, dmax = 0.f, discmax = 0.f, pr[3] = { 0.f, 0.f, 0.f };
                int32_t imax = 0;
                for (uint32_t k = rs; k < re; k++) {
                    const uint32_t id = point_list[k];
                    const float* co = conic_opacity + 4 * (size_t)id;
                    const float power = o_power(means2D + 2 * (size_t)id, co, px, py);
                    if (power > 0.0f) continue;
                    const float alpha = o_fminf(0.99f, co[3] * o_expf(power));
                    if (alpha < alpha_min) continue;
                    const float test_T = T_ * (1.0f - alpha);
                    if (test_T < 0.0001f) break;
                    for (int c = 0; c < 3; c++) C[c] = fmaf(colors[3 * (size_t)id + c] * alpha, T_, C[c]);
                    const float* q = rotations + 4 * (size_t)id;
                    const float qr = q[0], qx = q[1], qy = q[2], qz = q[3];
                    const float m0 = 1.f - 2.f * (qy * qy + qz * qz), m1 = 2.f * (qx * qy - qr * qz);
                    const float m2 = 2.f * (qx * qz + qr * qy), m3 = 2.f * (qx * qy + qr * qz);
                    const float m4 = 1.f - 2.f * (qx * qx + qz * qz), m5 = 2.f * (qy * qz - qr * qx);
                    const float m6 = 2.f * (qx * qz - qr * qy), m7 = 2.f * (qy * qz + qr * qx);
                    const float m8 = 1.f - 2.f * (qx * qx + qy * qy);
                    const float* mu = means3D + 3 * (size_t)id;
                    const float ex = cx - mu[0], ey = cy - mu[1], ez = cz - mu[2];
                    const float rox = m0 * ex + m3 * ey + m6 * ez;
                    const float roy = m1 * ex + m4 * ey + m7 * ez;
                    const float roz = m2 * ex + m5 * ey + m8 * ez;
                    const float rdx2 = m0 * nx + m3 * ny + m6 * nz;
                    const float rdy2 = m1 * nx + m4 * ny + m7 * nz;
                    const float rdz2 = m2 * nx + m5 * ny + m8 * nz;
                    const float* sc = scales + 3 * (size_t)id;
                    const float sx = sc[0] * 3.0f, sy = sc[1] * 3.0f, sz = sc[2] * 3.0f;
                    const float a = rdx2 / sx * rdx2 / sx + rdy2 / sy * rdy2 / sy + rdz2 / sz * rdz2 / sz;
                    const float b = 2.0f * (rdx2 / sx * rox / sx + rdy2 / sy * roy / sy + rdz2 / sz * roz / sz);
                    const float cc = rox / sx * rox / sx + roy / sy * roy / sy + roz / sz * roz / sz - 1.0f;
                    const float disc = b * b - 4.0f * a * cc;
                    const float tpar = -b / 2.0f / a;
                    const float depth = tpar / len;
                    if (depth < 0.0f) continue;
                    const float wgt = alpha * T_;
                    if (wmax < wgt) {
                        wmax = wgt;
                        dmax = depth;
                        discmax = disc;
                        imax = (int32_t)id;
                        pr[0] = cx + tpar * nx;
                        pr[1] = cy + tpar * ny;
                        pr[2] = cz + tpar * nz;
                    }
                    T_ = test_T;
                }
                const size_t pid = (size_t)y * W + x;
                for (int c = 0; c < 3; c++) {
                    out_color[(size_t)c * HW + pid] = fmaf(T_, bg[c], C[c]);
                    out_pts[(size_t)c * HW + pid] = pr[c];
                }
                out_depth[pid] = dmax;
                accum_alpha[pid] = T_;
                discriminants[pid] = discmax;
                gidx[pid] = imax;
            }
    }
}

void o_vec_expf(int n, const float* x, float* y)
{
    for (int i = 0; i < n; i++) y[i] = o_expf(x[i]);
}
void o_vec_logf(int n, const float* x, float* y)
{
    for (int i = 0; i < n; i++) y[i] = o_logf(x[i]);
}

#ifdef _OPENMP
#include <omp.h>
int o_num_threads(void) { return omp_get_max_threads(); }
#else
int o_num_threads(void) { return 1; }
#endif
