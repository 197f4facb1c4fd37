/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, never linked into the product.
 *
 * Restatement of the reference's Gaussian -> rank routing of the
 * image-distributed step (/root/reference/submodule/diff-gaussian-rasterization_f):
 *   getTouchedIdsBool             rasterize_points.cu:212-256
 *   GetLocal2jIdsBoolCUDA         rasterize_points.cu:258-289
 *   getTouchedIdsBoolAdjustMode6  rasterize_points.cu:291-335
 *   GetLocal2jIdsBoolAdjustMode6CUDA rasterize_points.cu:337-367
 *   getRect(float2, int)          cuda_rasterizer/auxiliary.h:51-61
 * Both write a (P, world) bool matrix: row i says which ranks' tile ranges a
 * Gaussian's screen rectangle reaches.  Neither looks at whether the Gaussian
 * was culled (radius 0): the rectangle alone decides, as in the reference.
 *
 * Integer semantics follow the reference's types exactly: the rectangle is
 * unsigned, the linear tile indices are computed in 32-bit unsigned
 * arithmetic and then read as signed int (so an empty rectangle at the image
 * origin gives a negative maximum index), the rank bounds are signed int, and
 * the rectangle test of mode 6 compares unsigned against int, which C
 * promotes to unsigned.
 */
#include "gs_oracle.h"
#include "o_math.h"

#define OT 16  /* BLOCK_X = BLOCK_Y = 16 (config.h) */

static inline unsigned clamp_tile(int v, unsigned g)
{
    v = v < 0 ? 0 : v;
    return (unsigned)v > g ? g : (unsigned)v;
}

/* getRect(float2, int): float arithmetic left to right, (int) truncation,
 * clamped to [0, grid] (auxiliary.h:51-61). */
static inline void rect(const float* p, int r, unsigned gx, unsigned gy,
                        unsigned* x0, unsigned* y0, unsigned* x1, unsigned* y1)
{
    const float rf = (float)r;
    *x0 = clamp_tile(o_f2i_sat((p[0] - rf) / 16.0f), gx);
    *y0 = clamp_tile(o_f2i_sat((p[1] - rf) / 16.0f), gy);
    *x1 = clamp_tile(o_f2i_sat(((p[0] + rf) + 16.0f - 1.0f) / 16.0f), gx);
    *y1 = clamp_tile(o_f2i_sat(((p[1] + rf) + 16.0f - 1.0f) / 16.0f), gy);
}

void o_local2j_ids_bool(int P, int H, int W, int world, const float* means2D, const int* radii,
                        const int* strategy, int avoid, uint8_t* out)
{
    const unsigned gx = (unsigned)((W + OT - 1) / OT), gy = (unsigned)((H + OT - 1) / OT);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < P; i++) {
        uint8_t* row = out + (size_t)i * (size_t)world;
        for (int rk = 0; rk < world; rk++) row[rk] = 0;
        unsigned x0, y0, x1, y1;
        rect(means2D + 2 * (size_t)i, radii[i], gx, gy, &x0, &y0, &x1, &y1);
        const int lo = (int)(y0 * gx + x0);
        const int hi = (int)((y1 - 1u) * gx + x1 - 1u);
        if (hi < lo) continue;
        for (int rk = 0; rk < world; rk++) {
            int tl = strategy[rk], tr = strategy[rk + 1];
            if (avoid) {
                tl = (int)((unsigned)tl - (gx + 1u));
                tr = (int)((unsigned)tr + (gx + 1u));
            }
            if (hi < tl || lo >= tr) continue;
            row[rk] = 1;
        }
    }
}

void o_local2j_ids_bool_rect(int P, int H, int W, int world, const float* means2D, const int* radii,
                             const int* rectangles, int avoid, uint8_t* out)
{
    const unsigned gx = (unsigned)((W + OT - 1) / OT), gy = (unsigned)((H + OT - 1) / OT);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < P; i++) {
        uint8_t* row = out + (size_t)i * (size_t)world;
        unsigned x0, y0, x1, y1;
        rect(means2D + 2 * (size_t)i, radii[i], gx, gy, &x0, &y0, &x1, &y1);
        for (int rk = 0; rk < world; rk++) {
            int yl = rectangles[4 * rk + 0], yr = rectangles[4 * rk + 1];
            int xl = rectangles[4 * rk + 2], xr = rectangles[4 * rk + 3];
            if (avoid) {
                if (yl > 0) yl -= 1;
                if (xl > 0) xl -= 1;
                yr += 1;
                xr += 1;
            }
            /* unsigned versus int: the int side converts to unsigned */
            row[rk] = !(y1 <= (unsigned)yl || (unsigned)yr <= y0 || x1 <= (unsigned)xl || (unsigned)xr <= x0);
        }
    }
}
