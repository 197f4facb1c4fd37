/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, never linked into the product.
 *
 * Sparse Adam step (/root/reference/submodule/diff-gaussian-rasterization_f/
 * cuda_rasterizer/adam.cu:9-38, bound at rasterize_points.cu:807-832, driven by
 * SparseGaussianAdam.step in diff_gaussian_rasterization_f/__init__.py:832-863):
 * for every element p of a (N, M) parameter whose Gaussian p / M is visible,
 *   m = b1 * m + (1 - b1) * g
 *   v = b2 * v + ((1 - b2) * g) * g
 *   param += ((-lr) * m) / (sqrt(v) + eps)
 * in fp32, left to right, no fused multiply-add, IEEE sqrt and division.
 * Elements of invisible Gaussians are not touched.
 */
#include "gs_oracle.h"
#include <math.h>

void o_adam_update(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, const uint8_t* visible,
                   float lr, float b1, float b2, float eps, int64_t N, int64_t M)
{
    const int64_t cnt = N * M;
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < cnt; p++) {
        if (!visible[p / M]) continue;
        const float g = grad[p];
        const float m = b1 * exp_avg[p] + (1.0f - b1) * g;
        const float v = b2 * exp_avg_sq[p] + ((1.0f - b2) * g) * g;
        const float step = ((-lr) * m) / (sqrtf(v) + eps);
        param[p] += step;
        exp_avg[p] = m;
        exp_avg_sq[p] = v;
    }
}
