// fused-ssim forward / backward for gfx950.
//
// Reference: BlitzGS submodule/fused-ssim/ssim.cu:8-441 (fusedssimCUDA,
// fusedssim_backwardCUDA, host wrappers) and fused_ssim/__init__.py:8-41.
// The 11x11 Gaussian window (sigma 1.5) is separable; images are zero padded
// ("same" output size).
//
// Design: one block per 32x32 output tile of one (batch, channel) plane (the
// reference runs the channels sequentially inside the block).  The block
// stages the zero-padded 42x42 input tiles in LDS, runs the horizontal pass for
// all 42 rows of the five (forward) or three (backward) quantities at once,
// keeps those rows in LDS, and runs the vertical pass per output pixel.  Every
// sum is accumulated tap by tap from -5 to +5 with separate multiplies and
// adds (the library is built with -ffp-contract=off), the same order as the
// CPU oracle, so the results are reproducible bit for bit on the CPU.
#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {

constexpr int TX = 32, TY = 32, HALO = 5;
constexpr int SX = TX + 2 * HALO, SY = TY + 2 * HALO;   // 42 x 42 staged input
constexpr int SXP = SX + 1;                              // LDS row pitch
constexpr int NT = 256;

// reference float values of the normalised window (ssim.cu:8-18)
__device__ __forceinline__ float gwin(int t)
{
    const uint32_t h[6] = {0x3a86cab6u, 0x3bf8ff01u, 0x3d13758cu, 0x3ddff87fu, 0x3e5a1e1fu, 0x3e8832b0u};
    return __uint_as_float(h[t < 6 ? t : 10 - t]);
}

__device__ __forceinline__ void stage(float (*dst)[SXP], const float* __restrict__ plane, int H, int W, int x0,
                                      int y0)
{
    for (int i = threadIdx.x; i < SX * SY; i += NT) {
        const int ly = i / SX, lx = i - ly * SX;
        const int y = y0 + ly - HALO, x = x0 + lx - HALO;
        dst[ly][lx] = (y >= 0 && y < H && x >= 0 && x < W) ? plane[(size_t)y * W + x] : 0.0f;
    }
}

__global__ __launch_bounds__(NT) void ssim_fwd_kernel(int H, int W, float C1, float C2,
                                                      const float* __restrict__ img1, const float* __restrict__ img2,
                                                      float* __restrict__ ssim_map, float* __restrict__ dm_dmu1,
                                                      float* __restrict__ dm_dsigma1_sq, float* __restrict__ dm_dsigma12)
{
    __shared__ float s1[SY][SXP];
    __shared__ float s2[SY][SXP];
    __shared__ float hz[5][SY][TX];
    const int x0 = blockIdx.x * TX, y0 = blockIdx.y * TY;
    const size_t plane = (size_t)blockIdx.z * H * W;
    stage(s1, img1 + plane, H, W, x0, y0);
    stage(s2, img2 + plane, H, W, x0, y0);
    __syncthreads();
    // horizontal pass: rows 0..41 (image rows y0-5 .. y0+36), columns 0..31
    for (int i = threadIdx.x; i < SY * TX; i += NT) {
        const int r = i / TX, c = i - r * TX;
        float a = 0.f, b = 0.f, aa = 0.f, bb = 0.f, ab = 0.f;
#pragma unroll
        for (int t = 0; t < 11; t++) {
            const float g = gwin(t);
            const float p = s1[r][c + t], q = s2[r][c + t];
            a += g * p;
            b += g * q;
            aa += g * (p * p);
            bb += g * (q * q);
            ab += g * (p * q);
        }
        hz[0][r][c] = a; hz[1][r][c] = b; hz[2][r][c] = aa; hz[3][r][c] = bb; hz[4][r][c] = ab;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < TY * TX; i += NT) {
        const int r = i / TX, c = i - r * TX;
        const int y = y0 + r, x = x0 + c;
        if (y >= H || x >= W) continue;
        float v[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 11; t++) {
            const float g = gwin(t);
#pragma unroll
            for (int k = 0; k < 5; k++) v[k] += g * hz[k][r + t][c];
        }
        const float m1 = v[0], m2 = v[1];
        const float sigma1_sq = v[2] - m1 * m1;
        const float sigma2_sq = v[3] - m2 * m2;
        const float sigma12 = v[4] - m1 * m2;
        const float mu1_sq = m1 * m1, mu2_sq = m2 * m2, mu1_mu2 = m1 * m2;
        const float Cn = (2.0f * mu1_mu2 + C1);
        const float Dn = (2.0f * sigma12 + C2);
        const float A = (mu1_sq + mu2_sq + C1);
        const float Bd = (sigma1_sq + sigma2_sq + C2);
        const size_t o = plane + (size_t)y * W + x;
        ssim_map[o] = (Cn * Dn) / (A * Bd);
        if (dm_dmu1) {
            dm_dmu1[o] = ((m2 * 2.0f * Dn) / (A * Bd) - (m2 * 2.0f * Cn) / (A * Bd) -
                          (m1 * 2.0f * Cn * Dn) / (A * A * Bd) + (m1 * 2.0f * Cn * Dn) / (A * Bd * Bd));
            dm_dsigma1_sq[o] = ((-Cn * Dn) / (A * Bd * Bd));
            dm_dsigma12[o] = ((2 * Cn) / (A * Bd));
        }
    }
}

// stage the product dm * dL_dmap (zero padded)
__device__ __forceinline__ void stage_prod(float (*dst)[SXP], const float* __restrict__ a, const float* __restrict__ b,
                                           int H, int W, int x0, int y0)
{
    for (int i = threadIdx.x; i < SX * SY; i += NT) {
        const int ly = i / SX, lx = i - ly * SX;
        const int y = y0 + ly - HALO, x = x0 + lx - HALO;
        float v = 0.0f;
        if (y >= 0 && y < H && x >= 0 && x < W) {
            const size_t o = (size_t)y * W + x;
            v = a[o] * b[o];
        }
        dst[ly][lx] = v;
    }
}

__global__ __launch_bounds__(NT) void ssim_bwd_kernel(int H, int W, const float* __restrict__ img1,
                                                      const float* __restrict__ img2, const float* __restrict__ dL_dmap,
                                                      const float* __restrict__ dm_dmu1,
                                                      const float* __restrict__ dm_dsigma1_sq,
                                                      const float* __restrict__ dm_dsigma12, float* __restrict__ dL_dimg1)
{
    __shared__ float sp[3][SY][SXP];
    __shared__ float hz[3][SY][TX];
    const int x0 = blockIdx.x * TX, y0 = blockIdx.y * TY;
    const size_t plane = (size_t)blockIdx.z * H * W;
    stage_prod(sp[0], dm_dmu1 + plane, dL_dmap + plane, H, W, x0, y0);
    stage_prod(sp[1], dm_dsigma1_sq + plane, dL_dmap + plane, H, W, x0, y0);
    stage_prod(sp[2], dm_dsigma12 + plane, dL_dmap + plane, H, W, x0, y0);
    __syncthreads();
    for (int i = threadIdx.x; i < SY * TX; i += NT) {
        const int r = i / TX, c = i - r * TX;
        float v[3] = {0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 11; t++) {
            const float g = gwin(t);
#pragma unroll
            for (int k = 0; k < 3; k++) v[k] += g * sp[k][r][c + t];
        }
        hz[0][r][c] = v[0]; hz[1][r][c] = v[1]; hz[2][r][c] = v[2];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < TY * TX; i += NT) {
        const int r = i / TX, c = i - r * TX;
        const int y = y0 + r, x = x0 + c;
        if (y >= H || x >= W) continue;
        float v[3] = {0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 11; t++) {
            const float g = gwin(t);
#pragma unroll
            for (int k = 0; k < 3; k++) v[k] += g * hz[k][r + t][c];
        }
        const size_t o = plane + (size_t)y * W + x;
        float d = 0.0f;
        d += v[0];
        d += img1[o] * 2.0f * v[1];
        d += img2[o] * v[2];
        dL_dimg1[o] = d;
    }
}

}  // namespace

extern "C" int gs_ssim_forward(int B, int C, int H, int W, float C1, float C2, const float* img1, const float* img2,
                               float* ssim_map, float* dm_dmu1, float* dm_dsigma1_sq, float* dm_dsigma12,
                               hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(B >= 0 && C >= 0 && H >= 0 && W >= 0, "invalid image shape (%d,%d,%d,%d)", B, C, H, W);
    GS_REQUIRE((dm_dmu1 == nullptr) == (dm_dsigma1_sq == nullptr) && (dm_dmu1 == nullptr) == (dm_dsigma12 == nullptr),
               "the three dm_* outputs must be all given or all null");
    GS_REQUIRE((size_t)B * C <= 65535u, "B*C must be <= 65535");
    if ((size_t)B * C * H * W == 0) return GS_OK;
    const dim3 grid(gs_div_up(W, TX), gs_div_up(H, TY), B * C);
    GS_TIMED("ssim_fwd_kernel", stream,
             hipLaunchKernelGGL(ssim_fwd_kernel, grid, dim3(NT), 0, stream, H, W, C1, C2, img1, img2, ssim_map,
                                dm_dmu1, dm_dsigma1_sq, dm_dsigma12));
    GS_LAUNCH_CHECK("ssim_fwd_kernel");
    return GS_OK;
}

extern "C" int gs_ssim_backward(int B, int C, int H, int W, float C1, float C2, const float* img1, const float* img2,
                                const float* dL_dmap, const float* dm_dmu1, const float* dm_dsigma1_sq,
                                const float* dm_dsigma12, float* dL_dimg1, hipStream_t stream)
{
    gs::clear_error();
    (void)C1; (void)C2;
    GS_REQUIRE(B >= 0 && C >= 0 && H >= 0 && W >= 0, "invalid image shape (%d,%d,%d,%d)", B, C, H, W);
    GS_REQUIRE((size_t)B * C <= 65535u, "B*C must be <= 65535");
    if ((size_t)B * C * H * W == 0) return GS_OK;
    GS_REQUIRE(dm_dmu1 && dm_dsigma1_sq && dm_dsigma12, "the backward needs the forward's dm_* partials (train=True)");
    const dim3 grid(gs_div_up(W, TX), gs_div_up(H, TY), B * C);
    GS_TIMED("ssim_bwd_kernel", stream,
             hipLaunchKernelGGL(ssim_bwd_kernel, grid, dim3(NT), 0, stream, H, W, img1, img2, dL_dmap, dm_dmu1,
                                dm_dsigma1_sq, dm_dsigma12, dL_dimg1));
    GS_LAUNCH_CHECK("ssim_bwd_kernel");
    return GS_OK;
}
