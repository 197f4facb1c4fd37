// fused-ssim forward / backward for gfx950.
//
// Reference: BlitzGS submodule/fused-ssim/ssim.cu:8-441 (fusedssimCUDA,
// fusedssim_backwardCUDA, host wrappers) and fused_ssim/__init__.py:8-41.
// The 11x11 Gaussian window (sigma 1.5) is separable; images are zero padded
// ("same" output size).
//
// Design: the sliding-window form described at the kernels (one thread per
// column of a strip, horizontal sums staged row by row through LDS, the last
// 11 rows of sums in registers).  Every sum is accumulated tap by tap from -5
// to +5 with one fused multiply-add per tap (explicit fmaf; the library is
// built with -ffp-contract=off), the same operations in the same order as the
// CPU oracle, so the results are reproducible bit for bit on the CPU.
#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {

constexpr int HALO = 5;

// reference float values of the normalised window (ssim.cu:8-18)
__device__ __forceinline__ float gwin(int t)
{
    const uint32_t h[6] = {0x3a86cab6u, 0x3bf8ff01u, 0x3d13758cu, 0x3ddff87fu, 0x3e5a1e1fu, 0x3e8832b0u};
    return __uint_as_float(h[t < 6 ? t : 10 - t]);
}

// Sliding-window form: a block owns a strip of SW columns (one per thread)
// and SHR output rows.  It walks the strip's input rows top to bottom: each
// step stages one zero-padded input row (SW + 10 values per quantity) in LDS,
// every thread computes its column's horizontal 11-tap sums for that row, and
// keeps the last 11 rows of sums in registers (a ring whose slot is static
// because the row loop is unrolled by 11); once a row's 11-row window is
// complete the vertical sums and the output follow.  Input rows are read once
// per strip (halo 10 / SHR rows and 10 / SW columns), the next row's loads are
// in flight while the current row is processed.  Every sum is accumulated tap
// by tap from -5 to +5 with one fmaf per tap, as the CPU oracle does.
constexpr int SW = 256;       // strip width: threads per block
constexpr int SHR = 64;       // output rows per strip
constexpr int RW = SW + 2 * HALO;

template <int Q>
struct Rows {
    float v[Q][2];            // this thread's staged values: column tid and (tid < 2 HALO) column tid + SW
};

// one input row of the strip for the forward: the two images (zero outside the image)
__device__ __forceinline__ void load_row_fwd(Rows<2>& r, const float* __restrict__ a, const float* __restrict__ b,
                                             int H, int W, int y, int xs)
{
    const int t = threadIdx.x;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int lx = t + h * SW;
        const int x = xs + lx;
        const bool ok = (h == 0 || t < 2 * HALO) && y >= 0 && y < H && x >= 0 && x < W;
        r.v[0][h] = ok ? a[(size_t)y * W + x] : 0.f;
        r.v[1][h] = ok ? b[(size_t)y * W + x] : 0.f;
    }
}

// one input row for the backward: the three products dm_* x dL_dmap
__device__ __forceinline__ void load_row_bwd(Rows<3>& r, const float* __restrict__ d0, const float* __restrict__ d1,
                                             const float* __restrict__ d2, const float* __restrict__ dl, int H, int W,
                                             int y, int xs)
{
    const int t = threadIdx.x;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int lx = t + h * SW;
        const int x = xs + lx;
        const bool ok = (h == 0 || t < 2 * HALO) && y >= 0 && y < H && x >= 0 && x < W;
        float g = 0.f, p0 = 0.f, p1 = 0.f, p2 = 0.f;
        if (ok) {
            const size_t o = (size_t)y * W + x;
            g = dl[o];
            p0 = d0[o];
            p1 = d1[o];
            p2 = d2[o];
        }
        r.v[0][h] = p0 * g;
        r.v[1][h] = p1 * g;
        r.v[2][h] = p2 * g;
    }
}

template <int Q>
__device__ __forceinline__ void put_row(float (*buf)[RW], const Rows<Q>& r)
{
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        buf[q][t] = r.v[q][0];
        if (t < 2 * HALO) buf[q][t + SW] = r.v[q][1];
    }
}

__global__ __launch_bounds__(SW) void ssim_fwd_kernel(int H, int W, float C1, float C2,
                                                      const float* __restrict__ img1, const float* __restrict__ img2,
                                                      float* __restrict__ ssim_map, float* __restrict__ dm_dmu1,
                                                      float* __restrict__ dm_dsigma1_sq, float* __restrict__ dm_dsigma12)
{
    __shared__ float buf[2][2][RW];
    const int t = threadIdx.x;
    const int x0 = blockIdx.x * SW, y0 = blockIdx.y * SHR;
    const int xs = x0 - HALO;
    const size_t plane = (size_t)blockIdx.z * H * W;
    const float* a = img1 + plane;
    const float* b = img2 + plane;
    const int x = x0 + t;
    const int nsteps = SHR + 2 * HALO;    // input rows y0-5 .. y0+SHR+4
    float ring[11][5];
    Rows<2> nxt;
    load_row_fwd(nxt, a, b, H, W, y0 - HALO, xs);
    for (int s0 = 0; s0 < nsteps; s0 += 11) {
#pragma unroll
        for (int j = 0; j < 11; j++) {
            const int step = s0 + j;
            if (step >= nsteps) break;
            float (*cur)[RW] = buf[step & 1];
            put_row<2>(cur, nxt);
            if (step + 1 < nsteps) load_row_fwd(nxt, a, b, H, W, y0 - HALO + step + 1, xs);
            __syncthreads();
            float sa = 0.f, sb = 0.f, saa = 0.f, sbb = 0.f, sab = 0.f;
#pragma unroll
            for (int k = 0; k < 11; k++) {
                const float g = gwin(k);
                const float u = cur[0][t + k], w = cur[1][t + k];
                sa = __builtin_fmaf(g, u, sa);
                sb = __builtin_fmaf(g, w, sb);
                saa = __builtin_fmaf(g, u * u, saa);
                sbb = __builtin_fmaf(g, w * w, sbb);
                sab = __builtin_fmaf(g, u * w, sab);
            }
            ring[j][0] = sa; ring[j][1] = sb; ring[j][2] = saa; ring[j][3] = sbb; ring[j][4] = sab;
            // output row y = row of this step - 5, once rows y-5 .. y+5 are in the ring
            const int y = y0 - HALO + step - HALO;
            if (step >= 2 * HALO && y < H && x < W) {
                float v[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < 11; k++) {
                    const float g = gwin(k);
                    const int slot = (j + 1 + k) % 11;   // rows y-5+k in ascending order
#pragma unroll
                    for (int q = 0; q < 5; q++) v[q] = __builtin_fmaf(g, ring[slot][q], v[q]);
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
                const size_t oo = plane + (size_t)y * W + x;
                ssim_map[oo] = (Cn * Dn) / (A * Bd);
                if (dm_dmu1) {
                    dm_dmu1[oo] = ((m2 * 2.0f * Dn) / (A * Bd) - (m2 * 2.0f * Cn) / (A * Bd) -
                                   (m1 * 2.0f * Cn * Dn) / (A * A * Bd) + (m1 * 2.0f * Cn * Dn) / (A * Bd * Bd));
                    dm_dsigma1_sq[oo] = ((-Cn * Dn) / (A * Bd * Bd));
                    dm_dsigma12[oo] = ((2 * Cn) / (A * Bd));
                }
            }
        }
    }
}

__global__ __launch_bounds__(SW) void ssim_bwd_kernel(int H, int W, const float* __restrict__ img1,
                                                      const float* __restrict__ img2, const float* __restrict__ dL_dmap,
                                                      const float* __restrict__ dm_dmu1,
                                                      const float* __restrict__ dm_dsigma1_sq,
                                                      const float* __restrict__ dm_dsigma12, float* __restrict__ dL_dimg1)
{
    __shared__ float buf[2][3][RW];
    const int t = threadIdx.x;
    const int x0 = blockIdx.x * SW, y0 = blockIdx.y * SHR;
    const int xs = x0 - HALO;
    const size_t plane = (size_t)blockIdx.z * H * W;
    const float* d0 = dm_dmu1 + plane;
    const float* d1 = dm_dsigma1_sq + plane;
    const float* d2 = dm_dsigma12 + plane;
    const float* dl = dL_dmap + plane;
    const int x = x0 + t;
    const int nsteps = SHR + 2 * HALO;
    float ring[11][3];
    Rows<3> nxt;
    load_row_bwd(nxt, d0, d1, d2, dl, H, W, y0 - HALO, xs);
    for (int s0 = 0; s0 < nsteps; s0 += 11) {
#pragma unroll
        for (int j = 0; j < 11; j++) {
            const int step = s0 + j;
            if (step >= nsteps) break;
            float (*cur)[RW] = buf[step & 1];
            put_row<3>(cur, nxt);
            if (step + 1 < nsteps) load_row_bwd(nxt, d0, d1, d2, dl, H, W, y0 - HALO + step + 1, xs);
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 3; q++) {
                float acc = 0.f;
#pragma unroll
                for (int k = 0; k < 11; k++) acc = __builtin_fmaf(gwin(k), cur[q][t + k], acc);
                ring[j][q] = acc;
            }
            const int y = y0 - HALO + step - HALO;
            if (step >= 2 * HALO && y < H && x < W) {
                float v[3] = {0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < 11; k++) {
                    const float g = gwin(k);
                    const int slot = (j + 1 + k) % 11;
#pragma unroll
                    for (int q = 0; q < 3; q++) v[q] = __builtin_fmaf(g, ring[slot][q], v[q]);
                }
                const size_t oo = plane + (size_t)y * W + x;
                float d = 0.0f;
                d += v[0];
                d += img1[oo] * 2.0f * v[1];
                d += img2[oo] * v[2];
                gs::st_stream(&dL_dimg1[oo], d);   // streaming store: written once, not re-read here
            }
        }
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
    const dim3 grid(gs_div_up(W, SW), gs_div_up(H, SHR), B * C);
    GS_TIMED("ssim_fwd_kernel", stream,
             hipLaunchKernelGGL(ssim_fwd_kernel, grid, dim3(SW), 0, stream, H, W, C1, C2, img1, img2, ssim_map,
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
    const dim3 grid(gs_div_up(W, SW), gs_div_up(H, SHR), B * C);
    GS_TIMED("ssim_bwd_kernel", stream,
             hipLaunchKernelGGL(ssim_bwd_kernel, grid, dim3(SW), 0, stream, H, W, img1, img2, dL_dmap, dm_dmu1,
                                dm_dsigma1_sq, dm_dsigma12, dL_dimg1));
    GS_LAUNCH_CHECK("ssim_bwd_kernel");
    return GS_OK;
}
