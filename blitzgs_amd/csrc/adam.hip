// Sparse Adam step for Gaussian parameters (the SparseGaussianAdam optimiser).
//
// Reference: BlitzGS submodule/diff-gaussian-rasterization_f
//   cuda_rasterizer/adam.cu:9-67       adamUpdateCUDA, one launch per parameter
//   rasterize_points.cu:807-832        adamUpdate binding
//   diff_gaussian_rasterization_f/__init__.py:832-863  SparseGaussianAdam.step
// For every element p of a (N, M) parameter whose Gaussian p / M is visible:
//   m = b1 m + (1 - b1) g;  v = b2 v + ((1 - b2) g) g;  param += (-lr m) / (sqrt(v) + eps)
// in fp32, left to right, without contraction (so the CPU oracle reproduces
// it bit for bit); elements of invisible Gaussians keep their values.
//
// Design: all parameter groups of one optimiser step go in one launch.  The
// groups' float4 work items are concatenated; a block finds its group from a
// small table of block offsets.  A thread handles four consecutive elements
// and loads nothing when none of their Gaussians is visible (about four in
// five for a large scene), so the step moves only the visible rows.
#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {

constexpr int ADAM_THREADS = 256;
constexpr int ADAM_MAX_GROUPS = 8;

struct AdamGroupDev {
    float* param;
    const float* grad;
    float* m;
    float* v;
    uint32_t M;        // elements per Gaussian
    uint32_t vec;      // 1: the four arrays are 16-byte aligned
    uint64_t cnt;      // N * M elements
    float lr, eps;
};

struct AdamBatch {
    AdamGroupDev g[ADAM_MAX_GROUPS];
    uint32_t block_start[ADAM_MAX_GROUPS + 1];   // first block of each group; [n] = total
    int n;
};

__device__ __forceinline__ void adam_one(float& p, float& m, float& v, float g, float lr, float b1, float b2,
                                         float eps)
{
    const float mn = b1 * m + (1.0f - b1) * g;
    const float vn = b2 * v + ((1.0f - b2) * g) * g;
    const float step = ((-lr) * mn) / (__builtin_sqrtf(vn) + eps);
    p = p + step;
    m = mn;
    v = vn;
}

__global__ __launch_bounds__(ADAM_THREADS) void adam_kernel(AdamBatch B, const uint8_t* __restrict__ visible,
                                                            float b1, float b2)
{
    const uint32_t b = blockIdx.x;
    int gi = 0;
#pragma unroll
    for (int k = 1; k < ADAM_MAX_GROUPS; k++)
        if (k < B.n && b >= B.block_start[k]) gi = k;
    const AdamGroupDev G = B.g[gi];
    const uint64_t item = (uint64_t)(b - B.block_start[gi]) * ADAM_THREADS + threadIdx.x;
    const uint64_t e0 = item * 4;
    if (e0 >= G.cnt) return;
    const uint32_t n_el = (uint32_t)min((uint64_t)4, G.cnt - e0);
    // the Gaussian of element e0 + k: one division per item (32-bit when the
    // group fits), the other three rows follow by comparison (k < 4, M >= 1)
    const uint64_t row0 = G.cnt <= 0xffffffffull ? (uint64_t)((uint32_t)e0 / G.M) : e0 / G.M;
    const uint32_t rem = (uint32_t)(e0 - row0 * G.M);
    bool vis[4];
    bool any = false;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t t = rem + (uint32_t)k;
        const uint64_t row = row0 + (uint64_t)((t >= G.M) + (t >= 2 * G.M) + (t >= 3 * G.M));
        vis[k] = (uint32_t)k < n_el && visible[row] != 0;
        any = any || vis[k];
    }
    if (!any) return;
    if (G.vec && n_el == 4) {
        const float4 g4 = reinterpret_cast<const float4*>(G.grad)[item];
        float4 p4 = reinterpret_cast<float4*>(G.param)[item];
        float4 m4 = reinterpret_cast<float4*>(G.m)[item];
        float4 v4 = reinterpret_cast<float4*>(G.v)[item];
        float p[4] = {p4.x, p4.y, p4.z, p4.w}, m[4] = {m4.x, m4.y, m4.z, m4.w}, v[4] = {v4.x, v4.y, v4.z, v4.w};
        const float g[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float pk = p[k], mk = m[k], vk = v[k];
            adam_one(pk, mk, vk, g[k], G.lr, b1, b2, G.eps);
            if (vis[k]) { p[k] = pk; m[k] = mk; v[k] = vk; }
        }
        reinterpret_cast<float4*>(G.param)[item] = make_float4(p[0], p[1], p[2], p[3]);
        reinterpret_cast<float4*>(G.m)[item] = make_float4(m[0], m[1], m[2], m[3]);
        reinterpret_cast<float4*>(G.v)[item] = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        for (uint32_t k = 0; k < n_el; k++) {
            if (!vis[k]) continue;
            const uint64_t e = e0 + k;
            float pk = G.param[e], mk = G.m[e], vk = G.v[e];
            adam_one(pk, mk, vk, G.grad[e], G.lr, b1, b2, G.eps);
            G.param[e] = pk;
            G.m[e] = mk;
            G.v[e] = vk;
        }
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int gs_adam_update_groups(int n_groups, const gs_adam_group* groups, int64_t N, const uint8_t* visible,
                                     float b1, float b2, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(n_groups >= 0 && n_groups <= ADAM_MAX_GROUPS, "n_groups must be in [0, %d]", ADAM_MAX_GROUPS);
    GS_REQUIRE(N >= 0, "N must be >= 0");
    if (n_groups == 0 || N == 0) return GS_OK;
    GS_REQUIRE(groups != nullptr && visible != nullptr, "groups and visible must be non-null");
    AdamBatch B{};
    B.n = n_groups;
    uint64_t blocks = 0;
    for (int i = 0; i < n_groups; i++) {
        const gs_adam_group& s = groups[i];
        GS_REQUIRE(s.M >= 1 && s.M <= 0x7fffffff, "group %d: elements per Gaussian must be >= 1", i);
        GS_REQUIRE(s.param && s.grad && s.exp_avg && s.exp_avg_sq, "group %d: null pointer", i);
        AdamGroupDev& d = B.g[i];
        d.param = s.param;
        d.grad = s.grad;
        d.m = s.exp_avg;
        d.v = s.exp_avg_sq;
        d.M = (uint32_t)s.M;
        d.vec = aligned16(s.param) && aligned16(s.grad) && aligned16(s.exp_avg) && aligned16(s.exp_avg_sq);
        d.cnt = (uint64_t)N * (uint64_t)s.M;
        d.lr = s.lr;
        d.eps = s.eps;
        B.block_start[i] = (uint32_t)blocks;
        blocks += (d.cnt + 4ull * ADAM_THREADS - 1) / (4ull * ADAM_THREADS);
        GS_REQUIRE(blocks < 0x7fffffffull, "too many elements for one launch");
    }
    for (int i = n_groups; i <= ADAM_MAX_GROUPS; i++) B.block_start[i] = (uint32_t)blocks;
    if (blocks == 0) return GS_OK;
    GS_TIMED("adam_kernel", stream,
             hipLaunchKernelGGL(adam_kernel, dim3((unsigned)blocks), dim3(ADAM_THREADS), 0, stream, B, visible, b1,
                                b2));
    GS_LAUNCH_CHECK("adam_kernel");
    return GS_OK;
}

extern "C" int gs_adam_update(float* param, const float* param_grad, float* exp_avg, float* exp_avg_sq,
                              const uint8_t* visible, float lr, float b1, float b2, float eps, int64_t N, int64_t M,
                              hipStream_t stream)
{
    const gs_adam_group g{param, param_grad, exp_avg, exp_avg_sq, M, lr, eps};
    return gs_adam_update_groups(1, &g, N, visible, b1, b2, stream);
}
