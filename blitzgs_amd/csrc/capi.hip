// Library-wide C-ABI pieces: version, thread-local error text, and the
// device-math diagnostic entry point.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {
thread_local char g_err[1024] = {0};
}

namespace gs {
void set_error(const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}
void clear_error() { g_err[0] = 0; }
}  // namespace gs

// ------------------------------------------------------------ kernel timing
namespace {
struct PendingMark {
    std::string name;
    hipEvent_t start, stop;
};
struct TimingState {
    std::mutex mu;
    int on = 0;   // 0 off, 1 every kernel and the stages, 2 the stages only
    std::vector<hipEvent_t> pool;
    std::vector<PendingMark> pending;
    std::vector<PendingMark> open_stages;   // stages begun and not yet ended
    std::vector<std::string> names;
    std::vector<double> total_ms;
    std::vector<int> counts;
};
TimingState& timing()
{
    static TimingState* s = new TimingState();   // lives until process exit
    return *s;
}
hipEvent_t take_event(TimingState& t)
{
    if (!t.pool.empty()) {
        hipEvent_t e = t.pool.back();
        t.pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
void drain(TimingState& t)
{
    for (auto& m : t.pending) {
        float ms = 0.f;
        if (m.start && m.stop && hipEventSynchronize(m.stop) == hipSuccess &&
            hipEventElapsedTime(&ms, m.start, m.stop) == hipSuccess) {
            size_t k = 0;
            while (k < t.names.size() && t.names[k] != m.name) k++;
            if (k == t.names.size()) { t.names.push_back(m.name); t.total_ms.push_back(0.0); t.counts.push_back(0); }
            t.total_ms[k] += ms;
            t.counts[k] += 1;
        }
        if (m.start) t.pool.push_back(m.start);
        if (m.stop) t.pool.push_back(m.stop);
    }
    t.pending.clear();
}
}  // namespace

namespace gs {
bool timing_on() { return timing().on != 0; }
bool timing_kernels_on() { return timing().on == 1; }
void timing_mark_begin(hipStream_t stream, const char* name)
{
    TimingState& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    PendingMark m{name, take_event(t), nullptr};
    if (m.start) (void)hipEventRecord(m.start, stream);
    t.pending.push_back(m);
}
void timing_mark_end(hipStream_t stream)
{
    TimingState& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    if (t.pending.empty()) return;
    PendingMark& m = t.pending.back();
    m.stop = take_event(t);
    if (m.stop) (void)hipEventRecord(m.stop, stream);
}
void timing_stage_begin(hipStream_t stream, const char* name)
{
    TimingState& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    PendingMark m{name, take_event(t), nullptr};
    if (m.start) (void)hipEventRecord(m.start, stream);
    t.open_stages.push_back(m);
}
void timing_stage_end(hipStream_t stream, const char* name)
{
    TimingState& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    for (size_t i = t.open_stages.size(); i-- > 0;) {
        if (t.open_stages[i].name != name) continue;
        PendingMark m = t.open_stages[i];
        t.open_stages.erase(t.open_stages.begin() + (long)i);
        m.stop = take_event(t);
        if (m.stop) (void)hipEventRecord(m.stop, stream);
        t.pending.push_back(m);
        return;
    }
}
}  // namespace gs

extern "C" int gs_timing_enable(int on)
{
    TimingState& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    if (on < 0 || on > 2) {
        gs::set_error("timing mode must be 0, 1 or 2 (got %d)", on);
        return GS_ERR_ARG;
    }
    t.on = on;
    return GS_OK;
}

extern "C" int gs_timing_reset(void)
{
    TimingState& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    drain(t);
    for (auto& m : t.open_stages)
        if (m.start) t.pool.push_back(m.start);
    t.open_stages.clear();
    t.names.clear(); t.total_ms.clear(); t.counts.clear();
    return GS_OK;
}

extern "C" int gs_timing_read(int max_entries, char* names, double* total_ms, int* counts)
{
    TimingState& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    drain(t);
    const int n = (int)t.names.size();
    for (int i = 0; i < n && i < max_entries; i++) {
        strncpy(names + 64 * i, t.names[i].c_str(), 63);
        names[64 * i + 63] = 0;
        total_ms[i] = t.total_ms[i];
        counts[i] = t.counts[i];
    }
    return n;
}

extern "C" int gs_version(void) { return 100; }
extern "C" const char* gs_last_error(void) { return g_err; }

namespace {
// op 3: x holds 12 x 64 values ([value][lane]); y[k] = sum over lanes of value k
__global__ void diag_sum12_kernel(const float* __restrict__ x, float* __restrict__ y)
{
    float v[12];
#pragma unroll
    for (int k = 0; k < 12; k++) v[k] = x[k * 64 + threadIdx.x];
    const float t = gs::wave_sum12(v);
    const int k = gs::wave_sum12_index((int)threadIdx.x);
    if (k >= 0) y[k] = t;
}

__global__ void diag_math_kernel(int op, int n, const float* __restrict__ x, float* __restrict__ y)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r;
    if (op == 0) r = gs::expf_full(v);
    else if (op == 1) r = gs::logf_full(v);
    else if (op == 6) gs::blend_alpha(1.0f, v, gs::alpha_cut_power(1.0f), r);
    else r = (v <= 0.0f || v != v) ? gs::expf_nonpos(v) : gs::expf_full(v);
    y[i] = r;
}

// op 4: plain copy of n floats (n % 4 == 0), 16-byte loads and stores; the
// known-size reference against which HBM byte counters are calibrated
__global__ void diag_copy_kernel(size_t n4, const float4* __restrict__ x, float4* __restrict__ y)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) y[i] = x[i];
}

// op 5: VALU issue-rate reference.  Every wave runs `iters` rounds of 32
// independent-chain fp32 FMAs (8 chains, 4 deep), i.e. 32 * iters VALU
// instructions; the result is stored only in the (never met) case that it
// equals a sentinel, so nothing is optimised away and nothing is written.
constexpr int DIAG_VALU_BLOCKS = 8192;
__global__ __launch_bounds__(256) void diag_valu_kernel(int iters, float a, float b, float* __restrict__ y)
{
    float x0 = threadIdx.x * 1e-3f, x1 = x0 + 1e-4f, x2 = x0 + 2e-4f, x3 = x0 + 3e-4f;
    float x4 = x0 + 4e-4f, x5 = x0 + 5e-4f, x6 = x0 + 6e-4f, x7 = x0 + 7e-4f;
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            x0 = __builtin_fmaf(x0, a, b); x1 = __builtin_fmaf(x1, a, b);
            x2 = __builtin_fmaf(x2, a, b); x3 = __builtin_fmaf(x3, a, b);
            x4 = __builtin_fmaf(x4, a, b); x5 = __builtin_fmaf(x5, a, b);
            x6 = __builtin_fmaf(x6, a, b); x7 = __builtin_fmaf(x7, a, b);
        }
    }
    const float s = ((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7));
    if (s == 12345.0f) y[0] = s;
}
}  // namespace

extern "C" int gs_diag_math(int op, int n, const float* x, float* y, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(op >= 0 && op <= 9,
               "op must be 0 (exp), 1 (log), 2 (exact blend exp), 3 (wave sum of 12 values), 4 (copy), "
               "5 (VALU rate), 6 (the blend's falloff G), 7, 8 or 9 (forward / backward / half-tile backward "
               "blend VALU probe)");
    GS_REQUIRE(n >= 0, "n must be >= 0");
    if (op >= 7 && op <= 9) return gs::render_valu_probe(op - 7, n, y, stream);
    if (op == 5) {
        GS_REQUIRE(y != nullptr, "op 5 needs y (one float)");
        if (n == 0) return GS_OK;
        GS_TIMED("diag_valu_kernel", stream,
                 hipLaunchKernelGGL(diag_valu_kernel, dim3(DIAG_VALU_BLOCKS), dim3(256), 0, stream, n, 0.999f, 1e-3f,
                                    y));
        GS_LAUNCH_CHECK("diag_valu_kernel");
        return GS_OK;
    }
    if (op == 3) {
        GS_REQUIRE(n == 12 * 64, "op 3 takes 12 x 64 inputs");
        hipLaunchKernelGGL(diag_sum12_kernel, dim3(1), dim3(64), 0, stream, x, y);
        GS_LAUNCH_CHECK("diag_sum12_kernel");
        return GS_OK;
    }
    if (n == 0) return GS_OK;
    if (op == 4) {
        GS_REQUIRE(n % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0,
                   "op 4 copies whole 16-byte groups from 16-byte aligned buffers");
        const size_t n4 = (size_t)n / 4;
        const unsigned blocks = (unsigned)std::min<size_t>(gs_div_up(n4, 256), 32768);
        GS_TIMED("diag_copy_kernel", stream,
                 hipLaunchKernelGGL(diag_copy_kernel, dim3(blocks), dim3(256), 0, stream, n4,
                                    (const float4*)x, (float4*)y));
        GS_LAUNCH_CHECK("diag_copy_kernel");
        return GS_OK;
    }
    hipLaunchKernelGGL(diag_math_kernel, dim3(gs_div_up((size_t)n, 256)), dim3(256), 0, stream, op, n, x, y);
    GS_LAUNCH_CHECK("diag_math_kernel");
    return GS_OK;
}
