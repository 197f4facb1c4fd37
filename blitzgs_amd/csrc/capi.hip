// Library-wide C-ABI pieces: version, thread-local error text, and the
// device-math diagnostic entry point.
#include <stdarg.h>
#include <stdio.h>

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

extern "C" int gs_version(void) { return 100; }
extern "C" const char* gs_last_error(void) { return g_err; }

namespace {
__global__ void diag_math_kernel(int op, int n, const float* __restrict__ x, float* __restrict__ y)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r;
    if (op == 0) r = gs::expf_full(v);
    else if (op == 1) r = gs::logf_full(v);
    else r = (v <= 0.0f || v != v) ? gs::expf_nonpos(v) : gs::expf_full(v);
    y[i] = r;
}
}  // namespace

extern "C" int gs_diag_math(int op, int n, const float* x, float* y, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(op >= 0 && op <= 2, "op must be 0 (exp), 1 (log) or 2 (blend exp)");
    GS_REQUIRE(n >= 0, "n must be >= 0");
    if (n == 0) return GS_OK;
    hipLaunchKernelGGL(diag_math_kernel, dim3(gs_div_up((size_t)n, 256)), dim3(256), 0, stream, op, n, x, y);
    GS_LAUNCH_CHECK("diag_math_kernel");
    return GS_OK;
}
