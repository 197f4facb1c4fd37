// Host-side helpers for the C-ABI entry points: error reporting and launch
// checks.  Every entry point returns 0 on success or a negative code, and
// leaves a message for gs_last_error().
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gs {
void set_error(const char* fmt, ...);
void clear_error();

// Optional per-kernel timing (gs_timing_enable): in mode 1 every launch made
// through GS_TIMED is bracketed by HIP events on its stream and the elapsed
// times are accumulated per kernel name by gs_timing_read; stages (below) are
// timed in modes 1 and 2.
bool timing_on();          // mode 1 or 2: stage marks
bool timing_kernels_on();  // mode 1: per-launch marks
void timing_mark_begin(hipStream_t stream, const char* name);
void timing_mark_end(hipStream_t stream);
// A named stage spanning several launches (and entry points) on one stream:
// its time runs from the begin mark to the end mark of the same name.
void timing_stage_begin(hipStream_t stream, const char* name);
void timing_stage_end(hipStream_t stream, const char* name);
// The blend kernels' VALU probes (render.hip): which 0 forward, 1 backward.
int render_valu_probe(int which, int iters, float* y, hipStream_t stream);
}  // namespace gs

#define GS_TIMED(name, stream, launch)                                                 \
    do {                                                                               \
        const bool gs_t_ = gs::timing_kernels_on();                                    \
        if (gs_t_) gs::timing_mark_begin(stream, name);                                \
        launch;                                                                        \
        if (gs_t_) gs::timing_mark_end(stream);                                        \
    } while (0)

#define GS_OK 0
#define GS_ERR_ARG -1
#define GS_ERR_HIP -2
#define GS_ERR_SIZE -3

#define GS_HIP(expr)                                                                   \
    do {                                                                               \
        hipError_t gs_e_ = (expr);                                                     \
        if (gs_e_ != hipSuccess) {                                                     \
            gs::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(gs_e_),    \
                          __FILE__, __LINE__);                                         \
            return GS_ERR_HIP;                                                         \
        }                                                                              \
    } while (0)

#define GS_LAUNCH_CHECK(name)                                                          \
    do {                                                                               \
        hipError_t gs_e_ = hipGetLastError();                                          \
        if (gs_e_ != hipSuccess) {                                                     \
            gs::set_error("launch of %s failed: %s", name, hipGetErrorString(gs_e_));  \
            return GS_ERR_HIP;                                                         \
        }                                                                              \
    } while (0)

#define GS_REQUIRE(cond, ...)                                                          \
    do {                                                                               \
        if (!(cond)) {                                                                 \
            gs::set_error(__VA_ARGS__);                                                \
            return GS_ERR_ARG;                                                         \
        }                                                                              \
    } while (0)

static inline unsigned gs_div_up(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }
