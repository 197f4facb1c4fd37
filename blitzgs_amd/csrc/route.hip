// Gaussian -> rank routing of the image-distributed training step, and the
// row moves around its all-to-all (pack, unpack, gradient scatter).
//
// Reference: BlitzGS submodule/diff-gaussian-rasterization_f
//   rasterize_points.cu:212-289   getTouchedIdsBool / GetLocal2jIdsBoolCUDA
//   rasterize_points.cu:291-367   getTouchedIdsBoolAdjustMode6 / GetLocal2jIdsBoolAdjustMode6CUDA
//   cuda_rasterizer/auxiliary.h:51-61   getRect(float2, int)
// and the Python around them:
//   gaussian_renderer/workload_division.py:682-704  bool matrix -> per-rank ids (nonzero, one host sync per rank)
//   gaussian_renderer/__init__.py:22-189            cat + index per rank (pack), all_to_all,
//                                                   split + cat + radii.int() (unpack)
//
// Routing rule (both modes look only at the rectangle, never at whether the
// Gaussian was culled):
//   interval mode: rank rk gets Gaussian i when the row-major tile-index span
//     [y0*gx + x0, (y1-1)*gx + x1 - 1] of its rect meets [s[rk], s[rk+1]),
//     both ends widened by gx + 1 when avoid_pixel_all2all is set.  The span
//     is computed in 32-bit unsigned arithmetic and read as int, as the
//     reference's types do (an empty rect at the origin gives a negative end).
//   rectangle mode: rank rk owns tile rows [y_l, y_r) and columns [x_l, x_r)
//     (widened by one tile on each side when avoid is set, the low ends not
//     below 0); rect overlap with unsigned-versus-int comparisons.
//
// Design: the reference writes a (P, world) bool matrix, then takes one
// nonzero() per rank (a device->host sync each) and gathers rows with
// torch.cat + index + split.  Here one counting pass (bool matrix optional)
// and one writing pass produce every rank's id list at once, in Gaussian id
// order, concatenated rank after rank, with a single host read of the counts;
// a generic row mover does the pack, the unpack and the gradient scatter, each
// in one launch with coalesced stores.
#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {

using gs::ballot;
using gs::f2i_sat;
using gs::lane_id;
using gs::rank_below;
using gs::rect_int;

constexpr int ROUTE_THREADS = 256;
constexpr int ROUTE_WAVES = ROUTE_THREADS / 64;
constexpr int ROUTE_MAX_BLOCKS = 2048;
constexpr int ROUTE_MAX_WORLD_IDS = 64;   // ranks handled by the id-list path (one bit per rank)
constexpr int MOVE_MAX_FIELDS = 8;
constexpr int MOVE_MAX_COLS = 32;
constexpr int MOVE_ROWS = 256;            // rows per block of the row mover (LDS: 32 KB of staged rows)
constexpr int MOVE_MAX_CHUNKS = 16;       // <= 4-column chunks: 8 fields, 32 columns split at most this far

struct RouteGeom {
    unsigned gx, gy;
    int world;
    int avoid;
};

// Rank test for Gaussian rect [x0,x1) x [y0,y1) against rank rk.
template <bool RECT>
__device__ __forceinline__ bool route_hit(const RouteGeom& G, const int* __restrict__ table, int rk, unsigned x0,
                                          unsigned y0, unsigned x1, unsigned y1)
{
    if constexpr (!RECT) {
        const int lo = (int)(y0 * G.gx + x0);
        const int hi = (int)((y1 - 1u) * G.gx + x1 - 1u);
        if (hi < lo) return false;
        int tl = table[rk], tr = table[rk + 1];
        if (G.avoid) {
            tl = (int)((unsigned)tl - (G.gx + 1u));
            tr = (int)((unsigned)tr + (G.gx + 1u));
        }
        return !(hi < tl || lo >= tr);
    } else {
        int yl = table[4 * rk + 0], yr = table[4 * rk + 1];
        int xl = table[4 * rk + 2], xr = table[4 * rk + 3];
        if (G.avoid) {
            if (yl > 0) yl -= 1;
            if (xl > 0) xl -= 1;
            yr += 1;
            xr += 1;
        }
        return !(y1 <= (unsigned)yl || (unsigned)yr <= y0 || x1 <= (unsigned)xl || (unsigned)xr <= x0);
    }
}

__device__ __forceinline__ void route_rect(const RouteGeom& G, const float* __restrict__ means2D,
                                           const int* __restrict__ radii, int i, unsigned& x0, unsigned& y0,
                                           unsigned& x1, unsigned& y1)
{
    const float2 m = reinterpret_cast<const float2*>(means2D)[i];
    rect_int(m.x, m.y, radii[i], G.gx, G.gy, x0, y0, x1, y1);
}

// Bit rk of the result: rank rk gets Gaussian i (world <= 64).
template <bool RECT>
__device__ __forceinline__ uint64_t route_mask(const RouteGeom& G, const int* __restrict__ table,
                                               const float* __restrict__ means2D, const int* __restrict__ radii, int i)
{
    unsigned x0, y0, x1, y1;
    route_rect(G, means2D, radii, i, x0, y0, x1, y1);
    uint64_t m = 0;
    for (int rk = 0; rk < G.world; rk++)
        if (route_hit<RECT>(G, table, rk, x0, y0, x1, y1)) m |= 1ull << rk;
    return m;
}

// The (P, world) bool matrix alone, for any world size.
template <bool RECT>
__global__ __launch_bounds__(ROUTE_THREADS) void route_bool_kernel(int P, RouteGeom G, const float* __restrict__ means2D,
                                                                   const int* __restrict__ radii,
                                                                   const int* __restrict__ table,
                                                                   uint8_t* __restrict__ out)
{
    const int i = blockIdx.x * ROUTE_THREADS + threadIdx.x;
    if (i >= P) return;
    unsigned x0, y0, x1, y1;
    route_rect(G, means2D, radii, i, x0, y0, x1, y1);
    uint8_t* row = out + (size_t)i * (size_t)G.world;
    if (G.world == 1) {
        row[0] = route_hit<RECT>(G, table, 0, x0, y0, x1, y1) ? 1 : 0;
        return;
    }
    for (int rk = 0; rk < G.world; rk++) row[rk] = route_hit<RECT>(G, table, rk, x0, y0, x1, y1) ? 1 : 0;
}

// Per block (a contiguous span of Gaussians) and rank: how many Gaussians go
// to that rank.  blk_cnt is rank-major: [rk * NB + b].  Optionally writes the
// bool matrix on the way.
template <bool RECT>
__global__ __launch_bounds__(ROUTE_THREADS) void route_count_kernel(int P, int span, RouteGeom G,
                                                                    const float* __restrict__ means2D,
                                                                    const int* __restrict__ radii,
                                                                    const int* __restrict__ table,
                                                                    uint8_t* __restrict__ out_bool,
                                                                    uint32_t* __restrict__ blk_cnt)
{
    __shared__ uint32_t s_cnt[ROUTE_MAX_WORLD_IDS];
    const int lane = lane_id();
    if (threadIdx.x < ROUTE_MAX_WORLD_IDS) s_cnt[threadIdx.x] = 0;
    __syncthreads();
    const int b = blockIdx.x;
    const int begin = b * span;
    const int end = min(P, begin + span);
    uint32_t acc = 0;   // lane rk: this wave's count for rank rk
    for (int c0 = begin; c0 < end; c0 += ROUTE_THREADS) {
        const int i = c0 + (int)threadIdx.x;
        const uint64_t m = i < end ? route_mask<RECT>(G, table, means2D, radii, i) : 0ull;
        if (out_bool && i < end) {
            uint8_t* row = out_bool + (size_t)i * (size_t)G.world;
            for (int rk = 0; rk < G.world; rk++) row[rk] = (uint8_t)((m >> rk) & 1ull);
        }
        for (int rk = 0; rk < G.world; rk++) {
            const uint32_t c = (uint32_t)__builtin_popcountll(ballot(((m >> rk) & 1ull) != 0));
            if (lane == rk) acc += c;
        }
    }
    if (lane < G.world && acc) atomicAdd(&s_cnt[lane], acc);
    __syncthreads();
    if ((int)threadIdx.x < G.world) blk_cnt[(size_t)threadIdx.x * gridDim.x + b] = s_cnt[threadIdx.x];
}

// Exclusive scan of the rank-major block counts in place (one 1024-thread
// block); counts[rk] = number of ids rank rk receives, counts[world] = total.
__global__ __launch_bounds__(1024) void route_scan_kernel(int NB, int world, uint32_t* __restrict__ blk,
                                                          int64_t* __restrict__ counts)
{
    __shared__ uint32_t s_wave[32];
    const int N = NB * world;
    uint32_t base = 0;
    for (int c0 = 0; c0 < N; c0 += 1024) {
        const int k = c0 + (int)threadIdx.x;
        const uint32_t v = k < N ? blk[k] : 0u;
        uint32_t tot;
        const uint32_t pre = gs::block_excl_scan_1024(v, s_wave, &tot);
        if (k < N) blk[k] = base + pre;
        base += tot;
    }
    __syncthreads();
    for (int rk = (int)threadIdx.x; rk <= world; rk += 1024) {
        if (rk < world) {
            const uint32_t s = blk[(size_t)rk * NB];
            const uint32_t e = rk + 1 < world ? blk[(size_t)(rk + 1) * NB] : base;
            counts[rk] = (int64_t)(e - s);
        } else {
            counts[world] = (int64_t)base;
        }
    }
}

// Writes every rank's ids (ascending) at the block offsets of the scan.
template <bool RECT>
__global__ __launch_bounds__(ROUTE_THREADS) void route_write_kernel(int P, int span, RouteGeom G,
                                                                    const float* __restrict__ means2D,
                                                                    const int* __restrict__ radii,
                                                                    const int* __restrict__ table,
                                                                    const uint32_t* __restrict__ blk_off,
                                                                    int64_t* __restrict__ ids, uint32_t n_ids)
{
    __shared__ uint32_t s_wcnt[ROUTE_WAVES][ROUTE_MAX_WORLD_IDS];
    __shared__ uint32_t s_run[ROUTE_MAX_WORLD_IDS];
    const int lane = lane_id();
    const int wid = (int)threadIdx.x >> 6;
    const int b = blockIdx.x;
    if ((int)threadIdx.x < G.world) s_run[threadIdx.x] = blk_off[(size_t)threadIdx.x * gridDim.x + b];
    const int begin = b * span;
    const int end = min(P, begin + span);
    __syncthreads();
    for (int c0 = begin; c0 < end; c0 += ROUTE_THREADS) {
        const int i = c0 + (int)threadIdx.x;
        const uint64_t m = i < end ? route_mask<RECT>(G, table, means2D, radii, i) : 0ull;
        uint32_t mine = 0;   // lane rk: this wave's count for rank rk
        for (int rk = 0; rk < G.world; rk++) {
            const uint32_t c = (uint32_t)__builtin_popcountll(ballot(((m >> rk) & 1ull) != 0));
            if (lane == rk) mine = c;
        }
        if (lane < G.world) s_wcnt[wid][lane] = mine;
        __syncthreads();
        uint32_t wbase = 0;   // lane rk: first slot of this wave for rank rk
        if (lane < G.world) {
            wbase = s_run[lane];
            for (int w = 0; w < wid; w++) wbase += s_wcnt[w][lane];
        }
        for (int rk = 0; rk < G.world; rk++) {
            const bool hit = ((m >> rk) & 1ull) != 0;
            const uint64_t bal = ballot(hit);
            if (bal == 0) continue;
            const uint32_t wb = (uint32_t)__builtin_amdgcn_readlane((int)wbase, rk);
            const uint32_t pos = wb + (uint32_t)rank_below(bal);
            if (hit && pos < n_ids) ids[pos] = (int64_t)i;   // n_ids: the counted total
        }
        __syncthreads();
        if ((int)threadIdx.x < G.world) {
            uint32_t t = 0;
            for (int w = 0; w < ROUTE_WAVES; w++) t += s_wcnt[w][threadIdx.x];
            s_run[threadIdx.x] += t;
        }
        __syncthreads();
    }
}

// One chunk of at most 4 columns of a field (wider fields are split on the
// host), so every thread handles at most 4 elements of a chunk per block.
struct MoveField {
    const void* src;
    void* dst;
    int64_t src_stride, dst_stride;   // elements
    int width;                        // 1..4
    int off;                          // first column of the chunk in a staged row
    uint32_t magic;                   // ceil(2^20 / width): k / width = (k * magic) >> 20 for k < 2^13
    int src_i32, dst_i32;
};

struct MoveSpec {
    MoveField f[MOVE_MAX_CHUNKS];
    int n, cols;
    const uint32_t* src_linear;       // non-null: the sources are one row-major buffer of `cols` words per
                                      // row, read without a source map
    uint32_t* dst_linear;             // non-null: likewise the destinations, written without a destination map
};

// Word conversion between the field types (torch's .float() / .int()).
__device__ __forceinline__ uint32_t convert_word(uint32_t w, int src_i32, int dst_i32)
{
    if (src_i32 == dst_i32) return w;
    return dst_i32 ? (uint32_t)f2i_sat(__uint_as_float(w)) : __float_as_uint((float)(int)w);
}

__device__ __forceinline__ int div_small(int k, uint32_t magic) { return (int)(((uint64_t)(uint32_t)k * magic) >> 20); }

// Row mover, staged through LDS: a block moves MOVE_ROWS rows.  Phase 1
// gathers the rows' fields into LDS rows of `cols` 32-bit words (element k of
// a chunk is (row k / width, column k % width), so consecutive lanes read
// consecutive elements of consecutive source rows) and converts them to the
// destination type; every thread issues all its loads (up to 4 per chunk)
// before its first LDS store, so each wave keeps many loads in flight.  A
// row-major source is instead copied as one contiguous span (words keep the
// source type; phase 2 converts).  Phase 2 writes the rows out the same way
// per chunk, or as one contiguous span when the destination is a row-major
// buffer.
// Row-interleaved (packed) and field-separated layouts are both read and
// written with coalesced accesses.  A source row outside [0, n_src) reads as
// zero; a destination row outside [0, n_dst) is skipped.
__global__ __launch_bounds__(ROUTE_THREADS) void move_rows_kernel(int64_t n_rows, const int64_t* __restrict__ smap,
                                                                  const int64_t* __restrict__ dmap, int64_t n_src,
                                                                  int64_t n_dst, MoveSpec S, int accumulate)
{
    __shared__ __align__(16) uint32_t s_rows[MOVE_ROWS * MOVE_MAX_COLS];
    __shared__ int64_t s_src[MOVE_ROWS], s_dst[MOVE_ROWS];
    const int64_t r0 = (int64_t)blockIdx.x * MOVE_ROWS;
    const int nr = (int)min((int64_t)MOVE_ROWS, n_rows - r0);
    const int cols = S.cols;
    const int tid = (int)threadIdx.x;
    const int n_words = nr * cols;
    if (tid < nr) {
        const int64_t sr = smap ? smap[r0 + tid] : r0 + tid;
        const int64_t dr = dmap ? dmap[r0 + tid] : r0 + tid;
        s_src[tid] = (sr >= 0 && sr < n_src) ? sr : -1;
        s_dst[tid] = (dr >= 0 && dr < n_dst) ? dr : -1;
    }
    // phase 1: sources -> LDS
    const bool lds_src_typed = S.src_linear != nullptr;
    if (lds_src_typed) {
        // contiguous span of n_words words, 16-byte aligned (r0 * cols * 4 is a multiple of 1024)
        const uint32_t* src = S.src_linear + r0 * cols;
        const int n4 = n_words >> 2;
        uint4 v[MOVE_MAX_COLS / 4];
#pragma unroll
        for (int i = 0; i < MOVE_MAX_COLS / 4; i++) {
            const int q = tid + i * ROUTE_THREADS;
            v[i] = q < n4 ? reinterpret_cast<const uint4*>(src)[q] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int i = 0; i < MOVE_MAX_COLS / 4; i++) {
            const int q = tid + i * ROUTE_THREADS;
            if (q < n4) reinterpret_cast<uint4*>(s_rows)[q] = v[i];
        }
        const int k = (n4 << 2) + tid;
        if (k < n_words) s_rows[k] = src[k];
        __syncthreads();
    } else {
        __syncthreads();   // s_src ready
        uint32_t v[MOVE_MAX_CHUNKS][4] = {};
#pragma unroll
        for (int f = 0; f < MOVE_MAX_CHUNKS; f++) {
            if (f < S.n) {
                const MoveField& F = S.f[f];
                const uint32_t* src = static_cast<const uint32_t*>(F.src);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int k = tid + i * ROUTE_THREADS;
                    if (i < F.width && k < nr * F.width) {
                        const int row = div_small(k, F.magic);
                        const int c = k - row * F.width;
                        const int64_t sr = s_src[row];
                        v[f][i] = sr >= 0 ? convert_word(src[sr * F.src_stride + c], F.src_i32, F.dst_i32) : 0u;
                    }
                }
            }
        }
#pragma unroll
        for (int f = 0; f < MOVE_MAX_CHUNKS; f++) {
            if (f < S.n) {
                const MoveField& F = S.f[f];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int k = tid + i * ROUTE_THREADS;
                    if (i < F.width && k < nr * F.width) {
                        const int row = div_small(k, F.magic);
                        const int c = k - row * F.width;
                        s_rows[row * cols + F.off + c] = v[f][i];
                    }
                }
            }
        }
        __syncthreads();
    }
    // phase 2: LDS -> destinations
    if (S.dst_linear && !accumulate) {
        uint32_t* dst = S.dst_linear + r0 * cols;
        const int n4 = n_words >> 2;
        for (int q = tid; q < n4; q += ROUTE_THREADS)
            reinterpret_cast<uint4*>(dst)[q] = reinterpret_cast<const uint4*>(s_rows)[q];
        const int k = (n4 << 2) + tid;
        if (k < n_words) dst[k] = s_rows[k];
        return;
    }
    for (int f = 0; f < S.n; f++) {
        const MoveField F = S.f[f];
        for (int k = tid; k < nr * F.width; k += ROUTE_THREADS) {
            const int row = div_small(k, F.magic);
            const int c = k - row * F.width;
            const int64_t dr = s_dst[row];
            if (dr < 0) continue;
            uint32_t w = s_rows[row * cols + F.off + c];
            if (lds_src_typed) w = convert_word(w, F.src_i32, F.dst_i32);
            const int64_t di = dr * F.dst_stride + c;
            if (F.dst_i32) {
                int* d = static_cast<int*>(F.dst) + di;
                *d = accumulate ? *d + (int)w : (int)w;
            } else {
                float* d = static_cast<float*>(F.dst) + di;
                *d = accumulate ? *d + __uint_as_float(w) : __uint_as_float(w);
            }
        }
    }
}

struct RoutePlan {
    int NB, span;
};

RoutePlan route_plan(int P)
{
    const int chunks = (P + ROUTE_THREADS - 1) / ROUTE_THREADS;
    RoutePlan p;
    p.NB = chunks < ROUTE_MAX_BLOCKS ? chunks : ROUTE_MAX_BLOCKS;
    if (p.NB < 1) p.NB = 1;
    p.span = ((chunks + p.NB - 1) / p.NB) * ROUTE_THREADS;
    return p;
}

int route_check(int mode, int P, int H, int W, int world, const float* means2D, const int* radii, const int* table,
                RouteGeom& G)
{
    GS_REQUIRE(mode == GS_ROUTE_INTERVAL || mode == GS_ROUTE_RECT, "mode must be GS_ROUTE_INTERVAL or GS_ROUTE_RECT");
    GS_REQUIRE(P >= 0 && H > 0 && W > 0, "bad sizes P=%d H=%d W=%d", P, H, W);
    GS_REQUIRE(world >= 1, "world_size must be >= 1");
    GS_REQUIRE(P <= 0x7ff00000, "P must be below 2^31 - 2^20");
    GS_REQUIRE(P == 0 || (means2D && radii && table), "null input");
    G.gx = (unsigned)((W + 15) / 16);
    G.gy = (unsigned)((H + 15) / 16);
    G.world = world;
    return GS_OK;
}

}  // namespace

extern "C" int gs_local2j_ids_bool(int mode, int P, int H, int W, int world_size, const float* means2D,
                                   const int* radii, const int* table, int avoid_pixel_all2all, uint8_t* out,
                                   hipStream_t stream)
{
    gs::clear_error();
    RouteGeom G{};
    if (int rc = route_check(mode, P, H, W, world_size, means2D, radii, table, G)) return rc;
    G.avoid = avoid_pixel_all2all ? 1 : 0;
    if (P == 0) return GS_OK;
    GS_REQUIRE(out != nullptr, "out must be non-null");
    const dim3 grid((unsigned)((P + ROUTE_THREADS - 1) / ROUTE_THREADS));
    if (mode == GS_ROUTE_INTERVAL) {
        GS_TIMED("route_bool_kernel", stream,
                 hipLaunchKernelGGL(route_bool_kernel<false>, grid, dim3(ROUTE_THREADS), 0, stream, P, G, means2D,
                                    radii, table, out));
    } else {
        GS_TIMED("route_bool_kernel", stream,
                 hipLaunchKernelGGL(route_bool_kernel<true>, grid, dim3(ROUTE_THREADS), 0, stream, P, G, means2D,
                                    radii, table, out));
    }
    GS_LAUNCH_CHECK("route_bool_kernel");
    return GS_OK;
}

extern "C" size_t gs_local2j_workspace_bytes(int P, int world_size)
{
    if (P < 0 || world_size < 1) return 0;
    const RoutePlan p = route_plan(P);
    return (size_t)p.NB * (size_t)world_size * sizeof(uint32_t);
}

extern "C" int gs_local2j_count(int mode, int P, int H, int W, int world_size, const float* means2D, const int* radii,
                                const int* table, int avoid_pixel_all2all, uint8_t* out_bool, int64_t* counts,
                                void* workspace, hipStream_t stream)
{
    gs::clear_error();
    RouteGeom G{};
    if (int rc = route_check(mode, P, H, W, world_size, means2D, radii, table, G)) return rc;
    G.avoid = avoid_pixel_all2all ? 1 : 0;
    GS_REQUIRE(world_size <= ROUTE_MAX_WORLD_IDS, "world_size %d exceeds %d for the id lists", world_size,
               ROUTE_MAX_WORLD_IDS);
    GS_REQUIRE((uint64_t)P * (uint64_t)world_size < 0xffffffffull, "P * world_size must be below 2^32");
    GS_REQUIRE(counts != nullptr && workspace != nullptr, "counts and workspace must be non-null");
    const RoutePlan p = route_plan(P);
    uint32_t* blk = static_cast<uint32_t*>(workspace);
    // with P == 0 the one block writes zero counts
    if (mode == GS_ROUTE_INTERVAL) {
        GS_TIMED("route_count_kernel", stream,
                 hipLaunchKernelGGL(route_count_kernel<false>, dim3(p.NB), dim3(ROUTE_THREADS), 0, stream, P, p.span,
                                    G, means2D, radii, table, out_bool, blk));
    } else {
        GS_TIMED("route_count_kernel", stream,
                 hipLaunchKernelGGL(route_count_kernel<true>, dim3(p.NB), dim3(ROUTE_THREADS), 0, stream, P, p.span,
                                    G, means2D, radii, table, out_bool, blk));
    }
    GS_LAUNCH_CHECK("route_count_kernel");
    GS_TIMED("route_scan_kernel", stream,
             hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(1024), 0, stream, p.NB, world_size, blk, counts));
    GS_LAUNCH_CHECK("route_scan_kernel");
    return GS_OK;
}

extern "C" int gs_local2j_write(int mode, int P, int H, int W, int world_size, const float* means2D, const int* radii,
                                const int* table, int avoid_pixel_all2all, const void* workspace, int64_t* ids,
                                int64_t n_ids, hipStream_t stream)
{
    gs::clear_error();
    RouteGeom G{};
    if (int rc = route_check(mode, P, H, W, world_size, means2D, radii, table, G)) return rc;
    G.avoid = avoid_pixel_all2all ? 1 : 0;
    GS_REQUIRE(world_size <= ROUTE_MAX_WORLD_IDS, "world_size %d exceeds %d for the id lists", world_size,
               ROUTE_MAX_WORLD_IDS);
    GS_REQUIRE(workspace != nullptr, "workspace must be non-null");
    GS_REQUIRE(n_ids >= 0 && (uint64_t)n_ids <= (uint64_t)P * (uint64_t)world_size, "n_ids out of range");
    if (P == 0 || n_ids == 0) return GS_OK;
    GS_REQUIRE(ids != nullptr, "ids must be non-null");
    const RoutePlan p = route_plan(P);
    const uint32_t* blk = static_cast<const uint32_t*>(workspace);
    if (mode == GS_ROUTE_INTERVAL) {
        GS_TIMED("route_write_kernel", stream,
                 hipLaunchKernelGGL(route_write_kernel<false>, dim3(p.NB), dim3(ROUTE_THREADS), 0, stream, P, p.span,
                                    G, means2D, radii, table, blk, ids, (uint32_t)n_ids));
    } else {
        GS_TIMED("route_write_kernel", stream,
                 hipLaunchKernelGGL(route_write_kernel<true>, dim3(p.NB), dim3(ROUTE_THREADS), 0, stream, P, p.span,
                                    G, means2D, radii, table, blk, ids, (uint32_t)n_ids));
    }
    GS_LAUNCH_CHECK("route_write_kernel");
    return GS_OK;
}

extern "C" int gs_move_rows(int64_t n_rows, const int64_t* src_rows, int64_t n_src_rows, const int64_t* dst_rows,
                            int64_t n_dst_rows, int n_fields, const gs_row_field* fields, int accumulate,
                            hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(n_rows >= 0 && n_src_rows >= 0 && n_dst_rows >= 0, "row counts must be >= 0");
    GS_REQUIRE(src_rows != nullptr || n_rows <= n_src_rows, "n_rows exceeds the source rows");
    GS_REQUIRE(dst_rows != nullptr || n_rows <= n_dst_rows, "n_rows exceeds the destination rows");
    GS_REQUIRE(n_fields >= 1 && n_fields <= MOVE_MAX_FIELDS, "n_fields must be in [1, %d]", MOVE_MAX_FIELDS);
    GS_REQUIRE(fields != nullptr, "fields must be non-null");
    MoveSpec S{};
    int cols = 0, n = 0;
    bool same_types = true, src_lin = true, dst_lin = true;
    const char* src0 = static_cast<const char*>(fields[0].src);
    const char* dst0 = static_cast<const char*>(fields[0].dst);
    for (int f = 0; f < n_fields; f++) {
        const gs_row_field& d = fields[f];
        GS_REQUIRE(d.width >= 1, "field %d: width must be >= 1", f);
        GS_REQUIRE(cols + d.width <= MOVE_MAX_COLS, "more than %d columns in one move", MOVE_MAX_COLS);
        GS_REQUIRE(d.src_type == GS_ROW_F32 || d.src_type == GS_ROW_I32, "field %d: bad src_type", f);
        GS_REQUIRE(d.dst_type == GS_ROW_F32 || d.dst_type == GS_ROW_I32, "field %d: bad dst_type", f);
        GS_REQUIRE(d.src_stride >= d.width && d.dst_stride >= d.width, "field %d: stride below width", f);
        GS_REQUIRE(n_rows == 0 || (d.src && d.dst), "field %d: null pointer", f);
        GS_REQUIRE(!(accumulate && d.dst_type != d.src_type), "field %d: accumulate needs equal types", f);
        same_types = same_types && d.src_type == d.dst_type;
        // one row-major buffer on a side: fields at consecutive columns, row stride = all columns
        src_lin = src_lin && static_cast<const char*>(d.src) == src0 + 4 * (int64_t)cols;
        dst_lin = dst_lin && static_cast<const char*>(d.dst) == dst0 + 4 * (int64_t)cols;
        for (int j = 0; j < d.width; j += 4) {
            const int w = d.width - j < 4 ? d.width - j : 4;
            S.f[n++] = MoveField{static_cast<const char*>(d.src) + 4 * (int64_t)j,
                                 static_cast<char*>(d.dst) + 4 * (int64_t)j, d.src_stride, d.dst_stride, w, cols + j,
                                 (uint32_t)(((1u << 20) + (uint32_t)w - 1) / (uint32_t)w), d.src_type == GS_ROW_I32,
                                 d.dst_type == GS_ROW_I32};
        }
        cols += d.width;
    }
    for (int f = 0; f < n_fields; f++) {
        src_lin = src_lin && fields[f].src_stride == cols;
        dst_lin = dst_lin && fields[f].dst_stride == cols;
    }
    S.n = n;
    S.cols = cols;
    S.src_linear = (src_lin && src_rows == nullptr && ((uintptr_t)src0 & 15) == 0)
                       ? reinterpret_cast<const uint32_t*>(src0)
                       : nullptr;
    // a linear copy out needs the staged words in the destination type: either
    // phase 1 converted them (gathered sources) or no field converts
    S.dst_linear = (dst_lin && dst_rows == nullptr && ((uintptr_t)dst0 & 15) == 0 && (!S.src_linear || same_types))
                       ? reinterpret_cast<uint32_t*>(const_cast<char*>(dst0))
                       : nullptr;
    if (n_rows == 0) return GS_OK;
    const int64_t blocks = (n_rows + MOVE_ROWS - 1) / MOVE_ROWS;
    GS_REQUIRE(blocks < 0x7fffffffll, "too many rows for one launch");
    GS_TIMED("move_rows_kernel", stream,
             hipLaunchKernelGGL(move_rows_kernel, dim3((unsigned)blocks), dim3(ROUTE_THREADS), 0, stream, n_rows,
                                src_rows, dst_rows, n_src_rows, n_dst_rows, S, accumulate ? 1 : 0));
    GS_LAUNCH_CHECK("move_rows_kernel");
    return GS_OK;
}
