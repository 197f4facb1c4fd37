// Binning (tile instances, per-tile depth sort, ranges) and the 16x16-tile
// alpha blend, forward and backward, for gfx950.
//
// Reference (BlitzGS submodule/diff-gaussian-rasterization_r):
//   updateTileTouched        cuda_rasterizer/rasterizer_impl.cu:258-282
//   InclusiveSum + R readback rasterizer_impl.cu:616-625
//   duplicateWithKeys        rasterizer_impl.cu:74-111
//   SortPairs (CUB)          rasterizer_impl.cu:643-652
//   identifyTileRanges       rasterizer_impl.cu:116-138
//   get_n_render / reduce_data_per_block  rasterizer_impl.cu:213-256
//   renderCUDA forward       cuda_rasterizer/forward.cu:263-413
//   renderCUDA backward      cuda_rasterizer/backward.cu:324-530
//
// Binning design.  The reference duplicates every Gaussian/tile instance with
// a 64-bit (tile | depth) key in Gaussian order and radix-sorts all R pairs
// globally (about six passes over 12 bytes per instance).  Here the tiles are
// bucketed first and each bucket is sorted on chip:
//   1. count   : each block takes a chunk of Gaussians and histograms their
//                tile instances in LDS (one counter per local tile), then
//                writes its histogram row.
//   2. scan    : a column scan over the chunk rows gives each block a private
//                write cursor per tile; a scan over tiles gives tile offsets
//                (these are the reference's ranges).
//   3. scatter : each block re-walks its chunk and appends (depth bits, id)
//                to its cursors (LDS atomics only).
//   4. sort    : one block per tile sorts its bucket by (depth bits, id) in
//                LDS (bitonic) and writes the sorted ids and the
//                (tile << 32 | depth bits) keys.
// Sorting each bucket by (depth bits, Gaussian id) yields exactly the order
// of a stable sort of the reference's duplicated keys, so the sorted arrays
// and the ranges are bit-identical to the reference algorithm's.
// When more than LDS_TILES tiles are local, steps 1 and 3 use global atomics
// instead of the LDS histogram (same result after step 4).
//
// Blend design.  One wave64 per 8x8 quadrant of a tile, one pixel per lane,
// no block-wide barriers: a wave stages batches of 64 Gaussians in its own
// LDS slots and stops as soon as all of its 64 pixels are saturated.  The
// backward walks each quadrant's list back to front from the largest last
// contributor of its pixels, reduces every Gaussian's eleven gradient terms
// across the wave with DPP row shifts / row broadcasts, and issues one set of
// global atomics per (wave, Gaussian) instead of one per (pixel, Gaussian).
#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {

constexpr int LDS_TILES = 16384;     // local tiles histogrammed in LDS (64 KB)
constexpr int BIN_THREADS = 512;
constexpr int MAX_CHUNKS = 512;
constexpr int SORT_CAP = 4096;       // bucket size sorted entirely in LDS
constexpr int SORT_THREADS = 512;
constexpr int BIG_SORT_THREADS = 1024;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct GeomLayout {
    int T, NC, CH;
    size_t loc_map, tile_of_local, meta, hist, tile_count, tile_start, cursor, total;
};

GeomLayout geom_layout(int P, int W, int H)
{
    GeomLayout g;
    const int gx = (W + 15) / 16, gy = (H + 15) / 16;
    g.T = gx * gy;
    long nc = ((long)P + 2047) / 2048;
    if (nc < 1) nc = 1;
    if (nc > MAX_CHUNKS) nc = MAX_CHUNKS;
    g.NC = (int)nc;
    g.CH = (int)(((long)P + g.NC - 1) / g.NC);
    size_t o = 0;
    g.loc_map = o; o = align256(o + sizeof(int) * (size_t)g.T);
    g.tile_of_local = o; o = align256(o + sizeof(int) * (size_t)g.T);
    g.meta = o; o = align256(o + 64);
    g.hist = o; o = align256(o + sizeof(uint32_t) * (size_t)g.NC * (size_t)(g.T < LDS_TILES ? g.T : LDS_TILES));
    g.tile_count = o; o = align256(o + sizeof(uint32_t) * (size_t)g.T);
    g.tile_start = o; o = align256(o + sizeof(uint32_t) * (size_t)g.T);
    g.cursor = o; o = align256(o + sizeof(uint32_t) * (size_t)g.T);
    g.total = o;
    return g;
}

struct ImgLayout {
    size_t ranges, final_T, n_contrib, n_contrib2loss, total;
};

ImgLayout img_layout(int W, int H)
{
    ImgLayout l;
    const int gx = (W + 15) / 16, gy = (H + 15) / 16;
    const size_t N = (size_t)W * H;
    size_t o = 0;
    l.ranges = o; o = align256(o + sizeof(uint32_t) * 2 * (size_t)gx * gy);
    l.final_T = o; o = align256(o + sizeof(float) * N);
    l.n_contrib = o; o = align256(o + sizeof(uint32_t) * N);
    l.n_contrib2loss = o; o = align256(o + sizeof(uint32_t) * N);
    l.total = o;
    return l;
}

struct BinLayout {
    size_t sortkey, point_list, keys, total;
};

BinLayout bin_layout(int64_t R)
{
    BinLayout b;
    size_t o = 0;
    b.sortkey = o; o = align256(o + sizeof(uint64_t) * (size_t)R);
    b.point_list = o; o = align256(o + sizeof(uint32_t) * (size_t)R);
    b.keys = o; o = align256(o + sizeof(uint64_t) * (size_t)R);
    b.total = o < 256 ? 256 : o;
    return b;
}

template <typename T>
T* at(void* base, size_t off) { return reinterpret_cast<T*>(static_cast<char*>(base) + off); }
template <typename T>
const T* at(const void* base, size_t off) { return reinterpret_cast<const T*>(static_cast<const char*>(base) + off); }

// ---------------------------------------------------------------- scans

// Exclusive scan of one value per thread over a 1024-thread block; returns
// the prefix and writes the block total to *total (all threads).
__device__ __forceinline__ uint32_t block_excl_scan_1024(uint32_t v, uint32_t* s_wave, uint32_t* total)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) s_wave[wid] = x;
    __syncthreads();
    if (wid == 0) {
        uint32_t w = lane < 16 ? s_wave[lane] : 0;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const uint32_t y = __shfl_up(w, off, 64);
            if (lane >= off) w += y;
        }
        if (lane < 16) s_wave[16 + lane] = w;
    }
    __syncthreads();
    const uint32_t wbase = wid == 0 ? 0 : s_wave[16 + wid - 1];
    *total = s_wave[31];
    __syncthreads();
    return wbase + x - v;
}

// compute_locally -> local tile numbering; clears the per-tile counters
__global__ __launch_bounds__(1024) void localmap_kernel(int T, const uint8_t* __restrict__ cl,
                                                        int* __restrict__ loc_map, int* __restrict__ tile_of_local,
                                                        uint32_t* __restrict__ tile_count, uint32_t* __restrict__ meta)
{
    __shared__ uint32_t s_wave[32];
    uint32_t base = 0;
    for (int t0 = 0; t0 < T; t0 += 1024) {
        const int t = t0 + threadIdx.x;
        const uint32_t f = (t < T && cl[t]) ? 1u : 0u;
        uint32_t tot;
        const uint32_t pre = block_excl_scan_1024(f, s_wave, &tot);
        if (t < T) {
            loc_map[t] = f ? (int)(base + pre) : -1;
            if (f) tile_of_local[base + pre] = t;
            tile_count[t] = 0;
        }
        base += tot;
    }
    if (threadIdx.x == 0) meta[0] = base;
}

// ------------------------------------------------------------- counting

__global__ __launch_bounds__(BIN_THREADS) void count_kernel(
    int P, int CH, unsigned gx, unsigned gy, const float2* __restrict__ means2D, const int* __restrict__ radii,
    const int* __restrict__ loc_map, const uint32_t* __restrict__ meta, uint32_t* __restrict__ hist,
    uint32_t* __restrict__ tile_count)
{
    __shared__ uint32_t s_hist[LDS_TILES];
    const int TL = (int)meta[0];
    const bool lds = TL <= LDS_TILES;
    const int c = blockIdx.x;
    if (lds) {
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) s_hist[l] = 0;
        __syncthreads();
    }
    const int i0 = c * CH;
    const int i1 = min(P, i0 + CH);
    for (int i = i0 + threadIdx.x; i < i1; i += BIN_THREADS) {
        const int r = radii[i];
        if (r <= 0) continue;
        const float2 p = means2D[i];
        unsigned x0, y0, x1, y1;
        gs::rect_int(p.x, p.y, r, gx, gy, x0, y0, x1, y1);
        for (unsigned y = y0; y < y1; y++)
            for (unsigned x = x0; x < x1; x++) {
                const int l = loc_map[y * gx + x];
                if (l >= 0) {
                    if (lds) atomicAdd(&s_hist[l], 1u);
                    else atomicAdd(&tile_count[l], 1u);
                }
            }
    }
    if (lds) {
        __syncthreads();
        uint32_t* row = hist + (size_t)c * TL;
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) row[l] = s_hist[l];
    }
}

// per local tile: exclusive prefix of the chunk histograms (in place) and total
__global__ __launch_bounds__(256) void colscan_kernel(int NC, const uint32_t* __restrict__ meta,
                                                      uint32_t* __restrict__ hist, uint32_t* __restrict__ tile_count)
{
    const int TL = (int)meta[0];
    if (TL > LDS_TILES) return;
    const int l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= TL) return;
    uint32_t run = 0;
    for (int c = 0; c < NC; c++) {
        uint32_t* p = hist + (size_t)c * TL + l;
        const uint32_t v = *p;
        *p = run;
        run += v;
    }
    tile_count[l] = run;
}

// exclusive scan over local tiles -> tile_start, R -> meta[2..3]
__global__ __launch_bounds__(1024) void tilescan_kernel(uint32_t* __restrict__ meta, const uint32_t* __restrict__ tile_count,
                                                        uint32_t* __restrict__ tile_start, uint32_t* __restrict__ cursor)
{
    __shared__ uint32_t s_wave[32];
    const int TL = (int)meta[0];
    uint64_t base = 0;
    for (int t0 = 0; t0 < TL; t0 += 1024) {
        const int l = t0 + threadIdx.x;
        const uint32_t v = l < TL ? tile_count[l] : 0u;
        uint32_t tot;
        const uint32_t pre = block_excl_scan_1024(v, s_wave, &tot);
        if (l < TL) {
            tile_start[l] = (uint32_t)(base + pre);
            cursor[l] = (uint32_t)(base + pre);
        }
        base += tot;
    }
    if (threadIdx.x == 0) {
        meta[2] = (uint32_t)(base & 0xffffffffu);
        meta[3] = (uint32_t)(base >> 32);
    }
}

// per tile: ranges, n_render; clears the per-tile blend statistics
__global__ __launch_bounds__(256) void ranges_kernel(int T, const int* __restrict__ loc_map,
                                                     const uint32_t* __restrict__ tile_count,
                                                     const uint32_t* __restrict__ tile_start, uint2* __restrict__ ranges,
                                                     int32_t* __restrict__ n_render, int32_t* __restrict__ n_consider,
                                                     int32_t* __restrict__ n_contrib)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const int l = loc_map[t];
    uint32_t cnt = 0, s = 0;
    if (l >= 0) { cnt = tile_count[l]; s = tile_start[l]; }
    ranges[t] = cnt ? make_uint2(s, s + cnt) : make_uint2(0u, 0u);
    n_render[t] = (int32_t)cnt;
    n_consider[t] = 0;
    n_contrib[t] = 0;
}

// ------------------------------------------------------------- scatter

__global__ __launch_bounds__(BIN_THREADS) void scatter_kernel(
    int P, int CH, unsigned gx, unsigned gy, const float2* __restrict__ means2D, const float* __restrict__ depths,
    const int* __restrict__ radii, const int* __restrict__ loc_map, const uint32_t* __restrict__ meta,
    const uint32_t* __restrict__ hist, const uint32_t* __restrict__ tile_start, uint32_t* __restrict__ cursor,
    uint64_t* __restrict__ sortkey)
{
    __shared__ uint32_t s_cur[LDS_TILES];
    const int TL = (int)meta[0];
    const bool lds = TL <= LDS_TILES;
    const int c = blockIdx.x;
    if (lds) {
        const uint32_t* row = hist + (size_t)c * TL;
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) s_cur[l] = tile_start[l] + row[l];
        __syncthreads();
    }
    const int i0 = c * CH;
    const int i1 = min(P, i0 + CH);
    for (int i = i0 + threadIdx.x; i < i1; i += BIN_THREADS) {
        const int r = radii[i];
        if (r <= 0) continue;
        const float2 p = means2D[i];
        const uint64_t key = ((uint64_t)gs::f2u(depths[i]) << 32) | (uint32_t)i;
        unsigned x0, y0, x1, y1;
        gs::rect_int(p.x, p.y, r, gx, gy, x0, y0, x1, y1);
        for (unsigned y = y0; y < y1; y++)
            for (unsigned x = x0; x < x1; x++) {
                const int l = loc_map[y * gx + x];
                if (l >= 0) {
                    const uint32_t pos = lds ? atomicAdd(&s_cur[l], 1u) : atomicAdd(&cursor[l], 1u);
                    sortkey[pos] = key;
                }
            }
    }
}

// ------------------------------------------------------- per-tile sort

__device__ __forceinline__ void cswap(uint64_t* a, uint64_t* b)
{
    const uint64_t x = *a, y = *b;
    if (y < x) { *a = y; *b = x; }
}

// Bitonic sort (all comparators put the minimum at the lower index, so a
// virtual +inf tail beyond n needs no storage) of s[0..N), N = pow2 >= n.
template <int NT>
__device__ __forceinline__ void bitonic_lds(uint64_t* s, int N)
{
    for (int k = 2; k <= N; k <<= 1) {
        const int hk = k >> 1;
        for (int p = threadIdx.x; p < (N >> 1); p += NT) {
            const int blk = p / hk, off = p - blk * hk;
            cswap(&s[blk * k + off], &s[blk * k + k - 1 - off]);
        }
        __syncthreads();
        for (int j = k >> 2; j >= 1; j >>= 1) {
            for (int p = threadIdx.x; p < (N >> 1); p += NT) {
                const int blk = p / j, off = p - blk * j;
                const int a = blk * 2 * j + off;
                cswap(&s[a], &s[a + j]);
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ void write_sorted(uint32_t tile, uint32_t start, int n, const uint64_t* src,
                                             uint32_t* __restrict__ point_list, uint64_t* __restrict__ keys, int nt)
{
    for (int i = threadIdx.x; i < n; i += nt) {
        const uint64_t k = src[i];
        point_list[start + i] = (uint32_t)k;
        keys[start + i] = ((uint64_t)tile << 32) | (k >> 32);
    }
}

__global__ __launch_bounds__(SORT_THREADS) void tilesort_kernel(
    const uint32_t* __restrict__ meta, const int* __restrict__ tile_of_local, const uint32_t* __restrict__ tile_count,
    const uint32_t* __restrict__ tile_start, const uint64_t* __restrict__ sortkey, uint32_t* __restrict__ point_list,
    uint64_t* __restrict__ keys)
{
    __shared__ uint64_t s[SORT_CAP];
    const int l = blockIdx.x;
    if (l >= (int)meta[0]) return;
    const int n = (int)tile_count[l];
    if (n == 0 || n > SORT_CAP) return;
    const uint32_t start = tile_start[l];
    int N = 1;
    while (N < n) N <<= 1;
    for (int i = threadIdx.x; i < N; i += SORT_THREADS) s[i] = i < n ? sortkey[start + i] : ~(uint64_t)0;
    __syncthreads();
    bitonic_lds<SORT_THREADS>(s, N);
    write_sorted((uint32_t)tile_of_local[l], start, n, s, point_list, keys, SORT_THREADS);
}

// Buckets larger than SORT_CAP: the same network in global memory (in place)
__global__ __launch_bounds__(BIG_SORT_THREADS) void tilesort_big_kernel(
    const uint32_t* __restrict__ meta, const int* __restrict__ tile_of_local, const uint32_t* __restrict__ tile_count,
    const uint32_t* __restrict__ tile_start, uint64_t* __restrict__ sortkey, uint32_t* __restrict__ point_list,
    uint64_t* __restrict__ keys)
{
    const int l = blockIdx.x;
    if (l >= (int)meta[0]) return;
    const int n = (int)tile_count[l];
    if (n <= SORT_CAP) return;
    const uint32_t start = tile_start[l];
    uint64_t* s = sortkey + start;
    int N = 1;
    while (N < n) N <<= 1;
    for (int k = 2; k <= N; k <<= 1) {
        const int hk = k >> 1;
        for (int p = threadIdx.x; p < (N >> 1); p += BIG_SORT_THREADS) {
            const int blk = p / hk, off = p - blk * hk;
            const int a = blk * k + off, b = blk * k + k - 1 - off;
            if (b < n) cswap(&s[a], &s[b]);
        }
        __syncthreads();
        for (int j = k >> 2; j >= 1; j >>= 1) {
            for (int p = threadIdx.x; p < (N >> 1); p += BIG_SORT_THREADS) {
                const int blk = p / j, off = p - blk * j;
                const int a = blk * 2 * j + off;
                if (a + j < n) cswap(&s[a], &s[a + j]);
            }
            __syncthreads();
        }
    }
    write_sorted((uint32_t)tile_of_local[l], start, n, s, point_list, keys, BIG_SORT_THREADS);
}

// ------------------------------------------------------------- blend

// block b -> (tile, quadrant): the four quadrant waves of a tile land on the
// same XCD (workgroups are dispatched to the 8 XCDs round-robin)
__device__ __forceinline__ void block_to_tile(unsigned b, unsigned& tile, unsigned& quad)
{
    const unsigned xcd = b & 7u, slot = b >> 3;
    quad = slot & 3u;
    tile = (slot >> 2) * 8u + xcd;
}

__global__ __launch_bounds__(64) void render_fwd_kernel(
    int W, int H, unsigned gx, unsigned T, const uint2* __restrict__ ranges, const uint32_t* __restrict__ point_list,
    const float2* __restrict__ means2D, const float4* __restrict__ conic_opacity, const float* __restrict__ rgb,
    const uint8_t* __restrict__ cl, const float* __restrict__ bg, float* __restrict__ out_color,
    float* __restrict__ final_T, uint32_t* __restrict__ n_contrib_px, uint32_t* __restrict__ n_contrib2loss_px,
    int32_t* __restrict__ out_observe, int32_t* __restrict__ n_consider, int32_t* __restrict__ n_contrib_tile)
{
    unsigned tile, quad;
    block_to_tile(blockIdx.x, tile, quad);
    if (tile >= T) return;
    const int lane = threadIdx.x;
    const int px = (int)(tile % gx) * 16 + (int)(quad & 1u) * 8 + (lane & 7);
    const int py = (int)(tile / gx) * 16 + (int)(quad >> 1) * 8 + (lane >> 3);
    const bool inside = px < W && py < H;
    const size_t pid = (size_t)py * W + px;
    const size_t HW = (size_t)H * W;
    if (!cl[tile]) {
        if (inside) {
            out_color[pid] = 0.f; out_color[HW + pid] = 0.f; out_color[2 * HW + pid] = 0.f;
            final_T[pid] = 0.f; n_contrib_px[pid] = 0; n_contrib2loss_px[pid] = 0;
        }
        return;
    }
    __shared__ float4 s_a[64];   // x, y, -a/2, -b
    __shared__ float4 s_b[64];   // -c/2, opacity, r, g
    __shared__ float2 s_c[64];   // blue, id bits

    const uint2 range = ranges[tile];
    const int n = (int)(range.y - range.x);
    const float pxf = (float)px, pyf = (float)py;
    const float alpha_min = 1.0f / 255.0f;
    float T_ = 1.0f, C0 = 0.f, C1 = 0.f, C2 = 0.f;
    uint32_t contributor = 0, last = 0, n2l = 0;
    bool done = !inside;

    for (int base = 0; base < n; base += 64) {
        if (gs::ballot(!done) == 0) break;
        const int k = base + lane;
        if (k < n) {
            const uint32_t id = point_list[range.x + k];
            const float2 xy = means2D[id];
            const float4 co = conic_opacity[id];
            s_a[lane] = make_float4(xy.x, xy.y, -0.5f * co.x, -co.y);
            s_b[lane] = make_float4(-0.5f * co.z, co.w, rgb[3 * id], rgb[3 * id + 1]);
            s_c[lane] = make_float2(rgb[3 * id + 2], __uint_as_float(id));
        }
        __syncthreads();
        const int cnt = min(64, n - base);
        for (int j = 0; j < cnt; j++) {
            if (gs::ballot(!done) == 0) break;
            const float4 A = s_a[j];
            const float4 B = s_b[j];
            const float2 Cc = s_c[j];
            bool blend = false, observe = false;
            if (!done) {
                contributor++;
                const float dx = A.x - pxf, dy = A.y - pyf;
                const float power = gs::power_of(A.z, A.w, B.x, dx, dy);
                const float alpha = __builtin_fminf(0.99f, B.y * gs::expf_nonpos(power));
                if (!(power > 0.0f) && !(alpha < alpha_min)) {
                    const float test_T = T_ * (1.0f - alpha);
                    if (test_T < 0.0001f) {
                        done = true;
                    } else {
                        blend = true;
                        observe = T_ > 0.5f;
                        n2l++;
                        const float wgt = alpha * T_;
                        C0 = __builtin_fmaf(B.z, wgt, C0);
                        C1 = __builtin_fmaf(B.w, wgt, C1);
                        C2 = __builtin_fmaf(Cc.x, wgt, C2);
                        T_ = test_T;
                        last = contributor;
                    }
                }
            }
            (void)blend;
            const uint64_t m = gs::ballot(observe);
            if (m != 0 && lane == (int)__builtin_ctzll(m))
                atomicAdd(&out_observe[__float_as_uint(Cc.y)], (int)__builtin_popcountll(m));
        }
        __syncthreads();
    }

    if (inside) {
        final_T[pid] = T_;
        n_contrib_px[pid] = last;
        n_contrib2loss_px[pid] = n2l;
        out_color[pid] = __builtin_fmaf(T_, bg[0], C0);
        out_color[HW + pid] = __builtin_fmaf(T_, bg[1], C1);
        out_color[2 * HW + pid] = __builtin_fmaf(T_, bg[2], C2);
    }
    const int s_last = gs::wave_sum_i(inside ? (int)last : 0);
    const int s_n2l = gs::wave_sum_i(inside ? (int)n2l : 0);
    if (lane == 0) {
        if (s_last) atomicAdd(&n_consider[tile], s_last);
        if (s_n2l) atomicAdd(&n_contrib_tile[tile], s_n2l);
    }
}

__global__ __launch_bounds__(256) void zero_i32_kernel(int n, int32_t* __restrict__ p)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

__global__ __launch_bounds__(256) void zero_grads_kernel(int P, int m2d_stride, float* __restrict__ g_m2d,
                                                         float* __restrict__ g_m2d_abs, float4* __restrict__ g_con,
                                                         float* __restrict__ g_col)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= P) return;
    for (int k = 0; k < m2d_stride; k++) g_m2d[(size_t)i * m2d_stride + k] = 0.f;
    g_m2d_abs[3 * (size_t)i] = 0.f; g_m2d_abs[3 * (size_t)i + 1] = 0.f; g_m2d_abs[3 * (size_t)i + 2] = 0.f;
    g_con[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    g_col[3 * (size_t)i] = 0.f; g_col[3 * (size_t)i + 1] = 0.f; g_col[3 * (size_t)i + 2] = 0.f;
}

__global__ __launch_bounds__(64) void render_bwd_kernel(
    int W, int H, unsigned gx, unsigned T, const uint2* __restrict__ ranges, const uint32_t* __restrict__ point_list,
    const float2* __restrict__ means2D, const float4* __restrict__ conic_opacity, const float* __restrict__ rgb,
    const uint8_t* __restrict__ cl, const float* __restrict__ bg, const float* __restrict__ final_T,
    const uint32_t* __restrict__ n_contrib_px, const float* __restrict__ dL_dpixels, float* __restrict__ g_m2d,
    int m2d_stride, float* __restrict__ g_m2d_abs, float* __restrict__ g_con, float* __restrict__ g_col)
{
    unsigned tile, quad;
    block_to_tile(blockIdx.x, tile, quad);
    if (tile >= T || !cl[tile]) return;
    const int lane = threadIdx.x;
    const int px = (int)(tile % gx) * 16 + (int)(quad & 1u) * 8 + (lane & 7);
    const int py = (int)(tile / gx) * 16 + (int)(quad >> 1) * 8 + (lane >> 3);
    const bool inside = px < W && py < H;
    const size_t pid = (size_t)py * W + px;
    const size_t HW = (size_t)H * W;

    const float T_final = inside ? final_T[pid] : 0.f;
    const int last = inside ? (int)n_contrib_px[pid] : 0;
    float dp0 = 0.f, dp1 = 0.f, dp2 = 0.f;
    if (inside) { dp0 = dL_dpixels[pid]; dp1 = dL_dpixels[HW + pid]; dp2 = dL_dpixels[2 * HW + pid]; }
    const int maxlast = gs::wave_max_i(last);
    if (maxlast == 0) return;

    __shared__ float4 s_a[64];   // x, y, -a/2, -b
    __shared__ float4 s_b[64];   // -c/2, opacity, r, g
    __shared__ float2 s_c[64];   // blue, id bits

    const uint2 range = ranges[tile];
    const float pxf = (float)px, pyf = (float)py;
    const float alpha_min = 1.0f / 255.0f;
    const float ddelx_dx = 0.5f * (float)W, ddely_dy = 0.5f * (float)H;
    const float bg_dot = bg[0] * dp0 + bg[1] * dp1 + bg[2] * dp2;
    float T_ = T_final;
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f;
    float lc0 = 0.f, lc1 = 0.f, lc2 = 0.f, last_alpha = 0.f;

    // walk positions maxlast-1 .. 0 of the tile's list, back to front
    for (int top = maxlast; top > 0; top -= 64) {
        const int cnt = min(64, top);
        if (lane < cnt) {
            const uint32_t id = point_list[range.x + top - 1 - lane];
            const float2 xy = means2D[id];
            const float4 co = conic_opacity[id];
            s_a[lane] = make_float4(xy.x, xy.y, -0.5f * co.x, -co.y);
            s_b[lane] = make_float4(-0.5f * co.z, co.w, rgb[3 * id], rgb[3 * id + 1]);
            s_c[lane] = make_float2(rgb[3 * id + 2], __uint_as_float(id));
        }
        __syncthreads();
        for (int j = 0; j < cnt; j++) {
            const int ci = top - 1 - j;   // position in the tile's list
            const float4 A = s_a[j];
            const float4 B = s_b[j];
            const float2 Cc = s_c[j];
            float gmx = 0.f, gmy = 0.f, gca = 0.f, gcb = 0.f, gcc = 0.f, gop = 0.f;
            float gc0 = 0.f, gc1 = 0.f, gc2 = 0.f;
            bool valid = false;
            if (ci < last) {
                const float dx = A.x - pxf, dy = A.y - pyf;
                const float power = gs::power_of(A.z, A.w, B.x, dx, dy);
                const float G = gs::expf_nonpos(power);
                const float alpha = __builtin_fminf(0.99f, B.y * G);
                if (!(power > 0.0f) && !(alpha < alpha_min)) {
                    valid = true;
                    const float one_m = 1.f - alpha;
                    T_ = T_ / one_m;
                    const float dchannel_dcolor = alpha * T_;
                    acc0 = last_alpha * lc0 + (1.f - last_alpha) * acc0;
                    acc1 = last_alpha * lc1 + (1.f - last_alpha) * acc1;
                    acc2 = last_alpha * lc2 + (1.f - last_alpha) * acc2;
                    lc0 = B.z; lc1 = B.w; lc2 = Cc.x;
                    float dL_dalpha = (B.z - acc0) * dp0 + (B.w - acc1) * dp1 + (Cc.x - acc2) * dp2;
                    gc0 = dchannel_dcolor * dp0;
                    gc1 = dchannel_dcolor * dp1;
                    gc2 = dchannel_dcolor * dp2;
                    dL_dalpha *= T_;
                    last_alpha = alpha;
                    dL_dalpha += (-T_final / one_m) * bg_dot;
                    const float a = -2.0f * A.z, b = -A.w, c = -2.0f * B.x;
                    const float dL_dG = B.y * dL_dalpha;
                    const float gdx = G * dx, gdy = G * dy;
                    const float dG_ddelx = -gdx * a - gdy * b;
                    const float dG_ddely = -gdy * c - gdx * b;
                    gmx = dL_dG * dG_ddelx * ddelx_dx;
                    gmy = dL_dG * dG_ddely * ddely_dy;
                    gca = -0.5f * gdx * dx * dL_dG;
                    gcb = -0.5f * gdx * dy * dL_dG;
                    gcc = -0.5f * gdy * dy * dL_dG;
                    gop = G * dL_dalpha;
                }
            }
            if (gs::ballot(valid) == 0) continue;
            const float s_mx = gs::wave_sum(gmx), s_my = gs::wave_sum(gmy);
            const float s_ax = gs::wave_sum(__builtin_fabsf(gmx)), s_ay = gs::wave_sum(__builtin_fabsf(gmy));
            const float s_ca = gs::wave_sum(gca), s_cb = gs::wave_sum(gcb), s_cc = gs::wave_sum(gcc);
            const float s_op = gs::wave_sum(gop);
            const float s_c0 = gs::wave_sum(gc0), s_c1 = gs::wave_sum(gc1), s_c2 = gs::wave_sum(gc2);
            // eleven atomics, one lane each, in one instruction
            const uint32_t id = __float_as_uint(Cc.y);
            float v = 0.f;
            float* dst = nullptr;
            switch (lane) {
                case 0: v = s_mx; dst = g_m2d + (size_t)id * m2d_stride; break;
                case 1: v = s_my; dst = g_m2d + (size_t)id * m2d_stride + 1; break;
                case 2: v = s_ax; dst = g_m2d_abs + 3 * (size_t)id; break;
                case 3: v = s_ay; dst = g_m2d_abs + 3 * (size_t)id + 1; break;
                case 4: v = s_ca; dst = g_con + 4 * (size_t)id; break;
                case 5: v = s_cb; dst = g_con + 4 * (size_t)id + 1; break;
                case 6: v = s_cc; dst = g_con + 4 * (size_t)id + 2; break;
                case 7: v = s_op; dst = g_con + 4 * (size_t)id + 3; break;
                case 8: v = s_c0; dst = g_col + 3 * (size_t)id; break;
                case 9: v = s_c1; dst = g_col + 3 * (size_t)id + 1; break;
                case 10: v = s_c2; dst = g_col + 3 * (size_t)id + 2; break;
                default: break;
            }
            if (dst != nullptr && v != 0.f) atomicAdd(dst, v);
        }
        __syncthreads();
    }
}

}  // namespace

// ====================================================================== C ABI

extern "C" size_t gs_render_geom_bytes(int P, int W, int H) { return geom_layout(P, W, H).total; }
extern "C" size_t gs_render_binning_bytes(int64_t R) { return bin_layout(R).total; }
extern "C" size_t gs_render_img_bytes(int W, int H) { return img_layout(W, H).total; }

extern "C" int gs_render_buffer_views(int64_t R, int W, int H, void* binning, void* img, uint32_t** point_list,
                                      uint64_t** point_list_keys, uint32_t** ranges, float** final_T,
                                      uint32_t** n_contrib, uint32_t** n_contrib2loss)
{
    const BinLayout b = bin_layout(R);
    const ImgLayout l = img_layout(W, H);
    if (point_list) *point_list = at<uint32_t>(binning, b.point_list);
    if (point_list_keys) *point_list_keys = at<uint64_t>(binning, b.keys);
    if (ranges) *ranges = at<uint32_t>(img, l.ranges);
    if (final_T) *final_T = at<float>(img, l.final_T);
    if (n_contrib) *n_contrib = at<uint32_t>(img, l.n_contrib);
    if (n_contrib2loss) *n_contrib2loss = at<uint32_t>(img, l.n_contrib2loss);
    return GS_OK;
}

extern "C" int gs_render_forward_count(int P, int W, int H, const float* means2D, const int* radii,
                                       const uint8_t* compute_locally, void* geom, int64_t* num_rendered,
                                       hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0 && W > 0 && H > 0, "invalid sizes P=%d W=%d H=%d", P, W, H);
    GS_REQUIRE(geom != nullptr && num_rendered != nullptr, "geom and num_rendered must be non-null");
    const GeomLayout g = geom_layout(P, W, H);
    const unsigned gx = (unsigned)((W + 15) / 16), gy = (unsigned)((H + 15) / 16);
    int* loc_map = at<int>(geom, g.loc_map);
    int* tile_of_local = at<int>(geom, g.tile_of_local);
    uint32_t* meta = at<uint32_t>(geom, g.meta);
    uint32_t* hist = at<uint32_t>(geom, g.hist);
    uint32_t* tile_count = at<uint32_t>(geom, g.tile_count);
    uint32_t* tile_start = at<uint32_t>(geom, g.tile_start);
    uint32_t* cursor = at<uint32_t>(geom, g.cursor);

    GS_TIMED("localmap_kernel", stream, hipLaunchKernelGGL(localmap_kernel, dim3(1), dim3(1024), 0, stream, g.T, compute_locally, loc_map,
                       tile_of_local, tile_count, meta));
    GS_LAUNCH_CHECK("localmap_kernel");
    if (P > 0) {
        GS_TIMED("count_kernel", stream, hipLaunchKernelGGL(count_kernel, dim3(g.NC), dim3(BIN_THREADS), 0, stream, P, g.CH, gx, gy,
                           reinterpret_cast<const float2*>(means2D), radii, loc_map, meta, hist, tile_count));
        GS_LAUNCH_CHECK("count_kernel");
        GS_TIMED("colscan_kernel", stream, hipLaunchKernelGGL(colscan_kernel, dim3(gs_div_up((size_t)(g.T < LDS_TILES ? g.T : LDS_TILES), 256)),
                           dim3(256), 0, stream, g.NC, meta, hist, tile_count));
        GS_LAUNCH_CHECK("colscan_kernel");
    }
    GS_TIMED("tilescan_kernel", stream, hipLaunchKernelGGL(tilescan_kernel, dim3(1), dim3(1024), 0, stream, meta, tile_count, tile_start, cursor));
    GS_LAUNCH_CHECK("tilescan_kernel");
    uint32_t hR[2] = {0, 0};
    GS_HIP(hipMemcpyAsync(hR, meta + 2, sizeof(hR), hipMemcpyDeviceToHost, stream));
    GS_HIP(hipStreamSynchronize(stream));
    const uint64_t R = (uint64_t)hR[0] | ((uint64_t)hR[1] << 32);
    if (R > 0xffffffffull) {
        gs::set_error("number of tile instances %llu exceeds 2^32-1", (unsigned long long)R);
        return GS_ERR_SIZE;
    }
    *num_rendered = (int64_t)R;
    return GS_OK;
}

extern "C" int gs_render_forward(int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                                 const float* depths, const int* radii, const float* conic_opacity, const float* rgb,
                                 const uint8_t* compute_locally, void* geom, void* binning, void* img,
                                 float* out_color, int32_t* n_render, int32_t* n_consider, int32_t* n_contrib,
                                 int32_t* out_observe, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0 && W > 0 && H > 0 && R >= 0, "invalid sizes P=%d W=%d H=%d R=%lld", P, W, H, (long long)R);
    GS_REQUIRE(((uintptr_t)conic_opacity & 15) == 0 && ((uintptr_t)means2D & 7) == 0,
               "conic_opacity must be 16-byte and means2D 8-byte aligned");
    const GeomLayout g = geom_layout(P, W, H);
    const ImgLayout il = img_layout(W, H);
    const BinLayout bl = bin_layout(R);
    const unsigned gx = (unsigned)((W + 15) / 16), gy = (unsigned)((H + 15) / 16);
    int* loc_map = at<int>(geom, g.loc_map);
    int* tile_of_local = at<int>(geom, g.tile_of_local);
    uint32_t* meta = at<uint32_t>(geom, g.meta);
    uint32_t* hist = at<uint32_t>(geom, g.hist);
    uint32_t* tile_count = at<uint32_t>(geom, g.tile_count);
    uint32_t* tile_start = at<uint32_t>(geom, g.tile_start);
    uint32_t* cursor = at<uint32_t>(geom, g.cursor);
    uint2* ranges = at<uint2>(img, il.ranges);
    uint64_t* sortkey = at<uint64_t>(binning, bl.sortkey);
    uint32_t* point_list = at<uint32_t>(binning, bl.point_list);
    uint64_t* keys = at<uint64_t>(binning, bl.keys);

    const unsigned T = (unsigned)g.T;
    GS_TIMED("ranges_kernel", stream, hipLaunchKernelGGL(ranges_kernel, dim3(gs_div_up(T, 256)), dim3(256), 0, stream, g.T, loc_map, tile_count,
                       tile_start, ranges, n_render, n_consider, n_contrib));
    GS_LAUNCH_CHECK("ranges_kernel");
    if (P > 0) {
        GS_TIMED("zero_i32_kernel", stream, hipLaunchKernelGGL(zero_i32_kernel, dim3(gs_div_up((size_t)P, 256)), dim3(256), 0, stream, P, out_observe));
        GS_LAUNCH_CHECK("zero_i32_kernel");
    }
    if (R > 0) {
        GS_TIMED("scatter_kernel", stream, hipLaunchKernelGGL(scatter_kernel, dim3(g.NC), dim3(BIN_THREADS), 0, stream, P, g.CH, gx, gy,
                           reinterpret_cast<const float2*>(means2D), depths, radii, loc_map, meta, hist,
                           tile_start, cursor, sortkey));
        GS_LAUNCH_CHECK("scatter_kernel");
        GS_TIMED("tilesort_kernel", stream, hipLaunchKernelGGL(tilesort_kernel, dim3(T), dim3(SORT_THREADS), 0, stream, meta, tile_of_local, tile_count,
                           tile_start, sortkey, point_list, keys));
        GS_LAUNCH_CHECK("tilesort_kernel");
        GS_TIMED("tilesort_big_kernel", stream, hipLaunchKernelGGL(tilesort_big_kernel, dim3(T), dim3(BIG_SORT_THREADS), 0, stream, meta, tile_of_local,
                           tile_count, tile_start, sortkey, point_list, keys));
        GS_LAUNCH_CHECK("tilesort_big_kernel");
    }
    const unsigned nblk = ((T + 7u) / 8u) * 32u;
    GS_TIMED("render_fwd_kernel", stream, hipLaunchKernelGGL(render_fwd_kernel, dim3(nblk), dim3(64), 0, stream, W, H, gx, T, ranges, point_list,
                       reinterpret_cast<const float2*>(means2D), reinterpret_cast<const float4*>(conic_opacity), rgb,
                       compute_locally, bg, out_color, at<float>(img, il.final_T), at<uint32_t>(img, il.n_contrib),
                       at<uint32_t>(img, il.n_contrib2loss), out_observe, n_consider, n_contrib));
    GS_LAUNCH_CHECK("render_fwd_kernel");
    (void)gy;
    return GS_OK;
}

extern "C" int gs_render_backward(int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                                  const float* conic_opacity, const float* rgb, const uint8_t* compute_locally,
                                  const void* binning, const void* img, const float* dL_dpixels, float* dL_dmeans2D,
                                  int dL_dmeans2D_stride, float* dL_dmeans2D_abs, float* dL_dconic_opacity,
                                  float* dL_dcolors, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0 && W > 0 && H > 0 && R >= 0, "invalid sizes P=%d W=%d H=%d R=%lld", P, W, H, (long long)R);
    GS_REQUIRE(dL_dmeans2D_stride >= 2, "dL_dmeans2D row stride must be >= 2");
    GS_REQUIRE(((uintptr_t)conic_opacity & 15) == 0 && ((uintptr_t)dL_dconic_opacity & 15) == 0 &&
               ((uintptr_t)means2D & 7) == 0,
               "conic_opacity / dL_dconic_opacity must be 16-byte and means2D 8-byte aligned");
    if (P == 0) return GS_OK;
    const ImgLayout il = img_layout(W, H);
    const BinLayout bl = bin_layout(R);
    const unsigned gx = (unsigned)((W + 15) / 16), gy = (unsigned)((H + 15) / 16);
    const unsigned T = gx * gy;
    GS_TIMED("zero_grads_kernel", stream, hipLaunchKernelGGL(zero_grads_kernel, dim3(gs_div_up((size_t)P, 256)), dim3(256), 0, stream, P,
                       dL_dmeans2D_stride, dL_dmeans2D, dL_dmeans2D_abs, reinterpret_cast<float4*>(dL_dconic_opacity),
                       dL_dcolors));
    GS_LAUNCH_CHECK("zero_grads_kernel");
    if (R == 0) return GS_OK;
    const unsigned nblk = ((T + 7u) / 8u) * 32u;
    GS_TIMED("render_bwd_kernel", stream, hipLaunchKernelGGL(render_bwd_kernel, dim3(nblk), dim3(64), 0, stream, W, H, gx, T,
                       at<uint2>(img, il.ranges), at<uint32_t>(binning, bl.point_list),
                       reinterpret_cast<const float2*>(means2D), reinterpret_cast<const float4*>(conic_opacity), rgb,
                       compute_locally, bg, at<float>(img, il.final_T), at<uint32_t>(img, il.n_contrib), dL_dpixels,
                       dL_dmeans2D, dL_dmeans2D_stride, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors));
    GS_LAUNCH_CHECK("render_bwd_kernel");
    return GS_OK;
}
