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
//   1. count   : each block takes a chunk of Gaussians, expands their tile
//                instances wave-cooperatively (one instance per lane per
//                round, whatever the rect sizes) and histograms them in LDS
//                (one counter per local tile); it then reserves its slice of
//                every tile bucket with one global atomic per non-empty tile.
//   2. scan    : a scan over the tile totals gives the tile offsets (these
//                are the reference's ranges) and R.
//   3. scatter : each block re-walks its chunk and appends (depth bits, id)
//                to its reserved slices (LDS cursors).
//   4. sort    : one block per tile sorts its bucket by (depth bits, id) in
//                LDS (bitonic, three size classes) and writes the sorted ids
//                and the (tile << 32 | depth bits) keys.
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
constexpr int SORT_CAP_S = 2048;     // bucket size classes sorted entirely in LDS
constexpr int SORT_CAP_M = 4096;
constexpr int SORT_CAP_L = 8192;
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

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(v, off, 64);
        if (lane >= off) v += y;
    }
    return v;
}

// Wave-cooperative instance expansion.  Each lane holds one Gaussian with
// `cnt` tile instances (its w-wide rect starting at (x0, y0)); the wave walks
// the concatenated instance list 64 at a time, so every lane handles one
// instance per round however unevenly the rect sizes are spread.
struct Expansion {
    int incl, total;
};

__device__ __forceinline__ Expansion expansion_begin(int cnt)
{
    Expansion e;
    e.incl = wave_incl_scan(cnt);
    e.total = __shfl(e.incl, 63, 64);
    return e;
}

// Owner lane and tile of instance k.  All 64 lanes must call this (it
// shuffles); the result is meaningful when k < total.
__device__ __forceinline__ void expansion_at(const Expansion& e, int cnt, unsigned x0, unsigned y0, unsigned w, int k,
                                             int& owner, unsigned& tx, unsigned& ty)
{
    int lo = 0;
#pragma unroll
    for (int step = 32; step > 0; step >>= 1) {
        const int probe = __shfl(e.incl, lo + step - 1, 64);
        if (probe <= k) lo += step;
    }
    owner = lo < 64 ? lo : 63;
    const int o_excl = __shfl(e.incl - cnt, owner, 64);
    const unsigned ox0 = (unsigned)__shfl((int)x0, owner, 64);
    const unsigned oy0 = (unsigned)__shfl((int)y0, owner, 64);
    const unsigned ow = (unsigned)__shfl((int)w, owner, 64);
    const unsigned local = (unsigned)(k - o_excl);
    const unsigned q = ow ? local / ow : 0u;
    tx = ox0 + (local - q * ow);
    ty = oy0 + q;
}

// tile rect of Gaussian i (binning rule); returns its tile count
__device__ __forceinline__ int rect_of(int i, int i1, const float2* __restrict__ means2D, const int* __restrict__ radii,
                                       unsigned gx, unsigned gy, unsigned& x0, unsigned& y0, unsigned& w)
{
    x0 = y0 = w = 0;
    if (i >= i1) return 0;
    const int r = radii[i];
    if (r <= 0) return 0;
    const float2 p = means2D[i];
    unsigned x1, y1;
    gs::rect_int(p.x, p.y, r, gx, gy, x0, y0, x1, y1);
    w = x1 - x0;
    return (int)(w * (y1 - y0));
}

// Per chunk of Gaussians: histogram of its tile instances in LDS; the chunk
// then reserves its slice of every tile's bucket with one atomic per
// non-empty tile and keeps the returned base in its histogram row.  With more
// local tiles than LDS_TILES, instances are counted with global atomics.
__global__ __launch_bounds__(BIN_THREADS) void count_kernel(
    int P, int CH, unsigned gx, unsigned gy, const float2* __restrict__ means2D, const int* __restrict__ radii,
    const int* __restrict__ loc_map, const uint32_t* __restrict__ meta, uint32_t* __restrict__ hist,
    uint32_t* __restrict__ tile_count)
{
    __shared__ uint32_t s_hist[LDS_TILES];
    const int TL = (int)meta[0];
    const bool lds = TL <= LDS_TILES;
    const bool all_local = TL == (int)(gx * gy);
    const int c = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lds) {
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) s_hist[l] = 0;
        __syncthreads();
    }
    const int i0 = c * CH;
    const int i1 = min(P, i0 + CH);
    for (int wb = i0 + wave * 64; wb < i1; wb += BIN_THREADS) {
        unsigned x0, y0, w;
        const int cnt = rect_of(wb + lane, i1, means2D, radii, gx, gy, x0, y0, w);
        const Expansion e = expansion_begin(cnt);
        for (int k0 = 0; k0 < e.total; k0 += 64) {
            int owner;
            unsigned tx, ty;
            expansion_at(e, cnt, x0, y0, w, k0 + lane, owner, tx, ty);
            if (k0 + lane < e.total) {
                const unsigned t = ty * gx + tx;
                const int l = all_local ? (int)t : loc_map[t];
                if (l >= 0) {
                    if (lds) atomicAdd(&s_hist[l], 1u);
                    else atomicAdd(&tile_count[l], 1u);
                }
            }
        }
    }
    if (lds) {
        __syncthreads();
        uint32_t* row = hist + (size_t)c * TL;
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) {
            const uint32_t v = s_hist[l];
            row[l] = v ? atomicAdd(&tile_count[l], v) : 0u;
        }
    }
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

// Re-walks the chunk and appends (depth bits << 32 | Gaussian id) to the
// chunk's reserved slice of each tile bucket (LDS cursors).
__global__ __launch_bounds__(BIN_THREADS) void scatter_kernel(
    int P, int CH, unsigned gx, unsigned gy, const float2* __restrict__ means2D, const float* __restrict__ depths,
    const int* __restrict__ radii, const int* __restrict__ loc_map, const uint32_t* __restrict__ meta,
    const uint32_t* __restrict__ hist, const uint32_t* __restrict__ tile_start, uint32_t* __restrict__ cursor,
    uint64_t* __restrict__ sortkey)
{
    __shared__ uint32_t s_cur[LDS_TILES];
    const int TL = (int)meta[0];
    const bool lds = TL <= LDS_TILES;
    const bool all_local = TL == (int)(gx * gy);
    const int c = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lds) {
        const uint32_t* row = hist + (size_t)c * TL;
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) s_cur[l] = tile_start[l] + row[l];
        __syncthreads();
    }
    const int i0 = c * CH;
    const int i1 = min(P, i0 + CH);
    for (int wb = i0 + wave * 64; wb < i1; wb += BIN_THREADS) {
        const int i = wb + lane;
        unsigned x0, y0, w;
        const int cnt = rect_of(i, i1, means2D, radii, gx, gy, x0, y0, w);
        const uint32_t dbits = cnt ? gs::f2u(depths[i]) : 0u;
        const Expansion e = expansion_begin(cnt);
        for (int k0 = 0; k0 < e.total; k0 += 64) {
            int owner;
            unsigned tx, ty;
            expansion_at(e, cnt, x0, y0, w, k0 + lane, owner, tx, ty);
            const uint32_t odb = (uint32_t)__shfl((int)dbits, owner, 64);
            if (k0 + lane < e.total) {
                const unsigned t = ty * gx + tx;
                const int l = all_local ? (int)t : loc_map[t];
                if (l >= 0) {
                    const uint32_t pos = lds ? atomicAdd(&s_cur[l], 1u) : atomicAdd(&cursor[l], 1u);
                    sortkey[pos] = ((uint64_t)odb << 32) | (uint32_t)(wb + owner);
                }
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

// Bitonic sort of s[0..N), N a power of two, n real keys (the rest are
// treated as +inf): every comparator puts the minimum at the lower index
// (the "flip" first stage of each merge), so keys past n never move and need
// no storage; pairs touching them are skipped.
template <int NT>
__device__ __forceinline__ void bitonic(uint64_t* s, int n, int N)
{
    for (int k = 2; k <= N; k <<= 1) {
        const int lh = __builtin_ctz((unsigned)k) - 1;            // log2(k/2)
        for (int p = threadIdx.x; p < (N >> 1); p += NT) {
            const int blk = p >> lh, off = p & ((1 << lh) - 1);
            const int a = (blk << (lh + 1)) + off;
            const int b = a + k - 1 - 2 * off;
            if (b < n) cswap(&s[a], &s[b]);
        }
        __syncthreads();
        for (int j = k >> 2; j >= 1; j >>= 1) {
            const int lj = __builtin_ctz((unsigned)j);
            for (int p = threadIdx.x; p < (N >> 1); p += NT) {
                const int blk = p >> lj, off = p & (j - 1);
                const int a = (blk << (lj + 1)) + off;
                if (a + j < n) cswap(&s[a], &s[a + j]);
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

// One block per local tile whose bucket size lies in (LO, CAP]: the bucket is
// sorted by (depth bits, Gaussian id) in LDS.  Three size classes keep the
// LDS footprint (and so the occupancy) matched to the bucket.
template <int CAP, int NT, int LO>
__global__ __launch_bounds__(NT) void tilesort_kernel(
    const uint32_t* __restrict__ meta, const int* __restrict__ tile_of_local, const uint32_t* __restrict__ tile_count,
    const uint32_t* __restrict__ tile_start, const uint64_t* __restrict__ sortkey, uint32_t* __restrict__ point_list,
    uint64_t* __restrict__ keys)
{
    __shared__ uint64_t s[CAP];
    const int l = blockIdx.x;
    if (l >= (int)meta[0]) return;
    const int n = (int)tile_count[l];
    if (n <= LO || n > CAP) return;
    const uint32_t start = tile_start[l];
    int N = 1;
    while (N < n) N <<= 1;
    for (int i = threadIdx.x; i < n; i += NT) s[i] = sortkey[start + i];
    __syncthreads();
    bitonic<NT>(s, n, N);
    write_sorted((uint32_t)tile_of_local[l], start, n, s, point_list, keys, NT);
}

// Buckets larger than the biggest LDS class: the same network in global
// memory, in place.
__global__ __launch_bounds__(BIG_SORT_THREADS) void tilesort_big_kernel(
    const uint32_t* __restrict__ meta, const int* __restrict__ tile_of_local, const uint32_t* __restrict__ tile_count,
    const uint32_t* __restrict__ tile_start, uint64_t* __restrict__ sortkey, uint32_t* __restrict__ point_list,
    uint64_t* __restrict__ keys)
{
    const int l = blockIdx.x;
    if (l >= (int)meta[0]) return;
    const int n = (int)tile_count[l];
    if (n <= SORT_CAP_L) return;
    const uint32_t start = tile_start[l];
    uint64_t* s = sortkey + start;
    int N = 1;
    while (N < n) N <<= 1;
    bitonic<BIG_SORT_THREADS>(s, n, N);
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
    __shared__ int s_pos[64];    // position in the tile's list

    const uint2 range = ranges[tile];
    const int n = (int)(range.y - range.x);
    const float pxf = (float)px, pyf = (float)py;
    const float qx0 = (float)((int)(tile % gx) * 16 + (int)(quad & 1u) * 8);
    const float qy0 = (float)((int)(tile / gx) * 16 + (int)(quad >> 1) * 8);
    const float alpha_min = 1.0f / 255.0f;
    float T_ = 1.0f, C0 = 0.f, C1 = 0.f, C2 = 0.f;
    uint32_t last = 0, n2l = 0;
    bool done = !inside;

    for (int base = 0; base < n; base += 64) {
        if (gs::ballot(!done) == 0) break;
        // stage the batch, keeping only Gaussians that can reach this quadrant
        const int k = base + lane;
        bool keep = false;
        uint32_t id = 0;
        float2 xy = make_float2(0.f, 0.f);
        float4 co = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < n) {
            id = point_list[range.x + k];
            xy = means2D[id];
            co = conic_opacity[id];
            keep = gs::may_touch(xy.x, xy.y, co.x, co.y, co.z, co.w, qx0, qy0, qx0 + 7.0f, qy0 + 7.0f);
        }
        const uint64_t km = gs::ballot(keep);
        if (keep) {
            const int slot = gs::rank_below(km);
            s_a[slot] = make_float4(xy.x, xy.y, -0.5f * co.x, -co.y);
            s_b[slot] = make_float4(-0.5f * co.z, co.w, rgb[3 * id], rgb[3 * id + 1]);
            s_c[slot] = make_float2(rgb[3 * id + 2], __uint_as_float(id));
            s_pos[slot] = k;
        }
        __syncthreads();
        const int cnt = (int)__builtin_popcountll(km);
        for (int j = 0; j < cnt; j++) {
            if (gs::ballot(!done) == 0) break;
            const float4 A = s_a[j];
            const float4 B = s_b[j];
            const float2 Cc = s_c[j];
            bool observe = false;
            if (!done) {
                const float dx = A.x - pxf, dy = A.y - pyf;
                const float power = gs::power_of(A.z, A.w, B.x, dx, dy);
                const float alpha = __builtin_fminf(0.99f, B.y * gs::expf_nonpos(power));
                if (!(power > 0.0f) && !(alpha < alpha_min)) {
                    const float test_T = T_ * (1.0f - alpha);
                    if (test_T < 0.0001f) {
                        done = true;
                    } else {
                        observe = T_ > 0.5f;
                        n2l++;
                        const float wgt = alpha * T_;
                        C0 = __builtin_fmaf(B.z, wgt, C0);
                        C1 = __builtin_fmaf(B.w, wgt, C1);
                        C2 = __builtin_fmaf(Cc.x, wgt, C2);
                        T_ = test_T;
                        last = (uint32_t)s_pos[j] + 1u;
                    }
                }
            }
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
    __shared__ int s_pos[64];    // position in the tile's list

    const uint2 range = ranges[tile];
    const float pxf = (float)px, pyf = (float)py;
    const float qx0 = (float)((int)(tile % gx) * 16 + (int)(quad & 1u) * 8);
    const float qy0 = (float)((int)(tile / gx) * 16 + (int)(quad >> 1) * 8);
    const float alpha_min = 1.0f / 255.0f;
    const float ddelx_dx = 0.5f * (float)W, ddely_dy = 0.5f * (float)H;
    const float bg_dot = bg[0] * dp0 + bg[1] * dp1 + bg[2] * dp2;
    // after the wave reduction this lane holds the total of one gradient term:
    // its array, row stride and offset
    float* my_dst = nullptr;
    int my_stride = 0;
    switch (gs::wave_sum12_index(lane)) {
        case 0: my_dst = g_m2d; my_stride = m2d_stride; break;
        case 1: my_dst = g_m2d + 1; my_stride = m2d_stride; break;
        case 2: my_dst = g_m2d_abs; my_stride = 3; break;
        case 3: my_dst = g_m2d_abs + 1; my_stride = 3; break;
        case 4: my_dst = g_con; my_stride = 4; break;
        case 5: my_dst = g_con + 1; my_stride = 4; break;
        case 6: my_dst = g_con + 2; my_stride = 4; break;
        case 7: my_dst = g_con + 3; my_stride = 4; break;
        case 8: my_dst = g_col; my_stride = 3; break;
        case 9: my_dst = g_col + 1; my_stride = 3; break;
        case 10: my_dst = g_col + 2; my_stride = 3; break;
        default: break;
    }
    float T_ = T_final;
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f;
    float lc0 = 0.f, lc1 = 0.f, lc2 = 0.f, last_alpha = 0.f;

    // walk positions maxlast-1 .. 0 of the tile's list, back to front
    for (int top = maxlast; top > 0; top -= 64) {
        // stage positions top-1, top-2, ... keeping only Gaussians that can reach this quadrant
        const int k = top - 1 - lane;
        bool keep = false;
        uint32_t id = 0;
        float2 xy = make_float2(0.f, 0.f);
        float4 co = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k >= 0) {
            id = point_list[range.x + k];
            xy = means2D[id];
            co = conic_opacity[id];
            keep = gs::may_touch(xy.x, xy.y, co.x, co.y, co.z, co.w, qx0, qy0, qx0 + 7.0f, qy0 + 7.0f);
        }
        const uint64_t km = gs::ballot(keep);
        if (keep) {
            const int slot = gs::rank_below(km);
            s_a[slot] = make_float4(xy.x, xy.y, -0.5f * co.x, -co.y);
            s_b[slot] = make_float4(-0.5f * co.z, co.w, rgb[3 * id], rgb[3 * id + 1]);
            s_c[slot] = make_float2(rgb[3 * id + 2], __uint_as_float(id));
            s_pos[slot] = k;
        }
        __syncthreads();
        const int cnt = (int)__builtin_popcountll(km);
        for (int j = 0; j < cnt; j++) {
            const int ci = s_pos[j];   // position in the tile's list
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
                    const float inv_one_m = __builtin_amdgcn_rcpf(one_m);   // 1 ulp; gradients only
                    T_ = T_ * inv_one_m;
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
                    dL_dalpha += (-T_final * inv_one_m) * bg_dot;
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
            const uint64_t vm = gs::ballot(valid);
            if (vm == 0) continue;
            const uint32_t id = __float_as_uint(Cc.y);
            const float vals[12] = {gmx, gmy, __builtin_fabsf(gmx), __builtin_fabsf(gmy), gca, gcb, gcc, gop,
                                    gc0, gc1, gc2, 0.f};
            const float tot = gs::wave_sum12(vals);
            if (my_dst != nullptr && tot != 0.f) unsafeAtomicAdd(my_dst + (size_t)id * my_stride, tot);
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
        GS_TIMED("tilesort_kernel_s", stream,
                 hipLaunchKernelGGL((tilesort_kernel<SORT_CAP_S, 256, 0>), dim3(T), dim3(256), 0, stream, meta,
                                    tile_of_local, tile_count, tile_start, sortkey, point_list, keys));
        GS_LAUNCH_CHECK("tilesort_kernel<S>");
        GS_TIMED("tilesort_kernel_m", stream,
                 hipLaunchKernelGGL((tilesort_kernel<SORT_CAP_M, 512, SORT_CAP_S>), dim3(T), dim3(512), 0, stream,
                                    meta, tile_of_local, tile_count, tile_start, sortkey, point_list, keys));
        GS_LAUNCH_CHECK("tilesort_kernel<M>");
        GS_TIMED("tilesort_kernel_l", stream,
                 hipLaunchKernelGGL((tilesort_kernel<SORT_CAP_L, 1024, SORT_CAP_M>), dim3(T), dim3(1024), 0, stream,
                                    meta, tile_of_local, tile_count, tile_start, sortkey, point_list, keys));
        GS_LAUNCH_CHECK("tilesort_kernel<L>");
        GS_TIMED("tilesort_big_kernel", stream,
                 hipLaunchKernelGGL(tilesort_big_kernel, dim3(T), dim3(BIG_SORT_THREADS), 0, stream, meta,
                                    tile_of_local, tile_count, tile_start, sortkey, point_list, keys));
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
