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
//   1. count   : each block takes a chunk of Gaussians (each wave a
//                contiguous run of it), expands their tile instances
//                wave-cooperatively (one instance per lane per round, whatever
//                the rect sizes) and histograms them in LDS (one counter per
//                local tile); it then reserves its slice of every tile bucket
//                with one global atomic per non-empty tile.  Each wave also
//                counts its listed Gaussians (non-empty rect).
//   2. scan    : a scan over the tile totals gives the tile offsets (these
//                are the reference's ranges) and R; a scan over the per-wave
//                listed counts numbers the listed Gaussians densely in id
//                order (compact index).
//   3. scatter : each block re-walks its chunk, appends (depth bits, compact
//                index) to its reserved slices (LDS cursors) and writes each
//                listed Gaussian's 64-byte blend record at its compact index.
//   4. sort    : one block (or wave) per tile sorts its bucket by (depth
//                bits, compact index) on chip -- a register bitonic network
//                up to 512 keys, an LDS radix sort up to 8192, a bitonic
//                network in global memory beyond -- in size classes, each
//                class walking its own list of buckets, and writes the
//                compact list the blend walks (the reference's sorted ids and
//                keys are derived from it on request).
// The compact index is increasing in Gaussian id, so each sorted bucket is
// exactly the order of a stable sort of the reference's duplicated keys, and
// the sorted arrays and the ranges are bit-identical to the reference
// algorithm's.  When more than LDS_TILES tiles are local, steps 1 and 3 use
// global atomics instead of the LDS histogram (same result after step 4).
//
// Blend design.  One wave64 per 8x8 quadrant of a tile, one pixel per lane,
// no block-wide barriers: a wave stages batches of 64 list entries (their
// records gathered while the previous batch blends) in its own LDS slots,
// dropping those that provably cannot reach the quadrant, and stops as soon as
// all of its 64 pixels are saturated.  The backward walks each quadrant's
// list back to front from the largest last contributor of its pixels, reduces
// every Gaussian's eleven gradient terms across the wave and adds them into
// the Gaussian's 64-byte accumulator with one atomic instruction per (wave,
// Gaussian) instead of eleven atomics per (pixel, Gaussian); a final pass
// writes the reference's gradient arrays from the accumulators.
#include <mutex>

#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {

constexpr int LDS_TILES = 16384;     // local tiles histogrammed in LDS (64 KB)
constexpr int BIN_THREADS = 512;
constexpr int WAVES_PER_BIN = BIN_THREADS / 64;
constexpr int MAX_CHUNKS = 512;
constexpr int SORT_CAP_MAX = 8192;   // largest bucket sorted on chip (8 keys per thread, 1024 threads)
constexpr int SORT_CLASSES = 6;      // bucket size classes: <= 512, 1k, 2k, 4k, 8k keys, larger
// Regions of the split path: RS x RS-tile blocks (RS = 2, or 4 / 8 for very
// large tile grids) tiling the local-tile box from its corner.
constexpr int REGION_SIDE = 2;       // preferred region side (tiles)
constexpr int MAX_REGIONS = 16384;   // regions of the full tile grid
constexpr int LDS_REGIONS = 4096;    // region counters / cursors held in LDS by the count and the scatter
constexpr int LDS_GRID = 12288;      // entries of the tile-count difference grid held in LDS
constexpr int GRID_PARTS = 16;       // partial difference grids (chunk c adds into part c % GRID_PARTS)
constexpr int REGION_CLASSES = 5;    // region list size classes: <= 1k, 2k, 4k, 8k entries, larger
constexpr int REGION_CAP = 8192;     // longest region list sorted on chip in one piece
constexpr const char* BINNING_STAGE = "binning (wall)";   // per-kernel timing: the whole binning stage
// Listed Gaussians (non-empty tile rect) are numbered densely, in Gaussian id
// order ("compact index").  Per listed Gaussian the scatter writes a blend
// record of 4 x float4 at its compact index:
//   [0] mean x, mean y, conic a, conic b
//   [1] conic c, opacity, red, green
//   [2] blue, cull threshold, cull slopes -b/c and -b/a
//   [3] Gaussian id bits, alpha cut-off power -log(255 opacity), 0, 0
// so the blend gathers one aligned 64-byte segment per list entry.
constexpr size_t REC_BYTES = 64;
// Per-Gaussian gradient accumulator of the backward (16 floats, 11 used):
//   dmean x, dmean y, |dmean x|, |dmean y|, dconic a, b, c, dopacity, drgb x 3
constexpr size_t GACC_BYTES = 64;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Blend blocks are grouped into supertiles of SUPER x SUPER tiles, supertile s
// on XCD s % 8 (block_to_tile); an XCD's tiles, in supertile order, number at
// most sched_cap of them.
constexpr unsigned SUPER = 8;
__host__ __device__ __forceinline__ unsigned sched_cap(unsigned NS) { return ((NS + 7u) / 8u) * SUPER * SUPER; }

struct GeomLayout {
    int T, NC, CH, WS;
    int RS, NR, G;                // region side (0: grid too large), regions and difference-grid entries of the full grid
    size_t cls_count, cls_list;   // per size class: number of local tiles, their local indices (T per class)
    size_t loc_map, tile_of_local, meta, hist, tile_count, tile_start, cursor, wcount, cidx_of, cid2id, rec, gacc;
    // split path: per-region local-tile masks, list lengths, offsets and
    // cursors, per-chunk region bases, per-class region lists and the partial
    // per-tile count difference grids
    size_t regmask, rcount, rstart, rcursor, rhist, rcls_count, rcls_list, grid;
    size_t qwork, sched, scnt;   // split path: per-quadrant work (forward), backward block order
    size_t total;
};

// region side for a gx x gy tile grid: the smallest of REGION_SIDE, 4 and 8
// that gives at most MAX_REGIONS regions; 0 when 8 does not
inline int region_side(int gx, int gy)
{
    for (int rs = REGION_SIDE; rs <= 8; rs *= 2)
        if ((long)((gx + rs - 1) / rs) * (long)((gy + rs - 1) / rs) <= MAX_REGIONS) return rs;
    return 0;
}

GeomLayout geom_layout(int P, int W, int H)
{
    GeomLayout g;
    const int gx = (W + 15) / 16, gy = (H + 15) / 16;
    g.T = gx * gy;
    g.RS = region_side(gx, gy);
    {
        const int rs = g.RS > 0 ? g.RS : 8;
        g.NR = ((gx + rs - 1) / rs) * ((gy + rs - 1) / rs);
    }
    g.G = ((gx + 1) * (gy + 1) + 3) & ~3;   // a multiple of four cells: the scan reads the partials as 16-byte vectors
    long nc = ((long)P + 2047) / 2048;
    if (nc < 1) nc = 1;
    if (nc > MAX_CHUNKS) nc = MAX_CHUNKS;
    g.NC = (int)nc;
    g.CH = (int)(((long)P + g.NC - 1) / g.NC);
    // each of a block's waves takes a contiguous run of WS Gaussians (whole groups of 64)
    g.WS = (int)((((long)g.CH + WAVES_PER_BIN - 1) / WAVES_PER_BIN + 63) / 64 * 64);
    size_t o = 0;
    g.loc_map = o; o = align256(o + sizeof(int) * (size_t)g.T);
    g.tile_of_local = o; o = align256(o + sizeof(int) * (size_t)g.T);
    g.meta = o; o = align256(o + 64);
    g.hist = o; o = align256(o + sizeof(uint32_t) * (size_t)g.NC * (size_t)(g.T < LDS_TILES ? g.T : LDS_TILES));
    g.tile_count = o; o = align256(o + sizeof(uint32_t) * (size_t)g.T);
    g.tile_start = o; o = align256(o + sizeof(uint32_t) * (size_t)g.T);
    g.cursor = o; o = align256(o + sizeof(uint32_t) * (size_t)g.T);
    g.wcount = o; o = align256(o + sizeof(uint32_t) * (size_t)g.NC * WAVES_PER_BIN);
    g.cls_count = o; o = align256(o + sizeof(uint32_t) * SORT_CLASSES);
    g.cls_list = o; o = align256(o + sizeof(int) * (size_t)SORT_CLASSES * (size_t)g.T);
    g.cidx_of = o; o = align256(o + sizeof(int) * (size_t)P);
    g.cid2id = o; o = align256(o + sizeof(uint32_t) * (size_t)P);
    g.rec = o; o = align256(o + REC_BYTES * (size_t)P);
    g.gacc = o; o = align256(o + GACC_BYTES * (size_t)P);
    g.regmask = o; o = align256(o + sizeof(uint64_t) * (size_t)g.NR);
    g.rcount = o; o = align256(o + sizeof(uint32_t) * (size_t)g.NR);
    g.rstart = o; o = align256(o + sizeof(uint32_t) * (size_t)g.NR);
    g.rcursor = o; o = align256(o + sizeof(uint32_t) * (size_t)g.NR);
    g.rhist = o; o = align256(o + sizeof(uint32_t) * (size_t)g.NC * (size_t)(g.NR < LDS_REGIONS ? g.NR : LDS_REGIONS));
    g.rcls_count = o; o = align256(o + sizeof(uint32_t) * REGION_CLASSES);
    g.rcls_list = o; o = align256(o + sizeof(int) * (size_t)REGION_CLASSES * (size_t)g.NR);
    g.grid = o; o = align256(o + sizeof(uint32_t) * (size_t)GRID_PARTS * (size_t)g.G);
    {
        const unsigned NS = (unsigned)(((gx + SUPER - 1) / SUPER) * ((gy + SUPER - 1) / SUPER));
        g.qwork = o; o = align256(o + sizeof(uint32_t) * 4 * (size_t)g.T);
        g.sched = o; o = align256(o + sizeof(uint32_t) * 8 * (size_t)sched_cap(NS));
        g.scnt = o; o = align256(o + sizeof(uint32_t) * 8);
    }
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
    size_t sortkey, point_list, keys, clist, total;
};

// The compact list comes first: it is the only array the blend, the backward
// and the depth pass read.  The point list and its keys (written on request,
// after the forward) follow it, and the forward's unsorted keys use their
// space as scratch.  Nothing at or past an offset depends on R except through
// that offset, so a buffer laid out for a capacity C >= R serves R: its
// compact list is at the same place and the point list fits.
BinLayout bin_layout(int64_t R)
{
    BinLayout b;
    size_t o = 0;
    b.clist = o; o = align256(o + sizeof(uint32_t) * (size_t)R);
    b.point_list = o;
    b.sortkey = o;                                   // 8R bytes inside point list + keys
    o = align256(o + sizeof(uint32_t) * (size_t)R);
    b.keys = o; o = align256(o + sizeof(uint64_t) * (size_t)R);
    b.total = o < 256 ? 256 : o;
    return b;
}

template <typename T>
T* at(void* base, size_t off) { return reinterpret_cast<T*>(static_cast<char*>(base) + off); }
template <typename T>
const T* at(const void* base, size_t off) { return reinterpret_cast<const T*>(static_cast<const char*>(base) + off); }

// ---------------------------------------------------------------- scans

// Per-call state of the split path's region binning, cleared by the local
// tile map (null pointers: not used by the caller's path).  Thread i of n
// clears entries i, i + n, ...
struct ClearRegions {
    uint64_t* regmask;   // per-region local-tile masks (null when every tile is local)
    uint32_t* rcount;    // per-region list lengths
    uint32_t* grid;      // partial per-tile count difference grids
    int NR, G;           // regions; entries of all partial grids
    unsigned lrs;        // log2 of the region side

    __device__ __forceinline__ void clear(int i, int n) const
    {
        clear_bulk(i, n);
        clear_masks(i, n);
    }
    // the partial grids and the list lengths
    __device__ __forceinline__ void clear_bulk(int i, int n) const
    {
        for (int k = i; k < G && grid != nullptr; k += n) grid[k] = 0u;
        for (int k = i; k < NR && rcount != nullptr; k += n) rcount[k] = 0u;
    }
    // the local-tile masks
    __device__ __forceinline__ void clear_masks(int i, int n) const
    {
        for (int k = i; k < NR && regmask != nullptr; k += n) regmask[k] = 0ull;
    }
};

// compute_locally (null: every tile) -> local tile numbering and the
// bounding box of the local tiles (meta[5..8] = x0, y0, x1, y1, exclusive
// ends; empty box if none); clears the per-tile counters and the region
// state, then sets the regions' local-tile masks.  Block 0 (16 waves) does
// the numbering: each wave owns a contiguous run of 64-tile rounds, counts
// its local tiles (ballots), one barrier publishes the 16 counts, and a
// second walk numbers the tiles in order with coalesced loads and stores.
// The other blocks clear the partial count grids and list lengths, which
// block 0 does not touch (alone it took ~70 us for a 256 x 171-tile grid).
__global__ __launch_bounds__(1024) void localmap_kernel(int T, unsigned gx, const uint8_t* __restrict__ cl,
                                                        int* __restrict__ loc_map, int* __restrict__ tile_of_local,
                                                        uint32_t* __restrict__ tile_count, uint32_t* __restrict__ meta,
                                                        ClearRegions CR, int lds_rounds)
{
    if (gridDim.x == 1) {
        CR.clear_bulk(threadIdx.x, 1024);
    } else if (blockIdx.x > 0) {
        CR.clear_bulk((int)((blockIdx.x - 1) * 1024 + threadIdx.x), (int)((gridDim.x - 1) * 1024));
        return;
    }
    CR.clear_masks(threadIdx.x, 1024);
    // dynamic LDS: the mask as one 64-bit word per 64-tile round, when the
    // grid has at most lds_rounds rounds (else the mask is re-read from memory)
    extern __shared__ uint64_t s_bits[];
    __shared__ uint32_t s_cnt[16];
    __shared__ uint32_t s_box[4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (threadIdx.x == 0) { s_box[0] = 0xffffffffu; s_box[1] = 0xffffffffu; s_box[2] = 0u; s_box[3] = 0u; }
    const int rounds = (T + 63) / 64;
    const bool in_lds = rounds <= lds_rounds;
    const int per = (rounds + 15) / 16;
    const int r0 = min(rounds, w * per), r1 = min(rounds, r0 + per);
    auto flag = [&](int t) { return t < T && cl[t] != 0; };
    // pass 1: the wave's local-tile count; the mask bytes of eight rounds are
    // loaded at once (unconditionally, at clamped indices, then masked)
    uint32_t cnt = 0;
    for (int rb = r0; rb < r1; rb += 8) {
        uint8_t byte[8];
#pragma unroll
        for (int k = 0; k < 8; k++) byte[k] = cl[min((rb + k) * 64 + lane, T - 1)];
        bool f[8];
#pragma unroll
        for (int k = 0; k < 8; k++) f[k] = rb + k < r1 && (rb + k) * 64 + lane < T && byte[k] != 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint64_t m = gs::ballot(f[k]);
            cnt += (uint32_t)__builtin_popcountll(m);
            if (in_lds && lane == 0 && rb + k < r1) s_bits[rb + k] = m;
        }
    }
    if (lane == 0) s_cnt[w] = cnt;
    __syncthreads();
    uint32_t base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t c = s_cnt[i];
        base += i < w ? c : 0u;
        tot += c;
    }
    // pass 2: number the tiles in order; the lane's tile (tx, ty) advances by
    // 64 tiles a round without a division
    uint32_t bx0 = 0xffffffffu, by0 = 0xffffffffu, bx1 = 0u, by1 = 0u;
    const uint32_t step_x = 64u % gx, step_y = 64u / gx;
    uint32_t tx = (uint32_t)(r0 * 64 + lane) % gx, ty = (uint32_t)(r0 * 64 + lane) / gx;
    for (int r = r0; r < r1; r++) {
        const int t = r * 64 + lane;
        const uint64_t m = in_lds ? s_bits[r] : gs::ballot(flag(t));
        const bool f = (m >> lane) & 1ull;
        const uint32_t l = base + (uint32_t)gs::rank_below(m);
        if (t < T) {
            loc_map[t] = f ? (int)l : -1;
            tile_count[t] = 0;
        }
        if (f) {
            tile_of_local[l] = t;
            bx0 = min(bx0, tx); by0 = min(by0, ty);
            bx1 = max(bx1, tx + 1); by1 = max(by1, ty + 1);
        }
        base += (uint32_t)__builtin_popcountll(m);
        tx += step_x;
        ty += step_y;
        if (tx >= gx) { tx -= gx; ty++; }
    }
    atomicMin(&s_box[0], bx0); atomicMin(&s_box[1], by0);
    atomicMax(&s_box[2], bx1); atomicMax(&s_box[3], by1);
    __syncthreads();
    if (threadIdx.x == 0) {
        meta[0] = tot;
        const bool any = tot > 0;
        meta[5] = any ? s_box[0] : 0u; meta[6] = any ? s_box[1] : 0u;
        meta[7] = any ? s_box[2] : 0u; meta[8] = any ? s_box[3] : 0u;
    }
    // local-tile mask of every region of the box (the cleared masks and the
    // box are visible after the barrier above; every local tile lies in the
    // box), needed only when the local tiles do not fill their box
    const bool box_full = tot == (s_box[2] - s_box[0]) * (s_box[3] - s_box[1]);
    if (CR.regmask != nullptr && tot > 0 && !box_full) {
        const unsigned rs = 1u << CR.lrs, nrx = (s_box[2] - s_box[0] + rs - 1) >> CR.lrs;
        const uint32_t sx = 1024u % gx, sy = 1024u / gx;
        uint32_t px = threadIdx.x % gx, py = threadIdx.x / gx;   // (px, py): tile t
        for (int t = threadIdx.x; t < T; t += 1024, px += sx, py += sy) {
            if (px >= gx) { px -= gx; py++; }
            if (!(in_lds ? (bool)((s_bits[t >> 6] >> (t & 63)) & 1ull) : flag(t))) continue;
            const unsigned ax = px - s_box[0], ay = py - s_box[1];
            const unsigned r = (ay >> CR.lrs) * nrx + (ax >> CR.lrs);
            atomicOr(reinterpret_cast<unsigned long long*>(&CR.regmask[r]),
                     1ull << (((ay & (rs - 1)) << CR.lrs) + (ax & (rs - 1))));
        }
    }
}
__global__ __launch_bounds__(256) void localmap_all_kernel(int T, unsigned gx, unsigned gy, int* __restrict__ loc_map,
                                                            int* __restrict__ tile_of_local,
                                                            uint32_t* __restrict__ tile_count,
                                                            uint32_t* __restrict__ meta, ClearRegions CR)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    CR.clear(t, (int)(gridDim.x * blockDim.x));
    if (t < T) {
        loc_map[t] = t;
        tile_of_local[t] = t;
        tile_count[t] = 0;
    }
    if (t == 0) {
        meta[0] = (uint32_t)T;
        meta[5] = 0u; meta[6] = 0u; meta[7] = gx; meta[8] = gy;
    }
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

// Local-tile bounding box: tiles outside it are never local, so rects are
// clipped to it before their instances are expanded.
struct TileBox {
    unsigned x0, y0, x1, y1;
};

__device__ __forceinline__ TileBox tile_box(const uint32_t* __restrict__ meta)
{
    return TileBox{meta[5], meta[6], meta[7], meta[8]};
}

// tile rect of a Gaussian with radius r and mean p (binning rule), clipped to
// the local-tile box; returns its tile count there
__device__ __forceinline__ int rect_from(int r, float2 p, unsigned gx, unsigned gy, const TileBox& box, unsigned& x0,
                                         unsigned& y0, unsigned& w)
{
    x0 = y0 = w = 0;
    if (r <= 0) return 0;
    unsigned x1, y1;
    gs::rect_int(p.x, p.y, r, gx, gy, x0, y0, x1, y1);
    x0 = max(x0, box.x0); y0 = max(y0, box.y0);
    x1 = min(x1, box.x1); y1 = min(y1, box.y1);
    if (x1 <= x0 || y1 <= y0) { x0 = y0 = 0; return 0; }
    w = x1 - x0;
    return (int)(w * (y1 - y0));
}

// float-extent rect of the full-image path (ext = the preprocess's rect
// extents), clipped to the local-tile box; returns its tile count there
__device__ __forceinline__ int rect_from_ext(int r, float2 p, float2 ext, unsigned gx, unsigned gy,
                                             const TileBox& box, unsigned& x0, unsigned& y0, unsigned& w)
{
    x0 = y0 = w = 0;
    if (r <= 0) return 0;
    unsigned x1, y1;
    gs::rect_float(p.x, p.y, ext.x, ext.y, gx, gy, x0, y0, x1, y1);
    x0 = max(x0, box.x0); y0 = max(y0, box.y0);
    x1 = min(x1, box.x1); y1 = min(y1, box.y1);
    if (x1 <= x0 || y1 <= y0) { x0 = y0 = 0; return 0; }
    w = x1 - x0;
    return (int)(w * (y1 - y0));
}

// Per-Gaussian constants of the full path's tile test, carried by the lane
// that holds the Gaussian and shuffled to the lanes expanding its tiles.
struct KeepTest {
    float mx, my, a, b, c, thr;
};

__device__ __forceinline__ KeepTest keep_test_of(float2 m, float4 co)
{
    return KeepTest{m.x, m.y, co.x, co.y, co.z, gs::logf_full(co.w / (1.0f / 255.0f))};
}

// does instance (owner's Gaussian, tile tx, ty) survive the tile test
__device__ __forceinline__ bool keep_instance(const KeepTest& k, int owner, unsigned tx, unsigned ty)
{
    const float mx = __shfl(k.mx, owner, 64), my = __shfl(k.my, owner, 64);
    const float a = __shfl(k.a, owner, 64), b = __shfl(k.b, owner, 64), c = __shfl(k.c, owner, 64);
    const float thr = __shfl(k.thr, owner, 64);
    return gs::full_tile_keep(mx, my, a, b, c, thr, tx, ty);
}

// radius and mean of Gaussian i of a wave's run ending at i1 (radius 0 past it)
__device__ __forceinline__ void load_rm(int i, int i1, const int* __restrict__ radii,
                                        const float2* __restrict__ means2D, int& r, float2& m)
{
    r = 0;
    m = make_float2(0.f, 0.f);
    if (i < i1) {
        r = radii[i];
        m = means2D[i];
    }
}

// Per chunk of Gaussians: histogram of its tile instances in LDS; the chunk
// then reserves its slice of every tile's bucket with one atomic per
// non-empty tile and keeps the returned base in its histogram row.  With more
// local tiles than LDS_TILES, instances are counted with global atomics.
//
// Each wave takes a contiguous run of WS Gaussians of the chunk and also
// counts its listed Gaussians (wcount), from which the scan derives the
// compact indices.
//
// FULL (the full-image path): rects come from the preprocess's float extents
// and an instance counts only if it passes the tile test (full_tile_keep).
template <bool FULL>
__global__ __launch_bounds__(BIN_THREADS) void count_kernel(
    int P, int CH, int WS, unsigned gx, unsigned gy, const float2* __restrict__ means2D, const int* __restrict__ radii,
    const int* __restrict__ loc_map, const uint32_t* __restrict__ meta, uint32_t* __restrict__ hist,
    uint32_t* __restrict__ tile_count, uint32_t* __restrict__ wcount, const float2* __restrict__ rects,
    const float4* __restrict__ conic_opacity)
{
    extern __shared__ uint4 s_dyn[];   // min(T, LDS_TILES) tile counters
    uint32_t* s_hist = reinterpret_cast<uint32_t*>(s_dyn);
    const int TL = (int)meta[0];
    const bool lds = TL <= LDS_TILES;
    const bool all_local = TL == (int)(gx * gy);
    const TileBox box = tile_box(meta);
    const int c = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lds) {
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) s_hist[l] = 0;
        __syncthreads();
    }
    const int i1c = min(P, c * CH + CH);
    const int ws = min(i1c, c * CH + wave * WS);
    const int i1 = min(i1c, ws + WS);
    uint32_t listed = 0;
    // the next group's radii and means are loaded while this group expands
    int r_n;
    float2 m_n;
    load_rm(ws + lane, i1, radii, means2D, r_n, m_n);
    for (int wb = ws; wb < i1; wb += 64) {
        const int r = r_n;
        const float2 m = m_n;
        load_rm(wb + 64 + lane, i1, radii, means2D, r_n, m_n);
        unsigned x0, y0, w;
        int cnt;
        KeepTest kt{};
        if (FULL) {
            const int i = wb + lane;
            cnt = rect_from_ext(r, m, r > 0 ? rects[i] : make_float2(0.f, 0.f), gx, gy, box, x0, y0, w);
            if (cnt > 0) kt = keep_test_of(m, conic_opacity[i]);
        } else {
            cnt = rect_from(r, m, gx, gy, box, x0, y0, w);
        }
        listed += (uint32_t)__builtin_popcountll(gs::ballot(cnt > 0));
        const Expansion e = expansion_begin(cnt);
        for (int k0 = 0; k0 < e.total; k0 += 64) {
            int owner;
            unsigned tx, ty;
            expansion_at(e, cnt, x0, y0, w, k0 + lane, owner, tx, ty);
            const bool kept = !FULL || keep_instance(kt, owner, tx, ty);
            if (k0 + lane < e.total && kept) {
                const unsigned t = ty * gx + tx;
                const int l = all_local ? (int)t : loc_map[t];
                if (l >= 0) {
                    if (lds) atomicAdd(&s_hist[l], 1u);
                    else atomicAdd(&tile_count[l], 1u);
                }
            }
        }
    }
    if (lane == 0) wcount[(size_t)c * WAVES_PER_BIN + wave] = listed;
    if (lds) {
        __syncthreads();
        uint32_t* row = hist + (size_t)c * TL;
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) {
            const uint32_t v = s_hist[l];
            row[l] = v ? atomicAdd(&tile_count[l], v) : 0u;
        }
    }
}

// inclusive scan over the 64 lanes of a wave (DPP: row_shr 1, 2, 4, 8 inside
// each 16-lane row, then row_bcast 15 / 31 across rows); all lanes active
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, true);
}

__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v)
{
    v += dpp_u<0x111>(v);          // row_shr:1
    v += dpp_u<0x112>(v);          // row_shr:2
    v += dpp_u<0x114>(v);          // row_shr:4
    v += dpp_u<0x118>(v);          // row_shr:8
    v += dpp_u<0x142, 0xa>(v);     // row_bcast:15 into rows 1 and 3
    v += dpp_u<0x143, 0xc>(v);     // row_bcast:31 into rows 2 and 3
    return v;
}


// inclusive max over the 64 lanes of a wave, for values >= 0 (the DPP steps
// read 0 past the row edges); all lanes active
__device__ __forceinline__ uint32_t wave_incl_max_u32(uint32_t v)
{
    v = max(v, dpp_u<0x111>(v));
    v = max(v, dpp_u<0x112>(v));
    v = max(v, dpp_u<0x114>(v));
    v = max(v, dpp_u<0x118>(v));
    v = max(v, dpp_u<0x142, 0xa>(v));
    v = max(v, dpp_u<0x143, 0xc>(v));
    return v;
}

// ---- split path: region binning
//
// The local-tile box is tiled by regions of RS x RS tiles from its corner
// (region (rx, ry) = box-relative tiles [rx RS, rx RS + RS) x [ry RS, ...)).
// A listed Gaussian enters the list of every region where its rect meets a
// local tile; the lists are sorted per region on chip and filtered into the
// region's tiles in order.

struct RegionGrid {
    unsigned bx0, by0, bw, bh, lrs, nrx, nry;
};

// LDS words of count_regions_kernel's region counters: min(NR, LDS_REGIONS)
// of the full grid, plus the extra row and column of a region difference grid
__host__ __device__ __forceinline__ int count_region_words(unsigned gx, unsigned gy, unsigned lrs)
{
    const unsigned rs = 1u << lrs, nx = (gx + rs - 1) >> lrs, ny = (gy + rs - 1) >> lrs;
    const int nr = (int)(nx * ny);
    return (nr < LDS_REGIONS ? nr : LDS_REGIONS) + (int)(nx + ny + 1);
}

__device__ __forceinline__ RegionGrid region_grid(const uint32_t* __restrict__ meta, unsigned lrs)
{
    RegionGrid g;
    g.bx0 = meta[5];
    g.by0 = meta[6];
    g.bw = meta[7] - meta[5];
    g.bh = meta[8] - meta[6];
    g.lrs = lrs;
    const unsigned rs = 1u << lrs;
    g.nrx = (g.bw + rs - 1) >> lrs;
    g.nry = (g.bh + rs - 1) >> lrs;
    return g;
}

// tile rect of a Gaussian with radius r and mean p (binning rule) clipped to
// the local-tile box: [x0, x1) x [y0, y1); false when empty (not listed)
__device__ __forceinline__ bool clip_rect(int r, float2 p, unsigned gx, unsigned gy, const TileBox& box, unsigned& x0,
                                          unsigned& y0, unsigned& x1, unsigned& y1)
{
    x0 = y0 = x1 = y1 = 0;
    if (r <= 0) return false;
    gs::rect_int(p.x, p.y, r, gx, gy, x0, y0, x1, y1);
    x0 = max(x0, box.x0); y0 = max(y0, box.y0);
    x1 = min(x1, box.x1); y1 = min(y1, box.y1);
    return x1 > x0 && y1 > y0;
}

// tiles of the box-relative rect [ax0, ax1) x [ay0, ay1) inside region
// (rx, ry) as a mask over the region's tiles (bit y RS + x, RS <= 8); the
// rect meets the region
__device__ __forceinline__ uint64_t rect_bits_in_region(unsigned ax0, unsigned ay0, unsigned ax1, unsigned ay1,
                                                        unsigned rx, unsigned ry, unsigned lrs)
{
    const unsigned rs = 1u << lrs;
    const unsigned ox = rx << lrs, oy = ry << lrs;
    const unsigned cx0 = max(ax0, ox) - ox, cx1 = min(ax1, ox + rs) - ox;
    const unsigned cy0 = max(ay0, oy) - oy, cy1 = min(ay1, oy + rs) - oy;
    const uint64_t row = ((1ull << (cx1 - cx0)) - 1ull) << cx0;
    const uint64_t ones = rs == 8u ? 0x0101010101010101ull : rs == 4u ? 0x1111ull : 0x5ull;   // bit 0 of every row
    const uint64_t rows = (ones >> ((rs - (cy1 - cy0)) << lrs)) << (cy0 << lrs);
    return rows * row;
}

// tiles of the box-relative rect [ax0, ax1) x [ay0, ay1) in region (rx, ry),
// which it meets, as masks over the region's tile columns (bits 0-7) and rows
// (bits 8-15): tile (jx, jy) of the region is in the rect iff bits jx and
// 8 + jy are both set
__device__ __forceinline__ uint32_t region_mask(unsigned ax0, unsigned ay0, unsigned ax1, unsigned ay1, unsigned rx,
                                                unsigned ry, unsigned lrs)
{
    const unsigned rs = 1u << lrs;
    auto span = [&](unsigned a0, unsigned a1, unsigned o) {
        const unsigned c0 = a0 > o ? a0 - o : 0u, c1 = min(a1 - o, rs);
        return ((1u << c1) - 1u) & ~((1u << c0) - 1u);
    };
    return span(ax0, ax1, rx << lrs) | (span(ay0, ay1, ry << lrs) << 8);
}

// LDS a wave needs for expand_regions: per lane its staged data (two
// uint4), then 64 segment marks
constexpr int EXPAND_WORDS = 64 * 8 + 64;

// Wave-cooperative walk over the regions each lane's box-relative rect
// [ax0, ax1) x [ay0, ay1) meets (all 64 lanes call it; in = false: no rect).
// The wave walks the concatenated (lane, region) pairs 64 at a time, one pair
// per lane per round however the rect sizes are spread, and calls
// f(q, rx, ry, owner's rect, owner's pa, pb, lbits) for the pairs whose region
// list the owner enters: the regions that hold a local tile of its rect
// (every region it meets when every tile of the box is local; lbits: the rect's local
// tiles in the region, rect_bits_in_region layout -- 0 when all are local).  pa / pb: per-lane payload
// handed to f as the owner's.  The lanes' data are staged in the wave's LDS
// (s, EXPAND_WORDS words); the owner of each position is found by marking the
// segment starts of the round and a max-scan over the marks.
template <typename F>
__device__ __forceinline__ void expand_regions(const RegionGrid& rg, bool all_local,
                                               const uint64_t* __restrict__ regmask, bool in, unsigned ax0,
                                               unsigned ay0, unsigned ax1, unsigned ay1, uint32_t pa, uint32_t pb,
                                               uint32_t* s, F&& f)
{
    const int lane = threadIdx.x & 63;
    uint4* s_own = reinterpret_cast<uint4*>(s);
    uint32_t* s_mark = s + 64 * 8;
    unsigned rx0 = 0u, ry0 = 0u, w = 0u;
    uint32_t cnt = 0u;
    if (in) {
        rx0 = ax0 >> rg.lrs;
        ry0 = ay0 >> rg.lrs;
        w = ((ax1 - 1) >> rg.lrs) + 1 - rx0;
        cnt = w * (((ay1 - 1) >> rg.lrs) + 1 - ry0);
    }
    const uint32_t incl = wave_incl_scan_u32(cnt);
    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    if (total == 0u) return;
    const uint32_t excl = incl - cnt;
    s_own[2 * lane] = make_uint4(rx0 | (ry0 << 16), w, excl, ax0 | (ax1 << 16));
    s_own[2 * lane + 1] = make_uint4(ay0 | (ay1 << 16), pa, pb, 0u);
    for (uint32_t k0 = 0; k0 < total; k0 += 64) {
        s_mark[lane] = 0u;
        __builtin_amdgcn_wave_barrier();
        if (cnt > 0u && excl >= k0 && excl < k0 + 64u) s_mark[excl - k0] = (uint32_t)lane + 1u;
        // the lane whose segment holds position k0: the first with incl > k0
        const uint32_t own0 = (uint32_t)__builtin_popcountll(gs::ballot(incl <= k0));
        __builtin_amdgcn_wave_barrier();
        uint32_t v = s_mark[lane];
        if (lane == 0 && v == 0u) v = own0 + 1u;
        const int owner = (int)wave_incl_max_u32(v) - 1;
        const uint4 o0 = s_own[2 * owner], o1 = s_own[2 * owner + 1];
        const uint32_t k = k0 + (uint32_t)lane;
        if (k < total) {
            const uint32_t local = k - o0.z, ow = o0.y;
            const uint32_t qy = local / ow;
            const unsigned rx = (o0.x & 0xffffu) + (local - qy * ow), ry = (o0.x >> 16) + qy;
            const unsigned oax0 = o0.w & 0xffffu, oax1 = o0.w >> 16, oay0 = o1.x & 0xffffu, oay1 = o1.x >> 16;
            const unsigned q = ry * rg.nrx + rx;
            const uint64_t lbits = all_local ? 0ull : regmask[q] & rect_bits_in_region(oax0, oay0, oax1, oay1, rx, ry, rg.lrs);
            if (all_local || lbits != 0ull) f(q, rx, ry, oax0, oay0, oax1, oay1, o1.y, o1.z, lbits);
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// In-place 2D inclusive prefix sum of the w x h grid g (row stride w) in LDS
// by an NT-thread block: rows one wave each, 64 columns at a time (DPP scan),
// then columns one thread each.  Barriers before and after are the caller's.
template <int NT>
__device__ __forceinline__ void lds_prefix_2d(uint32_t* g, unsigned w, unsigned h)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    for (unsigned y = (unsigned)wid; y < h; y += NT / 64) {
        uint32_t carry = 0u;
        for (unsigned x0 = 0; x0 < w; x0 += 64) {
            const unsigned x = x0 + (unsigned)lane;
            const uint32_t v = x < w ? g[y * w + x] : 0u;
            const uint32_t sum = wave_incl_scan_u32(v) + carry;
            if (x < w) g[y * w + x] = sum;
            carry = (uint32_t)__builtin_amdgcn_readlane((int)sum, 63);
        }
    }
    __syncthreads();
    for (unsigned x = threadIdx.x; x < w; x += NT) {
        uint32_t acc = 0u;
        for (unsigned y = 0; y < h; y++) {
            acc += g[y * w + x];
            g[y * w + x] = acc;
        }
    }
}

// Split path, step 1 (count).  Per chunk of Gaussians (each wave a
// contiguous run of it, as count_kernel): each wave's listed count; per
// region, how many of the chunk's listed Gaussians enter its list (LDS
// histogram; the chunk then reserves its slice of every region list with one
// atomic per non-empty region and keeps the returned base in its histogram
// row); and the per-tile instance counts as a difference grid over the box
// (+1 at (x0, y0) and (x1, y1), -1 at (x1, y0) and (x0, y1) per rect; the
// scan sums it in 2D), added into partial grid c % GRID_PARTS so that the
// chunks' additions do not all meet at the same addresses.  Beyond
// LDS_REGIONS regions or LDS_GRID grid entries the counters are global
// atomics.  Dynamic LDS: per wave EXPAND_WORDS, then min(NR, LDS_REGIONS) +
// min(G, LDS_GRID) words for the full tile grid.
__global__ __launch_bounds__(BIN_THREADS) void count_regions_kernel(
    int P, int CH, int WS, unsigned gx, unsigned gy, unsigned lrs, const float2* __restrict__ means2D,
    const int* __restrict__ radii, const uint32_t* __restrict__ meta, const uint64_t* __restrict__ regmask,
    uint32_t* __restrict__ rhist, uint32_t* __restrict__ rcount, uint32_t* __restrict__ grid, int Gfull,
    uint32_t* __restrict__ wcount)
{
    extern __shared__ uint4 s_dyn[];
    const RegionGrid rg = region_grid(meta, lrs);
    const int NRb = (int)(rg.nrx * rg.nry);
    const bool lds_r = NRb <= LDS_REGIONS;
    const unsigned gw = rg.bw + 1;
    const int G = (int)(gw * (rg.bh + 1));
    const bool lds_g = G <= LDS_GRID;
    const int c = blockIdx.x;
    // every tile of the local box is local (no mask, or a mask that fills its box):
    // each region a rect meets holds a local tile of it, and no mask test is needed
    const bool all_local = meta[0] == (meta[7] - meta[5]) * (meta[8] - meta[6]);
    // then the chunk's region counts come from a difference grid over the box's
    // regions too ((nrx + 1) x (nry + 1) entries, in the region words)
    const unsigned rgw = rg.nrx + 1;
    const bool rdiff = all_local && lds_r;
    uint32_t* s_exp = reinterpret_cast<uint32_t*>(s_dyn) + (threadIdx.x >> 6) * EXPAND_WORDS;
    uint32_t* s_rh = reinterpret_cast<uint32_t*>(s_dyn) + WAVES_PER_BIN * EXPAND_WORDS;
    uint32_t* s_grid = s_rh + (lds_r ? count_region_words(gx, gy, lrs) : 0);
    uint32_t* rc = lds_r ? s_rh : rcount;
    uint32_t* part = grid + (size_t)(c % GRID_PARTS) * (size_t)Gfull;
    uint32_t* gp = lds_g ? s_grid : part;
    const TileBox box = tile_box(meta);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    {
        for (int i = threadIdx.x; lds_r && i < (rdiff ? (int)(rgw * (rg.nry + 1)) : NRb); i += BIN_THREADS) s_rh[i] = 0u;
        for (int i = threadIdx.x; lds_g && i < G; i += BIN_THREADS) s_grid[i] = 0u;
        __syncthreads();
    }
    const int i1c = min(P, c * CH + CH);
    const int ws = min(i1c, c * CH + wave * WS);
    const int i1 = min(i1c, ws + WS);
    uint32_t listed = 0;
    // the inputs of the next two groups are loaded while this group is counted
    int r_n, r_nn;
    float2 m_n, m_nn;
    load_rm(ws + lane, i1, radii, means2D, r_n, m_n);
    load_rm(ws + 64 + lane, i1, radii, means2D, r_nn, m_nn);
    for (int wb = ws; wb < i1; wb += 64) {
        const int r = r_n;
        const float2 m = m_n;
        r_n = r_nn;
        m_n = m_nn;
        load_rm(wb + 128 + lane, i1, radii, means2D, r_nn, m_nn);
        unsigned x0, y0, x1, y1;
        const bool in = clip_rect(r, m, gx, gy, box, x0, y0, x1, y1);
        listed += (uint32_t)__builtin_popcountll(gs::ballot(in));
        const unsigned ax0 = x0 - rg.bx0, ax1 = x1 - rg.bx0, ay0 = y0 - rg.by0, ay1 = y1 - rg.by0;
        if (in) {
            atomicAdd(&gp[ay0 * gw + ax0], 1u);
            atomicAdd(&gp[ay0 * gw + ax1], ~0u);
            atomicAdd(&gp[ay1 * gw + ax0], ~0u);
            atomicAdd(&gp[ay1 * gw + ax1], 1u);
            if (rdiff) {
                // the rect's regions [rx0, rx1] x [ry0, ry1], corners of the region difference grid
                const unsigned rx0 = ax0 >> lrs, rx1 = ((ax1 - 1) >> lrs) + 1;
                const unsigned ry0 = ay0 >> lrs, ry1 = ((ay1 - 1) >> lrs) + 1;
                atomicAdd(&s_rh[ry0 * rgw + rx0], 1u);
                atomicAdd(&s_rh[ry0 * rgw + rx1], ~0u);
                atomicAdd(&s_rh[ry1 * rgw + rx0], ~0u);
                atomicAdd(&s_rh[ry1 * rgw + rx1], 1u);
            }
        }
        if (!rdiff)
            expand_regions(rg, all_local, regmask, in, ax0, ay0, ax1, ay1, 0u, 0u, s_exp,
                           [&](unsigned q, unsigned, unsigned, unsigned, unsigned, unsigned, unsigned, uint32_t,
                               uint32_t, uint64_t) { atomicAdd(&rc[q], 1u); });
    }
    if (lane == 0) wcount[(size_t)c * WAVES_PER_BIN + wave] = listed;
    __syncthreads();
    if (rdiff) {
        lds_prefix_2d<BIN_THREADS>(s_rh, rgw, rg.nry + 1);
        __syncthreads();
    }
    if (lds_r) {
        uint32_t* row = rhist + (size_t)c * NRb;
        // the bases of up to four regions per thread are requested at once
        for (int q0 = 0; q0 < NRb; q0 += 4 * BIN_THREADS) {
            uint32_t b[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int q = q0 + u * BIN_THREADS + (int)threadIdx.x;
                uint32_t v = 0u;
                if (q < NRb) v = rdiff ? s_rh[((unsigned)q / rg.nrx) * rgw + (unsigned)q % rg.nrx] : s_rh[q];
                b[u] = v ? atomicAdd(&rcount[q], v) : 0u;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int q = q0 + u * BIN_THREADS + (int)threadIdx.x;
                if (q < NRb) row[q] = b[u];
            }
        }
    }
    if (lds_g) {
        for (int i = threadIdx.x; i < G; i += BIN_THREADS) {
            const uint32_t v = s_grid[i];
            if (v) atomicAdd(&part[i], v);
        }
    }
}

// exclusive scans: over local tiles -> tile_start, R -> meta[2..3]; over the
// per-wave listed counts (in place) -> compact index bases, L -> meta[4]
__device__ __forceinline__ int sort_class(uint32_t n)
{
    return n <= 512u ? 0 : n <= 1024u ? 1 : n <= 2048u ? 2 : n <= 4096u ? 3 : n <= (uint32_t)SORT_CAP_MAX ? 4 : 5;
}

// The instance count as the host reads it back: one 64-bit word, so that a
// single store publishes it -- bits 0-31 R (mod 2^32), bit 32 set when R does
// not fit in 32 bits, bits 33-63 the caller's sequence number (31 bits), by
// which the host tells this call's word from an earlier one.
__host__ __device__ __forceinline__ uint64_t readback_word(uint64_t R, uint32_t seq)
{
    return (R & 0xffffffffull) | ((R >> 32) != 0 ? (1ull << 32) : 0ull) | ((uint64_t)(seq & 0x7fffffffu) << 33);
}

//
// cap: the instance capacity of the caller's binning buffer.  When R exceeds
// it, meta[9] is set and the class lists are left empty: the ranges, the
// scatter and the sorts then do nothing (the caller redoes the forward with a
// buffer for R).  host_R (device address of mapped, coherent pinned host
// memory, or null): R is also stored there in one 8-byte store, tagged with
// the caller's sequence number seq, for the host to poll (readback_word).
__global__ __launch_bounds__(1024) void tilescan_kernel(uint32_t* __restrict__ meta, const uint32_t* __restrict__ tile_count,
                                                        uint32_t* __restrict__ tile_start, uint32_t* __restrict__ cursor,
                                                        uint32_t* __restrict__ wcount, int NW, int T,
                                                        uint32_t* __restrict__ cls_count, int* __restrict__ cls_list,
                                                        uint64_t cap, uint64_t* __restrict__ host_R, uint32_t seq)
{
    __shared__ uint32_t s_wave[32];
    __shared__ uint32_t s_cls[SORT_CLASSES];
    if (threadIdx.x < SORT_CLASSES) s_cls[threadIdx.x] = 0u;
    const int TL = (int)meta[0];
    {
        uint32_t base = 0;
        for (int w0 = 0; w0 < NW; w0 += 1024) {
            const int wi = w0 + threadIdx.x;
            const uint32_t v = wi < NW ? wcount[wi] : 0u;
            uint32_t tot;
            const uint32_t pre = gs::block_excl_scan_1024(v, s_wave, &tot);
            if (wi < NW) wcount[wi] = base + pre;
            base += tot;
        }
        if (threadIdx.x == 0) meta[4] = base;
    }
    uint64_t base = 0;
    for (int t0 = 0; t0 < TL; t0 += 1024) {
        const int l = t0 + threadIdx.x;
        const uint32_t v = l < TL ? tile_count[l] : 0u;
        uint32_t tot;
        const uint32_t pre = gs::block_excl_scan_1024(v, s_wave, &tot);
        if (l < TL) {
            tile_start[l] = (uint32_t)(base + pre);
            cursor[l] = (uint32_t)(base + pre);
            // the sort launches walk per-class lists of non-empty buckets
            if (v > 0u) {
                const int c = sort_class(v);
                cls_list[(size_t)c * T + atomicAdd(&s_cls[c], 1u)] = l;
            }
        }
        base += tot;
    }
    __syncthreads();
    const bool over = base > cap;
    if (threadIdx.x < SORT_CLASSES) cls_count[threadIdx.x] = over ? 0u : s_cls[threadIdx.x];
    if (threadIdx.x == 0) {
        meta[2] = (uint32_t)(base & 0xffffffffu);
        meta[3] = (uint32_t)(base >> 32);
        meta[9] = over ? 1u : 0u;
        if (host_R != nullptr) *host_R = readback_word(base, seq);
    }
}

// per tile: ranges, n_render; clears the per-tile blend statistics (all
// ranges empty when R exceeded the caller's capacity)
struct RangesOut {
    int T;
    const int* loc_map;
    const uint32_t* tile_count;
    const uint32_t* tile_start;
    uint2* ranges;
    int32_t* n_render;     // null: the full-image path (no per-tile statistics)
    int32_t* n_consider;
    int32_t* n_contrib;

    __device__ __forceinline__ void tile(int t, bool over) const
    {
        const int l = loc_map[t];
        uint32_t cnt = 0, s = 0;
        if (l >= 0 && !over) { cnt = tile_count[l]; s = tile_start[l]; }
        ranges[t] = cnt ? make_uint2(s, s + cnt) : make_uint2(0u, 0u);
        if (n_render != nullptr) {
            n_render[t] = (int32_t)cnt;
            n_consider[t] = 0;
            n_contrib[t] = 0;
        }
    }
};

__global__ __launch_bounds__(256) void ranges_kernel(const uint32_t* __restrict__ meta, RangesOut ro)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < ro.T) ro.tile(t, meta[9] != 0u);
}

// ------------------------------------------------------------- scatter

// per-Gaussian int32 accumulators of the blend (null: not used by the mode),
// zeroed by the scatter, which visits every Gaussian once
struct ZeroOut {
    int32_t* p[4];
};

// Re-walks the chunk (each wave its run, as in the count) and appends
// (depth bits << 32 | compact index) to the chunk's reserved slice of each
// tile bucket (LDS cursors).  Compact indices follow Gaussian id order, so
// sorting by them breaks depth ties exactly as sorting by id does.  Every
// Gaussian gets its compact index or -1 (cidx_of); listed ones also get their
// blend record, id (cid2id) and a zeroed gradient accumulator.
template <bool FULL>
__global__ __launch_bounds__(BIN_THREADS) void scatter_kernel(
    int P, int CH, int WS, unsigned gx, unsigned gy, const float2* __restrict__ means2D,
    const float* __restrict__ depths, const int* __restrict__ radii, const float4* __restrict__ conic_opacity,
    const float* __restrict__ rgb, const int* __restrict__ loc_map, const uint32_t* __restrict__ meta,
    const uint32_t* __restrict__ hist, const uint32_t* __restrict__ tile_start, uint32_t* __restrict__ cursor,
    const uint32_t* __restrict__ wbase, uint64_t* __restrict__ sortkey, int* __restrict__ cidx_of,
    uint32_t* __restrict__ cid2id, float4* __restrict__ rec, const float2* __restrict__ rects, ZeroOut Z)
{
    if (meta[9] != 0u) return;   // R exceeded the caller's capacity: nothing to write
    // dynamic LDS: per wave 64 staged records, then min(T, LDS_TILES) cursors
    extern __shared__ uint4 s_dyn[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float4* stage = reinterpret_cast<float4*>(s_dyn) + wave * 256;
    uint32_t* s_cur = reinterpret_cast<uint32_t*>(s_dyn + WAVES_PER_BIN * 256);
    const int TL = (int)meta[0];
    const bool lds = TL <= LDS_TILES;
    const bool all_local = TL == (int)(gx * gy);
    const TileBox box = tile_box(meta);
    const int c = blockIdx.x;
    if (lds) {
        const uint32_t* row = hist + (size_t)c * TL;
        for (int l = threadIdx.x; l < TL; l += BIN_THREADS) s_cur[l] = tile_start[l] + row[l];
        __syncthreads();
    }
    const int i1c = min(P, c * CH + CH);
    const int ws = min(i1c, c * CH + wave * WS);
    const int i1 = min(i1c, ws + WS);
    uint32_t next = wbase[(size_t)c * WAVES_PER_BIN + wave];
    // software pipeline: all of the next group's inputs (radii, means, depth,
    // conic, colour) are loaded while this group expands -- unconditionally,
    // so that no load waits for the radius (the culled Gaussians' lines are
    // mostly fetched anyway: a line holds several Gaussians)
    int r_n;
    float2 m_n;
    float d_n = 0.f;
    float4 co_n = make_float4(0.f, 0.f, 0.f, 0.f);
    float3 c_n = make_float3(0.f, 0.f, 0.f);
    auto load_next = [&](int in) {
        load_rm(in, i1, radii, means2D, r_n, m_n);
        if (in < i1) {
            d_n = depths[in];
            co_n = conic_opacity[in];
            c_n = make_float3(rgb[3 * (size_t)in], rgb[3 * (size_t)in + 1], rgb[3 * (size_t)in + 2]);
        }
    };
    load_next(ws + lane);
    for (int wb = ws; wb < i1; wb += 64) {
        const int i = wb + lane;
        const int r = r_n;
        const float2 xy = m_n;
        const float dep = d_n;
        const float4 co = co_n;
        const float3 col = c_n;
        load_next(i + 64);
        unsigned x0, y0, w;
        int cnt;
        KeepTest kt{};
        if (FULL) {
            cnt = rect_from_ext(r, xy, r > 0 ? rects[i] : make_float2(0.f, 0.f), gx, gy, box, x0, y0, w);
            if (cnt > 0) kt = keep_test_of(xy, co);
        } else {
            cnt = rect_from(r, xy, gx, gy, box, x0, y0, w);
        }
        const uint64_t lm = gs::ballot(cnt > 0);
        const int nl = (int)__builtin_popcountll(lm);
        const int rank = gs::rank_below(lm);
        const uint32_t first = next;
        const uint32_t cidx = first + (uint32_t)rank;
        next += (uint32_t)nl;
        uint32_t dbits = 0;
        if (i < i1) {
            cidx_of[i] = cnt > 0 ? (int)cidx : -1;
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (Z.p[q] != nullptr) Z.p[q][i] = 0;
        }
        if (cnt > 0) {
            dbits = gs::f2u(dep);
            const gs::CullPrep cp = gs::cull_prepare(xy.x, xy.y, co.x, co.y, co.z, co.w);
            float4* sp = stage + 4 * rank;
            sp[0] = make_float4(xy.x, xy.y, co.x, co.y);
            sp[1] = make_float4(co.z, co.w, col.x, col.y);
            sp[2] = make_float4(col.z, cp.thresh, cp.nbc, cp.nba);
            sp[3] = make_float4(__uint_as_float((uint32_t)i), gs::alpha_cut_power(co.w), 0.f, 0.f);
            cid2id[cidx] = (uint32_t)i;
        }
        // the group's records are one contiguous run: write them with
        // consecutive 16-byte stores (wave-private staging, so a wave-level
        // barrier suffices)
        __builtin_amdgcn_wave_barrier();
        {
            float4* rdst = rec + 4 * (size_t)first;
            for (int j = lane; j < 4 * nl; j += 64) rdst[j] = stage[j];
        }
        __builtin_amdgcn_wave_barrier();
        const Expansion e = expansion_begin(cnt);
        for (int k0 = 0; k0 < e.total; k0 += 64) {
            int owner;
            unsigned tx, ty;
            expansion_at(e, cnt, x0, y0, w, k0 + lane, owner, tx, ty);
            const uint32_t odb = (uint32_t)__shfl((int)dbits, owner, 64);
            const uint32_t ocx = (uint32_t)__shfl((int)cidx, owner, 64);
            const bool kept = !FULL || keep_instance(kt, owner, tx, ty);
            if (k0 + lane < e.total && kept) {
                const unsigned t = ty * gx + tx;
                const int l = all_local ? (int)t : loc_map[t];
                if (l >= 0) {
                    const uint32_t pos = lds ? atomicAdd(&s_cur[l], 1u) : atomicAdd(&cursor[l], 1u);
                    sortkey[pos] = ((uint64_t)odb << 32) | ocx;
                }
            }
        }
    }
}

// Split path, step 3 (scatter).  Re-walks the chunk (each wave its run, as
// in the count) and appends the entry (depth bits, compact index, tile mask
// over the region -- region_mask) to the chunk's reserved slice of each
// region list it enters (LDS cursors; global cursors beyond LDS_REGIONS
// regions).  Every Gaussian gets its compact index or -1 (cidx_of); listed
// ones also get their blend record and id (cid2id) and their accumulators
// zeroed, as in scatter_kernel.  The blocks also write the tiles' ranges
// (ranges_kernel's work; tiles t = block * 512 + thread, strided by the grid).
__global__ __launch_bounds__(BIN_THREADS) void scatter_regions_kernel(
    int P, int CH, int WS, unsigned gx, unsigned gy, unsigned lrs, const float2* __restrict__ means2D,
    const float* __restrict__ depths, const int* __restrict__ radii, const float4* __restrict__ conic_opacity,
    const float* __restrict__ rgb, const uint32_t* __restrict__ meta, const uint64_t* __restrict__ regmask,
    const uint32_t* __restrict__ rhist, const uint32_t* __restrict__ rstart, uint32_t* __restrict__ rcursor,
    const uint32_t* __restrict__ wbase, uint3* __restrict__ rent, int* __restrict__ cidx_of,
    uint32_t* __restrict__ cid2id, float4* __restrict__ rec, ZeroOut Z, RangesOut ro)
{
    const bool over = meta[9] != 0u;
    for (int t = blockIdx.x * BIN_THREADS + threadIdx.x; t < ro.T; t += gridDim.x * BIN_THREADS) ro.tile(t, over);
    if (over) return;   // R exceeded the caller's capacity: nothing to write
    // dynamic LDS: per wave 64 staged records, then min(NR, LDS_REGIONS) cursors
    extern __shared__ uint4 s_dyn[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float4* stage = reinterpret_cast<float4*>(s_dyn) + wave * 256;
    uint32_t* s_exp = reinterpret_cast<uint32_t*>(s_dyn + WAVES_PER_BIN * 256) + wave * EXPAND_WORDS;
    uint32_t* s_cur = reinterpret_cast<uint32_t*>(s_dyn + WAVES_PER_BIN * 256) + WAVES_PER_BIN * EXPAND_WORDS;
    const RegionGrid rg = region_grid(meta, lrs);
    const int NRb = (int)(rg.nrx * rg.nry);
    const bool lds_r = NRb <= LDS_REGIONS;
    uint32_t* cur = lds_r ? s_cur : rcursor;
    // every tile of the local box is local (no mask, or a mask that fills its box):
    // each region a rect meets holds a local tile of it, and no mask test is needed
    const bool all_local = meta[0] == (meta[7] - meta[5]) * (meta[8] - meta[6]);
    const TileBox box = tile_box(meta);
    const int c = blockIdx.x;
    if (lds_r) {
        const uint32_t* row = rhist + (size_t)c * NRb;
        for (int q = threadIdx.x; q < NRb; q += BIN_THREADS) s_cur[q] = rstart[q] + row[q];
        __syncthreads();
    }
    const int i1c = min(P, c * CH + CH);
    const int ws = min(i1c, c * CH + wave * WS);
    const int i1 = min(i1c, ws + WS);
    uint32_t next = wbase[(size_t)c * WAVES_PER_BIN + wave];
    // Radius and mean of the group after next, and depth, conic and colour of
    // the next group -- the latter only for Gaussians with a radius (the
    // others are not listed and their lines need not be fetched) -- are loaded
    // while this group is written.
    struct Ext {
        float d;
        float4 co;
        float3 c;
    };
    auto load_ext = [&](int in, int r, Ext& v) {
        v.d = 0.f;
        v.co = make_float4(0.f, 0.f, 0.f, 0.f);
        v.c = make_float3(0.f, 0.f, 0.f);
        if (in < i1 && r > 0) {
            v.d = depths[in];
            v.co = conic_opacity[in];
            v.c = make_float3(rgb[3 * (size_t)in], rgb[3 * (size_t)in + 1], rgb[3 * (size_t)in + 2]);
        }
    };
    int r0, r1;
    float2 m0, m1;
    Ext e0;
    load_rm(ws + lane, i1, radii, means2D, r0, m0);
    load_rm(ws + 64 + lane, i1, radii, means2D, r1, m1);
    load_ext(ws + lane, r0, e0);
    for (int wb = ws; wb < i1; wb += 64) {
        const int i = wb + lane;
        const int r = r0;
        const float2 xy = m0;
        const float dep = e0.d;
        const float4 co = e0.co;
        const float3 col = e0.c;
        r0 = r1;
        m0 = m1;
        load_rm(i + 128, i1, radii, means2D, r1, m1);
        load_ext(i + 64, r0, e0);
        unsigned x0, y0, x1, y1;
        const bool in = clip_rect(r, xy, gx, gy, box, x0, y0, x1, y1);
        const uint64_t lm = gs::ballot(in);
        const int nl = (int)__builtin_popcountll(lm);
        const int rank = gs::rank_below(lm);
        const uint32_t first = next;
        const uint32_t cidx = first + (uint32_t)rank;
        next += (uint32_t)nl;
        if (i < i1) {
            cidx_of[i] = in ? (int)cidx : -1;
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (Z.p[q] != nullptr) Z.p[q][i] = 0;
        }
        if (in) {
            const gs::CullPrep cp = gs::cull_prepare(xy.x, xy.y, co.x, co.y, co.z, co.w);
            float4* sp = stage + 4 * rank;
            sp[0] = make_float4(xy.x, xy.y, co.x, co.y);
            sp[1] = make_float4(co.z, co.w, col.x, col.y);
            sp[2] = make_float4(col.z, cp.thresh, cp.nbc, cp.nba);
            sp[3] = make_float4(__uint_as_float((uint32_t)i), gs::alpha_cut_power(co.w), 0.f, 0.f);
            cid2id[cidx] = (uint32_t)i;
        }
        expand_regions(rg, all_local, regmask, in, x0 - rg.bx0, y0 - rg.by0, x1 - rg.bx0, y1 - rg.by0, gs::f2u(dep),
                       cidx, s_exp,
                       [&](unsigned q, unsigned rx, unsigned ry, unsigned ax0, unsigned ay0, unsigned ax1, unsigned ay1,
                           uint32_t dbits, uint32_t ocidx, uint64_t) {
                           rent[atomicAdd(&cur[q], 1u)] =
                               make_uint3(dbits, ocidx, region_mask(ax0, ay0, ax1, ay1, rx, ry, lrs));
                       });
        // the group's records are one contiguous run (wave-private staging)
        __builtin_amdgcn_wave_barrier();
        {
            float4* rdst = rec + 4 * (size_t)first;
            for (int j = lane; j < 4 * nl; j += 64) rdst[j] = stage[j];
        }
        __builtin_amdgcn_wave_barrier();
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

// A sorted bucket is written as the blend's compact list only (clist: compact
// index per list position).  The reference's sorted Gaussian ids and
// (tile << 32 | depth bits) keys are derived from it on request
// (pointlist_kernel, gs_render_point_list).
__device__ __forceinline__ void write_sorted(uint32_t start, int n, const uint64_t* src, uint32_t* __restrict__ clist,
                                             int nt)
{
    for (int i = threadIdx.x; i < n; i += nt) clist[start + i] = (uint32_t)src[i];
}

// ---- register-resident bitonic sort (buckets of up to 512 keys, one wave):
// each lane holds 8 consecutive keys (position i = 8 lane + r), so a
// compare-exchange between positions i and i ^ M is in-lane for M < 8 and
// between lanes (ds_swizzle / permlane32 exchanges, no barrier) up to M < 512.

// value of v held by lane (lane ^ D) of this wave, 0 < D < 64 (all lanes active)
template <int D>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v)
{
    if constexpr ((D & 32) != 0) {
        // permlane32_swap(v, v): first result = (v[0..31], v[0..31]), second = (v[32..63], v[32..63])
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = (threadIdx.x & 32u) ? r[0] : r[1];
    }
    if constexpr ((D & 31) != 0) v = (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, ((D & 31) << 10) | 0x1f);
    return v;
}

template <int D>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v)
{
    return ((uint64_t)lane_xor<D>((uint32_t)(v >> 32)) << 32) | (uint64_t)lane_xor<D>((uint32_t)v);
}

template <int X>
struct TopBit {
    static constexpr int value = X <= 1 ? 0 : 1 + TopBit<X / 2>::value;
};
template <>
struct TopBit<0> {
    static constexpr int value = 0;
};

// compare-exchanges (i, i ^ M), M < 8, inside each lane
template <int M>
__device__ __forceinline__ void sort_stage_in(uint64_t (&k)[8])
{
    constexpr int HB = 1 << TopBit<M>::value;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        if ((r & HB) == 0) {
            const uint64_t x = k[r], y = k[r ^ M];
            k[r] = x < y ? x : y;
            k[r ^ M] = x < y ? y : x;
        }
    }
}

// compare-exchanges (i, i ^ M), 8 <= M < 512: the partner is register
// r ^ (M & 7) of lane l ^ (M >> 3); the lower position keeps the minimum
template <int M>
__device__ __forceinline__ void sort_stage_cross(uint64_t (&k)[8])
{
    constexpr int DT = M >> 3, RX = M & 7;
    const bool lower = ((threadIdx.x >> TopBit<DT>::value) & 1u) == 0;
    uint64_t p[8];
#pragma unroll
    for (int r = 0; r < 8; r++) p[r] = lane_xor64<DT>(k[r ^ RX]);
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const uint64_t x = k[r], y = p[r];
        k[r] = lower ? (x < y ? x : y) : (x < y ? y : x);
    }
}

// half-cleaners j = J, J/2, ..., 1
template <int J>
__device__ __forceinline__ void sort_cleaners(uint64_t (&k)[8])
{
    if constexpr (J >= 8) {
        sort_stage_cross<J>(k);
        sort_cleaners<J / 2>(k);
    } else if constexpr (J >= 1) {
        sort_stage_in<J>(k);
        sort_cleaners<J / 2>(k);
    }
}

// merges of size K2, 2 K2, ..., 512: a flip (i, i ^ (K2 - 1)) then the half-cleaners
template <int K2>
__device__ __forceinline__ void sort_merges(uint64_t (&k)[8])
{
    if constexpr (K2 <= 512) {
        if constexpr (K2 <= 8) sort_stage_in<K2 - 1>(k);
        else sort_stage_cross<K2 - 1>(k);
        sort_cleaners<K2 / 4>(k);
        sort_merges<K2 * 2>(k);
    }
}

// A bucket of up to 512 keys sorted by one wave (lane = this thread's lane),
// by (depth bits, compact index), padded with all-ones keys.
__device__ __forceinline__ void wave_sort_bucket(uint32_t start, int n, const uint64_t* __restrict__ sortkey,
                                                 uint32_t* __restrict__ clist, int lane)
{
    uint64_t k[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int i = 8 * lane + r;
        k[r] = i < n ? sortkey[start + i] : ~0ull;
    }
    sort_merges<2>(k);
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int i = 8 * lane + r;
        if (i < n) clist[start + i] = (uint32_t)k[r];
    }
}

// ---- LDS radix sort of one bucket (least-significant digit first, 4-bit
// digits; Merrill & Grimshaw's per-thread counter ranking):
//   items = (depth bits, compact index); each thread owns K consecutive
//   positions of the bucket (blocked), stored in LDS with one pad slot per K
//   items so that the blocked reads are conflict-free.  Per digit:
//     count  : every item adds 1 to its thread's counter for its digit
//              (ds_add_rtn: the old value is the item's rank among the
//              thread's earlier items of that digit); the counters form a
//              digit-major (digit, thread) table,
//     scan   : an exclusive scan of that table in digit-major order gives
//              each (digit, thread) its first output position (raking: each
//              thread scans 16 consecutive entries, then one block-wide scan
//              of the 16-entry totals),
//     scatter: every item goes to its (digit, thread) base + rank.
//   Each pass is stable, so after the digits of the depth bits the bucket is
//   ordered by depth, items of equal depth in input order.  Digits on which
//   all keys agree are skipped.  Runs of equal depth (the reference orders
//   them by Gaussian id, i.e. by compact index) are then sorted by compact
//   index in place, one thread per run; a run longer than MAX_TIE_RUN sends
//   the bucket to the 64-bit bitonic network in global memory instead.
constexpr int RADIX_DIGITS = 16;
constexpr int MAX_TIE_RUN = 32;

template <int K>
struct Log2 {
    static constexpr int value = K <= 1 ? 0 : 1 + Log2<K / 2>::value;
};

// slot of item i: one pad slot after every K items, so that the K items of
// thread t start at t (K + 1) and the blocked reads (consecutive threads at an
// odd stride) are free of bank conflicts
template <int K>
__device__ __forceinline__ int rpad(int i) { return i + i / K; }


// exclusive scan of one value per thread over an NT-thread block (block
// total in *total); s_tmp holds NT / 64 words
template <int NT>
__device__ __forceinline__ uint32_t radix_block_scan(uint32_t v, uint32_t* s_tmp, uint32_t* total)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint32_t x = wave_incl_scan_u32(v);
    if (lane == 63) s_tmp[wid] = x;
    __syncthreads();
    uint32_t base = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) {
        const uint32_t sv = s_tmp[w];
        base += w < wid ? sv : 0u;
        tot += sv;
    }
    *total = tot;
    return base + x - v;
}

// The (digit, thread) counter table, flattened digit-major (f = digit * NT +
// thread), is stored with its 16-byte chunks XOR-swizzled inside each
// 256-byte row (word bits 2-5 ^= bits 4-7, a bijection): the per-item
// atomics (one column, consecutive threads) and the raking reads (16
// consecutive entries per thread, as 16-byte vectors) are then both free of
// bank conflicts, with 32 or 64 four-byte banks.
__device__ __forceinline__ int cnt_slot(int f) { return f ^ (((f >> 4) & 15) << 2); }

template <int NT, int K>
struct alignas(16) RadixLds {
    uint2 items[NT * K + NT];
    uint32_t cnt[RADIX_DIGITS * NT];
    uint32_t misc[3 * (NT / 64) + 4];
};

// Loads a bucket's n keys into S.items (all-ones padding from n up to the
// capacity NT K); kor / kand: OR and AND of the depth bits this thread loaded.
template <int NT, int K>
__device__ __forceinline__ void radix_load(uint32_t start, int n, const uint64_t* __restrict__ src,
                                           RadixLds<NT, K>& S, uint32_t& kor, uint32_t& kand)
{
    kor = 0u;
    kand = ~0u;
    // all K loads are issued before the first is used
    uint64_t v[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = (int)threadIdx.x + k * NT;
        v[k] = i < n ? src[start + i] : ~0ull;
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = (int)threadIdx.x + k * NT;
        const uint2 it = make_uint2((uint32_t)(v[k] >> 32), (uint32_t)v[k]);
        if (i < n) {
            kor |= it.x;
            kand &= it.x;
        }
        S.items[rpad<K>(i)] = it;
    }
}

// the compact index of an item whose second word is that index
struct TieIdentity {
    __device__ __forceinline__ uint32_t operator()(uint32_t y) const { return y; }
};

// Sorts the n items in S.items (padding above them, as radix_load leaves it)
// by (depth bits, compact index), the compact index of an item being
// tk(second word).  kor / kand: OR and AND of the depth bits of the items
// this thread placed.  Returns true (block-uniform) when a run of equal
// depths is longer than MAX_TIE_RUN: the items are then ordered by depth only
// and the caller sorts the bucket another way.
template <int NT, int K, typename TieKey = TieIdentity>
__device__ __forceinline__ bool radix_sort_items(int n, RadixLds<NT, K>& S, uint32_t kor, uint32_t kand,
                                                 TieKey tk = TieKey())
{
    constexpr int NW = NT / 64;
    const int t = threadIdx.x;
    const int lane = t & 63, wid = t >> 6;
    // which key bits vary over the bucket (digits that do not are skipped)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        kor |= (uint32_t)__shfl_xor((int)kor, off, 64);
        kand &= (uint32_t)__shfl_xor((int)kand, off, 64);
    }
    if (lane == 0) { S.misc[wid] = kor; S.misc[NW + wid] = kand; }
    if (t == 0) S.misc[2 * NW] = 0u;   // long-tie-run flag
    // this thread's raking segment of the counter table: four 16-byte chunks
    auto seg = [&](int i) -> uint4* { return reinterpret_cast<uint4*>(&S.cnt[cnt_slot(RADIX_DIGITS * t + 4 * i)]); };
    const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int i = 0; i < 4; i++) *seg(i) = z4;
    __syncthreads();
    uint32_t vor = 0u, vand = ~0u;
#pragma unroll
    for (int w = 0; w < NW; w++) { vor |= S.misc[w]; vand &= S.misc[NW + w]; }
    const uint32_t vary = vor ^ vand;
    uint32_t* s_tmp = S.misc + 2 * NW + 1;   // NW words for the block scan

    uint32_t* cnt = S.cnt;
    for (int shift = 0; shift < 32; shift += 4) {
        if (((vary >> shift) & 15u) == 0u) continue;   // uniform over the block
        uint32_t key[K], val[K], rk[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            const uint2 it = S.items[rpad<K>(t * K + k)];
            key[k] = it.x;
            val[k] = it.y;
        }
        // the table is all zero here (cleared before the first pass, and by
        // every thread's column at the end of each pass)
#pragma unroll
        for (int k = 0; k < K; k++) rk[k] = atomicAdd(&cnt[cnt_slot((int)((key[k] >> shift) & 15u) * NT + t)], 1u);
        __syncthreads();
        {
            uint4 q[4];
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = *seg(i);
            uint32_t run = 0u;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t a = q[i].x, b = q[i].y, c = q[i].z, d = q[i].w;
                q[i].x = run; run += a;
                q[i].y = run; run += b;
                q[i].z = run; run += c;
                q[i].w = run; run += d;
            }
            uint32_t tot;
            const uint32_t base = radix_block_scan<NT>(run, s_tmp, &tot);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                q[i].x += base; q[i].y += base; q[i].z += base; q[i].w += base;
                *seg(i) = q[i];
            }
        }
        __syncthreads();
        // all K bases are read before the first item moves (the compiler
        // cannot tell the item stores from the counter table, so interleaved
        // reads would each wait for the previous store)
#pragma unroll
        for (int k = 0; k < K; k++) rk[k] += cnt[cnt_slot((int)((key[k] >> shift) & 15u) * NT + t)];
#pragma unroll
        for (int k = 0; k < K; k++) S.items[rpad<K>((int)rk[k])] = make_uint2(key[k], val[k]);
        // only this thread reads its column (digit, t) in the scatter: clear
        // it for the next pass
#pragma unroll
        for (int d = 0; d < RADIX_DIGITS; d++) cnt[cnt_slot(d * NT + t)] = 0u;
        __syncthreads();
    }

    // runs of equal depth: order by compact index (one thread per run); the
    // thread's keys and its two neighbours' are read at once
    uint32_t kn[K + 2];
#pragma unroll
    for (int j = 0; j < K + 2; j++) {
        const int i = t * K - 1 + j;
        kn[j] = (i >= 0 && i < n) ? S.items[rpad<K>(i)].x : 0u;
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = t * K + k;
        if (i + 1 >= n) break;
        const uint32_t key_i = kn[k + 1];
        if (kn[k + 2] != key_i) continue;
        if (i > 0 && kn[k] == key_i) continue;   // not the run's first item
        int e = i + 2;
        while (e < n && e - i <= MAX_TIE_RUN && S.items[rpad<K>(e)].x == key_i) e++;
        if (e - i > MAX_TIE_RUN) {
            S.misc[2 * NW] = 1u;
            continue;
        }
        for (int a = i + 1; a < e; a++) {
            const uint32_t v = S.items[rpad<K>(a)].y;
            const uint32_t kv = tk(v);
            int b = a - 1;
            while (b >= i && tk(S.items[rpad<K>(b)].y) > kv) {
                S.items[rpad<K>(b + 1)].y = S.items[rpad<K>(b)].y;
                b--;
            }
            S.items[rpad<K>(b + 1)].y = v;
        }
    }
    __syncthreads();
    return S.misc[2 * NW] != 0u;
}

template <int NT, int K>
__device__ void radix_sort_bucket(uint32_t start, int n, uint64_t* __restrict__ sortkey, uint32_t* __restrict__ clist,
                                  RadixLds<NT, K>& S)
{
    uint32_t kor, kand;
    radix_load<NT, K>(start, n, sortkey, S, kor, kand);
    if (radix_sort_items<NT, K>(n, S, kor, kand)) {
        // a long run of equal depths: the full 64-bit sort in global memory
        // (the bucket there is still the unsorted input)
        uint64_t* s = sortkey + start;
        int N = 1;
        while (N < n) N <<= 1;
        bitonic<NT>(s, n, N);
        write_sorted(start, n, s, clist, NT);
        return;
    }
    for (int i = threadIdx.x; i < n; i += NT) clist[start + i] = S.items[rpad<K>(i)].y;
}

// One launch per size class; its blocks walk the class's list of buckets
// (block b takes entries b, b + gridDim.x, ...).  A launch also takes a
// second list (xcount / xlist) when EXTRA says so, so that the smallest and
// the largest buckets need no launches of their own:
//   EXTRA_WAVE: buckets of up to 512 keys, one per wave (wave_sort_bucket);
//   EXTRA_BIG : buckets of more than SORT_CAP_MAX keys, one per block (the
//               64-bit bitonic network in global memory, in place).
constexpr int EXTRA_NONE = 0, EXTRA_WAVE = 1, EXTRA_BIG = 2;

template <int NT, int K, int EXTRA = EXTRA_NONE>
__global__ __launch_bounds__(NT) void tilesort_radix_kernel(const uint32_t* __restrict__ cls_count,
                                                           const int* __restrict__ cls_list,
                                                           const uint32_t* __restrict__ tile_count,
                                                           const uint32_t* __restrict__ tile_start,
                                                           uint64_t* __restrict__ sortkey, uint32_t* __restrict__ clist,
                                                           const uint32_t* __restrict__ xcount,
                                                           const int* __restrict__ xlist)
{
    __shared__ RadixLds<NT, K> S;
    const int nl = (int)*cls_count;
    for (int e = blockIdx.x; e < nl; e += gridDim.x) {
        if (e != (int)blockIdx.x) __syncthreads();   // the previous bucket's reads of LDS are done
        const int l = cls_list[e];
        radix_sort_bucket<NT, K>(tile_start[l], (int)tile_count[l], sortkey, clist, S);
    }
    if constexpr (EXTRA == EXTRA_WAVE) {
        // no block barrier from here on: every wave sorts its own buckets
        constexpr int NW = NT / 64;
        const int nx = (int)*xcount;
        for (int e = blockIdx.x * NW + (int)(threadIdx.x >> 6); e < nx; e += gridDim.x * NW) {
            const int l = xlist[e];
            wave_sort_bucket(tile_start[l], (int)tile_count[l], sortkey, clist, threadIdx.x & 63);
        }
    } else if constexpr (EXTRA == EXTRA_BIG) {
        const int nx = (int)*xcount;
        for (int e = blockIdx.x; e < nx; e += gridDim.x) {
            const int l = xlist[e];
            const int n = (int)tile_count[l];
            const uint32_t start = tile_start[l];
            uint64_t* s = sortkey + start;
            int N = 1;
            while (N < n) N <<= 1;
            __syncthreads();
            bitonic<NT>(s, n, N);
            write_sorted(start, n, s, clist, NT);
        }
    }
}

// size class of a region list of n entries
__device__ __forceinline__ int region_class(uint32_t n)
{
    return n <= 1024u ? 0 : n <= 2048u ? 1 : n <= 4096u ? 2 : n <= (uint32_t)REGION_CAP ? 3 : 4;
}

// Exclusive scan of N values over a 1024-thread block, each thread taking 8
// consecutive values per round of 8192 (one block scan per round):
// put(i, prefix, value) for every i < N; returns the total.  A value is
// value(i, fetch(i, j)), j the value's place among the thread's 8 (i = 8 tid
// + j in the first round, unless clamped): the 8 fetches of a thread (global
// loads) are all issued before the first value is formed (they read index
// min(i, N - 1), so that none is conditional), and value may then read LDS.
template <typename Fetch, typename Value, typename Put>
__device__ __forceinline__ uint64_t block_scan_runs(int N, uint32_t* s_wave, Fetch&& fetch, Value&& value, Put&& put)
{
    uint64_t base = 0;
    for (int r0 = 0; r0 < N; r0 += 8192) {
        const int i0 = r0 + (int)threadIdx.x * 8;
        uint32_t f[8], v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) f[j] = fetch(min(i0 + j, N - 1), j);
        uint32_t sum = 0u;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            v[j] = i0 + j < N ? value(i0 + j, f[j]) : 0u;
            sum += v[j];
        }
        uint32_t tot;
        uint32_t run = gs::block_excl_scan_1024(sum, s_wave, &tot);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (i0 + j < N) put(i0 + j, (uint32_t)(base + run), v[j]);
            run += v[j];
        }
        base += tot;
    }
    return base;
}

// Split path, step 2 (scan): three blocks, independent of one another.
//   block 0: the difference grid (the sum of the partial grids) summed in 2D
//     (rows, then columns; in LDS when it fits) -> each local tile's instance
//     count (tile_count) and, by a scan in local order, its offset
//     (tile_start) and R -> meta[2..3]; meta[9] = R > cap (then nothing
//     further is written: the scatter and the sorts check it); R stored
//     for the host (host_R, seq: as tilescan_kernel);
//   block 1: the per-wave listed counts -> compact index bases (in place),
//     L -> meta[4];
//   block 2: the region list lengths -> offsets (rstart, and rcursor for the
//     global cursors) and per-class region lists; the total E -> meta[10]
//     (E <= R: a region entry stands for one or more instances).
__global__ __launch_bounds__(1024) void scan_regions_kernel(uint32_t* __restrict__ meta, unsigned gx, unsigned lrs,
                                                            const int* __restrict__ tile_of_local,
                                                            uint32_t* __restrict__ grid, int Gfull,
                                                            uint32_t* __restrict__ tile_count,
                                                            uint32_t* __restrict__ tile_start,
                                                            uint32_t* __restrict__ wcount, int NW,
                                                            const uint32_t* __restrict__ rcount,
                                                            uint32_t* __restrict__ rstart,
                                                            uint32_t* __restrict__ rcursor,
                                                            uint32_t* __restrict__ rcls_count,
                                                            int* __restrict__ rcls_list, int NR, uint64_t cap,
                                                            uint64_t* __restrict__ host_R, uint32_t seq)
{
    __shared__ uint32_t s_grid[LDS_GRID];
    __shared__ uint32_t s_wave[32];
    __shared__ uint32_t s_cls[REGION_CLASSES];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const RegionGrid rg = region_grid(meta, lrs);
    if (blockIdx.x == 1) {
        const uint64_t L = block_scan_runs(
            NW, s_wave, [&](int i, int) { return wcount[i]; }, [&](int, uint32_t f) { return f; },
            [&](int i, uint32_t pre, uint32_t) { wcount[i] = pre; });
        if (tid == 0) meta[4] = (uint32_t)L;
        return;
    }
    if (blockIdx.x == 2) {
        // regions: offsets and size classes
        if (tid < REGION_CLASSES) s_cls[tid] = 0u;
        __syncthreads();
        const int NRb = (int)(rg.nrx * rg.nry);
        const uint64_t E = block_scan_runs(
            NRb, s_wave, [&](int r, int) { return rcount[r]; }, [&](int, uint32_t f) { return f; },
            [&](int r, uint32_t pre, uint32_t v) {
                rstart[r] = pre;
                rcursor[r] = pre;
                if (v > 0u) {
                    const int c = region_class(v);
                    rcls_list[(size_t)c * NR + atomicAdd(&s_cls[c], 1u)] = r;
                }
            });
        __syncthreads();
        if (tid < REGION_CLASSES) rcls_count[tid] = s_cls[tid];
        if (tid == 0) meta[10] = (uint32_t)E;
        return;
    }
    const unsigned gw = rg.bw + 1;
    const int G = (int)(gw * (rg.bh + 1));
    const bool lds_g = G <= LDS_GRID;
    // the local tiles' indices, read while the grid is summed
    const int TL = (int)meta[0];
    uint32_t t_pre[8];
#pragma unroll
    for (int j = 0; j < 8; j++) t_pre[j] = TL > 0 ? (uint32_t)tile_of_local[min(tid * 8 + j, TL - 1)] : 0u;
    // the partial grids summed (into LDS, or into partial 0): four
    // consecutive cells per thread, one 16-byte load per partial (Gfull, the
    // partials' stride, is a multiple of four cells and at least G rounded up
    // to four), all 16 loads in flight
    uint32_t* gp = lds_g ? s_grid : grid;
    for (int i0 = tid * 4; i0 < G; i0 += 4096) {
        uint4 v[GRID_PARTS];
#pragma unroll
        for (int k = 0; k < GRID_PARTS; k++) v[k] = *reinterpret_cast<const uint4*>(grid + (size_t)k * Gfull + i0);
        uint4 sum = v[0];
#pragma unroll
        for (int k = 1; k < GRID_PARTS; k++) {
            sum.x += v[k].x;
            sum.y += v[k].y;
            sum.z += v[k].z;
            sum.w += v[k].w;
        }
        const uint32_t sv[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int c = 0; c < 4; c++)
            if (i0 + c < G) gp[i0 + c] = sv[c];
    }
    __syncthreads();
    // rows: one wave per row, 64 columns at a time
    for (unsigned y = (unsigned)wid; y < rg.bh; y += 16) {
        uint32_t carry = 0u;
        for (unsigned x0 = 0; x0 < rg.bw; x0 += 64) {
            const unsigned x = x0 + (unsigned)lane;
            const uint32_t v = x < rg.bw ? gp[y * gw + x] : 0u;
            const uint32_t sum = wave_incl_scan_u32(v) + carry;
            if (x < rg.bw) gp[y * gw + x] = sum;
            carry = (uint32_t)__builtin_amdgcn_readlane((int)sum, 63);
        }
    }
    __syncthreads();
    // columns: one thread per column, 8 rows per step
    for (unsigned x = (unsigned)tid; x < rg.bw; x += 1024) {
        uint32_t acc = 0u;
        unsigned y = 0;
        for (; y + 8 <= rg.bh; y += 8) {
            uint32_t v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = gp[(y + k) * gw + x];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                acc += v[k];
                gp[(y + k) * gw + x] = acc;
            }
        }
        for (; y < rg.bh; y++) {
            acc += gp[y * gw + x];
            gp[y * gw + x] = acc;
        }
    }
    __syncthreads();
    // local tiles in order: counts, offsets, R (the first 8192 tiles' indices
    // were read above)
    const uint64_t R = block_scan_runs(
        TL, s_wave,
        [&](int l, int j) { return l < 8192 ? t_pre[j] : (uint32_t)tile_of_local[l]; },
        [&](int, uint32_t t) { return gp[(t / gx - rg.by0) * gw + (t % gx - rg.bx0)]; },
        [&](int l, uint32_t pre, uint32_t v) {
            tile_count[l] = v;
            tile_start[l] = pre;
        });
    if (tid == 0) {
        const bool over = R > cap;
        meta[2] = (uint32_t)(R & 0xffffffffu);
        meta[3] = (uint32_t)(R >> 32);
        meta[9] = over ? 1u : 0u;
        if (host_R != nullptr) *host_R = readback_word(R, seq);
    }
}

// ---- split path: per-region sort and tile filter

// the tiles of region r: origin and extent (clipped to the box)
struct RegionTiles {
    unsigned tx0, ty0, tw, th;
};

__device__ __forceinline__ RegionTiles region_tiles(const RegionGrid& rg, int r)
{
    const unsigned rx = (unsigned)r % rg.nrx, ry = (unsigned)r / rg.nrx;
    const unsigned rs = 1u << rg.lrs;
    RegionTiles t;
    t.tx0 = rg.bx0 + (rx << rg.lrs);
    t.ty0 = rg.by0 + (ry << rg.lrs);
    t.tw = min(rs, rg.bw - (rx << rg.lrs));
    t.th = min(rs, rg.bh - (ry << rg.lrs));
    return t;
}

// where the filter writes: tile t's list is clist[tile_start[l], + tile_count[l])
// for its local index l
struct TileOut {
    const int* loc_map;
    const uint32_t* tile_start;
    const uint32_t* tile_count;
    uint32_t* clist;
    unsigned gx, gy;
};

// Region lists hold 12-byte entries (uint3): depth bits, compact index and
// the entry's tile mask over the region (region_mask), written with one store.

// LDS of a region sort.  An item is (depth bits, slot | tile mask << 16): the
// slot it was loaded into (its compact index is cidx[slot]) and its tile mask.
template <int NT, int K>
struct RegionLds {
    RadixLds<NT, K> R;
    uint32_t cidx[NT * K];
    uint32_t tslot[64 * 2];        // per tile of the region: list start (~0u: not local) and end
    uint32_t tab[(NT / 64) * 4];   // filter: per wave and tile of a pass, the wave's count, then its offset
    uint32_t piece[4 * 2];         // filter: per tile of a pass, this call's output start (~0u: none) and length
};

// words the filter may stage output in: the item slots and the counter
// table, which are free once every wave holds its items in registers
template <int NT, int K>
constexpr int stage_words() { return 2 * (NT * K + NT) + RADIX_DIGITS * NT; }

// list start (~0u: the tile is outside the box or not local) and end of tile
// j (row-major in the region, RS per row)
__device__ __forceinline__ void tile_slot(unsigned j, unsigned lrs, const RegionTiles& rt, const TileOut& to,
                                          bool all_local, uint32_t& b, uint32_t& e)
{
    b = ~0u;
    e = 0u;
    const unsigned rs = 1u << lrs, jx = j & (rs - 1), jy = j >> lrs;
    if (jx < rt.tw && jy < rt.th) {
        const unsigned tt = (rt.ty0 + jy) * to.gx + rt.tx0 + jx;
        const int l = all_local ? (int)tt : to.loc_map[tt];
        if (l >= 0) {
            b = to.tile_start[l];
            e = b + to.tile_count[l];
        }
    }
}

// Loads region list entries [start, start + n) (n <= NT K) into slots 0..n-1
// (all-ones padding above); kor / kand: OR and AND of this thread's depths.
template <int NT, int K>
__device__ __forceinline__ void region_load(uint32_t start, int n, const uint3* __restrict__ rent,
                                            RegionLds<NT, K>& L, uint32_t& kor, uint32_t& kand)
{
    kor = 0u;
    kand = ~0u;
    uint3 v[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = (int)threadIdx.x + k * NT;
        v[k] = i < n ? rent[start + i] : make_uint3(~0u, 0u, 0u);
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = (int)threadIdx.x + k * NT;
        uint2 it = make_uint2(~0u, ~0u);
        if (i < n) {
            it = make_uint2(v[k].x, (uint32_t)i | (v[k].z << 16));
            kor |= it.x;
            kand &= it.x;
            L.cidx[i] = v[k].y;
        }
        L.R.items[rpad<K>(i)] = it;
    }
}

// Bitonic sort of the n items in LDS by (depth bits, tk(second word)) -- the
// way out when radix_sort_items finds a long run of equal depths; pairs
// touching slots past n are skipped (those slots hold padding, which sorts last)
template <int NT, int K, typename TieKey>
__device__ void lds_bitonic_items(int n, RadixLds<NT, K>& S, TieKey tk)
{
    int N = 1;
    while (N < n) N <<= 1;
    auto cx = [&](int a, int b) {
        const uint2 A = S.items[rpad<K>(a)], B = S.items[rpad<K>(b)];
        if (B.x < A.x || (B.x == A.x && tk(B.y) < tk(A.y))) {
            S.items[rpad<K>(a)] = B;
            S.items[rpad<K>(b)] = A;
        }
    };
    for (int k = 2; k <= N; k <<= 1) {
        const int lh = __builtin_ctz((unsigned)k) - 1;
        for (int p = threadIdx.x; p < (N >> 1); p += NT) {
            const int blk = p >> lh, off = p & ((1 << lh) - 1);
            const int a = (blk << (lh + 1)) + off;
            const int b = a + k - 1 - 2 * off;
            if (b < n) cx(a, b);
        }
        __syncthreads();
        for (int j = k >> 2; j >= 1; j >>= 1) {
            const int lj = __builtin_ctz((unsigned)j);
            for (int p = threadIdx.x; p < (N >> 1); p += NT) {
                const int blk = p >> lj, off = p & (j - 1);
                const int a = (blk << (lj + 1)) + off;
                if (a + j < n) cx(a, a + j);
            }
            __syncthreads();
        }
    }
}

// copies len words from LDS to global memory (all NT threads): 16-byte
// stores once dst is aligned, single words at the ends
template <int NT>
__device__ __forceinline__ void copy_out(uint32_t* __restrict__ dst, const uint32_t* src, uint32_t len)
{
    const uint32_t mis = (uint32_t)(((uintptr_t)dst >> 2) & 3u);
    const uint32_t head = min(len, (4u - mis) & 3u);
    if (threadIdx.x < head) dst[threadIdx.x] = src[threadIdx.x];
    const uint32_t nb = (len - head) >> 2;
    uint4* d4 = reinterpret_cast<uint4*>(dst + head);
    for (uint32_t i = threadIdx.x; i < nb; i += NT) {
        const uint32_t o = head + 4u * i;
        d4[i] = make_uint4(src[o], src[o + 1], src[o + 2], src[o + 3]);
    }
    const uint32_t t0 = head + 4u * nb;
    if (threadIdx.x < len - t0) dst[t0 + threadIdx.x] = src[t0 + threadIdx.x];
}

// Filters the n sorted items into the region's local tiles, in order, four
// tiles at a time (row-major).  Wave w holds items [w c, w c + c) in registers
// (c = n / (NT/64) rounded up to 64, at most 64 K), 64 per step.  Per pass:
// each wave counts, per tile, its items whose mask holds the tile (one ballot
// per step and tile); 4 threads turn the counts into each wave's offset in
// each tile's piece; a second walk puts each wave's items there (ballot ranks
// give consecutive positions), into LDS when the pass's pieces fit there, and
// the pieces are then written out with 16-byte stores (each piece is one
// contiguous run of the tile's list).  tb / te: this thread's tile slot
// (threads below RS^2; tile_slot); s_tcur (optional): per-tile offsets
// carried over from earlier calls for the same region, advanced by this call.
template <int NT, int K>
__device__ void filter_region(int n, RegionLds<NT, K>& L, const RegionTiles& rt, const TileOut& to, unsigned lrs,
                              uint32_t tb, uint32_t te, uint32_t* s_tcur)
{
    constexpr int NW = NT / 64, SW = stage_words<NT, K>();
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int chunk = ((n + NW - 1) / NW + 63) & ~63;
    const int i0 = wid * chunk, i1 = min(n, i0 + chunk);
    const int steps = i1 > i0 ? (i1 - i0 + 63) >> 6 : 0;
    const unsigned rs = 1u << lrs;
    uint32_t pm[K], cx[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = i0 + 64 * k + lane;
        pm[k] = 0u;
        cx[k] = 0u;
        if (i < i1) {
            const uint32_t y = L.R.items[rpad<K>(i)].y;
            pm[k] = y >> 16;
            cx[k] = L.cidx[y & 0xffffu];
        }
    }
    if (threadIdx.x < rs * rs) {
        L.tslot[2 * threadIdx.x] = tb;
        L.tslot[2 * threadIdx.x + 1] = te;
    }
    __syncthreads();   // every wave holds its items: item slots and counters are staging space
    uint32_t* stage = reinterpret_cast<uint32_t*>(L.R.items);
    // the region's tiles four at a time in row-major order (RS = 2: the whole
    // region in one pass; RS = 4: a row per pass; RS = 8: half a row)
    for (unsigned j0 = 0; j0 < rs * rs; j0 += 4) {
        {
            // tile j0 + q: column j & (RS - 1), row j >> lrs; bits: its mask test
            uint32_t bits[4];
            bool tin[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const unsigned j = j0 + (unsigned)q, jx = j & (rs - 1u), jy = j >> lrs;
                tin[q] = jx < rt.tw && jy < rt.th;
                bits[q] = (1u << jx) | (1u << (8 + jy));
            }
            uint32_t cnt[4];
#pragma unroll
            for (int q = 0; q < 4; q++) cnt[q] = 0u;
#pragma unroll
            for (int k = 0; k < K; k++) {
                if (k < steps) {
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        if (tin[q]) cnt[q] += (uint32_t)__builtin_popcountll(gs::ballot((pm[k] & bits[q]) == bits[q]));
                    }
                }
            }
            if (lane == 0) {
#pragma unroll
                for (int q = 0; q < 4; q++) L.tab[wid * 4 + q] = cnt[q];
            }
            __syncthreads();
            if (threadIdx.x < 4) {
                const unsigned q = threadIdx.x, j = j0 + q;
                uint32_t b = ~0u, e = 0u;
                if ((j & (rs - 1u)) < rt.tw && (j >> lrs) < rt.th) {
                    b = L.tslot[2 * j];
                    e = L.tslot[2 * j + 1];
                }
                uint32_t run = 0u;
#pragma unroll
                for (int w = 0; w < NW; w++) {
                    const uint32_t v = L.tab[w * 4 + q];
                    L.tab[w * 4 + q] = run;
                    run += v;
                }
                uint32_t gs0 = b;
                if (b != ~0u && s_tcur != nullptr) gs0 += s_tcur[j];
                // a piece that would overrun its list (never by construction) is not written
                const bool ok = b != ~0u && gs0 + run <= e;
                L.piece[2 * q] = ok ? gs0 : ~0u;
                L.piece[2 * q + 1] = ok ? run : 0u;
                if (ok && s_tcur != nullptr) s_tcur[j] += run;
            }
            __syncthreads();
            uint32_t gq[4], so[4], pos[4];
            uint32_t total = 0u;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                gq[q] = __builtin_amdgcn_readfirstlane(L.piece[2 * q]);
                so[q] = total;
                total += __builtin_amdgcn_readfirstlane(L.piece[2 * q + 1]);
                pos[q] = __builtin_amdgcn_readfirstlane(L.tab[wid * 4 + q]);
            }
            const bool staged = total <= (uint32_t)SW;
#pragma unroll
            for (int k = 0; k < K; k++) {
                if (k < steps) {
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        if (gq[q] == ~0u) continue;
                        const bool hit = (pm[k] & bits[q]) == bits[q];
                        const uint64_t m = gs::ballot(hit);
                        if (hit) {
                            const uint32_t p = pos[q] + (uint32_t)gs::rank_below(m);
                            if (staged) stage[so[q] + p] = cx[k];
                            else to.clist[gq[q] + p] = cx[k];
                        }
                        pos[q] += (uint32_t)__builtin_popcountll(m);
                    }
                }
            }
            __syncthreads();
            if (staged) {
#pragma unroll 1
                for (int q = 0; q < 4; q++) {
                    const uint32_t len = __builtin_amdgcn_readfirstlane(L.piece[2 * q + 1]);
                    if (gq[q] != ~0u && len > 0u) copy_out<NT>(to.clist + gq[q], stage + so[q], len);
                }
            }
            __syncthreads();
        }
    }
}

// Bitonic sort of n region entries in global memory by (depth bits, compact
// index), in place (one block; pairs touching positions past n are skipped)
template <int NT>
__device__ void bitonic_entries(uint3* s, int n, int N)
{
    auto cx = [&](int a, int b) {
        const uint3 A = s[a], B = s[b];
        if (B.x < A.x || (B.x == A.x && B.y < A.y)) {
            s[a] = B;
            s[b] = A;
        }
    };
    for (int k = 2; k <= N; k <<= 1) {
        const int lh = __builtin_ctz((unsigned)k) - 1;
        for (int p = threadIdx.x; p < (N >> 1); p += NT) {
            const int blk = p >> lh, off = p & ((1 << lh) - 1);
            const int a = (blk << (lh + 1)) + off;
            const int b = a + k - 1 - 2 * off;
            if (b < n) cx(a, b);
        }
        __syncthreads();
        for (int j = k >> 2; j >= 1; j >>= 1) {
            const int lj = __builtin_ctz((unsigned)j);
            for (int p = threadIdx.x; p < (N >> 1); p += NT) {
                const int blk = p >> lj, off = p & (j - 1);
                const int a = (blk << (lj + 1)) + off;
                if (a + j < n) cx(a, a + j);
            }
            __syncthreads();
        }
    }
}

// Fallback filter over a region list sorted in global memory: one wave per tile.
template <int NT>
__device__ void filter_global(uint32_t start, int n, const uint3* __restrict__ rent, const RegionTiles& rt,
                              const TileOut& to, bool all_local)
{
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63;
    const int ntile = (int)(rt.tw * rt.th);
    for (int j = (int)(threadIdx.x >> 6); j < ntile; j += NW) {
        const unsigned jx = (unsigned)j % rt.tw, jy = (unsigned)j / rt.tw;
        const unsigned tt = (rt.ty0 + jy) * to.gx + rt.tx0 + jx;
        const int l = all_local ? (int)tt : to.loc_map[tt];
        if (l < 0) continue;
        const uint32_t bits = (1u << jx) | (1u << (8 + jy));
        const uint32_t base = to.tile_start[l], end = base + to.tile_count[l];
        uint32_t cur = 0u;
        for (int b = 0; b < n; b += 64) {
            const int i = b + lane;
            uint32_t m = 0u, cidx = 0u;
            if (i < n) {
                const uint3 v = rent[start + i];
                cidx = v.y;
                m = v.z;
            }
            const bool hit = (m & bits) == bits;
            const uint64_t mb = gs::ballot(hit);
            const uint32_t pos = base + cur + (uint32_t)gs::rank_below(mb);
            if (hit && pos < end) to.clist[pos] = cidx;
            cur += (uint32_t)__builtin_popcountll(mb);
        }
    }
}

// A region list longer than CAP = NT K: its entries are split into depth
// ranges of at most CAP (digit = 12 bits of the depth from its highest varying
// bit; range k = the digits whose exclusive prefix lies in [k CAP/2,
// (k+1) CAP/2), so a range holds at most CAP/2 plus its last digit's count),
// which are gathered, sorted and filtered one after another, the tile
// positions carried over.  A digit holding more than CAP/2 entries or a list
// of one depth: the whole list is sorted in global memory (bitonic, in place)
// and filtered from there (filter_global).  s_big: 4096 digit prefixes, then
// 64 tile positions.
template <int NT, int K>
__device__ void sort_filter_big(uint32_t start, int n, uint3* __restrict__ rent, RegionLds<NT, K>& L,
                                uint32_t* s_big, const RegionGrid& rg, int r, const TileOut& to, bool all_local)
{
    constexpr int CAP = NT * K, C = CAP / 2, NW = NT / 64, NDIG = 4096;
    const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
    RadixLds<NT, K>& S = L.R;
    const RegionTiles rt = region_tiles(rg, r);
    uint32_t* s_pre = s_big;
    uint32_t* s_tcur = s_big + NDIG;
    uint32_t* s_gather = S.misc + 3 * NW + 1;
    uint32_t* s_max = S.misc + 3 * NW + 2;
    uint32_t tb = ~0u, te = 0u;
    if ((unsigned)t < (1u << (2 * rg.lrs))) tile_slot((unsigned)t, rg.lrs, rt, to, all_local, tb, te);
    // passes over the list read 8 entries per thread at a time, all in flight
    constexpr int U = 8;
    auto pass = [&](auto&& f) {
        for (int i0 = 0; i0 < n; i0 += U * NT) {
            uint3 v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = i0 + t + u * NT;
                v[u] = i < n ? rent[start + i] : make_uint3(0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (i0 + t + u * NT < n) f(v[u]);
        }
    };
    uint32_t kor = 0u, kand = ~0u;
    pass([&](const uint3& v) {
        kor |= v.x;
        kand &= v.x;
    });
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        kor |= (uint32_t)__shfl_xor((int)kor, off, 64);
        kand &= (uint32_t)__shfl_xor((int)kand, off, 64);
    }
    if (lane == 0) { S.misc[wid] = kor; S.misc[NW + wid] = kand; }
    for (int i = t; i < NDIG; i += NT) s_pre[i] = 0u;
    if (t < 64) s_tcur[t] = 0u;
    if (t == 0) *s_max = 0u;
    __syncthreads();
    uint32_t vor = 0u, vand = ~0u;
#pragma unroll
    for (int w = 0; w < NW; w++) { vor |= S.misc[w]; vand &= S.misc[NW + w]; }
    const uint32_t vary = vor ^ vand;
    bool global_sort = vary == 0u;
    unsigned shift = 0u;
    if (!global_sort) {
        const int hb = 31 - __builtin_clz(vary);
        shift = hb >= 11 ? (unsigned)(hb - 11) : 0u;
        pass([&](const uint3& v) { atomicAdd(&s_pre[(v.x >> shift) & (NDIG - 1)], 1u); });
        __syncthreads();
        // exclusive scan of the digit counts in place; the largest count
        constexpr int PER = (NDIG + NT - 1) / NT;
        uint32_t loc[PER];
        uint32_t sum = 0u, mx = 0u;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int d = t * PER + j;
            const uint32_t v = d < NDIG ? s_pre[d] : 0u;
            loc[j] = v;
            sum += v;
            mx = max(mx, v);
        }
        uint32_t tot;
        uint32_t run = radix_block_scan<NT>(sum, S.misc + 2 * NW + 1, &tot);
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int d = t * PER + j;
            if (d < NDIG) s_pre[d] = run;
            run += loc[j];
        }
        atomicMax(s_max, mx);
        __syncthreads();
        global_sort = *s_max > (uint32_t)(CAP - C);
    }
    if (!global_sort) {
        auto tk = [&](uint32_t y) { return L.cidx[y & 0xffffu]; };
        const int nr = (n + C - 1) / C;
        for (int k = 0; k < nr; k++) {
            for (int i = t; i < CAP; i += NT) S.items[rpad<K>(i)] = make_uint2(~0u, ~0u);
            if (t == 0) *s_gather = 0u;
            __syncthreads();
            uint32_t gor = 0u, gand = ~0u;
            pass([&](const uint3& v) {
                if (s_pre[(v.x >> shift) & (NDIG - 1)] / (uint32_t)C == (uint32_t)k) {
                    const uint32_t p = atomicAdd(s_gather, 1u);
                    S.items[rpad<K>((int)p)] = make_uint2(v.x, p | (v.z << 16));
                    L.cidx[p] = v.y;
                    gor |= v.x;
                    gand &= v.x;
                }
            });
            __syncthreads();
            const int m = (int)*s_gather;
            if (radix_sort_items<NT, K>(m, S, gor, gand, tk)) lds_bitonic_items<NT, K>(m, S, tk);
            filter_region<NT, K>(m, L, rt, to, rg.lrs, tb, te, s_tcur);
        }
    } else {
        __syncthreads();
        int N = 1;
        while (N < n) N <<= 1;
        bitonic_entries<NT>(rent + start, n, N);
        filter_global<NT>(start, n, rent, rt, to, all_local);
    }
}

// One region: its list sorted on chip (radix_sort_items; a long run of equal
// depths: a bitonic network in LDS) and filtered into its tiles.  The caller
// separates consecutive regions with a barrier.
template <int NT, int K>
__device__ __forceinline__ void sort_filter_region(int r, const uint32_t* __restrict__ rcount,
                                                   const uint32_t* __restrict__ rstart, const uint3* __restrict__ rent,
                                                   RegionLds<NT, K>& L, const RegionGrid& rg, const TileOut& to,
                                                   bool all_local)
{
    auto tk = [&](uint32_t y) { return L.cidx[y & 0xffffu]; };
    const int n = (int)rcount[r];
    const RegionTiles rt = region_tiles(rg, r);
    uint32_t tb = ~0u, te = 0u;   // this thread's tile slot, loaded while the region sorts
    if (threadIdx.x < (1u << (2 * rg.lrs))) tile_slot(threadIdx.x, rg.lrs, rt, to, all_local, tb, te);
    uint32_t kor, kand;
    region_load<NT, K>(rstart[r], n, rent, L, kor, kand);
    if (radix_sort_items<NT, K>(n, L.R, kor, kand, tk)) lds_bitonic_items<NT, K>(n, L.R, tk);
    filter_region<NT, K>(n, L, rt, to, rg.lrs, tb, te, nullptr);
}

// Split path, step 4: one launch per region size class; its blocks walk the
// class's region list (block b takes entries b, b + gridDim.x, ...) and sort
// and filter each region (sort_filter_region).
template <int NT, int K>
__global__ __launch_bounds__(NT) void regionsort_kernel(const uint32_t* __restrict__ cls_count,
                                                        const int* __restrict__ cls_list,
                                                        const uint32_t* __restrict__ rcount,
                                                        const uint32_t* __restrict__ rstart,
                                                        const uint3* __restrict__ rent,
                                                        const uint32_t* __restrict__ meta, unsigned lrs, TileOut to)
{
    __shared__ RegionLds<NT, K> L;
    const RegionGrid rg = region_grid(meta, lrs);
    const bool all_local = meta[0] == to.gx * to.gy;
    if (meta[9] != 0u) return;   // R exceeded the caller's capacity: the lists were not written
    const int nl = (int)*cls_count;
    for (int e = blockIdx.x; e < nl; e += gridDim.x) {
        if (e != (int)blockIdx.x) __syncthreads();   // the previous region's reads of LDS are done
        sort_filter_region<NT, K>(cls_list[e], rcount, rstart, rent, L, rg, to, all_local);
    }
}

// The regions of up to 4096 entries (size classes 0..2) in one launch of
// 256-thread blocks: block b takes entries b, b + gridDim.x, ... of the class
// lists concatenated largest class first; a list of up to 2048 entries is
// sorted with 8 keys per thread, a longer one with 16 (the two layouts share
// the block's LDS).
__global__ __launch_bounds__(256, 2) void regionsort_small_kernel(const uint32_t* __restrict__ cls_count,
                                                               const int* __restrict__ cls_list, int NR,
                                                               const uint32_t* __restrict__ rcount,
                                                               const uint32_t* __restrict__ rstart,
                                                               const uint3* __restrict__ rent,
                                                               const uint32_t* __restrict__ meta, unsigned lrs,
                                                               TileOut to)
{
    static_assert(sizeof(RegionLds<256, 8>) <= sizeof(RegionLds<256, 16>), "shared layout");
    __shared__ RegionLds<256, 16> L16;
    RegionLds<256, 8>& L8 = *reinterpret_cast<RegionLds<256, 8>*>(&L16);
    const RegionGrid rg = region_grid(meta, lrs);
    const bool all_local = meta[0] == to.gx * to.gy;
    if (meta[9] != 0u) return;   // R exceeded the caller's capacity: the lists were not written
    const int n2 = (int)cls_count[2], n1 = (int)cls_count[1], n0 = (int)cls_count[0];
    for (int e = blockIdx.x; e < n2 + n1 + n0; e += gridDim.x) {
        if (e != (int)blockIdx.x) __syncthreads();   // the previous region's reads of LDS are done
        const int r = e < n2 ? cls_list[2 * (size_t)NR + e]
                             : e < n2 + n1 ? cls_list[(size_t)NR + (e - n2)] : cls_list[e - n2 - n1];
        if (rcount[r] > 2048u) sort_filter_region<256, 16>(r, rcount, rstart, rent, L16, rg, to, all_local);
        else sort_filter_region<256, 8>(r, rcount, rstart, rent, L8, rg, to, all_local);
    }
}

// the regions longer than NT K (sort_filter_big), one block each
template <int NT, int K>
__global__ __launch_bounds__(NT) void regionsort_big_kernel(const uint32_t* __restrict__ xcount,
                                                            const int* __restrict__ xlist,
                                                            const uint32_t* __restrict__ rcount,
                                                            const uint32_t* __restrict__ rstart,
                                                            uint3* __restrict__ rent,
                                                            const uint32_t* __restrict__ meta, unsigned lrs, TileOut to)
{
    __shared__ RegionLds<NT, K> L;
    __shared__ uint32_t s_big[4096 + 64];
    const RegionGrid rg = region_grid(meta, lrs);
    const bool all_local = meta[0] == to.gx * to.gy;
    if (meta[9] != 0u) return;   // R exceeded the caller's capacity: the lists were not written
    const int nx = (int)*xcount;
    for (int e = blockIdx.x; e < nx; e += gridDim.x) {
        if (e != (int)blockIdx.x) __syncthreads();
        const int r = xlist[e];
        sort_filter_big<NT, K>(rstart[r], (int)rcount[r], rent, L, s_big, rg, r, to, all_local);
    }
}

// The reference's sorted arrays from the compact list, on request: per
// local tile, point_list[i] = Gaussian id and point_list_keys[i] =
// (tile << 32) | depth bits of list position i.
__global__ __launch_bounds__(256) void pointlist_kernel(const uint2* __restrict__ ranges,
                                                        const uint32_t* __restrict__ clist,
                                                        const uint32_t* __restrict__ cid2id,
                                                        const float* __restrict__ depths,
                                                        uint32_t* __restrict__ point_list, uint64_t* __restrict__ keys)
{
    const uint32_t tile = blockIdx.x;
    const uint2 r = ranges[tile];
    for (uint32_t i = r.x + threadIdx.x; i < r.y; i += 256) {
        const uint32_t id = cid2id[clist[i]];
        point_list[i] = id;
        keys[i] = ((uint64_t)tile << 32) | (uint64_t)__float_as_uint(depths[id]);
    }
}

// ------------------------------------------------------------- blend

// Blend blocks -> (tile, quadrant).  Workgroups are dispatched to the 8 XCDs
// round-robin (block b runs on XCD b % 8) and each XCD has its own L2.  Tiles
// are grouped into 8x8-tile supertiles; supertile s belongs to XCD s % 8, and
// an XCD's blocks walk its supertiles in order, four quadrant waves per tile,
// so the waves resident on one XCD cover a compact patch of the image and
// share the records of the Gaussians overlapping it in that XCD's L2.
constexpr unsigned BLOCKS_PER_SUPER = SUPER * SUPER * 4;

__device__ __forceinline__ bool block_to_tile(unsigned b, unsigned gx, unsigned gy, unsigned sgx, unsigned NS,
                                              unsigned& tile, unsigned& quad, unsigned& tx, unsigned& ty)
{
    const unsigned xcd = b & 7u, slot = b >> 3;
    const unsigned st = (slot / BLOCKS_PER_SUPER) * 8u + xcd;
    if (st >= NS) return false;
    const unsigned loc = slot % BLOCKS_PER_SUPER;
    quad = loc & 3u;
    const unsigned t = loc >> 2;
    tx = (st % sgx) * SUPER + (t % SUPER);
    ty = (st / sgx) * SUPER + (t / SUPER);
    if (tx >= gx || ty >= gy) return false;
    tile = ty * gx + tx;
    return true;
}

struct Rec {
    float4 q0, q1, q2;
    uint32_t gid;      // Gaussian id (loaded only WITH_ID)
    float cut_power;   // alpha cut-off power of the blend's exact-exp window
};

template <bool WITH_ID>
__device__ __forceinline__ Rec load_rec(const float4* __restrict__ rec, uint32_t cx)
{
    const float4* r = rec + 4 * (size_t)cx;
    const float2 q3 = *reinterpret_cast<const float2*>(&r[3]);
    Rec o{r[0], r[1], r[2], 0u, q3.y};
    if (WITH_ID) o.gid = __float_as_uint(q3.x);
    return o;
}

__device__ __forceinline__ bool rec_may_touch(const Rec& r, float x0, float y0, float x1, float y1)
{
    return gs::may_touch_prepared(r.q2.y, r.q2.z, r.q2.w, r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, x0, y0, x1, y1);
}

// The pixel rectangle [x0, x1] x [y0, y1] spanned by the lanes set in m
// (m != 0; lane 8 y + x is pixel (qx0 + x, qy0 + y) of the quadrant): the
// staging cull of a batch tests against the pixels that can still take part
// in it.  Scalar bit arithmetic on the wave-uniform mask.
__device__ __forceinline__ void active_rect(uint64_t m, float qx0, float qy0, float& x0, float& y0, float& x1,
                                            float& y1)
{
    uint32_t c = (uint32_t)m | (uint32_t)(m >> 32);   // columns: OR of the eight row bytes
    c |= c >> 16;
    c |= c >> 8;
    c &= 0xffu;
    x0 = qx0 + (float)__builtin_ctz(c);
    x1 = qx0 + (float)(31 - __builtin_clz(c));
    y0 = qy0 + (float)(__builtin_ctzll(m) >> 3);
    y1 = qy0 + (float)((63 - __builtin_clzll(m)) >> 3);
}

// wave-private staging slots of one batch of 64 list entries
struct Stage {
    float4 a[64];   // x, y, -a/2, -b
    float4 b[64];   // -c/2, opacity, r, g
    float4 c[64];   // blue, tag bits, 1-based position in the tile's list (bits), alpha cut-off power
};

// Per-pixel state of the forward blend, and the blend of one staged entry
// (A, B, Cc as staged by stage_put) into it.  Branch-free: every lane
// evaluates the entry and the state changes are selects.  Shared by the
// forward kernels and the VALU probe (render_valu_probe), which therefore
// issue the same instructions per entry.
struct FwdPixel {
    float T;   // transmittance; negated once the pixel has finished (its final value is |T|)
    float C0, C1, C2;
    uint32_t last, n2l;
};

struct FwdStep {
    bool upd;
    uint64_t observe;   // the wave's pixels that observe the entry (ballot)
    float wgt;
};

__device__ __forceinline__ FwdStep fwd_blend_step(FwdPixel& p, const float4& A, const float4& B, const float4& Cc,
                                                  float pxf, float pyf)
{
    const float dx = A.x - pxf, dy = A.y - pyf;
    const float power = gs::power_of(A.z, A.w, B.x, dx, dy);
    float G;
    const float alpha = gs::blend_alpha(B.y, power, Cc.w, G);
    const float test_T = p.T * (1.0f - alpha);
    const bool use = p.T > 0.0f && !(power > 0.0f) && !(alpha < 1.0f / 255.0f);
    const bool fin = use && test_T < 0.0001f;
    const bool upd = use && !fin;
    // observed: taken (upd) with T > 0.5.  Then T (1 - alpha) >= 0.5 (1 - 0.99)
    // > 1e-4, so the pixel does not finish and the test is T > 0.5 && power
    // <= 0 && alpha >= 1/255: a ballot of each compare (scalar masks, no
    // vector select to re-form a predicate)
    const uint64_t observe =
        gs::ballot(p.T > 0.5f) & gs::ballot(!(power > 0.0f)) & gs::ballot(!(alpha < 1.0f / 255.0f));
    const float wgt = alpha * p.T;
    // a pixel that does not take the entry adds colour * 0 (exactly its colour)
    const float w = upd ? wgt : 0.f;
    p.C0 = __builtin_fmaf(B.z, w, p.C0);
    p.C1 = __builtin_fmaf(B.w, w, p.C1);
    p.C2 = __builtin_fmaf(Cc.x, w, p.C2);
    // a pixel finishes (the reference's T < 1e-4 stop) by negating T: the
    // sign is the live test (one compare, no separate flag), |T| its value
    p.T = upd ? test_T : (fin ? -p.T : p.T);
    p.n2l += upd ? 1u : 0u;
    p.last = upd ? (uint32_t)__float_as_int(Cc.z) : p.last;   // (staged 1-based)
    return FwdStep{upd, observe, wgt};
}

// stages entry k of the list; `tag` (Gaussian id in the forward, compact
// index in the backward) rides along in the blue slot's partner, and the
// entry's 1-based position k + 1 (the value a pixel's last contributor takes)
// in the next slot
__device__ __forceinline__ void stage_put(Stage& st, int slot, const Rec& r, uint32_t tag, int k)
{
    st.a[slot] = make_float4(r.q0.x, r.q0.y, -0.5f * r.q0.z, -r.q0.w);
    st.b[slot] = make_float4(-0.5f * r.q1.x, r.q1.y, r.q1.z, r.q1.w);
    st.c[slot] = make_float4(r.q2.x, __uint_as_float(tag), __int_as_float(k + 1), r.cut_power);
}

// Blend modes: the split path's render (observation counts and per-tile
// statistics), the full-image path's render (per pixel, the Gaussian of the
// largest blend weight alpha * T gets one count in accum_max_count, when that
// pointer is set) and its render_simp (the same plus every contribution's
// alpha * T and a count added to the Gaussian's accumulators, one atomic per
// wave and Gaussian).
constexpr int BLEND_SPLIT = 0, BLEND_FULL = 1, BLEND_SIMP = 2;
// render_geo of the split path (reference _r forward.cu:381-384,407-412): a
// second walk of the split render's lists that blends the five geometry
// maps (all_map, P x 5) with the colour's weights and writes them and the
// plane depth, and nothing else
constexpr int BLEND_GEO = 4;
// the split path's render and render_geo's maps in one walk: the colour
// outputs and statistics of BLEND_SPLIT, the maps and plane depth of BLEND_GEO
constexpr int BLEND_SPLIT_GEO = 5;
__host__ __device__ constexpr bool is_split(int mode) { return mode == BLEND_SPLIT || mode == BLEND_SPLIT_GEO; }
__host__ __device__ constexpr bool is_geo(int mode) { return mode == BLEND_GEO || mode == BLEND_SPLIT_GEO; }
constexpr int NUM_MAPS = 5;   // NUM_ALL_MAP (_r config.h:24)

// A caller's buffer that a blend kernel clears while it runs (n16: 16-byte
// words; none when 0): each block, after its walk, writes zeros over its
// share with streaming stores.  The blend kernels are VALU-bound and leave
// HBM bandwidth unused, so the clearing costs them little; the buffer is an
// output of a later step that then writes only its non-zero part (the
// preprocess backward's dL/dsh, cleared by the render backward) or stays
// zero (the render forward's geometry maps when render_geo is off).  The
// stores come after the walk: on this target vmcnt also counts stores, so
// stores issued first would hold up the walk's loads.
struct ClearBuf {
    float4* p;
    size_t n16;
};

__device__ __forceinline__ void clear_share(const ClearBuf& c)
{
    if (c.n16 == 0) return;
    const size_t share = (c.n16 + gridDim.x - 1) / gridDim.x;
    const size_t b0 = (size_t)blockIdx.x * share, b1 = min(c.n16, b0 + share);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    for (size_t i = b0 + threadIdx.x; i < b1; i += blockDim.x) gs::st_stream(&c.p[i], z);
}

// clears its buffer when the block leaves, by whichever return
struct ClearAtExit {
    const ClearBuf& c;
    __device__ ~ClearAtExit() { clear_share(c); }
};

struct FwdOut {
    float* out_color;
    float* final_T;
    uint32_t* n_contrib_px;
    uint32_t* n_contrib2loss_px;   // split
    int32_t* out_observe;          // split
    int32_t* n_consider;           // split
    int32_t* n_contrib_tile;       // split
    uint32_t* qwork;               // split: per quadrant (4 tile + quad) the largest last contributor
    float* accum_max_count;        // full (null: flag_max_count off), simp
    float* accum_weights;          // simp
    int32_t* accum_weights_count;  // simp
    const float* all_map;          // geo: (P,5)
    float* out_all_map;            // geo: (5,H,W)
    float* out_plane_depth;        // geo: (H,W)
    float focal_x, focal_y, cx, cy;   // geo: the plane depth's pixel rays
    ClearBuf clr;                  // split: a caller's buffer cleared after the walks (none: n16 == 0)
};

template <int MODE>
// (Waves per SIMD.  The split path's walk: seven (72 VGPRs; one 8-byte value
// spilled around the loop, none inside it): measured 2.5 % faster than six,
// and six was 3 % faster than the 84 VGPRs the compiler picks unbounded;
// eight force spills inside the loop and were slower.  The other paths: six;
// the fused render_geo walk carries five more accumulators: five, no spills.)
__global__ __launch_bounds__(64, MODE == BLEND_SPLIT ? 7 : (MODE == BLEND_SPLIT_GEO ? 5 : 6)) void render_fwd_kernel(
    int W, int H, unsigned gx, unsigned gy, unsigned sgx, unsigned NS, const uint2* __restrict__ ranges,
    const uint32_t* __restrict__ clist, const float4* __restrict__ rec, const uint8_t* __restrict__ cl,
    const float* __restrict__ bg, FwdOut O)
{
    [[maybe_unused]] const ClearAtExit clear_at_exit{O.clr};
    unsigned tile, quad, tx, ty;
    if (!block_to_tile(blockIdx.x, gx, gy, sgx, NS, tile, quad, tx, ty)) return;
    const int lane = threadIdx.x;
    const int qx = (int)tx * 16 + (int)(quad & 1u) * 8, qy = (int)ty * 16 + (int)(quad >> 1) * 8;
    const int px = qx + (lane & 7), py = qy + (lane >> 3);
    const bool inside = px < W && py < H;
    const size_t pid = (size_t)py * W + px;
    const size_t HW = (size_t)H * W;
    float* __restrict__ out_color = O.out_color;
    if (cl != nullptr && !cl[tile]) {
        if (inside) {
            if constexpr (is_geo(MODE)) {
                for (int c = 0; c < NUM_MAPS; c++) O.out_all_map[c * HW + pid] = 0.f;
                O.out_plane_depth[pid] = 0.f;
            }
            if constexpr (MODE != BLEND_GEO) {
                out_color[pid] = 0.f; out_color[HW + pid] = 0.f; out_color[2 * HW + pid] = 0.f;
                O.final_T[pid] = 0.f; O.n_contrib_px[pid] = 0;
                if (is_split(MODE)) O.n_contrib2loss_px[pid] = 0;
            }
        }
        if (is_split(MODE) && lane == 0) O.qwork[4 * tile + quad] = 0u;
        return;
    }
    __shared__ Stage st;
    __shared__ float st_map[is_geo(MODE) ? NUM_MAPS * 64 : 1];   // geo: the staged entries' maps
    [[maybe_unused]] float Mv[NUM_MAPS] = {0.f, 0.f, 0.f, 0.f, 0.f};

    const uint2 range = ranges[tile];
    const int n = (int)(range.y - range.x);
    const uint32_t* list = clist + range.x;
    const float pxf = (float)px, pyf = (float)py;
    const float qx0 = (float)qx, qy0 = (float)qy;
    FwdPixel px_st{inside ? 1.0f : -1.0f, 0.f, 0.f, 0.f, 0u, 0u};
    float wmax = 0.f;      // largest blend weight so far, and its Gaussian (full / simp)
    uint32_t imax = 0u;

    // software pipeline: while a batch blends, the next batch's records and
    // the list entries of the batch after it are in flight
    uint32_t id_cur = lane < n ? list[lane] : 0u;
    uint32_t id_nxt = 64 + lane < n ? list[64 + lane] : 0u;
    Rec r_cur{};
    if (lane < n) r_cur = load_rec<true>(rec, id_cur);

    for (int base = 0; base < n; base += 64) {
        const uint64_t live = gs::ballot(px_st.T > 0.0f);
        if (live == 0) break;
        const int k = base + lane;
        Rec r_nxt{};
        uint32_t id_nn = 0;
        if (k + 64 < n) r_nxt = load_rec<true>(rec, id_nxt);
        if (k + 128 < n) id_nn = list[k + 128];
        // stage the batch, keeping only Gaussians that can reach a pixel of
        // the quadrant that is still blending (a finished pixel takes no
        // further entry, so the others cannot change any output)
        float cx0, cy0, cx1, cy1;
        active_rect(live, qx0, qy0, cx0, cy0, cx1, cy1);
        const bool keep = k < n && rec_may_touch(r_cur, cx0, cy0, cx1, cy1);
        const uint64_t km = gs::ballot(keep);
        if (keep) stage_put(st, gs::rank_below(km), r_cur, r_cur.gid, k);
        if constexpr (is_geo(MODE)) {
            if (keep) {
                const int slot = gs::rank_below(km);
                const float* m = O.all_map + (size_t)NUM_MAPS * r_cur.gid;
                for (int c = 0; c < NUM_MAPS; c++) st_map[c * 64 + slot] = m[c];
            }
        }
        __syncthreads();
        const int cnt = (int)__builtin_popcountll(km);
        // Branch-free blend of one staged entry: every lane evaluates it and
        // the state changes are selects, so no exec-mask bookkeeping.  OBS
        // (split path): lane jj of obs_cnt takes the number of pixels that
        // observe entry jj (T > 0.5 when they blend it), added to the
        // Gaussian's out_observe after the batch, one atomic per entry.
        auto blend = [&](auto OBS, const float4& A, const float4& B, const float4& Cc, [[maybe_unused]] int jj,
                         [[maybe_unused]] uint32_t& obs_cnt) {
            const FwdStep f = fwd_blend_step(px_st, A, B, Cc, pxf, pyf);
            const bool upd = f.upd;
            const float wgt = f.wgt;
            if constexpr (is_geo(MODE)) {
                // the colour's update rule: a pixel that does not take the
                // entry adds map * 0
                const float w = upd ? wgt : 0.f;
                for (int c = 0; c < NUM_MAPS; c++) Mv[c] = __builtin_fmaf(st_map[c * 64 + jj], w, Mv[c]);
            }
            if constexpr (MODE == BLEND_GEO) {
            } else if constexpr (is_split(MODE)) {
                if constexpr (decltype(OBS)::value) {
                    const uint32_t m = (uint32_t)__builtin_popcountll(f.observe);
                    obs_cnt = gs::write_lane(obs_cnt, m, jj);
                }
            } else {
                const bool better = upd && wmax < wgt;
                wmax = better ? wgt : wmax;
                imax = better ? __float_as_uint(Cc.y) : imax;
                if (MODE == BLEND_SIMP) {
                    const uint64_t um = gs::ballot(upd);
                    if (um != 0) {
                        const float ws = gs::wave_sum(upd ? wgt : 0.f);
                        if (lane == (int)__builtin_ctzll(um)) {
                            atomicAdd(&O.accum_weights[__float_as_uint(Cc.y)], ws);
                            atomicAdd(&O.accum_weights_count[__float_as_uint(Cc.y)], (int)__builtin_popcountll(um));
                        }
                    }
                }
            }
        };
        // two register sets in turn: the next entry's LDS reads are issued
        // before this entry's arithmetic
        auto blend_batch = [&](auto OBS) {
            uint32_t obs_cnt = 0u;
            float4 A0 = st.a[0], B0 = st.b[0], D0 = st.c[0];
            float4 A1, B1, D1;
            for (int j = 0; j < cnt; j += 2) {
                if (gs::ballot(px_st.T > 0.0f) == 0) break;
                A1 = st.a[(j + 1) & 63]; B1 = st.b[(j + 1) & 63]; D1 = st.c[(j + 1) & 63];
                blend(OBS, A0, B0, D0, j, obs_cnt);
                if (j + 1 >= cnt) break;   // (the finished-pixel test runs once per pair)
                A0 = st.a[(j + 2) & 63]; B0 = st.b[(j + 2) & 63]; D0 = st.c[(j + 2) & 63];
                blend(OBS, A1, B1, D1, j + 1, obs_cnt);
            }
            if constexpr (decltype(OBS)::value) {
                if (obs_cnt != 0u) atomicAdd(&O.out_observe[__float_as_uint(st.c[lane].y)], (int)obs_cnt);
            }
        };
        // T only decreases, so a batch that starts with no live pixel above
        // T = 0.5 cannot observe (split path): it runs without the counts
        if (is_split(MODE) && gs::ballot(px_st.T > 0.5f) != 0)
            blend_batch(std::integral_constant<bool, is_split(MODE)>{});
        else
            blend_batch(std::false_type{});
        __syncthreads();
        r_cur = r_nxt;
        id_cur = id_nxt;
        id_nxt = id_nn;
    }

    if constexpr (is_geo(MODE)) {
        // plane depth (reference _r forward.cu:411): M4 / -(M0 rx + M1 ry + M2
        // + 1e-8), the 1e-8 a double literal there: the sum in float, the rest
        // in double
        if (inside) {
            for (int c = 0; c < NUM_MAPS; c++) O.out_all_map[c * HW + pid] = Mv[c];
            const float rx = (pxf - O.cx) / O.focal_x, ry = (pyf - O.cy) / O.focal_y;
            const float sdot = __builtin_fmaf(Mv[0], rx, Mv[1] * ry) + Mv[2];
            O.out_plane_depth[pid] = (float)((double)Mv[4] / -((double)sdot + 1.0e-8));
        }
        if constexpr (MODE == BLEND_GEO) return;
    }
    if (inside) {
        const float Tf = __builtin_fabsf(px_st.T);
        O.final_T[pid] = Tf;
        O.n_contrib_px[pid] = px_st.last;
        if (is_split(MODE)) O.n_contrib2loss_px[pid] = px_st.n2l;
        out_color[pid] = __builtin_fmaf(Tf, bg[0], px_st.C0);
        out_color[HW + pid] = __builtin_fmaf(Tf, bg[1], px_st.C1);
        out_color[2 * HW + pid] = __builtin_fmaf(Tf, bg[2], px_st.C2);
    }
    if (is_split(MODE)) {
        const int s_last = gs::wave_sum_i(inside ? (int)px_st.last : 0);
        const int s_n2l = gs::wave_sum_i(inside ? (int)px_st.n2l : 0);
        const int m_last = gs::wave_max_i(inside ? (int)px_st.last : 0);
        if (lane == 0) {
            if (s_last) atomicAdd(&O.n_consider[tile], s_last);
            if (s_n2l) atomicAdd(&O.n_contrib_tile[tile], s_n2l);
            O.qwork[4 * tile + quad] = (uint32_t)m_last;   // the backward's work for this wave
        }
    } else if (O.accum_max_count != nullptr && inside && px_st.last > 0) {
        atomicAdd(&O.accum_max_count[imax], 1.0f);
    }
}

__global__ __launch_bounds__(256) void zero_i32_kernel(int n, int32_t* __restrict__ p)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// ---------------------------------------------------------------- depth render
//
// render_depth of the full-image path (reference: _f/cuda_rasterizer/forward.cu:616-835,
// host rasterizer_impl.cu:671-847): the forward blend plus, per pixel, the
// intersection of the camera ray with each blended Gaussian's 3-sigma
// ellipsoid; the Gaussian of the largest blend weight alpha * T gives the
// pixel's depth, ray discriminant, hit point and id.  The reference's rules,
// kept as they are:
//   * the pixel ray runs from campos to inv(projmatrix) * (ndc.x * 1.0000001,
//     ndc.y * 1.0000001, z_far, 1) taken WITHOUT the division by w;
//   * the quaternion is used unnormalised; the ellipsoid radii are 3 * scale;
//   * a Gaussian whose ray parameter gives depth < 0 still adds its colour but
//     leaves T (and the depth state) unchanged;
//   * the per-pixel contributor count stays 0.
// Everything a Gaussian contributes independently of the pixel (rotation,
// ray origin in its frame, the constant term of the quadratic) is computed
// once when it is staged; the inverse projection is computed in double by
// every wave (64 lanes, ~200 double operations) from the device matrix.
constexpr int BLEND_DEPTH = 3;

struct DepthIO {
    const float* means3D;
    const float* scales;
    const float* rotations;
    const float* projmatrix;   // (4,4) as the settings tensor: column-major for the kernels
    const float* campos;
    float* out_pts;            // (3,H,W)
    float* out_depth;          // (1,H,W)
    float* accum_alpha;        // (1,H,W): final T
    int32_t* gidx;             // (1,H,W)
    float* discriminants;      // (1,H,W)
};

// Inverse of the 4x4 matrix whose element (r, c) is m[4c + r], by the
// expansion in complementary 2x2 minors, in double; written the same way.
__device__ void inv4_colmajor(const float* __restrict__ mf, float* __restrict__ out)
{
    double a[4][4];
    for (int c = 0; c < 4; c++)
        for (int r = 0; r < 4; r++) a[r][c] = (double)mf[4 * c + r];
    const double s0 = a[0][0] * a[1][1] - a[1][0] * a[0][1];
    const double s1 = a[0][0] * a[1][2] - a[1][0] * a[0][2];
    const double s2 = a[0][0] * a[1][3] - a[1][0] * a[0][3];
    const double s3 = a[0][1] * a[1][2] - a[1][1] * a[0][2];
    const double s4 = a[0][1] * a[1][3] - a[1][1] * a[0][3];
    const double s5 = a[0][2] * a[1][3] - a[1][2] * a[0][3];
    const double c5 = a[2][2] * a[3][3] - a[3][2] * a[2][3];
    const double c4 = a[2][1] * a[3][3] - a[3][1] * a[2][3];
    const double c3 = a[2][1] * a[3][2] - a[3][1] * a[2][2];
    const double c2 = a[2][0] * a[3][3] - a[3][0] * a[2][3];
    const double c1 = a[2][0] * a[3][2] - a[3][0] * a[2][2];
    const double c0 = a[2][0] * a[3][1] - a[3][0] * a[2][1];
    const double det = s0 * c5 - s1 * c4 + s2 * c3 + s3 * c2 - s4 * c1 + s5 * c0;
    const double id = 1.0 / det;
    double b[4][4];
    b[0][0] = (a[1][1] * c5 - a[1][2] * c4 + a[1][3] * c3) * id;
    b[0][1] = (-a[0][1] * c5 + a[0][2] * c4 - a[0][3] * c3) * id;
    b[0][2] = (a[3][1] * s5 - a[3][2] * s4 + a[3][3] * s3) * id;
    b[0][3] = (-a[2][1] * s5 + a[2][2] * s4 - a[2][3] * s3) * id;
    b[1][0] = (-a[1][0] * c5 + a[1][2] * c2 - a[1][3] * c1) * id;
    b[1][1] = (a[0][0] * c5 - a[0][2] * c2 + a[0][3] * c1) * id;
    b[1][2] = (-a[3][0] * s5 + a[3][2] * s2 - a[3][3] * s1) * id;
    b[1][3] = (a[2][0] * s5 - a[2][2] * s2 + a[2][3] * s1) * id;
    b[2][0] = (a[1][0] * c4 - a[1][1] * c2 + a[1][3] * c0) * id;
    b[2][1] = (-a[0][0] * c4 + a[0][1] * c2 - a[0][3] * c0) * id;
    b[2][2] = (a[3][0] * s4 - a[3][1] * s2 + a[3][3] * s0) * id;
    b[2][3] = (-a[2][0] * s4 + a[2][1] * s2 - a[2][3] * s0) * id;
    b[3][0] = (-a[1][0] * c3 + a[1][1] * c1 - a[1][2] * c0) * id;
    b[3][1] = (a[0][0] * c3 - a[0][1] * c1 + a[0][2] * c0) * id;
    b[3][2] = (-a[3][0] * s3 + a[3][1] * s1 - a[3][2] * s0) * id;
    b[3][3] = (a[2][0] * s3 - a[2][1] * s1 + a[2][2] * s0) * id;
    for (int c = 0; c < 4; c++)
        for (int r = 0; r < 4; r++) out[4 * c + r] = (float)b[r][c];
}

// staging slots of one batch for the depth render
struct DepthStage {
    float4 a[64];    // x, y, -a/2, -b
    float4 b[64];    // -c/2, opacity, r, g
    float4 c[64];    // blue, Gaussian id (bits), 0, alpha cut-off power
    float4 r0[64];   // rotation entries m0..m3 (glm column order)
    float4 r1[64];   // m4..m7
    float4 r2[64];   // m8, ray origin in the Gaussian's frame
    float4 s[64];    // 3 * scale, constant term of the quadratic
};

// glm::mat3(m0..m8) * v: m0..m2 is the first column
__device__ __forceinline__ float3 rot_apply(const float4& r0, const float4& r1, const float4& r2, float x, float y,
                                            float z)
{
    return make_float3(r0.x * x + r0.w * y + r1.z * z, r0.y * x + r1.x * y + r1.w * z, r0.z * x + r1.y * y + r2.x * z);
}

__global__ __launch_bounds__(64) void render_depth_kernel(int W, int H, unsigned gx, unsigned gy, unsigned sgx,
                                                          unsigned NS, const uint2* __restrict__ ranges,
                                                          const uint32_t* __restrict__ clist,
                                                          const float4* __restrict__ rec, const float* __restrict__ bg,
                                                          FwdOut O, DepthIO D)
{
    unsigned tile, quad, tx, ty;
    if (!block_to_tile(blockIdx.x, gx, gy, sgx, NS, tile, quad, tx, ty)) return;
    const int lane = threadIdx.x;
    const int qx = (int)tx * 16 + (int)(quad & 1u) * 8, qy = (int)ty * 16 + (int)(quad >> 1) * 8;
    const int px = qx + (lane & 7), py = qy + (lane >> 3);
    const bool inside = px < W && py < H;
    const size_t pid = (size_t)py * W + px;
    const size_t HW = (size_t)H * W;
    __shared__ DepthStage st;

    // the pixel's ray
    float inv[16];
    inv4_colmajor(D.projmatrix, inv);
    const float cx = D.campos[0], cy = D.campos[1], cz = D.campos[2];
    const float pxf = (float)px, pyf = (float)py;
    const float ndx = (2.0f * pxf + 1.0f) / (float)W - 1.0f;
    const float ndy = (2.0f * pyf + 1.0f) / (float)H - 1.0f;
    const float hx = (float)((double)ndx * 1.0000001), hy = (float)((double)ndy * 1.0000001);
    const float hz = (float)((100.0 - 100.0 * 0.01) / (100.0 - 0.01));
    const float ox = inv[0] * hx + inv[4] * hy + inv[8] * hz + inv[12];
    const float oy = inv[1] * hx + inv[5] * hy + inv[9] * hz + inv[13];
    const float oz = inv[2] * hx + inv[6] * hy + inv[10] * hz + inv[14];
    const float rdx = ox - cx, rdy = oy - cy, rdz = oz - cz;
    const float len = sqrtf(rdx * rdx + rdy * rdy + rdz * rdz);
    const float il = 1.0f / len;
    const float nx = rdx * il, ny = rdy * il, nz = rdz * il;

    const uint2 range = ranges[tile];
    const int n = (int)(range.y - range.x);
    const uint32_t* list = clist + range.x;
    const float qx0 = (float)qx, qy0 = (float)qy;
    const float alpha_min = 1.0f / 255.0f;
    float T_ = 1.0f, C0 = 0.f, C1 = 0.f, C2 = 0.f;
    float wmax = 0.f, dmax = 0.f, discmax = 0.f, prx = 0.f, pry = 0.f, prz = 0.f;
    uint32_t imax = 0u;
    bool done = !inside;

    for (int base = 0; base < n; base += 64) {
        if (gs::ballot(!done) == 0) break;
        const int k = base + lane;
        Rec r{};
        if (k < n) r = load_rec<true>(rec, list[k]);
        const bool keep = k < n && rec_may_touch(r, qx0, qy0, qx0 + 7.0f, qy0 + 7.0f);
        const uint64_t km = gs::ballot(keep);
        if (keep) {
            const int slot = gs::rank_below(km);
            st.a[slot] = make_float4(r.q0.x, r.q0.y, -0.5f * r.q0.z, -r.q0.w);
            st.b[slot] = make_float4(-0.5f * r.q1.x, r.q1.y, r.q1.z, r.q1.w);
            st.c[slot] = make_float4(r.q2.x, __uint_as_float(r.gid), 0.f, r.cut_power);
            const uint32_t g = r.gid;
            const float4 q = reinterpret_cast<const float4*>(D.rotations)[g];
            const float qr = q.x, qxx = q.y, qy_ = q.z, qz = q.w;
            const float m0 = 1.f - 2.f * (qy_ * qy_ + qz * qz), m1 = 2.f * (qxx * qy_ - qr * qz);
            const float m2 = 2.f * (qxx * qz + qr * qy_), m3 = 2.f * (qxx * qy_ + qr * qz);
            const float m4 = 1.f - 2.f * (qxx * qxx + qz * qz), m5 = 2.f * (qy_ * qz - qr * qxx);
            const float m6 = 2.f * (qxx * qz - qr * qy_), m7 = 2.f * (qy_ * qz + qr * qxx);
            const float m8 = 1.f - 2.f * (qxx * qxx + qy_ * qy_);
            const float4 R0 = make_float4(m0, m1, m2, m3), R1 = make_float4(m4, m5, m6, m7);
            const float tx_ = cx - D.means3D[3 * (size_t)g], ty_ = cy - D.means3D[3 * (size_t)g + 1],
                        tz_ = cz - D.means3D[3 * (size_t)g + 2];
            const float4 R2p = make_float4(m8, 0.f, 0.f, 0.f);
            const float3 ro = rot_apply(R0, R1, R2p, tx_, ty_, tz_);
            const float sx = D.scales[3 * (size_t)g] * 3.0f, sy = D.scales[3 * (size_t)g + 1] * 3.0f,
                        sz = D.scales[3 * (size_t)g + 2] * 3.0f;
            const float cc = ro.x / sx * ro.x / sx + ro.y / sy * ro.y / sy + ro.z / sz * ro.z / sz - 1.0f;
            st.r0[slot] = R0;
            st.r1[slot] = R1;
            st.r2[slot] = make_float4(m8, ro.x, ro.y, ro.z);
            st.s[slot] = make_float4(sx, sy, sz, cc);
        }
        __syncthreads();
        const int cnt = (int)__builtin_popcountll(km);
        for (int j = 0; j < cnt; j++) {
            if (gs::ballot(!done) == 0) break;
            if (done) continue;
            const float4 A = st.a[j], B = st.b[j], Cc = st.c[j];
            const float dx = A.x - pxf, dy = A.y - pyf;
            const float power = gs::power_of(A.z, A.w, B.x, dx, dy);
            if (power > 0.0f) continue;
            float G;
            const float alpha = gs::blend_alpha(B.y, power, Cc.w, G);
            if (alpha < alpha_min) continue;
            const float test_T = T_ * (1.0f - alpha);
            if (test_T < 0.0001f) { done = true; continue; }
            C0 = __builtin_fmaf(B.z * alpha, T_, C0);
            C1 = __builtin_fmaf(B.w * alpha, T_, C1);
            C2 = __builtin_fmaf(Cc.x * alpha, T_, C2);
            const float4 R0 = st.r0[j], R1 = st.r1[j], R2 = st.r2[j], S = st.s[j];
            const float3 rd = rot_apply(R0, R1, R2, nx, ny, nz);
            const float a = rd.x / S.x * rd.x / S.x + rd.y / S.y * rd.y / S.y + rd.z / S.z * rd.z / S.z;
            const float b = 2.0f * (rd.x / S.x * R2.y / S.x + rd.y / S.y * R2.z / S.y + rd.z / S.z * R2.w / S.z);
            const float disc = b * b - 4.0f * a * S.w;
            const float tpar = -b / 2.0f / a;
            const float depth = tpar / len;
            if (depth < 0.0f) continue;
            const float wgt = alpha * T_;
            if (wmax < wgt) {
                wmax = wgt;
                dmax = depth;
                discmax = disc;
                imax = __float_as_uint(Cc.y);
                prx = cx + tpar * nx;
                pry = cy + tpar * ny;
                prz = cz + tpar * nz;
            }
            T_ = test_T;
        }
        __syncthreads();
    }

    if (inside) {
        O.final_T[pid] = T_;
        O.n_contrib_px[pid] = 0u;
        O.out_color[pid] = __builtin_fmaf(T_, bg[0], C0);
        O.out_color[HW + pid] = __builtin_fmaf(T_, bg[1], C1);
        O.out_color[2 * HW + pid] = __builtin_fmaf(T_, bg[2], C2);
        D.out_pts[pid] = prx;
        D.out_pts[HW + pid] = pry;
        D.out_pts[2 * HW + pid] = prz;
        D.out_depth[pid] = dmax;
        D.accum_alpha[pid] = T_;
        D.discriminants[pid] = discmax;
        D.gidx[pid] = (int32_t)imax;
    }
}

// Clears the gradient accumulators of the listed Gaussians (meta[4] of them)
// before a backward accumulates into them (blocks nsched and up), beside the
// backward's block order (blocks 0 .. nsched - 1, bwd_schedule_block; nsched
// is 8, or 0 without a schedule).
__device__ void bwd_schedule_block(unsigned x, unsigned gx, unsigned gy, unsigned sgx, unsigned NS,
                                   const uint32_t* __restrict__ qwork, uint32_t* __restrict__ sched,
                                   uint32_t* __restrict__ scnt);

__global__ __launch_bounds__(1024) void zero_gacc_kernel(const uint32_t* __restrict__ meta, float4* __restrict__ gacc,
                                                         unsigned nsched, unsigned gx, unsigned gy, unsigned sgx,
                                                         unsigned NS, const uint32_t* __restrict__ qwork,
                                                         uint32_t* __restrict__ sched, uint32_t* __restrict__ scnt)
{
    if (blockIdx.x < nsched) {
        bwd_schedule_block(blockIdx.x, gx, gy, sgx, NS, qwork, sched, scnt);
        return;
    }
    const size_t n4 = 4 * (size_t)meta[4];
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    for (size_t i = (size_t)(blockIdx.x - nsched) * blockDim.x + threadIdx.x; i < n4;
         i += (size_t)(gridDim.x - nsched) * blockDim.x)
        gacc[i] = z;
}

// Writes the k-float rows (k = 2 or 3) of a wave's 64 consecutive Gaussians
// as one contiguous run: the rows are staged in the wave's LDS slice and
// leave as 16-byte streaming stores that fill whole cache lines.
__device__ __forceinline__ void emit_rows(float* __restrict__ S, int lane, int k, float* __restrict__ out,
                                          int base, float v0, float v1, float v2)
{
    S[lane * k] = v0;
    S[lane * k + 1] = v1;
    if (k == 3) S[lane * k + 2] = v2;
    __builtin_amdgcn_wave_barrier();
    float4* dst = reinterpret_cast<float4*>(out + (size_t)base * k);
    const float4* src = reinterpret_cast<const float4*>(S);
    for (int e = lane; e < 16 * k; e += 64) gs::st_stream(dst + e, src[e]);
    __builtin_amdgcn_wave_barrier();
}

// Writes the render backward's outputs for every Gaussian from its
// accumulator (listed Gaussians) or zeros, one Gaussian per thread, applying
// the factors the blend leaves to the sums: dmean/dpixel (sx = W/2, sy = H/2)
// to the mean terms, -1/2 to the conic terms.  A wave whose 64 Gaussians are
// all in range writes its rows through emit_rows when the outputs are 16-byte
// aligned (vec); otherwise element by element.
__global__ __launch_bounds__(256) void unpack_grads_kernel(int P, const int* __restrict__ cidx_of,
                                                           const float4* __restrict__ gacc, int m2d_stride,
                                                           float* __restrict__ g_m2d, float* __restrict__ g_m2d_abs,
                                                           float4* __restrict__ g_con, float* __restrict__ g_col,
                                                           bool vec, float sx, float sy)
{
    __shared__ __align__(16) float stage[4][64 * 3];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int base = (int)(blockIdx.x * 4 + w) * 64;
    if (base >= P) return;                         // the whole wave leaves; no block barrier follows
    const int i = base + lane;
    const bool in = i < P;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    // a = dmean x, dmean y, |dmean x|, |dmean y|; b = dconic a, b, c, dopacity; c = drgb
    float4 a = z, b = z, c = z;
    if (in && cidx_of != nullptr) {
        const int cx = cidx_of[i];
        if (cx >= 0) {
            const float4* g = gacc + 4 * (size_t)cx;
            a = g[0]; b = g[1]; c = g[2];
            a = make_float4(a.x * sx, a.y * sy, a.z * sx, a.w * sy);
            b = make_float4(-0.5f * b.x, -0.5f * b.y, -0.5f * b.z, b.w);
        }
    }
    if (in) gs::st_stream(&g_con[i], b);
    if (vec && base + 64 <= P) {
        float* S = stage[w];
        emit_rows(S, lane, m2d_stride, g_m2d, base, a.x, a.y, 0.f);
        if (g_m2d_abs != nullptr) emit_rows(S, lane, 3, g_m2d_abs, base, a.z, a.w, 0.f);
        emit_rows(S, lane, 3, g_col, base, c.x, c.y, c.z);
        return;
    }
    if (!in) return;
    float* m = g_m2d + (size_t)i * m2d_stride;
    gs::st_stream(&m[0], a.x);
    gs::st_stream(&m[1], a.y);
    if (m2d_stride == 3) gs::st_stream(&m[2], 0.f);
    if (g_m2d_abs != nullptr) {
        gs::st_stream(&g_m2d_abs[3 * (size_t)i], a.z);
        gs::st_stream(&g_m2d_abs[3 * (size_t)i + 1], a.w);
        gs::st_stream(&g_m2d_abs[3 * (size_t)i + 2], 0.f);
    }
    gs::st_stream(&g_col[3 * (size_t)i], c.x);
    gs::st_stream(&g_col[3 * (size_t)i + 1], c.y);
    gs::st_stream(&g_col[3 * (size_t)i + 2], c.z);
}

// render_geo: dL/dall_map (P,5) from accumulator slots 11..15 of the listed
// Gaussians (cidx_of[i] >= 0), zeros for the others and when nothing was
// listed (cidx_of null)
__global__ __launch_bounds__(256) void unpack_map_grads_kernel(int P, const int* __restrict__ cidx_of,
                                                               const float* __restrict__ gacc,
                                                               float* __restrict__ g_map)
{
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= P) return;
    const int cx = cidx_of != nullptr ? cidx_of[i] : -1;
    for (int c = 0; c < NUM_MAPS; c++)
        g_map[(size_t)NUM_MAPS * i + c] = cx >= 0 ? gacc[(size_t)cx * 16 + 11 + c] : 0.f;
}

// Per-pixel state and constants of the backward blend, and the backward of
// one staged entry for one pixel: updates the state and returns whether the
// pixel blends the entry, with its eleven gradient terms in vals (dmean x, y,
// |dmean x|, |dmean y|, dconic a, b, c, dopacity, drgb; vals[11] = 0).
// Shared by the backward kernels and the VALU probe (render_valu_probe).
// Per-pixel state of the backward walk.  The accumulated colour behind the
// current entry and the last blended colour enter the gradient only through
// their dot products with dL/dpixel, and the accumulation is linear, so the
// state keeps those two dot products instead of the six channel values.
struct BwdPixel {
    float T;            // transmittance in front of the current entry
    float acc_dp;       // (colour accumulated behind it) . dL/dpixel
    float last_dp;      // (colour of the last blended entry) . dL/dpixel
    float last_alpha;
};

struct BwdConst {
    float pxf, pyf, dp0, dp1, dp2, nT_bg;
    int last;
};

// One entry of the backward for this lane's pixel, in two parts: bwd_eval
// decides whether the pixel blends the entry (the forward's exact alpha
// expressions), and bwd_apply, which the caller skips when no lane of the
// wave blends it (the state update is then the identity for every lane),
// updates the pixel's state and yields the entry's twelve gradient terms.
struct BwdEval {
    float dx, dy, hadx, hcdy, nbdx, alpha, G0;
    bool valid;
};

__device__ __forceinline__ BwdEval bwd_eval(const BwdConst& k, const float4& A, const float4& B, const float4& Cc)
{
    BwdEval e;
    const int ci1 = __float_as_int(Cc.z);   // 1-based position in the tile's list
    e.dx = A.x - k.pxf;
    e.dy = A.y - k.pyf;
    // gs::power_of's operations, with the products ha dx, hc dy, nb dx kept
    // for the gradient
    e.hadx = A.z * e.dx;
    e.hcdy = B.x * e.dy;
    e.nbdx = A.w * e.dx;
    const float power = __builtin_fmaf(e.hadx, e.dx, __builtin_fmaf(e.hcdy, e.dy, e.nbdx * e.dy));
    e.alpha = gs::blend_alpha(B.y, power, Cc.w, e.G0);
    e.valid = ci1 <= k.last && !(power > 0.0f) && !(e.alpha < (1.0f / 255.0f));
    return e;
}

// Branch-free: every lane applies the entry; a lane whose pixel does not
// blend it (past its last contributor, power > 0, alpha < 1/255) gets zero
// gradient factors and unchanged state, through selects on three factors
// instead of per-value zeroing.  GEO (render_geo): m_dp is the entry's five
// maps dotted with the pixel's map gradients; the maps join the colour in
// every dot product (the accumulation is the same linear rule for all eight
// channels).  Returns alpha T, the factor of the colour and map gradients.
template <bool FULL, bool GEO = false>
__device__ __forceinline__ float bwd_apply(BwdPixel& p, const BwdConst& k, const float4& A, const float4& B,
                                           const float4& Cc, const BwdEval& e, float (&vals)[12],
                                           [[maybe_unused]] float m_dp = 0.f)
{
    const bool valid = e.valid;
    const float dx = e.dx, dy = e.dy;
    // a lane that does not blend the entry runs it with alpha = 0 and G = 0:
    // T is unchanged (1 / (1 - 0) is exactly 1), and every gradient term
    // carries a factor alpha (colour) or G (the others; dL/dalpha stays finite)
    const float alpha = valid ? e.alpha : 0.f;
    const float G = valid ? e.G0 : 0.f;
    const float inv_one_m = __builtin_amdgcn_rcpf(1.f - alpha);   // 1 ulp; gradients only
    p.T = p.T * inv_one_m;
    const float dchannel_dcolor = alpha * p.T;
    // the reference's expressions, regrouped into fused multiply-adds and
    // taken in their dot products with dL/dpixel (gradients carry a
    // tolerance, not bit-exactness):
    //   acc = la * lc + (1 - la) * acc        -> acc.dp += la * (lc.dp - acc.dp)
    //   dL/dalpha = sum_ch (c - acc) dp_ch    -> c.dp - acc.dp
    //   (ha = -a/2, nb = -b, hc = -c/2 are the staged conic terms);
    // a lane that does not blend the entry updates acc with factor 0
    const float la = valid ? p.last_alpha : 0.f;
    p.acc_dp = __builtin_fmaf(la, p.last_dp - p.acc_dp, p.acc_dp);
    float c_dp = __builtin_fmaf(B.z, k.dp0, __builtin_fmaf(B.w, k.dp1, Cc.x * k.dp2));
    if constexpr (GEO) c_dp += m_dp;
    p.last_dp = valid ? c_dp : p.last_dp;
    p.last_alpha = valid ? alpha : p.last_alpha;
    float dL_dalpha = c_dp - p.acc_dp;
    const float gc0 = dchannel_dcolor * k.dp0;
    const float gc1 = dchannel_dcolor * k.dp1;
    const float gc2 = dchannel_dcolor * k.dp2;
    dL_dalpha = __builtin_fmaf(dL_dalpha, p.T, inv_one_m * k.nT_bg);
    const float dL_dG = B.y * dL_dalpha;
    // dG/ddelx = G (2 ha dx + nb dy), dG/ddely = G (2 hc dy + nb dx)
    const float dpx = __builtin_fmaf(2.0f, e.hadx, A.w * dy);
    const float dpy = __builtin_fmaf(2.0f, e.hcdy, e.nbdx);
    const float wG = dL_dG * G;
    // the constant factors dmean/dpixel (W/2, H/2) and the conic terms' -1/2
    // are applied once to the sums (unpack_grads_kernel), not per entry
    const float gmx = wG * dpx;
    const float gmy = wG * dpy;
    const float wdx = wG * dx;
    const bool clamped = FULL && B.y * G > 0.99f;
    const float gca = clamped ? 0.f : wdx * dx;
    const float gcb = clamped ? 0.f : wdx * dy;
    const float gcc = clamped ? 0.f : (wG * dy) * dy;
    const float gop = clamped ? 0.f : G * dL_dalpha;
    // vals[2], vals[3]: |dmean| terms, made absolute by wave_sum12<true>
    vals[0] = gmx; vals[1] = gmy; vals[2] = gmx; vals[3] = gmy;
    vals[4] = gca; vals[5] = gcb; vals[6] = gcc; vals[7] = gop;
    // slot 11 is never read back: any register that is dead here fills it
    // (no zero has to be materialised for it)
    vals[8] = gc0; vals[9] = gc1; vals[10] = gc2; vals[11] = dx;
    return dchannel_dcolor;
}

// render_geo's backward inputs (reference _r backward.cu:335-347)
struct GeoBwd {
    const float* all_map;     // (P,5)
    const float* map_px;      // (5,H,W): the forward's out_all_map
    const float* dL_dmaps;    // (5,H,W)
    const float* dL_dplane;   // (H,W)
    float fx, fy;             // focal lengths
};

// The backward's block order: per XCD (one block each), the tiles of its
// supertiles (supertile s on XCD s % 8, as block_to_tile) with any work,
// heaviest first -- a tile's work is the largest last contributor of its four
// quadrants, which the forward recorded (qwork; the backward walks each
// quadrant's list from that position to 0).  Waves are dispatched in block
// order, so the long ones start first and the short ones fill in at the end
// instead of a long one starting last.  The order is by work class (two per
// octave of the work, heaviest first) and, inside a class, the supertile
// order, so that the tiles walked at the same time on an XCD are mostly
// neighbours and share the records they read in its L2: an exact sort on the
// work scattered them and raised the kernel's HBM reads at config 2 from 0.30
// to 0.51 GB at the same speed; one class per octave reads 0.21 GB but was 2 %
// slower.  A stable counting sort: per round of 1024 tiles, each wave ranks its
// tiles of a class by a ballot, then the waves' counts are scanned in order.
// (one 1024-thread block per XCD x, inside zero_gacc_kernel)
__device__ void bwd_schedule_block(unsigned x, unsigned gx, unsigned gy, unsigned sgx, unsigned NS,
                                   const uint32_t* __restrict__ qwork, uint32_t* __restrict__ sched,
                                   uint32_t* __restrict__ scnt)
{
    constexpr int NB = 32;   // work classes, two per octave, heaviest first
    __shared__ uint32_t s_base[NB];
    __shared__ uint32_t s_wcnt[16][NB];
    const unsigned cap = sched_cap(NS);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    // i-th tile of the XCD in supertile order -> tile index, or -1
    auto tile_of = [&](unsigned i) -> int {
        const unsigned st = (i / (SUPER * SUPER)) * 8u + x, t = i % (SUPER * SUPER);
        if (st >= NS) return -1;
        const unsigned tx = (st % sgx) * SUPER + t % SUPER, ty = (st / sgx) * SUPER + t / SUPER;
        return tx < gx && ty < gy ? (int)(ty * gx + tx) : -1;
    };
    auto class_of = [&](int tile) -> int {
        const uint4 q = reinterpret_cast<const uint4*>(qwork)[tile];
        const uint32_t w = min(max(max(q.x, q.y), max(q.z, q.w)), 0xffffu);
        if (w == 0u) return -1;
        const int lg = 31 - __builtin_clz(w);
        const int c = 2 * lg + (lg > 0 ? (int)((w >> (lg - 1)) & 1u) : 0);
        return NB - 1 - c;
    };
    if (threadIdx.x < NB) s_base[threadIdx.x] = 0u;
    __syncthreads();
    for (unsigned i = threadIdx.x; i < cap; i += 1024) {
        const int t = tile_of(i);
        const int c = t >= 0 ? class_of(t) : -1;
        if (c >= 0) atomicAdd(&s_base[c], 1u);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0u;
        for (int c = 0; c < NB; c++) {
            const uint32_t v = s_base[c];
            s_base[c] = run;
            run += v;
        }
        scnt[x] = run;
    }
    __syncthreads();
    // in each class, the tiles in supertile order (neighbours stay together)
    for (unsigned r0 = 0; r0 < cap; r0 += 1024) {
        const unsigned i = r0 + threadIdx.x;
        const int t = i < cap ? tile_of(i) : -1;
        const int cls = t >= 0 ? class_of(t) : -1;
        uint32_t rank = 0u;
        for (int c = 0; c < NB; c++) {
            const uint64_t m = gs::ballot(cls == c);
            if (cls == c) rank = (uint32_t)gs::rank_below(m);
            if (lane == 0) s_wcnt[wid][c] = (uint32_t)__builtin_popcountll(m);
        }
        __syncthreads();
        if (cls >= 0) {
            uint32_t off = s_base[cls];
            for (int w = 0; w < wid; w++) off += s_wcnt[w][cls];
            sched[(size_t)x * cap + off + rank] = (uint32_t)t;
        }
        __syncthreads();
        if (threadIdx.x < NB) {
            uint32_t tot = 0u;
            for (int w = 0; w < 16; w++) tot += s_wcnt[w][threadIdx.x];
            s_base[threadIdx.x] += tot;
        }
        __syncthreads();
    }
}

// The split path's backward over a 16x8 half tile (half 0: pixel rows 0-7,
// 1: rows 8-15) in one wave, two pixels per lane: lane l takes the pixels
// (x0 + l % 8, y) and (x0 + 8 + l % 8, y), y = y0 + l / 8.  Each staged
// entry is evaluated for both pixels and their twelve terms enter one wave
// reduction (the |dmean| terms as |a| + |b| per lane), so the reduction and
// the atomics are paid once per two pixels.  It pays when the Gaussians are
// wide enough that an entry the wave admits usually touches both 8x8 halves
// of the 16x8 footprint: the blocks take it when a Gaussian has
// TWO_PX_MIN_INSTANCES tile instances or more on average (two_px_lanes).
// Measured: config 1 (R / L = 55) 0.402 -> 0.366 ms, config 2 (R / L = 7.2)
// 0.651 -> 0.727 ms; a model of the two walks' admitted entries puts the
// break-even at R / L ~ 24 on both scene families.
constexpr uint64_t TWO_PX_MIN_INSTANCES = 24;

__device__ __forceinline__ bool two_px_lanes(const uint32_t* __restrict__ meta)
{
    const uint64_t R = (uint64_t)meta[2] | ((uint64_t)meta[3] << 32), L = meta[4];
    return R >= TWO_PX_MIN_INSTANCES * L;
}

__device__ __forceinline__ void bwd_half_tile(int W, int H, unsigned gx, unsigned tile, unsigned half,
                                              const uint2* __restrict__ ranges, const uint32_t* __restrict__ clist,
                                              const float4* __restrict__ rec, const float* __restrict__ bg,
                                              const float* __restrict__ final_T,
                                              const uint32_t* __restrict__ n_contrib_px,
                                              const float* __restrict__ dL_dpixels, float* __restrict__ gacc,
                                              Stage& st)
{
    const unsigned tx = tile % gx, ty = tile / gx;
    const int lane = threadIdx.x;
    const int qx = (int)tx * 16, qy = (int)ty * 16 + (int)half * 8;
    const int pxa = qx + (lane & 7), pxb = pxa + 8, py = qy + (lane >> 3);
    const bool ina = pxa < W && py < H, inb = pxb < W && py < H;
    const size_t pida = (size_t)py * W + pxa, pidb = pida + 8;
    const size_t HW = (size_t)H * W;
    const float Tfa = ina ? final_T[pida] : 0.f, Tfb = inb ? final_T[pidb] : 0.f;
    const int lasta = ina ? (int)n_contrib_px[pida] : 0, lastb = inb ? (int)n_contrib_px[pidb] : 0;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, b0 = 0.f, b1 = 0.f, b2 = 0.f;
    if (ina) { a0 = dL_dpixels[pida]; a1 = dL_dpixels[HW + pida]; a2 = dL_dpixels[2 * HW + pida]; }
    if (inb) { b0 = dL_dpixels[pidb]; b1 = dL_dpixels[HW + pidb]; b2 = dL_dpixels[2 * HW + pidb]; }
    const int maxlast = gs::wave_max_i(max(lasta, lastb));
    if (maxlast == 0) return;

    const uint32_t* list = clist + ranges[tile].x;
    const float qx0 = (float)qx, qy0 = (float)qy;
    const float bga = bg[0] * a0 + bg[1] * a1 + bg[2] * a2, bgb = bg[0] * b0 + bg[1] * b1 + bg[2] * b2;
    const BwdConst ka{(float)pxa, (float)py, a0, a1, a2, -Tfa * bga, lasta};
    const BwdConst kb{(float)pxb, (float)py, b0, b1, b2, -Tfb * bgb, lastb};
    const int my_k = gs::wave_sum12_index(lane);
    BwdPixel pa{Tfa, 0.f, 0.f, 0.f}, pb{Tfb, 0.f, 0.f, 0.f};

    // the same walk and software pipeline as the 8x8 quadrant waves
    uint32_t id_cur = maxlast - 1 - lane >= 0 ? list[maxlast - 1 - lane] : 0u;
    uint32_t id_nxt = maxlast - 65 - lane >= 0 ? list[maxlast - 65 - lane] : 0u;
    Rec r_cur{};
    if (maxlast - 1 - lane >= 0) r_cur = load_rec<false>(rec, id_cur);

    for (int top = maxlast; top > 0; top -= 64) {
        const int k = top - 1 - lane;
        Rec r_nxt{};
        uint32_t id_nn = 0;
        if (k - 64 >= 0) r_nxt = load_rec<false>(rec, id_nxt);
        if (k - 128 >= 0) id_nn = list[k - 128];
        // the staging cull tests the rectangle of both halves' pixels whose
        // last contributor lies past top - 64 (one of the two sets is not empty)
        const int thr = max(top - 64, 0);
        const uint64_t ma = gs::ballot(lasta > thr), mb = gs::ballot(lastb > thr);
        float cx0 = 3.0e38f, cy0 = 3.0e38f, cx1 = -3.0e38f, cy1 = -3.0e38f;
        if (ma != 0) active_rect(ma, qx0, qy0, cx0, cy0, cx1, cy1);
        if (mb != 0) {
            float x0, y0, x1, y1;
            active_rect(mb, qx0 + 8.f, qy0, x0, y0, x1, y1);
            cx0 = __builtin_fminf(cx0, x0);
            cy0 = __builtin_fminf(cy0, y0);
            cx1 = __builtin_fmaxf(cx1, x1);
            cy1 = __builtin_fmaxf(cy1, y1);
        }
        const bool keep = k >= 0 && rec_may_touch(r_cur, cx0, cy0, cx1, cy1);
        const uint64_t km = gs::ballot(keep);
        if (keep) stage_put(st, gs::rank_below(km), r_cur, id_cur, k);
        __syncthreads();
        const int cnt = (int)__builtin_popcountll(km);
        for (int j = 0; j < cnt; j++) {
            const float4 A = st.a[j];
            const float4 B = st.b[j];
            const float4 Cc = st.c[j];
            const BwdEval ea = bwd_eval(ka, A, B, Cc);
            const BwdEval eb = bwd_eval(kb, A, B, Cc);
            if (gs::ballot(ea.valid || eb.valid) == 0) continue;
            float va[12], vb[12], v[12];
            bwd_apply<false>(pa, ka, A, B, Cc, ea, va);
            bwd_apply<false>(pb, kb, A, B, Cc, eb, vb);
#pragma unroll
            for (int q = 0; q < 11; q++) v[q] = va[q] + vb[q];
            v[2] = __builtin_fabsf(va[2]) + __builtin_fabsf(vb[2]);
            v[3] = __builtin_fabsf(va[3]) + __builtin_fabsf(vb[3]);
            v[11] = va[11];   // never read back
            const uint32_t cx = __builtin_amdgcn_readfirstlane(__float_as_uint(Cc.y));
            const float tot = gs::wave_sum12<true>(v);
            if (my_k >= 0 && my_k < 11) unsafeAtomicAdd(gacc + (size_t)cx * 16 + my_k, tot);
        }
        __syncthreads();
        r_cur = r_nxt;
        id_cur = id_nxt;
        id_nxt = id_nn;
    }
}

// FULL: the full-image path's rule (reference _f backward.cu:560-566): no
// conic or opacity gradient from a pixel where opacity * G > 0.99 (the alpha
// clamp is active); |dL/dmean2D| is accumulated but not written out.
// GEO: render_geo (reference _r backward.cu:393-405,427-432,476-490): the five
// maps enter dL/dalpha beside the colour, and their gradients
// alpha T dL/dmap go to accumulator slots 11..15.
// The split path without render_geo (!FULL && !GEO) walks 16x8 half tiles
// instead of quadrants when the scene's Gaussians are wide (two_px_lanes,
// from the forward's counts in meta; block-uniform).  Occupancy: six waves
// per SIMD (80 VGPRs) except with render_geo's map terms.
template <bool FULL, bool GEO>
__device__ __forceinline__ void render_bwd_body(
    int W, int H, unsigned gx, unsigned gy, unsigned sgx, unsigned NS, const uint2* __restrict__ ranges,
    const uint32_t* __restrict__ clist, const float4* __restrict__ rec, const uint8_t* __restrict__ cl,
    const float* __restrict__ bg, const float* __restrict__ final_T, const uint32_t* __restrict__ n_contrib_px,
    const float* __restrict__ dL_dpixels, float* __restrict__ gacc, const GeoBwd& G,
    const uint32_t* __restrict__ sched, const uint32_t* __restrict__ scnt, const uint32_t* __restrict__ meta,
    Stage& st)
{
    unsigned tile, quad, tx, ty;
    if (sched != nullptr) {
        // bwd_schedule_kernel's order: XCD b % 8 takes its tiles heaviest first,
        // four quadrant waves per tile (or two half-tile waves: the grid's
        // other half of the blocks then has nothing to do)
        const unsigned xcd = blockIdx.x & 7u, slot = blockIdx.x >> 3;
        if constexpr (!FULL && !GEO) {
            if (two_px_lanes(meta)) {
                const unsigned i = slot >> 1;
                if (i >= scnt[xcd]) return;
                const unsigned t = sched[(size_t)xcd * sched_cap(NS) + i];
                if (cl != nullptr && !cl[t]) return;
                bwd_half_tile(W, H, gx, t, slot & 1u, ranges, clist, rec, bg, final_T, n_contrib_px, dL_dpixels,
                              gacc, st);
                return;
            }
        }
        const unsigned i = slot >> 2;
        if (i >= scnt[xcd]) return;
        quad = slot & 3u;
        tile = sched[(size_t)xcd * sched_cap(NS) + i];
        tx = tile % gx;
        ty = tile / gx;
    } else if (!block_to_tile(blockIdx.x, gx, gy, sgx, NS, tile, quad, tx, ty)) {
        return;
    }
    if (cl != nullptr && !cl[tile]) return;
    const int lane = threadIdx.x;
    const int qx = (int)tx * 16 + (int)(quad & 1u) * 8, qy = (int)ty * 16 + (int)(quad >> 1) * 8;
    const int px = qx + (lane & 7), py = qy + (lane >> 3);
    const bool inside = px < W && py < H;
    const size_t pid = (size_t)py * W + px;
    const size_t HW = (size_t)H * W;

    const float T_final = inside ? final_T[pid] : 0.f;
    const int last = inside ? (int)n_contrib_px[pid] : 0;
    float dp0 = 0.f, dp1 = 0.f, dp2 = 0.f;
    if (inside) { dp0 = dL_dpixels[pid]; dp1 = dL_dpixels[HW + pid]; dp2 = dL_dpixels[2 * HW + pid]; }
    const int maxlast = gs::wave_max_i(last);
    if (maxlast == 0) return;

    // render_geo: the pixel's map gradients, plus the plane depth's
    // D = M4 / -(n . ray + 1e-8) through n = M0..2 and M4 (the ray as the
    // reference's backward takes it: (x - W / 2) / fx in double)
    [[maybe_unused]] float dm[NUM_MAPS] = {0.f, 0.f, 0.f, 0.f, 0.f};
    if constexpr (GEO) {
        if (inside) {
            for (int c = 0; c < NUM_MAPS; c++) dm[c] = G.dL_dmaps[c * HW + pid];
            const float rx = (float)(((double)px - (double)W * 0.5) / (double)G.fx);
            const float ry = (float)(((double)py - (double)H * 0.5) / (double)G.fy);
            const float n0 = G.map_px[pid], n1 = G.map_px[HW + pid], n2 = G.map_px[2 * HW + pid];
            const float distance = G.map_px[4 * HW + pid];
            const float tmp = (float)((double)(n0 * rx + n1 * ry + n2) + 1.0e-8);
            const float g = G.dL_dplane[pid];
            const float q = distance / (tmp * tmp);
            dm[4] += -g / tmp;
            dm[0] += g * (q * rx);
            dm[1] += g * (q * ry);
            dm[2] += g * q;
        }
    }

    __shared__ float st_map[GEO ? NUM_MAPS * 64 : 1];

    const uint32_t* list = clist + ranges[tile].x;
    const float qx0 = (float)qx, qy0 = (float)qy;
    const float bg_dot = bg[0] * dp0 + bg[1] * dp1 + bg[2] * dp2;
    // nT_bg: the background term of dL/dalpha, before 1/(1-alpha)
    const BwdConst kc{(float)px, (float)py, dp0, dp1, dp2, -T_final * bg_dot, last};
    // after the wave reduction this lane holds the total of gradient term
    // my_k (accumulator slot), or nothing (my_k < 0)
    const int my_k = gs::wave_sum12_index(lane);
    BwdPixel px_st{T_final, 0.f, 0.f, 0.f};

    // walk positions maxlast-1 .. 0 of the tile's list, back to front, with
    // the same software pipeline as the forward
    uint32_t id_cur = maxlast - 1 - lane >= 0 ? list[maxlast - 1 - lane] : 0u;
    uint32_t id_nxt = maxlast - 65 - lane >= 0 ? list[maxlast - 65 - lane] : 0u;
    Rec r_cur{};
    if (maxlast - 1 - lane >= 0) r_cur = load_rec<GEO>(rec, id_cur);

    for (int top = maxlast; top > 0; top -= 64) {
        const int k = top - 1 - lane;
        Rec r_nxt{};
        uint32_t id_nn = 0;
        if (k - 64 >= 0) r_nxt = load_rec<GEO>(rec, id_nxt);
        if (k - 128 >= 0) id_nn = list[k - 128];
        // stage positions top-1, top-2, ..., top-64, keeping only Gaussians
        // that can reach a pixel whose last contributor lies past top-64
        // (the other pixels blend no entry of this batch); that pixel set is
        // never empty: it holds the pixels of the largest last contributor
        float cx0, cy0, cx1, cy1;
        active_rect(gs::ballot(last > max(top - 64, 0)), qx0, qy0, cx0, cy0, cx1, cy1);
        const bool keep = k >= 0 && rec_may_touch(r_cur, cx0, cy0, cx1, cy1);
        const uint64_t km = gs::ballot(keep);
        if (keep) stage_put(st, gs::rank_below(km), r_cur, id_cur, k);
        if constexpr (GEO) {
            if (keep) {
                const int slot = gs::rank_below(km);
                const float* m = G.all_map + (size_t)NUM_MAPS * r_cur.gid;
                for (int c = 0; c < NUM_MAPS; c++) st_map[c * 64 + slot] = m[c];
            }
        }
        __syncthreads();
        const int cnt = (int)__builtin_popcountll(km);
        for (int j = 0; j < cnt; j++) {
            const float4 A = st.a[j];
            const float4 B = st.b[j];
            const float4 Cc = st.c[j];
            const BwdEval e = bwd_eval(kc, A, B, Cc);
            if (gs::ballot(e.valid) == 0) continue;   // no lane blends the entry: nothing changes
            float vals[12];
            if constexpr (GEO) {
                float mv[NUM_MAPS];
                for (int c = 0; c < NUM_MAPS; c++) mv[c] = st_map[c * 64 + j];
                float m_dp = mv[0] * dm[0];
                for (int c = 1; c < NUM_MAPS; c++) m_dp = __builtin_fmaf(mv[c], dm[c], m_dp);
                const float dcc = bwd_apply<FULL, true>(px_st, kc, A, B, Cc, e, vals, m_dp);
                const uint32_t cx = __builtin_amdgcn_readfirstlane(__float_as_uint(Cc.y));
                // slot 11: the first map's gradient; the other four in a
                // second reduction, into slots 12..15
                vals[11] = dcc * dm[0];
                float v2[12] = {dcc * dm[1], dcc * dm[2], dcc * dm[3], dcc * dm[4], 0.f, 0.f,
                                0.f,         0.f,         0.f,         0.f,         0.f, 0.f};
                const float tot = gs::wave_sum12<true>(vals);
                const float tot2 = gs::wave_sum12<false>(v2);
                if (my_k >= 0) unsafeAtomicAdd(gacc + (size_t)cx * 16 + my_k, tot);
                if (my_k >= 0 && my_k < 4) unsafeAtomicAdd(gacc + (size_t)cx * 16 + 12 + my_k, tot2);
            } else {
                bwd_apply<FULL>(px_st, kc, A, B, Cc, e, vals);
                const uint32_t cx = __builtin_amdgcn_readfirstlane(__float_as_uint(Cc.y));   // one Gaussian per entry
                const float tot = gs::wave_sum12<true>(vals);
                // the eleven totals of one Gaussian land in one 64-byte accumulator
                if (my_k >= 0 && my_k < 11) unsafeAtomicAdd(gacc + (size_t)cx * 16 + my_k, tot);
            }
        }
        __syncthreads();
        r_cur = r_nxt;
        id_cur = id_nxt;
        id_nxt = id_nn;
    }
}

template <bool FULL, bool GEO = false>
__global__ __launch_bounds__(64, GEO ? 5 : 6) void render_bwd_kernel(
    int W, int H, unsigned gx, unsigned gy, unsigned sgx, unsigned NS, const uint2* __restrict__ ranges,
    const uint32_t* __restrict__ clist, const float4* __restrict__ rec, const uint8_t* __restrict__ cl,
    const float* __restrict__ bg, const float* __restrict__ final_T, const uint32_t* __restrict__ n_contrib_px,
    const float* __restrict__ dL_dpixels, float* __restrict__ gacc, GeoBwd G,
    const uint32_t* __restrict__ sched, const uint32_t* __restrict__ scnt, const uint32_t* __restrict__ meta,
    ClearBuf clr)
{
    __shared__ Stage st;
    render_bwd_body<FULL, GEO>(W, H, gx, gy, sgx, NS, ranges, clist, rec, cl, bg, final_T, n_contrib_px, dL_dpixels,
                               gacc, G, sched, scnt, meta, st);
    clear_share(clr);
}

// the clearing when no blend kernel runs
__global__ __launch_bounds__(256) void clear_kernel(ClearBuf clr)
{
    clear_share(clr);
}

// ---- VALU probes: the blend kernels' per-entry arithmetic (fwd_blend_step;
// bwd_eval + bwd_apply + wave_sum12), on 64 entries staged in LDS once, with no
// global memory traffic, in the blend kernels' 64-thread blocks.  Their VALU
// instruction rate is the ceiling the blend kernels' rate is compared with.
constexpr int VALU_PROBE_BLOCKS = 16384;

__device__ __forceinline__ void probe_stage(Stage& st, int lane)
{
    // entries centred on the quadrant's pixels, wide and faint enough that
    // every pixel blends every entry
    const float mx = (float)(lane & 7) + 0.25f, my = (float)(lane >> 3) + 0.5f;
    const float a = 0.02f + 0.0005f * (float)lane, b = 0.002f, c = 0.03f - 0.0003f * (float)lane;
    const float op = 0.02f + 0.0004f * (float)lane;
    st.a[lane] = make_float4(mx, my, -0.5f * a, -b);
    st.b[lane] = make_float4(-0.5f * c, op, 0.3f, 0.6f);
    st.c[lane] = make_float4(0.9f, __uint_as_float((uint32_t)lane), __int_as_float(lane + 1), gs::alpha_cut_power(op));
}

template <int WHICH>
__global__ __launch_bounds__(64) void valu_probe_kernel(int iters, float* __restrict__ y)
{
    __shared__ Stage st;
    const int lane = threadIdx.x;
    probe_stage(st, lane);
    __syncthreads();
    const float pxf = (float)(lane & 7), pyf = (float)(lane >> 3);
    float out = 0.f;
    if (WHICH == 0) {
        // the forward: the two-register-set loop of render_fwd_kernel, with
        // the observe ballot of its split mode (counted, not stored)
        int observed = 0;
        for (int it = 0; it < iters; it++) {
            FwdPixel p{1.0f, 0.f, 0.f, 0.f, 0u, 0u};
            auto blend = [&](const float4& A, const float4& B, const float4& Cc) {
                const FwdStep f = fwd_blend_step(p, A, B, Cc, pxf, pyf);
                const uint64_t m = f.observe;
                if (m != 0) observed += (int)__builtin_popcountll(m);
            };
            float4 A0 = st.a[0], B0 = st.b[0], D0 = st.c[0];
            float4 A1, B1, D1;
            for (int j = 0; j < 64; j += 2) {
                if (gs::ballot(p.T > 0.0f) == 0) break;
                A1 = st.a[(j + 1) & 63]; B1 = st.b[(j + 1) & 63]; D1 = st.c[(j + 1) & 63];
                blend(A0, B0, D0);
                if (j + 1 >= 64 || gs::ballot(p.T > 0.0f) == 0) break;
                A0 = st.a[(j + 2) & 63]; B0 = st.b[(j + 2) & 63]; D0 = st.c[(j + 2) & 63];
                blend(A1, B1, D1);
            }
            out += p.C0 + p.C1 + p.C2 + p.T + (float)(p.last + p.n2l);
        }
        out += (float)observed;
    } else if (WHICH == 2) {
        // the backward's half-tile walk (bwd_half_tile): two pixels per lane
        // (here at one position, so that both blend every entry), one
        // reduction per entry, the atomics replaced by a sum
        const int my_k = gs::wave_sum12_index(lane);
        const BwdConst ka{pxf, pyf, 0.3f, -0.2f, 0.1f, -0.05f, 64};
        const BwdConst kb{pxf, pyf, -0.1f, 0.25f, 0.2f, -0.04f, 64};
        for (int it = 0; it < iters; it++) {
            BwdPixel pa{0.2f, 0.f, 0.f, 0.f}, pb{0.25f, 0.f, 0.f, 0.f};
            for (int j = 0; j < 64; j++) {
                const float4 A = st.a[j], B = st.b[j], Cc = st.c[j];
                const BwdEval ea = bwd_eval(ka, A, B, Cc);
                const BwdEval eb = bwd_eval(kb, A, B, Cc);
                if (gs::ballot(ea.valid || eb.valid) == 0) continue;
                float va[12], vb[12], v[12];
                bwd_apply<false>(pa, ka, A, B, Cc, ea, va);
                bwd_apply<false>(pb, kb, A, B, Cc, eb, vb);
#pragma unroll
                for (int q = 0; q < 11; q++) v[q] = va[q] + vb[q];
                v[2] = __builtin_fabsf(va[2]) + __builtin_fabsf(vb[2]);
                v[3] = __builtin_fabsf(va[3]) + __builtin_fabsf(vb[3]);
                v[11] = va[11];
                const float tot = gs::wave_sum12<true>(v);
                if (my_k >= 0 && my_k < 11 && tot != 0.f) out += tot;
            }
            out += pa.T + pb.T;
        }
    } else {
        // the backward: render_bwd_kernel's entry loop, the accumulator
        // atomics replaced by a sum
        const int my_k = gs::wave_sum12_index(lane);
        const BwdConst kc{pxf, pyf, 0.3f, -0.2f, 0.1f, -0.05f, 64};
        for (int it = 0; it < iters; it++) {
            BwdPixel p{0.2f, 0.f, 0.f, 0.f};
            for (int j = 0; j < 64; j++) {
                const float4 A = st.a[j], B = st.b[j], Cc = st.c[j];
                const BwdEval e = bwd_eval(kc, A, B, Cc);
                if (gs::ballot(e.valid) == 0) continue;
                float vals[12];
                bwd_apply<false>(p, kc, A, B, Cc, e, vals);
                const float tot = gs::wave_sum12<true>(vals);
                if (my_k >= 0 && my_k < 11 && tot != 0.f) out += tot;
            }
            out += p.T;
        }
    }
    if (out == 12345.0f) y[0] = out;   // keeps the work; never true for these inputs in practice
}

}  // namespace

// ====================================================================== C ABI

namespace {
size_t count_lds_bytes(int T) { return sizeof(uint32_t) * (size_t)(T < LDS_TILES ? T : LDS_TILES); }
size_t count_regions_lds_bytes(const GeomLayout& g, unsigned gx, unsigned gy, unsigned lrs)
{
    return sizeof(uint32_t) * ((size_t)WAVES_PER_BIN * EXPAND_WORDS + (size_t)count_region_words(gx, gy, lrs) +
                               (size_t)(g.G < LDS_GRID ? g.G : LDS_GRID));
}
size_t scatter_regions_lds_bytes(const GeomLayout& g)
{
    return sizeof(float4) * 256 * WAVES_PER_BIN +
           sizeof(uint32_t) * ((size_t)WAVES_PER_BIN * EXPAND_WORDS + (size_t)(g.NR < LDS_REGIONS ? g.NR : LDS_REGIONS));
}
// log2 of the region side: the caller's side (0: the smallest the grid
// allows, g.RS), never below g.RS -- the layout's region arrays are sized for
// g.RS, so any larger side fits them.  The results do not depend on it; the
// cost does: larger regions give fewer, longer lists to sort, which pays when
// each Gaussian covers many tiles.
unsigned region_lrs(const GeomLayout& g, int side)
{
    const int rs = std::max(g.RS, side);
    return rs >= 8 ? 3u : rs == 4 ? 2u : 1u;
}

size_t scatter_lds_bytes(int T) { return sizeof(float4) * 256 * WAVES_PER_BIN + count_lds_bytes(T); }

// grid of the blend kernels: whole supertiles per XCD
unsigned blend_grid(unsigned gx, unsigned gy, unsigned& sgx, unsigned& NS)
{
    sgx = (gx + SUPER - 1) / SUPER;
    NS = sgx * ((gy + SUPER - 1) / SUPER);
    return ((NS + 7u) / 8u) * 8u * BLOCKS_PER_SUPER;
}
}  // namespace

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

extern "C" int gs_render_point_list(int P, int64_t R, int W, int H, const float* depths, const void* geom,
                                    void* binning, const void* img, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0 && W > 0 && H > 0 && R >= 0, "invalid sizes P=%d W=%d H=%d R=%lld", P, W, H, (long long)R);
    if (R == 0) return GS_OK;
    GS_REQUIRE(depths != nullptr && geom != nullptr && binning != nullptr && img != nullptr,
               "depths and the forward's workspaces must be non-null");
    const GeomLayout g = geom_layout(P, W, H);
    const ImgLayout il = img_layout(W, H);
    const BinLayout b = bin_layout(R);
    GS_TIMED("pointlist_kernel", stream,
             hipLaunchKernelGGL(pointlist_kernel, dim3((unsigned)g.T), dim3(256), 0, stream,
                                at<const uint2>(img, il.ranges), at<const uint32_t>(binning, b.clist),
                                at<const uint32_t>(geom, g.cid2id), depths, at<uint32_t>(binning, b.point_list),
                                at<uint64_t>(binning, b.keys)));
    GS_LAUNCH_CHECK("pointlist_kernel");
    return GS_OK;
}

namespace {

// Side streams for the bucket sort: the size classes sort disjoint buckets,
// and the largest classes are a few single blocks whose bitonic networks are
// latency-bound, so the classes run side by side (forked from and joined back
// to the caller's stream with events).  Created once per device, at the
// default priority, never destroyed.
// Pinned host words for R, one slot per forward in flight: a reserved
// forward copies R there and records the slot's event, and waits for that
// event only after the rest of the forward is queued.
// A reserved forward's slot for R: one word of mapped, coherent pinned host
// memory that the scan kernel stores readback_word(R, seq) into and the host
// polls, so that nothing is queued on the stream between the scan and the
// scatter (an event there costs the stream a gap of several microseconds).
struct Readback {
    uint64_t* host = nullptr;   // the word, host side
    uint64_t* dev = nullptr;    // its device address
    uint32_t seq = 0;           // this use's sequence number (31 bits, never 0)
    int device = -1;
    bool busy = false;
};
constexpr int READBACK_SLOTS = 64;
std::mutex g_rb_mu;

// Two more streams per device for the region sorts of the largest lists
// (one per size class), which run beside those of the smaller ones (forked
// from and joined back to the caller's stream with events): created once, at
// the default priority, never destroyed.  g_side_mu is held from the fork to
// the join, so that forwards queued from several host threads use the events
// one after another.
struct SideStream {
    hipStream_t s[2] = {nullptr, nullptr};
    hipEvent_t fork = nullptr, join[2] = {nullptr, nullptr};
};
constexpr int MAX_DEVICES = 64;
std::mutex g_side_mu;
SideStream g_side[MAX_DEVICES];

int side_stream(SideStream*& out)
{
    int dev = 0;
    GS_HIP(hipGetDevice(&dev));
    GS_REQUIRE(dev >= 0 && dev < MAX_DEVICES, "device %d out of range", dev);
    SideStream& ss = g_side[dev];
    if (ss.fork == nullptr) {
        // the events order work of one device: a device-scope release is
        // enough (a system-scope one writes the L2s back to memory at every
        // record)
        constexpr unsigned ev_flags = hipEventDisableTiming | hipEventDisableSystemFence;
        for (int k = 0; k < 2; k++) {
            GS_HIP(hipStreamCreateWithFlags(&ss.s[k], hipStreamNonBlocking));
            GS_HIP(hipEventCreateWithFlags(&ss.join[k], ev_flags));
        }
        GS_HIP(hipEventCreateWithFlags(&ss.fork, ev_flags));
    }
    out = &ss;
    return GS_OK;
}
Readback g_rb[READBACK_SLOTS];

int readback_acquire(Readback*& out)
{
    out = nullptr;
    int dev = 0;
    GS_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_rb_mu);
    for (Readback& r : g_rb) {
        if (r.busy || (r.device >= 0 && r.device != dev)) continue;
        if (r.device < 0) {
            GS_HIP(hipHostMalloc(reinterpret_cast<void**>(&r.host), sizeof(uint64_t),
                                 hipHostMallocMapped | hipHostMallocCoherent));
            GS_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&r.dev), r.host, 0));
            __atomic_store_n(r.host, 0ull, __ATOMIC_RELEASE);   // sequence 0: never a use's
            r.device = dev;
        }
        r.seq = (r.seq + 1u) & 0x7fffffffu;
        if (r.seq == 0u) r.seq = 1u;
        r.busy = true;
        out = &r;
        return GS_OK;
    }
    gs::set_error("more than %d reserved forwards in flight", READBACK_SLOTS);
    return GS_ERR_SIZE;
}

void readback_release(Readback* r)
{
    std::lock_guard<std::mutex> lk(g_rb_mu);
    r->busy = false;
}

// count + scan + R readback, shared by the split and the full-image path.
// Without a readback slot (rb null) R is copied back synchronously into
// *num_rendered; with one, the copy into the slot and its event are only
// queued, and cap is the caller's instance capacity (see tilescan_kernel).
int render_count_impl(bool full, int P, int W, int H, const float* means2D, const int* radii,
                      const uint8_t* compute_locally, const float* rects, const float* conic_opacity, void* geom,
                      int64_t* num_rendered, hipStream_t stream, uint64_t cap = ~0ull, Readback* rb = nullptr,
                      int region_side = 0)
{
    GS_REQUIRE(P >= 0 && W > 0 && H > 0, "invalid sizes P=%d W=%d H=%d", P, W, H);
    GS_REQUIRE(geom != nullptr && (num_rendered != nullptr || rb != nullptr), "geom and num_rendered must be non-null");
    GS_REQUIRE(!full || P == 0 || (rects != nullptr && conic_opacity != nullptr),
               "the full path needs rects and conic_opacity");
    GS_REQUIRE(((uintptr_t)means2D & 7) == 0 && ((uintptr_t)rects & 7) == 0 && ((uintptr_t)conic_opacity & 15) == 0,
               "means2D / rects must be 8-byte and conic_opacity 16-byte aligned");
    const GeomLayout g = geom_layout(P, W, H);
    const unsigned gx = (unsigned)((W + 15) / 16), gy = (unsigned)((H + 15) / 16);
    int* loc_map = at<int>(geom, g.loc_map);
    int* tile_of_local = at<int>(geom, g.tile_of_local);
    uint32_t* meta = at<uint32_t>(geom, g.meta);
    uint32_t* hist = at<uint32_t>(geom, g.hist);
    uint32_t* tile_count = at<uint32_t>(geom, g.tile_count);
    uint32_t* tile_start = at<uint32_t>(geom, g.tile_start);
    uint32_t* cursor = at<uint32_t>(geom, g.cursor);

    // the binning's wall time on the caller's stream: from here to the end of
    // the sorts in the forward call (the R readback and the caller's
    // allocation between the two calls included)
    // the split path bins through regions (count_regions / scan_regions /
    // scatter_regions / regionsort); the full-image path through per-tile
    // buckets (count / tilescan / scatter / tilesort)
    const bool split = !full;
    GS_REQUIRE(!split || g.RS > 0, "a %ux%u tile grid has more than %d regions of 8x8 tiles", gx, gy, MAX_REGIONS);
    GS_REQUIRE(region_side == 0 || region_side == 2 || region_side == 4 || region_side == 8,
               "region_side must be 0, 2, 4 or 8 (got %d)", region_side);
    const unsigned lrs = region_lrs(g, region_side);
    ClearRegions CR{nullptr, nullptr, nullptr, 0, 0, lrs};
    if (split)
        CR = ClearRegions{compute_locally != nullptr ? at<uint64_t>(geom, g.regmask) : nullptr,
                          at<uint32_t>(geom, g.rcount), at<uint32_t>(geom, g.grid), g.NR, GRID_PARTS * g.G, lrs};
    if (gs::timing_on()) gs::timing_stage_begin(stream, BINNING_STAGE);
    if (compute_locally == nullptr) {
        const size_t nclear = std::max<size_t>((size_t)g.T, split ? (size_t)std::max(GRID_PARTS * g.G, g.NR) : 0);
        GS_TIMED("localmap_kernel", stream,
                 hipLaunchKernelGGL(localmap_all_kernel, dim3(gs_div_up(nclear, 256)), dim3(256), 0, stream, g.T,
                                    gx, gy, loc_map, tile_of_local, tile_count, meta, CR));
    } else {
        // block 0 numbers the tiles, the others clear the region state (about
        // 4 words per thread)
        const size_t nbulk = split ? (size_t)std::max(GRID_PARTS * g.G, g.NR) : 0;
        const unsigned nb = 1u + (unsigned)std::min<size_t>(gs_div_up(nbulk, 4096), 1024);
        // the tile mask held in LDS as bits: one 64-bit word per 64-tile round, up to 64 KB
        const int rounds = (g.T + 63) / 64, lds_rounds = 8192;
        const size_t lds = rounds <= lds_rounds ? sizeof(uint64_t) * (size_t)rounds : 0;
        GS_TIMED("localmap_kernel", stream,
                 hipLaunchKernelGGL(localmap_kernel, dim3(nb), dim3(1024), lds, stream, g.T, gx, compute_locally,
                                    loc_map, tile_of_local, tile_count, meta, CR, lds_rounds));
    }
    GS_LAUNCH_CHECK("localmap_kernel");
    if (split) {
        if (P > 0) {
            GS_TIMED("count_regions_kernel", stream,
                     hipLaunchKernelGGL(count_regions_kernel, dim3(g.NC), dim3(BIN_THREADS), count_regions_lds_bytes(g, gx, gy, lrs),
                                        stream, P, g.CH, g.WS, gx, gy, lrs, reinterpret_cast<const float2*>(means2D),
                                        radii, meta, at<const uint64_t>(geom, g.regmask), at<uint32_t>(geom, g.rhist),
                                        at<uint32_t>(geom, g.rcount), at<uint32_t>(geom, g.grid), g.G,
                                        at<uint32_t>(geom, g.wcount)));
            GS_LAUNCH_CHECK("count_regions_kernel");
        }
        GS_TIMED("scan_regions_kernel", stream,
                 hipLaunchKernelGGL(scan_regions_kernel, dim3(3), dim3(1024), 0, stream, meta, gx, lrs, tile_of_local,
                                    at<uint32_t>(geom, g.grid), g.G, tile_count, tile_start,
                                    at<uint32_t>(geom, g.wcount), P > 0 ? g.NC * WAVES_PER_BIN : 0,
                                    at<const uint32_t>(geom, g.rcount),
                                    at<uint32_t>(geom, g.rstart), at<uint32_t>(geom, g.rcursor),
                                    at<uint32_t>(geom, g.rcls_count), at<int>(geom, g.rcls_list), g.NR, cap,
                                    rb != nullptr ? rb->dev : nullptr, rb != nullptr ? rb->seq : 0u));
        GS_LAUNCH_CHECK("scan_regions_kernel");
    }
    if (!split && P > 0) {
        GS_TIMED("count_kernel", stream,
                 hipLaunchKernelGGL(count_kernel<true>, dim3(g.NC), dim3(BIN_THREADS), count_lds_bytes(g.T), stream, P,
                                    g.CH, g.WS, gx, gy, reinterpret_cast<const float2*>(means2D), radii, loc_map,
                                    meta, hist, tile_count, at<uint32_t>(geom, g.wcount),
                                    reinterpret_cast<const float2*>(rects),
                                    reinterpret_cast<const float4*>(conic_opacity)));
        GS_LAUNCH_CHECK("count_kernel");
    }
    if (!split) {
        GS_TIMED("tilescan_kernel", stream,
                 hipLaunchKernelGGL(tilescan_kernel, dim3(1), dim3(1024), 0, stream, meta, tile_count, tile_start, cursor,
                                    at<uint32_t>(geom, g.wcount), P > 0 ? g.NC * WAVES_PER_BIN : 0, g.T,
                                    at<uint32_t>(geom, g.cls_count), at<int>(geom, g.cls_list), cap,
                                    rb != nullptr ? rb->dev : nullptr, rb != nullptr ? rb->seq : 0u));
        GS_LAUNCH_CHECK("tilescan_kernel");
    }
    if (rb != nullptr) return GS_OK;   // the scan stores R into rb's word (reserved_forward polls it)
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

// a caller's buffer for a blend kernel to clear: 16-byte aligned, a
// multiple of 16 bytes (none: 0 bytes)
int clear_buf(void* dst, int64_t bytes, ClearBuf& out)
{
    GS_REQUIRE(bytes >= 0 && (bytes & 15) == 0 && ((uintptr_t)dst & 15) == 0 && (bytes == 0 || dst != nullptr),
               "clear_dst and clear_bytes must be 16-byte aligned (clear_bytes=%lld)", (long long)bytes);
    out = ClearBuf{static_cast<float4*>(dst), (size_t)bytes / 16};
    return GS_OK;
}

// duplicate + sort + ranges + blend, shared by the split and the full-image path
int render_forward_impl(int mode, int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                        const float* depths, const int* radii, const float* conic_opacity, const float* rgb,
                        const uint8_t* compute_locally, const float* rects, void* geom, void* binning, void* img,
                        FwdOut O, int32_t* n_render, hipStream_t stream, const DepthIO* depth_io = nullptr, int region_side = 0)
{
    GS_REQUIRE(P >= 0 && W > 0 && H > 0 && R >= 0, "invalid sizes P=%d W=%d H=%d R=%lld", P, W, H, (long long)R);
    GS_REQUIRE(((uintptr_t)conic_opacity & 15) == 0 && ((uintptr_t)means2D & 7) == 0 && ((uintptr_t)rects & 7) == 0,
               "conic_opacity must be 16-byte and means2D / rects 8-byte aligned");
    const bool full = !is_split(mode);
    GS_REQUIRE(!full || P == 0 || rects != nullptr, "the full path needs rects");
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

    const unsigned T = (unsigned)g.T;
    const RangesOut ro{g.T, loc_map, tile_count, tile_start, ranges, n_render, O.n_consider, O.n_contrib_tile};
    if (R == 0 || full) {   // the split path's scatter writes the ranges itself
        GS_TIMED("ranges_kernel", stream,
                 hipLaunchKernelGGL(ranges_kernel, dim3(gs_div_up(T, 256)), dim3(256), 0, stream, meta, ro));
        GS_LAUNCH_CHECK("ranges_kernel");
    }
    // per-Gaussian accumulators start at zero: inside the scatter when there
    // are instances, else with a fill kernel each
    ZeroOut Z{{is_split(mode) ? O.out_observe : nullptr, reinterpret_cast<int32_t*>(O.accum_max_count),
                mode == BLEND_SIMP ? reinterpret_cast<int32_t*>(O.accum_weights) : nullptr,
                mode == BLEND_SIMP ? O.accum_weights_count : nullptr}};
    if (P > 0 && R == 0) {
        const dim3 zg(gs_div_up((size_t)P, 256));
        for (int32_t* z : Z.p) {
            if (z == nullptr) continue;
            GS_TIMED("zero_i32_kernel", stream, hipLaunchKernelGGL(zero_i32_kernel, zg, dim3(256), 0, stream, P, z));
            GS_LAUNCH_CHECK("zero_i32_kernel");
        }
    }
    if (R > 0 && !full) {
        // split path: region lists, then per region a sort and the filter
        // into its tiles.  One sort launch per region size class, largest
        // first, one after another on the caller's stream; the grids are
        // bounded by how many regions of the class the region entries (at
        // most R) can fill and by what fits on the chip at once.
        GS_REQUIRE(region_side == 0 || region_side == 2 || region_side == 4 || region_side == 8,
                   "region_side must be 0, 2, 4 or 8 (got %d)", region_side);
        const unsigned lrs = region_lrs(g, region_side);
        uint32_t* clist = at<uint32_t>(binning, bl.clist);
        // region lists (12 bytes per entry, at most R entries) in the point
        // list and key areas of the binning buffer (12 R bytes from point_list)
        uint3* rent = at<uint3>(binning, bl.point_list);
        const uint32_t* rcount = at<const uint32_t>(geom, g.rcount);
        const uint32_t* rstart = at<const uint32_t>(geom, g.rstart);
        GS_TIMED("scatter_regions_kernel", stream,
                 hipLaunchKernelGGL(scatter_regions_kernel, dim3(g.NC), dim3(BIN_THREADS), scatter_regions_lds_bytes(g),
                                    stream, P, g.CH, g.WS, gx, gy, lrs, reinterpret_cast<const float2*>(means2D),
                                    depths, radii, reinterpret_cast<const float4*>(conic_opacity), rgb, meta,
                                    at<const uint64_t>(geom, g.regmask), at<const uint32_t>(geom, g.rhist),
                                    at<const uint32_t>(geom, g.rstart), at<uint32_t>(geom, g.rcursor),
                                    at<const uint32_t>(geom, g.wcount), rent, at<int>(geom, g.cidx_of),
                                    at<uint32_t>(geom, g.cid2id), at<float4>(geom, g.rec), Z, ro));
        GS_LAUNCH_CHECK("scatter_regions_kernel");
        const uint32_t* cc = at<const uint32_t>(geom, g.rcls_count);
        const int* cls = at<const int>(geom, g.rcls_list);
        const TileOut to{loc_map, tile_start, tile_count, clist, gx, gy};
        auto grid_of = [&](int lo, int cap) {
            const int64_t fit = R / (int64_t)(lo + 1);
            return (unsigned)std::min<int64_t>(std::min<int64_t>((int64_t)g.NR, fit), (int64_t)cap);
        };
        auto list = [&](int c) { return cls + (size_t)c * g.NR; };
        const unsigned g4 = grid_of(REGION_CAP, 256), g3 = grid_of(4096, 256), g0 = grid_of(0, 2048);
        const unsigned gs = std::min<unsigned>(g0, 512u);
        // The lists of 4097..8192 entries (one 512-thread block per region,
        // one block per CU) sort on the caller's stream: they end last, so the
        // joins of the side streams -- the longer lists (sort_filter_big) on
        // the first, the lists of up to 4096 entries on the second -- are
        // already complete when the caller's stream reaches them.
        std::lock_guard<std::mutex> side_lock(g_side_mu);
        SideStream* ss = nullptr;
        if (int rc = side_stream(ss); rc != GS_OK) return rc;
        if (g4 > 0 || gs > 0) GS_HIP(hipEventRecord(ss->fork, stream));
        if (g3 > 0) {
            GS_TIMED("regionsort_kernel_8k", stream,
                     hipLaunchKernelGGL((regionsort_kernel<512, 16>), dim3(g3), dim3(512), 0, stream, cc + 3,
                                        list(3), rcount, rstart, rent, meta, lrs, to));
            GS_LAUNCH_CHECK("regionsort_kernel_8k");
        }
        if (g4 > 0) {
            GS_HIP(hipStreamWaitEvent(ss->s[0], ss->fork, 0));
            GS_TIMED("regionsort_big_kernel", ss->s[0],
                     hipLaunchKernelGGL((regionsort_big_kernel<512, 16>), dim3(g4), dim3(512), 0, ss->s[0], cc + 4,
                                        list(4), rcount, rstart, rent, meta, lrs, to));
            GS_LAUNCH_CHECK("regionsort_big_kernel");
            GS_HIP(hipEventRecord(ss->join[0], ss->s[0]));
        }
        if (gs > 0) {
            GS_HIP(hipStreamWaitEvent(ss->s[1], ss->fork, 0));
            GS_TIMED("regionsort_small_kernel", ss->s[1],
                     hipLaunchKernelGGL(regionsort_small_kernel, dim3(gs), dim3(256), 0, ss->s[1], cc, cls, g.NR,
                                        rcount, rstart, rent, meta, lrs, to));
            GS_LAUNCH_CHECK("regionsort_small_kernel");
            GS_HIP(hipEventRecord(ss->join[1], ss->s[1]));
        }
        if (g4 > 0) GS_HIP(hipStreamWaitEvent(stream, ss->join[0], 0));
        if (gs > 0) GS_HIP(hipStreamWaitEvent(stream, ss->join[1], 0));
    }
    if (R > 0 && full) {
        const float2* m2 = reinterpret_cast<const float2*>(means2D);
        const float4* co = reinterpret_cast<const float4*>(conic_opacity);
        GS_TIMED("scatter_kernel", stream,
                 hipLaunchKernelGGL(scatter_kernel<true>, dim3(g.NC), dim3(BIN_THREADS), scatter_lds_bytes(g.T), stream,
                                    P, g.CH, g.WS, gx, gy, m2, depths, radii, co, rgb, loc_map, meta, hist, tile_start,
                                    cursor, at<const uint32_t>(geom, g.wcount), sortkey, at<int>(geom, g.cidx_of),
                                    at<uint32_t>(geom, g.cid2id), at<float4>(geom, g.rec),
                                    reinterpret_cast<const float2*>(rects), Z));
        GS_LAUNCH_CHECK("scatter_kernel");
        uint32_t* clist = at<uint32_t>(binning, bl.clist);
        // one launch per LDS size class over that class's bucket list, one
        // after another on the caller's stream (run side by side on streams
        // of their own they contend for the same CUs and add a fork and a
        // join, which measured slower); the buckets of up to 512 keys ride
        // with the 1024-key class, those above SORT_CAP_MAX with the 8192-key
        // class.  The grid is bounded by how many buckets of the class R
        // instances can fill and by what fits on the chip at once.
        const uint32_t* cc = at<const uint32_t>(geom, g.cls_count);
        const int* cls = at<const int>(geom, g.cls_list);
        auto grid_of = [&](int lo, int cap) {
            const int64_t fit = R / (int64_t)(lo + 1);
            return (unsigned)std::min<int64_t>(std::min<int64_t>((int64_t)T, fit), (int64_t)cap);
        };
        auto list = [&](int c) { return cls + (size_t)c * T; };
        const unsigned g_wave = (grid_of(0, 8192) + 1) / 2;   // two waves per 128-thread block
        const unsigned g1 = std::max(grid_of(512, 4096), g_wave);
        const unsigned g2 = grid_of(1024, 2048), g3 = grid_of(2048, 2048);
        const unsigned g4 = std::max(grid_of(4096, 1024), grid_of(SORT_CAP_MAX, 256));
        if (g4 > 0) {
            GS_TIMED("tilesort_kernel_8k", stream,
                     hipLaunchKernelGGL((tilesort_radix_kernel<512, 16, EXTRA_BIG>), dim3(g4), dim3(512), 0, stream,
                                        cc + 4, list(4), tile_count, tile_start, sortkey, clist, cc + 5, list(5)));
            GS_LAUNCH_CHECK("tilesort_kernel_8k");
        }
        if (g3 > 0) {
            GS_TIMED("tilesort_kernel_4k", stream,
                     hipLaunchKernelGGL((tilesort_radix_kernel<256, 16>), dim3(g3), dim3(256), 0, stream, cc + 3,
                                        list(3), tile_count, tile_start, sortkey, clist, nullptr, nullptr));
            GS_LAUNCH_CHECK("tilesort_kernel_4k");
        }
        if (g2 > 0) {
            GS_TIMED("tilesort_kernel_2k", stream,
                     hipLaunchKernelGGL((tilesort_radix_kernel<256, 8>), dim3(g2), dim3(256), 0, stream, cc + 2,
                                        list(2), tile_count, tile_start, sortkey, clist, nullptr, nullptr));
            GS_LAUNCH_CHECK("tilesort_kernel_2k");
        }
        if (g1 > 0) {
            GS_TIMED("tilesort_kernel_1k", stream,
                     hipLaunchKernelGGL((tilesort_radix_kernel<128, 8, EXTRA_WAVE>), dim3(g1), dim3(128), 0, stream,
                                        cc + 1, list(1), tile_count, tile_start, sortkey, clist, cc + 0, list(0)));
            GS_LAUNCH_CHECK("tilesort_kernel_1k");
        }
    }
    if (gs::timing_on()) gs::timing_stage_end(stream, BINNING_STAGE);
    unsigned sgx, NS;
    const unsigned nblk = blend_grid(gx, gy, sgx, NS);
    O.final_T = at<float>(img, il.final_T);
    O.n_contrib_px = at<uint32_t>(img, il.n_contrib);
    O.n_contrib2loss_px = at<uint32_t>(img, il.n_contrib2loss);
    O.qwork = at<uint32_t>(geom, g.qwork);
    const uint32_t* clist = at<const uint32_t>(binning, bl.clist);
    const float4* recs = at<const float4>(geom, g.rec);
    if (mode == BLEND_SPLIT) {
        GS_TIMED("render_fwd_kernel", stream,
                 hipLaunchKernelGGL(render_fwd_kernel<BLEND_SPLIT>, dim3(nblk), dim3(64), 0, stream, W, H, gx, gy, sgx,
                                    NS, ranges, clist, recs, compute_locally, bg, O));
    } else if (mode == BLEND_SPLIT_GEO) {
        GS_TIMED("render_fwd_geo_kernel", stream,
                 hipLaunchKernelGGL(render_fwd_kernel<BLEND_SPLIT_GEO>, dim3(nblk), dim3(64), 0, stream, W, H, gx, gy,
                                    sgx, NS, ranges, clist, recs, compute_locally, bg, O));
    } else if (mode == BLEND_FULL) {
        GS_TIMED("render_fwd_kernel", stream,
                 hipLaunchKernelGGL(render_fwd_kernel<BLEND_FULL>, dim3(nblk), dim3(64), 0, stream, W, H, gx, gy, sgx,
                                    NS, ranges, clist, recs, compute_locally, bg, O));
    } else if (mode == BLEND_SIMP) {
        GS_TIMED("render_fwd_kernel", stream,
                 hipLaunchKernelGGL(render_fwd_kernel<BLEND_SIMP>, dim3(nblk), dim3(64), 0, stream, W, H, gx, gy, sgx,
                                    NS, ranges, clist, recs, compute_locally, bg, O));
    } else {
        GS_REQUIRE(mode == BLEND_DEPTH && depth_io != nullptr, "bad blend mode %d", mode);
        GS_TIMED("render_depth_kernel", stream,
                 hipLaunchKernelGGL(render_depth_kernel, dim3(nblk), dim3(64), 0, stream, W, H, gx, gy, sgx, NS,
                                    ranges, clist, recs, bg, O, *depth_io));
        GS_LAUNCH_CHECK("render_depth_kernel");
        return GS_OK;
    }
    GS_LAUNCH_CHECK("render_fwd_kernel");
    return GS_OK;
}

int render_backward_impl(bool full, int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                         const float* conic_opacity, const uint8_t* compute_locally, void* geom, const void* binning,
                         const void* img, const float* dL_dpixels, float* dL_dmeans2D, int dL_dmeans2D_stride,
                         float* dL_dmeans2D_abs, float* dL_dconic_opacity, float* dL_dcolors, hipStream_t stream,
                         const GeoBwd* geo = nullptr, float* dL_dall_map = nullptr, void* clear_dst = nullptr,
                         int64_t clear_bytes = 0)
{
    GS_REQUIRE(geo == nullptr || (!full && dL_dall_map != nullptr), "render_geo: split path, dL_dall_map non-null");
    GS_REQUIRE(P >= 0 && W > 0 && H > 0 && R >= 0, "invalid sizes P=%d W=%d H=%d R=%lld", P, W, H, (long long)R);
    GS_REQUIRE(dL_dmeans2D_stride == 2 || dL_dmeans2D_stride == 3, "dL_dmeans2D row stride must be 2 or 3");
    GS_REQUIRE(((uintptr_t)conic_opacity & 15) == 0 && ((uintptr_t)dL_dconic_opacity & 15) == 0 &&
               ((uintptr_t)means2D & 7) == 0,
               "conic_opacity / dL_dconic_opacity must be 16-byte and means2D 8-byte aligned");
    GS_REQUIRE(geom != nullptr, "geom must be the forward's geometry workspace");
    ClearBuf clr{};
    if (int rc = clear_buf(clear_dst, clear_bytes, clr); rc != GS_OK) return rc;
    if (P == 0) {
        if (clr.n16 != 0) {
            GS_TIMED("clear_kernel", stream,
                     hipLaunchKernelGGL(clear_kernel, dim3((unsigned)std::min<size_t>(gs_div_up(clr.n16, 256), 4096)),
                                        dim3(256), 0, stream, clr));
            GS_LAUNCH_CHECK("clear_kernel");
        }
        return GS_OK;
    }
    const GeomLayout g = geom_layout(P, W, H);
    const ImgLayout il = img_layout(W, H);
    const BinLayout bl = bin_layout(R);
    const unsigned gx = (unsigned)((W + 15) / 16), gy = (unsigned)((H + 15) / 16);
    float4* gacc = at<float4>(geom, g.gacc);
    if (R > 0) {
        unsigned sgx, NS;
        const unsigned nblk = blend_grid(gx, gy, sgx, NS);
        const uint2* rng = at<uint2>(img, il.ranges);
        const uint32_t* clist = at<const uint32_t>(binning, bl.clist);
        const float4* recs = at<const float4>(geom, g.rec);
        // the split path's waves heaviest first (the forward recorded each
        // quadrant's work): the order is computed by eight blocks of the
        // kernel that clears the listed Gaussians' accumulators (every
        // backward starts from zero)
        uint32_t* sched = full ? nullptr : at<uint32_t>(geom, g.sched);
        uint32_t* scnt = full ? nullptr : at<uint32_t>(geom, g.scnt);
        const unsigned nsched = full ? 0u : 8u;
        const unsigned zb = std::min<unsigned>(gs_div_up(4 * (size_t)P, 1024), 512u) + nsched;
        GS_TIMED("zero_gacc_kernel", stream,
                 hipLaunchKernelGGL(zero_gacc_kernel, dim3(zb), dim3(1024), 0, stream,
                                    at<const uint32_t>(geom, g.meta), gacc, nsched, gx, gy, sgx, NS,
                                    at<const uint32_t>(geom, g.qwork), sched, scnt));
        GS_LAUNCH_CHECK("zero_gacc_kernel");
        if (full) {
            GS_TIMED("render_bwd_kernel", stream,
                     hipLaunchKernelGGL(render_bwd_kernel<true>, dim3(nblk), dim3(64), 0, stream, W, H, gx, gy, sgx,
                                        NS, rng, clist, recs, compute_locally, bg, at<float>(img, il.final_T),
                                        at<uint32_t>(img, il.n_contrib), dL_dpixels, reinterpret_cast<float*>(gacc),
                                        GeoBwd{}, nullptr, nullptr, nullptr, ClearBuf{nullptr, 0}));
        } else if (geo != nullptr) {
            GS_TIMED("render_bwd_geo_kernel", stream,
                     hipLaunchKernelGGL((render_bwd_kernel<false, true>), dim3(nblk), dim3(64), 0, stream, W, H, gx,
                                        gy, sgx, NS, rng, clist, recs, compute_locally, bg,
                                        at<float>(img, il.final_T), at<uint32_t>(img, il.n_contrib), dL_dpixels,
                                        reinterpret_cast<float*>(gacc), *geo, sched, scnt, nullptr, clr));
        } else {
            GS_TIMED("render_bwd_kernel", stream,
                     hipLaunchKernelGGL(render_bwd_kernel<false>, dim3(nblk), dim3(64), 0, stream, W, H, gx, gy, sgx,
                                        NS, rng, clist, recs, compute_locally, bg, at<float>(img, il.final_T),
                                        at<uint32_t>(img, il.n_contrib), dL_dpixels, reinterpret_cast<float*>(gacc),
                                        GeoBwd{}, sched, scnt, at<const uint32_t>(geom, g.meta), clr));
        }
        GS_LAUNCH_CHECK("render_bwd_kernel");
    } else if (clr.n16 != 0) {
        GS_TIMED("clear_kernel", stream,
                 hipLaunchKernelGGL(clear_kernel, dim3((unsigned)std::min<size_t>(gs_div_up(clr.n16, 256), 4096)),
                                    dim3(256), 0, stream, clr));
        GS_LAUNCH_CHECK("clear_kernel");
    }
    // without instances the forward wrote no flags: every output is zero
    GS_TIMED("unpack_grads_kernel", stream,
             hipLaunchKernelGGL(unpack_grads_kernel, dim3(gs_div_up((size_t)P, 256)), dim3(256), 0, stream, P,
                                R > 0 ? at<const int>(geom, g.cidx_of) : nullptr, gacc, dL_dmeans2D_stride,
                                dL_dmeans2D, dL_dmeans2D_abs, reinterpret_cast<float4*>(dL_dconic_opacity),
                                dL_dcolors,
                                (((uintptr_t)dL_dmeans2D | (uintptr_t)dL_dmeans2D_abs | (uintptr_t)dL_dcolors) & 15) == 0,
                                0.5f * (float)W, 0.5f * (float)H));
    GS_LAUNCH_CHECK("unpack_grads_kernel");
    if (geo != nullptr) {
        GS_TIMED("unpack_map_grads_kernel", stream,
                 hipLaunchKernelGGL(unpack_map_grads_kernel, dim3(gs_div_up((size_t)P, 256)), dim3(256), 0, stream,
                                    P, R > 0 ? at<const int>(geom, g.cidx_of) : nullptr,
                                    reinterpret_cast<const float*>(gacc), dL_dall_map));
        GS_LAUNCH_CHECK("unpack_map_grads_kernel");
    }
    return GS_OK;
}

// render_geo's maps (reference _r forward.cu:381-384,407-412): a second walk
// of a completed split forward's lists (geom / binning / img, R as there).
int render_geo_forward_impl(int P, int64_t R, int W, int H, float tan_fovx, float tan_fovy, const float* all_map,
                            const uint8_t* compute_locally, const void* geom, const void* binning, const void* img,
                            float* out_all_map, float* out_plane_depth, hipStream_t stream)
{
    GS_REQUIRE(P >= 0 && W > 0 && H > 0 && R >= 0, "invalid sizes P=%d W=%d H=%d R=%lld", P, W, H, (long long)R);
    GS_REQUIRE(geom != nullptr && img != nullptr && (R == 0 || binning != nullptr),
               "geom, binning and img must be the forward's workspaces");
    GS_REQUIRE((P == 0 || all_map != nullptr) && out_all_map != nullptr && out_plane_depth != nullptr,
               "all_map, out_all_map and out_plane_depth must be non-null");
    GS_REQUIRE(tan_fovx > 0.f && tan_fovy > 0.f, "tan_fovx / tan_fovy must be positive");
    const GeomLayout g = geom_layout(P, W, H);
    const ImgLayout il = img_layout(W, H);
    const BinLayout bl = bin_layout(R);
    const unsigned gx = (unsigned)((W + 15) / 16), gy = (unsigned)((H + 15) / 16);
    FwdOut O{};
    O.all_map = all_map;
    O.out_all_map = out_all_map;
    O.out_plane_depth = out_plane_depth;
    // the render host's camera (rasterize_points.cu:325-326,339): focal
    // lengths W / (2 tan_fovx), H / (2 tan_fovy) and centre (W / 2, H / 2), in float
    O.focal_x = (float)W / (2.0f * tan_fovx);
    O.focal_y = (float)H / (2.0f * tan_fovy);
    O.cx = (float)W * 0.5f;
    O.cy = (float)H * 0.5f;
    unsigned sgx, NS;
    const unsigned nblk = blend_grid(gx, gy, sgx, NS);
    GS_TIMED("render_geo_kernel", stream,
             hipLaunchKernelGGL(render_fwd_kernel<BLEND_GEO>, dim3(nblk), dim3(64), 0, stream, W, H, gx, gy, sgx, NS,
                                at<const uint2>(img, il.ranges),
                                R > 0 ? at<const uint32_t>(binning, bl.clist) : nullptr,
                                at<const float4>(geom, g.rec), compute_locally, nullptr, O));
    GS_LAUNCH_CHECK("render_geo_kernel");
    return GS_OK;
}

// Queues the count, the scan and the rest of the forward (forward()) against
// a binning buffer laid out for `cap` instances, and waits only for R, which
// arrives while the scatter, sorts and blend still run.  R > cap: the scatter
// and sorts did nothing (tilescan_kernel) and the caller redoes the forward
// with a buffer for R.
template <typename Fwd>
int reserved_forward(bool full, int P, int64_t cap, int W, int H, const float* means2D, const int* radii,
                     const uint8_t* compute_locally, const float* rects, const float* conic_opacity, void* geom,
                     int64_t* num_rendered, hipStream_t stream, int region_side, Fwd&& forward)
{
    GS_REQUIRE(cap > 0 && cap <= 0xffffffffll, "capacity must be in [1, 2^32 - 1] (got %lld)", (long long)cap);
    GS_REQUIRE(num_rendered != nullptr, "num_rendered must be non-null");
    Readback* rb = nullptr;
    if (int rc = readback_acquire(rb); rc != GS_OK) return rc;
    int rc = render_count_impl(full, P, W, H, means2D, radii, compute_locally, rects, conic_opacity, geom, nullptr,
                               stream, (uint64_t)cap, rb, region_side);
    if (rc == GS_OK) rc = forward();
    if (rc != GS_OK) {
        // a scan already queued may still store into the slot: let it land first
        (void)hipStreamSynchronize(stream);
        readback_release(rb);
        return rc;
    }
    // poll the slot's word for this use's sequence number; every 256 polls the
    // stream is queried, and once it is idle (or failed) the word is final
    uint64_t v = 0;
    hipError_t e = hipSuccess;
    for (uint32_t poll = 1;; poll++) {
        v = __atomic_load_n(rb->host, __ATOMIC_ACQUIRE);
        if ((uint32_t)(v >> 33) == rb->seq) break;
        if ((poll & 255u) == 0u) {
            const hipError_t q = hipStreamQuery(stream);
            if (q == hipErrorNotReady) continue;
            v = __atomic_load_n(rb->host, __ATOMIC_ACQUIRE);
            if ((uint32_t)(v >> 33) != rb->seq) e = q != hipSuccess ? q : hipErrorUnknown;
            break;
        }
        __builtin_ia32_pause();
    }
    readback_release(rb);
    if (e != hipSuccess) {
        gs::set_error("waiting for the instance count failed: %s", hipGetErrorString(e));
        return GS_ERR_HIP;
    }
    if (v & (1ull << 32)) {
        gs::set_error("number of tile instances exceeds 2^32-1");
        return GS_ERR_SIZE;
    }
    *num_rendered = (int64_t)(v & 0xffffffffull);
    return GS_OK;
}

}  // namespace

extern "C" int gs_render_accumulators(const void* geom, int P, int W, int H, int64_t R, const void** acc,
                                      const int** cidx_of)
{
    gs::clear_error();
    GS_REQUIRE(geom != nullptr && acc != nullptr && cidx_of != nullptr && P >= 0 && W > 0 && H > 0 && R >= 0,
               "invalid arguments");
    const GeomLayout g = geom_layout(P, W, H);
    *acc = static_cast<const char*>(geom) + g.gacc;
    *cidx_of = R > 0 ? reinterpret_cast<const int*>(static_cast<const char*>(geom) + g.cidx_of) : nullptr;
    return GS_OK;
}

extern "C" int gs_render_forward_count(int P, int W, int H, const float* means2D, const int* radii,
                                       const uint8_t* compute_locally, void* geom, int64_t* num_rendered,
                                       int region_side, hipStream_t stream)
{
    gs::clear_error();
    return render_count_impl(false, P, W, H, means2D, radii, compute_locally, nullptr, nullptr, geom, num_rendered,
                             stream, ~0ull, nullptr, region_side);
}

extern "C" int gs_render_forward(int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                                 const float* depths, const int* radii, const float* conic_opacity, const float* rgb,
                                 const uint8_t* compute_locally, void* geom, void* binning, void* img,
                                 float* out_color, int32_t* n_render, int32_t* n_consider, int32_t* n_contrib,
                                 int32_t* out_observe, int region_side, void* clear_dst, int64_t clear_bytes,
                                 hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(n_render && n_consider && n_contrib && out_observe && out_color, "null output");
    FwdOut O{};
    O.out_color = out_color;
    O.out_observe = out_observe;
    O.n_consider = n_consider;
    O.n_contrib_tile = n_contrib;
    if (int rc = clear_buf(clear_dst, clear_bytes, O.clr); rc != GS_OK) return rc;
    return render_forward_impl(BLEND_SPLIT, P, R, W, H, bg, means2D, depths, radii, conic_opacity, rgb,
                               compute_locally, nullptr, geom, binning, img, O, n_render, stream, nullptr,
                               region_side);
}

extern "C" int gs_render_forward_reserved(int P, int64_t capacity, int W, int H, const float* bg,
                                          const float* means2D, const float* depths, const int* radii,
                                          const float* conic_opacity, const float* rgb,
                                          const uint8_t* compute_locally, void* geom, void* binning, void* img,
                                          float* out_color, int32_t* n_render, int32_t* n_consider,
                                          int32_t* n_contrib, int32_t* out_observe, int64_t* num_rendered,
                                          int region_side, void* clear_dst, int64_t clear_bytes,
                                          hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(n_render && n_consider && n_contrib && out_observe && out_color, "null output");
    FwdOut O{};
    O.out_color = out_color;
    O.out_observe = out_observe;
    O.n_consider = n_consider;
    O.n_contrib_tile = n_contrib;
    if (int rc = clear_buf(clear_dst, clear_bytes, O.clr); rc != GS_OK) return rc;
    return reserved_forward(false, P, capacity, W, H, means2D, radii, compute_locally, nullptr, nullptr, geom,
                            num_rendered, stream, region_side, [&] {
                                return render_forward_impl(BLEND_SPLIT, P, capacity, W, H, bg, means2D, depths, radii,
                                                           conic_opacity, rgb, compute_locally, nullptr, geom, binning,
                                                           img, O, n_render, stream, nullptr, region_side);
                            });
}

namespace {
// render_geo's inputs and outputs on a FwdOut; the render host's camera
// (rasterize_points.cu:325-326,339): focal lengths W / (2 tan_fovx),
// H / (2 tan_fovy) and centre (W / 2, H / 2), in float
int set_geo(FwdOut& O, int P, int W, int H, float tan_fovx, float tan_fovy, const float* all_map, float* out_all_map,
            float* out_plane_depth)
{
    GS_REQUIRE((P == 0 || all_map != nullptr) && out_all_map != nullptr && out_plane_depth != nullptr,
               "all_map, out_all_map and out_plane_depth must be non-null");
    GS_REQUIRE(tan_fovx > 0.f && tan_fovy > 0.f, "tan_fovx / tan_fovy must be positive");
    O.all_map = all_map;
    O.out_all_map = out_all_map;
    O.out_plane_depth = out_plane_depth;
    O.focal_x = (float)W / (2.0f * tan_fovx);
    O.focal_y = (float)H / (2.0f * tan_fovy);
    O.cx = (float)W * 0.5f;
    O.cy = (float)H * 0.5f;
    return GS_OK;
}
}  // namespace

extern "C" int gs_render_forward_geo(int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                                     const float* depths, const int* radii, const float* conic_opacity,
                                     const float* rgb, const uint8_t* compute_locally, void* geom, void* binning,
                                     void* img, float* out_color, int32_t* n_render, int32_t* n_consider,
                                     int32_t* n_contrib, int32_t* out_observe, float tan_fovx, float tan_fovy,
                                     const float* all_map, float* out_all_map, float* out_plane_depth,
                                     int region_side, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(n_render && n_consider && n_contrib && out_observe && out_color, "null output");
    FwdOut O{};
    O.out_color = out_color;
    O.out_observe = out_observe;
    O.n_consider = n_consider;
    O.n_contrib_tile = n_contrib;
    if (int rc = set_geo(O, P, W, H, tan_fovx, tan_fovy, all_map, out_all_map, out_plane_depth); rc != GS_OK)
        return rc;
    return render_forward_impl(BLEND_SPLIT_GEO, P, R, W, H, bg, means2D, depths, radii, conic_opacity, rgb,
                               compute_locally, nullptr, geom, binning, img, O, n_render, stream, nullptr,
                               region_side);
}

extern "C" int gs_render_forward_reserved_geo(int P, int64_t capacity, int W, int H, const float* bg,
                                              const float* means2D, const float* depths, const int* radii,
                                              const float* conic_opacity, const float* rgb,
                                              const uint8_t* compute_locally, void* geom, void* binning, void* img,
                                              float* out_color, int32_t* n_render, int32_t* n_consider,
                                              int32_t* n_contrib, int32_t* out_observe, int64_t* num_rendered,
                                              float tan_fovx, float tan_fovy, const float* all_map,
                                              float* out_all_map, float* out_plane_depth, int region_side,
                                              hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(n_render && n_consider && n_contrib && out_observe && out_color, "null output");
    FwdOut O{};
    O.out_color = out_color;
    O.out_observe = out_observe;
    O.n_consider = n_consider;
    O.n_contrib_tile = n_contrib;
    if (int rc = set_geo(O, P, W, H, tan_fovx, tan_fovy, all_map, out_all_map, out_plane_depth); rc != GS_OK)
        return rc;
    return reserved_forward(false, P, capacity, W, H, means2D, radii, compute_locally, nullptr, nullptr, geom,
                            num_rendered, stream, region_side, [&] {
                                return render_forward_impl(BLEND_SPLIT_GEO, P, capacity, W, H, bg, means2D, depths,
                                                           radii, conic_opacity, rgb, compute_locally, nullptr, geom,
                                                           binning, img, O, n_render, stream, nullptr, region_side);
                            });
}

extern "C" int gs_render_backward(int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                                  const float* conic_opacity, const float* rgb, const uint8_t* compute_locally,
                                  void* geom, const void* binning, const void* img, const float* dL_dpixels,
                                  float* dL_dmeans2D, int dL_dmeans2D_stride, float* dL_dmeans2D_abs,
                                  float* dL_dconic_opacity, float* dL_dcolors, void* clear_dst, int64_t clear_bytes,
                                  hipStream_t stream)
{
    gs::clear_error();
    (void)rgb;
    GS_REQUIRE(dL_dmeans2D_abs != nullptr, "dL_dmeans2D_abs must be non-null");
    return render_backward_impl(false, P, R, W, H, bg, means2D, conic_opacity, compute_locally, geom, binning, img,
                                dL_dpixels, dL_dmeans2D, dL_dmeans2D_stride, dL_dmeans2D_abs, dL_dconic_opacity,
                                dL_dcolors, stream, nullptr, nullptr, clear_dst, clear_bytes);
}

extern "C" int gs_render_geo_forward(int P, int64_t R, int W, int H, float tan_fovx, float tan_fovy,
                                     const float* all_map, const uint8_t* compute_locally, const void* geom,
                                     const void* binning, const void* img, float* out_all_map,
                                     float* out_plane_depth, hipStream_t stream)
{
    gs::clear_error();
    return render_geo_forward_impl(P, R, W, H, tan_fovx, tan_fovy, all_map, compute_locally, geom, binning, img,
                                   out_all_map, out_plane_depth, stream);
}

extern "C" int gs_render_backward_geo(int P, int64_t R, int W, int H, const float* bg, float tan_fovx,
                                      float tan_fovy, const float* all_map_pixels, const float* all_maps,
                                      const float* means2D, const float* conic_opacity, const float* rgb,
                                      const uint8_t* compute_locally, void* geom, const void* binning,
                                      const void* img, const float* dL_dpixels, const float* dL_dout_all_map,
                                      const float* dL_dout_plane_depth, float* dL_dmeans2D, int dL_dmeans2D_stride,
                                      float* dL_dmeans2D_abs, float* dL_dconic_opacity, float* dL_dcolors,
                                      float* dL_dall_map, void* clear_dst, int64_t clear_bytes, hipStream_t stream)
{
    gs::clear_error();
    (void)rgb;
    GS_REQUIRE(dL_dmeans2D_abs != nullptr && dL_dall_map != nullptr, "dL_dmeans2D_abs and dL_dall_map must be non-null");
    GS_REQUIRE(P == 0 || (all_map_pixels != nullptr && all_maps != nullptr && dL_dout_all_map != nullptr &&
                          dL_dout_plane_depth != nullptr),
               "all_map_pixels, all_maps, dL_dout_all_map and dL_dout_plane_depth must be non-null");
    GS_REQUIRE(tan_fovx > 0.f && tan_fovy > 0.f, "tan_fovx / tan_fovy must be positive");
    // the backward host's focal lengths (rasterizer_impl.cu:760-761)
    const GeoBwd geo{all_maps, all_map_pixels, dL_dout_all_map, dL_dout_plane_depth, (float)W / (2.0f * tan_fovx),
                     (float)H / (2.0f * tan_fovy)};
    return render_backward_impl(false, P, R, W, H, bg, means2D, conic_opacity, compute_locally, geom, binning, img,
                                dL_dpixels, dL_dmeans2D, dL_dmeans2D_stride, dL_dmeans2D_abs, dL_dconic_opacity,
                                dL_dcolors, stream, &geo, dL_dall_map, clear_dst, clear_bytes);
}

extern "C" int gs_render_full_count(int P, int W, int H, const float* means2D, const int* radii, const float* rects,
                                    const float* conic_opacity, void* geom, int64_t* num_rendered, hipStream_t stream)
{
    gs::clear_error();
    return render_count_impl(true, P, W, H, means2D, radii, nullptr, rects, conic_opacity, geom, num_rendered,
                             stream);
}

extern "C" int gs_render_full_forward(int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                                      const float* depths, const int* radii, const float* rects,
                                      const float* conic_opacity, const float* colors, void* geom, void* binning,
                                      void* img, float* out_color, float* accum_max_count, float* accum_weights,
                                      int32_t* accum_weights_count, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(out_color != nullptr, "out_color must be non-null");
    GS_REQUIRE((accum_weights == nullptr) == (accum_weights_count == nullptr),
               "accum_weights and accum_weights_count go together");
    GS_REQUIRE(accum_weights == nullptr || accum_max_count != nullptr, "render_simp needs accum_max_count");
    FwdOut O{};
    O.out_color = out_color;
    O.accum_max_count = accum_max_count;
    O.accum_weights = accum_weights;
    O.accum_weights_count = accum_weights_count;
    return render_forward_impl(accum_weights != nullptr ? BLEND_SIMP : BLEND_FULL, P, R, W, H, bg, means2D, depths,
                               radii, conic_opacity, colors, nullptr, rects, geom, binning, img, O, nullptr, stream);
}

extern "C" int gs_render_full_forward_reserved(int P, int64_t capacity, int W, int H, const float* bg,
                                               const float* means2D, const float* depths, const int* radii,
                                               const float* rects, const float* conic_opacity, const float* colors,
                                               void* geom, void* binning, void* img, float* out_color,
                                               float* accum_max_count, float* accum_weights,
                                               int32_t* accum_weights_count, int64_t* num_rendered, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(out_color != nullptr, "out_color must be non-null");
    GS_REQUIRE((accum_weights == nullptr) == (accum_weights_count == nullptr),
               "accum_weights and accum_weights_count go together");
    GS_REQUIRE(accum_weights == nullptr || accum_max_count != nullptr, "render_simp needs accum_max_count");
    FwdOut O{};
    O.out_color = out_color;
    O.accum_max_count = accum_max_count;
    O.accum_weights = accum_weights;
    O.accum_weights_count = accum_weights_count;
    return reserved_forward(true, P, capacity, W, H, means2D, radii, nullptr, rects, conic_opacity, geom,
                            num_rendered, stream, 0, [&] {
                                return render_forward_impl(accum_weights != nullptr ? BLEND_SIMP : BLEND_FULL, P,
                                                           capacity, W, H, bg, means2D, depths, radii, conic_opacity,
                                                           colors, nullptr, rects, geom, binning, img, O, nullptr,
                                                           stream);
                            });
}

extern "C" int gs_render_full_depth(int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                                    const float* depths, const int* radii, const float* rects,
                                    const float* conic_opacity, const float* colors, const float* means3D,
                                    const float* scales, const float* rotations, const float* projmatrix,
                                    const float* campos, void* geom, void* binning, void* img, float* out_color,
                                    float* out_pts, float* out_depth, float* accum_alpha, int32_t* gidx,
                                    float* discriminants, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(out_color && out_pts && out_depth && accum_alpha && gidx && discriminants,
               "every output must be non-null");
    GS_REQUIRE(projmatrix && campos, "projmatrix and campos must be non-null");
    GS_REQUIRE(P == 0 || (means3D && scales && rotations), "means3D, scales and rotations must be non-null");
    GS_REQUIRE(((uintptr_t)rotations & 15) == 0, "rotations must be 16-byte aligned");
    FwdOut O{};
    O.out_color = out_color;
    DepthIO D{means3D, scales, rotations, projmatrix, campos, out_pts, out_depth, accum_alpha, gidx, discriminants};
    return render_forward_impl(BLEND_DEPTH, P, R, W, H, bg, means2D, depths, radii, conic_opacity, colors, nullptr,
                               rects, geom, binning, img, O, nullptr, stream, &D);
}

extern "C" int gs_render_full_backward(int P, int64_t R, int W, int H, const float* bg, const float* means2D,
                                       const float* conic_opacity, void* geom, const void* binning, const void* img,
                                       const float* dL_dpixels, float* dL_dmeans2D, float* dL_dconic_opacity,
                                       float* dL_dcolors, hipStream_t stream)
{
    gs::clear_error();
    return render_backward_impl(true, P, R, W, H, bg, means2D, conic_opacity, nullptr, geom, binning, img, dL_dpixels,
                                dL_dmeans2D, 3, nullptr, dL_dconic_opacity, dL_dcolors, stream);
}

namespace gs {
// The VALU probes (which 0: forward, 1: backward) over `iters` passes of 64
// entries per wave, VALU_PROBE_BLOCKS waves.
int render_valu_probe(int which, int iters, float* y, hipStream_t stream)
{
    GS_REQUIRE(which >= 0 && which <= 2, "which must be 0 (forward), 1 (backward) or 2 (backward, half tiles)");
    GS_REQUIRE(iters >= 0 && y != nullptr, "iters must be >= 0 and y non-null");
    if (iters == 0) return GS_OK;
    if (which == 0) {
        GS_TIMED("valu_probe_fwd_kernel", stream,
                 hipLaunchKernelGGL(valu_probe_kernel<0>, dim3(VALU_PROBE_BLOCKS), dim3(64), 0, stream, iters, y));
    } else if (which == 1) {
        GS_TIMED("valu_probe_bwd_kernel", stream,
                 hipLaunchKernelGGL(valu_probe_kernel<1>, dim3(VALU_PROBE_BLOCKS), dim3(64), 0, stream, iters, y));
    } else {
        GS_TIMED("valu_probe_bwd2_kernel", stream,
                 hipLaunchKernelGGL(valu_probe_kernel<2>, dim3(VALU_PROBE_BLOCKS), dim3(64), 0, stream, iters, y));
    }
    GS_LAUNCH_CHECK("valu_probe_kernel");
    return GS_OK;
}
}  // namespace gs
