// Vertex records of the 3DGS PLY file <-> the Gaussian parameter tensors.
//
// Reference: BlitzGS scene/gaussian_model.py
//   :434-446  construct_list_of_attributes  (x y z nx ny nz f_dc_* f_rest_* opacity scale_* rot_* [lod_level])
//   :447-520  save_ply   normals written as 0; f_dc / f_rest transposed (P,K,3) -> (P,3,K) and flattened,
//                        so file column f_rest_{c*K+k} holds features_rest[:, k, c]; all values float32
//   :522-575  load_ply   the inverse, by property name; lod_level read as float and cast to int8
// The file I/O itself goes through the plyfile package (binary little-endian,
// one 'vertex' element whose records are the properties back to back).
//
// Design: the reference builds the records on the host (numpy concatenate and
// a per-row tuple conversion) and reads them field by field into float64
// arrays before the tensors go to the GPU.  Here the host moves only the raw
// record bytes (one contiguous copy each way) and one kernel per direction
// turns the array-of-records into the separate row-major tensors (or back).
// A block stages PLY_ROWS whole records in LDS with one contiguous, 16-byte
// vectorised sweep; every tensor's slice of those rows is then a contiguous
// span of the tensor, written (or read) with float4 accesses through a column
// map held in LDS.  Both directions are pure HBM streams: each byte of the
// records and of the tensors crosses HBM once.
#include "gs_device.h"
#include "gs_host.h"
#include "../../include/blitzgs_amd.h"

namespace {

constexpr int PLY_THREADS = 256;
constexpr int PLY_ROWS = 128;             // records per block: with 62 columns (SH 3) 31 KB of LDS
constexpr int PLY_MAX_COLS = 120;         // record columns (and tensor columns) of one call: <= 60 KB of LDS
constexpr int PLY_MAX_TENSORS = 8;
constexpr int PLY_BATCH = 8;              // float4 loads a thread issues before its first LDS store

struct PlyTensor {
    void* ptr;
    int width;
    int i8;          // 1: int8 tensor (lod_level), 0: float32
    int col0;        // first entry of this tensor in the column map
    uint32_t magic;  // ceil(2^24 / width): k / width for k < 2^24 / width
};

struct PlySpec {
    PlyTensor t[PLY_MAX_TENSORS];
    int n_t;
    int rec_cols;
    int total;                 // sum of the tensors' widths
    short col[PLY_MAX_COLS];   // record column of tensor column j (tensors concatenated)
};

__device__ __forceinline__ int div_w(int k, uint32_t magic) { return (int)(((uint64_t)(uint32_t)k * magic) >> 24); }

// float -> int8 as numpy's astype(np.int8) does on the host: truncate to a
// 32-bit integer (out of range and NaN give INT_MIN), keep the low byte.
__device__ __forceinline__ signed char f2i8(float v)
{
    const int iv = (v >= -2147483648.0f && v < 2147483648.0f) ? (int)v : (int)0x80000000;
    return (signed char)(iv & 0xff);
}

// Contiguous copy of n words from global to LDS (or back), float4 where both
// ends are 16-byte aligned; loads are batched so each wave has several in flight.
__device__ __forceinline__ void span_to_lds(const float* __restrict__ src, float* __restrict__ s, int n, bool vec)
{
    const int tid = (int)threadIdx.x;
    if (vec) {
        const int n4 = n >> 2;
        const float4* s4 = reinterpret_cast<const float4*>(src);
        for (int base = 0; base < n4; base += PLY_BATCH * PLY_THREADS) {
            float4 v[PLY_BATCH];
#pragma unroll
            for (int i = 0; i < PLY_BATCH; i++) {
                const int q = base + tid + i * PLY_THREADS;
                v[i] = q < n4 ? s4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int i = 0; i < PLY_BATCH; i++) {
                const int q = base + tid + i * PLY_THREADS;
                if (q < n4) reinterpret_cast<float4*>(s)[q] = v[i];
            }
        }
        for (int k = (n4 << 2) + tid; k < n; k += PLY_THREADS) s[k] = src[k];
    } else {
        for (int k = tid; k < n; k += PLY_THREADS) s[k] = src[k];
    }
}

// whole 16-byte groups leave as streaming stores (written once, not re-read)
__device__ __forceinline__ void lds_to_span(const float* __restrict__ s, float* __restrict__ dst, int n, bool vec)
{
    const int tid = (int)threadIdx.x;
    if (vec) {
        const int n4 = n >> 2;
        for (int q = tid; q < n4; q += PLY_THREADS)
            gs::st_stream(&reinterpret_cast<float4*>(dst)[q], reinterpret_cast<const float4*>(s)[q]);
        for (int k = (n4 << 2) + tid; k < n; k += PLY_THREADS) dst[k] = s[k];
    } else {
        for (int k = tid; k < n; k += PLY_THREADS) dst[k] = s[k];
    }
}

// records (P, rec_cols) float32 -> tensors.  Tensor t's rows [r0, r0+nr) are
// the contiguous span [r0*w, (r0+nr)*w) of it; element k of the span is
// (row k / w, column k % w) and reads LDS record column col[col0 + k % w].
__global__ __launch_bounds__(PLY_THREADS) void ply_unpack_kernel(int64_t P, const float* __restrict__ rec,
                                                                 PlySpec S, int rec_vec)
{
    extern __shared__ __align__(16) float s_rec[];
    __shared__ int s_col[PLY_MAX_COLS];
    const int tid = (int)threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * PLY_ROWS;
    const int nr = (int)min((int64_t)PLY_ROWS, P - r0);
    const int rc = S.rec_cols;
    if (tid < S.total) s_col[tid] = S.col[tid];
    // r0 * rc is a multiple of 128 words: the span is 16-byte aligned when the records are
    span_to_lds(rec + r0 * rc, s_rec, nr * rc, rec_vec != 0);
    __syncthreads();
    for (int t = 0; t < S.n_t; t++) {
        const PlyTensor T = S.t[t];
        const int w = T.width;
        const int n = nr * w;
        const int* cm = s_col + T.col0;
        if (T.i8) {
            signed char* dst = static_cast<signed char*>(T.ptr) + r0 * w;
            for (int k = tid; k < n; k += PLY_THREADS) {
                const int row = div_w(k, T.magic);
                dst[k] = f2i8(s_rec[row * rc + cm[k - row * w]]);
            }
            continue;
        }
        float* dst = static_cast<float*>(T.ptr) + r0 * w;
        // r0 * w is a multiple of 128 words: 16-byte aligned when the tensor is
        const bool vec = ((reinterpret_cast<uintptr_t>(T.ptr) & 15) == 0);
        const int n4 = vec ? (n >> 2) : 0;
        for (int q = tid; q < n4; q += PLY_THREADS) {
            const int k = q << 2;
            int row = div_w(k, T.magic);
            int col = k - row * w;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[e] = s_rec[row * rc + cm[col]];
                if (++col == w) { col = 0; row++; }
            }
            gs::st_stream(&reinterpret_cast<float4*>(dst)[q], make_float4(v[0], v[1], v[2], v[3]));
        }
        for (int k = (n4 << 2) + tid; k < n; k += PLY_THREADS) {
            const int row = div_w(k, T.magic);
            dst[k] = s_rec[row * rc + cm[k - row * w]];
        }
    }
}

// tensors -> records (P, rec_cols) float32; record columns no tensor column
// maps to are written as 0 (the reference's zero normals).
__global__ __launch_bounds__(PLY_THREADS) void ply_pack_kernel(int64_t P, float* __restrict__ rec, PlySpec S,
                                                               int rec_vec)
{
    extern __shared__ __align__(16) float s_rec[];
    __shared__ int s_col[PLY_MAX_COLS];
    const int tid = (int)threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * PLY_ROWS;
    const int nr = (int)min((int64_t)PLY_ROWS, P - r0);
    const int rc = S.rec_cols;
    const int n_words = nr * rc;
    if (tid < S.total) s_col[tid] = S.col[tid];
    for (int k = tid; k < n_words; k += PLY_THREADS) s_rec[k] = 0.f;
    __syncthreads();
    for (int t = 0; t < S.n_t; t++) {
        const PlyTensor T = S.t[t];
        const int w = T.width;
        const int n = nr * w;
        const int* cm = s_col + T.col0;
        if (T.i8) {
            const signed char* src = static_cast<const signed char*>(T.ptr) + r0 * w;
            for (int k = tid; k < n; k += PLY_THREADS) {
                const int row = div_w(k, T.magic);
                s_rec[row * rc + cm[k - row * w]] = (float)src[k];
            }
            continue;
        }
        const float* src = static_cast<const float*>(T.ptr) + r0 * w;
        const bool vec = ((reinterpret_cast<uintptr_t>(T.ptr) & 15) == 0);
        const int n4 = vec ? (n >> 2) : 0;
        for (int base = 0; base < n4; base += PLY_BATCH * PLY_THREADS) {
            float4 v[PLY_BATCH];
#pragma unroll
            for (int i = 0; i < PLY_BATCH; i++) {
                const int q = base + tid + i * PLY_THREADS;
                v[i] = q < n4 ? reinterpret_cast<const float4*>(src)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int i = 0; i < PLY_BATCH; i++) {
                const int q = base + tid + i * PLY_THREADS;
                if (q < n4) {
                    const int k = q << 2;
                    int row = div_w(k, T.magic);
                    int col = k - row * w;
                    const float e4[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        s_rec[row * rc + cm[col]] = e4[e];
                        if (++col == w) { col = 0; row++; }
                    }
                }
            }
        }
        for (int k = (n4 << 2) + tid; k < n; k += PLY_THREADS) {
            const int row = div_w(k, T.magic);
            s_rec[row * rc + cm[k - row * w]] = src[k];
        }
    }
    __syncthreads();
    lds_to_span(s_rec, rec + r0 * rc, n_words, rec_vec != 0);
}

int make_spec(int n_tensors, const gs_ply_tensor* tensors, const int32_t* colmap, int rec_cols, bool pack,
              PlySpec& S)
{
    GS_REQUIRE(rec_cols >= 1 && rec_cols <= PLY_MAX_COLS, "rec_cols must be in [1, %d]", PLY_MAX_COLS);
    GS_REQUIRE(n_tensors >= 1 && n_tensors <= PLY_MAX_TENSORS, "n_tensors must be in [1, %d]", PLY_MAX_TENSORS);
    GS_REQUIRE(tensors != nullptr && colmap != nullptr, "tensors and colmap must be non-null");
    S = PlySpec{};
    int total = 0;
    for (int t = 0; t < n_tensors; t++) {
        const gs_ply_tensor& d = tensors[t];
        GS_REQUIRE(d.width >= 1, "tensor %d: width must be >= 1", t);
        GS_REQUIRE(d.type == GS_PLY_F32 || d.type == GS_PLY_I8, "tensor %d: type must be GS_PLY_F32 or GS_PLY_I8", t);
        GS_REQUIRE(total + d.width <= PLY_MAX_COLS, "more than %d tensor columns", PLY_MAX_COLS);
        S.t[t] = PlyTensor{d.ptr, d.width, d.type == GS_PLY_I8 ? 1 : 0, total,
                           (uint32_t)(((1u << 24) + (uint32_t)d.width - 1) / (uint32_t)d.width)};
        total += d.width;
    }
    bool used[PLY_MAX_COLS] = {};
    for (int j = 0; j < total; j++) {
        GS_REQUIRE(colmap[j] >= 0 && colmap[j] < rec_cols, "colmap[%d] = %d is outside [0, %d)", j, colmap[j],
                   rec_cols);
        // packing writes each record column from at most one tensor column
        GS_REQUIRE(!(pack && used[colmap[j]]), "colmap maps two tensor columns to record column %d", colmap[j]);
        used[colmap[j]] = true;
        S.col[j] = (short)colmap[j];
    }
    S.n_t = n_tensors;
    S.rec_cols = rec_cols;
    S.total = total;
    return GS_OK;
}

}  // namespace

extern "C" int gs_ply_unpack(int64_t P, const float* records, int32_t rec_cols, int32_t n_tensors,
                             const gs_ply_tensor* tensors, const int32_t* colmap, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0, "P must be >= 0");
    PlySpec S;
    if (make_spec(n_tensors, tensors, colmap, rec_cols, false, S) != GS_OK) return GS_ERR_ARG;
    if (P == 0) return GS_OK;
    GS_REQUIRE(records != nullptr, "records must be non-null");
    for (int t = 0; t < n_tensors; t++) GS_REQUIRE(tensors[t].ptr != nullptr, "tensor %d: null pointer", t);
    const int64_t blocks = (P + PLY_ROWS - 1) / PLY_ROWS;
    GS_REQUIRE(blocks < 0x7fffffffll && P * rec_cols < (1ll << 40), "too many records for one launch");
    const int rec_vec = (reinterpret_cast<uintptr_t>(records) & 15) == 0;
    const size_t lds = sizeof(float) * PLY_ROWS * rec_cols;
    GS_TIMED("ply_unpack_kernel", stream,
             hipLaunchKernelGGL(ply_unpack_kernel, dim3((unsigned)blocks), dim3(PLY_THREADS), lds, stream, P,
                                records, S, rec_vec));
    GS_LAUNCH_CHECK("ply_unpack_kernel");
    return GS_OK;
}

extern "C" int gs_ply_pack(int64_t P, int32_t n_tensors, const gs_ply_tensor* tensors, const int32_t* colmap,
                           int32_t rec_cols, float* records, hipStream_t stream)
{
    gs::clear_error();
    GS_REQUIRE(P >= 0, "P must be >= 0");
    PlySpec S;
    if (make_spec(n_tensors, tensors, colmap, rec_cols, true, S) != GS_OK) return GS_ERR_ARG;
    if (P == 0) return GS_OK;
    GS_REQUIRE(records != nullptr, "records must be non-null");
    for (int t = 0; t < n_tensors; t++) GS_REQUIRE(tensors[t].ptr != nullptr, "tensor %d: null pointer", t);
    const int64_t blocks = (P + PLY_ROWS - 1) / PLY_ROWS;
    GS_REQUIRE(blocks < 0x7fffffffll && P * rec_cols < (1ll << 40), "too many records for one launch");
    const int rec_vec = (reinterpret_cast<uintptr_t>(records) & 15) == 0;
    const size_t lds = sizeof(float) * PLY_ROWS * rec_cols;
    GS_TIMED("ply_pack_kernel", stream,
             hipLaunchKernelGGL(ply_pack_kernel, dim3((unsigned)blocks), dim3(PLY_THREADS), lds, stream, P, records,
                                S, rec_vec));
    GS_LAUNCH_CHECK("ply_pack_kernel");
    return GS_OK;
}
