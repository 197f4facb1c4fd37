/*
 * blitzgs_amd -- C ABI of the MI355X (gfx950) differentiable Gaussian
 * rasterizer, simple-knn distCUDA2 and fused-ssim replacements.
 *
 * Conventions
 *   - Every pointer argument named after a tensor is a device pointer to a
 *     contiguous row-major array on the current HIP device; fp32 unless the
 *     type says otherwise.  bool tensors are uint8_t (0/1).
 *   - Every entry point is asynchronous on `stream` (a hipStream_t; 0 is the
 *     null stream) unless documented otherwise, returns 0 on success and a
 *     negative code on error; gs_last_error() then returns a message
 *     (thread-local, valid until the next call on this thread).
 *   - Argument validation mirrors the reference's checks; error text is
 *     returned, never printed.
 *   - Outputs are fully written by the library (no caller-side zeroing) unless
 *     stated.
 *   - Workspaces are plain device byte buffers sized by the *_bytes queries and
 *     owned by the caller (the Python layer allocates them as torch uint8
 *     tensors, as the reference keeps its geom/binning/img buffers).
 *
 * Reference interfaces replaced (paths under /root/reference/submodule, except
 *   the scene/ one, which is under /root/reference):
 *   diff-gaussian-rasterization_f/rasterize_points.cu:834-923  PreprocessGaussiansCUDA
 *   diff-gaussian-rasterization_f/rasterize_points.cu:926-1029 PreprocessGaussiansBackwardCUDA
 *   diff-gaussian-rasterization_r/rasterize_points.cu:273-361  RenderGaussiansCUDA
 *   diff-gaussian-rasterization_r/rasterize_points.cu:363-436  RenderGaussiansBackwardCUDA
 *   simple-knn/spatial.cu:15-26                                distCUDA2
 *   fused-ssim/ssim.cu:367-402                                 fusedssim
 *   fused-ssim/ssim.cu:404-441                                 fusedssim_backward
 *   diff-gaussian-rasterization_f/rasterize_points.cu:258-289  GetLocal2jIdsBoolCUDA
 *   diff-gaussian-rasterization_f/rasterize_points.cu:337-367  GetLocal2jIdsBoolAdjustMode6CUDA
 *   diff-gaussian-rasterization_f/rasterize_points.cu:807-832  adamUpdate
 *   scene/gaussian_model.py:434-575 (save_ply / load_ply record layout)  gs_ply_pack / gs_ply_unpack
 */
#ifndef BLITZGS_AMD_H
#define BLITZGS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* gs_stream_t; /* == hipStream_t */

/* Library version (major*10000 + minor*100 + patch) and last error text. */
int gs_version(void);
const char* gs_last_error(void);

/* ------------------------------------------------------------------------ *
 * Preprocess forward.  Replaces PreprocessGaussiansCUDA
 * (diff-gaussian-rasterization_f/rasterize_points.cu:834-923; kernel
 * cuda_rasterizer/forward.cu:164-284).
 *   P Gaussians, SH degree D (0..3), K = sh.size(1) >= (D+1)^2 coefficients.
 *   means3D (P,3), scales (P,3), rotations (P,4) quaternions (r,x,y,z),
 *   sh (P,K,3), opacities (P,1).  viewmatrix/projmatrix (4,4) and campos (3)
 *   are device tensors laid out as the reference's settings tensors.
 *   Outputs: means2D (P,2), depths (P), radii int32 (P), cov3D (P,6),
 *   conic_opacity (P,4), rgb (P,3), clamped uint8 (P,3).  cov3D may be
 *   NULL (not written; gs_preprocess_backward then recomputes it).
 *   rotations and conic_opacity must be 16-byte aligned.
 * ------------------------------------------------------------------------ */
int gs_preprocess_forward(int P, int D, int K, const float* means3D, const float* scales,
                          const float* rotations, const float* sh, const float* opacities,
                          float scale_modifier, const float* viewmatrix, const float* projmatrix,
                          const float* campos, float tanfovx, float tanfovy, int image_height,
                          int image_width, float* means2D, float* depths, int* radii, float* cov3D,
                          float* conic_opacity, float* rgb, uint8_t* clamped, gs_stream_t stream);

/* Preprocess backward.  Replaces PreprocessGaussiansBackwardCUDA
 * (diff-gaussian-rasterization_f/rasterize_points.cu:926-1029; kernels
 * cuda_rasterizer/backward.cu:146-276 and 348-400).
 *   dL_dmeans2D has row stride dL_dmeans2D_stride floats (2, or 3 for the
 *   reference's padded (P,3) layout); dL_dconic_opacity (P,4); dL_drgb (P,3).
 *   cov3D: the forward's output, or NULL to recompute it from scales and
 *   rotations (the same arithmetic as the forward's).
 *   Outputs: dL_dmeans3D (P,3), dL_dscales (P,3), dL_drotations (P,4),
 *   dL_dsh (P,K,3), dL_dopacity (P,1) = dL_dconic_opacity[:,3]. */
int gs_preprocess_backward(int P, int D, int K, const float* means3D, const float* scales,
                           const float* rotations, const float* sh, float scale_modifier,
                           const float* viewmatrix, const float* projmatrix, const float* campos,
                           float tanfovx, float tanfovy, int image_height, int image_width,
                           const int* radii, const float* cov3D, const uint8_t* clamped,
                           const float* dL_dmeans2D, int dL_dmeans2D_stride,
                           const float* dL_dconic_opacity, const float* dL_drgb, float* dL_dmeans3D,
                           float* dL_dscales, float* dL_drotations, float* dL_dsh,
                           float* dL_dopacity, gs_stream_t stream);

/* Preprocess forward and backward through a record buffer: the forward packs
 * each visible Gaussian's mean, scale, rotation and clamp flags into 48 bytes
 * (with a 64-bit visibility mask per 64 Gaussians) and the backward reads
 * those instead of means3D, scales, rotations, radii and clamped, which it
 * does not take.  The counterpart of the reference's geomBuffer, which its
 * forward fills for its backward (rasterizer_impl.cu:982-1067 writes it,
 * 1069-1129 reads it); outputs are bit-identical to gs_preprocess_forward /
 * gs_preprocess_backward on the same inputs.
 *   bwd_records: gs_preprocess_record_bytes(P) bytes, 256-byte aligned,
 *   written by gs_preprocess_forward_rec and read by gs_preprocess_backward_rec
 *   of the same P (records naming a Gaussian outside their own group of 64
 *   are skipped).  clamped may be NULL here (not written: the records hold
 *   the flags).
 *   outputs_zeroed (backward): nonzero when dL_dsh already holds zeros (the
 *   render backward cleared it while it ran: gs_render_backward's clear_dst):
 *   only the visible Gaussians' dL_dsh rows are written then (every other
 *   output is written whole either way; the reference allocates them all
 *   with torch::zeros, rasterize_points.cu:960-966). */
int64_t gs_preprocess_record_bytes(int P);
int gs_preprocess_forward_rec(int P, int D, int K, const float* means3D, const float* scales,
                              const float* rotations, const float* sh, const float* opacities,
                              float scale_modifier, const float* viewmatrix, const float* projmatrix,
                              const float* campos, float tanfovx, float tanfovy, int image_height,
                              int image_width, float* means2D, float* depths, int* radii, float* cov3D,
                              float* conic_opacity, float* rgb, uint8_t* clamped, void* bwd_records,
                              gs_stream_t stream);
int gs_preprocess_backward_rec(int P, int D, int K, const void* bwd_records, const float* sh,
                               float scale_modifier, const float* viewmatrix, const float* projmatrix,
                               const float* campos, float tanfovx, float tanfovy, int image_height,
                               int image_width, const float* cov3D, const float* dL_dmeans2D,
                               int dL_dmeans2D_stride, const float* dL_dconic_opacity,
                               const float* dL_drgb, float* dL_dmeans3D, float* dL_dscales,
                               float* dL_drotations, float* dL_dsh, float* dL_dopacity,
                               int outputs_zeroed, gs_stream_t stream);

/* gs_preprocess_backward_rec with outputs_zeroed = 1 whose incoming
 * gradients are exactly what a split render backward returned: instead of
 * the dense dL_dmeans2D / dL_dconic_opacity / dL_drgb it reads that render's
 * per-Gaussian accumulators (render_acc, render_cidx_of: gs_render_accumulators
 * of the render's geom, after its gs_render_backward and before any other
 * call on that geom) and applies the same factors as the render backward's
 * outputs (dmean/dpixel W/2, H/2; -1/2 on the conic terms), so the gradients
 * are bit-identical; an invisible Gaussian's dL_dopacity is zero (the render
 * listed it nowhere).  Needs 16-byte SH rows (K a multiple of 4, sh and
 * dL_dsh 16-byte aligned) and dL_dsh cleared.  No counterpart in the
 * reference: it saves the dense arrays' gathers (one visible Gaussian in
 * five at the benchmark's scene touches nearly every line of them). */
int gs_preprocess_backward_rec_acc(int P, int D, int K, const void* bwd_records, const float* sh,
                                   float scale_modifier, const float* viewmatrix, const float* projmatrix,
                                   const float* campos, float tanfovx, float tanfovy, int image_height,
                                   int image_width, const float* cov3D, const void* render_acc,
                                   const int* render_cidx_of, float* dL_dmeans3D, float* dL_dscales,
                                   float* dL_drotations, float* dL_dsh, float* dL_dopacity,
                                   gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Render forward, in two calls because the size of the instance buffers
 * (R = number of Gaussian/tile instances) is known only after counting.
 * Together they replace RenderGaussiansCUDA
 * (diff-gaussian-rasterization_r/rasterize_points.cu:273-361;
 * cuda_rasterizer/rasterizer_impl.cu:556-723, forward.cu:263-413).
 *
 *   geom    : gs_render_geom_bytes(P, W, H) bytes  (counts, offsets)
 *   binning : gs_render_binning_bytes(R) bytes     (the blend's sorted list;
 *             the point list and its keys on request; a buffer sized for a
 *             capacity >= R serves R)
 *   img     : gs_render_img_bytes(W, H) bytes      (tile ranges, per-pixel
 *             final transmittance and contributor counts)
 * compute_locally is a uint8 (ceil(H/16), ceil(W/16)) tile mask, or NULL
 * when every tile is local.
 * region_side: 0, 2, 4 or 8 -- the side, in tiles, of the square regions the
 * split path bins through (0: the smallest the tile grid allows; a side below
 * that is raised to it).  Every output is the same for every side; larger
 * regions suit Gaussians that each cover many tiles (fewer region entries,
 * longer lists to sort).  A count call and the forward call after it take
 * the same value.
 * ------------------------------------------------------------------------ */
size_t gs_render_geom_bytes(int P, int image_width, int image_height);
size_t gs_render_binning_bytes(int64_t R);
size_t gs_render_img_bytes(int image_width, int image_height);

/* Count the tile instances: per-tile counts and offsets (and, for the
 * sorts, per-region list lengths and offsets over 2x2-tile regions) go to
 * `geom`; R is copied to *num_rendered.  Synchronises `stream` (the
 * reference reads R back with cudaMemcpy at rasterizer_impl.cu:621). */
int gs_render_forward_count(int P, int image_width, int image_height, const float* means2D,
                            const int* radii, const uint8_t* compute_locally, void* geom,
                            int64_t* num_rendered, int region_side, gs_stream_t stream);

/* Duplicate, sort, range and blend.  Outputs: out_color (3,H,W),
 * n_render / n_consider / n_contrib int32 (tiles), out_observe int32 (P).
 * The per-tile sorted lists (compact Gaussian indices) stay in `binning`
 * (gs_render_point_list turns them into the reference's point list and
 * keys), the ranges and per-pixel state in `img`, and a packed 64-byte copy
 * of each listed Gaussian's means2D / conic_opacity / rgb in `geom`, for
 * gs_render_backward.  The sorts of the longest lists run on a second stream
 * of the library's (one per device, default priority), forked from `stream`
 * and joined back to it with events: work queued on `stream` afterwards sees
 * every result.  clear_dst / clear_bytes: NULL / 0, or a caller buffer
 * (16-byte aligned, clear_bytes a multiple of 16) that the call fills with
 * zeros while its blend runs -- the blend is VALU-bound and leaves HBM
 * bandwidth unused -- e.g. the zero geometry maps the render returns when
 * render_geo is off.  No counterpart in the reference (it allocates those
 * outputs with torch::full(..., 0.0) before its forward). */
int gs_render_forward(int P, int64_t R, int image_width, int image_height, const float* bg,
                      const float* means2D, const float* depths, const int* radii,
                      const float* conic_opacity, const float* rgb, const uint8_t* compute_locally,
                      void* geom, void* binning, void* img, float* out_color, int32_t* n_render,
                      int32_t* n_consider, int32_t* n_contrib, int32_t* out_observe,
                      int region_side, void* clear_dst, int64_t clear_bytes, gs_stream_t stream);

/* The two calls above in one, without the host round trip between them: the
 * count, the duplication, the sorts and the blend are all queued at once
 * against a binning buffer of gs_render_binning_bytes(capacity) bytes, and
 * the call waits only for R (copied back as soon as the count is done, while
 * the rest still runs).  R is returned in *num_rendered.  If R > capacity the
 * duplication, sorts and blend did nothing useful: the caller sizes a binning
 * buffer for R and repeats the forward with gs_render_forward_count and
 * gs_render_forward.  Same outputs and workspaces as those two calls; the
 * forward of rasterize_points.cu:273-361, whose host reads R back
 * (rasterizer_impl.cu:621) before it can size and launch the duplication.
 * clear_dst / clear_bytes as gs_render_forward (cleared whether or not R
 * fits the capacity). */
int gs_render_forward_reserved(int P, int64_t capacity, int image_width, int image_height,
                               const float* bg, const float* means2D, const float* depths,
                               const int* radii, const float* conic_opacity, const float* rgb,
                               const uint8_t* compute_locally, void* geom, void* binning, void* img,
                               float* out_color, int32_t* n_render, int32_t* n_consider,
                               int32_t* n_contrib, int32_t* out_observe, int64_t* num_rendered,
                               int region_side, void* clear_dst, int64_t clear_bytes,
                               gs_stream_t stream);

/* Render backward.  Replaces RenderGaussiansBackwardCUDA
 * (diff-gaussian-rasterization_r/rasterize_points.cu:363-436; kernel
 * cuda_rasterizer/backward.cu:324-530).
 *   geom / binning / img: the forward's workspaces (geom also holds the
 *   gradient accumulators, cleared at the start of each call, so calls
 *   sharing one geom must not overlap).  means2D / conic_opacity / rgb: the forward's inputs
 *   (the kernels read the forward's packed copy of them in geom).
 *   dL_dpixels (3,H,W).  Outputs: dL_dmeans2D (row stride dL_dmeans2D_stride,
 *   2 or 3; the third column, when present, is zero), dL_dmeans2D_abs (P,3),
 *   dL_dconic_opacity (P,4) = [c00, c01, c11, opacity], dL_dcolors (P,3).
 *   clear_dst / clear_bytes: NULL / 0, or a caller buffer (16-byte aligned,
 *   clear_bytes a multiple of 16) that the call fills with zeros while its
 *   blend runs -- the blend is VALU-bound and leaves HBM bandwidth unused --
 *   e.g. the preprocess backward's dL_dsh, which that call then writes only
 *   at the visible rows (gs_preprocess_backward_rec's outputs_zeroed).  No
 *   counterpart in the reference (it allocates that output with
 *   torch::zeros before its preprocess backward). */
int gs_render_backward(int P, int64_t R, int image_width, int image_height, const float* bg,
                       const float* means2D, const float* conic_opacity, const float* rgb,
                       const uint8_t* compute_locally, void* geom, const void* binning, const void* img,
                       const float* dL_dpixels, float* dL_dmeans2D, int dL_dmeans2D_stride,
                       float* dL_dmeans2D_abs, float* dL_dconic_opacity, float* dL_dcolors,
                       void* clear_dst, int64_t clear_bytes, gs_stream_t stream);

/* Device addresses of a split render's per-Gaussian gradient accumulators
 * in its geom (64 bytes per listed Gaussian) and of the Gaussians'
 * accumulator rows (cidx_of: int per Gaussian, -1 when not listed; NULL when
 * R == 0), as gs_render_backward leaves them: the input of
 * gs_preprocess_backward_rec_acc.  No device work.  No counterpart in the
 * reference. */
int gs_render_accumulators(const void* geom, int P, int image_width, int image_height, int64_t R,
                           const void** acc, const int** cidx_of);

/* render_geo of the render forward (rasterize_points.cu:273-361 with
 * render_geo = true; kernel cuda_rasterizer/forward.cu:381-384,407-412):
 * the five geometry maps all_map (P,5) blended with the colour's weights
 * into out_all_map (5,H,W), and the plane depth out_plane_depth (H,W) =
 * map4 / -(map0 rx + map1 ry + map2 + 1e-8) with the pixel ray
 * (rx, ry) = ((x - W/2) / focal_x, (y - H/2) / focal_y), focal = W / (2 tan_fovx),
 * H / (2 tan_fovy).  Runs after a completed gs_render_forward or
 * gs_render_forward_reserved (same P, R, W, H, compute_locally and
 * workspaces), as a second walk of its lists: the colour outputs are
 * untouched.  Non-local tiles get zeros. */
int gs_render_geo_forward(int P, int64_t R, int image_width, int image_height, float tan_fovx,
                          float tan_fovy, const float* all_map, const uint8_t* compute_locally,
                          const void* geom, const void* binning, const void* img, float* out_all_map,
                          float* out_plane_depth, gs_stream_t stream);

/* gs_render_forward / gs_render_forward_reserved with render_geo = true
 * (RenderGaussiansCUDA, diff-gaussian-rasterization_r/rasterize_points.cu:
 * 273-361; kernel cuda_rasterizer/forward.cu:381-384,407-412): every output
 * of those calls, and in the same walk of the sorted lists the five
 * geometry maps out_all_map (5,H,W) -- all_map (P,5) blended with the
 * colour's weights -- and out_plane_depth (H,W) = all_map[4] /
 * -(n . ray + 1e-8), n = maps 0..2, ray = ((x - W/2) / fx, (y - H/2) / fy, 1),
 * fx = W / (2 tan_fovx), fy = H / (2 tan_fovy).  Non-local tiles get zeros. */
int gs_render_forward_geo(int P, int64_t R, int image_width, int image_height, const float* bg,
                          const float* means2D, const float* depths, const int* radii,
                          const float* conic_opacity, const float* rgb, const uint8_t* compute_locally,
                          void* geom, void* binning, void* img, float* out_color, int32_t* n_render,
                          int32_t* n_consider, int32_t* n_contrib, int32_t* out_observe, float tan_fovx,
                          float tan_fovy, const float* all_map, float* out_all_map, float* out_plane_depth,
                          int region_side, gs_stream_t stream);
int gs_render_forward_reserved_geo(int P, int64_t capacity, int image_width, int image_height,
                                   const float* bg, const float* means2D, const float* depths,
                                   const int* radii, const float* conic_opacity, const float* rgb,
                                   const uint8_t* compute_locally, void* geom, void* binning, void* img,
                                   float* out_color, int32_t* n_render, int32_t* n_consider,
                                   int32_t* n_contrib, int32_t* out_observe, int64_t* num_rendered,
                                   float tan_fovx, float tan_fovy, const float* all_map,
                                   float* out_all_map, float* out_plane_depth, int region_side,
                                   gs_stream_t stream);

/* gs_render_backward with render_geo = true (RenderGaussiansBackwardCUDA,
 * rasterize_points.cu:363-436; kernel backward.cu:393-405,427-432,476-490):
 * the maps enter dL/dalpha beside the colour.  all_map_pixels: the
 * forward's out_all_map; all_maps (P,5); dL_dout_all_map (5,H,W);
 * dL_dout_plane_depth (H,W).  Writes dL_dall_map (P,5) as well as every
 * output of gs_render_backward. */
int gs_render_backward_geo(int P, int64_t R, int image_width, int image_height, const float* bg,
                           float tan_fovx, float tan_fovy, const float* all_map_pixels,
                           const float* all_maps, const float* means2D, const float* conic_opacity,
                           const float* rgb, const uint8_t* compute_locally, void* geom,
                           const void* binning, const void* img, const float* dL_dpixels,
                           const float* dL_dout_all_map, const float* dL_dout_plane_depth,
                           float* dL_dmeans2D, int dL_dmeans2D_stride, float* dL_dmeans2D_abs,
                           float* dL_dconic_opacity, float* dL_dcolors, float* dL_dall_map,
                           void* clear_dst, int64_t clear_bytes, gs_stream_t stream);

/* Views into the opaque buffers, for tests and tools:
 *   binning: point_list uint32 (R), point_list_keys uint64 (R) -- written by
 *            gs_render_point_list, not by the forward
 *   img    : ranges uint32 (T,2), final_T float (H,W), n_contrib uint32 (H,W),
 *            n_contrib2loss uint32 (H,W)                                    */
int gs_render_buffer_views(int64_t R, int image_width, int image_height, void* binning, void* img,
                           uint32_t** point_list, uint64_t** point_list_keys, uint32_t** ranges,
                           float** final_T, uint32_t** n_contrib, uint32_t** n_contrib2loss);

/* The reference's sorted instance arrays (the point_list and
 * point_list_keys its binningBuffer holds after SortPairs,
 * diff-gaussian-rasterization_r/cuda_rasterizer/rasterizer_impl.cu:643-652),
 * written into `binning` on request: the forward itself keeps only the
 * blend's compact list, so these 12 bytes per instance are spent only by
 * callers that read them.  point_list[i] = Gaussian id, point_list_keys[i] =
 * (tile << 32) | bits of depths[id].  geom / binning / img: a completed
 * gs_render_forward or gs_render_full_forward (P, R, W, H as passed there);
 * depths: the depths the forward was given. */
int gs_render_point_list(int P, int64_t R, int image_width, int image_height, const float* depths,
                         const void* geom, void* binning, const void* img, gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * distCUDA2 (simple-knn/spatial.cu:15-26, simple_knn.cu:186-221):
 * out[i] = mean of the squared distances from points[i] to its 3 nearest
 * other points.  points (P,3), out (P).  Synchronises `stream`.
 * ------------------------------------------------------------------------ */
size_t gs_knn_workspace_bytes(int P);
int gs_knn_meandist3(int P, const float* points, float* out, void* workspace, gs_stream_t stream);

/* Allocation-free distCUDA2.  No counterpart in the reference: for callers
 * that cannot allocate device memory (tight serving loops, harnesses that
 * forbid hipMalloc).  Same result as gs_knn_meandist3, with the workspace in
 * a device array inside the library (about 38 MB, held on every GPU the
 * library runs on until the process ends) instead of a caller buffer;
 * allocates nothing.  Not for HIP graph capture: it reads the points'
 * bounding box back to the host mid-call and synchronises `stream`.
 * P <= 1048576 (larger P: error, use gs_knn_meandist3).  `stream` must belong
 * to the current device.  All calls on one GPU share that GPU's array; a
 * per-device lock held for the whole call (which returns after its kernels
 * finish) makes calls from several host threads run one after another. */
int gs_knn_meandist3_noalloc(int P, const float* points, float* out, gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * fused-ssim (fused-ssim/ssim.cu:367-441).  Images (B,C,H,W).
 * Forward writes ssim_map and, when the three dm_* pointers are non-null
 * (train=True), the partial derivatives dm/dmu1, dm/dsigma1^2, dm/dsigma12.
 * Backward writes dL_dimg1.
 * ------------------------------------------------------------------------ */
int gs_ssim_forward(int B, int C, int H, int W, float C1, float C2, const float* img1,
                    const float* img2, float* ssim_map, float* dm_dmu1, float* dm_dsigma1_sq,
                    float* dm_dsigma12, gs_stream_t stream);
int gs_ssim_backward(int B, int C, int H, int W, float C1, float C2, const float* img1,
                     const float* img2, const float* dL_dmap, const float* dm_dmu1,
                     const float* dm_dsigma1_sq, const float* dm_dsigma12, float* dL_dimg1,
                     gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Sparse Adam step.  gs_adam_update replaces the reference's adamUpdate
 * (diff-gaussian-rasterization_f/rasterize_points.cu:807-832, kernel
 * cuda_rasterizer/adam.cu:9-67): for every element p of a (N, M) parameter
 * whose Gaussian p / M has visible != 0,
 *   m = b1 m + (1 - b1) g,  v = b2 v + (1 - b2) g g,  param += -lr m / (sqrt(v) + eps);
 * other elements are left unchanged.  gs_adam_update_groups applies the step
 * to up to 8 parameter groups (SparseGaussianAdam.step's loop over
 * param_groups, diff_gaussian_rasterization_f/__init__.py:836-863) in one
 * launch.  All arrays are contiguous fp32; visible is one byte per Gaussian.
 * ------------------------------------------------------------------------ */
typedef struct gs_adam_group {
    float* param;
    const float* grad;
    float* exp_avg;
    float* exp_avg_sq;
    int64_t M;   /* elements per Gaussian */
    float lr;
    float eps;
} gs_adam_group;

int gs_adam_update(float* param, const float* param_grad, float* exp_avg, float* exp_avg_sq,
                   const uint8_t* visible, float lr, float b1, float b2, float eps, int64_t N,
                   int64_t M, gs_stream_t stream);
int gs_adam_update_groups(int n_groups, const gs_adam_group* groups, int64_t N,
                          const uint8_t* visible, float b1, float b2, gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Full-image path (GaussianRasterizer.forward / render_simp / markVisible of
 * diff-gaussian-rasterization_f).  Together these replace
 * RasterizeGaussiansCUDA (_f/rasterize_points.cu:370-475),
 * RasterizeGaussiansSimpCUDA (:477-583), RasterizeGaussiansBackwardCUDA
 * (:697-783) and markVisible (:785-805), i.e. Rasterizer::forward /
 * forward_simp / backward (_f/cuda_rasterizer/rasterizer_impl.cu:336-660,
 * 850-955) and their kernels (forward.cu:165-614, backward.cu:146-596,
 * rasterizer_impl.cu:56-253).
 *
 * gs_preprocess_forward_full: preprocessCUDA with the full path's inputs --
 *   culling (P) uint8 (nonzero = skip), colors_precomp (P,3) or NULL,
 *   cov3D_precomp (P,6) or NULL (then scales / rotations are used), SH as dc
 *   (P,1,3) + rest (P,M,3), M >= (D+1)^2 - 1 unless colours are given.
 *   Outputs as gs_preprocess_forward plus rects (P,2) float tile-rect extents
 *   and tiles_touched (P) uint32 rect tile counts (their sum is the reference's
 *   num_rendered).  prefiltered is not an input: near-culled points are
 *   skipped (the reference traps on them when prefiltered is set).
 * gs_render_full_count / gs_render_full_forward: binning with the float
 *   rects and the per-tile culling test of duplicateWithKeys, then the blend;
 *   *num_rendered is the number of instances that pass the test (the sizes of
 *   the workspaces; not the reference's num_rendered).  colors: the preprocess
 *   rgb or colors_precomp.  accum_max_count (P) float: per pixel, the Gaussian
 *   of the largest alpha * T gets +1 (NULL: flag_max_count off).  render_simp:
 *   accum_weights (P) float (sum of alpha * T) and accum_weights_count (P)
 *   int32 non-NULL.  All accumulators are zeroed by the call.
 * gs_render_full_backward: dL_dmeans2D (P,3), dL_dconic_opacity (P,4) =
 *   [c00, c01, c11, opacity] (16-byte aligned), dL_dcolors (P,3); conic and
 *   opacity gradients skip pixels where the alpha clamp is active.
 * gs_preprocess_backward_full: from those gradients, dL_dmeans3D (P,3),
 *   dL_dcov3D (P,6), dL_ddc (P,1,3), dL_drest (P,M,3), dL_dscales (P,3),
 *   dL_drotations (P,4), dL_dopacity (P,1); SH gradients only with SH colours
 *   and M > 0, scale / rotation gradients only without cov3D_precomp.
 * gs_render_full_depth: render_depth (RasterizeGaussiansDepthCUDA,
 *   _f/rasterize_points.cu:588-690; Rasterizer::forward_depth,
 *   rasterizer_impl.cu:671-847; render_depthCUDA, forward.cu:616-835): the
 *   same binning as gs_render_full_forward, then the blend with, per pixel,
 *   the camera ray's intersection with each blended Gaussian's 3-sigma
 *   ellipsoid (means3D (P,3), scales (P,3) activated, rotations (P,4)
 *   unnormalised, 16-byte aligned; projmatrix (4,4) and campos (3) device
 *   tensors as in the settings).  Outputs: out_color (3,H,W), out_pts (3,H,W)
 *   hit point, out_depth (1,H,W), accum_alpha (1,H,W) final T, gidx (1,H,W)
 *   int32 Gaussian id and discriminants (1,H,W), each from the Gaussian of
 *   the largest alpha * T (0 where none).  No backward.
 * gs_mark_visible: present (P) uint8 = view-space z > 0.2.
 * ------------------------------------------------------------------------ */
int gs_preprocess_forward_full(int P, int D, int M, const float* means3D, const float* scales,
                               const float* rotations, const float* dc, const float* rest,
                               const float* opacities, const float* colors_precomp,
                               const float* cov3D_precomp, const uint8_t* culling, float scale_modifier,
                               const float* viewmatrix, const float* projmatrix, const float* campos,
                               float tanfovx, float tanfovy, int image_height, int image_width,
                               float* means2D, float* depths, int* radii, float* cov3D,
                               float* conic_opacity, float* rgb, uint8_t* clamped, float* rects,
                               uint32_t* tiles_touched, gs_stream_t stream);
int gs_render_full_count(int P, int image_width, int image_height, const float* means2D, const int* radii,
                         const float* rects, const float* conic_opacity, void* geom,
                         int64_t* num_rendered, gs_stream_t stream);
int gs_render_full_forward(int P, int64_t R, int image_width, int image_height, const float* bg,
                           const float* means2D, const float* depths, const int* radii, const float* rects,
                           const float* conic_opacity, const float* colors, void* geom, void* binning,
                           void* img, float* out_color, float* accum_max_count, float* accum_weights,
                           int32_t* accum_weights_count, gs_stream_t stream);
/* gs_render_full_count + gs_render_full_forward in one call with a reserved
 * binning capacity, as gs_render_forward_reserved. */
int gs_render_full_forward_reserved(int P, int64_t capacity, int image_width, int image_height,
                                    const float* bg, const float* means2D, const float* depths,
                                    const int* radii, const float* rects, const float* conic_opacity,
                                    const float* colors, void* geom, void* binning, void* img,
                                    float* out_color, float* accum_max_count, float* accum_weights,
                                    int32_t* accum_weights_count, int64_t* num_rendered,
                                    gs_stream_t stream);
int gs_render_full_depth(int P, int64_t R, int image_width, int image_height, const float* bg,
                         const float* means2D, const float* depths, const int* radii, const float* rects,
                         const float* conic_opacity, const float* colors, const float* means3D,
                         const float* scales, const float* rotations, const float* projmatrix,
                         const float* campos, void* geom, void* binning, void* img, float* out_color,
                         float* out_pts, float* out_depth, float* accum_alpha, int32_t* gidx,
                         float* discriminants, gs_stream_t stream);
int gs_render_full_backward(int P, int64_t R, int image_width, int image_height, const float* bg,
                            const float* means2D, const float* conic_opacity, void* geom,
                            const void* binning, const void* img, const float* dL_dpixels,
                            float* dL_dmeans2D, float* dL_dconic_opacity, float* dL_dcolors,
                            gs_stream_t stream);
int gs_preprocess_backward_full(int P, int D, int M, const float* means3D, const float* scales,
                                const float* rotations, const float* dc, const float* rest,
                                const float* colors_precomp, const float* cov3D_precomp,
                                float scale_modifier, const float* viewmatrix, const float* projmatrix,
                                const float* campos, float tanfovx, float tanfovy, int image_height,
                                int image_width, const int* radii, const float* cov3D,
                                const uint8_t* clamped, const float* dL_dmeans2D,
                                const float* dL_dconic_opacity, const float* dL_dcolors,
                                float* dL_dmeans3D, float* dL_dcov3D, float* dL_ddc, float* dL_drest,
                                float* dL_dscales, float* dL_drotations, float* dL_dopacity,
                                gs_stream_t stream);
int gs_mark_visible(int P, const float* means3D, const float* viewmatrix, const float* projmatrix,
                    uint8_t* present, gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Gaussian -> rank routing of the image-distributed step.
 *
 * gs_local2j_ids_bool replaces GetLocal2jIdsBoolCUDA (mode GS_ROUTE_INTERVAL,
 * diff-gaussian-rasterization_f/rasterize_points.cu:258-289, kernel :212-256)
 * and GetLocal2jIdsBoolAdjustMode6CUDA (mode GS_ROUTE_RECT, :337-367, kernel
 * :291-335).  It writes every byte of the (P, world_size) bool matrix `out`
 * (1 = rank rk's tiles meet Gaussian i's rect).  table: GS_ROUTE_INTERVAL ->
 * world_size + 1 ascending tile indices (dist_global_strategy);
 * GS_ROUTE_RECT -> world_size rows of (y_l, y_r, x_l, x_r) tile bounds.
 * means2D (P, 2) fp32, radii (P) int32, table int32, all device memory.
 * Any world_size >= 1.
 *
 * gs_local2j_count + gs_local2j_write replace the bool matrix followed by one
 * nonzero() per rank (gaussian_renderer/workload_division.py:698-704, also
 * :161-167 and :460-468): count writes counts[rk] (int64 device array of
 * world_size + 1; counts[world_size] = total) and, if out_bool is non-null, the
 * bool matrix; after the caller has read the counts, write stores every rank's
 * ids (int64, ascending) into `ids`, concatenated rank after rank (rank rk's
 * list starts at counts[0] + ... + counts[rk-1]); n_ids = counts[world_size],
 * the size of `ids` (no id is stored at or past it).  world_size <= 64 and
 * P * world_size < 2^32.  workspace: gs_local2j_workspace_bytes(P, world_size)
 * bytes of device memory, passed unchanged from count to write.
 * ------------------------------------------------------------------------ */
#define GS_ROUTE_INTERVAL 0
#define GS_ROUTE_RECT 1

int gs_local2j_ids_bool(int mode, int P, int H, int W, int world_size, const float* means2D,
                        const int* radii, const int* table, int avoid_pixel_all2all, uint8_t* out,
                        gs_stream_t stream);
size_t gs_local2j_workspace_bytes(int P, int world_size);
int gs_local2j_count(int mode, int P, int H, int W, int world_size, const float* means2D,
                     const int* radii, const int* table, int avoid_pixel_all2all, uint8_t* out_bool,
                     int64_t* counts, void* workspace, gs_stream_t stream);
int gs_local2j_write(int mode, int P, int H, int W, int world_size, const float* means2D,
                     const int* radii, const int* table, int avoid_pixel_all2all,
                     const void* workspace, int64_t* ids, int64_t n_ids, gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Row mover for the screen-space exchange: replaces, in one launch each, the
 * torch.cat(fields, 1)[ids] pack per destination rank, the split + cat +
 * .contiguous() + radii .float()/.int() unpack of what was received
 * (gaussian_renderer/__init__.py:64-189) and the autograd backward of the
 * pack (index_put of gradient rows into zero-filled per-field gradients).
 * Output row r takes source row src_rows[r] (r if NULL; an entry outside
 * [0, n_src_rows) reads as zeros) and stores into destination row dst_rows[r]
 * (r if NULL; an entry outside [0, n_dst_rows) is skipped), for each
 * field: `width` elements at src + row*src_stride -> dst + row*dst_stride
 * (strides in elements).  Types convert as torch's .float() / .int() do.
 * accumulate != 0 adds into the destination (equal types only).  Up to 8
 * fields and 32 columns in all; rows named twice in dst_rows race.
 * ------------------------------------------------------------------------ */
#define GS_ROW_F32 0
#define GS_ROW_I32 1

typedef struct gs_row_field {
    const void* src;
    void* dst;
    int64_t src_stride;
    int64_t dst_stride;
    int32_t width;
    int32_t src_type;   /* GS_ROW_F32 or GS_ROW_I32 */
    int32_t dst_type;
} gs_row_field;

int gs_move_rows(int64_t n_rows, const int64_t* src_rows, int64_t n_src_rows, const int64_t* dst_rows,
                 int64_t n_dst_rows, int n_fields, const gs_row_field* fields, int accumulate,
                 gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * PLY vertex records <-> Gaussian parameter tensors.  Replaces the record
 * assembly of save_ply and the per-property reads of load_ply
 * (scene/gaussian_model.py:434-446 construct_list_of_attributes, :447-520
 * save_ply, :522-575 load_ply); the file bytes themselves are read and
 * written by the host (binary little-endian 'vertex' element).
 *   records: (P, rec_cols) float32 device array, one PLY vertex per row,
 *     16-byte aligned for the vectorised path.
 *   tensors: up to 8 row-major (P, width) device tensors, float32 or int8.
 *   colmap: HOST array, one entry per tensor column (tensors concatenated in
 *     the order given): the record column that tensor column is read from
 *     (unpack) or written to (pack).
 * gs_ply_unpack fills the tensors (int8 tensors take numpy's astype(int8)
 * of the float: truncation, low byte).  gs_ply_pack writes every record
 * column: the mapped ones from their tensor column (int8 as float), the
 * others as 0 (the zero normals); two tensor columns may not map to one
 * record column.  rec_cols <= 120, at most 120 tensor columns.
 * ------------------------------------------------------------------------ */
#define GS_PLY_F32 0
#define GS_PLY_I8 1

typedef struct gs_ply_tensor {
    void* ptr;
    int32_t width;
    int32_t type;   /* GS_PLY_F32 or GS_PLY_I8 */
} gs_ply_tensor;

int gs_ply_unpack(int64_t P, const float* records, int32_t rec_cols, int32_t n_tensors,
                  const gs_ply_tensor* tensors, const int32_t* colmap, gs_stream_t stream);
int gs_ply_pack(int64_t P, int32_t n_tensors, const gs_ply_tensor* tensors, const int32_t* colmap,
                int32_t rec_cols, float* records, gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Diagnostics (no counterpart in the reference): evaluate the device exp / log
 * used by the kernels on n inputs (op 0 = exp, 1 = log, 2 = the exact exp of
 * the blend's guard,
 * 3 = the 12-value wave reduction on 12 x 64 inputs), so tests can compare them
 * bit for bit with the CPU; op 6 evaluates the blend's falloff G = exp(x),
 * x <= 0 (hardware exp2, exact within a window around the 1/255 alpha
 * cut-off at opacity 1); op 4 copies n floats (n % 4 == 0, 16-byte aligned),
 * the known-size kernel that HBM byte counters are calibrated against; op 5
 * runs 8192 blocks of 256 threads, each wave issuing 32 * n fp32 FMAs (x unused,
 * y one float that is never written), the reference for the VALU issue rate;
 * ops 7, 8 and 9 run the forward / backward (8x8 quadrant walk) / backward
 * (16x8 half-tile walk, two pixels per lane) blend kernels' per-entry
 * arithmetic (the same device functions) n times over 64 entries staged in
 * LDS, in 16384 waves with no global memory traffic (x unused, y one float
 * that is never written): the VALU issue rate of the blend's own instruction
 * mix.
 * ------------------------------------------------------------------------ */
int gs_diag_math(int op, int n, const float* x, float* y, gs_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Per-kernel timing (the counterpart of the reference's MyTimerOnGPU,
 * diff-gaussian-rasterization_r/cuda_rasterizer/timers.cu:11-79).  on = 1:
 * every kernel launch is bracketed by HIP events on its stream, and so are
 * the stages; on = 2: only the stages (so that their wall times carry no
 * per-kernel event overhead); on = 0: off.  gs_timing_read synchronises on the recorded events and returns, per kernel
 * name (64-byte slots in `names`), the summed milliseconds and launch count;
 * the return value is the number of distinct kernels.  One entry is a stage,
 * not a kernel: "binning (wall)", the render's binning from its first kernel
 * (gs_render_forward_count / gs_render_full_count) to the end of the sorts
 * (gs_render_forward / _full_forward / _full_depth), on the caller's stream,
 * the R readback and the caller's work between the two calls included.
 * ------------------------------------------------------------------------ */
int gs_timing_enable(int on);
int gs_timing_reset(void);
int gs_timing_read(int max_entries, char* names, double* total_ms, int* counts);

#ifdef __cplusplus
}
#endif
#endif
