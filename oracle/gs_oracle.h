/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle (checker) for the HIP rasterizer.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product library never does.
 *
 * A plain-C fp32 restatement of the reference's differentiable Gaussian
 * rasterizer hot path (BlitzGS diff-gaussian-rasterization_f preprocess +
 * diff-gaussian-rasterization_r binning/render), simple-knn's distCUDA2 and
 * fused-ssim.  Each function cites the reference file:line it follows.
 * All arrays are host memory, row-major, fp32 unless stated.
 */
#ifndef GS_ORACLE_H
#define GS_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int W, H;              /* image width / height                          */
    float tanfovx, tanfovy;
    float scale_modifier;
    int sh_degree;         /* D                                              */
    float view[16];        /* viewmatrix, flat, as the reference tensors     */
    float proj[16];        /* full projection matrix, flat                   */
    float campos[3];
} o_camera;

/* Per-Gaussian preprocess forward (reference _f/cuda_rasterizer/forward.cu:164-284).
 * sh is (P, K, 3), K >= (D+1)^2.  All outputs are fully written (zeros for
 * culled Gaussians, except cov3D which is written once the near cull passes). */
void o_preprocess_fwd(int P, int K, const o_camera* cam,
                      const float* means3D, const float* scales, const float* rotations,
                      const float* sh, const float* opacities,
                      float* means2D, float* depths, int* radii, float* cov3D,
                      float* conic_opacity, float* rgb, uint8_t* clamped);

/* Per-Gaussian preprocess backward: computeCov2DCUDA + preprocessCUDA
 * (reference _f/cuda_rasterizer/backward.cu:146-400).  dL_dmeans2D has row
 * stride m2d_stride floats (2 or 3).  Outputs fully written. */
void o_preprocess_bwd(int P, int K, const o_camera* cam,
                      const float* means3D, const float* scales, const float* rotations,
                      const float* sh, const int* radii, const float* cov3D,
                      const uint8_t* clamped,
                      const float* dL_dmeans2D, int m2d_stride,
                      const float* dL_dconic_opacity, const float* dL_drgb,
                      float* dL_dmeans3D, float* dL_dscales, float* dL_drotations,
                      float* dL_dsh, float* dL_dopacity);

/* Reference tile-count rule (_r rasterizer_impl.cu:258-282): returns R. */
int64_t o_binning_count(int P, int W, int H, const float* means2D, const int* radii,
                        const uint8_t* compute_locally, uint32_t* tiles_touched);

/* Reference binning: inclusive scan, duplicateWithKeys, stable sort of the
 * 64-bit keys, identifyTileRanges (_r rasterizer_impl.cu:74-138,556-660).
 * keys/values: R entries; ranges: 2*T uint32 (start,end). */
void o_binning(int P, int W, int H, const float* means2D, const float* depths,
               const int* radii, const uint8_t* compute_locally,
               const uint32_t* tiles_touched, int64_t R,
               uint64_t* keys, uint32_t* values, uint32_t* ranges);

/* getHigherMsb (_r rasterizer_impl.cu:39-54). */
uint32_t o_higher_msb(uint32_t n);

/* Render forward (_r/cuda_rasterizer/forward.cu:263-413) plus the per-tile
 * statistics (_r rasterizer_impl.cu:213-256).  out_color (3,H,W) and the
 * per-pixel state are written for local tiles; non-local tiles get zeros. */
void o_render_fwd(int P, int W, int H, const float* bg,
                  const float* means2D, const float* conic_opacity, const float* rgb,
                  const uint8_t* compute_locally,
                  const uint32_t* ranges, const uint32_t* point_list,
                  float* out_color, float* final_T, uint32_t* n_contrib,
                  uint32_t* n_contrib2loss, int32_t* out_observe,
                  int32_t* n_render, int32_t* n_consider, int32_t* n_contrib_tile,
                  int32_t* obs_near, uint8_t* stop_near);

/* Decision margins of o_render_fwd (test infrastructure: they say which
 * integer outputs a blend whose exp differs from o_expf by a relative
 * O_EXP_REL may change).  Along each pixel's walk a first-order bound on the
 * relative error of T is carried: every blended entry adds
 * O_EXP_REL * alpha / (1 - alpha) (the factor (1 - alpha)'s error) plus two
 * fp32 roundings.  obs_near (P, or NULL): per Gaussian, the number of blends
 * whose T > 0.5 test had |T - 0.5| <= 0.5 * bound.  stop_near (H*W, or NULL):
 * 1 where some alpha-passing entry had |test_T - 1e-4| <= 1e-4 * bound. */
#define O_EXP_REL 4e-6f
void o_set_blend_margin_model(float exp_delta, float bound_rel);

/* Render backward (_r/cuda_rasterizer/backward.cu:324-530).  dL_dmean2D and
 * dL_dmean2D_abs are (P,3); dL_dconic is (P,4) in the reference's float4
 * slot layout (.x=c00, .y=c01, .w=c11); dL_dopacity (P); dL_dcolors (P,3).
 * Outputs are accumulated (caller zeroes them). */
void o_render_bwd(int P, int W, int H, const float* bg,
                  const float* means2D, const float* conic_opacity, const float* rgb,
                  const uint8_t* compute_locally,
                  const uint32_t* ranges, const uint32_t* point_list,
                  const float* final_T, const uint32_t* n_contrib,
                  const float* dL_dpixels,
                  float* dL_dmean2D, float* dL_dmean2D_abs, float* dL_dconic,
                  float* dL_dopacity, float* dL_dcolors);

/* render_geo of the _r render (NUM_ALL_MAP = 5 channels, config.h:24). */
#define O_NUM_MAPS 5

/* The forward's geometry maps (_r forward.cu:381-384,407-412), by a walk of
 * the same blend as o_render_fwd: out_all_map (5,H,W) = the all_map (P,5)
 * channels blended with the colour's weights alpha T; out_plane_depth (H,W) =
 * all_map[4] / -(n . ray + 1e-8), n = channels 0..2, ray = ((x - cx) / focal_x,
 * (y - cy) / focal_y, 1).  Non-local tiles: zeros. */
void o_render_geo_fwd(int W, int H, float focal_x, float focal_y, float cx, float cy,
                      const float* means2D, const float* conic_opacity, const float* all_map,
                      const uint8_t* compute_locally, const uint32_t* ranges, const uint32_t* point_list,
                      float* out_all_map, float* out_plane_depth);

/* The backward's render_geo inputs and output (_r backward.cu:335-347). */
typedef struct {
    float fx, fy;                  /* focal lengths W / (2 tan_fovx), H / (2 tan_fovy) */
    const float* all_maps;         /* (P,5) */
    const float* all_map_pixels;   /* (5,H,W): the forward's out_all_map */
    const float* dL_dmaps;         /* (5,H,W) */
    const float* dL_dplane;        /* (H,W) */
    float* dL_dall_map;            /* (P,5), accumulated */
} OGeoBwd;

/* o_render_bwd with render_geo on (_r backward.cu:393-405,427-432,476-490). */
void o_render_bwd_geo(int P, int W, int H, const float* bg,
                      const float* means2D, const float* conic_opacity, const float* rgb,
                      const uint8_t* compute_locally,
                      const uint32_t* ranges, const uint32_t* point_list,
                      const float* final_T, const uint32_t* n_contrib,
                      const float* dL_dpixels,
                      float* dL_dmean2D, float* dL_dmean2D_abs, float* dL_dconic,
                      float* dL_dopacity, float* dL_dcolors, const OGeoBwd* geo);

/* ---- full-image path (_f GaussianRasterizer.forward / render_simp) ---- */

/* preprocessCUDA with the full path's arguments (_f forward.cu:165-284,
 * rasterizer_impl.cu:396-424): culling mask (nonzero = skip), precomputed
 * colours / 3D covariances (NULL = compute), SH as dc (P,1,3) + rest
 * (P,M,3); also writes the float tile-rect extents rects (P,2) and the rect
 * tile counts tiles_touched (P). */
void o_preprocess_fwd_full(int P, int M, const o_camera* cam,
                           const float* means3D, const float* scales, const float* rotations,
                           const float* dc, const float* rest, const float* opacities,
                           const float* colors_precomp, const float* cov3D_precomp, const uint8_t* culling,
                           float* means2D, float* depths, int* radii, float* cov3D,
                           float* conic_opacity, float* rgb, uint8_t* clamped,
                           float* rects, uint32_t* tiles_touched);

/* BACKWARD::preprocess with the full path's arguments (_f backward.cu:759-827,
 * rasterizer_impl.cu:931-954).  dL_dmeans2D (P,3), dL_dconic (P,4) float4
 * slots (.x=c00, .y=c01, .w=c11), dL_dcolors (P,3).  Outputs fully written. */
void o_preprocess_bwd_full(int P, int M, const o_camera* cam,
                           const float* means3D, const float* scales, const float* rotations,
                           const float* dc, const float* rest, const float* colors_precomp,
                           const float* cov3D_precomp, const int* radii, const float* cov3D,
                           const uint8_t* clamped, const float* dL_dmeans2D, const float* dL_dconic,
                           const float* dL_dcolors,
                           float* dL_dmeans3D, float* dL_dcov3D, float* dL_ddc, float* dL_drest,
                           float* dL_dscales, float* dL_drotations);

/* The tile-culling test of the full path's duplicateWithKeys
 * (rasterizer_impl.cu:56-95,144-167); 1 = keep tile (tx, ty). */
int o_full_tile_keep(const float* xy, const float* co, unsigned tx, unsigned ty);

/* Binning of the full path (rasterizer_impl.cu:119-210,440-480).  R = sum of
 * tiles_touched; keys/values hold R entries (culled slots padded with the
 * invalid key, sorted last).  Returns the valid instances; *num_buckets =
 * sum of ceil(tile length / 32). */
int64_t o_binning_full(int P, int W, int H, const float* means2D, const float* depths, const int* radii,
                       const float* rects, const float* conic_opacity, const uint32_t* tiles_touched,
                       int64_t R, uint64_t* keys, uint32_t* values, uint32_t* ranges, int64_t* num_buckets);

/* renderCUDA / render_simpCUDA of the full path (forward.cu:291-607).
 * accum_weights / accum_weights_count NULL for renderCUDA.  Accumulators
 * are added to (caller zeroes them). */
void o_inv4_colmajor(const float* m, float* out);
void o_render_depth_full(int W, int H, const float* bg, const float* means2D, const float* conic_opacity,
                         const float* colors, const uint32_t* ranges, const uint32_t* point_list,
                         const float* means3D, const float* scales, const float* rotations, const float* projmatrix,
                         const float* campos, float* out_color, float* out_pts, float* out_depth, float* accum_alpha,
                         int32_t* gidx, float* discriminants);
void o_render_fwd_full(int P, int W, int H, const float* bg, const float* means2D, const float* conic_opacity,
                       const float* colors, const uint32_t* ranges, const uint32_t* point_list, int flag_max_count,
                       float* out_color, float* final_T, uint32_t* n_contrib, uint32_t* max_contrib,
                       float* accum_max_count, float* accum_weights, int32_t* accum_weights_count);

/* Render backward of the full path: the split path's per-pixel gradients
 * with PerGaussianRenderCUDA's rule (_f backward.cu:403-588): no
 * |dL/dmean2D|, no conic / opacity gradient where opacity * G > 0.99.
 * dL_dmean2D (P,3), dL_dconic (P,4) float4 slots, dL_dopacity (P),
 * dL_dcolors (P,3); accumulated (caller zeroes them). */
void o_render_bwd_full(int P, int W, int H, const float* bg,
                       const float* means2D, const float* conic_opacity, const float* colors,
                       const uint32_t* ranges, const uint32_t* point_list,
                       const float* final_T, const uint32_t* n_contrib,
                       const float* dL_dpixels,
                       float* dL_dmean2D, float* dL_dconic, float* dL_dopacity, float* dL_dcolors);

/* distCUDA2 (simple-knn simple_knn.cu:148-221): mean of the three smallest
 * squared distances to other points.  Exact; O(P log P) grid search. */
void o_knn_meandist3(int P, const float* points, float* out);

/* fused-ssim forward / backward (fused-ssim ssim.cu:186-365).  img (B,C,H,W). */
void o_ssim_fwd(int B, int C, int H, int W, float C1, float C2,
                const float* img1, const float* img2, float* ssim_map,
                float* dm_dmu1, float* dm_dsigma1_sq, float* dm_dsigma12);
void o_ssim_bwd(int B, int C, int H, int W, float C1, float C2,
                const float* img1, const float* img2, const float* dL_dmap,
                const float* dm_dmu1, const float* dm_dsigma1_sq, const float* dm_dsigma12,
                float* dL_dimg1);

void o_ssim_window(float* w);

/* Scalar math used by the oracle, exported so tests can pin it. */
/* sparse Adam step over a (N, M) parameter (adam.cu:9-38) */
void o_adam_update(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, const uint8_t* visible,
                   float lr, float b1, float b2, float eps, int64_t N, int64_t M);

/* Gaussian -> rank routing, (P, world) bool rows (rasterize_points.cu:212-289):
 * rank rk gets Gaussian i when the linear tile-index span of its rect meets
 * [strategy[rk], strategy[rk+1]) (widened by one tile row + 1 when avoid). */
void o_local2j_ids_bool(int P, int H, int W, int world, const float* means2D, const int* radii,
                        const int* strategy, int avoid, uint8_t* out);
/* Same with one tile rectangle (y_l, y_r, x_l, x_r) per rank (rasterize_points.cu:291-367). */
void o_local2j_ids_bool_rect(int P, int H, int W, int world, const float* means2D, const int* radii,
                             const int* rectangles, int avoid, uint8_t* out);

void o_vec_expf(int n, const float* x, float* y);
void o_vec_logf(int n, const float* x, float* y);

int o_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
