/*
 * gsx_oracle.h -- CPU restatement of mlx3D's tile-based Gaussian-splatting
 * rasterizer, used ONLY as test infrastructure (the checker in tests/, the
 * cpu_baseline leg of bench.py and __graft_entry__.smoke()).  Nothing in the
 * product package links, loads or calls this code.
 *
 * Every function restates one piece of the reference (paths relative to the
 * reference repository root):
 *   orc_expf            -- own exp (Cody-Waite reduction + degree-7 Taylor)
 *                          for the activations of model.py:116-122
 *   orc_splat_expf,     -- the compositing loops' exp and power (metal::exp
 *   orc_splat_power        and the power of rasterize.py:77-80,169-171)
 *   orc_project         -- src/mlx3d/splatting/projection.py:24-146
 *   orc_eval_sh         -- src/mlx3d/splatting/sh.py:41-78
 *   orc_preprocess_fwd  -- render.py:73-80 + projection + model.py:116-126
 *   orc_bin             -- src/mlx3d/splatting/tiles.py:19-182 (refine_tiles
 *                          when conics are given)
 *   orc_raster_fwd      -- rasterize.py:28-98 (+ depth rasterize.py:223-290)
 *   orc_raster_bwd      -- rasterize.py:100-221, vjp wiring :364-403
 *   orc_project_ut      -- projection.py:149-205 + cameras.py:42-77, 290-311
 *                          (ut_oracle.c; orc_preprocess_* under ORC_PROJECT_UT)
 *   orc_mesh_raster     -- renderer/rasterizer.py:29-87 (mesh_oracle.c)
 *   orc_photometric, orc_adam, orc_accum_screen_grads -- train_oracle.c
 *   orc_project_bwd /
 *   orc_preprocess_bwd  -- hand-derived VJP of projection.py:56-138,
 *                          sh.py:52-78, render.py:75-80, model.py:116-122
 *                          (what MLX autodiff computes for the reference)
 *
 * Arithmetic is IEEE float32 in the reference's operation order, compiled
 * with -ffp-contract=off so no multiply-add is fused behind our back; the
 * explicit fmaf calls (the compositing power and accumulation) are the
 * contractions a fast-math compiler applies to the reference's expressions.
 *
 * The camera struct has the same layout as gsx_camera in include/gsx.h.
 */
#ifndef GSX_ORACLE_H
#define GSX_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_camera {
    float R[9];
    float t[3];
    float center[3];
    float fx, fy, cx, cy;
    float lim_x, lim_y;
    float znear;
    int32_t width, height;
    int32_t orthographic;   /* UT projection only (cameras.py:158-160)   */
    int32_t lens;           /* ORC_LENS_*                                 */
    float dist[8];          /* Brown: k1 k2 p1 p2 k3 2p1 2p2; fisheye k1..k4 */
} orc_camera;

enum {
    ORC_LOG_SCALES = 1,     /* scales given as log-sigma: apply exp      */
    ORC_LOGIT_OPACITY = 2,  /* opacities given as logits: apply sigmoid  */
    ORC_ANTIALIAS = 4,      /* Mip-Splatting compensation (blur > 0)     */
    ORC_PROJECT_UT = 8      /* unscented-transform projection            */
};

enum { ORC_LENS_NONE = 0, ORC_LENS_BROWN = 1, ORC_LENS_FISHEYE = 2 };

float orc_expf(float x);
void orc_expf_array(int64_t n, const float* x, float* y);
float orc_splat_expf(float x);
void orc_splat_expf_array(int64_t n, const float* x, float* y);
float orc_splat_power(float a, float b, float c, float dx, float dy);

void orc_project(const orc_camera* cam, int64_t n, const float* means,
                 const float* quats, const float* scales, float blur,
                 int antialias, float* means2d, float* conics, float* depths,
                 float* radii, float* comp, int nthreads);

void orc_project_bwd(const orc_camera* cam, int64_t n, const float* means,
                     const float* quats, const float* scales, float blur,
                     int antialias, const float* g_means2d,
                     const float* g_conics, const float* g_depths,
                     const float* g_comp, float* g_means, float* g_quats,
                     float* g_scales, int nthreads);

void orc_eval_sh(int64_t n, int K, int C, int degree, const float* sh,
                 const float* dirs, float* out, int nthreads);

void orc_eval_sh_bwd(int64_t n, int K, int C, int degree, const float* sh,
                     const float* dirs, const float* g_out, float* g_sh,
                     float* g_dirs, int nthreads);

/* sh == NULL selects colors mode: colors are used as given (no clamp). */
void orc_preprocess_fwd(const orc_camera* cam, int64_t n, const float* means,
                        const float* quats, const float* scales,
                        const float* opacities, const float* sh, int K,
                        int degree, uint32_t flags, float blur,
                        float* means2d, float* conics, float* depths,
                        float* radii, float* comp, float* opac_eff,
                        float* colors_out, int nthreads);

void orc_preprocess_bwd(const orc_camera* cam, int64_t n, const float* means,
                        const float* quats, const float* scales,
                        const float* opacities, const float* colors_out,
                        int K, int degree, uint32_t flags, float blur,
                        const float* g_means2d, const float* g_conics,
                        const float* g_opac_eff, const float* g_colors,
                        const float* g_depths, const float* g_comp,
                        float* g_means, float* g_quats, float* g_scales,
                        float* g_opacities, float* g_sh, int nthreads);

/* Returns D (number of duplicates).  Writes sorted_ids only if D <= cap.
 * tile_ranges (tiles_x*tiles_y, 2) is always written. */
int64_t orc_bin(int64_t n, const float* means2d, const float* radii,
                const float* depths, const float* conics, int64_t conic_stride,
                int width, int height, int32_t* sorted_ids, int64_t cap,
                int32_t* tile_ranges, int nthreads);

/* tiles == NULL renders every tile; else only the listed tile ids (outputs
 * of other tiles are left untouched). */
void orc_raster_fwd(int64_t n, int C, const float* means2d,
                    const float* conics, const float* opacities,
                    const float* feats, const float* depths,
                    const int32_t* sorted_ids, const int32_t* tile_ranges,
                    const float* bg, int width, int height, float* out,
                    float* final_T, int32_t* n_contrib, float* depth_out,
                    const int32_t* tiles, int64_t n_tiles, int nthreads);

/* orc_raster_fwd with the arithmetic chosen by `arith` (0: as orc_raster_fwd;
 * bits below: the reference's literal expressions, for measuring how many
 * decisions the shipped arithmetic changes).  Not a parity target. */
#define ORC_ARITH_LITERAL_POWER 1 /* rasterize.py:75-76 unfactored, op by op */
#define ORC_ARITH_SEPARATE_ACC 2  /* rasterize.py:84 multiply then add */
#define ORC_ARITH_ROUNDED_EXP 4   /* float32 rounding of the double exp */
float orc_literal_power(float a, float b, float c, float dx, float dy);
void orc_raster_fwd_arith(int64_t n, int C, const float* means2d,
                          const float* conics, const float* opacities,
                          const float* feats, const float* depths,
                          const int32_t* sorted_ids, const int32_t* tile_ranges,
                          const float* bg, int width, int height, float* out,
                          float* final_T, int32_t* n_contrib, float* depth_out,
                          const int32_t* tiles, int64_t n_tiles, int nthreads, int arith);

void orc_raster_bwd(int64_t n, int C, const float* means2d,
                    const float* conics, const float* opacities,
                    const float* feats, const int32_t* sorted_ids,
                    const int32_t* tile_ranges, const float* bg, int width,
                    int height, const float* final_T,
                    const int32_t* n_contrib, const float* grad_out,
                    const float* grad_final_T, float* g_means2d,
                    float* g_conics, float* g_feats, float* g_opac,
                    int nthreads);

/* ------------------------------------------------ UT projection (ut_oracle.c) */

float orc_atanf(float r);  /* r >= 0 */

void orc_project_ut(const orc_camera* cam, int64_t n, const float* means, const float* quats,
                    const float* scales, float blur, int antialias, float* means2d,
                    float* conics, float* depths, float* radii, float* comp, int nthreads);

void orc_project_ut_bwd(const orc_camera* cam, int64_t n, const float* means,
                        const float* quats, const float* scales, float blur, int antialias,
                        const float* g_means2d, const float* g_conics, const float* g_depths,
                        const float* g_comp, float* g_means, float* g_quats, float* g_scales,
                        int nthreads);

/* One Gaussian (used by orc_preprocess_* under ORC_PROJECT_UT):
 * out = {u, v, A, B, C, z, radius, comp};
 * g_in = cotangents {u, v, A, B, C, z, comp}. */
void orc_ut_project_one(const orc_camera* cam, const float* m, const float* q, const float* s,
                        float blur, int aa, float* out);
void orc_ut_project_vjp_one(const orc_camera* cam, const float* m, const float* q,
                            const float* s, float blur, int aa, const float* g_in, float* g_m,
                            float* g_q, float* g_s);

/* -------------------------------------------------- mesh raster (mesh_oracle.c) */

/* renderer/rasterizer.py:29-87: nearest face per pixel over its tile's
 * list; tri_xy (F,6), tri_z (F,3); pix_to_face (H*W) (-1 empty), zbuf. */
void orc_mesh_raster(int64_t n_faces, const float* tri_xy, const float* tri_z,
                     const int32_t* sorted_ids, const int32_t* tile_ranges, int width,
                     int height, float znear, int32_t* pix_to_face, float* zbuf,
                     int nthreads);

/* ------------------------------------------------ training step (train_oracle.c) */

/* Mean L1 and mean SSIM of pred vs target (H,W,C), double precision, direct
 * 2D window; out[2] = {mean L1, mean SSIM}.  grad (H,W,C) or NULL receives
 * g_l1 d(mean L1)/dpred + g_ssim d(mean SSIM)/dpred. */
void orc_photometric(int H, int W, int C, const float* pred, const float* target, int window,
                     double sigma, double max_val, double g_l1, double g_ssim, double* out,
                     double* grad);

/* One Adam update in place (mlx.optimizers.Adam, bias_correction off). */
void orc_adam(int64_t n, float* p, const float* g, float* m, float* v, float lr, float b1,
              float b2, float eps);

/* Density-control statistics of trainer.py:357-365, in place. */
void orc_accum_screen_grads(int64_t n, const float* g, const float* radii, int W, int H,
                            float* accum, float* count);

#ifdef __cplusplus
}
#endif
#endif
