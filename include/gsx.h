/*
 * gsx.h -- C ABI of the MI355X (gfx950) Gaussian-splatting rasterizer.
 *
 * This is the drop-in boundary for mlx3D's tile-based 3DGS path.  The
 * reference (amirhossein-razlighi/mlx3D v0.2.0, paths under src/mlx3d/) is
 * pure Python on MLX; its device boundary is the set of mx.fast.metal_kernel
 * launches and MLX-op pipelines listed beside each entry point below.  The
 * Python package mlx3d_amd binds these symbols with ctypes (see
 * mlx3d_amd/_lib.py) behind the reference's own function names.
 *
 * Conventions
 *  - Every pointer is device memory (hipMalloc/torch CUDA tensors) unless
 *    documented otherwise, contiguous, float32 or int32/uint32 as named.
 *  - The caller owns all buffers; no entry point allocates device memory.
 *    Scratch space comes in through an explicit workspace argument (the one
 *    exception, gsx_l1_fwd_noalloc, uses a fixed file-scope device array).
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = default stream).
 *    Only gsx_bin_sort synchronises the stream (one 8-byte readback of the
 *    duplicate count, as the reference does at tiles.py:68);
 *    gsx_bin_sort_async leaves that count on the device so the caller can
 *    enqueue the rasterizer first and read it afterwards.
 *  - Return value: GSX_OK (0) on success, > 0 = required capacity (retry
 *    with a larger buffer), < 0 = error code (gsx_strerror).
 *  - No C++ exception crosses the ABI.  Entry points are reentrant; calls
 *    on different streams may run concurrently, with one exception:
 *    gsx_l1_fwd_noalloc shares one scratch array per GPU, so the caller
 *    must order its calls on one GPU (overlapping calls race).
 */
#ifndef GSX_H
#define GSX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GSX_ABI_VERSION 7
#define GSX_TILE_SIZE 16 /* tiles.py:14 */

enum gsx_status {
    GSX_OK = 0,
    GSX_ERR_INVALID = -1,     /* bad size / null pointer / unsupported shape */
    GSX_ERR_HIP = -2,         /* a HIP runtime call failed                   */
    GSX_ERR_WORKSPACE = -3,   /* workspace smaller than gsx_*_workspace_bytes */
    GSX_ERR_TOO_LARGE = -4,   /* a count exceeds the supported index range   */
    GSX_ERR_DEVICE = -5       /* a device-side check failed (bounded wait)    */
};

/* Error bits of the device status word written by gsx_bin_sort_async. */
enum gsx_bin_error {
    GSX_BIN_ERR_LOOKBACK = 1, /* a chained-scan wait exceeded its bound       */
    GSX_BIN_ERR_OVERFLOW = 2  /* the duplicate count exceeds 2^30 - 1         */
};

/* Flags of gsx_preprocess_fwd/bwd. */
enum gsx_flags {
    GSX_LOG_SCALES = 1,     /* scales are log-sigma: exp applied (model.py:116-118)  */
    GSX_LOGIT_OPACITY = 2,  /* opacities are logits: sigmoid (model.py:120-122)      */
    GSX_ANTIALIAS = 4,      /* Mip-Splatting compensation (projection.py:125-129)    */
    GSX_PROJECT_UT = 8      /* unscented-transform projection (projection.py:149-205)
                               instead of EWA                                       */
};

/* Lens model of a gsx_camera (cameras.py:154-172). */
enum gsx_lens {
    GSX_LENS_NONE = 0,
    GSX_LENS_BROWN = 1,     /* Brown-Conrady k1 k2 p1 p2 [k3] (cameras.py:42-51)      */
    GSX_LENS_FISHEYE = 2    /* OpenCV equidistant k1..k4 (cameras.py:69-77)           */
};

/* Pinhole camera, OpenCV convention, X_cam = R X_world + t
 * (cameras/cameras.py:139-173).  All values are the float32 numbers the
 * reference's float32 arithmetic sees: fx..cy rounded from the Python
 * floats, lim_x/lim_y = float32(1.3 * 0.5 * width / fx) computed in double
 * (projection.py:70-73), center = -(R^T t) (cameras.py:270-273). */
typedef struct gsx_camera {
    float R[9];
    float t[3];
    float center[3];
    float fx, fy, cx, cy;
    float lim_x, lim_y;
    float znear;
    int32_t width, height;
    /* Lens model, used by the UT projection only (the EWA projection is a
     * pinhole model, as in the reference; cameras.py:290-325).
     * orthographic != 0: u = fx x_cam + cx, v = fy y_cam + cy.
     * lens = GSX_LENS_BROWN: dist = {k1, k2, p1, p2, k3, 2 p1, 2 p2} (the
     * doubled constants formed in double and rounded once, as the
     * reference's Python scalars reach its float32 arithmetic);
     * GSX_LENS_FISHEYE: dist = {k1, k2, k3, k4}; unused entries zero. */
    int32_t orthographic;
    int32_t lens;
    float dist[8];
} gsx_camera;

const char* gsx_strerror(int status);
int gsx_abi_version(void);
/* Name of the GPU the library runs on and whether its code object matches. */
int gsx_device_check(char* name_out, int name_len);

/* ---------------------------------------------------------- projection --
 * Replaces project_gaussians (splatting/projection.py:24-146): EWA
 * projection to means2d (N,2), conics (N,3), depths (N), radii (N, float
 * holding integers), compensation (N). */
int gsx_project_fwd(const gsx_camera* cam, int64_t n, const float* means,
                    const float* quats, const float* scales, float blur,
                    int32_t antialias, float* means2d, float* conics,
                    float* depths, float* radii, float* compensation,
                    void* stream);

/* VJP of project_gaussians (what MLX autodiff computes through
 * projection.py:56-138).  Any cotangent may be NULL (= zero). */
int gsx_project_bwd(const gsx_camera* cam, int64_t n, const float* means,
                    const float* quats, const float* scales, float blur,
                    int32_t antialias, const float* g_means2d,
                    const float* g_conics, const float* g_depths,
                    const float* g_compensation, float* g_means,
                    float* g_quats, float* g_scales, void* stream);

/* Replaces project_gaussians_ut (splatting/projection.py:149-205): six
 * sigma points mean +- sqrt(3) R diag(s) e_k through the camera's
 * project_points (cameras.py:290-311: perspective or orthographic, with
 * Brown-Conrady or fisheye distortion), their mean and covariance, then the
 * EWA path's blur, conic, compensation, radius and validity; depths are the
 * centres' camera z.  Same arguments and outputs as gsx_project_fwd. */
int gsx_project_ut_fwd(const gsx_camera* cam, int64_t n, const float* means,
                       const float* quats, const float* scales, float blur,
                       int32_t antialias, float* means2d, float* conics,
                       float* depths, float* radii, float* compensation,
                       void* stream);

/* VJP of project_gaussians_ut (what MLX autodiff computes through
 * projection.py:149-205 and cameras.py:42-77, 290-311).  Any cotangent may
 * be NULL (= zero). */
int gsx_project_ut_bwd(const gsx_camera* cam, int64_t n, const float* means,
                       const float* quats, const float* scales, float blur,
                       int32_t antialias, const float* g_means2d,
                       const float* g_conics, const float* g_depths,
                       const float* g_compensation, float* g_means,
                       float* g_quats, float* g_scales, void* stream);

/* ------------------------------------------------------------------ SH --
 * Replaces eval_sh (splatting/sh.py:41-78): sh (N,K,C), dirs (N,3) ->
 * out (N,C) = sum_k basis_k(dir) sh[:,k] + 0.5, degree 0..3. */
int gsx_eval_sh_fwd(int64_t n, int32_t K, int32_t C, int32_t degree,
                    const float* sh, const float* dirs, float* out,
                    void* stream);
/* VJP of eval_sh: g_sh (N,K,C) fully written; g_dirs (N,3) may be NULL. */
int gsx_eval_sh_bwd(int64_t n, int32_t K, int32_t C, int32_t degree,
                    const float* sh, const float* dirs, const float* g_out,
                    float* g_sh, float* g_dirs, void* stream);

/* --------------------------------------------------- fused preprocess --
 * One pass per Gaussian replacing GaussianModel.render's activations
 * (model.py:116-126), project_gaussians, render_gaussians' opacity
 * compensation, view directions and SH colour (render.py:73-80), and the
 * per-Gaussian half of bin_gaussians (tiles.py:54-65).
 *
 * SH coefficients are read as coefficient 0 from sh0 (float3 per Gaussian,
 * stride sh0_stride floats) and coefficients 1..K-1 from sh_rest (stride
 * sh_rest_stride floats), so both a packed (N,K,3) tensor and the model's
 * separate sh_dc (N,1,3) / sh_rest (N,K-1,3) tensors are read in place.
 * sh0 == NULL selects colours mode: no colour is computed here (the
 * caller's own (N,C) colours or features go to gsx_raster_fwd) and
 * colors_out may be NULL.
 *
 * Outputs: means2d (N,2), depths (N), radii (N), compensation (N),
 * conic_opacity (N,4) = (conic a, b, c, opacity*compensation),
 * colors_out (N,3) (SH mode only), and for binning tile_counts (N),
 * depth_keys (N) and tile_rects (N,2) (packed xmin|ymin<<16, w|h<<16).
 * depth_keys order the binned Gaussians by depth: the orderable bits of z
 * minus those of the camera's znear (binned Gaussians have z > znear), so
 * the depth sort's top 2-bit pass is skipped for every z below about 2^30
 * float32 ulps past znear; Gaussians with a zero tile count get key 0 and
 * rectangle (0, 0). */
int gsx_preprocess_fwd(const gsx_camera* cam, int64_t n, const float* means,
                       const float* quats, const float* scales,
                       const float* opacities, const float* sh0,
                       int64_t sh0_stride, const float* sh_rest,
                       int64_t sh_rest_stride, int32_t K, int32_t degree,
                       uint32_t flags, float blur, float* means2d,
                       float* depths, float* radii, float* compensation,
                       float* conic_opacity, float* colors_out,
                       uint32_t* tile_counts, uint32_t* depth_keys,
                       uint32_t* tile_rects, void* stream);

/* VJP of gsx_preprocess_fwd (MLX autodiff of the same expressions,
 * render.py:75-80 with dirs under stop_gradient, colour clamp mask from
 * colors_out).  g_means2d/g_conics/g_opac_eff/g_colors come from
 * gsx_raster_bwd: four arrays with grad_stride = 0, or with grad_stride > 0
 * its gradient record (g_means2d points at it, the other three are NULL;
 * grad_stride a multiple of 4, at least 12 with SH, 8 without);
 * g_means2d_extra, g_depths, g_compensation are extra cotangents of the
 * returned means2d/depths/compensation and may be NULL.  g_sh0/g_sh_rest
 * use the strides of the forward; coefficients >= (degree+1)^2 are written
 * as zero. */
int gsx_preprocess_bwd(const gsx_camera* cam, int64_t n, const float* means,
                       const float* quats, const float* scales,
                       const float* opacities, const float* colors_out,
                       int32_t K, int32_t degree, uint32_t flags, float blur,
                       const float* g_means2d, const float* g_conics,
                       const float* g_opac_eff, const float* g_colors,
                       const float* g_means2d_extra, const float* g_depths,
                       const float* g_compensation, float* g_means,
                       float* g_quats, float* g_scales, float* g_opacities,
                       float* g_sh0, int64_t sh0_stride, float* g_sh_rest,
                       int64_t sh_rest_stride, int32_t grad_stride, void* stream);

/* ------------------------------------------------------------- binning --
 * Replaces bin_gaussians (splatting/tiles.py:19-182, refine_tiles off).
 *
 * gsx_bin_prepare: tiles.py:54-65 for externally supplied means2d (N,2),
 * radii (N), depths (N) -> tile_counts, depth_keys (the orderable bits of
 * any float depth; 0 for Gaussians with a zero count), tile_rects. */
int gsx_bin_prepare(int64_t n, const float* means2d, const float* radii,
                    const float* depths, int32_t width, int32_t height,
                    uint32_t* tile_counts, uint32_t* depth_keys,
                    uint32_t* tile_rects, void* stream);

/* Bytes of workspace gsx_bin_sort(_async) needs for n Gaussians,
 * `capacity` duplicates and num_tiles tiles. */
int64_t gsx_bin_workspace_bytes(int64_t n, int64_t capacity, int32_t num_tiles);

/* tiles.py:67-182: depth-sort, duplicate per tile, sort by tile, ranges.
 * Order within a tile is (depth ascending, Gaussian index ascending) --
 * the order of key = tile*N + rank(depth) with a stable argsort.  Writes
 * sorted_ids (D) int32 and tile_ranges (num_tiles,2) int32 [start,end),
 * (0,0) for empty tiles.  With conics != NULL (N rows of conic_stride >= 3
 * floats, a b c first; means2d (N,2) required) a duplicate is kept only if
 * the conic quadratic's minimum over the tile rectangle is <= 12
 * (refine_tiles, tiles.py:91-164).  Synchronises `stream` once to read D
 * into *num_dups.  Returns 1 if the duplicates exceed capacity (then
 * *num_dups is the capacity needed; retry with at least that).  n and
 * capacity < 2^30; sorted_ids must be 16-byte aligned.  tile_rects of
 * Gaussians with a zero tile count must be (0, 0) (as gsx_bin_prepare and
 * gsx_preprocess_fwd write them).
 *
 * Up to 256 x 256 tiles without refine_tiles the duplicates are placed
 * without a sort over them: Gaussians go into per-row lists by a stable
 * radix pass over their rows, and each row's duplicates are ranked by
 * column within 4096-duplicate segments whose per-column offsets a scan
 * over the row has fixed.  Larger images and refine_tiles run the general
 * path: emission of (tile, id) pairs and a stable radix sort of the tile
 * ids. */
int gsx_bin_sort(int64_t n, const uint32_t* tile_counts,
                 const uint32_t* depth_keys, const uint32_t* tile_rects,
                 const float* means2d, const float* conics, int64_t conic_stride,
                 int32_t width, int32_t height, void* workspace,
                 int64_t workspace_bytes, int64_t capacity,
                 int32_t* sorted_ids, int32_t* tile_ranges,
                 int64_t* num_dups, void* stream);

/* The same pipeline without the readback: bin_status (8 device words)
 * gets [0] the number of duplicates emitted, [1] the gsx_bin_error bits,
 * [2] the number refine_tiles dropped (they sort after all kept ones),
 * [3] the sum of the tile counts and [4] the sum of the binned rectangles'
 * heights (see gsx_bin_count_async); [5..7] are reserved (zero).  If the
 * emitted duplicates exceed capacity, sorted_ids/tile_ranges hold an
 * incomplete (but in-bounds: ids < n, ranges within [0, capacity]; on the
 * row-placement path all ranges (0,0)) binning, so kernels enqueued behind
 * it stay safe; the caller copies bin_status to the host when it needs D,
 * checks it with gsx_bin_status_check and re-runs with a larger capacity if
 * asked to. */
int gsx_bin_sort_async(int64_t n, const uint32_t* tile_counts,
                       const uint32_t* depth_keys, const uint32_t* tile_rects,
                       const float* means2d, const float* conics,
                       int64_t conic_stride, int32_t width, int32_t height,
                       void* workspace, int64_t workspace_bytes,
                       int64_t capacity, int32_t* sorted_ids,
                       int32_t* tile_ranges, uint32_t* bin_status,
                       void* stream);

/* The same pipeline in three calls, for callers that size the duplicate
 * buffers exactly instead of guessing a capacity.
 *
 * gsx_bin_count_async: zeroes tile_ranges and bin_status words 0 and 2..7,
 * builds the depth keys' digit histograms in depth_ws
 * (gsx_bin_depth_workspace_bytes(n)), adds the tile counts into
 * bin_status[3] (the number of duplicates emission will write before
 * refine_tiles drops any, with GSX_BIN_ERR_OVERFLOW in bin_status[1] past
 * 2^30 - 1) and the binned rectangles' heights into bin_status[4], and, for
 * images up to 256 x 256 tiles, per-row histograms of the rectangles.
 * bin_status[1] is not cleared: the error bits of every call on one
 * bin_status accumulate until the caller clears the word, so a readback
 * behind this call also reports the checks of earlier calls' tile phases.
 *
 * gsx_bin_depth_async: the stable depth sort (tiles.py:67-72) of the same
 * n depth keys in the same depth_ws, in passes of 9, 9, 9 and 5 bits
 * (the last is skipped on the device when all keys share its digit, as
 * the renderer's near-plane-relative keys do).  With host_status != NULL
 * (pinned host memory of 8 uint64 words, e.g. the first half of
 * gsx_host_status_alloc's 16) its first kernel writes host_status[k] =
 * (uint64_t)seq << 32 | bin_status[k] for k = 0..7 after the count phase
 * has finished: the host polls for `seq` instead of enqueueing a copy.
 *
 * gsx_bin_tiles_async: the rest of tiles.py:73-182 on the depth sort's
 * output, with the same n, tile_counts, tile_rects, width and height and
 * the same depth_ws, plus tile_ws (gsx_bin_tile_workspace_bytes(capacity,
 * num_tiles)).  bin_status then holds what gsx_bin_sort_async documents;
 * with capacity = bin_status[3] the duplicates always fit.  With
 * host_status != NULL (8 words) its last kernel writes the final status
 * there the same way.  tile_order: NULL, or the gsx_tile_order_words(W, H)
 * buffer of the frame's gsx_raster_fwd: the call writes the forward's tile
 * order for the ranges it produces into words [T, 2T) (the placement's
 * first workgroups compute it beside the placement; it is what
 * gsx_raster_fwd would compute), to be passed with order_ready = 1.
 *
 * gsx_bin_sort_async is the three in sequence on one workspace (depth part
 * first, all bin_status words cleared); gsx_bin_workspace_bytes is the sum
 * of the two sizes. */
int64_t gsx_bin_depth_workspace_bytes(int64_t n);
int64_t gsx_bin_tile_workspace_bytes(int64_t capacity, int32_t num_tiles);
int gsx_bin_count_async(int64_t n, const uint32_t* tile_counts,
                        const uint32_t* depth_keys, const uint32_t* tile_rects,
                        int32_t width, int32_t height, void* depth_ws,
                        int64_t depth_ws_bytes, int32_t* tile_ranges,
                        uint32_t* bin_status, void* stream);
int gsx_bin_depth_async(int64_t n, const uint32_t* depth_keys, void* depth_ws,
                        int64_t depth_ws_bytes, uint32_t* bin_status,
                        uint64_t* host_status, uint32_t seq, void* stream);
int gsx_bin_tiles_async(int64_t n, const uint32_t* tile_counts,
                        const uint32_t* tile_rects, const float* means2d,
                        const float* conics, int64_t conic_stride,
                        int32_t width, int32_t height, void* depth_ws,
                        int64_t depth_ws_bytes, void* tile_ws,
                        int64_t tile_ws_bytes, int64_t capacity,
                        int32_t* sorted_ids, int32_t* tile_ranges,
                        uint32_t* bin_status, uint64_t* host_status,
                        uint32_t seq, int32_t* tile_order, void* stream);

/* Host-side: interprets a host copy of the bin_status words.  Returns
 * GSX_OK with *num_dups = D (duplicates kept), 1 with *num_dups = the
 * capacity needed, GSX_ERR_TOO_LARGE or GSX_ERR_DEVICE. */
int gsx_bin_status_check(const uint32_t* host_status, int64_t capacity,
                         int64_t* num_dups);

/* Pinned, device-coherent host memory of 16 uint64 words (two host_status
 * targets), zeroed; the one allocation in this library, of host memory, for
 * the status polling above.  Released with gsx_host_status_free. */
int gsx_host_status_alloc(uint64_t** words);
int gsx_host_status_free(uint64_t* words);

/* ---------------------------------------------------------- rasterizer --
 * Packs conics (N,3) and opacities (N) into conic_opacity (N,4), the
 * layout the rasterizer gathers (rasterize.py:432-438 inputs). */
int gsx_pack_conic_opacity(int64_t n, const float* conics,
                           const float* opacities, float* conic_opacity,
                           void* stream);

/* Replaces gs_rasterize_forward (rasterize.py:28-98) for C channels in one
 * pass (rasterize_features, rasterize.py:449-545, chunks of 3), with the
 * expected depth of gs_rasterize_depth (rasterize.py:223-290) fused as an
 * extra output when depths != NULL.  features (N,C); sorted_ids
 * (num_ids); tile ranges are clamped to [0, num_ids] and ids outside [0, n)
 * are treated as transparent, so malformed inputs cannot read out of
 * bounds; background (C) or NULL (zeros); out (H,W,C); final_T (H,W);
 * n_contrib (H,W) int32; depth_out (H,W) when depths != NULL; alpha_out
 * (H,W) = 1 - final_T (rasterize.py:443) or NULL.
 * tile_order: NULL (tiles in launch order), or gsx_tile_order_words(W, H)
 * int32 words that the call fills: words [0, T) (T = ceil(W/16)
 * ceil(H/16)) each tile's largest n_contrib, which gsx_raster_bwd orders
 * its tiles by; words [T, 2T) the order the workgroups take the tiles in
 * (each XCD's contiguous band of tiles, longest lists first).  With
 * order_ready != 0 words [T, 2T) already hold that order, written by
 * gsx_bin_tiles_async for these ranges, and the call only reads them.  The
 * outputs do not depend on the order.  The buffer has no counterpart in the
 * reference (whose Metal dispatch has no such control). */
int gsx_raster_fwd(int64_t n, int32_t C, const float* means2d,
                   const float* conic_opacity, const float* features,
                   const float* depths, const int32_t* sorted_ids,
                   int64_t num_ids, const int32_t* tile_ranges,
                   const float* background,
                   int32_t width, int32_t height, float* out, float* final_T,
                   int32_t* n_contrib, float* depth_out, float* alpha_out,
                   int32_t* tile_order, int32_t order_ready, void* stream);

/* Replaces gs_rasterize_backward (rasterize.py:100-221) and the vjp wiring
 * of _rasterize_core (rasterize.py:364-403).  grad_out (H,W,C);
 * grad_final_T (H,W) or NULL.  Outputs (zeroed here, then accumulated):
 * g_means2d (N,2), g_conics (N,3), g_features (N,C), g_opacities (N) with
 * grad_stride = 0; with grad_stride > 0 (a multiple of 4, >= 6 + C) one
 * 16-byte aligned record per Gaussian at g_means2d, [means2d 2 | conic 3 |
 * opacity 1 | features C | padding], and the other three outputs NULL: a
 * Gaussian's float atomics from one tile then land in one or two cache
 * lines instead of one per array.  No gradient is produced for the
 * background (rasterize.py:401).  tile_order: NULL (launch order), or the
 * buffer gsx_raster_fwd filled for this frame: from the contributor bounds
 * in words [0, T) the call writes its order to the words after them (the
 * tiles cut into 8 contiguous bands of equal work, one per XCD, each band
 * heaviest first).  Any contents give a valid order; the gradients do not
 * depend on it beyond float atomic ordering. */
/* Size in int32 words of the rasterizers' tile_order buffer for a
 * width x height image: T + 16 ceil(T / 8) (0 for an empty image). */
int64_t gsx_tile_order_words(int32_t width, int32_t height);

int gsx_raster_bwd(int64_t n, int32_t C, const float* means2d,
                   const float* conic_opacity, const float* features,
                   const int32_t* sorted_ids, int64_t num_ids,
                   const int32_t* tile_ranges,
                   const float* background, int32_t width, int32_t height,
                   const float* final_T, const int32_t* n_contrib,
                   const float* grad_out, const float* grad_final_T,
                   float* g_means2d, float* g_conics, float* g_features,
                   float* g_opacities, int32_t grad_stride,
                   int32_t* tile_order, void* stream);

/* -------------------------------------------------------- training step --
 * The calls GaussianTrainer.step (splatting/trainer.py:319-421) makes
 * around the render. */

/* Workspace for one image of the photometric loss: three (H,W,C) float
 * maps of SSIM partial derivatives plus per-tile partial sums. */
int64_t gsx_photometric_workspace_bytes(int32_t height, int32_t width,
                                        int32_t channels);

/* Replaces l1 = mean|pred - target| and ssim(pred, target, max_val,
 * window_size, sigma) (trainer.py:303-305; losses/image_metrics.py:23-55,
 * 66-85: Gaussian window, zero-padded depthwise correlation, c1 =
 * (0.01 max_val)^2, c2 = (0.03 max_val)^2, mean over H*W*C).  pred and
 * target (H,W,C); window_size odd, at most 15.  out (2 floats, device):
 * [mean |pred - target|, mean SSIM].  The workspace keeps what
 * gsx_photometric_bwd needs; it must not change in between. */
int gsx_photometric_fwd(int32_t height, int32_t width, int32_t channels,
                        const float* pred, const float* target,
                        int32_t window_size, float sigma, float max_val,
                        void* workspace, int64_t workspace_bytes, float* out,
                        void* stream);

/* Gradient of both outputs of gsx_photometric_fwd with respect to pred:
 * grad_pred = grad_out[0] d(mean L1)/dpred + grad_out[1] d(mean SSIM)/dpred,
 * with grad_out (2 floats) on the device (what MLX autodiff of
 * image_metrics.py:29-55 computes).  sign(0) = 0 for the L1 term. */
int gsx_photometric_bwd(int32_t height, int32_t width, int32_t channels,
                        const float* pred, const float* target,
                        int32_t window_size, float sigma,
                        const void* workspace, int64_t workspace_bytes,
                        const float* grad_out, float* grad_pred, void* stream);

/* The trainer's objective loss = (1 - lambda) l1 + lambda (1 - ssim)
 * (trainer.py:303-305) in one call: gsx_photometric_fwd, and out3 (3
 * floats, device) = [l1, ssim, loss], the loss in the float32 steps of
 * that expression with 1 - lambda and lambda each rounded once to float32
 * (as the Python scalars reach float32 arithmetic).  0 <= lambda <= 1. */
int gsx_photometric_loss_fwd(int32_t height, int32_t width, int32_t channels,
                             const float* pred, const float* target,
                             int32_t window_size, float sigma, float max_val,
                             double lambda, void* workspace,
                             int64_t workspace_bytes, float* out3, void* stream);

/* Gradient of that loss: gsx_photometric_bwd with grad_out = (g (1 -
 * lambda), -(g lambda)) formed on the device from the loss cotangent g
 * (g_loss, 1 float, device), the values autodiff of the expression
 * gives. */
int gsx_photometric_loss_bwd(int32_t height, int32_t width, int32_t channels,
                             const float* pred, const float* target,
                             int32_t window_size, float sigma, double lambda,
                             const void* workspace, int64_t workspace_bytes,
                             const float* g_loss, float* grad_pred, void* stream);

/* Replaces l1_loss(pred, target) = mean |pred - target|
 * (losses/image_metrics.py:13-14) for n contiguous floats: out (1 float,
 * device); partial sums in double, added in a fixed order.  The workspace
 * holds the partials (gsx_l1_workspace_bytes). */
int64_t gsx_l1_workspace_bytes(int64_t n);
int gsx_l1_fwd(int64_t n, const float* pred, const float* target,
               void* workspace, int64_t workspace_bytes, float* out,
               void* stream);

/* gsx_l1_fwd without a workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  The partial sums go
 * to a file-scope device array (512 KiB per GPU, held until the process
 * ends), so n is at most gsx_l1_noalloc_max_elements() (2^28); larger n
 * returns GSX_ERR_TOO_LARGE.  The call allocates nothing: the array's
 * address is looked up once per device (GSX_ERR_HIP if that fails).  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, different host threads) race and must be ordered by
 * the caller.  Same kernels and summation order as gsx_l1_fwd, so the
 * results are bit-identical. */
int64_t gsx_l1_noalloc_max_elements(void);
int gsx_l1_fwd_noalloc(int64_t n, const float* pred, const float* target, float* out,
                       void* stream);

/* Its gradient: grad_pred = sign(pred - target) grad_out[0] / n (sign(0) =
 * 0), grad_out (1 float) on the device. */
int gsx_l1_bwd(int64_t n, const float* pred, const float* target,
               const float* grad_out, float* grad_pred, void* stream);

/* The same pair with the signs of pred - target kept between them (the
 * autodiff of losses/image_metrics.py:13-14 reads pred and target again):
 * gsx_l1_fwd_signs is gsx_l1_fwd that also writes one code byte per element
 * to signs (n bytes, device; 0: d > 0, 1: d < 0, 2: d == 0, 3: NaN), and
 * gsx_l1_bwd_signs writes gsx_l1_bwd's gradient from those codes, reading
 * pred and target only where the code is NaN (the gradient is then
 * pred - target).  Bit-identical to gsx_l1_fwd / gsx_l1_bwd; the backward
 * moves 5 bytes per element instead of 12. */
int gsx_l1_fwd_signs(int64_t n, const float* pred, const float* target,
                     void* workspace, int64_t workspace_bytes, uint8_t* signs,
                     float* out, void* stream);
int gsx_l1_bwd_signs(int64_t n, const uint8_t* signs, const float* pred,
                     const float* target, const float* grad_out,
                     float* grad_pred, void* stream);

#define GSX_ADAM_MAX_GROUPS 8

/* One parameter group of gsx_adam_step: n floats each (host struct). */
typedef struct gsx_adam_group {
    float* param;
    const float* grad;
    float* m;
    float* v;
    int64_t n;
    float lr;
} gsx_adam_group;

/* Replaces the per-group mlx.optimizers.Adam(learning_rate=lr, eps=eps)
 * updates of trainer.py:128, 339-342 (mlx >= 0.31, bias_correction off):
 * m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2; p -= lr m / (sqrt(v) + eps),
 * float32, in place, all groups in one launch.  m and v start at zero. */
int gsx_adam_step(int32_t num_groups, const gsx_adam_group* groups,
                  float beta1, float beta2, float eps, void* stream);

/* gsx_preprocess_bwd followed by gsx_adam_step on the six parameter groups
 * of GaussianTrainer.step (trainer.py:339-342 after the autodiff VJP of
 * render.py:73-80 / model.py:116-126), fused: every gradient goes from
 * registers into the Adam update of its parameter, so the gradients are
 * never written out and read back.  The reference has no single call for
 * this; the updates are those gsx_adam_step applies to the gradients
 * gsx_preprocess_bwd writes, bit for bit.  groups[6]: means, quats, scales,
 * opacities, sh_dc, sh_rest (param = the tensor passed here, n = its float
 * count, grad unused); SH in split layout with contiguous rows (sh_dc (N,3),
 * sh_rest (N, 3 (K-1)), K >= 1), moments with the parameters' layouts,
 * quats and its moments 16-byte aligned.  Parameters and moments are
 * updated in place.  K = 1: groups[5] is not read.  The rasterizer
 * gradients come as in gsx_preprocess_bwd (grad_stride). */
int gsx_preprocess_bwd_adam(const gsx_camera* cam, int64_t n, float* means, float* quats,
                            float* scales, float* opacities, float* sh_dc, float* sh_rest,
                            const float* colors_out, int32_t K, int32_t degree, uint32_t flags,
                            float blur, const float* g_means2d, const float* g_conics,
                            const float* g_opac_eff, const float* g_colors,
                            const float* g_means2d_extra, const float* g_depths,
                            const float* g_compensation, const gsx_adam_group* groups,
                            float beta1, float beta2, float eps, int32_t grad_stride,
                            void* stream);

/* Replaces the density-control statistics of trainer.py:357-365:
 * grad_accum += |(g.x W/2, g.y H/2)| * (radii > 0); grad_count += (radii > 0).
 * g_means2d (N,2) is dL/dmeans2d of the rasterizer (the reference's
 * means2d probe gradient, trainer.py:264-275, 337); with grad_stride > 0
 * (even) the (x, y) pairs are grad_stride floats apart (a gradient record). */
int gsx_accum_screen_grads(int64_t n, const float* g_means2d,
                           const float* radii, int32_t width, int32_t height,
                           float* grad_accum, float* grad_count, int32_t grad_stride,
                           void* stream);

/* ------------------------------------------------------ table edits --
 * A Gaussian table: up to GSX_TABLE_MAX float32 tensors of N rows, tensor k
 * holding width[k] contiguous floats per row (the parameter groups, and in
 * training their Adam moments).  src and dst are the tensors before and
 * after the edit (the same pointers for in-place edits).  Host struct. */
#define GSX_TABLE_MAX 20
enum gsx_row_role {
    GSX_ROW_PARAM = 1,   /* a parameter tensor: rows are copied or edited     */
    GSX_ROW_MOMENT = 2   /* an optimizer moment: new or moved rows are zero    */
};
typedef struct gsx_row_table {
    int32_t count;
    int32_t width[GSX_TABLE_MAX];
    int32_t role[GSX_TABLE_MAX];
    const float* src[GSX_TABLE_MAX];
    float* dst[GSX_TABLE_MAX];
} gsx_row_table;

/* Replaces the nearest-neighbour scale of GaussianModel.from_points
 * (splatting/model.py:72-92 with ops/knn.py:121-177): for each of n_query
 * points the k nearest of n_ref reference points (squared distance = sum of
 * the squared coordinate differences, ties to the lower index), the mean of
 * the k - 1 nearest skipping a self hit (first distance <= 1e-12), clamped
 * at 1e-8, written as log(sqrt(mean)) capped at log_cap.  2 <= k <= 8,
 * k <= n_ref. */
int gsx_knn_log_scale(int64_t n_query, const float* query, int64_t n_ref,
                      const float* ref, int32_t k, float log_cap, float* log_scale,
                      void* stream);

/* Replaces densify_and_prune (splatting/model.py:406-480), in two calls.
 * gsx_density_classify: per row, avg = grad_accum / max(grad_count, 1),
 * s = max of exp(log_scales); clone if avg > grad_threshold and s <=
 * dense_scale, split if avg > grad_threshold and s > dense_scale; pruned
 * (not kept) if sigmoid(clip(logit, -50, 50)) < min_opacity, split, or s >
 * prune_scale.  totals (3 uint32, device) = (kept, cloned, split).  The
 * workspace (gsx_density_workspace_bytes) carries the classes to the second
 * call.  gsx_density_emit: with the new tensors sized kept + cloned +
 * 2 split rows, writes rows [kept originals, clones, split pairs], each part
 * in source order; a split pair's means move by R(q) (s * xi) with xi from
 * split_samples ((2 split, 3) float64 standard normals, pair-major, as the
 * reference draws them) and R from the normalised quaternion, log-scales drop
 * by log_shrink; GSX_ROW_MOMENT tensors keep kept rows' values and are zero in
 * new rows. */
int64_t gsx_density_workspace_bytes(int64_t n);
int gsx_density_classify(int64_t n, const float* log_scales, const float* logit_opacities,
                         const float* grad_accum, const float* grad_count,
                         float grad_threshold, float dense_scale, float prune_scale,
                         float min_opacity, void* workspace, int64_t workspace_bytes,
                         uint32_t* totals, void* stream);
int gsx_density_emit(int64_t n, const void* workspace, int64_t workspace_bytes,
                     const uint32_t* totals, const gsx_row_table* table, int32_t means_col,
                     int32_t scales_col, int32_t quats_col, const double* split_samples,
                     float log_shrink, void* stream);

/* Replaces the scores relocate_mcmc selects by (splatting/model.py:497-512):
 * target_score = 2 - sigmoid(o) where the row is underused (sigmoid(o) <
 * min_opacity or grad_count <= 0), else -sigmoid(o); source_score =
 * grad_accum / max(grad_count, 1); *under_count (device, caller-zeroed) +=
 * the number of underused rows.  The caller picks the k largest of each
 * (sources among rows that are not destinations). */
int gsx_relocate_scores(int64_t n, const float* grad_accum, const float* grad_count,
                        const float* logit_opacities, float min_opacity, float* target_score,
                        float* source_score, uint32_t* under_count, void* stream);

/* Replaces the row rewrite of relocate_mcmc (splatting/model.py:517-529), in
 * place: row dst_rows[j] takes source row src_rows[j] (k pairs, int64,
 * device) with means + noise[j] * exp(log-scale) * jitter, the opacity
 * logit reset_logit and log-scales - log_shrink, written as old + (new -
 * old) (the reference's scatter-add); moments of the destination rows
 * become zero.  staging: k times the sum of the parameter widths floats. */
int gsx_density_relocate(int64_t k, const int64_t* src_rows, const int64_t* dst_rows,
                         const gsx_row_table* table, int32_t means_col, int32_t scales_col,
                         int32_t opac_col, const float* noise, float jitter,
                         float reset_logit, float log_shrink, float* staging,
                         int64_t staging_floats, void* stream);

/* ---------------------------------------------------- 2DGS geometry --
 * Replaces the 2DGS regularisers of GaussianTrainer._geometry_loss_2dgs
 * (splatting/trainer.py:187-259).
 * gsx_geom_features: features (N,5) = (z, z^2, n), n the normalised third
 * column of the rotation of the normalised quaternion, negated when
 * n . (center - mean) < 0; center = the camera centre (3 floats, host).
 * gsx_geom_features_bwd: the VJP into depths (N) and quaternions (N,4).
 * gsx_geom_loss_fwd: on the alpha-normalised render F (H,W,5) of those
 * features and alpha (H,W), with unprojection maps P = base + z dir
 * ((H,W,3) each, the world point of a pixel centre at z-depth z):
 *   depth variance = sum over alpha > min_alpha of max(F1 - F0^2, 0) / max(count, 1)
 *   normal term    = sum over 2x2 quads whose 4 pixels pass of
 *                    1 - |unit(F[2:5]) . unit((P01 - P00) x (P10 - P00))| / max(count, 1)
 * out (5 floats, device) = [lam_dv dv + lam_nc nc, dv, nc, dv divisor, nc
 * divisor]; a term with lambda <= 0 is off (and the normal term needs W, H
 * > 1).  gsx_geom_loss_bwd: dL/dF (H,W,5) from fwd_out and the loss
 * cotangent grad_loss (1 float, device); alpha gets no gradient (its test
 * is a step). */
int gsx_geom_features(int64_t n, const float* means, const float* quats, const float* depths,
                      const float* center, float* features, void* stream);
int gsx_geom_features_bwd(int64_t n, const float* means, const float* quats,
                          const float* depths, const float* center, const float* g_features,
                          float* g_depths, float* g_quats, void* stream);
int64_t gsx_geom_loss_workspace_bytes(int32_t width, int32_t height);
int gsx_geom_loss_fwd(int32_t width, int32_t height, const float* features, const float* alpha,
                      const float* base, const float* dir, float min_alpha, float lam_dv,
                      float lam_nc, void* workspace, int64_t workspace_bytes, float* out,
                      void* stream);
int gsx_geom_loss_bwd(int32_t width, int32_t height, const float* features, const float* alpha,
                      const float* base, const float* dir, float min_alpha, float lam_dv,
                      float lam_nc, const float* fwd_out, const float* grad_loss,
                      float* g_features, void* stream);

/* --------------------------------------------------------- mesh raster --
 * Replaces the hard z-buffer kernel of rasterize_meshes
 * (renderer/rasterizer.py:29-87), the mesh consumer of bin_gaussians: the
 * caller bins faces by centroid, bounding-circle radius and mean depth
 * (rasterizer.py:140-146) and passes the screen-space vertices tri_xy
 * (F,6) = (ax, ay, bx, by, cx, cy), camera depths tri_z (F,3), sorted ids
 * and tile ranges.  Per pixel (centre +0.5) the nearest face with all
 * barycentrics >= -1e-5 and interpolated depth > znear wins (first in list
 * order on ties); pix_to_face (H,W) int32 (-1 = empty), zbuf (H,W) (0 where
 * empty). */
int gsx_mesh_raster(int64_t n_faces, const float* tri_xy, const float* tri_z,
                    const int32_t* sorted_ids, int64_t num_ids,
                    const int32_t* tile_ranges, int32_t width, int32_t height,
                    float znear, int32_t* pix_to_face, float* zbuf, void* stream);

/* ---------------------------------------------------------- diagnostics --
 * Evaluates the device exp used by the rasterizer (the stand-in for
 * metal::exp at rasterize.py:80,171,274) on n inputs; tests check it
 * bit-for-bit against the CPU oracle. */
int gsx_debug_expf(int64_t n, const float* x, float* y, void* stream);

/* Evaluates the device arctan of the fisheye lens model (the stand-in for
 * the arctan at cameras.py:72) on n inputs >= 0; tests check it bit for bit
 * against the CPU oracle. */
int gsx_debug_atanf(int64_t n, const float* x, float* y, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GSX_H */
