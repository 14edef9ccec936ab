// preprocess.hip -- per-Gaussian kernels (one lane per Gaussian):
//   projection   (splatting/projection.py:24-146)       fwd + VJP
//   eval_sh      (splatting/sh.py:41-78)                fwd + VJP
//   fused preprocess of render_gaussians / GaussianModel.render
//                (model.py:116-126, render.py:73-80, tiles.py:54-65) fwd + VJP
//   bin_prepare  (tiles.py:54-65 on given means2d/radii/depths)
//   conic/opacity packing for the rasterizer
#include "gsx_device.h"

using namespace gsx;

namespace {

constexpr int kThreads = 256;

inline unsigned grid_for(int64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

// SH coefficient rows are moved between HBM and LDS by the whole workgroup
// with consecutive lanes on consecutive floats, instead of each lane
// touching its own 180-192 strided bytes (which costs one cache-line request
// per lane per load).  LDS rows are padded to an odd length so that lane r
// walking its own row hits distinct banks.
enum ShMode { kShDirect = 0, kShSplit = 1, kShPacked = 2 };
constexpr int kShMaxCols = 48;  // 16 coefficients x 3 channels
constexpr int kShPad = kShMaxCols + 1;

// Row r and column c of the flattened index j (cols >= 1, j < 2^20).
__device__ __forceinline__ void row_col(int j, int cols, float inv, int& r, int& c) {
    r = (int)(((float)j + 0.5f) * inv);
    c = j - r * cols;
    if (c < 0) {
        --r;
        c += cols;
    } else if (c >= cols) {
        ++r;
        c -= cols;
    }
}

// Rows [g0, g0 + rows) of `cols` floats (row r at base + (g0 + r) * stride)
// into LDS rows of `pad` floats.  Loads go out kBatch at a time so their
// latencies overlap; 48 covers a whole workgroup's rows (<= 48 columns) in
// one batch.
__device__ __forceinline__ void rows_to_lds(float* s, int pad, const float* __restrict__ base,
                                            int64_t stride, int64_t g0, int rows, int cols) {
    constexpr int kBatch = 48;
    const int total = rows * cols;
    const float inv = 1.0f / (float)cols;
    for (int j0 = threadIdx.x; j0 < total; j0 += kBatch * kThreads) {
        float v[kBatch];
        int at[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int j = j0 + u * kThreads;
            at[u] = -1;
            v[u] = 0.0f;
            if (j < total) {
                int r, c;
                row_col(j, cols, inv, r, c);
                v[u] = base[(g0 + r) * stride + c];
                at[u] = r * pad + c;
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (at[u] >= 0) s[at[u]] = v[u];
    }
}

// Contiguous rows (stride == cols, odd cols so that lane r walking its own
// row of the unpadded copy hits distinct banks): `total` floats from src
// (16-byte aligned) into LDS by direct-to-LDS loads (global_load_lds_dwordx4:
// each lane's 16 bytes land at the wave's LDS base + 16 lane), no VGPR
// round trip; the < 4 tail floats go through registers.  The caller waits
// for the loads (vmcnt) before its barrier.
__device__ __forceinline__ void rows_to_lds_direct(float* s, const float* __restrict__ src,
                                                   int total) {
    const int n4 = total >> 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int b4 = wave * kWave; b4 < n4; b4 += kThreads) {
        if (b4 + lane < n4)
            __builtin_amdgcn_global_load_lds(
                src + 4 * (b4 + lane),
                (__attribute__((address_space(3))) void*)(s + 4 * b4), 16, 0, 0);
    }
    const int t = 4 * n4 + (int)threadIdx.x;
    if (t < total) s[t] = src[t];
}

// The reverse: LDS rows of `pad` floats out to rows of `cols` floats.
__device__ __forceinline__ void lds_to_rows(const float* s, int pad, float* __restrict__ base,
                                            int64_t stride, int64_t g0, int rows, int cols) {
    const int total = rows * cols;
    const float inv = 1.0f / (float)cols;
    for (int j = threadIdx.x; j < total; j += kThreads) {
        int r, c;
        row_col(j, cols, inv, r, c);
        base[(g0 + r) * stride + c] = s[r * pad + c];
    }
}

template <bool UT>
__global__ __launch_bounds__(kThreads) void k_project_fwd(
    gsx_camera cam, int64_t n, const float* __restrict__ means, const float4* __restrict__ quats,
    const float* __restrict__ scales, float blur, bool aa, float2* __restrict__ means2d,
    float* __restrict__ conics, float* __restrict__ depths, float* __restrict__ radii,
    float* __restrict__ comp) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float4 q = quats[i];
    typename ProjOf<UT>::T p;
    project_any<UT>(cam, means[3 * i], means[3 * i + 1], means[3 * i + 2], q.x, q.y, q.z, q.w,
                    scales[3 * i], scales[3 * i + 1], scales[3 * i + 2], blur, aa, p);
    means2d[i] = make_float2(p.u, p.v);
    conics[3 * i] = p.A;
    conics[3 * i + 1] = p.B;
    conics[3 * i + 2] = p.C;
    depths[i] = p.z;
    radii[i] = p.radius;
    comp[i] = p.comp;
}

template <bool UT>
__global__ __launch_bounds__(kThreads) void k_project_bwd(
    gsx_camera cam, int64_t n, const float* __restrict__ means, const float4* __restrict__ quats,
    const float* __restrict__ scales, float blur, bool aa, const float2* __restrict__ g_means2d,
    const float* __restrict__ g_conics, const float* __restrict__ g_depths,
    const float* __restrict__ g_comp, float* __restrict__ g_means, float4* __restrict__ g_quats,
    float* __restrict__ g_scales) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float4 q = quats[i];
    const float m0 = means[3 * i], m1 = means[3 * i + 1], m2 = means[3 * i + 2];
    typename ProjOf<UT>::T p;
    project_any<UT>(cam, m0, m1, m2, q.x, q.y, q.z, q.w, scales[3 * i], scales[3 * i + 1],
                    scales[3 * i + 2], blur, aa, p);
    const float2 gm2 = g_means2d ? g_means2d[i] : make_float2(0.0f, 0.0f);
    float gm[3], gq[4], gs[3];
    project_any_vjp<UT>(cam, p, m0, m1, m2, aa, gm2.x, gm2.y,
                        g_conics ? g_conics[3 * i] : 0.0f, g_conics ? g_conics[3 * i + 1] : 0.0f,
                        g_conics ? g_conics[3 * i + 2] : 0.0f, g_depths ? g_depths[i] : 0.0f,
                        g_comp ? g_comp[i] : 0.0f, gm, gq, gs);
    g_means[3 * i] = gm[0];
    g_means[3 * i + 1] = gm[1];
    g_means[3 * i + 2] = gm[2];
    g_quats[i] = make_float4(gq[0], gq[1], gq[2], gq[3]);
    g_scales[3 * i] = gs[0];
    g_scales[3 * i + 1] = gs[1];
    g_scales[3 * i + 2] = gs[2];
}

// eval_sh over (N, K, C) coefficients, one lane per (Gaussian, channel).
__global__ __launch_bounds__(kThreads) void k_eval_sh_fwd(int64_t n, int K, int C, int degree,
                                                          const float* __restrict__ sh,
                                                          const float* __restrict__ dirs,
                                                          float* __restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= n * C) return;
    const int64_t i = t / C;
    const int ch = (int)(t - i * C);
    const float x = dirs[3 * i], y = dirs[3 * i + 1], z = dirs[3 * i + 2];
    float bk[16], c[16];
    sh_basis(degree, x, y, z, bk);
    const int Ka = (degree + 1) * (degree + 1);
    const float* shi = sh + i * (int64_t)K * C + ch;
#pragma unroll
    for (int k = 0; k < 16; ++k) c[k] = (k < Ka) ? shi[(int64_t)k * C] : 0.0f;
    out[t] = sh_eval(degree, bk, c, x, y, z);
}

// Partial derivatives of the basis functions w.r.t. the direction.
__device__ __forceinline__ void sh_basis_grad(int degree, float x, float y, float z, float* dx,
                                              float* dy, float* dz) {
#pragma unroll
    for (int k = 0; k < 16; ++k) dx[k] = dy[k] = dz[k] = 0.0f;
    if (degree < 1) return;
    dy[1] = -GSX_SH_C1;
    dz[2] = GSX_SH_C1;
    dx[3] = -GSX_SH_C1;
    if (degree < 2) return;
    dx[4] = GSX_SH_C2_0 * y;
    dy[4] = GSX_SH_C2_0 * x;
    dy[5] = GSX_SH_C2_1 * z;
    dz[5] = GSX_SH_C2_1 * y;
    dx[6] = GSX_SH_C2_2 * -2.0f * x;
    dy[6] = GSX_SH_C2_2 * -2.0f * y;
    dz[6] = GSX_SH_C2_2 * 4.0f * z;
    dx[7] = GSX_SH_C2_3 * z;
    dz[7] = GSX_SH_C2_3 * x;
    dx[8] = GSX_SH_C2_4 * 2.0f * x;
    dy[8] = GSX_SH_C2_4 * -2.0f * y;
    if (degree < 3) return;
    const float xx = x * x, yy = y * y, zz = z * z;
    dx[9] = GSX_SH_C3_0 * 6.0f * x * y;
    dy[9] = GSX_SH_C3_0 * (3.0f * xx - 3.0f * yy);
    dx[10] = GSX_SH_C3_1 * y * z;
    dy[10] = GSX_SH_C3_1 * x * z;
    dz[10] = GSX_SH_C3_1 * x * y;
    dx[11] = GSX_SH_C3_2 * -2.0f * x * y;
    dy[11] = GSX_SH_C3_2 * (4.0f * zz - xx - 3.0f * yy);
    dz[11] = GSX_SH_C3_2 * 8.0f * y * z;
    dx[12] = GSX_SH_C3_3 * -6.0f * x * z;
    dy[12] = GSX_SH_C3_3 * -6.0f * y * z;
    dz[12] = GSX_SH_C3_3 * (6.0f * zz - 3.0f * xx - 3.0f * yy);
    dx[13] = GSX_SH_C3_4 * (4.0f * zz - 3.0f * xx - yy);
    dy[13] = GSX_SH_C3_4 * -2.0f * x * y;
    dz[13] = GSX_SH_C3_4 * 8.0f * x * z;
    dx[14] = GSX_SH_C3_5 * 2.0f * x * z;
    dy[14] = GSX_SH_C3_5 * -2.0f * y * z;
    dz[14] = GSX_SH_C3_5 * (xx - yy);
    dx[15] = GSX_SH_C3_6 * (3.0f * xx - 3.0f * yy);
    dy[15] = GSX_SH_C3_6 * -6.0f * x * y;
}

// VJP of eval_sh, one lane per Gaussian (the direction gradient sums over
// channels).
__global__ __launch_bounds__(kThreads) void k_eval_sh_bwd(int64_t n, int K, int C, int degree,
                                                          const float* __restrict__ sh,
                                                          const float* __restrict__ dirs,
                                                          const float* __restrict__ g_out,
                                                          float* __restrict__ g_sh,
                                                          float* __restrict__ g_dirs) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float x = dirs[3 * i], y = dirs[3 * i + 1], z = dirs[3 * i + 2];
    float bk[16], dx[16], dy[16], dz[16];
    sh_basis(degree, x, y, z, bk);
    sh_basis_grad(degree, x, y, z, dx, dy, dz);
    const int Ka = (degree + 1) * (degree + 1);
    const float* shi = sh + i * (int64_t)K * C;
    float* gsh = g_sh + i * (int64_t)K * C;
    float gd0 = 0.0f, gd1 = 0.0f, gd2 = 0.0f;
    for (int k = 0; k < K; ++k)
        for (int ch = 0; ch < C; ++ch) {
            const float go = g_out[i * C + ch];
            const bool act = k < Ka;
            gsh[k * C + ch] = act ? bk[k < 16 ? k : 0] * go : 0.0f;
            if (act) {
                const float cv = shi[k * C + ch];
                gd0 += dx[k] * cv * go;
                gd1 += dy[k] * cv * go;
                gd2 += dz[k] * cv * go;
            }
        }
    if (g_dirs) {
        g_dirs[3 * i] = gd0;
        g_dirs[3 * i + 1] = gd1;
        g_dirs[3 * i + 2] = gd2;
    }
}

// Fused forward preprocess: activations, projection, compensation, SH colour,
// binning rectangle/count and depth key for one Gaussian per lane.  SH
// coefficients come through LDS (sh_mode: split = rest rows staged, DC read
// directly; packed = whole rows of 3 Ka floats staged; direct = no staging).
template <bool UT>
__global__ __launch_bounds__(kThreads) void k_preprocess_fwd(
    gsx_camera cam, int64_t n, const float* __restrict__ means, const float4* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ opacities,
    const float* __restrict__ sh0, int64_t s0, const float* __restrict__ shr, int64_t sr, int K,
    int degree, int sh_mode, int sh_cols, uint32_t flags, float blur, bool aa, int tiles_x,
    int tiles_y, float2* __restrict__ means2d, float* __restrict__ depths,
    float* __restrict__ radii, float* __restrict__ comp, float4* __restrict__ conic_opac,
    float* __restrict__ colors_out, uint32_t* __restrict__ counts, uint32_t* __restrict__ dkeys,
    uint2* __restrict__ rects) {
    __shared__ float s_sh[kThreads * kShPad];
    const int64_t g0 = (int64_t)blockIdx.x * kThreads;
    const int64_t i = g0 + threadIdx.x;
    const int pad = sh_cols | 1;
    // the Gaussian's own inputs are requested before the SH rows, so both
    // loads are in flight together (lanes past n re-read row n - 1; the host
    // launches nothing for n == 0)
    const int64_t il = i < n ? i : n - 1;
    const float m0 = means[3 * il], m1 = means[3 * il + 1], m2 = means[3 * il + 2];
    const float4 q = quats[il];
    const float r0 = scales[3 * il], r1 = scales[3 * il + 1], r2 = scales[3 * il + 2];
    const float ro = opacities[il];
    if (sh_mode != kShDirect) {
        const int rows = (int)min<int64_t>(kThreads, n - g0);
        const float* base = sh_mode == kShPacked ? sh0 : shr;
        const int64_t stride = sh_mode == kShPacked ? s0 : sr;
        if (stride == sh_cols && pad == sh_cols &&
            ((uintptr_t)(base + g0 * stride) & 15u) == 0u) {
            rows_to_lds_direct(s_sh, base + g0 * stride, rows * sh_cols);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            rows_to_lds(s_sh, pad, base, stride, g0, rows, sh_cols);
        }
        __syncthreads();
    }
    if (i >= n) return;
    const float sx = act_scale(r0, flags);
    const float sy = act_scale(r1, flags);
    const float sz = act_scale(r2, flags);
    const float o = act_opacity(ro, flags);
    typename ProjOf<UT>::T p;
    project_any<UT>(cam, m0, m1, m2, q.x, q.y, q.z, q.w, sx, sy, sz, blur, aa, p);
    means2d[i] = make_float2(p.u, p.v);
    depths[i] = p.z;
    radii[i] = p.radius;
    comp[i] = p.comp;
    conic_opac[i] = make_float4(p.A, p.B, p.C, o * p.comp);
    if (sh0) {
        float dx, dy, dz;
        view_dir(cam, m0, m1, m2, dx, dy, dz);
        float bk[16];
        sh_basis(degree, dx, dy, dz, bk);
        const int Ka = (degree + 1) * (degree + 1);
        const float* a = sh0 + i * s0;
        const float* b = shr + i * sr;
        const float* row = s_sh + threadIdx.x * pad;
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
            float c[16];
            c[0] = sh_mode == kShPacked ? row[ch] : a[ch];
#pragma unroll
            for (int k = 1; k < 16; ++k) {
                float v = 0.0f;
                if (k < Ka) {
                    if (sh_mode == kShPacked) v = row[3 * k + ch];
                    else if (sh_mode == kShSplit) v = row[3 * (k - 1) + ch];
                    else v = b[3 * (k - 1) + ch];
                }
                c[k] = v;
            }
            colors_out[3 * i + ch] = fmaxf(sh_eval(degree, bk, c, dx, dy, dz), 0.0f);
        }
    }
    uint2 rect;
    const uint32_t cnt = tile_rect(p.u, p.v, p.radius, cam.width, cam.height, tiles_x, tiles_y, rect);
    counts[i] = cnt;
    dkeys[i] = cnt ? depth_key(p.z) : 0xFFFFFFFFu;
    rects[i] = rect;
}

// VJP of k_preprocess_fwd, one Gaussian per lane.  SH gradients (zero for
// coefficients >= Ka) are written through LDS rows in the same sh_mode
// layouts as the forward reads.
template <bool UT>
__global__ __launch_bounds__(kThreads) void k_preprocess_bwd(
    gsx_camera cam, int64_t n, const float* __restrict__ means, const float4* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ opacities,
    const float* __restrict__ colors_out, int K, int degree, int sh_mode, int sh_cols,
    uint32_t flags, float blur, bool aa, const float2* __restrict__ g_means2d,
    const float* __restrict__ g_conics, const float* __restrict__ g_opac_eff,
    const float* __restrict__ g_colors, const float2* __restrict__ g_means2d_extra,
    const float* __restrict__ g_depths, const float* __restrict__ g_comp,
    float* __restrict__ g_means, float4* __restrict__ g_quats, float* __restrict__ g_scales,
    float* __restrict__ g_opacities, float* __restrict__ g_sh0, int64_t s0,
    float* __restrict__ g_shr, int64_t sr) {
    __shared__ float s_sh[kThreads * kShPad];
    const int64_t g0 = (int64_t)blockIdx.x * kThreads;
    const int64_t i = g0 + threadIdx.x;
    const int pad = sh_cols | 1;
    if (i < n) {
        const float m0 = means[3 * i], m1 = means[3 * i + 1], m2 = means[3 * i + 2];
        const float4 q = quats[i];
        const float sx = act_scale(scales[3 * i], flags);
        const float sy = act_scale(scales[3 * i + 1], flags);
        const float sz = act_scale(scales[3 * i + 2], flags);
        const float o = act_opacity(opacities[i], flags);
        typename ProjOf<UT>::T p;
        project_any<UT>(cam, m0, m1, m2, q.x, q.y, q.z, q.w, sx, sy, sz, blur, aa, p);
        const float goe = g_opac_eff[i];
        const float g_o = goe * p.comp;
        const float g_comp_total = (g_comp ? g_comp[i] : 0.0f) + goe * o;
        float2 gm2 = g_means2d[i];
        if (g_means2d_extra) {
            const float2 e = g_means2d_extra[i];
            gm2.x += e.x;
            gm2.y += e.y;
        }
        float gm[3], gq[4], gs[3];
        project_any_vjp<UT>(cam, p, m0, m1, m2, aa, gm2.x, gm2.y, g_conics[3 * i],
                            g_conics[3 * i + 1], g_conics[3 * i + 2],
                            g_depths ? g_depths[i] : 0.0f, g_comp_total, gm, gq, gs);
        g_means[3 * i] = gm[0];
        g_means[3 * i + 1] = gm[1];
        g_means[3 * i + 2] = gm[2];
        g_quats[i] = make_float4(gq[0], gq[1], gq[2], gq[3]);
        const bool ls = flags & GSX_LOG_SCALES;
        g_scales[3 * i] = ls ? gs[0] * sx : gs[0];
        g_scales[3 * i + 1] = ls ? gs[1] * sy : gs[1];
        g_scales[3 * i + 2] = ls ? gs[2] * sz : gs[2];
        g_opacities[i] = (flags & GSX_LOGIT_OPACITY) ? g_o * o * (1.0f - o) : g_o;
        if (g_sh0) {
            float dx, dy, dz;
            view_dir(cam, m0, m1, m2, dx, dy, dz);
            float bk[16];
            sh_basis(degree, dx, dy, dz, bk);
            const int Ka = (degree + 1) * (degree + 1);
            float gc[3];
#pragma unroll
            for (int ch = 0; ch < 3; ++ch)
                gc[ch] = (colors_out[3 * i + ch] > 0.0f) ? g_colors[3 * i + ch] : 0.0f;
            float* row = s_sh + threadIdx.x * pad;
            if (sh_mode == kShPacked) {
                for (int k = 0; k < K; ++k) {
                    const float bv = (k < Ka) ? bk[k < 16 ? k : 0] : 0.0f;
#pragma unroll
                    for (int ch = 0; ch < 3; ++ch) row[3 * k + ch] = bv * gc[ch];
                }
            } else {
                float* a = g_sh0 + i * s0;
#pragma unroll
                for (int ch = 0; ch < 3; ++ch) a[ch] = bk[0] * gc[ch];
                float* b = sh_mode == kShSplit ? row : g_shr + i * sr;
                for (int k = 1; k < K; ++k) {
                    const float bv = (k < Ka) ? bk[k < 16 ? k : 0] : 0.0f;
#pragma unroll
                    for (int ch = 0; ch < 3; ++ch) b[3 * (k - 1) + ch] = bv * gc[ch];
                }
            }
        }
    }
    if (sh_mode != kShDirect) {
        __syncthreads();
        const int rows = (int)min<int64_t>(kThreads, n - g0);
        lds_to_rows(s_sh, pad, sh_mode == kShPacked ? g_sh0 : g_shr,
                    sh_mode == kShPacked ? s0 : sr, g0, rows, sh_cols);
    }
}

__global__ __launch_bounds__(kThreads) void k_bin_prepare(
    int64_t n, const float2* __restrict__ means2d, const float* __restrict__ radii,
    const float* __restrict__ depths, int width, int height, int tiles_x, int tiles_y,
    uint32_t* __restrict__ counts, uint32_t* __restrict__ dkeys, uint2* __restrict__ rects) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float2 m = means2d[i];
    uint2 rect;
    const uint32_t cnt = tile_rect(m.x, m.y, radii[i], width, height, tiles_x, tiles_y, rect);
    counts[i] = cnt;
    dkeys[i] = cnt ? depth_key(depths[i]) : 0xFFFFFFFFu;
    rects[i] = rect;
}

__global__ __launch_bounds__(kThreads) void k_pack_conic_opacity(int64_t n,
                                                                 const float* __restrict__ conics,
                                                                 const float* __restrict__ opac,
                                                                 float4* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    out[i] = make_float4(conics[3 * i], conics[3 * i + 1], conics[3 * i + 2], opac[i]);
}

__global__ __launch_bounds__(kThreads) void k_debug_atanf(int64_t n, const float* __restrict__ x,
                                                         float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) y[i] = datan_pos(x[i]);
}

__global__ __launch_bounds__(kThreads) void k_debug_expf(int64_t n, const float* __restrict__ x,
                                                         float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) y[i] = dexp(x[i]);
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline bool aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }

inline bool lens_ok(const gsx_camera* cam) {
    return cam->lens == GSX_LENS_NONE || cam->lens == GSX_LENS_BROWN ||
           cam->lens == GSX_LENS_FISHEYE;
}

template <bool UT>
int project_fwd_impl(const gsx_camera* cam, int64_t n, const float* means, const float* quats,
                     const float* scales, float blur, int32_t antialias, float* means2d,
                     float* conics, float* depths, float* radii, float* compensation,
                     void* stream) {
    if (!cam || n < 0 || !lens_ok(cam)) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!means || !quats || !scales || !means2d || !conics || !depths || !radii || !compensation)
        return GSX_ERR_INVALID;
    if (!aligned16(quats) || !aligned8(means2d)) return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_project_fwd<UT>, dim3(grid_for(n)), dim3(kThreads), 0,
                       (hipStream_t)stream, *cam, n, means, (const float4*)quats, scales, blur,
                       antialias != 0 && blur > 0.0f, (float2*)means2d, conics, depths, radii,
                       compensation);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

template <bool UT>
int project_bwd_impl(const gsx_camera* cam, int64_t n, const float* means, const float* quats,
                     const float* scales, float blur, int32_t antialias, const float* g_means2d,
                     const float* g_conics, const float* g_depths, const float* g_compensation,
                     float* g_means, float* g_quats, float* g_scales, void* stream) {
    if (!cam || n < 0 || !lens_ok(cam)) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!means || !quats || !scales || !g_means || !g_quats || !g_scales) return GSX_ERR_INVALID;
    if (!aligned16(quats) || !aligned16(g_quats) || (g_means2d && !aligned8(g_means2d)))
        return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_project_bwd<UT>, dim3(grid_for(n)), dim3(kThreads), 0,
                       (hipStream_t)stream, *cam, n, means, (const float4*)quats, scales, blur,
                       antialias != 0 && blur > 0.0f, (const float2*)g_means2d, g_conics,
                       g_depths, g_compensation, g_means, (float4*)g_quats, g_scales);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // namespace

extern "C" {

int gsx_project_fwd(const gsx_camera* cam, int64_t n, const float* means, const float* quats,
                    const float* scales, float blur, int32_t antialias, float* means2d,
                    float* conics, float* depths, float* radii, float* compensation,
                    void* stream) {
    return project_fwd_impl<false>(cam, n, means, quats, scales, blur, antialias, means2d,
                                   conics, depths, radii, compensation, stream);
}

int gsx_project_bwd(const gsx_camera* cam, int64_t n, const float* means, const float* quats,
                    const float* scales, float blur, int32_t antialias, const float* g_means2d,
                    const float* g_conics, const float* g_depths, const float* g_compensation,
                    float* g_means, float* g_quats, float* g_scales, void* stream) {
    return project_bwd_impl<false>(cam, n, means, quats, scales, blur, antialias, g_means2d,
                                   g_conics, g_depths, g_compensation, g_means, g_quats,
                                   g_scales, stream);
}

int gsx_project_ut_fwd(const gsx_camera* cam, int64_t n, const float* means, const float* quats,
                       const float* scales, float blur, int32_t antialias, float* means2d,
                       float* conics, float* depths, float* radii, float* compensation,
                       void* stream) {
    return project_fwd_impl<true>(cam, n, means, quats, scales, blur, antialias, means2d,
                                  conics, depths, radii, compensation, stream);
}

int gsx_project_ut_bwd(const gsx_camera* cam, int64_t n, const float* means, const float* quats,
                       const float* scales, float blur, int32_t antialias,
                       const float* g_means2d, const float* g_conics, const float* g_depths,
                       const float* g_compensation, float* g_means, float* g_quats,
                       float* g_scales, void* stream) {
    return project_bwd_impl<true>(cam, n, means, quats, scales, blur, antialias, g_means2d,
                                  g_conics, g_depths, g_compensation, g_means, g_quats,
                                  g_scales, stream);
}

int gsx_eval_sh_fwd(int64_t n, int32_t K, int32_t C, int32_t degree, const float* sh,
                    const float* dirs, float* out, void* stream) {
    if (n < 0 || C <= 0 || degree < 0 || degree > 3 || K < (degree + 1) * (degree + 1))
        return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!sh || !dirs || !out) return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_eval_sh_fwd, dim3(grid_for(n * C)), dim3(kThreads), 0,
                       (hipStream_t)stream, n, K, C, degree, sh, dirs, out);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_eval_sh_bwd(int64_t n, int32_t K, int32_t C, int32_t degree, const float* sh,
                    const float* dirs, const float* g_out, float* g_sh, float* g_dirs,
                    void* stream) {
    if (n < 0 || C <= 0 || degree < 0 || degree > 3 || K < (degree + 1) * (degree + 1))
        return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!sh || !dirs || !g_out || !g_sh) return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_eval_sh_bwd, dim3(grid_for(n)), dim3(kThreads), 0, (hipStream_t)stream,
                       n, K, C, degree, sh, dirs, g_out, g_sh, g_dirs);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_preprocess_fwd(const gsx_camera* cam, int64_t n, const float* means, const float* quats,
                       const float* scales, const float* opacities, const float* sh0,
                       int64_t sh0_stride, const float* sh_rest, int64_t sh_rest_stride,
                       int32_t K, int32_t degree, uint32_t flags, float blur, float* means2d,
                       float* depths, float* radii, float* compensation, float* conic_opacity,
                       float* colors_out, uint32_t* tile_counts, uint32_t* depth_keys,
                       uint32_t* tile_rects, void* stream) {
    if (!cam || n < 0 || cam->width <= 0 || cam->height <= 0 || !lens_ok(cam))
        return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!means || !quats || !scales || !opacities || !means2d || !depths || !radii ||
        !compensation || !conic_opacity || !tile_counts || !depth_keys || !tile_rects)
        return GSX_ERR_INVALID;
    if (sh0) {
        if (degree < 0 || degree > 3 || K < (degree + 1) * (degree + 1) || !colors_out)
            return GSX_ERR_INVALID;
        if (K > 1 && !sh_rest) return GSX_ERR_INVALID;
    }
    if (!aligned16(quats) || !aligned16(conic_opacity) || !aligned8(means2d) ||
        !aligned8(tile_rects))
        return GSX_ERR_INVALID;
    const int tiles_x = (cam->width + kTile - 1) / kTile;
    const int tiles_y = (cam->height + kTile - 1) / kTile;
    int sh_mode = kShDirect, sh_cols = 1;
    if (sh0) {
        const int Ka = (degree + 1) * (degree + 1);
        if (sh_rest == sh0 + 3 && sh0_stride == sh_rest_stride && sh0_stride >= 3 * Ka &&
            3 * Ka <= kShMaxCols && Ka > 1) {
            sh_mode = kShPacked;  // one (N, K, 3) tensor: stage rows of 3 Ka floats
            sh_cols = 3 * Ka;
        } else if (Ka > 1 && 3 * (Ka - 1) <= kShMaxCols && sh_rest_stride >= 3 * (Ka - 1)) {
            sh_mode = kShSplit;  // separate DC / rest tensors: stage the rest rows
            sh_cols = 3 * (Ka - 1);
        }
    }
    auto kern = (flags & GSX_PROJECT_UT) ? k_preprocess_fwd<true> : k_preprocess_fwd<false>;
    hipLaunchKernelGGL(kern, dim3(grid_for(n)), dim3(kThreads), 0,
                       (hipStream_t)stream, *cam, n, means, (const float4*)quats, scales,
                       opacities, sh0, sh0_stride, sh_rest, sh_rest_stride, K, degree, sh_mode,
                       sh_cols, flags, blur, (flags & GSX_ANTIALIAS) != 0 && blur > 0.0f,
                       tiles_x, tiles_y,
                       (float2*)means2d, depths, radii, compensation, (float4*)conic_opacity,
                       colors_out, tile_counts, depth_keys, (uint2*)tile_rects);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_preprocess_bwd(const gsx_camera* cam, int64_t n, const float* means, const float* quats,
                       const float* scales, const float* opacities, const float* colors_out,
                       int32_t K, int32_t degree, uint32_t flags, float blur,
                       const float* g_means2d, const float* g_conics, const float* g_opac_eff,
                       const float* g_colors, const float* g_means2d_extra,
                       const float* g_depths, const float* g_compensation, float* g_means,
                       float* g_quats, float* g_scales, float* g_opacities, float* g_sh0,
                       int64_t sh0_stride, float* g_sh_rest, int64_t sh_rest_stride,
                       void* stream) {
    if (!cam || n < 0 || !lens_ok(cam)) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!means || !quats || !scales || !opacities || !g_means2d || !g_conics || !g_opac_eff ||
        !g_means || !g_quats || !g_scales || !g_opacities)
        return GSX_ERR_INVALID;
    if (g_sh0) {
        if (!colors_out || !g_colors || degree < 0 || degree > 3 ||
            K < (degree + 1) * (degree + 1))
            return GSX_ERR_INVALID;
        if (K > 1 && !g_sh_rest) return GSX_ERR_INVALID;
    }
    if (!aligned16(quats) || !aligned16(g_quats) || !aligned8(g_means2d) ||
        (g_means2d_extra && !aligned8(g_means2d_extra)))
        return GSX_ERR_INVALID;
    int sh_mode = kShDirect, sh_cols = 1;
    if (g_sh0) {
        if (g_sh_rest == g_sh0 + 3 && sh0_stride == sh_rest_stride && sh0_stride >= 3 * K &&
            3 * K <= kShMaxCols && K > 1) {
            sh_mode = kShPacked;
            sh_cols = 3 * K;
        } else if (K > 1 && 3 * (K - 1) <= kShMaxCols && sh_rest_stride >= 3 * (K - 1)) {
            sh_mode = kShSplit;
            sh_cols = 3 * (K - 1);
        }
    }
    auto kern = (flags & GSX_PROJECT_UT) ? k_preprocess_bwd<true> : k_preprocess_bwd<false>;
    hipLaunchKernelGGL(kern, dim3(grid_for(n)), dim3(kThreads), 0,
                       (hipStream_t)stream, *cam, n, means, (const float4*)quats, scales,
                       opacities, colors_out, K, degree, sh_mode, sh_cols, flags, blur,
                       (flags & GSX_ANTIALIAS) != 0 && blur > 0.0f, (const float2*)g_means2d,
                       g_conics, g_opac_eff, g_colors, (const float2*)g_means2d_extra, g_depths,
                       g_compensation, g_means, (float4*)g_quats, g_scales, g_opacities, g_sh0,
                       sh0_stride, g_sh_rest, sh_rest_stride);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_bin_prepare(int64_t n, const float* means2d, const float* radii, const float* depths,
                    int32_t width, int32_t height, uint32_t* tile_counts, uint32_t* depth_keys,
                    uint32_t* tile_rects, void* stream) {
    if (n < 0 || width <= 0 || height <= 0) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!means2d || !radii || !depths || !tile_counts || !depth_keys || !tile_rects)
        return GSX_ERR_INVALID;
    if (!aligned8(means2d) || !aligned8(tile_rects)) return GSX_ERR_INVALID;
    const int tiles_x = (width + kTile - 1) / kTile;
    const int tiles_y = (height + kTile - 1) / kTile;
    hipLaunchKernelGGL(k_bin_prepare, dim3(grid_for(n)), dim3(kThreads), 0, (hipStream_t)stream,
                       n, (const float2*)means2d, radii, depths, width, height, tiles_x, tiles_y,
                       tile_counts, depth_keys, (uint2*)tile_rects);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_pack_conic_opacity(int64_t n, const float* conics, const float* opacities,
                           float* conic_opacity, void* stream) {
    if (n < 0) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!conics || !opacities || !conic_opacity || !aligned16(conic_opacity))
        return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_pack_conic_opacity, dim3(grid_for(n)), dim3(kThreads), 0,
                       (hipStream_t)stream, n, conics, opacities, (float4*)conic_opacity);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_debug_atanf(int64_t n, const float* x, float* y, void* stream) {
    if (n < 0) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!x || !y) return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_debug_atanf, dim3(grid_for(n)), dim3(kThreads), 0, (hipStream_t)stream,
                       n, x, y);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_debug_expf(int64_t n, const float* x, float* y, void* stream) {
    if (n < 0) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!x || !y) return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_debug_expf, dim3(grid_for(n)), dim3(kThreads), 0, (hipStream_t)stream,
                       n, x, y);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // extern "C"
