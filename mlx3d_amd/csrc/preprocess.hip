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

// Cache-policy operand of the direct-to-LDS load builtin: the non-temporal
// bit (the rows are read once; measured on MI355X at C3: 66.2 -> 62.4 us for
// the preprocess forward, bit-identical results).
constexpr int kCachePolicyNT = 2;

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
                (__attribute__((address_space(3))) void*)(s + 4 * b4), 16, 0, kCachePolicyNT);
    }
    const int t = 4 * n4 + (int)threadIdx.x;
    if (t < total) s[t] = src[t];
}

// Non-temporal 16-byte accesses for data touched once per call.
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 stream_load(const float4* p) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void stream_store(float4* p, float4 a) {
    const f32x4 v = {a.x, a.y, a.z, a.w};
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
}

// Contiguous rows the other way: `total` floats of an unpadded LDS copy (16-
// byte aligned) out to dst (16-byte aligned) as non-temporal float4 stores,
// the < 4 tail floats one by one.
__device__ __forceinline__ void lds_to_rows_direct(const float* s, float* __restrict__ dst,
                                                   int total) {
    const int n4 = total >> 2;
    const float4* s4 = reinterpret_cast<const float4*>(s);
    float4* d4 = reinterpret_cast<float4*>(dst);
    for (int j = threadIdx.x; j < n4; j += kThreads) stream_store(d4 + j, s4[j]);
    const int t = 4 * n4 + (int)threadIdx.x;
    if (t < total) dst[t] = s[t];
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
    // binned Gaussians have z > znear: the key is the distance from the
    // near plane in orderable float bits (small for every realistic depth)
    dkeys[i] = cnt ? depth_key(p.z) - depth_key(cam.znear) : 0u;
    rects[i] = rect;
}

// Gradients of one Gaussian's stored parameters (means, quaternion, scales
// and opacity as stored, before the activations `flags` select) from the
// cotangents of the forward's outputs, and with SH the colour cotangent
// after the clamp mask (gc), the basis (bk) and the active count (Ka).
struct RawGrads {
    float means[3], quat[4], scales[3], opacity;
    float gc[3], bk[16];
    int Ka;
};

// The rasterizer's per-Gaussian gradients: four arrays (means2d (N,2),
// conics (N,3), effective opacity (N), colours (N,3)), or with stride > 0 one
// record of `stride` floats per Gaussian, [means2d 2 | conic 3 | opacity 1 |
// colour 3 | ...], 16-byte aligned (read as three float4).
struct RasterGrads {
    const float* m2;
    const float* con;
    const float* op;
    const float* col;
    int stride;
};

struct GradRow {
    float gx, gy, ga, gb, gc, go;
    float col[3];
};

__device__ __forceinline__ GradRow load_grads(const RasterGrads& g, int64_t i, bool sh) {
    GradRow r;
    if (g.stride > 0) {
        const float4* p = reinterpret_cast<const float4*>(g.m2 + (int64_t)g.stride * i);
        const float4 a = p[0], b = p[1];
        r.gx = a.x;
        r.gy = a.y;
        r.ga = a.z;
        r.gb = a.w;
        r.gc = b.x;
        r.go = b.y;
        r.col[0] = b.z;
        r.col[1] = b.w;
        r.col[2] = sh ? p[2].x : 0.0f;
    } else {
        const float2 m = reinterpret_cast<const float2*>(g.m2)[i];
        r.gx = m.x;
        r.gy = m.y;
        r.ga = g.con[3 * i];
        r.gb = g.con[3 * i + 1];
        r.gc = g.con[3 * i + 2];
        r.go = g.op[i];
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) r.col[ch] = sh ? g.col[3 * i + ch] : 0.0f;
    }
    return r;
}

template <bool UT>
__device__ __forceinline__ void preprocess_vjp(
    const gsx_camera& cam, int64_t i, float m0, float m1, float m2, float4 q, float r0, float r1,
    float r2, float ro, uint32_t flags, float blur, bool aa, bool sh, int degree,
    const float* __restrict__ colors_out, const RasterGrads& rg,
    const float2* __restrict__ g_means2d_extra, const float* __restrict__ g_depths,
    const float* __restrict__ g_comp, RawGrads& G) {
    const float sx = act_scale(r0, flags);
    const float sy = act_scale(r1, flags);
    const float sz = act_scale(r2, flags);
    const float o = act_opacity(ro, flags);
    typename ProjOf<UT>::T p;
    project_any<UT>(cam, m0, m1, m2, q.x, q.y, q.z, q.w, sx, sy, sz, blur, aa, p);
    const GradRow gr = load_grads(rg, i, sh);
    const float goe = gr.go;
    const float g_o = goe * p.comp;
    const float g_comp_total = (g_comp ? g_comp[i] : 0.0f) + goe * o;
    float2 gm2 = make_float2(gr.gx, gr.gy);
    if (g_means2d_extra) {
        const float2 e = g_means2d_extra[i];
        gm2.x += e.x;
        gm2.y += e.y;
    }
    float gs[3];
    project_any_vjp<UT>(cam, p, m0, m1, m2, aa, gm2.x, gm2.y, gr.ga, gr.gb, gr.gc,
                        g_depths ? g_depths[i] : 0.0f, g_comp_total, G.means, G.quat, gs);
    const bool ls = flags & GSX_LOG_SCALES;
    G.scales[0] = ls ? gs[0] * sx : gs[0];
    G.scales[1] = ls ? gs[1] * sy : gs[1];
    G.scales[2] = ls ? gs[2] * sz : gs[2];
    G.opacity = (flags & GSX_LOGIT_OPACITY) ? g_o * o * (1.0f - o) : g_o;
    G.Ka = 0;
    if (sh) {
        float dx, dy, dz;
        view_dir(cam, m0, m1, m2, dx, dy, dz);
        sh_basis(degree, dx, dy, dz, G.bk);
        G.Ka = (degree + 1) * (degree + 1);
#pragma unroll
        for (int ch = 0; ch < 3; ++ch)
            G.gc[ch] = (colors_out[3 * i + ch] > 0.0f) ? gr.col[ch] : 0.0f;
    }
}

// The SH coefficient gradients bk[k] gc (zero for k >= Ka) of coefficients
// k0 .. K - 1 into dst[3 (k - k0) + ch].  The basis is indexed with
// compile-time constants (a runtime index would move it to scratch); the
// coefficients past 16 have no basis value, their gradient is zero.
__device__ __forceinline__ void sh_grad_rows(const RawGrads& G, int K, int k0, float* dst) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        if (k < k0 || k >= K) continue;
        const float bv = (k < G.Ka) ? G.bk[k] : 0.0f;
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) dst[3 * (k - k0) + ch] = bv * G.gc[ch];
    }
    for (int k = 16; k < K; ++k)
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) dst[3 * (k - k0) + ch] = 0.0f;
}

// VJP of k_preprocess_fwd, one Gaussian per lane.  SH gradients (zero for
// coefficients >= Ka) are written through LDS rows in the same sh_mode
// layouts as the forward reads.
template <bool UT>
__global__ __launch_bounds__(kThreads) void k_preprocess_bwd(
    gsx_camera cam, int64_t n, const float* __restrict__ means, const float4* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ opacities,
    const float* __restrict__ colors_out, int K, int degree, int sh_mode, int sh_cols,
    uint32_t flags, float blur, bool aa, RasterGrads rg,
    const float2* __restrict__ g_means2d_extra,
    const float* __restrict__ g_depths, const float* __restrict__ g_comp,
    float* __restrict__ g_means, float4* __restrict__ g_quats, float* __restrict__ g_scales,
    float* __restrict__ g_opacities, float* __restrict__ g_sh0, int64_t s0,
    float* __restrict__ g_shr, int64_t sr) {
    __shared__ __align__(16) float s_sh[kThreads * kShPad];
    const int64_t g0 = (int64_t)blockIdx.x * kThreads;
    const int64_t i = g0 + threadIdx.x;
    const int pad = sh_cols | 1;
    if (i < n) {
        RawGrads G;
        preprocess_vjp<UT>(cam, i, means[3 * i], means[3 * i + 1], means[3 * i + 2], quats[i],
                           scales[3 * i], scales[3 * i + 1], scales[3 * i + 2], opacities[i],
                           flags, blur, aa, g_sh0 != nullptr, degree, colors_out, rg,
                           g_means2d_extra, g_depths, g_comp, G);
        g_means[3 * i] = G.means[0];
        g_means[3 * i + 1] = G.means[1];
        g_means[3 * i + 2] = G.means[2];
        g_quats[i] = make_float4(G.quat[0], G.quat[1], G.quat[2], G.quat[3]);
        g_scales[3 * i] = G.scales[0];
        g_scales[3 * i + 1] = G.scales[1];
        g_scales[3 * i + 2] = G.scales[2];
        g_opacities[i] = G.opacity;
        if (g_sh0) {
            float* row = s_sh + threadIdx.x * pad;
            if (sh_mode == kShPacked) {
                sh_grad_rows(G, K, 0, row);
            } else {
                float* a = g_sh0 + i * s0;
#pragma unroll
                for (int ch = 0; ch < 3; ++ch) a[ch] = G.bk[0] * G.gc[ch];
                sh_grad_rows(G, K, 1, sh_mode == kShSplit ? row : g_shr + i * sr);
            }
        }
    }
    if (sh_mode != kShDirect) {
        __syncthreads();
        const int rows = (int)min<int64_t>(kThreads, n - g0);
        float* base = sh_mode == kShPacked ? g_sh0 : g_shr;
        const int64_t stride = sh_mode == kShPacked ? s0 : sr;
        // contiguous unpadded rows (odd width) into a 16-byte aligned block:
        // the block is one run of floats, written as non-temporal float4
        // (measured on MI355X at C3: 98.7 -> 71.4 us for this kernel)
        if (stride == sh_cols && pad == sh_cols &&
            ((uintptr_t)(base + g0 * stride) & 15u) == 0u)
            lds_to_rows_direct(s_sh, base + g0 * stride, rows * sh_cols);
        else
            lds_to_rows(s_sh, pad, base, stride, g0, rows, sh_cols);
    }
}

// The six parameter groups' Adam state for k_preprocess_bwd_adam, in the
// trainer's order: means, quats, scales, opacities, SH DC, SH rest.
struct AdamState6 {
    float* m[6];
    float* v[6];
    float lr[6];
};

// One Adam update of a parameter whose value p the lane holds already; the
// moments are read and written at M[k], V[k].  Returns the new value.
__device__ __forceinline__ float adam_reg(float p, float* __restrict__ M, float* __restrict__ V,
                                          int64_t k, float g, float lr, float b1, float omb1,
                                          float b2, float omb2, float eps) {
    float m = M[k], v = V[k];
    adam_update(p, g, m, v, lr, b1, omb1, b2, omb2, eps);
    M[k] = m;
    V[k] = v;
    return p;
}

__device__ __forceinline__ void adam4(float4& p, float4& m, float4& v, float4 g, float lr,
                                      float b1, float omb1, float b2, float omb2, float eps) {
    adam_update(p.x, g.x, m.x, v.x, lr, b1, omb1, b2, omb2, eps);
    adam_update(p.y, g.y, m.y, v.y, lr, b1, omb1, b2, omb2, eps);
    adam_update(p.z, g.z, m.z, v.z, lr, b1, omb1, b2, omb2, eps);
    adam_update(p.w, g.w, m.w, v.w, lr, b1, omb1, b2, omb2, eps);
}

// The SH rest gradient of a Gaussian is rank one: coefficient k, channel ch
// has bv(k) gc[ch] with bv(k) = bk[k] (0 from Ka on).  A workgroup stages
// each lane's bv(1 .. 16) and gc(0 .. 2) as one LDS row of kRank1Stride
// floats (odd, so each lane's own row hits distinct banks), and the SH rest
// block is then streamed against it.
constexpr int kRank1Stride = 19;

__device__ __forceinline__ void stage_rank1(const RawGrads& G, float* row) {
#pragma unroll
    for (int k = 1; k < 16; ++k) row[k - 1] = (k < G.Ka) ? G.bk[k] : 0.0f;
    row[15] = 0.0f;
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) row[16 + ch] = G.gc[ch];
}

// Gradient of SH rest column c (coefficient c / 3 + 1, channel c % 3) of a
// staged row: the product sh_grad_rows forms (coefficient 16 has no basis
// value and a gradient of +0, as there).
__device__ __forceinline__ float rank1_grad(const float* row, int c) {
    const int k1 = c / 3, ch = c - 3 * k1;
    return k1 == 15 ? 0.0f : row[k1] * row[16 + ch];
}

// Gradients of elements e .. e + 3 of a workgroup's SH rest block (row-major,
// `cols` per row).
__device__ __forceinline__ float4 rank1_grad4(const float* s, int e, int cols, float inv) {
    int r, c;
    row_col(e, cols, inv, r, c);
    float g[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        g[u] = rank1_grad(s + r * kRank1Stride, c);
        if (++c == cols) {
            c = 0;
            ++r;
        }
    }
    return make_float4(g[0], g[1], g[2], g[3]);
}

// The SH rest parameters and moments are read and written once per step, far
// more data than the caches hold: non-temporal 16-byte loads and stores keep
// the stream from evicting other data (measured on MI355X at 1M Gaussians,
// K = 16: 297 -> 241 us for the fused kernel; the same on the stride-3
// per-Gaussian moments made it slower, 339 us).  kStreamPieces 16-byte
// pieces per lane are in flight at once (1: 277 us, 2: 242, 4: 238).
constexpr int kStreamPieces = 4;

// k_preprocess_bwd followed by the Adam update of every parameter, fused:
// each lane's gradients stay in registers and go straight into the update
// of its Gaussian's parameters and moments, instead of being written out and
// read back by a separate Adam launch.  The SH rest gradients' rank-one
// factors go through LDS, and the workgroup then streams its contiguous
// block of SH rest parameters and moments in 16-byte pieces (vec: all three
// 16-byte aligned; otherwise element by element).  Parameters are read and
// updated in place: each lane reads its own Gaussian's inputs before it
// writes them, and no other lane reads them.  SH in split layout, contiguous rows: sh0 (N, 3),
// shr (N, 3 (K - 1)); the moments share the parameters' layouts, the
// quaternion moments 16-byte aligned.
template <bool UT>
__global__ __launch_bounds__(kThreads) void k_preprocess_bwd_adam(
    gsx_camera cam, int64_t n, float* __restrict__ means, float4* __restrict__ quats,
    float* __restrict__ scales, float* __restrict__ opacities, float* __restrict__ sh0,
    float* __restrict__ shr, int K, int degree, uint32_t flags, float blur, bool aa, bool vec,
    const float* __restrict__ colors_out, RasterGrads rg,
    const float2* __restrict__ g_means2d_extra,
    const float* __restrict__ g_depths, const float* __restrict__ g_comp, AdamState6 st,
    float b1, float omb1, float b2, float omb2, float eps) {
    __shared__ float s_r1[kThreads * kRank1Stride];
    const int64_t g0 = (int64_t)blockIdx.x * kThreads;
    const int64_t i = g0 + threadIdx.x;
    const int cols = 3 * (K - 1);
    if (i < n) {
        const float pm[3] = {means[3 * i], means[3 * i + 1], means[3 * i + 2]};
        const float4 q = quats[i];
        const float ps[3] = {scales[3 * i], scales[3 * i + 1], scales[3 * i + 2]};
        const float ro = opacities[i];
        RawGrads G;
        preprocess_vjp<UT>(cam, i, pm[0], pm[1], pm[2], q, ps[0], ps[1], ps[2], ro, flags, blur,
                           aa, true, degree, colors_out, rg, g_means2d_extra, g_depths, g_comp,
                           G);
#pragma unroll
        for (int k = 0; k < 3; ++k)
            means[3 * i + k] = adam_reg(pm[k], st.m[0], st.v[0], 3 * i + k, G.means[k], st.lr[0],
                                        b1, omb1, b2, omb2, eps);
        {
            float4 p = q;
            float4 m = reinterpret_cast<float4*>(st.m[1])[i];
            float4 v = reinterpret_cast<float4*>(st.v[1])[i];
            adam4(p, m, v, make_float4(G.quat[0], G.quat[1], G.quat[2], G.quat[3]), st.lr[1], b1,
                  omb1, b2, omb2, eps);
            quats[i] = p;
            reinterpret_cast<float4*>(st.m[1])[i] = m;
            reinterpret_cast<float4*>(st.v[1])[i] = v;
        }
#pragma unroll
        for (int k = 0; k < 3; ++k)
            scales[3 * i + k] = adam_reg(ps[k], st.m[2], st.v[2], 3 * i + k, G.scales[k],
                                         st.lr[2], b1, omb1, b2, omb2, eps);
        opacities[i] = adam_reg(ro, st.m[3], st.v[3], i, G.opacity, st.lr[3], b1, omb1, b2, omb2,
                                eps);
        float pd[3];
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) pd[ch] = sh0[3 * i + ch];
#pragma unroll
        for (int ch = 0; ch < 3; ++ch)
            sh0[3 * i + ch] = adam_reg(pd[ch], st.m[4], st.v[4], 3 * i + ch, G.bk[0] * G.gc[ch],
                                       st.lr[4], b1, omb1, b2, omb2, eps);
        stage_rank1(G, s_r1 + threadIdx.x * kRank1Stride);
    }
    if (cols > 0) {
        __syncthreads();
        const int rows = (int)min<int64_t>(kThreads, n - g0);
        const int total = rows * cols;
        const float inv = 1.0f / (float)cols;
        float* __restrict__ P = shr + g0 * cols;
        float* __restrict__ M = st.m[5] + g0 * cols;
        float* __restrict__ V = st.v[5] + g0 * cols;
        const float lr = st.lr[5];
        int done = 0;
        if (vec) {  // g0 cols is a multiple of 4 (g0 of kThreads), the block 16-byte aligned
            float4* P4 = reinterpret_cast<float4*>(P);
            float4* M4 = reinterpret_cast<float4*>(M);
            float4* V4 = reinterpret_cast<float4*>(V);
            const int total4 = total >> 2;
            for (int j = threadIdx.x; j < total4; j += kStreamPieces * kThreads) {
                // loads of every piece are unconditional (a piece past the end
                // re-reads the first), its stores guarded
                int jj[kStreamPieces];
                float4 pp[kStreamPieces], mm[kStreamPieces], vv[kStreamPieces];
#pragma unroll
                for (int u = 0; u < kStreamPieces; ++u) {
                    jj[u] = j + u * kThreads < total4 ? j + u * kThreads : j;
                    pp[u] = stream_load(P4 + jj[u]);
                    mm[u] = stream_load(M4 + jj[u]);
                    vv[u] = stream_load(V4 + jj[u]);
                }
#pragma unroll
                for (int u = 0; u < kStreamPieces; ++u)
                    adam4(pp[u], mm[u], vv[u], rank1_grad4(s_r1, 4 * jj[u], cols, inv), lr, b1,
                          omb1, b2, omb2, eps);
#pragma unroll
                for (int u = 0; u < kStreamPieces; ++u)
                    if (u == 0 || j + u * kThreads < total4) {
                        stream_store(P4 + jj[u], pp[u]);
                        stream_store(M4 + jj[u], mm[u]);
                        stream_store(V4 + jj[u], vv[u]);
                    }
            }
            done = total4 << 2;
        }
        for (int e = done + threadIdx.x; e < total; e += kThreads) {
            int r, c;
            row_col(e, cols, inv, r, c);
            P[e] = adam_reg(P[e], M, V, e, rank1_grad(s_r1 + r * kRank1Stride, c), lr, b1, omb1,
                            b2, omb2, eps);
        }
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
    dkeys[i] = cnt ? depth_key(depths[i]) : 0u;
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

}  // extern "C"

namespace {
// The rasterizer gradients of gsx_preprocess_bwd(_adam): grad_stride 0 =
// four arrays, > 0 = one record per Gaussian at g_means2d (the other three
// pointers NULL).  Returns false for an invalid combination.
bool raster_grads(const float* g_means2d, const float* g_conics, const float* g_opac_eff,
                  const float* g_colors, int32_t grad_stride, bool sh, RasterGrads& rg) {
    rg = RasterGrads{g_means2d, g_conics, g_opac_eff, g_colors, grad_stride};
    if (!g_means2d || grad_stride < 0) return false;
    if (grad_stride > 0)
        return grad_stride % 4 == 0 && grad_stride >= (sh ? 12 : 8) && aligned16(g_means2d) &&
               !g_conics && !g_opac_eff && !g_colors;
    return g_conics && g_opac_eff && (!sh || g_colors) && aligned8(g_means2d);
}
}  // namespace

extern "C" {

int gsx_preprocess_bwd_adam(const gsx_camera* cam, int64_t n, float* means, float* quats,
                            float* scales, float* opacities, float* sh_dc, float* sh_rest,
                            const float* colors_out, int32_t K, int32_t degree, uint32_t flags,
                            float blur, const float* g_means2d, const float* g_conics,
                            const float* g_opac_eff, const float* g_colors,
                            const float* g_means2d_extra, const float* g_depths,
                            const float* g_compensation, const gsx_adam_group* groups,
                            float beta1, float beta2, float eps, int32_t grad_stride,
                            void* stream) {
    if (!cam || n < 0 || !lens_ok(cam) || !groups) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    RasterGrads rg;
    if (!means || !quats || !scales || !opacities || !sh_dc || !colors_out ||
        !raster_grads(g_means2d, g_conics, g_opac_eff, g_colors, grad_stride, true, rg))
        return GSX_ERR_INVALID;
    if (degree < 0 || degree > 3 || K < (degree + 1) * (degree + 1) ||
        3 * (K - 1) > kShMaxCols || (K > 1 && !sh_rest))
        return GSX_ERR_INVALID;
    // the groups name the same tensors, with the element counts of their layouts
    float* const params[6] = {means, quats, scales, opacities, sh_dc, sh_rest};
    const int64_t counts[6] = {3 * n, 4 * n, 3 * n, n, 3 * n, 3 * (int64_t)(K - 1) * n};
    AdamState6 st;
    for (int k = 0; k < 6; ++k) {
        if (k == 5 && K == 1) {
            st.m[k] = st.v[k] = nullptr;
            st.lr[k] = 0.0f;
            continue;
        }
        if (groups[k].param != params[k] || groups[k].n != counts[k] || !groups[k].m ||
            !groups[k].v)
            return GSX_ERR_INVALID;
        st.m[k] = groups[k].m;
        st.v[k] = groups[k].v;
        st.lr[k] = groups[k].lr;
    }
    if (!aligned16(quats) || !aligned16(st.m[1]) || !aligned16(st.v[1]) ||
        (g_means2d_extra && !aligned8(g_means2d_extra)))
        return GSX_ERR_INVALID;
    const bool vec = K > 1 && aligned16(sh_rest) && aligned16(st.m[5]) && aligned16(st.v[5]);
    // b1, 1 - b1, b2, 1 - b2 in float32 as gsx_adam_step rounds them
    const float b1 = beta1, omb1 = (float)(1.0 - (double)beta1);
    const float b2 = beta2, omb2 = (float)(1.0 - (double)beta2);
    auto kern = (flags & GSX_PROJECT_UT) ? k_preprocess_bwd_adam<true>
                                         : k_preprocess_bwd_adam<false>;
    hipLaunchKernelGGL(kern, dim3(grid_for(n)), dim3(kThreads), 0, (hipStream_t)stream, *cam, n,
                       means, (float4*)quats, scales, opacities, sh_dc, sh_rest, K, degree, flags,
                       blur, (flags & GSX_ANTIALIAS) != 0 && blur > 0.0f, vec, colors_out, rg,
                       (const float2*)g_means2d_extra, g_depths, g_compensation, st, b1, omb1,
                       b2, omb2, eps);
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
                       int32_t grad_stride, void* stream) {
    if (!cam || n < 0 || !lens_ok(cam)) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    RasterGrads rg;
    if (!means || !quats || !scales || !opacities || !g_means || !g_quats || !g_scales ||
        !g_opacities ||
        !raster_grads(g_means2d, g_conics, g_opac_eff, g_colors, grad_stride, g_sh0 != nullptr,
                      rg))
        return GSX_ERR_INVALID;
    if (g_sh0) {
        if (!colors_out || degree < 0 || degree > 3 || K < (degree + 1) * (degree + 1))
            return GSX_ERR_INVALID;
        if (K > 1 && !g_sh_rest) return GSX_ERR_INVALID;
    }
    if (!aligned16(quats) || !aligned16(g_quats) ||
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
                       (flags & GSX_ANTIALIAS) != 0 && blur > 0.0f, rg,
                       (const float2*)g_means2d_extra, g_depths,
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
