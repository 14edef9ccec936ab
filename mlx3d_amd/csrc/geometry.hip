// geometry.hip -- the 2DGS geometry regularisers of the training step
// (splatting/trainer.py:187-259) as two kernel pairs.
//
//  1. Per-Gaussian features (N, 5) = (z, z^2, s n): n the third column of
//     the rotation of the normalised quaternion (the surfel normal),
//     normalised again, s = -1 when n points away from the camera
//     (n . (centre - mean) < 0) so every normal faces the viewer.  Its VJP
//     sends the feature cotangent to the depths and the quaternions (the
//     flip has zero derivative).
//  2. The per-pixel losses on the alpha-normalised feature render F (H, W, 5)
//     = (expected depth, expected depth^2, normal) and alpha:
//       depth variance   mean over pixels with alpha > min_alpha of
//                        max(E[z^2] - E[z]^2, 0);
//       normal agreement mean over 2x2 pixel quads whose four pixels pass of
//                        1 - |n_render . n_depth|, n_depth the normal of the
//                        surface the expected depths span: the cross product
//                        of the world-space differences to the right and
//                        lower neighbours of the unprojected pixel centre.
//     Unprojection is affine in depth, P = base + z dir per pixel (perspective:
//     base = camera centre, dir = R^T (undistorted x, y, 1); orthographic:
//     base on the image plane, dir = the view axis), so one pair of maps
//     serves every camera model.  The forward writes per-workgroup partial
//     sums reduced in double in a fixed order; the backward gives each pixel
//     its own cotangent by re-evaluating the (at most three) quads its point
//     belongs to -- no atomics, deterministic.
#include <hip/hip_runtime.h>

#include <cmath>

#include "gsx.h"
#include "gsx_device.h"

using namespace gsx;

namespace {

constexpr int kThreads = 256;

struct V3 {
    float x, y, z;
};
__device__ __forceinline__ V3 v3(float x, float y, float z) { return V3{x, y, z}; }
__device__ __forceinline__ V3 operator+(V3 a, V3 b) { return v3(a.x + b.x, a.y + b.y, a.z + b.z); }
__device__ __forceinline__ V3 operator-(V3 a, V3 b) { return v3(a.x - b.x, a.y - b.y, a.z - b.z); }
__device__ __forceinline__ V3 operator*(float s, V3 a) { return v3(s * a.x, s * a.y, s * a.z); }
__device__ __forceinline__ float dot(V3 a, V3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
__device__ __forceinline__ V3 cross(V3 a, V3 b) {
    return v3(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
__device__ __forceinline__ float norm(V3 a) { return sqrtf(dot(a, a)); }
__device__ __forceinline__ V3 load3(const float* p) { return v3(p[0], p[1], p[2]); }

// v / max(|v|, 1e-8) and its VJP: for |v| > 1e-8, (g - u (u . g)) / |v|;
// otherwise the divisor is the constant and the VJP is g / 1e-8.
__device__ __forceinline__ V3 unit(V3 v, float& len) {
    len = norm(v);
    return (1.0f / fmaxf(len, 1e-8f)) * v;
}
__device__ __forceinline__ V3 unit_vjp(V3 u, float len, V3 g) {
    if (len > 1e-8f) return (1.0f / len) * (g - dot(u, g) * u);
    return (1.0f / 1e-8f) * g;
}

// ------------------------------------------------------------ features --
__device__ __forceinline__ V3 surfel_axis(float w, float x, float y, float z) {
    // third column of the rotation matrix (rotations.py:30-49)
    return v3(2.0f * (x * z + w * y), 2.0f * (y * z - w * x), 1.0f - 2.0f * (x * x + y * y));
}

__global__ __launch_bounds__(kThreads) void k_geom_features(
    int64_t n, const float* __restrict__ means, const float4* __restrict__ quats,
    const float* __restrict__ depths, float cx, float cy, float cz, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float4 q = quats[i];
    const float qn = sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w);
    const V3 col = surfel_axis(q.x / qn, q.y / qn, q.z / qn, q.w / qn);
    float len;
    V3 nrm = unit(col, len);
    const V3 view = v3(cx - means[3 * i], cy - means[3 * i + 1], cz - means[3 * i + 2]);
    if (dot(nrm, view) < 0.0f) nrm = v3(-nrm.x, -nrm.y, -nrm.z);
    const float z = depths[i];
    float* o = out + 5 * i;
    o[0] = z;
    o[1] = z * z;
    o[2] = nrm.x;
    o[3] = nrm.y;
    o[4] = nrm.z;
}

__global__ __launch_bounds__(kThreads) void k_geom_features_bwd(
    int64_t n, const float* __restrict__ means, const float4* __restrict__ quats,
    const float* __restrict__ depths, float cx, float cy, float cz,
    const float* __restrict__ g_feat, float* __restrict__ g_depths, float4* __restrict__ g_quats) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float* g = g_feat + 5 * i;
    const float z = depths[i];
    g_depths[i] = g[0] + 2.0f * z * g[1];
    const float4 q = quats[i];
    const float qn = sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w);
    const float w = q.x / qn, x = q.y / qn, y = q.z / qn, zq = q.w / qn;
    const V3 col = surfel_axis(w, x, y, zq);
    float len;
    const V3 nrm = unit(col, len);
    const V3 view = v3(cx - means[3 * i], cy - means[3 * i + 1], cz - means[3 * i + 2]);
    const float s = dot(nrm, view) < 0.0f ? -1.0f : 1.0f;
    const V3 gn = s * v3(g[2], g[3], g[4]);
    const V3 gc = unit_vjp(nrm, len, gn);
    // d col / d (w, x, y, z) transposed onto gc
    const float gw = 2.0f * y * gc.x - 2.0f * x * gc.y;
    const float gx = 2.0f * zq * gc.x - 2.0f * w * gc.y - 4.0f * x * gc.z;
    const float gy = 2.0f * w * gc.x + 2.0f * zq * gc.y - 4.0f * y * gc.z;
    const float gz = 2.0f * x * gc.x + 2.0f * y * gc.y;
    // through the normalisation q / |q|
    const float d = w * gw + x * gx + y * gy + zq * gz;
    g_quats[i] = make_float4((gw - w * d) / qn, (gx - x * d) / qn, (gy - y * d) / qn,
                             (gz - zq * d) / qn);
}

// --------------------------------------------------------------- losses --
struct GeomMaps {
    const float* F;      // (H, W, 5)
    const float* alpha;  // (H, W)
    const float* base;   // (H, W, 3)
    const float* dir;    // (H, W, 3)
    int W, H;
    float min_alpha;
};

__device__ __forceinline__ bool valid_at(const GeomMaps& m, int y, int x) {
    return m.alpha[(int64_t)y * m.W + x] > m.min_alpha;
}
__device__ __forceinline__ V3 point_at(const GeomMaps& m, int y, int x) {
    const int64_t p = (int64_t)y * m.W + x;
    return load3(m.base + 3 * p) + m.F[5 * p] * load3(m.dir + 3 * p);
}

// All four pixels of the quad with top-left pixel (y, x) pass the alpha test.
__device__ __forceinline__ bool quad_valid(const GeomMaps& m, int y, int x) {
    return valid_at(m, y, x) && valid_at(m, y, x + 1) && valid_at(m, y + 1, x) &&
           valid_at(m, y + 1, x + 1);
}

// The 1 - |cos| term of a valid quad and, with qg, the cotangents of its three
// points and of the rendered normal at (y, x) for a term weight gw.
struct QuadGrad {
    V3 g00, g01, g10, gr;
};
__device__ __forceinline__ float quad_term(const GeomMaps& m, int y, int x, float gw,
                                           QuadGrad* qg) {
    const V3 p00 = point_at(m, y, x), p01 = point_at(m, y, x + 1), p10 = point_at(m, y + 1, x);
    const V3 tx = p01 - p00, ty = p10 - p00;
    const V3 c = cross(tx, ty);
    float lc, lr;
    const V3 dn = unit(c, lc);
    const int64_t p = (int64_t)y * m.W + x;
    const V3 r = load3(m.F + 5 * p + 2);
    const V3 rn = unit(r, lr);
    const float cs = dot(rn, dn);
    if (qg) {
        const float gcos = cs > 0.0f ? -gw : (cs < 0.0f ? gw : 0.0f);  // d(1 - |cos|)
        const V3 gc = unit_vjp(dn, lc, gcos * rn);
        qg->gr = unit_vjp(rn, lr, gcos * dn);
        const V3 gtx = cross(ty, gc), gty = cross(gc, tx);
        qg->g01 = gtx;
        qg->g10 = gty;
        qg->g00 = v3(-(gtx.x + gty.x), -(gtx.y + gty.y), -(gtx.z + gty.z));
    }
    return 1.0f - fabsf(cs);
}

// Per-workgroup partial sums (depth-variance sum, valid pixels, normal sum,
// valid quads) over a 16 x 16 pixel tile.
__global__ __launch_bounds__(kThreads) void k_geom_loss_partial(GeomMaps m, int use_dv,
                                                                int use_nc,
                                                                float* __restrict__ partials) {
    __shared__ float s_red[4][kThreads / kWave];
    const int tiles_x = (m.W + 15) / 16;
    const int tx = blockIdx.x % tiles_x, ty = blockIdx.x / tiles_x;
    const int x = tx * 16 + (threadIdx.x & 15), y = ty * 16 + (threadIdx.x >> 4);
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (x < m.W && y < m.H) {
        const bool v = valid_at(m, y, x);
        if (use_dv && v) {
            const int64_t p = (int64_t)y * m.W + x;
            const float ed = m.F[5 * p], ed2 = m.F[5 * p + 1];
            a[0] = fmaxf(ed2 - ed * ed, 0.0f);
            a[1] = 1.0f;
        }
        if (use_nc && x < m.W - 1 && y < m.H - 1 && quad_valid(m, y, x)) {
            a[2] = quad_term(m, y, x, 0.0f, nullptr);
            a[3] = 1.0f;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float s = wave_sum(a[k]);
        if (lane == 0) s_red[k][wave] = s;
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < kThreads / kWave; ++w) t += s_red[threadIdx.x][w];
        partials[4 * (int64_t)blockIdx.x + threadIdx.x] = t;
    }
}

// out = [loss, depth variance, normal term, max(valid pixels, 1),
// max(valid quads, 1)]; sums in double in a fixed order.
__global__ __launch_bounds__(256) void k_geom_loss_reduce(const float* __restrict__ partials,
                                                          int64_t nblk, float lam_dv,
                                                          float lam_nc, int use_dv, int use_nc,
                                                          float* __restrict__ out) {
    __shared__ double s[4][256];
    double a[4] = {0.0, 0.0, 0.0, 0.0};
    for (int64_t i = threadIdx.x; i < nblk; i += 256)
        for (int k = 0; k < 4; ++k) a[k] += (double)partials[4 * i + k];
    for (int k = 0; k < 4; ++k) s[k][threadIdx.x] = a[k];
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w)
            for (int k = 0; k < 4; ++k) s[k][threadIdx.x] += s[k][threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float den_dv = fmaxf((float)s[1][0], 1.0f), den_nc = fmaxf((float)s[3][0], 1.0f);
        const float dv = use_dv ? (float)s[0][0] / den_dv : 0.0f;
        const float nc = use_nc ? (float)s[2][0] / den_nc : 0.0f;
        out[0] = (use_dv ? lam_dv * dv : 0.0f) + (use_nc ? lam_nc * nc : 0.0f);
        out[1] = dv;
        out[2] = nc;
        out[3] = den_dv;
        out[4] = den_nc;
    }
}

__global__ __launch_bounds__(kThreads) void k_geom_loss_bwd(GeomMaps m, int use_dv, int use_nc,
                                                            float lam_dv, float lam_nc,
                                                            const float* __restrict__ fwd_out,
                                                            const float* __restrict__ g_loss,
                                                            float* __restrict__ g_F) {
    const int64_t p = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (p >= (int64_t)m.W * m.H) return;
    const int y = (int)(p / m.W), x = (int)(p - (int64_t)y * m.W);
    const float g = g_loss[0];
    float g0 = 0.0f, g1 = 0.0f;
    V3 gr = v3(0.0f, 0.0f, 0.0f);
    if (use_dv && valid_at(m, y, x)) {
        const float c = lam_dv * g / fwd_out[3];
        const float ed = m.F[5 * p], ed2 = m.F[5 * p + 1];
        if (ed2 - ed * ed > 0.0f) {
            g0 = -2.0f * ed * c;
            g1 = c;
        }
    }
    if (use_nc && m.W > 1 && m.H > 1) {
        const float gw = lam_nc * g / fwd_out[4];
        V3 gp = v3(0.0f, 0.0f, 0.0f);  // cotangent of this pixel's point
        QuadGrad q;
        // this pixel's point is the top-left of quad (y, x), the top-right of
        // quad (y, x - 1) and the bottom-left of quad (y - 1, x)
        if (x < m.W - 1 && y < m.H - 1 && quad_valid(m, y, x)) {
            quad_term(m, y, x, gw, &q);
            gp = gp + q.g00;
            gr = q.gr;
        }
        if (x > 0 && y < m.H - 1 && quad_valid(m, y, x - 1)) {
            quad_term(m, y, x - 1, gw, &q);
            gp = gp + q.g01;
        }
        if (y > 0 && x < m.W - 1 && quad_valid(m, y - 1, x)) {
            quad_term(m, y - 1, x, gw, &q);
            gp = gp + q.g10;
        }
        g0 = g0 + dot(gp, load3(m.dir + 3 * p));
    }
    float* o = g_F + 5 * p;
    o[0] = g0;
    o[1] = g1;
    o[2] = gr.x;
    o[3] = gr.y;
    o[4] = gr.z;
}

inline unsigned blocks_for(int64_t n, int threads) {
    return (unsigned)((n + threads - 1) / threads);
}

bool maps_ok(const float* F, const float* alpha, const float* base, const float* dir, int W,
             int H) {
    return F && alpha && base && dir && W > 0 && H > 0;
}

}  // namespace

extern "C" {

int gsx_geom_features(int64_t n, const float* means, const float* quats, const float* depths,
                      const float* center, float* features, void* stream) {
    if (n < 0 || !center) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!means || !quats || !depths || !features || ((uintptr_t)quats & 15u))
        return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_geom_features, dim3(blocks_for(n, kThreads)), dim3(kThreads), 0,
                       (hipStream_t)stream, n, means, (const float4*)quats, depths, center[0],
                       center[1], center[2], features);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_geom_features_bwd(int64_t n, const float* means, const float* quats,
                          const float* depths, const float* center, const float* g_features,
                          float* g_depths, float* g_quats, void* stream) {
    if (n < 0 || !center) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!means || !quats || !depths || !g_features || !g_depths || !g_quats ||
        ((uintptr_t)quats & 15u) || ((uintptr_t)g_quats & 15u))
        return GSX_ERR_INVALID;
    hipLaunchKernelGGL(k_geom_features_bwd, dim3(blocks_for(n, kThreads)), dim3(kThreads), 0,
                       (hipStream_t)stream, n, means, (const float4*)quats, depths, center[0],
                       center[1], center[2], g_features, g_depths, (float4*)g_quats);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int64_t gsx_geom_loss_workspace_bytes(int32_t width, int32_t height) {
    if (width <= 0 || height <= 0) return GSX_ERR_INVALID;
    const int64_t tiles = (int64_t)((width + 15) / 16) * ((height + 15) / 16);
    return 16 * tiles;
}

int gsx_geom_loss_fwd(int32_t width, int32_t height, const float* features, const float* alpha,
                      const float* base, const float* dir, float min_alpha, float lam_dv,
                      float lam_nc, void* workspace, int64_t workspace_bytes, float* out,
                      void* stream) {
    if (!maps_ok(features, alpha, base, dir, width, height) || !out || !workspace)
        return GSX_ERR_INVALID;
    if (workspace_bytes < gsx_geom_loss_workspace_bytes(width, height)) return GSX_ERR_WORKSPACE;
    const GeomMaps m{features, alpha, base, dir, width, height, min_alpha};
    const int use_dv = lam_dv > 0.0f, use_nc = lam_nc > 0.0f && width > 1 && height > 1;
    const int64_t tiles = (int64_t)((width + 15) / 16) * ((height + 15) / 16);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_geom_loss_partial, dim3((unsigned)tiles), dim3(kThreads), 0, st, m,
                       use_dv, use_nc, (float*)workspace);
    GSX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_geom_loss_reduce, dim3(1), dim3(256), 0, st, (const float*)workspace,
                       tiles, lam_dv, lam_nc, use_dv, use_nc, out);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_geom_loss_bwd(int32_t width, int32_t height, const float* features, const float* alpha,
                      const float* base, const float* dir, float min_alpha, float lam_dv,
                      float lam_nc, const float* fwd_out, const float* grad_loss,
                      float* g_features, void* stream) {
    if (!maps_ok(features, alpha, base, dir, width, height) || !fwd_out || !grad_loss ||
        !g_features)
        return GSX_ERR_INVALID;
    const GeomMaps m{features, alpha, base, dir, width, height, min_alpha};
    const int use_dv = lam_dv > 0.0f, use_nc = lam_nc > 0.0f && width > 1 && height > 1;
    hipLaunchKernelGGL(k_geom_loss_bwd, dim3(blocks_for((int64_t)width * height, kThreads)),
                       dim3(kThreads), 0, (hipStream_t)stream, m, use_dv, use_nc, lam_dv, lam_nc,
                       fwd_out, grad_loss, g_features);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // extern "C"
