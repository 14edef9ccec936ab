// gsx_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// Float arithmetic follows the reference's operation order exactly
// (src/mlx3d/splatting/*.py of amirhossein-razlighi/mlx3D v0.2.0) and every
// translation unit is compiled with -ffp-contract=off, so each + - * / sqrt
// is one correctly rounded IEEE operation -- the results that decide radii,
// tile rectangles and per-pixel contributor counts are bit-reproducible.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gsx.h"

namespace gsx {

constexpr int kTile = 16;            // tiles.py:14
constexpr int kTilePixels = 256;     // rasterize.py:26
constexpr int kWave = 64;            // CDNA wavefront

// exp(x): Cody-Waite reduction x = k ln2 + r (ln2 as a 16-bit head plus a
// tail), degree-7 Taylor polynomial of e^r in Horner form with fused
// multiply-adds, exact scaling by 2^k.  Returns 0 below -86 and +inf above
// 88.  The exp of the activations of model.py:116-122 (the compositing
// loops use their own splat_exp, raster.hip).  The CPU oracle evaluates the
// same sequence of correctly rounded operations, so both agree bit for bit.
__device__ __forceinline__ float dexp(float x) {
    if (x != x) return x;
    if (x < -86.0f) return 0.0f;
    if (x > 88.0f) return __builtin_huge_valf();
    const float k = rintf(x * 1.44269504088896341f);
    float r = fmaf(k, -0.693145751953125f, x);
    r = fmaf(k, -1.42860682030941723e-06f, r);
    float p = 1.98412698412698413e-04f;
    p = fmaf(p, r, 1.38888888888888889e-03f);
    p = fmaf(p, r, 8.33333333333333333e-03f);
    p = fmaf(p, r, 4.16666666666666667e-02f);
    p = fmaf(p, r, 1.66666666666666667e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

// One Adam update (mlx.optimizers.Adam.apply_single without bias
// correction, trainer.py:128, 339-342):
//   m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g^2;  p = p - lr m / (sqrt(v) + eps)
// in float32, each operation rounded once, in this order.
__device__ __forceinline__ void adam_update(float& p, float g, float& m, float& v, float lr,
                                            float b1, float omb1, float b2, float omb2,
                                            float eps) {
    m = b1 * m + omb1 * g;
    v = b2 * v + omb2 * (g * g);
    p = p - (lr * m) / (sqrtf(v) + eps);
}

// Sort key whose unsigned order is the float order of z (-0 folded onto +0,
// NaN after +inf).
__device__ __forceinline__ uint32_t depth_key(float z) {
    uint32_t u = __float_as_uint(z);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float act_scale(float s, uint32_t flags) {
    return (flags & GSX_LOG_SCALES) ? dexp(s) : s;
}
__device__ __forceinline__ float act_opacity(float o, uint32_t flags) {
    return (flags & GSX_LOGIT_OPACITY) ? 1.0f / (1.0f + dexp(-o)) : o;
}

// ---------------------------------------------------------------- EWA --
// projection.py:56-138 for one Gaussian.  The backward pass recomputes this
// and reads the intermediates it needs; in the forward kernels the unused
// ones are dead code.
struct Proj {
    float x, y, z, zs, u, v;
    float rx, ry, cxr, cyr, tx, ty, inv_z, inv_z2;
    float j00, j02, j11, j12;
    float T[6];
    float qnorm, qn[4];
    float Rq[9];
    float s[3];
    float P[6];
    float M[6];
    float a0, b, c0, a, c, det, ds;
    float A, B, C, comp, radius;
    bool valid;
};

__device__ __forceinline__ void project(const gsx_camera& cam, float m0, float m1, float m2,
                                        float q0, float q1, float q2, float q3, float s0,
                                        float s1, float s2, float blur, bool aa, Proj& p) {
    const float* R = cam.R;
    p.x = m0 * R[0] + m1 * R[1] + m2 * R[2] + cam.t[0];
    p.y = m0 * R[3] + m1 * R[4] + m2 * R[5] + cam.t[1];
    p.z = m0 * R[6] + m1 * R[7] + m2 * R[8] + cam.t[2];
    p.zs = fmaxf(p.z, 1e-6f);
    p.u = cam.fx * p.x / p.zs + cam.cx;
    p.v = cam.fy * p.y / p.zs + cam.cy;
    p.rx = p.x / p.zs;
    p.ry = p.y / p.zs;
    p.cxr = fminf(fmaxf(p.rx, -cam.lim_x), cam.lim_x);
    p.cyr = fminf(fmaxf(p.ry, -cam.lim_y), cam.lim_y);
    p.tx = p.cxr * p.zs;
    p.ty = p.cyr * p.zs;
    p.inv_z = 1.0f / p.zs;
    p.inv_z2 = p.inv_z * p.inv_z;
    p.j00 = cam.fx * p.inv_z;
    p.j02 = -cam.fx * p.tx * p.inv_z2;
    p.j11 = cam.fy * p.inv_z;
    p.j12 = -cam.fy * p.ty * p.inv_z2;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        p.T[k] = p.j00 * R[k] + p.j02 * R[6 + k];
        p.T[3 + k] = p.j11 * R[3 + k] + p.j12 * R[6 + k];
    }
    p.qnorm = sqrtf(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3);
    const float w = q0 / p.qnorm, x = q1 / p.qnorm, y = q2 / p.qnorm, z = q3 / p.qnorm;
    p.qn[0] = w;
    p.qn[1] = x;
    p.qn[2] = y;
    p.qn[3] = z;
    p.Rq[0] = 1.0f - 2.0f * (y * y + z * z);
    p.Rq[1] = 2.0f * (x * y - w * z);
    p.Rq[2] = 2.0f * (x * z + w * y);
    p.Rq[3] = 2.0f * (x * y + w * z);
    p.Rq[4] = 1.0f - 2.0f * (x * x + z * z);
    p.Rq[5] = 2.0f * (y * z - w * x);
    p.Rq[6] = 2.0f * (x * z - w * y);
    p.Rq[7] = 2.0f * (y * z + w * x);
    p.Rq[8] = 1.0f - 2.0f * (x * x + y * y);
    p.s[0] = s0;
    p.s[1] = s1;
    p.s[2] = s2;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            p.P[3 * r + k] = p.T[3 * r] * p.Rq[k] + p.T[3 * r + 1] * p.Rq[3 + k] +
                             p.T[3 * r + 2] * p.Rq[6 + k];
            p.M[3 * r + k] = p.P[3 * r + k] * p.s[k];
        }
    p.a0 = p.M[0] * p.M[0] + p.M[1] * p.M[1] + p.M[2] * p.M[2];
    p.b = p.M[0] * p.M[3] + p.M[1] * p.M[4] + p.M[2] * p.M[5];
    p.c0 = p.M[3] * p.M[3] + p.M[4] * p.M[4] + p.M[5] * p.M[5];
    p.a = p.a0 + blur;
    p.c = p.c0 + blur;
    p.det = p.a * p.c - p.b * p.b;
    p.ds = fmaxf(p.det, 1e-12f);
    p.A = p.c / p.ds;
    p.B = -p.b / p.ds;
    p.C = p.a / p.ds;
    p.comp = aa ? sqrtf(fmaxf(p.a0 * p.c0 - p.b * p.b, 0.0f) / p.ds) : 1.0f;
    const float mid = 0.5f * (p.a + p.c);
    const float lam1 = mid + sqrtf(fmaxf(mid * mid - p.det, 0.01f));
    p.radius = ceilf(3.0f * sqrtf(fmaxf(lam1, 0.0f)));
    p.valid = (p.z > cam.znear) && (p.det > 0.0f);
    if (!p.valid) {
        p.radius = 0.0f;
        p.comp = 0.0f;
    }
}

// Gradient of the raw quaternion from the gradient G of the rotation matrix
// of its normalisation qn = q / |q| (rotations.py:30-49, projection.py:94-105).
__device__ __forceinline__ void quat_vjp(const float* qn, float qnorm, const float* G,
                                         float* g_q) {
    const float w = qn[0], x = qn[1], y = qn[2], z = qn[3];
    float gqn[4];
    gqn[0] = 2.0f * (-z * G[1] + y * G[2] + z * G[3] - x * G[5] - y * G[6] + x * G[7]);
    gqn[1] = 2.0f * (y * G[1] + z * G[2] + y * G[3] - 2.0f * x * G[4] - w * G[5] + z * G[6] +
                     w * G[7] - 2.0f * x * G[8]);
    gqn[2] = 2.0f * (-2.0f * y * G[0] + x * G[1] + w * G[2] + x * G[3] + z * G[5] - w * G[6] +
                     z * G[7] - 2.0f * y * G[8]);
    gqn[3] = 2.0f * (-2.0f * z * G[0] - w * G[1] + x * G[2] + w * G[3] - 2.0f * z * G[4] +
                     y * G[5] + x * G[6] + y * G[7]);
    const float dot = w * gqn[0] + x * gqn[1] + y * gqn[2] + z * gqn[3];
#pragma unroll
    for (int k = 0; k < 4; ++k) g_q[k] = (gqn[k] - qn[k] * dot) / qnorm;
}

// Gradient of the screen covariance (a0, b, c0) (before blur) from the
// cotangents of the conic (A, B, C) = (c, -b, a) / max(det, 1e-12) and of the
// antialiasing compensation sqrt(max(a0 c0 - b^2, 0) / max(det, 1e-12))
// (projection.py:115-129); max passes gradient only strictly inside.
__device__ __forceinline__ void cov2d_vjp(float a0, float b, float c0, float a, float c,
                                          float det, float ds, float A, float B, float C,
                                          float comp, bool valid, bool aa, float gA, float gB,
                                          float gC, float gcomp, float& g_a0_out,
                                          float& g_b_out, float& g_c0_out) {
    float g_a = gC / ds, g_b = -gB / ds, g_c = gA / ds;
    float g_a0 = 0.0f, g_c0 = 0.0f;
    float g_ds = -(gA * A + gB * B + gC * C) / ds;
    if (aa && valid) {
        const float det0 = a0 * c0 - b * b;
        if (det0 > 0.0f && comp > 0.0f) {
            const float g_r = gcomp * 0.5f / comp;
            const float g_det0 = g_r / ds;
            g_ds += -g_r * (det0 / ds) / ds;
            g_a0 += g_det0 * c0;
            g_c0 += g_det0 * a0;
            g_b += -2.0f * b * g_det0;
        }
    }
    const float g_det = (det > 1e-12f) ? g_ds : 0.0f;
    g_a += g_det * c;
    g_c += g_det * a;
    g_b += -2.0f * b * g_det;
    g_a0_out = g_a0 + g_a;
    g_c0_out = g_c0 + g_c;
    g_b_out = g_b;
}

// Reverse-mode derivative of project(): cotangents of (u, v), conic
// (A, B, C), z and comp -> gradients of the mean, raw quaternion and
// (activated) scales.  max/clip pass gradient strictly inside their active
// branch; the quaternion normalisation is differentiated through.
__device__ __forceinline__ void project_vjp(const gsx_camera& cam, const Proj& p, bool aa,
                                            float gu, float gv, float gA, float gB, float gC,
                                            float gz_in, float gcomp, float* g_m, float* g_q,
                                            float* g_s) {
    const float* R = cam.R;
    float g_a0, g_b, g_c0;
    cov2d_vjp(p.a0, p.b, p.c0, p.a, p.c, p.det, p.ds, p.A, p.B, p.C, p.comp, p.valid, aa, gA,
              gB, gC, gcomp, g_a0, g_b, g_c0);
    float gM[6], gP[6];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        gM[k] = 2.0f * p.M[k] * g_a0 + p.M[3 + k] * g_b;
        gM[3 + k] = 2.0f * p.M[3 + k] * g_c0 + p.M[k] * g_b;
        gP[k] = gM[k] * p.s[k];
        gP[3 + k] = gM[3 + k] * p.s[k];
        g_s[k] = gM[k] * p.P[k] + gM[3 + k] * p.P[3 + k];
    }
    float gT[6], gRq[9];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int i = 0; i < 3; ++i)
            gT[3 * r + i] = gP[3 * r] * p.Rq[3 * i] + gP[3 * r + 1] * p.Rq[3 * i + 1] +
                            gP[3 * r + 2] * p.Rq[3 * i + 2];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int k = 0; k < 3; ++k) gRq[3 * i + k] = p.T[i] * gP[k] + p.T[3 + i] * gP[3 + k];
    float g_j00 = 0.0f, g_j02 = 0.0f, g_j11 = 0.0f, g_j12 = 0.0f;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        g_j00 += gT[k] * R[k];
        g_j02 += gT[k] * R[6 + k];
        g_j11 += gT[3 + k] * R[3 + k];
        g_j12 += gT[3 + k] * R[6 + k];
    }
    float g_invz = cam.fx * g_j00 + cam.fy * g_j11;
    const float g_tx = -cam.fx * p.inv_z2 * g_j02;
    const float g_ty = -cam.fy * p.inv_z2 * g_j12;
    const float g_invz2 = -cam.fx * p.tx * g_j02 - cam.fy * p.ty * g_j12;
    g_invz += 2.0f * p.inv_z * g_invz2;
    float g_zs = -p.inv_z2 * g_invz;
    g_zs += g_tx * p.cxr + g_ty * p.cyr;
    float g_x = 0.0f, g_y = 0.0f;
    const float zs2 = p.zs * p.zs;
    if (p.rx > -cam.lim_x && p.rx < cam.lim_x) {
        const float g_rx = g_tx * p.zs;
        g_x += g_rx / p.zs;
        g_zs += -g_rx * p.x / zs2;
    }
    if (p.ry > -cam.lim_y && p.ry < cam.lim_y) {
        const float g_ry = g_ty * p.zs;
        g_y += g_ry / p.zs;
        g_zs += -g_ry * p.y / zs2;
    }
    g_x += gu * cam.fx / p.zs;
    g_y += gv * cam.fy / p.zs;
    g_zs += -(gu * cam.fx * p.x + gv * cam.fy * p.y) / zs2;
    const float g_z = gz_in + ((p.z > 1e-6f) ? g_zs : 0.0f);
#pragma unroll
    for (int j = 0; j < 3; ++j) g_m[j] = R[j] * g_x + R[3 + j] * g_y + R[6 + j] * g_z;
    quat_vjp(p.qn, p.qnorm, gRq, g_q);
}

// ----------------------------------------------------------------- UT --
// project_gaussians_ut (projection.py:149-205) with the camera's
// project_points (cameras.py:290-311) and lens models (cameras.py:42-77).
// World-to-camera products are summed left to right as in project();
// means over the six sigma points are sums (in point order) times
// float32(1/6).  The CPU oracle evaluates the same operations.

constexpr float kSqrt3 = 1.73205077648162841796875f;  // float32(sqrt(3))
constexpr float kSixth = 0.16666667163372039794921875f;  // float32(1/6)

// arctan(r), r >= 0, from the Taylor series: arctan r = pi/2 - arctan(1/r)
// above 1 and arctan x = pi/4 + arctan((x - 1)/(x + 1)) above tan(pi/8) leave
// |y| <= tan(pi/8), where y - y^3/3 + ... - y^19/19 + y^21/21 (truncation
// below 2e-10 relative) is evaluated in Horner form with fused
// multiply-adds.  Stands in for the arctan of the fisheye model
// (cameras.py:72); the CPU oracle uses the same sequence.
__device__ __forceinline__ float datan_pos(float r) {
    const bool big = r > 1.0f;
    const float x = big ? 1.0f / r : r;
    const bool mid = x > 0.414213562373095049f;
    const float y = mid ? (x - 1.0f) / (x + 1.0f) : x;
    const float y2 = y * y;
    float q = 4.76190476190476191e-02f;
    q = fmaf(q, y2, -5.26315789473684211e-02f);
    q = fmaf(q, y2, 5.88235294117647059e-02f);
    q = fmaf(q, y2, -6.66666666666666667e-02f);
    q = fmaf(q, y2, 7.69230769230769231e-02f);
    q = fmaf(q, y2, -9.09090909090909091e-02f);
    q = fmaf(q, y2, 1.11111111111111111e-01f);
    q = fmaf(q, y2, -1.42857142857142857e-01f);
    q = fmaf(q, y2, 2.0e-01f);
    q = fmaf(q, y2, -3.33333333333333333e-01f);
    float a = fmaf(y * y2, q, y);
    // pi/4 and pi/2 as float32 head + tail: the tail joins the small term first
    if (mid) a = 0.785398185253143310546875f + (a + -2.18556950752568e-08f);
    return big ? 1.57079637050628662109375f + (-4.37113900018624e-08f - a) : a;
}

__device__ __forceinline__ void cam_point(const gsx_camera& cam, float px, float py, float pz,
                                          float& x, float& y, float& z) {
    const float* R = cam.R;
    x = px * R[0] + py * R[1] + pz * R[2] + cam.t[0];
    y = px * R[3] + py * R[4] + pz * R[5] + cam.t[1];
    z = px * R[6] + py * R[7] + pz * R[8] + cam.t[2];
}

// Lens distortion of normalised coordinates (cameras.py:42-51, 69-77).
__device__ __forceinline__ void distort(const gsx_camera& cam, float x, float y, float& xd,
                                        float& yd) {
    const float* d = cam.dist;
    if (cam.lens == GSX_LENS_BROWN) {
        const float r2 = x * x + y * y;
        const float radial = 1.0f + r2 * (d[0] + r2 * (d[1] + r2 * d[4]));
        xd = x * radial + d[5] * x * y + d[3] * (r2 + 2.0f * x * x);
        yd = y * radial + d[2] * (r2 + 2.0f * y * y) + d[6] * x * y;
    } else if (cam.lens == GSX_LENS_FISHEYE) {
        const float r = sqrtf(x * x + y * y);
        const float th = datan_pos(r);
        const float th2 = th * th;
        const float thd = th * (1.0f + th2 * (d[0] + th2 * (d[1] + th2 * (d[2] + th2 * d[3]))));
        const float scale = thd / fmaxf(r, 1e-9f);
        xd = x * scale;
        yd = y * scale;
    } else {
        xd = x;
        yd = y;
    }
}

// Cotangent of (x, y) from that of the distorted (xd, yd).
__device__ __forceinline__ void distort_vjp(const gsx_camera& cam, float x, float y, float gxd,
                                            float gyd, float& gx, float& gy) {
    const float* d = cam.dist;
    if (cam.lens == GSX_LENS_BROWN) {
        const float r2 = x * x + y * y;
        const float radial = 1.0f + r2 * (d[0] + r2 * (d[1] + r2 * d[4]));
        const float dr = d[0] + r2 * (2.0f * d[1] + 3.0f * d[4] * r2);  // d radial / d r2
        const float xy2 = 2.0f * x * y * dr;
        const float dxdx = radial + 2.0f * x * x * dr + 2.0f * d[2] * y + 6.0f * d[3] * x;
        const float dxdy = xy2 + 2.0f * d[2] * x + 2.0f * d[3] * y;
        const float dydy = radial + 2.0f * y * y * dr + 6.0f * d[2] * y + 2.0f * d[3] * x;
        gx = gxd * dxdx + gyd * dxdy;
        gy = gxd * dxdy + gyd * dydy;
    } else if (cam.lens == GSX_LENS_FISHEYE) {
        const float r = sqrtf(x * x + y * y);
        const float th = datan_pos(r);
        const float th2 = th * th;
        const float thd = th * (1.0f + th2 * (d[0] + th2 * (d[1] + th2 * (d[2] + th2 * d[3]))));
        const float rs = fmaxf(r, 1e-9f);
        const float scale = thd / rs;
        const float dthd = 1.0f + th2 * (3.0f * d[0] + th2 * (5.0f * d[1] +
                                         th2 * (7.0f * d[2] + th2 * 9.0f * d[3])));
        float ds_dr = dthd / (1.0f + r * r) / rs;
        if (r > 1e-9f) ds_dr -= thd / (rs * rs);
        gx = gxd * scale;
        gy = gyd * scale;
        if (r > 0.0f) {
            const float g_r = (gxd * x + gyd * y) * ds_dr;
            gx += g_r * x / r;
            gy += g_r * y / r;
        }
    } else {
        gx = gxd;
        gy = gyd;
    }
}

// Camera.project_points of one world point (cameras.py:290-311).
__device__ __forceinline__ void ut_point(const gsx_camera& cam, float px, float py, float pz,
                                         float& u, float& v) {
    float x, y, z;
    cam_point(cam, px, py, pz, x, y, z);
    if (cam.orthographic) {
        u = cam.fx * x + cam.cx;
        v = cam.fy * y + cam.cy;
        return;
    }
    const float inv = 1.0f / (fabsf(z) < 1e-8f ? 1e-8f : z);
    float xd, yd;
    distort(cam, x * inv, y * inv, xd, yd);
    u = cam.fx * xd + cam.cx;
    v = cam.fy * yd + cam.cy;
}

// Cotangent of the world point from that of its pixel coordinates.
__device__ __forceinline__ void ut_point_vjp(const gsx_camera& cam, float px, float py, float pz,
                                             float gu, float gv, float* gp) {
    float x, y, z;
    cam_point(cam, px, py, pz, x, y, z);
    float gcx, gcy, gcz = 0.0f;
    if (cam.orthographic) {
        gcx = cam.fx * gu;
        gcy = cam.fy * gv;
    } else {
        const bool tiny = fabsf(z) < 1e-8f;
        const float inv = 1.0f / (tiny ? 1e-8f : z);
        float gx, gy;
        distort_vjp(cam, x * inv, y * inv, cam.fx * gu, cam.fy * gv, gx, gy);
        gcx = gx * inv;
        gcy = gy * inv;
        if (!tiny) gcz = -(gx * x + gy * y) * inv * inv;
    }
    const float* R = cam.R;
#pragma unroll
    for (int j = 0; j < 3; ++j) gp[j] = R[j] * gcx + R[3 + j] * gcy + R[6 + j] * gcz;
}

struct ProjUT {
    float u, v, z, A, B, C, comp, radius;
    bool valid;
    float qnorm, qn[4], Rq[9], s[3];
    float a0, b, c0, a, c, det, ds;
    float du[6], dv[6];
};

// Sigma point k of the mean m: m + sqrt(3) (+-) column (k mod 3) of R diag(s).
__device__ __forceinline__ void ut_sigma(const ProjUT& p, float m0, float m1, float m2, int k,
                                         float* q) {
    const int j = k % 3;
    const float sg = k < 3 ? 1.0f : -1.0f;
    q[0] = m0 + kSqrt3 * (sg * (p.Rq[j] * p.s[j]));
    q[1] = m1 + kSqrt3 * (sg * (p.Rq[3 + j] * p.s[j]));
    q[2] = m2 + kSqrt3 * (sg * (p.Rq[6 + j] * p.s[j]));
}

__device__ __forceinline__ void project_ut(const gsx_camera& cam, float m0, float m1, float m2,
                                           float q0, float q1, float q2, float q3, float s0,
                                           float s1, float s2, float blur, bool aa, ProjUT& p) {
    p.qnorm = sqrtf(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3);
    const float w = q0 / p.qnorm, x = q1 / p.qnorm, y = q2 / p.qnorm, z = q3 / p.qnorm;
    p.qn[0] = w;
    p.qn[1] = x;
    p.qn[2] = y;
    p.qn[3] = z;
    p.Rq[0] = 1.0f - 2.0f * (y * y + z * z);
    p.Rq[1] = 2.0f * (x * y - w * z);
    p.Rq[2] = 2.0f * (x * z + w * y);
    p.Rq[3] = 2.0f * (x * y + w * z);
    p.Rq[4] = 1.0f - 2.0f * (x * x + z * z);
    p.Rq[5] = 2.0f * (y * z - w * x);
    p.Rq[6] = 2.0f * (x * z - w * y);
    p.Rq[7] = 2.0f * (y * z + w * x);
    p.Rq[8] = 1.0f - 2.0f * (x * x + y * y);
    p.s[0] = s0;
    p.s[1] = s1;
    p.s[2] = s2;
    float us[6], vs[6];
    float su = 0.0f, sv = 0.0f;
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        float q[3];
        ut_sigma(p, m0, m1, m2, k, q);
        ut_point(cam, q[0], q[1], q[2], us[k], vs[k]);
        su = k ? su + us[k] : us[k];
        sv = k ? sv + vs[k] : vs[k];
    }
    p.u = su * kSixth;
    p.v = sv * kSixth;
    float saa = 0.0f, sab = 0.0f, scc = 0.0f;
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        p.du[k] = us[k] - p.u;
        p.dv[k] = vs[k] - p.v;
        const float aa_k = p.du[k] * p.du[k], ab_k = p.du[k] * p.dv[k], cc_k = p.dv[k] * p.dv[k];
        saa = k ? saa + aa_k : aa_k;
        sab = k ? sab + ab_k : ab_k;
        scc = k ? scc + cc_k : cc_k;
    }
    p.a0 = saa * kSixth;
    p.b = sab * kSixth;
    p.c0 = scc * kSixth;
    p.a = p.a0 + blur;
    p.c = p.c0 + blur;
    p.det = p.a * p.c - p.b * p.b;
    p.ds = fmaxf(p.det, 1e-12f);
    p.A = p.c / p.ds;
    p.B = -p.b / p.ds;
    p.C = p.a / p.ds;
    p.comp = aa ? sqrtf(fmaxf(p.a0 * p.c0 - p.b * p.b, 0.0f) / p.ds) : 1.0f;
    const float mid = 0.5f * (p.a + p.c);
    const float lam1 = mid + sqrtf(fmaxf(mid * mid - p.det, 0.01f));
    p.radius = ceilf(3.0f * sqrtf(fmaxf(lam1, 0.0f)));
    const float* R = cam.R;
    p.z = m0 * R[6] + m1 * R[7] + m2 * R[8] + cam.t[2];
    p.valid = (p.z > cam.znear) && (p.det > 0.0f);
    if (!p.valid) {
        p.radius = 0.0f;
        p.comp = 0.0f;
    }
}

// Reverse-mode derivative of project_ut().  The sigma-point covariance
// is differentiated as (1/6) sum du dv^T with du = u_k - mean: the terms
// through the mean drop out because sum_k du_k = 0.
__device__ __forceinline__ void project_ut_vjp(const gsx_camera& cam, const ProjUT& p, float m0,
                                               float m1, float m2, bool aa, float gu, float gv,
                                               float gA, float gB, float gC, float gz_in,
                                               float gcomp, float* g_m, float* g_q,
                                               float* g_s) {
    float g_a0, g_b, g_c0;
    cov2d_vjp(p.a0, p.b, p.c0, p.a, p.c, p.det, p.ds, p.A, p.B, p.C, p.comp, p.valid, aa, gA,
              gB, gC, gcomp, g_a0, g_b, g_c0);
    float gM[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) gM[i] = 0.0f;
    g_m[0] = g_m[1] = g_m[2] = 0.0f;
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const float guk = (gu + 2.0f * p.du[k] * g_a0 + p.dv[k] * g_b) * kSixth;
        const float gvk = (gv + p.du[k] * g_b + 2.0f * p.dv[k] * g_c0) * kSixth;
        float q[3], gp[3];
        ut_sigma(p, m0, m1, m2, k, q);
        ut_point_vjp(cam, q[0], q[1], q[2], guk, gvk, gp);
        const int j = k % 3;
        const float sg = k < 3 ? kSqrt3 : -kSqrt3;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            g_m[i] += gp[i];
            gM[3 * i + j] += sg * gp[i];
        }
    }
    const float* R = cam.R;
#pragma unroll
    for (int j = 0; j < 3; ++j) g_m[j] += R[6 + j] * gz_in;
    float gRq[9];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        g_s[j] = gM[j] * p.Rq[j] + gM[3 + j] * p.Rq[3 + j] + gM[6 + j] * p.Rq[6 + j];
#pragma unroll
        for (int i = 0; i < 3; ++i) gRq[3 * i + j] = gM[3 * i + j] * p.s[j];
    }
    quat_vjp(p.qn, p.qnorm, gRq, g_q);
}

// Projection selected at compile time: EWA (project) or UT (project_ut).
template <bool UT>
struct ProjOf {
    using T = Proj;
};
template <>
struct ProjOf<true> {
    using T = ProjUT;
};

template <bool UT>
__device__ __forceinline__ void project_any(const gsx_camera& cam, float m0, float m1, float m2,
                                            float q0, float q1, float q2, float q3, float s0,
                                            float s1, float s2, float blur, bool aa,
                                            typename ProjOf<UT>::T& p) {
    if constexpr (UT)
        project_ut(cam, m0, m1, m2, q0, q1, q2, q3, s0, s1, s2, blur, aa, p);
    else
        project(cam, m0, m1, m2, q0, q1, q2, q3, s0, s1, s2, blur, aa, p);
}

template <bool UT>
__device__ __forceinline__ void project_any_vjp(const gsx_camera& cam,
                                                const typename ProjOf<UT>::T& p, float m0,
                                                float m1, float m2, bool aa, float gu, float gv,
                                                float gA, float gB, float gC, float gz,
                                                float gcomp, float* g_m, float* g_q,
                                                float* g_s) {
    if constexpr (UT)
        project_ut_vjp(cam, p, m0, m1, m2, aa, gu, gv, gA, gB, gC, gz, gcomp, g_m, g_q, g_s);
    else
        project_vjp(cam, p, aa, gu, gv, gA, gB, gC, gz, gcomp, g_m, g_q, g_s);
}

// ----------------------------------------------------------------- SH --
// sh.py:7-24 real-SH constants, float32.
#define GSX_SH_C0 0.28209479177387814f
#define GSX_SH_C1 0.4886025119029199f
#define GSX_SH_C2_0 1.0925484305920792f
#define GSX_SH_C2_1 -1.0925484305920792f
#define GSX_SH_C2_2 0.31539156525252005f
#define GSX_SH_C2_3 -1.0925484305920792f
#define GSX_SH_C2_4 0.5462742152960396f
#define GSX_SH_C3_0 -0.5900435899266435f
#define GSX_SH_C3_1 2.890611442640554f
#define GSX_SH_C3_2 -0.4570457994644658f
#define GSX_SH_C3_3 0.3731763325901154f
#define GSX_SH_C3_4 -0.4570457994644658f
#define GSX_SH_C3_5 1.445305721320277f
#define GSX_SH_C3_6 -0.5900435899266435f

// Basis value that multiplies coefficient k in eval_sh (sh.py:57-77), in the
// reference's operation order; bk[1] and bk[3] carry the sign of the
// subtracted terms.
__device__ __forceinline__ void sh_basis(int degree, float x, float y, float z, float* bk) {
    bk[0] = GSX_SH_C0;
    if (degree < 1) return;
    bk[1] = -(GSX_SH_C1 * y);
    bk[2] = GSX_SH_C1 * z;
    bk[3] = -(GSX_SH_C1 * x);
    if (degree < 2) return;
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, yz = y * z, xz = x * z;
    bk[4] = GSX_SH_C2_0 * xy;
    bk[5] = GSX_SH_C2_1 * yz;
    bk[6] = GSX_SH_C2_2 * (2.0f * zz - xx - yy);
    bk[7] = GSX_SH_C2_3 * xz;
    bk[8] = GSX_SH_C2_4 * (xx - yy);
    if (degree < 3) return;
    bk[9] = GSX_SH_C3_0 * y * (3.0f * xx - yy);
    bk[10] = GSX_SH_C3_1 * xy * z;
    bk[11] = GSX_SH_C3_2 * y * (4.0f * zz - xx - yy);
    bk[12] = GSX_SH_C3_3 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
    bk[13] = GSX_SH_C3_4 * x * (4.0f * zz - xx - yy);
    bk[14] = GSX_SH_C3_5 * z * (xx - yy);
    bk[15] = GSX_SH_C3_6 * x * (xx - 3.0f * yy);
}

// eval_sh for one channel given the 16 coefficients c[k] (sh.py:57-78):
// the running sum is formed term by term, left to right, as MLX does.
__device__ __forceinline__ float sh_eval(int degree, const float* bk, const float* c, float x,
                                         float y, float z) {
    float res = GSX_SH_C0 * c[0];
    if (degree > 0) {
        res = res - GSX_SH_C1 * y * c[1] + GSX_SH_C1 * z * c[2] - GSX_SH_C1 * x * c[3];
        if (degree > 1) {
            res = res + bk[4] * c[4] + bk[5] * c[5] + bk[6] * c[6] + bk[7] * c[7] + bk[8] * c[8];
            if (degree > 2)
                res = res + bk[9] * c[9] + bk[10] * c[10] + bk[11] * c[11] + bk[12] * c[12] +
                      bk[13] * c[13] + bk[14] * c[14] + bk[15] * c[15];
        }
    }
    return res + 0.5f;
}

// render.py:78-79 unit view direction (normalised with max(|d|, 1e-8)).
__device__ __forceinline__ void view_dir(const gsx_camera& cam, float m0, float m1, float m2,
                                         float& dx, float& dy, float& dz) {
    const float ex = m0 - cam.center[0], ey = m1 - cam.center[1], ez = m2 - cam.center[2];
    const float nrm = fmaxf(sqrtf(ex * ex + ey * ey + ez * ez), 1e-8f);
    dx = ex / nrm;
    dy = ey / nrm;
    dz = ez / nrm;
}

// tiles.py:55-65: inclusive tile rectangle of the 3-sigma square, packed as
// (xmin | ymin << 16, w | h << 16); returns the duplicate count (0 when the
// Gaussian is culled or off screen).
__device__ __forceinline__ uint32_t tile_rect(float x, float y, float r, int width, int height,
                                              int tiles_x, int tiles_y, uint2& rect) {
    const float fx0 = fminf(fmaxf(floorf((x - r) / 16.0f), 0.0f), (float)(tiles_x - 1));
    const float fx1 = fminf(fmaxf(floorf((x + r) / 16.0f), 0.0f), (float)(tiles_x - 1));
    const float fy0 = fminf(fmaxf(floorf((y - r) / 16.0f), 0.0f), (float)(tiles_y - 1));
    const float fy1 = fminf(fmaxf(floorf((y + r) / 16.0f), 0.0f), (float)(tiles_y - 1));
    const bool on = (r > 0.0f) && (x + r >= 0.0f) && (x - r < (float)width) &&
                    (y + r >= 0.0f) && (y - r < (float)height);
    if (!on) {
        rect = make_uint2(0u, 0u);
        return 0u;
    }
    const uint32_t x0 = (uint32_t)(int)fx0, y0 = (uint32_t)(int)fy0;
    const uint32_t w = (uint32_t)((int)fx1 - (int)fx0 + 1), h = (uint32_t)((int)fy1 - (int)fy0 + 1);
    rect = make_uint2(x0 | (y0 << 16), w | (h << 16));
    return w * h;
}

// ------------------------------------------------------------ waves --
__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    const int lane = lane_id();
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t t = __shfl_up(v, (unsigned)o, kWave);
        if (lane >= o) v += t;
    }
    return v;
}

// Maps a linear workgroup id to a work item so that the ~1/8 of the grid
// dispatched to each XCD (workgroups go round-robin over the 8 XCDs) is a
// contiguous range: neighbouring tiles share an L2.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t nb) {
    constexpr uint32_t kXcd = 8;
    const uint32_t q = nb / kXcd, r = nb % kXcd;
    const uint32_t x = b % kXcd, i = b / kXcd;
    return (x < r) ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

}  // namespace gsx

#define GSX_LAUNCH_CHECK()                                  \
    do {                                                    \
        if (hipGetLastError() != hipSuccess) return GSX_ERR_HIP; \
    } while (0)
