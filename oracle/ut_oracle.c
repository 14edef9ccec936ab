/*
 * ut_oracle.c -- CPU restatement of the unscented-transform projection.
 * TEST INFRASTRUCTURE ONLY (the checker of tests/); nothing in the product
 * package links, loads or calls it.
 *
 *   orc_atanf            -- arctan for the fisheye model (cameras.py:72),
 *                           Taylor series after range reduction
 *   orc_project_ut       -- project_gaussians_ut, projection.py:149-205, with
 *                           Camera.project_points (cameras.py:290-311) and the
 *                           Brown-Conrady / fisheye models (cameras.py:42-77)
 *   orc_project_ut_bwd   -- its VJP, derived by hand (what MLX autodiff
 *                           computes), with the sigma-point covariance
 *                           differentiated as (1/6) sum du dv^T (the terms
 *                           through the mean cancel, sum du = 0)
 *
 * Float32, each operation rounded once (-ffp-contract=off), in this order:
 * world-to-camera sums left to right as the EWA restatement; sums over the
 * six sigma points in point order, times float32(1/6); the lens formulas in
 * the reference's operation order, with the doubled Brown constants 2 p1,
 * 2 p2 taken from the camera (formed in double, rounded once).
 *
 * One deliberate difference from autodiff: a sigma point exactly on the
 * optical axis of a fisheye camera gets a finite gradient here, where the
 * reference's sqrt at 0 gives NaN.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "gsx_oracle.h"

#define SQRT3F 1.73205077648162841796875f   /* float32(sqrt(3)) */
#define SIXTHF 0.16666667163372039794921875f /* float32(1/6) */

static int clamp_threads(int n) { return n > 0 ? n : 1; }

/* arctan r for r >= 0: pi/2 - arctan(1/r) above 1, pi/4 + arctan((x-1)/(x+1))
 * above tan(pi/8); on |y| <= tan(pi/8) the series y - y^3/3 + ... + y^21/21 in
 * Horner form with fused multiply-adds. */
float orc_atanf(float r) {
    const int big = r > 1.0f;
    const float x = big ? 1.0f / r : r;
    const int mid = x > 0.414213562373095049f;
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
    /* pi/4 and pi/2 as float32 head + tail: the tail joins the small term first */
    if (mid) a = 0.785398185253143310546875f + (a + -2.18556950752568e-08f);
    return big ? 1.57079637050628662109375f + (-4.37113900018624e-08f - a) : a;
}

static void cam_point(const orc_camera* cam, const float* p, float* c) {
    const float* R = cam->R;
    c[0] = p[0] * R[0] + p[1] * R[1] + p[2] * R[2] + cam->t[0];
    c[1] = p[0] * R[3] + p[1] * R[4] + p[2] * R[5] + cam->t[1];
    c[2] = p[0] * R[6] + p[1] * R[7] + p[2] * R[8] + cam->t[2];
}

/* cameras.py:42-51 (Brown-Conrady) and 69-77 (fisheye) */
static void distort(const orc_camera* cam, float x, float y, float* xd, float* yd) {
    const float* d = cam->dist;
    if (cam->lens == ORC_LENS_BROWN) {
        const float r2 = x * x + y * y;
        const float radial = 1.0f + r2 * (d[0] + r2 * (d[1] + r2 * d[4]));
        *xd = x * radial + d[5] * x * y + d[3] * (r2 + 2.0f * x * x);
        *yd = y * radial + d[2] * (r2 + 2.0f * y * y) + d[6] * x * y;
    } else if (cam->lens == ORC_LENS_FISHEYE) {
        const float r = sqrtf(x * x + y * y);
        const float th = orc_atanf(r);
        const float th2 = th * th;
        const float thd = th * (1.0f + th2 * (d[0] + th2 * (d[1] + th2 * (d[2] + th2 * d[3]))));
        const float scale = thd / fmaxf(r, 1e-9f);
        *xd = x * scale;
        *yd = y * scale;
    } else {
        *xd = x;
        *yd = y;
    }
}

static void distort_vjp(const orc_camera* cam, float x, float y, float gxd, float gyd,
                        float* gx, float* gy) {
    const float* d = cam->dist;
    if (cam->lens == ORC_LENS_BROWN) {
        /* Jacobian of (xd, yd) in (x, y); radial' = d radial / d r2 */
        const float r2 = x * x + y * y;
        const float radial = 1.0f + r2 * (d[0] + r2 * (d[1] + r2 * d[4]));
        const float dr = d[0] + r2 * (2.0f * d[1] + 3.0f * d[4] * r2);
        const float xy2 = 2.0f * x * y * dr;
        const float dxdx = radial + 2.0f * x * x * dr + 2.0f * d[2] * y + 6.0f * d[3] * x;
        const float dxdy = xy2 + 2.0f * d[2] * x + 2.0f * d[3] * y;
        const float dydy = radial + 2.0f * y * y * dr + 6.0f * d[2] * y + 2.0f * d[3] * x;
        *gx = gxd * dxdx + gyd * dxdy;
        *gy = gxd * dxdy + gyd * dydy;
    } else if (cam->lens == ORC_LENS_FISHEYE) {
        /* scale = theta_d(atan r) / max(r, eps); r = |(x, y)| */
        const float r = sqrtf(x * x + y * y);
        const float th = orc_atanf(r);
        const float th2 = th * th;
        const float thd = th * (1.0f + th2 * (d[0] + th2 * (d[1] + th2 * (d[2] + th2 * d[3]))));
        const float rs = fmaxf(r, 1e-9f);
        const float scale = thd / rs;
        const float dthd = 1.0f + th2 * (3.0f * d[0] + th2 * (5.0f * d[1] +
                                         th2 * (7.0f * d[2] + th2 * 9.0f * d[3])));
        float ds_dr = dthd / (1.0f + r * r) / rs;
        if (r > 1e-9f) ds_dr -= thd / (rs * rs);
        *gx = gxd * scale;
        *gy = gyd * scale;
        if (r > 0.0f) {
            const float g_r = (gxd * x + gyd * y) * ds_dr;
            *gx += g_r * x / r;
            *gy += g_r * y / r;
        }
    } else {
        *gx = gxd;
        *gy = gyd;
    }
}

/* Camera.project_points of one world point (cameras.py:290-311) */
static void ut_point(const orc_camera* cam, const float* p, float* u, float* v) {
    float c[3];
    cam_point(cam, p, c);
    if (cam->orthographic) {
        *u = cam->fx * c[0] + cam->cx;
        *v = cam->fy * c[1] + cam->cy;
        return;
    }
    const float inv = 1.0f / (fabsf(c[2]) < 1e-8f ? 1e-8f : c[2]);
    float xd, yd;
    distort(cam, c[0] * inv, c[1] * inv, &xd, &yd);
    *u = cam->fx * xd + cam->cx;
    *v = cam->fy * yd + cam->cy;
}

static void ut_point_vjp(const orc_camera* cam, const float* p, float gu, float gv, float* gp) {
    float c[3];
    cam_point(cam, p, c);
    float gcx, gcy, gcz = 0.0f;
    if (cam->orthographic) {
        gcx = cam->fx * gu;
        gcy = cam->fy * gv;
    } else {
        const int tiny = fabsf(c[2]) < 1e-8f;
        const float inv = 1.0f / (tiny ? 1e-8f : c[2]);
        float gx, gy;
        distort_vjp(cam, c[0] * inv, c[1] * inv, cam->fx * gu, cam->fy * gv, &gx, &gy);
        gcx = gx * inv;
        gcy = gy * inv;
        if (!tiny) gcz = -(gx * c[0] + gy * c[1]) * inv * inv;
    }
    const float* R = cam->R;
    for (int j = 0; j < 3; ++j) gp[j] = R[j] * gcx + R[3 + j] * gcy + R[6 + j] * gcz;
}

typedef struct {
    float u, v, z, A, B, C, comp, radius;
    int valid;
    float qnorm, qn[4], Rq[9], s[3];
    float a0, b, c0, a, c, det, ds;
    float du[6], dv[6];
} ut_t;

/* sigma point k: m + sqrt(3) (+-) column (k mod 3) of R diag(s) (projection.py:165-168) */
static void ut_sigma(const ut_t* p, const float* m, int k, float* q) {
    const int j = k % 3;
    const float sg = k < 3 ? 1.0f : -1.0f;
    for (int i = 0; i < 3; ++i) q[i] = m[i] + SQRT3F * (sg * (p->Rq[3 * i + j] * p->s[j]));
}

static void ut_one(const orc_camera* cam, const float* m, const float* q, const float* s,
                   float blur, int aa, ut_t* p) {
    /* rotations.py:30-49 */
    p->qnorm = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
    for (int k = 0; k < 4; ++k) p->qn[k] = q[k] / p->qnorm;
    const float w = p->qn[0], x = p->qn[1], y = p->qn[2], z = p->qn[3];
    p->Rq[0] = 1.0f - 2.0f * (y * y + z * z);
    p->Rq[1] = 2.0f * (x * y - w * z);
    p->Rq[2] = 2.0f * (x * z + w * y);
    p->Rq[3] = 2.0f * (x * y + w * z);
    p->Rq[4] = 1.0f - 2.0f * (x * x + z * z);
    p->Rq[5] = 2.0f * (y * z - w * x);
    p->Rq[6] = 2.0f * (x * z - w * y);
    p->Rq[7] = 2.0f * (y * z + w * x);
    p->Rq[8] = 1.0f - 2.0f * (x * x + y * y);
    for (int k = 0; k < 3; ++k) p->s[k] = s[k];
    /* projection.py:170-176: pixel positions of the six points, mean, covariance */
    float us[6], vs[6], su = 0.0f, sv = 0.0f;
    for (int k = 0; k < 6; ++k) {
        float pt[3];
        ut_sigma(p, m, k, pt);
        ut_point(cam, pt, &us[k], &vs[k]);
        su = k ? su + us[k] : us[k];
        sv = k ? sv + vs[k] : vs[k];
    }
    p->u = su * SIXTHF;
    p->v = sv * SIXTHF;
    float saa = 0.0f, sab = 0.0f, scc = 0.0f;
    for (int k = 0; k < 6; ++k) {
        p->du[k] = us[k] - p->u;
        p->dv[k] = vs[k] - p->v;
        const float aa_k = p->du[k] * p->du[k], ab_k = p->du[k] * p->dv[k];
        const float cc_k = p->dv[k] * p->dv[k];
        saa = k ? saa + aa_k : aa_k;
        sab = k ? sab + ab_k : ab_k;
        scc = k ? scc + cc_k : cc_k;
    }
    p->a0 = saa * SIXTHF;
    p->b = sab * SIXTHF;
    p->c0 = scc * SIXTHF;
    /* projection.py:178-203, as the EWA path */
    p->a = p->a0 + blur;
    p->c = p->c0 + blur;
    p->det = p->a * p->c - p->b * p->b;
    p->ds = fmaxf(p->det, 1e-12f);
    p->A = p->c / p->ds;
    p->B = -p->b / p->ds;
    p->C = p->a / p->ds;
    p->comp = aa ? sqrtf(fmaxf(p->a0 * p->c0 - p->b * p->b, 0.0f) / p->ds) : 1.0f;
    const float mid = 0.5f * (p->a + p->c);
    const float lam1 = mid + sqrtf(fmaxf(mid * mid - p->det, 0.01f));
    p->radius = ceilf(3.0f * sqrtf(fmaxf(lam1, 0.0f)));
    const float* R = cam->R;
    p->z = m[0] * R[6] + m[1] * R[7] + m[2] * R[8] + cam->t[2];
    p->valid = (p->z > cam->znear) && (p->det > 0.0f);
    if (!p->valid) {
        p->radius = 0.0f;
        p->comp = 0.0f;
    }
}

static void ut_vjp(const orc_camera* cam, const ut_t* p, const float* m, int aa, float gu,
                   float gv, float gA, float gB, float gC, float gz, float gcomp, float* g_m,
                   float* g_q, float* g_s) {
    /* conic and compensation -> (a0, b, c0): as the EWA restatement */
    float g_a = gC / p->ds, g_b = -gB / p->ds, g_c = gA / p->ds;
    float g_a0 = 0.0f, g_c0 = 0.0f;
    float g_ds = -(gA * p->A + gB * p->B + gC * p->C) / p->ds;
    if (aa && p->valid) {
        const float det0 = p->a0 * p->c0 - p->b * p->b;
        if (det0 > 0.0f && p->comp > 0.0f) {
            const float g_r = gcomp * 0.5f / p->comp;
            const float g_det0 = g_r / p->ds;
            g_ds += -g_r * (det0 / p->ds) / p->ds;
            g_a0 += g_det0 * p->c0;
            g_c0 += g_det0 * p->a0;
            g_b += -2.0f * p->b * g_det0;
        }
    }
    const float g_det = (p->det > 1e-12f) ? g_ds : 0.0f;
    g_a += g_det * p->c;
    g_c += g_det * p->a;
    g_b += -2.0f * p->b * g_det;
    g_a0 = g_a0 + g_a;
    g_c0 = g_c0 + g_c;
    /* mean and covariance -> pixel positions -> sigma points */
    float gM[9];
    memset(gM, 0, sizeof(gM));
    g_m[0] = g_m[1] = g_m[2] = 0.0f;
    for (int k = 0; k < 6; ++k) {
        const float guk = (gu + 2.0f * p->du[k] * g_a0 + p->dv[k] * g_b) * SIXTHF;
        const float gvk = (gv + p->du[k] * g_b + 2.0f * p->dv[k] * g_c0) * SIXTHF;
        float pt[3], gp[3];
        ut_sigma(p, m, k, pt);
        ut_point_vjp(cam, pt, guk, gvk, gp);
        const int j = k % 3;
        const float sg = k < 3 ? SQRT3F : -SQRT3F;
        for (int i = 0; i < 3; ++i) {
            g_m[i] += gp[i];
            gM[3 * i + j] += sg * gp[i];
        }
    }
    const float* R = cam->R;
    for (int j = 0; j < 3; ++j) g_m[j] += R[6 + j] * gz;
    /* sqrt_cov = R diag(s) */
    float gRq[9];
    for (int j = 0; j < 3; ++j) {
        g_s[j] = gM[j] * p->Rq[j] + gM[3 + j] * p->Rq[3 + j] + gM[6 + j] * p->Rq[6 + j];
        for (int i = 0; i < 3; ++i) gRq[3 * i + j] = gM[3 * i + j] * p->s[j];
    }
    /* normalised quaternion -> rotation matrix */
    const float w = p->qn[0], x = p->qn[1], y = p->qn[2], z = p->qn[3];
    const float* G = gRq;
    float gqn[4];
    gqn[0] = 2.0f * (-z * G[1] + y * G[2] + z * G[3] - x * G[5] - y * G[6] + x * G[7]);
    gqn[1] = 2.0f * (y * G[1] + z * G[2] + y * G[3] - 2.0f * x * G[4] - w * G[5] + z * G[6] +
                     w * G[7] - 2.0f * x * G[8]);
    gqn[2] = 2.0f * (-2.0f * y * G[0] + x * G[1] + w * G[2] + x * G[3] + z * G[5] - w * G[6] +
                     z * G[7] - 2.0f * y * G[8]);
    gqn[3] = 2.0f * (-2.0f * z * G[0] - w * G[1] + x * G[2] + w * G[3] - 2.0f * z * G[4] +
                     y * G[5] + x * G[6] + y * G[7]);
    const float dot = w * gqn[0] + x * gqn[1] + y * gqn[2] + z * gqn[3];
    for (int k = 0; k < 4; ++k) g_q[k] = (gqn[k] - p->qn[k] * dot) / p->qnorm;
}

void orc_ut_project_one(const orc_camera* cam, const float* m, const float* q, const float* s,
                        float blur, int aa, float* out) {
    ut_t p;
    ut_one(cam, m, q, s, blur, aa, &p);
    out[0] = p.u;
    out[1] = p.v;
    out[2] = p.A;
    out[3] = p.B;
    out[4] = p.C;
    out[5] = p.z;
    out[6] = p.radius;
    out[7] = p.comp;
}

void orc_ut_project_vjp_one(const orc_camera* cam, const float* m, const float* q,
                            const float* s, float blur, int aa, const float* g_in, float* g_m,
                            float* g_q, float* g_s) {
    ut_t p;
    ut_one(cam, m, q, s, blur, aa, &p);
    ut_vjp(cam, &p, m, aa, g_in[0], g_in[1], g_in[2], g_in[3], g_in[4], g_in[5], g_in[6], g_m,
           g_q, g_s);
}

void orc_project_ut(const orc_camera* cam, int64_t n, const float* means, const float* quats,
                    const float* scales, float blur, int antialias, float* means2d,
                    float* conics, float* depths, float* radii, float* comp, int nthreads) {
    const int aa = antialias && blur > 0.0f;
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float o[8];
        orc_ut_project_one(cam, means + 3 * i, quats + 4 * i, scales + 3 * i, blur, aa, o);
        means2d[2 * i] = o[0];
        means2d[2 * i + 1] = o[1];
        conics[3 * i] = o[2];
        conics[3 * i + 1] = o[3];
        conics[3 * i + 2] = o[4];
        depths[i] = o[5];
        radii[i] = o[6];
        comp[i] = o[7];
    }
}

void orc_project_ut_bwd(const orc_camera* cam, int64_t n, const float* means,
                        const float* quats, const float* scales, float blur, int antialias,
                        const float* g_means2d, const float* g_conics, const float* g_depths,
                        const float* g_comp, float* g_means, float* g_quats, float* g_scales,
                        int nthreads) {
    const int aa = antialias && blur > 0.0f;
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float g[7] = {g_means2d ? g_means2d[2 * i] : 0.0f,
                            g_means2d ? g_means2d[2 * i + 1] : 0.0f,
                            g_conics ? g_conics[3 * i] : 0.0f,
                            g_conics ? g_conics[3 * i + 1] : 0.0f,
                            g_conics ? g_conics[3 * i + 2] : 0.0f,
                            g_depths ? g_depths[i] : 0.0f,
                            g_comp ? g_comp[i] : 0.0f};
        orc_ut_project_vjp_one(cam, means + 3 * i, quats + 4 * i, scales + 3 * i, blur, aa, g,
                               g_means + 3 * i, g_quats + 4 * i, g_scales + 3 * i);
    }
}
