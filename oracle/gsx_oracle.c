/*
 * gsx_oracle.c -- CPU restatement of mlx3D's Gaussian-splatting hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are
 * compared against (tests/), the CPU baseline bench.py times, and the
 * reference for __graft_entry__.smoke().  The product library never links it.
 *
 * Citations are paths under the reference repository
 * (amirhossein-razlighi/mlx3D v0.2.0), src/mlx3d/splatting/ unless noted.
 * Every float operation follows the reference's evaluation order; build with
 * -ffp-contract=off (see oracle/Makefile) so none is fused.
 */
#include "gsx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define TILE 16

static int clamp_threads(int n) { return n > 0 ? n : 1; }

/* ------------------------------------------------------------------ exp --
 * exp(x) by Cody & Waite's argument reduction x = k*ln2 + r with ln2 split
 * into a 16-bit head and a tail, then the degree-7 Taylor polynomial of e^r
 * on |r| <= ln2/2 in Horner form (truncation error < 6e-9 relative), and
 * exact scaling by 2^k.  Used for the exp/sigmoid activations of
 * model.py:116-122 (the compositing loops use orc_splat_expf below).
 * Returns 0 below -86 (so the scaled result is never subnormal) and +inf
 * above 88.
 */
float orc_expf(float x) {
    if (x != x) return x;
    if (x < -86.0f) return 0.0f;
    if (x > 88.0f) return INFINITY;
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

void orc_expf_array(int64_t n, const float* x, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

/* ------------------------------------------------------- splat exp/power --
 * The compositing loops' exp (metal::exp at rasterize.py:80,171,274): k =
 * the integer nearest x log2 e, from one fused multiply-add with the
 * rounding constant 1.5 * 2^23 (j = x log2 e + 1.5 * 2^23 rounded to float
 * lies in [2^23, 2^24), where the float spacing is 1, so j - 1.5 * 2^23 = k
 * exactly); r = x - k ln2 with ln2 rounded to float32 (one fused
 * multiply-add); e^r by the degree-5 polynomial p = 1 + r q(r) whose
 * coefficients were fitted for least maximum relative error on
 * |r| <= ln2/2; then 2^k p by adding k to p's exponent field (the low nine
 * bits of j's encoding are k mod 2^9, so j's bits shifted left by 23 add k
 * to the field modulo 2^32; for x in [-86, 88] the result is a normal
 * float, so the add is the exact scaling).  Same range handling as
 * orc_expf.  At most 2.02 ulp from exp on [-6, 0] (every power that can
 * pass the alpha test), 2.19 on [-12, 0] and 4.75 on [-87, 0] (float32
 * sweeps), exp(0) = 1.
 */
float orc_splat_expf(float x) {
    if (x != x) return x;
    if (x < -86.0f) return 0.0f;
    if (x > 88.0f) return INFINITY;
    const float j = fmaf(x, 1.44269504088896341f, 12582912.0f);
    const float k = j - 12582912.0f;
    const float r = fmaf(k, -0.693147182464599609375f, x);
    float q = 8.290260538610955e-03f;
    q = fmaf(q, r, 4.189814578274823e-02f);
    q = fmaf(q, r, 1.6667638172664237e-01f);
    q = fmaf(q, r, 4.9999147944277167e-01f);
    q = fmaf(q, r, 9.999997063356061e-01f);
    const float p = fmaf(q, r, 1.0f);
    uint32_t pb, jb;
    memcpy(&pb, &p, 4);
    memcpy(&jb, &j, 4);
    pb += jb << 23;
    float y;
    memcpy(&y, &pb, 4);
    return y;
}

void orc_splat_expf_array(int64_t n, const float* x, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_splat_expf(x[i]);
}

/* rasterize.py:77-78, power = -0.5 (a dx^2 + c dy^2) - b dx dy, evaluated
 * with the conic pre-scaled to (A, B, C) = (-a/2, -b, -c/2) (exact) and
 * factored as power = (A dx + B dy) dx + (C dy) dy (three products, two
 * multiply-adds; error <= 2 eps (|A| dx^2 + |B dx dy| + |C| dy^2) + eps |power|,
 * eps = 2^-24). */
float orc_splat_power(float a, float b, float c, float dx, float dy) {
    const float A = -0.5f * a, B = -b, C = -0.5f * c;
    return fmaf(fmaf(B, dy, A * dx), dx, (C * dy) * dy);
}

/* model.py:116-122 activations. */
static inline float act_scale(float s, uint32_t flags) {
    return (flags & ORC_LOG_SCALES) ? orc_expf(s) : s;
}
static inline float act_opacity(float o, uint32_t flags) {
    return (flags & ORC_LOGIT_OPACITY) ? 1.0f / (1.0f + orc_expf(-o)) : o;
}

/* ----------------------------------------------------------- projection --
 * projection.py:56-138, one Gaussian, keeping every intermediate the VJP
 * needs. */
typedef struct {
    float x, y, z, zs, u, v;
    float rx, ry;           /* x/z_safe, y/z_safe before the clip       */
    float cxr, cyr;         /* after the clip                           */
    float tx, ty, inv_z, inv_z2;
    float j00, j02, j11, j12;
    float T[6];             /* rows of J @ R                             */
    float qnorm, qn[4];
    float Rq[9];
    float s[3];
    float P[6];             /* (J R Rq) before the column scaling        */
    float M[6];
    float a0, b, c0, a, c, det, ds;
    float A, B, C, comp, radius;
    int valid;
} proj_t;

static void project_one(const orc_camera* cam, const float* m, const float* q,
                        const float* s, float blur, int aa, proj_t* p) {
    const float* R = cam->R;
    /* projection.py:58-61 */
    p->x = m[0] * R[0] + m[1] * R[1] + m[2] * R[2] + cam->t[0];
    p->y = m[0] * R[3] + m[1] * R[4] + m[2] * R[5] + cam->t[1];
    p->z = m[0] * R[6] + m[1] * R[7] + m[2] * R[8] + cam->t[2];
    p->zs = fmaxf(p->z, 1e-6f);
    /* :64-65 */
    p->u = cam->fx * p->x / p->zs + cam->cx;
    p->v = cam->fy * p->y / p->zs + cam->cy;
    /* :70-73 (the bounds are Python doubles rounded once to float32) */
    p->rx = p->x / p->zs;
    p->ry = p->y / p->zs;
    p->cxr = fminf(fmaxf(p->rx, -cam->lim_x), cam->lim_x);
    p->cyr = fminf(fmaxf(p->ry, -cam->lim_y), cam->lim_y);
    p->tx = p->cxr * p->zs;
    p->ty = p->cyr * p->zs;
    /* :75-85 */
    p->inv_z = 1.0f / p->zs;
    p->inv_z2 = p->inv_z * p->inv_z;
    p->j00 = cam->fx * p->inv_z;
    p->j02 = -cam->fx * p->tx * p->inv_z2;
    p->j11 = cam->fy * p->inv_z;
    p->j12 = -cam->fy * p->ty * p->inv_z2;
    /* :87-92 */
    for (int k = 0; k < 3; ++k) {
        p->T[k] = p->j00 * R[k] + p->j02 * R[6 + k];
        p->T[3 + k] = p->j11 * R[3 + k] + p->j12 * R[6 + k];
    }
    /* :94-105 */
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
    /* :107-113 */
    for (int k = 0; k < 3; ++k) p->s[k] = s[k];
    for (int r = 0; r < 2; ++r)
        for (int k = 0; k < 3; ++k) {
            const float* Tr = &p->T[3 * r];
            p->P[3 * r + k] = Tr[0] * p->Rq[k] + Tr[1] * p->Rq[3 + k] + Tr[2] * p->Rq[6 + k];
            p->M[3 * r + k] = p->P[3 * r + k] * s[k];
        }
    const float* M = p->M;
    /* :115-124 */
    p->a0 = M[0] * M[0] + M[1] * M[1] + M[2] * M[2];
    p->b = M[0] * M[3] + M[1] * M[4] + M[2] * M[5];
    p->c0 = M[3] * M[3] + M[4] * M[4] + M[5] * M[5];
    p->a = p->a0 + blur;
    p->c = p->c0 + blur;
    p->det = p->a * p->c - p->b * p->b;
    p->ds = fmaxf(p->det, 1e-12f);
    p->A = p->c / p->ds;
    p->B = -p->b / p->ds;
    p->C = p->a / p->ds;
    /* :125-129 */
    if (aa) {
        const float det0 = fmaxf(p->a0 * p->c0 - p->b * p->b, 0.0f);
        p->comp = sqrtf(det0 / p->ds);
    } else {
        p->comp = 1.0f;
    }
    /* :132-138 */
    const float mid = 0.5f * (p->a + p->c);
    const float lam1 = mid + sqrtf(fmaxf(mid * mid - p->det, 0.01f));
    p->radius = ceilf(3.0f * sqrtf(fmaxf(lam1, 0.0f)));
    p->valid = (p->z > cam->znear) && (p->det > 0.0f);
    if (!p->valid) {
        p->radius = 0.0f;
        p->comp = 0.0f;
    }
}

void orc_project(const orc_camera* cam, int64_t n, const float* means,
                 const float* quats, const float* scales, float blur,
                 int antialias, float* means2d, float* conics, float* depths,
                 float* radii, float* comp, int nthreads) {
    const int aa = antialias && blur > 0.0f;
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        proj_t p;
        project_one(cam, means + 3 * i, quats + 4 * i, scales + 3 * i, blur, aa, &p);
        means2d[2 * i] = p.u;
        means2d[2 * i + 1] = p.v;
        conics[3 * i] = p.A;
        conics[3 * i + 1] = p.B;
        conics[3 * i + 2] = p.C;
        depths[i] = p.z;
        radii[i] = p.radius;
        comp[i] = p.comp;
    }
}

/* VJP of projection.py:56-138 for one Gaussian.  Gradients pass through
 * max/clip only strictly inside the active branch, through the quaternion
 * normalisation, and (antialias) through sqrt(max(det0,0)/det_safe). */
static void project_vjp(const orc_camera* cam, const proj_t* p, int aa,
                        float gu, float gv, float gA, float gB, float gC,
                        float gz_in, float gcomp, float* g_m, float* g_q,
                        float* g_s) {
    const float* R = cam->R;
    float g_a = 0.0f, g_b = 0.0f, g_c = 0.0f, g_a0 = 0.0f, g_c0 = 0.0f;
    /* conics = (c, -b, a) / det_safe */
    g_c += gA / p->ds;
    g_b += -gB / p->ds;
    g_a += gC / p->ds;
    float g_ds = -(gA * p->A + gB * p->B + gC * p->C) / p->ds;
    /* compensation = sqrt(max(a0 c0 - b^2, 0) / det_safe), zero if invalid */
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
    /* det_safe = max(det, 1e-12); det = a c - b^2 */
    const float g_det = (p->det > 1e-12f) ? g_ds : 0.0f;
    g_a += g_det * p->c;
    g_c += g_det * p->a;
    g_b += -2.0f * p->b * g_det;
    g_a0 += g_a;
    g_c0 += g_c;
    /* a0, b, c0 from the rows of M */
    float gM[6];
    for (int k = 0; k < 3; ++k) {
        gM[k] = 2.0f * p->M[k] * g_a0 + p->M[3 + k] * g_b;
        gM[3 + k] = 2.0f * p->M[3 + k] * g_c0 + p->M[k] * g_b;
    }
    /* M = P diag(s) */
    float gP[6];
    for (int k = 0; k < 3; ++k) {
        gP[k] = gM[k] * p->s[k];
        gP[3 + k] = gM[3 + k] * p->s[k];
        g_s[k] = gM[k] * p->P[k] + gM[3 + k] * p->P[3 + k];
    }
    /* P = T Rq */
    float gT[6], gRq[9];
    for (int r = 0; r < 2; ++r)
        for (int i = 0; i < 3; ++i)
            gT[3 * r + i] = gP[3 * r] * p->Rq[3 * i] + gP[3 * r + 1] * p->Rq[3 * i + 1] +
                            gP[3 * r + 2] * p->Rq[3 * i + 2];
    for (int i = 0; i < 3; ++i)
        for (int k = 0; k < 3; ++k)
            gRq[3 * i + k] = p->T[i] * gP[k] + p->T[3 + i] * gP[3 + k];
    /* T rows = j00 R0 + j02 R2, j11 R1 + j12 R2 */
    float g_j00 = 0.0f, g_j02 = 0.0f, g_j11 = 0.0f, g_j12 = 0.0f;
    for (int k = 0; k < 3; ++k) {
        g_j00 += gT[k] * R[k];
        g_j02 += gT[k] * R[6 + k];
        g_j11 += gT[3 + k] * R[3 + k];
        g_j12 += gT[3 + k] * R[6 + k];
    }
    float g_invz = cam->fx * g_j00 + cam->fy * g_j11;
    const float g_tx = -cam->fx * p->inv_z2 * g_j02;
    const float g_ty = -cam->fy * p->inv_z2 * g_j12;
    const float g_invz2 = -cam->fx * p->tx * g_j02 - cam->fy * p->ty * g_j12;
    g_invz += 2.0f * p->inv_z * g_invz2;
    float g_zs = -p->inv_z2 * g_invz;
    /* tx = clip(x/zs) * zs */
    g_zs += g_tx * p->cxr + g_ty * p->cyr;
    float g_x = 0.0f, g_y = 0.0f;
    const float zs2 = p->zs * p->zs;
    if (p->rx > -cam->lim_x && p->rx < cam->lim_x) {
        const float g_rx = g_tx * p->zs;
        g_x += g_rx / p->zs;
        g_zs += -g_rx * p->x / zs2;
    }
    if (p->ry > -cam->lim_y && p->ry < cam->lim_y) {
        const float g_ry = g_ty * p->zs;
        g_y += g_ry / p->zs;
        g_zs += -g_ry * p->y / zs2;
    }
    /* u = fx x / zs + cx */
    g_x += gu * cam->fx / p->zs;
    g_y += gv * cam->fy / p->zs;
    g_zs += -(gu * cam->fx * p->x + gv * cam->fy * p->y) / zs2;
    const float g_z = gz_in + ((p->z > 1e-6f) ? g_zs : 0.0f);
    /* camera coordinates = R m + t */
    for (int j = 0; j < 3; ++j) g_m[j] = R[j] * g_x + R[3 + j] * g_y + R[6 + j] * g_z;
    /* rotation matrix of the normalised quaternion */
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
    const float dot = p->qn[0] * gqn[0] + p->qn[1] * gqn[1] + p->qn[2] * gqn[2] + p->qn[3] * gqn[3];
    for (int k = 0; k < 4; ++k) g_q[k] = (gqn[k] - p->qn[k] * dot) / p->qnorm;
}

void orc_project_bwd(const orc_camera* cam, int64_t n, const float* means,
                     const float* quats, const float* scales, float blur,
                     int antialias, const float* g_means2d,
                     const float* g_conics, const float* g_depths,
                     const float* g_comp, float* g_means, float* g_quats,
                     float* g_scales, int nthreads) {
    const int aa = antialias && blur > 0.0f;
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        proj_t p;
        project_one(cam, means + 3 * i, quats + 4 * i, scales + 3 * i, blur, aa, &p);
        project_vjp(cam, &p, aa, g_means2d ? g_means2d[2 * i] : 0.0f,
                    g_means2d ? g_means2d[2 * i + 1] : 0.0f,
                    g_conics ? g_conics[3 * i] : 0.0f, g_conics ? g_conics[3 * i + 1] : 0.0f,
                    g_conics ? g_conics[3 * i + 2] : 0.0f, g_depths ? g_depths[i] : 0.0f,
                    g_comp ? g_comp[i] : 0.0f, g_means + 3 * i, g_quats + 4 * i,
                    g_scales + 3 * i);
    }
}

/* ------------------------------------------------------------------ SH --
 * sh.py:7-24 constants (real SH, 3DGS sign convention), rounded to float32
 * where the reference multiplies float32 arrays by them. */
#define SH_C0 0.28209479177387814f
#define SH_C1 0.4886025119029199f
static const float SH_C2[5] = {1.0925484305920792f, -1.0925484305920792f,
                               0.31539156525252005f, -1.0925484305920792f,
                               0.5462742152960396f};
static const float SH_C3[7] = {-0.5900435899266435f, 2.890611442640554f,
                               -0.4570457994644658f, 0.3731763325901154f,
                               -0.4570457994644658f, 1.445305721320277f,
                               -0.5900435899266435f};

/* Basis value multiplying coefficient k in eval_sh (sh.py:57-77), in the
 * reference's operation order (the sign of a subtracted term folded in). */
static void sh_basis(int degree, float x, float y, float z, float* bk) {
    bk[0] = SH_C0;
    if (degree < 1) return;
    bk[1] = -(SH_C1 * y);
    bk[2] = SH_C1 * z;
    bk[3] = -(SH_C1 * x);
    if (degree < 2) return;
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, yz = y * z, xz = x * z;
    bk[4] = SH_C2[0] * xy;
    bk[5] = SH_C2[1] * yz;
    bk[6] = SH_C2[2] * (2.0f * zz - xx - yy);
    bk[7] = SH_C2[3] * xz;
    bk[8] = SH_C2[4] * (xx - yy);
    if (degree < 3) return;
    bk[9] = SH_C3[0] * y * (3.0f * xx - yy);
    bk[10] = SH_C3[1] * xy * z;
    bk[11] = SH_C3[2] * y * (4.0f * zz - xx - yy);
    bk[12] = SH_C3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
    bk[13] = SH_C3[4] * x * (4.0f * zz - xx - yy);
    bk[14] = SH_C3[5] * z * (xx - yy);
    bk[15] = SH_C3[6] * x * (xx - 3.0f * yy);
}

/* eval_sh for one Gaussian and channel: sh.py:52-78, term by term in the
 * reference's left-to-right order. */
static float sh_eval_one(int degree, const float* sh, int C, int ch, float x,
                         float y, float z) {
    float bk[16];
    sh_basis(degree, x, y, z, bk);
#define SHC(k) sh[(k) * C + ch]
    float res = SH_C0 * SHC(0);
    if (degree > 0) {
        res = res - SH_C1 * y * SHC(1) + SH_C1 * z * SHC(2) - SH_C1 * x * SHC(3);
        if (degree > 1) {
            res = res + bk[4] * SHC(4) + bk[5] * SHC(5) + bk[6] * SHC(6) + bk[7] * SHC(7) +
                  bk[8] * SHC(8);
            if (degree > 2)
                res = res + bk[9] * SHC(9) + bk[10] * SHC(10) + bk[11] * SHC(11) +
                      bk[12] * SHC(12) + bk[13] * SHC(13) + bk[14] * SHC(14) +
                      bk[15] * SHC(15);
        }
    }
#undef SHC
    return res + 0.5f;
}

void orc_eval_sh(int64_t n, int K, int C, int degree, const float* sh,
                 const float* dirs, float* out, int nthreads) {
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float* d = dirs + 3 * i;
        for (int ch = 0; ch < C; ++ch)
            out[i * C + ch] = sh_eval_one(degree, sh + i * (int64_t)K * C, C, ch, d[0], d[1], d[2]);
    }
}

/* Partial derivatives of the basis functions w.r.t. the direction. */
static void sh_basis_grad(int degree, float x, float y, float z, float* dx,
                          float* dy, float* dz) {
    for (int k = 0; k < 16; ++k) dx[k] = dy[k] = dz[k] = 0.0f;
    if (degree < 1) return;
    dy[1] = -SH_C1;
    dz[2] = SH_C1;
    dx[3] = -SH_C1;
    if (degree < 2) return;
    dx[4] = SH_C2[0] * y;  dy[4] = SH_C2[0] * x;
    dy[5] = SH_C2[1] * z;  dz[5] = SH_C2[1] * y;
    dx[6] = SH_C2[2] * -2.0f * x;  dy[6] = SH_C2[2] * -2.0f * y;  dz[6] = SH_C2[2] * 4.0f * z;
    dx[7] = SH_C2[3] * z;  dz[7] = SH_C2[3] * x;
    dx[8] = SH_C2[4] * 2.0f * x;  dy[8] = SH_C2[4] * -2.0f * y;
    if (degree < 3) return;
    const float xx = x * x, yy = y * y, zz = z * z;
    dx[9] = SH_C3[0] * 6.0f * x * y;
    dy[9] = SH_C3[0] * (3.0f * xx - 3.0f * yy);
    dx[10] = SH_C3[1] * y * z;  dy[10] = SH_C3[1] * x * z;  dz[10] = SH_C3[1] * x * y;
    dx[11] = SH_C3[2] * -2.0f * x * y;
    dy[11] = SH_C3[2] * (4.0f * zz - xx - 3.0f * yy);
    dz[11] = SH_C3[2] * 8.0f * y * z;
    dx[12] = SH_C3[3] * -6.0f * x * z;
    dy[12] = SH_C3[3] * -6.0f * y * z;
    dz[12] = SH_C3[3] * (6.0f * zz - 3.0f * xx - 3.0f * yy);
    dx[13] = SH_C3[4] * (4.0f * zz - 3.0f * xx - yy);
    dy[13] = SH_C3[4] * -2.0f * x * y;
    dz[13] = SH_C3[4] * 8.0f * x * z;
    dx[14] = SH_C3[5] * 2.0f * x * z;
    dy[14] = SH_C3[5] * -2.0f * y * z;
    dz[14] = SH_C3[5] * (xx - yy);
    dx[15] = SH_C3[6] * (3.0f * xx - 3.0f * yy);
    dy[15] = SH_C3[6] * -6.0f * x * y;
}

void orc_eval_sh_bwd(int64_t n, int K, int C, int degree, const float* sh,
                     const float* dirs, const float* g_out, float* g_sh,
                     float* g_dirs, int nthreads) {
    const int Ka = (degree + 1) * (degree + 1);
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float* d = dirs + 3 * i;
        float bk[16], dx[16], dy[16], dz[16];
        sh_basis(degree, d[0], d[1], d[2], bk);
        sh_basis_grad(degree, d[0], d[1], d[2], dx, dy, dz);
        const float* shi = sh + i * (int64_t)K * C;
        float* gsh = g_sh + i * (int64_t)K * C;
        float gd[3] = {0.0f, 0.0f, 0.0f};
        for (int k = 0; k < K; ++k)
            for (int ch = 0; ch < C; ++ch) {
                const float go = g_out[i * C + ch];
                gsh[k * C + ch] = (k < Ka) ? bk[k] * go : 0.0f;
                if (k < Ka) {
                    gd[0] += dx[k] * shi[k * C + ch] * go;
                    gd[1] += dy[k] * shi[k * C + ch] * go;
                    gd[2] += dz[k] * shi[k * C + ch] * go;
                }
            }
        if (g_dirs) {
            g_dirs[3 * i] = gd[0];
            g_dirs[3 * i + 1] = gd[1];
            g_dirs[3 * i + 2] = gd[2];
        }
    }
}

/* render.py:78-79: unit view direction from the camera centre. */
static void view_dir(const orc_camera* cam, const float* m, float* d) {
    const float dx = m[0] - cam->center[0];
    const float dy = m[1] - cam->center[1];
    const float dz = m[2] - cam->center[2];
    const float nrm = fmaxf(sqrtf(dx * dx + dy * dy + dz * dz), 1e-8f);
    d[0] = dx / nrm;
    d[1] = dy / nrm;
    d[2] = dz / nrm;
}

/* -------------------------------------------------- fused preprocess -- */
void orc_preprocess_fwd(const orc_camera* cam, int64_t n, const float* means,
                        const float* quats, const float* scales,
                        const float* opacities, const float* sh, int K,
                        int degree, uint32_t flags, float blur,
                        float* means2d, float* conics, float* depths,
                        float* radii, float* comp, float* opac_eff,
                        float* colors_out, int nthreads) {
    const int aa = (flags & ORC_ANTIALIAS) && blur > 0.0f;
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float s[3];
        for (int k = 0; k < 3; ++k) s[k] = act_scale(scales[3 * i + k], flags);
        const float o = act_opacity(opacities[i], flags);
        proj_t p;
        if (flags & ORC_PROJECT_UT) { /* render.py:14-26 */
            float r[8];
            orc_ut_project_one(cam, means + 3 * i, quats + 4 * i, s, blur, aa, r);
            p.u = r[0];
            p.v = r[1];
            p.A = r[2];
            p.B = r[3];
            p.C = r[4];
            p.z = r[5];
            p.radius = r[6];
            p.comp = r[7];
        } else {
            project_one(cam, means + 3 * i, quats + 4 * i, s, blur, aa, &p);
        }
        means2d[2 * i] = p.u;
        means2d[2 * i + 1] = p.v;
        conics[3 * i] = p.A;
        conics[3 * i + 1] = p.B;
        conics[3 * i + 2] = p.C;
        depths[i] = p.z;
        radii[i] = p.radius;
        comp[i] = p.comp;
        opac_eff[i] = o * p.comp; /* render.py:75 */
        if (sh) {
            float d[3];
            view_dir(cam, means + 3 * i, d);
            for (int ch = 0; ch < 3; ++ch) /* render.py:80 */
                colors_out[3 * i + ch] =
                    fmaxf(sh_eval_one(degree, sh + i * (int64_t)K * 3, 3, ch, d[0], d[1], d[2]), 0.0f);
        }
    }
}

void orc_preprocess_bwd(const orc_camera* cam, int64_t n, const float* means,
                        const float* quats, const float* scales,
                        const float* opacities, const float* colors_out,
                        int K, int degree, uint32_t flags, float blur,
                        const float* g_means2d, const float* g_conics,
                        const float* g_opac_eff, const float* g_colors,
                        const float* g_depths, const float* g_comp,
                        float* g_means, float* g_quats, float* g_scales,
                        float* g_opacities, float* g_sh, int nthreads) {
    const int aa = (flags & ORC_ANTIALIAS) && blur > 0.0f;
    const int Ka = (degree + 1) * (degree + 1);
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float s[3];
        for (int k = 0; k < 3; ++k) s[k] = act_scale(scales[3 * i + k], flags);
        const float o = act_opacity(opacities[i], flags);
        const int ut = (flags & ORC_PROJECT_UT) != 0;
        float comp_i;
        proj_t p;
        if (ut) {
            float r[8];
            orc_ut_project_one(cam, means + 3 * i, quats + 4 * i, s, blur, aa, r);
            comp_i = r[7];
        } else {
            project_one(cam, means + 3 * i, quats + 4 * i, s, blur, aa, &p);
            comp_i = p.comp;
        }
        const float goe = g_opac_eff ? g_opac_eff[i] : 0.0f;
        /* opac_eff = o * comp */
        const float g_o = goe * comp_i;
        const float g_comp_total = (g_comp ? g_comp[i] : 0.0f) + goe * o;
        float gs[3];
        const float g_in[7] = {g_means2d ? g_means2d[2 * i] : 0.0f,
                               g_means2d ? g_means2d[2 * i + 1] : 0.0f,
                               g_conics ? g_conics[3 * i] : 0.0f,
                               g_conics ? g_conics[3 * i + 1] : 0.0f,
                               g_conics ? g_conics[3 * i + 2] : 0.0f,
                               g_depths ? g_depths[i] : 0.0f, g_comp_total};
        if (ut)
            orc_ut_project_vjp_one(cam, means + 3 * i, quats + 4 * i, s, blur, aa, g_in,
                                   g_means + 3 * i, g_quats + 4 * i, gs);
        else
            project_vjp(cam, &p, aa, g_in[0], g_in[1], g_in[2], g_in[3], g_in[4], g_in[5],
                        g_in[6], g_means + 3 * i, g_quats + 4 * i, gs);
        for (int k = 0; k < 3; ++k)
            g_scales[3 * i + k] = (flags & ORC_LOG_SCALES) ? gs[k] * s[k] : gs[k];
        g_opacities[i] = (flags & ORC_LOGIT_OPACITY) ? g_o * o * (1.0f - o) : g_o;
        if (g_sh) {
            /* colours = max(eval_sh(dirs), 0) with dirs under stop_gradient */
            float d[3], bk[16];
            view_dir(cam, means + 3 * i, d);
            sh_basis(degree, d[0], d[1], d[2], bk);
            float* gsh = g_sh + i * (int64_t)K * 3;
            for (int ch = 0; ch < 3; ++ch) {
                const float gc = (colors_out[3 * i + ch] > 0.0f) ? g_colors[3 * i + ch] : 0.0f;
                for (int k = 0; k < K; ++k) gsh[k * 3 + ch] = (k < Ka) ? bk[k] * gc : 0.0f;
            }
        }
    }
}

/* ------------------------------------------------------------- binning -- */
static inline uint32_t depth_key(float z) {
    uint32_t u;
    memcpy(&u, &z, 4);
    if (u == 0x80000000u) u = 0; /* -0 ties with +0 */
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static int cmp_u64(const void* a, const void* b) {
    const uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x > y) - (x < y);
}

/* tiles.py:55-65 for one Gaussian: inclusive tile rectangle and count. */
static int64_t tile_rect(float x, float y, float r, int width, int height,
                         int tiles_x, int tiles_y, int* xmin, int* ymin,
                         int* w, int* h) {
    const float fx0 = fminf(fmaxf(floorf((x - r) / 16.0f), 0.0f), (float)(tiles_x - 1));
    const float fx1 = fminf(fmaxf(floorf((x + r) / 16.0f), 0.0f), (float)(tiles_x - 1));
    const float fy0 = fminf(fmaxf(floorf((y - r) / 16.0f), 0.0f), (float)(tiles_y - 1));
    const float fy1 = fminf(fmaxf(floorf((y + r) / 16.0f), 0.0f), (float)(tiles_y - 1));
    const int on = (r > 0.0f) && (x + r >= 0.0f) && (x - r < (float)width) &&
                   (y + r >= 0.0f) && (y - r < (float)height);
    if (!on) {
        *w = *h = 0;
        *xmin = *ymin = 0;
        return 0;
    }
    *xmin = (int)fx0;
    *ymin = (int)fy0;
    *w = (int)fx1 - (int)fx0 + 1;
    *h = (int)fy1 - (int)fy0 + 1;
    return (int64_t)(*w) * (*h);
}

/* tiles.py:91-146: with conics given, a (tile, Gaussian) duplicate is kept
 * only if the minimum of q(d) = a dx^2 + 2 b dx dy + c dy^2 over the tile's
 * continuous rectangle (clipped to the image) is <= 12; the minimum is taken
 * over the four corners and the four clipped edge minimisers, zero when the
 * mean is inside.  float32 in the reference's evaluation order. */
static float refine_q(float a, float b, float c, float dx, float dy) {
    return (a * dx * dx + 2.0f * b * dx * dy) + c * dy * dy;
}

static float clipf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

static int refine_keep(int tx, int ty, int width, int height, float gx, float gy,
                       const float* co) {
    const float x0 = (float)(tx * TILE), y0 = (float)(ty * TILE);
    const float x1 = (float)((tx + 1) * TILE < width ? (tx + 1) * TILE : width);
    const float y1 = (float)((ty + 1) * TILE < height ? (ty + 1) * TILE : height);
    const float dx_min = x0 - gx, dx_max = x1 - gx, dy_min = y0 - gy, dy_max = y1 - gy;
    if (dx_min <= 0.0f && dx_max >= 0.0f && dy_min <= 0.0f && dy_max >= 0.0f) return 1;
    const float a = co[0], b = co[1], c = co[2];
    const float dy_at_left = clipf(-(b / c) * dx_min, dy_min, dy_max);
    const float dy_at_right = clipf(-(b / c) * dx_max, dy_min, dy_max);
    const float dx_at_bottom = clipf(-(b / a) * dy_min, dx_min, dx_max);
    const float dx_at_top = clipf(-(b / a) * dy_max, dx_min, dx_max);
    float qmin = refine_q(a, b, c, dx_min, dy_min);
    qmin = fminf(qmin, refine_q(a, b, c, dx_min, dy_max));
    qmin = fminf(qmin, refine_q(a, b, c, dx_max, dy_min));
    qmin = fminf(qmin, refine_q(a, b, c, dx_max, dy_max));
    qmin = fminf(qmin, refine_q(a, b, c, dx_min, dy_at_left));
    qmin = fminf(qmin, refine_q(a, b, c, dx_max, dy_at_right));
    qmin = fminf(qmin, refine_q(a, b, c, dx_at_bottom, dy_min));
    qmin = fminf(qmin, refine_q(a, b, c, dx_at_top, dy_max));
    return qmin <= 12.0f;
}

int64_t orc_bin(int64_t n, const float* means2d, const float* radii,
                const float* depths, const float* conics, int64_t conic_stride,
                int width, int height, int32_t* sorted_ids, int64_t cap,
                int32_t* tile_ranges, int nthreads) {
    const int tiles_x = (width + TILE - 1) / TILE;
    const int tiles_y = (height + TILE - 1) / TILE;
    const int64_t T = (int64_t)tiles_x * tiles_y;
    const int nt = clamp_threads(nthreads);
    memset(tile_ranges, 0, sizeof(int32_t) * 2 * T);

    /* Gaussians are split into nt fixed chunks; every per-chunk table is
     * indexed by the chunk, never by the OpenMP thread that ran it. */
    const int nchunk = nt;
    int64_t* hist = (int64_t*)calloc((size_t)nchunk * (size_t)T, sizeof(int64_t));
    int64_t D = 0;
#pragma omp parallel for num_threads(nt) schedule(static, 1) reduction(+ : D)
    for (int k = 0; k < nchunk; ++k) {
        int64_t* h = hist + (size_t)k * T;
        const int64_t i0 = n * k / nchunk, i1 = n * (k + 1) / nchunk;
        for (int64_t i = i0; i < i1; ++i) {
            int x0, y0, w, hh;
            const int64_t c = tile_rect(means2d[2 * i], means2d[2 * i + 1], radii[i], width,
                                        height, tiles_x, tiles_y, &x0, &y0, &w, &hh);
            if (!conics) D += c;
            for (int ty = y0; ty < y0 + hh; ++ty)
                for (int tx = x0; tx < x0 + w; ++tx) {
                    if (conics && !refine_keep(tx, ty, width, height, means2d[2 * i],
                                               means2d[2 * i + 1], conics + i * conic_stride))
                        continue;
                    if (conics) ++D;
                    h[(int64_t)ty * tiles_x + tx]++;
                }
        }
    }
    if (D == 0 || D > cap) {
        free(hist);
        return D;
    }
    /* write cursors: tile-major, chunk-minor */
    int64_t* tile_start = (int64_t*)malloc(sizeof(int64_t) * (size_t)(T + 1));
    int64_t run = 0;
    for (int64_t t = 0; t < T; ++t) {
        tile_start[t] = run;
        for (int k = 0; k < nchunk; ++k) {
            int64_t* h = hist + (size_t)k * T;
            const int64_t c = h[t];
            h[t] = run;
            run += c;
        }
    }
    tile_start[T] = run;
    uint64_t* entries = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)D);
#pragma omp parallel for num_threads(nt) schedule(static, 1)
    for (int k = 0; k < nchunk; ++k) {
        int64_t* cur = hist + (size_t)k * T;
        const int64_t i0 = n * k / nchunk, i1 = n * (k + 1) / nchunk;
        for (int64_t i = i0; i < i1; ++i) {
            int x0, y0, w, hh;
            tile_rect(means2d[2 * i], means2d[2 * i + 1], radii[i], width, height, tiles_x,
                      tiles_y, &x0, &y0, &w, &hh);
            const uint64_t key = ((uint64_t)depth_key(depths[i]) << 32) | (uint32_t)i;
            for (int ty = y0; ty < y0 + hh; ++ty)
                for (int tx = x0; tx < x0 + w; ++tx) {
                    if (conics && !refine_keep(tx, ty, width, height, means2d[2 * i],
                                               means2d[2 * i + 1], conics + i * conic_stride))
                        continue;
                    entries[cur[(int64_t)ty * tiles_x + tx]++] = key;
                }
        }
    }
    /* Within a tile: depth ascending, ties by Gaussian index -- the order a
     * stable argsort of depths induces through key = tile*N + rank
     * (tiles.py:167-172). */
#pragma omp parallel for num_threads(nt) schedule(dynamic, 16)
    for (int64_t t = 0; t < T; ++t) {
        const int64_t s0 = tile_start[t], s1 = tile_start[t + 1];
        if (s1 - s0 > 1) qsort(entries + s0, (size_t)(s1 - s0), sizeof(uint64_t), cmp_u64);
        if (s1 > s0) { /* tiles.py:175-180: empty tiles keep (0, 0) */
            tile_ranges[2 * t] = (int32_t)s0;
            tile_ranges[2 * t + 1] = (int32_t)s1;
        }
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t d = 0; d < D; ++d) sorted_ids[d] = (int32_t)(uint32_t)entries[d];
    free(entries);
    free(tile_start);
    free(hist);
    return D;
}

/* ---------------------------------------------------------- rasterizer -- */
/* The shipped arithmetic (arith = 0) and, for measuring how far it lies
 * from the reference's literal expressions, three alternatives that can be
 * combined (ORC_ARITH_* bits):
 *  - LITERAL_POWER: rasterize.py:75-76 as written,
 *    -0.5f * (a dx dx + c dy dy) - b dx dy, every product and sum rounded
 *    separately in source order (the library builds with -ffp-contract=off);
 *  - SEPARATE_ACC: rasterize.py:84 `acc += rgb * (alpha * T)` as a rounded
 *    product then a rounded sum instead of one multiply-add;
 *  - ROUNDED_EXP: metal::exp replaced by the float32 rounding of the
 *    double-precision exp (the result a correctly rounded exp gives except in
 *    rare double-rounding ties) instead of orc_splat_expf. */
static inline float literal_power(float a, float b, float c, float dx, float dy) {
    const float ax = a * dx, axx = ax * dx;
    const float cy = c * dy, cyy = cy * dy;
    const float bx = b * dx, bxy = bx * dy;
    return -0.5f * (axx + cyy) - bxy;
}

float orc_literal_power(float a, float b, float c, float dx, float dy) {
    return literal_power(a, b, c, dx, dy);
}

static void raster_tile_fwd(int64_t tile, int C, const float* means2d,
                            const float* conics, const float* opacities,
                            const float* feats, const float* depths,
                            const int32_t* ids, const int32_t* ranges,
                            const float* bg, int width, int height,
                            int tiles_x, float* out, float* final_T,
                            int32_t* n_contrib, float* depth_out, int arith) {
    const int tx = (int)(tile % tiles_x), ty = (int)(tile / tiles_x);
    const int start = ranges[2 * tile], num = ranges[2 * tile + 1] - ranges[2 * tile];
    float acc[64];
    for (int ly = 0; ly < TILE; ++ly)
        for (int lx = 0; lx < TILE; ++lx) {
            const int px = tx * TILE + lx, py = ty * TILE + ly;
            if (px >= width || py >= height) continue;
            const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
            for (int c0 = 0; c0 < C; c0 += 64) {
                const int nc = (C - c0 < 64) ? C - c0 : 64;
                float T = 1.0f, dacc = 0.0f;
                int last = 0;
                for (int k = 0; k < nc; ++k) acc[k] = 0.0f;
                /* rasterize.py:60-88 */
                for (int j = 0; j < num; ++j) {
                    const int g = ids[start + j];
                    const float dx = means2d[2 * g] - pxf, dy = means2d[2 * g + 1] - pyf;
                    const float* cg = conics + 3 * g;
                    const float power =
                        (arith & ORC_ARITH_LITERAL_POWER)
                            ? literal_power(cg[0], cg[1], cg[2], dx, dy)
                            : orc_splat_power(cg[0], cg[1], cg[2], dx, dy);
                    if (power > 0.0f) continue;
                    const float e = (arith & ORC_ARITH_ROUNDED_EXP)
                                        ? (float)exp((double)power)
                                        : orc_splat_expf(power);
                    const float alpha = fminf(0.99f, opacities[g] * e);
                    if (alpha < 1.0f / 255.0f) continue;
                    const float next_T = T * (1.0f - alpha);
                    if (next_T < 1e-4f) break;
                    /* rasterize.py:84 `acc += rgb * (alpha * T)`, fused as Metal's
                     * default fast-math contraction compiles it */
                    const float w = alpha * T;
                    if (arith & ORC_ARITH_SEPARATE_ACC) {
                        for (int k = 0; k < nc; ++k) {
                            const float t = feats[(int64_t)g * C + c0 + k] * w;
                            acc[k] = acc[k] + t;
                        }
                        if (depths) {
                            const float t = depths[g] * w;
                            dacc = dacc + t;
                        }
                    } else {
                        for (int k = 0; k < nc; ++k)
                            acc[k] = fmaf(feats[(int64_t)g * C + c0 + k], w, acc[k]);
                        if (depths) dacc = fmaf(depths[g], w, dacc); /* rasterize.py:276-279 */
                    }
                    T = next_T;
                    last = j + 1;
                }
                const int64_t pid = (int64_t)py * width + px;
                for (int k = 0; k < nc; ++k) /* rasterize.py:90-96 */
                    out[pid * C + c0 + k] = acc[k] + T * (bg ? bg[c0 + k] : 0.0f);
                final_T[pid] = T;
                n_contrib[pid] = last;
                if (depth_out && c0 == 0) { /* rasterize.py:284-287 */
                    const float al = 1.0f - T;
                    depth_out[pid] = al > 1e-6f ? dacc / al : 0.0f;
                }
            }
        }
}

void orc_raster_fwd(int64_t n, int C, const float* means2d,
                    const float* conics, const float* opacities,
                    const float* feats, const float* depths,
                    const int32_t* sorted_ids, const int32_t* tile_ranges,
                    const float* bg, int width, int height, float* out,
                    float* final_T, int32_t* n_contrib, float* depth_out,
                    const int32_t* tiles, int64_t n_tiles, int nthreads) {
    orc_raster_fwd_arith(n, C, means2d, conics, opacities, feats, depths, sorted_ids,
                         tile_ranges, bg, width, height, out, final_T, n_contrib, depth_out,
                         tiles, n_tiles, nthreads, 0);
}

void orc_raster_fwd_arith(int64_t n, int C, const float* means2d,
                          const float* conics, const float* opacities,
                          const float* feats, const float* depths,
                          const int32_t* sorted_ids, const int32_t* tile_ranges,
                          const float* bg, int width, int height, float* out,
                          float* final_T, int32_t* n_contrib, float* depth_out,
                          const int32_t* tiles, int64_t n_tiles, int nthreads, int arith) {
    (void)n;
    const int tiles_x = (width + TILE - 1) / TILE;
    const int tiles_y = (height + TILE - 1) / TILE;
    const int64_t T = tiles ? n_tiles : (int64_t)tiles_x * tiles_y;
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(dynamic, 4)
    for (int64_t i = 0; i < T; ++i) {
        const int64_t tile = tiles ? tiles[i] : i;
        raster_tile_fwd(tile, C, means2d, conics, opacities, feats, depths, sorted_ids,
                        tile_ranges, bg, width, height, tiles_x, out, final_T, n_contrib,
                        depth_out, arith);
    }
}

/* rasterize.py:100-221 with the vjp wiring of :364-403.  Per-pair values are
 * computed in float32 exactly as the kernel does; sums accumulate in double
 * (the reference sums with unordered float atomics, so its order is not
 * defined anyway). */
void orc_raster_bwd(int64_t n, int C, const float* means2d,
                    const float* conics, const float* opacities,
                    const float* feats, const int32_t* sorted_ids,
                    const int32_t* tile_ranges, const float* bg, int width,
                    int height, const float* final_T,
                    const int32_t* n_contrib, const float* grad_out,
                    const float* grad_final_T, float* g_means2d,
                    float* g_conics, float* g_feats, float* g_opac,
                    int nthreads) {
    const int tiles_x = (width + TILE - 1) / TILE;
    const int tiles_y = (height + TILE - 1) / TILE;
    const int64_t T = (int64_t)tiles_x * tiles_y;
    const int nt = clamp_threads(nthreads);
    const int64_t stride = 6 + C;
    double* buf = (double*)calloc((size_t)nt * (size_t)n * (size_t)stride, sizeof(double));
#pragma omp parallel num_threads(nt)
    {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        double* gb = buf + (size_t)tid * (size_t)n * (size_t)stride;
        float* gpix = (float*)malloc(sizeof(float) * (size_t)C);
        float* accum = (float*)malloc(sizeof(float) * (size_t)C);
        float* lastc = (float*)malloc(sizeof(float) * (size_t)C);
#pragma omp for schedule(dynamic, 4)
        for (int64_t tile = 0; tile < T; ++tile) {
            const int tx = (int)(tile % tiles_x), ty = (int)(tile / tiles_x);
            const int start = tile_ranges[2 * tile];
            for (int ly = 0; ly < TILE; ++ly)
                for (int lx = 0; lx < TILE; ++lx) {
                    const int px = tx * TILE + lx, py = ty * TILE + ly;
                    if (px >= width || py >= height) continue;
                    const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
                    const int64_t pid = (int64_t)py * width + px;
                    const float T_final = final_T[pid];
                    float Tc = T_final;
                    const int last = n_contrib[pid];
                    float bg_dot = 0.0f;
                    for (int k = 0; k < C; ++k) {
                        gpix[k] = grad_out[pid * C + k];
                        bg_dot = bg_dot + (bg ? bg[k] : 0.0f) * gpix[k];
                        accum[k] = 0.0f;
                        lastc[k] = 0.0f;
                    }
                    bg_dot = bg_dot + (grad_final_T ? grad_final_T[pid] : 0.0f);
                    float last_alpha = 0.0f;
                    for (int j = last - 1; j >= 0; --j) {
                        const int g = sorted_ids[start + j];
                        const float dx = means2d[2 * g] - pxf, dy = means2d[2 * g + 1] - pyf;
                        const float a = conics[3 * g], b = conics[3 * g + 1], c = conics[3 * g + 2];
                        const float o = opacities[g];
                        const float power = orc_splat_power(a, b, c, dx, dy);
                        if (power > 0.0f) continue;
                        const float G = orc_splat_expf(power);
                        const float alpha = fminf(0.99f, o * G);
                        if (alpha < 1.0f / 255.0f) continue;
                        Tc = Tc / (1.0f - alpha);
                        const float aT = alpha * Tc;
                        const float* f = feats + (int64_t)g * C;
                        float dl = 0.0f;
                        for (int k = 0; k < C; ++k) {
                            accum[k] = last_alpha * lastc[k] + (1.0f - last_alpha) * accum[k];
                            lastc[k] = f[k];
                            dl = dl + (f[k] - accum[k]) * gpix[k];
                        }
                        last_alpha = alpha;
                        float dL_dalpha = dl * Tc;
                        dL_dalpha += (-T_final / (1.0f - alpha)) * bg_dot;
                        const float dL_dG = o * dL_dalpha;
                        const float gdx = G * dx, gdy = G * dy;
                        double* e = gb + (int64_t)g * stride;
                        e[0] += -(gdx * a + gdy * b) * dL_dG;
                        e[1] += -(gdy * c + gdx * b) * dL_dG;
                        e[2] += -0.5f * gdx * dx * dL_dG;
                        e[3] += -gdx * dy * dL_dG;
                        e[4] += -0.5f * gdy * dy * dL_dG;
                        e[5] += G * dL_dalpha;
                        for (int k = 0; k < C; ++k) e[6 + k] += aT * gpix[k];
                    }
                }
        }
        free(gpix);
        free(accum);
        free(lastc);
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t g = 0; g < n; ++g) {
        double v[6 + 64];
        for (int64_t k = 0; k < stride && k < 70; ++k) v[k] = 0.0;
        double* vv = (stride <= 70) ? v : (double*)calloc((size_t)stride, sizeof(double));
        for (int t = 0; t < nt; ++t) {
            const double* e = buf + ((size_t)t * (size_t)n + (size_t)g) * (size_t)stride;
            for (int64_t k = 0; k < stride; ++k) vv[k] += e[k];
        }
        g_means2d[2 * g] = (float)vv[0];
        g_means2d[2 * g + 1] = (float)vv[1];
        g_conics[3 * g] = (float)vv[2];
        g_conics[3 * g + 1] = (float)vv[3];
        g_conics[3 * g + 2] = (float)vv[4];
        g_opac[g] = (float)vv[5];
        for (int k = 0; k < C; ++k) g_feats[(int64_t)g * C + k] = (float)vv[6 + k];
        if (vv != v) free(vv);
    }
    free(buf);
}
