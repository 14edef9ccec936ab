/*
 * train_oracle.c -- CPU restatement of the training-step pieces around the
 * rasterizer.  TEST INFRASTRUCTURE ONLY: used by tests/ as the checker;
 * nothing in the product package links, loads or calls it.
 *
 *   orc_photometric         -- losses/image_metrics.py:23-55, 66-85 (ssim)
 *                              and trainer.py:303 (mean L1), forward value
 *                              and gradient with respect to pred
 *   orc_adam                -- mlx.optimizers.Adam.apply_single (mlx >= 0.31,
 *                              bias_correction=False) as trainer.py:128,
 *                              339-342 use it
 *   orc_accum_screen_grads  -- trainer.py:357-365
 *
 * orc_photometric evaluates in double precision with the full 2D window
 * g g^T applied directly (not separably): it is the accuracy reference for
 * the float32 GPU kernels, which differ from it only by float32 rounding.
 * orc_adam and orc_accum_screen_grads use float32 in the reference's
 * operation order, each operation rounded once (-ffp-contract=off), so the
 * GPU must agree bit for bit.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "gsx_oracle.h"

/* image_metrics.py:23-26: x = k - (size-1)/2, g = exp(-x^2 / (2 sigma^2)),
 * normalised to sum 1. */
static void window1d(int size, double sigma, double* g) {
    double sum = 0.0;
    for (int k = 0; k < size; ++k) {
        const double x = (double)k - (size - 1) / 2.0;
        g[k] = exp(-(x * x) / (2.0 * sigma * sigma));
        sum += g[k];
    }
    for (int k = 0; k < size; ++k) g[k] /= sum;
}

/* 'same' correlation with the 2D window w2 (size x size), zero padding
 * (mx.conv2d(x, weight, padding=size//2, groups=C), image_metrics.py:38-39),
 * of one channel plane src (H*W, stride C) into dst (H*W). */
static void filter2d(int H, int W, int C, int c, const double* src, int size, const double* w2,
                     double* dst) {
    const int r = size / 2;
    for (int y = 0; y < H; ++y) {
        for (int x = 0; x < W; ++x) {
            double acc = 0.0;
            for (int i = 0; i < size; ++i) {
                const int yy = y + i - r;
                if (yy < 0 || yy >= H) continue;
                for (int j = 0; j < size; ++j) {
                    const int xx = x + j - r;
                    if (xx < 0 || xx >= W) continue;
                    acc += w2[i * size + j] * src[((int64_t)yy * W + xx) * C + c];
                }
            }
            dst[(int64_t)y * W + x] = acc;
        }
    }
}

void orc_photometric(int H, int W, int C, const float* pred, const float* target, int window,
                     double sigma, double max_val, double g_l1, double g_ssim, double* out,
                     double* grad) {
    const int64_t np = (int64_t)H * W, n = np * C;
    double g[64], w2[64 * 64];
    window1d(window, sigma, g);
    for (int i = 0; i < window; ++i)
        for (int j = 0; j < window; ++j) w2[i * window + j] = g[i] * g[j];
    const double c1 = (0.01 * max_val) * (0.01 * max_val);
    const double c2 = (0.03 * max_val) * (0.03 * max_val);

    double* p = (double*)malloc(sizeof(double) * n);
    double* t = (double*)malloc(sizeof(double) * n);
    double* pp = (double*)malloc(sizeof(double) * n);
    double* tt = (double*)malloc(sizeof(double) * n);
    double* pt = (double*)malloc(sizeof(double) * n);
    double* f[5];
    for (int q = 0; q < 5; ++q) f[q] = (double*)malloc(sizeof(double) * np);
    double* d[3];
    for (int q = 0; q < 3; ++q) d[q] = (double*)malloc(sizeof(double) * np);
    double* fd = (double*)malloc(sizeof(double) * np);
    for (int64_t i = 0; i < n; ++i) {
        p[i] = pred[i];
        t[i] = target[i];
        pp[i] = p[i] * p[i];
        tt[i] = t[i] * t[i];
        pt[i] = p[i] * t[i];
    }
    double l1 = 0.0, ssum = 0.0;
    for (int64_t i = 0; i < n; ++i) l1 += fabs(p[i] - t[i]);
    if (grad)
        for (int64_t i = 0; i < n; ++i)
            grad[i] = g_l1 * (double)((p[i] > t[i]) - (p[i] < t[i])) / (double)n;
    for (int c = 0; c < C; ++c) {
        const double* srcs[5] = {p, t, pp, tt, pt};
        for (int q = 0; q < 5; ++q) filter2d(H, W, C, c, srcs[q], window, w2, f[q]);
        for (int64_t i = 0; i < np; ++i) {
            /* image_metrics.py:41-54 */
            const double mp = f[0][i], mt = f[1][i];
            const double mpp = mp * mp, mtt = mt * mt, mpt = mp * mt;
            const double sp = f[2][i] - mpp, st = f[3][i] - mtt, spt = f[4][i] - mpt;
            const double A = 2.0 * mpt + c1, B = mpp + mtt + c1;
            const double Cn = 2.0 * spt + c2, D = sp + st + c2;
            const double cs = Cn / D, l = A / B;
            ssum += l * cs;
            /* partial derivatives of S with respect to (mu_p, E_pp, E_pt) */
            d[0][i] = 2.0 * (mt - l * mp) * cs / B + 2.0 * l * (mp * cs - mt) / D;
            d[1][i] = -l * cs / D;
            d[2][i] = 2.0 * l / D;
        }
        if (!grad) continue;
        /* adjoint of the zero-padded correlation with a symmetric window is
         * the same correlation */
        for (int q = 0; q < 3; ++q) {
            filter2d(H, W, 1, 0, d[q], window, w2, fd);
            for (int64_t i = 0; i < np; ++i) {
                const int64_t k = i * C + c;
                const double m = q == 0 ? 1.0 : (q == 1 ? 2.0 * p[k] : t[k]);
                grad[k] += g_ssim * m * fd[i] / (double)n;
            }
        }
    }
    out[0] = l1 / (double)n;
    out[1] = ssum / (double)n;
    free(p);
    free(t);
    free(pp);
    free(tt);
    free(pt);
    for (int q = 0; q < 5; ++q) free(f[q]);
    for (int q = 0; q < 3; ++q) free(d[q]);
    free(fd);
}

/* m = b1 m + (1 - b1) g; v = b2 v + (1 - b2) square(g);
 * p = p - lr m / (sqrt(v) + eps).  The Python scalars 1 - b1 and 1 - b2 are
 * evaluated in double and meet float32 arrays as float32. */
void orc_adam(int64_t n, float* p, const float* g, float* m, float* v, float lr, float b1,
              float b2, float eps) {
    const float omb1 = (float)(1.0 - (double)b1), omb2 = (float)(1.0 - (double)b2);
    for (int64_t i = 0; i < n; ++i) {
        const float gi = g[i];
        const float mi = b1 * m[i] + omb1 * gi;
        const float vi = b2 * v[i] + omb2 * (gi * gi);
        m[i] = mi;
        v[i] = vi;
        p[i] = p[i] - (lr * mi) / (sqrtf(vi) + eps);
    }
}

/* gx = g[:, 0] * (W / 2.0); gy = g[:, 1] * (H / 2.0); norms = sqrt(gx gx + gy gy);
 * visible = radii > 0; accum += norms * visible; count += visible. */
void orc_accum_screen_grads(int64_t n, const float* g, const float* radii, int W, int H,
                            float* accum, float* count) {
    const float hw = (float)(W / 2.0), hh = (float)(H / 2.0);
    for (int64_t i = 0; i < n; ++i) {
        const float gx = g[2 * i] * hw, gy = g[2 * i + 1] * hh;
        const float norm = sqrtf(gx * gx + gy * gy);
        const float vis = radii[i] > 0.0f ? 1.0f : 0.0f;
        accum[i] = accum[i] + norm * vis;
        count[i] = count[i] + vis;
    }
}
