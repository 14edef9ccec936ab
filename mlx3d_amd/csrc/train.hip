// train.hip -- the training step around the rasterizer on gfx950:
//
//   * photometric loss: mean |pred - target| and mean SSIM in one pass over
//     the image (trainer.py:302-305; losses/image_metrics.py:23-55, 66-85),
//     with the analytic gradient of both in a second pass;
//   * Adam over several parameter groups in one launch (trainer.py:101-128,
//     339-342; mlx.optimizers.Adam, mlx >= 0.31);
//   * the screen-space gradient statistics of adaptive density control
//     (trainer.py:357-366).
//
// All of it is HBM-bound elementwise or stencil work: no MFMA, coalesced
// loads, LDS tiles for the 2D window.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "gsx.h"
#include "gsx_device.h"

namespace {

using gsx::kWave;

// ------------------------------------------------------------------- SSIM --
//
// mu_p = F(p), mu_t = F(t), E_pp = F(p p), E_tt = F(t t), E_pt = F(p t), with
// F the zero-padded 'same' correlation with the separable Gaussian window
// g g^T (image_metrics.py:23-45; mx.conv2d with padding = window // 2 pads
// with zeros).  Per pixel and channel
//   A = 2 mu_p mu_t + c1, B = mu_p^2 + mu_t^2 + c1,
//   Cn = 2 (E_pt - mu_p mu_t) + c2, D = (E_pp - mu_p^2) + (E_tt - mu_t^2) + c2,
//   S = (A / B) (Cn / D)                                 (image_metrics.py:47-54)
// and the loss uses mean(S) over every pixel and channel.  The forward keeps
// the partial derivatives of S with respect to (mu_p, E_pp, E_pt):
//   dS/dE_pt = 2 l / D,   dS/dE_pp = -l cs / D,
//   dS/dmu_p = 2 (mu_t - l mu_p) cs / B + 2 l (mu_p cs - mu_t) / D,
// (l = A / B, cs = Cn / D), and the backward applies F^T, which equals F for
// a symmetric window with zero padding:
//   dS_mean/dp = (F(dS/dmu_p) + 2 p F(dS/dE_pp) + t F(dS/dE_pt)) / n.

constexpr int kSsMaxR = 7;   // window radius up to 7 (15 taps)
constexpr int kSsMaxCh = 4;  // channels per launch
constexpr int kSsWaves = 4;  // strips (one per wave) per workgroup
constexpr int kSsThreads = kSsWaves * kWave;

struct SsimWindow {
    float g[2 * kSsMaxR + 1];
};

// Strip geometry.  A wave owns ssim_cols(CH) image columns of CH channels
// (lane = column * CH + channel) and walks down ssim_rows(R) input rows,
// which complete ssim_rows(R) - 2R output rows.  The input rows come in
// chunks of the window length K = 2R + 1, so the ring of the last K rows'
// horizontal sums is indexed by compile-time constants.  Each row is read
// once from global memory (the window's halo rows and columns being the only
// re-reads: (K - 1) / ssim_rows(R) and 2R / ssim_cols(CH) of the strip).
constexpr int ssim_cols(int ch) { return kWave / ch; }
constexpr int ssim_rows(int r) { return (2 * r + 1) * ((44 + 2 * r) / (2 * r + 1)); }

// Strip and lane bookkeeping shared by the two kernels.
template <int R, int CH>
struct SsimStrip {
    static constexpr int K = 2 * R + 1;
    static constexpr int COLS = ssim_cols(CH);
    static constexpr int SPAN = (COLS + 2 * R) * CH;  // floats of one input row
    static constexpr int NL = (SPAN + kWave - 1) / kWave;  // row floats per lane
    static constexpr int ROWS = ssim_rows(R);
    static constexpr int TB = ROWS - 2 * R;  // output rows
    int x0, y0, xl, ch;
    bool col_out;          // the lane's output column exists
    int off[NL];           // offsets of the lane's row elements within an image row
    bool ok[NL];           // and whether they lie inside the image
    __device__ SsimStrip(int strip, int strips_x, int W, int C, int c0, int lane) {
        const int sx = strip % strips_x, sy = strip / strips_x;
        x0 = sx * COLS;
        y0 = sy * TB;
        xl = lane / CH;
        ch = lane - xl * CH;
        col_out = xl < COLS && x0 + xl < W;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int e = lane + kWave * j, col = e / CH, c = e - col * CH;
            const int gx = x0 - R + col;
            ok[j] = e < SPAN && gx >= 0 && gx < W;
            off[j] = ok[j] ? gx * C + c0 + c : 0;
        }
    }
    // index of tap k of the lane's column in a staged row
    __device__ int tap(int k) const { return (xl + k) * CH + ch; }
};

// One input row of one array into registers (zero outside the image).  The
// loads are unconditional (outside the image they read element 0 and the
// value is dropped): loads under branches would make the compiler wait for
// every outstanding load, the prefetched rows included, at the next use.
template <int NL>
__device__ __forceinline__ void ssim_fetch(const float* __restrict__ src, int64_t row_base,
                                           bool row_ok, const int (&off)[NL],
                                           const bool (&ok)[NL], float (&v)[NL]) {
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const bool in = row_ok && ok[j];
        const float x = src[in ? row_base + off[j] : 0];
        v[j] = in ? x : 0.0f;
    }
}

// Keeps the compiler from moving the wave's LDS row accesses across the
// point (lanes read what other lanes of the wave wrote; the hardware
// executes one wave's LDS operations in order).
__device__ __forceinline__ void wave_lds_order() { asm volatile("" ::: "memory"); }

template <int R, int CH>
__global__ __launch_bounds__(kSsThreads) void k_ssim_fwd(
    const float* __restrict__ pred, const float* __restrict__ tgt, int H, int W, int C, int c0,
    int strips_x, int n_strips, SsimWindow win, float c1, float c2, float* __restrict__ maps,
    float* __restrict__ partials) {
    using S = SsimStrip<R, CH>;
    constexpr int K = S::K, NL = S::NL;
    __shared__ float s_row[kSsWaves][2][NL * kWave];
    __shared__ float s_red[2][kSsWaves];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int strip = (int)gsx::xcd_remap(blockIdx.x, gridDim.x) * kSsWaves + wave;
    float l1 = 0.0f, ssum = 0.0f;
    if (strip < n_strips) {
        const S s(strip, strips_x, W, C, c0, lane);
        float* sp = s_row[wave][0];
        float* stt = s_row[wave][1];
        const int64_t plane = (int64_t)H * W * C;
        const int64_t rstride = (int64_t)W * C;
        // rows i + 1 and i + 2 in flight while row i is filtered
        float p0[NL], t0[NL], p1[NL], t1[NL], p2[NL], t2[NL];
        auto fetch = [&](int i, float (&vp)[NL], float (&vt)[NL]) {
            const int gy = s.y0 - R + i;
            const bool row_ok = i < S::ROWS && gy >= 0 && gy < H;
            const int64_t base = row_ok ? (int64_t)gy * rstride : 0;
            ssim_fetch<NL>(pred, base, row_ok, s.off, s.ok, vp);
            ssim_fetch<NL>(tgt, base, row_ok, s.off, s.ok, vt);
        };
        fetch(0, p1, t1);
        fetch(1, p2, t2);
        float ring[K][5];  // horizontal sums of the last K rows: p, t, pp, tt, pt
#pragma unroll 1
        for (int i0 = 0; i0 < S::ROWS; i0 += K) {
#pragma unroll
            for (int u = 0; u < K; ++u) {
                const int i = i0 + u;
#pragma unroll
                for (int j = 0; j < NL; ++j) {
                    p0[j] = p1[j];
                    t0[j] = t1[j];
                    p1[j] = p2[j];
                    t1[j] = t2[j];
                }
                fetch(i + 2, p2, t2);
                wave_lds_order();
#pragma unroll
                for (int j = 0; j < NL; ++j) {
                    sp[lane + kWave * j] = p0[j];
                    stt[lane + kWave * j] = t0[j];
                }
                wave_lds_order();
                float a = 0.0f, b = 0.0f, pp = 0.0f, tt = 0.0f, pt = 0.0f, pc = 0.0f, tc = 0.0f;
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    const float w = win.g[k], p = sp[s.tap(k)], t = stt[s.tap(k)];
                    if (k == R) {
                        pc = p;
                        tc = t;
                    }
                    a = fmaf(w, p, a);
                    b = fmaf(w, t, b);
                    pp = fmaf(w, p * p, pp);
                    tt = fmaf(w, t * t, tt);
                    pt = fmaf(w, p * t, pt);
                }
                ring[u][0] = a;
                ring[u][1] = b;
                ring[u][2] = pp;
                ring[u][3] = tt;
                ring[u][4] = pt;
                // |p - t| at the centre of output row i - R
                const int oc = i - R;
                if (s.col_out && oc >= 0 && oc < S::TB && s.y0 + oc < H) l1 += fabsf(pc - tc);
                // output row o = i - 2R: rows o .. i sit in ring slots (u + 1 + k) mod K
                const int o = i - 2 * R;
                if (o >= 0 && o < S::TB) {
                    float mp = 0.0f, mt = 0.0f, epp = 0.0f, ett = 0.0f, ept = 0.0f;
#pragma unroll
                    for (int k = 0; k < K; ++k) {
                        const int q = (u + 1 + k) % K;
                        const float w = win.g[k];
                        mp = fmaf(w, ring[q][0], mp);
                        mt = fmaf(w, ring[q][1], mt);
                        epp = fmaf(w, ring[q][2], epp);
                        ett = fmaf(w, ring[q][3], ett);
                        ept = fmaf(w, ring[q][4], ept);
                    }
                    const int y = s.y0 + o;
                    if (s.col_out && y < H) {
                        const float mpp = mp * mp, mtt = mt * mt, mpt = mp * mt;
                        const float A = 2.0f * mpt + c1, B = mpp + mtt + c1;
                        const float Cn = 2.0f * (ept - mpt) + c2, D = (epp - mpp) + (ett - mtt) + c2;
                        // reciprocals to about 1 ulp (the loss is compared in
                        // float32 against a double-precision restatement)
                        const float rB = __builtin_amdgcn_rcpf(B), rD = __builtin_amdgcn_rcpf(D);
                        const float cs = Cn * rD, l = A * rB;
                        ssum += l * cs;
                        const int64_t pix = (int64_t)y * rstride + (int64_t)(s.x0 + s.xl) * C + c0 +
                                            s.ch;
                        maps[pix] = 2.0f * (mt - l * mp) * cs * rB + 2.0f * l * (mp * cs - mt) * rD;
                        maps[plane + pix] = -l * cs * rD;
                        maps[2 * plane + pix] = 2.0f * l * rD;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        l1 += __shfl_xor(l1, o, kWave);
        ssum += __shfl_xor(ssum, o, kWave);
    }
    if (lane == 0) {
        s_red[0][wave] = l1;
        s_red[1][wave] = ssum;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int w = 0; w < kSsWaves; ++w) {
            a += s_red[0][w];
            b += s_red[1][w];
        }
        partials[2 * (int64_t)blockIdx.x] = a;
        partials[2 * (int64_t)blockIdx.x + 1] = b;
    }
}

// The trainer's objective (1 - lambda) L1 + lambda (1 - SSIM) from the two
// means, in the float32 steps torch takes for it (trainer.py:303-305 with
// lambda a Python float): c_l1 = (float)(1 - lambda), c_ss = (float)lambda.
struct LossMix {
    float c_l1, c_ss;
    bool on;
};

// Sums the per-tile partials in a fixed order (double accumulators) and
// writes the first nout of [mean |pred - target|, mean SSIM]; with mix.on
// also out[2] = the mixed objective.
__global__ __launch_bounds__(256) void k_loss_reduce(const float* __restrict__ partials,
                                                     int64_t nblk, double inv_n,
                                                     float* __restrict__ out, int nout,
                                                     LossMix mix) {
    __shared__ double s[2][256];
    double a = 0.0, b = 0.0;
    // each thread adds partials threadIdx.x + 256 k in increasing k; the
    // loads of eight of them are issued together
    constexpr int kBatch = 8;
    for (int64_t i0 = threadIdx.x; i0 < nblk; i0 += 256 * kBatch) {
        float2 v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {  // unconditional (clamped) loads
            const int64_t i = min(i0 + 256 * k, nblk - 1);
            v[k] = *reinterpret_cast<const float2*>(partials + 2 * i);
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            if (i0 + 256 * k < nblk) {
                a += (double)v[k].x;
                b += (double)v[k].y;
            }
        }
    }
    s[0][threadIdx.x] = a;
    s[1][threadIdx.x] = b;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) {
            s[0][threadIdx.x] += s[0][threadIdx.x + w];
            s[1][threadIdx.x] += s[1][threadIdx.x + w];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float l1 = (float)(s[0][0] * inv_n), ss = (float)(s[1][0] * inv_n);
        out[0] = l1;
        if (nout > 1) out[1] = ss;
        if (mix.on) out[2] = mix.c_l1 * l1 + mix.c_ss * (1.0f - ss);
    }
}

// grad_pred = g_l1 sign(p - t) / n + g_ssim (F(dmu) + 2 p F(dpp) + t F(dpt)) / n,
// F over the three maps in the strip walk of k_ssim_fwd.
template <int R, int CH>
__global__ __launch_bounds__(kSsThreads) void k_ssim_bwd(
    const float* __restrict__ pred, const float* __restrict__ tgt, int H, int W, int C, int c0,
    int strips_x, int n_strips, SsimWindow win, const float* __restrict__ maps,
    const float* __restrict__ grad_in, LossMix mix, float inv_n, float* __restrict__ grad) {
    using S = SsimStrip<R, CH>;
    constexpr int K = S::K, NL = S::NL;
    __shared__ float s_row[kSsWaves][3][NL * kWave];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int strip = (int)gsx::xcd_remap(blockIdx.x, gridDim.x) * kSsWaves + wave;
    if (strip >= n_strips) return;
    const S s(strip, strips_x, W, C, c0, lane);
    // (g_l1, g_ssim): given, or from the mixed objective's cotangent g as
    // autograd forms them: (g c_l1, -(g c_ss))
    const float g_l1 = mix.on ? grad_in[0] * mix.c_l1 : grad_in[0];
    const float g_ss = mix.on ? -(grad_in[0] * mix.c_ss) : grad_in[1];
    const float gl = g_l1 * inv_n, gs = g_ss * inv_n;
    const int64_t plane = (int64_t)H * W * C;
    const int64_t rstride = (int64_t)W * C;
    const int64_t col = (int64_t)(s.x0 + s.xl) * C + c0 + s.ch;
    float* sm[3] = {s_row[wave][0], s_row[wave][1], s_row[wave][2]};
    // row i + 1 and i + 2 of the maps in flight, with pred and target at
    // the output pixel those rows complete
    struct Row {
        float m[3][NL];
        float p, t;
    };
    Row r0, r1, r2;
    auto fetch = [&](int i, Row& v) {
        const int gy = s.y0 - R + i;
        const bool row_ok = i < S::ROWS && gy >= 0 && gy < H;
        const int64_t base = row_ok ? (int64_t)gy * rstride : 0;
#pragma unroll
        for (int q = 0; q < 3; ++q) ssim_fetch<NL>(maps + q * plane, base, row_ok, s.off, s.ok, v.m[q]);
        const int yo = s.y0 + i - 2 * R;
        const bool out_ok = s.col_out && i >= 2 * R && i < S::ROWS && yo < H;
        const int64_t pix = out_ok ? (int64_t)yo * rstride + col : 0;
        v.p = pred[pix];  // element 0 when out_ok is false: unused
        v.t = tgt[pix];
    };
    fetch(0, r1);
    fetch(1, r2);
    float ring[K][3];
#pragma unroll 1
    for (int i0 = 0; i0 < S::ROWS; i0 += K) {
#pragma unroll
        for (int u = 0; u < K; ++u) {
            const int i = i0 + u;
            r0 = r1;
            r1 = r2;
            fetch(i + 2, r2);
            wave_lds_order();
#pragma unroll
            for (int q = 0; q < 3; ++q)
#pragma unroll
                for (int j = 0; j < NL; ++j) sm[q][lane + kWave * j] = r0.m[q][j];
            wave_lds_order();
            float a = 0.0f, b = 0.0f, d = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float w = win.g[k];
                a = fmaf(w, sm[0][s.tap(k)], a);
                b = fmaf(w, sm[1][s.tap(k)], b);
                d = fmaf(w, sm[2][s.tap(k)], d);
            }
            ring[u][0] = a;
            ring[u][1] = b;
            ring[u][2] = d;
            const int o = i - 2 * R;
            if (o >= 0 && o < S::TB) {
                float fm = 0.0f, fpp = 0.0f, fpt = 0.0f;
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    const int q = (u + 1 + k) % K;
                    const float w = win.g[k];
                    fm = fmaf(w, ring[q][0], fm);
                    fpp = fmaf(w, ring[q][1], fpp);
                    fpt = fmaf(w, ring[q][2], fpt);
                }
                const int y = s.y0 + o;
                if (s.col_out && y < H) {
                    const float p = r0.p, t = r0.t;
                    const float sgn = (float)((p > t) - (p < t));
                    const float gss = fm + 2.0f * p * fpp + t * fpt;
                    grad[(int64_t)y * rstride + col] = fmaf(gs, gss, gl * sgn);
                }
            }
        }
    }
}

// ------------------------------------------------------------------- Adam --
//
// mlx.optimizers.Adam.apply_single without bias correction (the default):
//   m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g^2;  p = p - lr m / (sqrt(v) + eps)
// in float32, each operation rounded once, in this order.

constexpr int kAdamMaxGroups = GSX_ADAM_MAX_GROUPS;
constexpr int kAdamThreads = 512;
constexpr int kAdamPerBlock = kAdamThreads * 4;  // four floats per thread

struct AdamArgs {
    float* p[kAdamMaxGroups];
    const float* g[kAdamMaxGroups];
    float* m[kAdamMaxGroups];
    float* v[kAdamMaxGroups];
    int64_t n[kAdamMaxGroups];
    float lr[kAdamMaxGroups];
    int64_t blk[kAdamMaxGroups + 1];
    int32_t vec[kAdamMaxGroups];
    int32_t count;
};

__device__ __forceinline__ void adam_one(float& p, float g, float& m, float& v, float lr, float b1,
                                         float omb1, float b2, float omb2, float eps) {
    gsx::adam_update(p, g, m, v, lr, b1, omb1, b2, omb2, eps);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Every element is read and written once per step, far more data than the
// caches hold: non-temporal loads and stores keep the stream from evicting
// other data (measured on MI355X: 5.4 -> 5.7-6.1 TB/s on 59M-float groups).
__global__ __launch_bounds__(kAdamThreads) void k_adam(AdamArgs a, float b1, float omb1, float b2,
                                                       float omb2, float eps) {
    const int64_t b = blockIdx.x;
    int gi = 0;
    while (gi + 1 < a.count && b >= a.blk[gi + 1]) ++gi;
    const int64_t n = a.n[gi];
    const int64_t i0 = (b - a.blk[gi]) * kAdamPerBlock + (int64_t)threadIdx.x * 4;
    if (i0 >= n) return;
    float* __restrict__ P = a.p[gi];
    const float* __restrict__ G = a.g[gi];
    float* __restrict__ M = a.m[gi];
    float* __restrict__ V = a.v[gi];
    const float lr = a.lr[gi];
    if (a.vec[gi] && i0 + 4 <= n) {
        const f32x4 p4 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(P + i0));
        const f32x4 g4 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(G + i0));
        const f32x4 m4 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(M + i0));
        const f32x4 v4 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(V + i0));
        float p[4] = {p4.x, p4.y, p4.z, p4.w}, m[4] = {m4.x, m4.y, m4.z, m4.w};
        float v[4] = {v4.x, v4.y, v4.z, v4.w};
        const float g[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) adam_one(p[k], g[k], m[k], v[k], lr, b1, omb1, b2, omb2, eps);
        const f32x4 po = {p[0], p[1], p[2], p[3]}, mo = {m[0], m[1], m[2], m[3]};
        const f32x4 vo = {v[0], v[1], v[2], v[3]};
        __builtin_nontemporal_store(po, reinterpret_cast<f32x4*>(P + i0));
        __builtin_nontemporal_store(mo, reinterpret_cast<f32x4*>(M + i0));
        __builtin_nontemporal_store(vo, reinterpret_cast<f32x4*>(V + i0));
        return;
    }
    const int64_t i1 = std::min<int64_t>(i0 + 4, n);
    for (int64_t i = i0; i < i1; ++i) {
        float p = P[i], m = M[i], v = V[i];
        adam_one(p, G[i], m, v, lr, b1, omb1, b2, omb2, eps);
        P[i] = p;
        M[i] = m;
        V[i] = v;
    }
}

// ------------------------------------------- density-control statistics --
// trainer.py:358-365: gx = g_x (W / 2), gy = g_y (H / 2),
// accum += sqrt(gx gx + gy gy) * visible, count += visible, visible = radii > 0.
// g: (x, y) pairs `stride` floats apart.
__global__ __launch_bounds__(256) void k_accum_screen_grads(int64_t n, const float* __restrict__ g,
                                                            int stride,
                                                            const float* __restrict__ radii,
                                                            float half_w, float half_h,
                                                            float* __restrict__ accum,
                                                            float* __restrict__ count) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float2 d = *reinterpret_cast<const float2*>(g + (int64_t)stride * i);
    const float gx = d.x * half_w, gy = d.y * half_h;
    const float norm = sqrtf(gx * gx + gy * gy);
    const float vis = radii[i] > 0.0f ? 1.0f : 0.0f;
    accum[i] = accum[i] + norm * vis;
    count[i] = count[i] + vis;
}

// ------------------------------------------------------------ host side --

bool make_window(int32_t window_size, float sigma, SsimWindow& w) {
    if (window_size < 1 || window_size > 2 * kSsMaxR + 1 || (window_size & 1) == 0) return false;
    if (!(sigma > 0.0f) || !std::isfinite(sigma)) return false;
    // image_metrics.py:23-26 in float32: x = k - (size - 1) / 2,
    // g = exp(-(x x) / (2 sigma sigma)), g / sum(g).
    float g[2 * kSsMaxR + 1];
    float sum = 0.0f;
    const float half = (float)((window_size - 1) / 2.0);
    const float den = (float)(2.0 * (double)sigma * (double)sigma);
    for (int k = 0; k < window_size; ++k) {
        const float x = (float)k - half;
        g[k] = std::exp(-(x * x) / den);
        sum += g[k];
    }
    for (int k = 0; k < window_size; ++k) w.g[k] = g[k] / sum;
    for (int k = window_size; k < 2 * kSsMaxR + 1; ++k) w.g[k] = 0.0f;
    return true;
}

// Strips of a launch over `ch` channels with window radius r, and its
// workgroups (one partial pair each).
struct SsimGeom {
    int strips_x;
    int n_strips;
    int64_t blocks;
};
SsimGeom ssim_geom(int32_t H, int32_t W, int r, int ch) {
    const int cols = ssim_cols(ch), tb = ssim_rows(r) - 2 * r;
    SsimGeom g;
    g.strips_x = (W + cols - 1) / cols;
    const int64_t n = (int64_t)g.strips_x * ((H + tb - 1) / tb);
    g.n_strips = (int)std::min<int64_t>(n, 0x7FFFFFFF);
    g.blocks = (n + kSsWaves - 1) / kSsWaves;
    return g;
}

// Partial pairs one launch may write, over every window radius and channel
// count (the workspace does not depend on the window).
int64_t photometric_blocks(int32_t H, int32_t W) {
    int64_t m = 0;
    for (int r = 0; r <= kSsMaxR; ++r)
        for (int ch = 1; ch <= kSsMaxCh; ++ch) m = std::max(m, ssim_geom(H, W, r, ch).blocks);
    return m;
}

int64_t photometric_groups(int32_t C) { return (C + kSsMaxCh - 1) / kSsMaxCh; }

// ------------------------------------------------------------------ L1 --
// mean |pred - target| (image_metrics.py:13-14): each workgroup sums 4096
// elements (float4 loads) in double into its partial (k_loss_reduce adds
// the partials in a fixed order), and the gradient sign(pred - target) g/n
// in one elementwise pass.
constexpr int kL1Threads = 256, kL1Per = 16, kL1Block = kL1Threads * kL1Per;

// Sign code of d = pred - target, one byte per element: 0 for d > 0, 1 for
// d < 0, 2 for d == 0, 3 for NaN (the gradient is then d itself).
__device__ __forceinline__ uint32_t l1_sign_code(float d) {
    return d > 0.0f ? 0u : (d < 0.0f ? 1u : (d == 0.0f ? 2u : 3u));
}

template <bool VEC>
__global__ __launch_bounds__(kL1Threads) void k_l1_partial(int64_t n,
                                                           const float* __restrict__ p,
                                                           const float* __restrict__ t,
                                                           float* __restrict__ partials,
                                                           uint8_t* __restrict__ signs) {
    __shared__ double s[kL1Threads];
    const int64_t base = (int64_t)blockIdx.x * kL1Block;
    double acc = 0.0;
    if (VEC && base + kL1Block <= n) {
        // a whole block: every load issued before the sums (same order)
        float4 a[kL1Per / 4], b[kL1Per / 4];
#pragma unroll
        for (int k = 0; k < kL1Per / 4; ++k) {
            const int64_t i = base + 4 * ((int64_t)k * kL1Threads + threadIdx.x);
            a[k] = *reinterpret_cast<const float4*>(p + i);
            b[k] = *reinterpret_cast<const float4*>(t + i);
        }
#pragma unroll
        for (int k = 0; k < kL1Per / 4; ++k) {
            const int64_t i = base + 4 * ((int64_t)k * kL1Threads + threadIdx.x);
            const float4 d = make_float4(a[k].x - b[k].x, a[k].y - b[k].y, a[k].z - b[k].z,
                                         a[k].w - b[k].w);
            acc += (double)fabsf(d.x) + (double)fabsf(d.y) + (double)fabsf(d.z) +
                   (double)fabsf(d.w);
            if (signs)
                *reinterpret_cast<uint32_t*>(signs + i) =
                    l1_sign_code(d.x) | (l1_sign_code(d.y) << 8) | (l1_sign_code(d.z) << 16) |
                    (l1_sign_code(d.w) << 24);
        }
    } else {
#pragma unroll
    for (int k = 0; k < kL1Per / 4; ++k) {
        const int64_t i = base + 4 * ((int64_t)k * kL1Threads + threadIdx.x);
        if (VEC && i + 3 < n) {
            const float4 a = *reinterpret_cast<const float4*>(p + i);
            const float4 b = *reinterpret_cast<const float4*>(t + i);
            const float4 d = make_float4(a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w);
            acc += (double)fabsf(d.x) + (double)fabsf(d.y) + (double)fabsf(d.z) +
                   (double)fabsf(d.w);
            if (signs)  // VEC: 4-byte aligned
                *reinterpret_cast<uint32_t*>(signs + i) =
                    l1_sign_code(d.x) | (l1_sign_code(d.y) << 8) | (l1_sign_code(d.z) << 16) |
                    (l1_sign_code(d.w) << 24);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (i + e < n) {
                    const float d = p[i + e] - t[i + e];
                    acc += (double)fabsf(d);
                    if (signs) signs[i + e] = (uint8_t)l1_sign_code(d);
                }
            }
        }
    }
    }
    s[threadIdx.x] = acc;
    __syncthreads();
    for (int w = kL1Threads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) s[threadIdx.x] += s[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        partials[2 * blockIdx.x] = (float)s[0];
        partials[2 * blockIdx.x + 1] = 0.0f;
    }
}

// grad = sign(pred - target) * (g / n); sign(0) = 0, NaN differences give NaN
template <bool VEC>
__global__ __launch_bounds__(kL1Threads) void k_l1_bwd(int64_t n, const float* __restrict__ p,
                                                       const float* __restrict__ t,
                                                       const float* __restrict__ g, float nf,
                                                       float* __restrict__ grad) {
    const float sc = g[0] / nf;
    auto sgn = [&](float d) { return d > 0.0f ? sc : (d < 0.0f ? -sc : (d == 0.0f ? 0.0f : d)); };
    const int64_t base = (int64_t)blockIdx.x * kL1Block;
#pragma unroll
    for (int k = 0; k < kL1Per / 4; ++k) {
        const int64_t i = base + 4 * ((int64_t)k * kL1Threads + threadIdx.x);
        if (VEC && i + 3 < n) {
            const float4 a = *reinterpret_cast<const float4*>(p + i);
            const float4 b = *reinterpret_cast<const float4*>(t + i);
            *reinterpret_cast<float4*>(grad + i) =
                make_float4(sgn(a.x - b.x), sgn(a.y - b.y), sgn(a.z - b.z), sgn(a.w - b.w));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (i + e < n) grad[i + e] = sgn(p[i + e] - t[i + e]);
        }
    }
}

// The same gradient from the sign codes k_l1_partial wrote: one byte read
// per element instead of two floats (pred and target are read only where
// the code is NaN).
template <bool VEC>
__global__ __launch_bounds__(kL1Threads) void k_l1_bwd_signs(int64_t n,
                                                             const uint8_t* __restrict__ signs,
                                                             const float* __restrict__ p,
                                                             const float* __restrict__ t,
                                                             const float* __restrict__ g,
                                                             float nf, float* __restrict__ grad) {
    const float sc = g[0] / nf;
    auto val = [&](uint32_t code, int64_t i) {
        return code == 0u ? sc : (code == 1u ? -sc : (code == 2u ? 0.0f : p[i] - t[i]));
    };
    const int64_t base = (int64_t)blockIdx.x * kL1Block;
    if (VEC && base + kL1Block <= n) {  // a whole block: the code loads issued together
        uint32_t c[kL1Per / 4];
#pragma unroll
        for (int k = 0; k < kL1Per / 4; ++k)
            c[k] = *reinterpret_cast<const uint32_t*>(
                signs + base + 4 * ((int64_t)k * kL1Threads + threadIdx.x));
#pragma unroll
        for (int k = 0; k < kL1Per / 4; ++k) {
            const int64_t i = base + 4 * ((int64_t)k * kL1Threads + threadIdx.x);
            *reinterpret_cast<float4*>(grad + i) =
                make_float4(val(c[k] & 0xFFu, i), val((c[k] >> 8) & 0xFFu, i + 1),
                            val((c[k] >> 16) & 0xFFu, i + 2), val(c[k] >> 24, i + 3));
        }
        return;
    }
#pragma unroll
    for (int k = 0; k < kL1Per / 4; ++k) {
        const int64_t i = base + 4 * ((int64_t)k * kL1Threads + threadIdx.x);
        if (VEC && i + 3 < n) {
            const uint32_t c = *reinterpret_cast<const uint32_t*>(signs + i);
            *reinterpret_cast<float4*>(grad + i) =
                make_float4(val(c & 0xFFu, i), val((c >> 8) & 0xFFu, i + 1),
                            val((c >> 16) & 0xFFu, i + 2), val(c >> 24, i + 3));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (i + e < n) grad[i + e] = val(signs[i + e], i + e);
        }
    }
}

inline int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

// Scratch of gsx_l1_fwd_noalloc: the per-workgroup partial sums of at most
// kL1NoAllocMaxN elements, in a file-scope device array instead of a
// caller workspace (512 KiB, held on every GPU the library runs on until the
// process ends).  Host code never hands the array's name to a kernel: the
// name is a host-side stand-in, so the kernels get the address that
// hipGetSymbolAddress reports for the current device.
constexpr int64_t kL1NoAllocMaxN = int64_t(1) << 28;
constexpr int64_t kL1NoAllocMaxBlocks = kL1NoAllocMaxN / kL1Block;
static __device__ __align__(256) float scratch[2 * kL1NoAllocMaxBlocks];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices];  // per device; filled once, under the mutex

// Address of `scratch` on `dev`, looked up once per device with that device
// current; nullptr if the lookup fails.
float* scratch_on(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p) return nullptr;
    g_scratch_ptr[dev] = static_cast<float*>(p);
    return g_scratch_ptr[dev];
}

// The L1 forward on given partials storage (the workspace or the scratch).
int l1_fwd_into(int64_t n, const float* pred, const float* target, float* partials,
                uint8_t* signs, float* out, hipStream_t st) {
    const int64_t nblk = (n + kL1Block - 1) / kL1Block;
    const bool vec =
        (((uintptr_t)pred | (uintptr_t)target) & 15u) == 0 && ((uintptr_t)signs & 3u) == 0;
    if (vec)
        hipLaunchKernelGGL(k_l1_partial<true>, dim3((unsigned)nblk), dim3(kL1Threads), 0, st, n,
                           pred, target, partials, signs);
    else
        hipLaunchKernelGGL(k_l1_partial<false>, dim3((unsigned)nblk), dim3(kL1Threads), 0, st, n,
                           pred, target, partials, signs);
    GSX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_loss_reduce, dim3(1), dim3(256), 0, st, (const float*)partials, nblk,
                       1.0 / (double)n, out, 1, LossMix{0.0f, 0.0f, false});
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

LossMix loss_mix(double lambda) {
    // the Python scalars 1 - lambda and lambda, each rounded once to float32
    return LossMix{(float)(1.0 - lambda), (float)lambda, true};
}

bool lambda_ok(double lambda) { return lambda >= 0.0 && lambda <= 1.0; }

int photometric_fwd(int32_t height, int32_t width, int32_t channels, const float* pred,
                    const float* target, int32_t window_size, float sigma, float max_val,
                    void* workspace, int64_t workspace_bytes, float* out, LossMix mix,
                    void* stream) {
    if (height <= 0 || width <= 0 || channels <= 0) return GSX_ERR_INVALID;
    if (!pred || !target || !out || !workspace) return GSX_ERR_INVALID;
    if ((int64_t)height * width * channels >= (int64_t(1) << 40)) return GSX_ERR_TOO_LARGE;
    SsimWindow win;
    if (!make_window(window_size, sigma, win)) return GSX_ERR_INVALID;
    if (workspace_bytes < gsx_photometric_workspace_bytes(height, width, channels))
        return GSX_ERR_WORKSPACE;
    // image_metrics.py:51-52
    const float c1 = (float)((0.01 * max_val) * (0.01 * max_val));
    const float c2 = (float)((0.03 * max_val) * (0.03 * max_val));
    float* maps = (float*)workspace;
    float* partials = (float*)((char*)workspace +
                               align256(3 * (int64_t)height * width * channels * 4));
    hipStream_t st = (hipStream_t)stream;
    int64_t n_part = 0;  // partial pairs written so far, launches back to back
    for (int c0 = 0; c0 < channels; c0 += kSsMaxCh) {
        const int nc = std::min(kSsMaxCh, channels - c0);
        const SsimGeom g = ssim_geom(height, width, window_size / 2, nc);
        if (g.blocks > 0x7FFFFFFF) return GSX_ERR_TOO_LARGE;
        float* part = partials + 2 * n_part;
        n_part += g.blocks;
        const int key = (window_size / 2) * 8 + nc;
        switch (key) {
#define GSX_SSIM_FWD(RR, CC)                                                                   \
    case RR * 8 + CC:                                                                          \
        hipLaunchKernelGGL((k_ssim_fwd<RR, CC>), dim3((unsigned)g.blocks), dim3(kSsThreads), 0, \
                           st, pred, target, height, width, channels, c0, g.strips_x,           \
                           g.n_strips, win, c1, c2, maps, part);                               \
        break;
#define GSX_SSIM_FWD_R(RR) GSX_SSIM_FWD(RR, 1) GSX_SSIM_FWD(RR, 2) GSX_SSIM_FWD(RR, 3) GSX_SSIM_FWD(RR, 4)
            GSX_SSIM_FWD_R(0)
            GSX_SSIM_FWD_R(1)
            GSX_SSIM_FWD_R(2)
            GSX_SSIM_FWD_R(3)
            GSX_SSIM_FWD_R(4)
            GSX_SSIM_FWD_R(5)
            GSX_SSIM_FWD_R(6)
            GSX_SSIM_FWD_R(7)
#undef GSX_SSIM_FWD_R
#undef GSX_SSIM_FWD
            default:
                return GSX_ERR_INVALID;
        }
        GSX_LAUNCH_CHECK();
    }
    const double inv_n = 1.0 / ((double)height * width * channels);
    hipLaunchKernelGGL(k_loss_reduce, dim3(1), dim3(256), 0, st, partials, n_part, inv_n, out,
                       2, mix);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int photometric_bwd(int32_t height, int32_t width, int32_t channels, const float* pred,
                    const float* target, int32_t window_size, float sigma,
                    const void* workspace, int64_t workspace_bytes, const float* grad_out,
                    LossMix mix, float* grad_pred, void* stream) {
    if (height <= 0 || width <= 0 || channels <= 0) return GSX_ERR_INVALID;
    if (!pred || !target || !workspace || !grad_out || !grad_pred) return GSX_ERR_INVALID;
    if ((int64_t)height * width * channels >= (int64_t(1) << 40)) return GSX_ERR_TOO_LARGE;
    SsimWindow win;
    if (!make_window(window_size, sigma, win)) return GSX_ERR_INVALID;
    if (workspace_bytes < gsx_photometric_workspace_bytes(height, width, channels))
        return GSX_ERR_WORKSPACE;
    const float inv_n = (float)(1.0 / ((double)height * width * channels));
    hipStream_t st = (hipStream_t)stream;
    const float* maps = (const float*)workspace;
    for (int c0 = 0; c0 < channels; c0 += kSsMaxCh) {
        const int nc = std::min(kSsMaxCh, channels - c0);
        const SsimGeom g = ssim_geom(height, width, window_size / 2, nc);
        if (g.blocks > 0x7FFFFFFF) return GSX_ERR_TOO_LARGE;
        const int key = (window_size / 2) * 8 + nc;
        switch (key) {
#define GSX_SSIM_BWD(RR, CC)                                                                   \
    case RR * 8 + CC:                                                                          \
        hipLaunchKernelGGL((k_ssim_bwd<RR, CC>), dim3((unsigned)g.blocks), dim3(kSsThreads), 0, \
                           st, pred, target, height, width, channels, c0, g.strips_x,           \
                           g.n_strips, win, maps, grad_out, mix, inv_n, grad_pred);            \
        break;
#define GSX_SSIM_BWD_R(RR) GSX_SSIM_BWD(RR, 1) GSX_SSIM_BWD(RR, 2) GSX_SSIM_BWD(RR, 3) GSX_SSIM_BWD(RR, 4)
            GSX_SSIM_BWD_R(0)
            GSX_SSIM_BWD_R(1)
            GSX_SSIM_BWD_R(2)
            GSX_SSIM_BWD_R(3)
            GSX_SSIM_BWD_R(4)
            GSX_SSIM_BWD_R(5)
            GSX_SSIM_BWD_R(6)
            GSX_SSIM_BWD_R(7)
#undef GSX_SSIM_BWD_R
#undef GSX_SSIM_BWD
            default:
                return GSX_ERR_INVALID;
        }
        GSX_LAUNCH_CHECK();
    }
    return GSX_OK;
}

}  // namespace

extern "C" {

int64_t gsx_photometric_workspace_bytes(int32_t height, int32_t width, int32_t channels) {
    if (height <= 0 || width <= 0 || channels <= 0) return 0;
    const int64_t maps = 3 * (int64_t)height * width * channels * (int64_t)sizeof(float);
    return align256(maps) + align256(2 * photometric_groups(channels) *
                                     photometric_blocks(height, width) * (int64_t)sizeof(float));
}


int gsx_photometric_fwd(int32_t height, int32_t width, int32_t channels, const float* pred,
                        const float* target, int32_t window_size, float sigma, float max_val,
                        void* workspace, int64_t workspace_bytes, float* out, void* stream) {
    return photometric_fwd(height, width, channels, pred, target, window_size, sigma, max_val,
                           workspace, workspace_bytes, out, LossMix{0.0f, 0.0f, false}, stream);
}

int gsx_photometric_bwd(int32_t height, int32_t width, int32_t channels, const float* pred,
                        const float* target, int32_t window_size, float sigma,
                        const void* workspace, int64_t workspace_bytes, const float* grad_out,
                        float* grad_pred, void* stream) {
    return photometric_bwd(height, width, channels, pred, target, window_size, sigma, workspace,
                           workspace_bytes, grad_out, LossMix{0.0f, 0.0f, false}, grad_pred,
                           stream);
}

int gsx_photometric_loss_fwd(int32_t height, int32_t width, int32_t channels, const float* pred,
                             const float* target, int32_t window_size, float sigma,
                             float max_val, double lambda, void* workspace,
                             int64_t workspace_bytes, float* out3, void* stream) {
    if (!lambda_ok(lambda)) return GSX_ERR_INVALID;
    return photometric_fwd(height, width, channels, pred, target, window_size, sigma, max_val,
                           workspace, workspace_bytes, out3, loss_mix(lambda), stream);
}

int gsx_photometric_loss_bwd(int32_t height, int32_t width, int32_t channels, const float* pred,
                             const float* target, int32_t window_size, float sigma,
                             double lambda, const void* workspace, int64_t workspace_bytes,
                             const float* g_loss, float* grad_pred, void* stream) {
    if (!lambda_ok(lambda)) return GSX_ERR_INVALID;
    return photometric_bwd(height, width, channels, pred, target, window_size, sigma, workspace,
                           workspace_bytes, g_loss, loss_mix(lambda), grad_pred, stream);
}

int64_t gsx_l1_workspace_bytes(int64_t n) {
    if (n <= 0) return 0;
    return align256(2 * ((n + kL1Block - 1) / kL1Block) * (int64_t)sizeof(float));
}

int gsx_l1_fwd(int64_t n, const float* pred, const float* target, void* workspace,
               int64_t workspace_bytes, float* out, void* stream) {
    if (n <= 0 || !pred || !target || !workspace || !out) return GSX_ERR_INVALID;
    if (workspace_bytes < gsx_l1_workspace_bytes(n)) return GSX_ERR_WORKSPACE;
    const int64_t nblk = (n + kL1Block - 1) / kL1Block;
    if (nblk > 0x7FFFFFFF) return GSX_ERR_TOO_LARGE;
    return l1_fwd_into(n, pred, target, (float*)workspace, nullptr, out, (hipStream_t)stream);
}

int gsx_l1_fwd_signs(int64_t n, const float* pred, const float* target, void* workspace,
                     int64_t workspace_bytes, uint8_t* signs, float* out, void* stream) {
    if (n <= 0 || !pred || !target || !workspace || !signs || !out) return GSX_ERR_INVALID;
    if (workspace_bytes < gsx_l1_workspace_bytes(n)) return GSX_ERR_WORKSPACE;
    const int64_t nblk = (n + kL1Block - 1) / kL1Block;
    if (nblk > 0x7FFFFFFF) return GSX_ERR_TOO_LARGE;
    return l1_fwd_into(n, pred, target, (float*)workspace, signs, out, (hipStream_t)stream);
}

int64_t gsx_l1_noalloc_max_elements(void) { return kL1NoAllocMaxN; }

int gsx_l1_fwd_noalloc(int64_t n, const float* pred, const float* target, float* out,
                       void* stream) {
    if (n <= 0 || !pred || !target || !out) return GSX_ERR_INVALID;
    if (n > kL1NoAllocMaxN) return GSX_ERR_TOO_LARGE;
    hipStream_t st = (hipStream_t)stream;
    int dev = -1;
    if (st) {
        hipDevice_t d;
        if (hipStreamGetDevice(st, &d) != hipSuccess) return GSX_ERR_HIP;
        dev = (int)d;
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return GSX_ERR_HIP;
    }
    float* partials = scratch_on(dev);
    if (!partials) return GSX_ERR_HIP;
    // every workgroup writes both of its partial words, and the reduction
    // reads only this call's nblk of them: nothing needs clearing first
    return l1_fwd_into(n, pred, target, partials, nullptr, out, st);
}

int gsx_l1_bwd(int64_t n, const float* pred, const float* target, const float* grad_out,
               float* grad_pred, void* stream) {
    if (n <= 0 || !pred || !target || !grad_out || !grad_pred) return GSX_ERR_INVALID;
    const int64_t nblk = (n + kL1Block - 1) / kL1Block;
    if (nblk > 0x7FFFFFFF) return GSX_ERR_TOO_LARGE;
    hipStream_t st = (hipStream_t)stream;
    const bool vec = (((uintptr_t)pred | (uintptr_t)target | (uintptr_t)grad_pred) & 15u) == 0;
    if (vec)
        hipLaunchKernelGGL(k_l1_bwd<true>, dim3((unsigned)nblk), dim3(kL1Threads), 0, st, n, pred,
                           target, grad_out, (float)n, grad_pred);
    else
        hipLaunchKernelGGL(k_l1_bwd<false>, dim3((unsigned)nblk), dim3(kL1Threads), 0, st, n,
                           pred, target, grad_out, (float)n, grad_pred);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_l1_bwd_signs(int64_t n, const uint8_t* signs, const float* pred, const float* target,
                     const float* grad_out, float* grad_pred, void* stream) {
    if (n <= 0 || !signs || !pred || !target || !grad_out || !grad_pred) return GSX_ERR_INVALID;
    const int64_t nblk = (n + kL1Block - 1) / kL1Block;
    if (nblk > 0x7FFFFFFF) return GSX_ERR_TOO_LARGE;
    hipStream_t st = (hipStream_t)stream;
    const bool vec = ((uintptr_t)grad_pred & 15u) == 0 && ((uintptr_t)signs & 3u) == 0;
    if (vec)
        hipLaunchKernelGGL(k_l1_bwd_signs<true>, dim3((unsigned)nblk), dim3(kL1Threads), 0, st,
                           n, signs, pred, target, grad_out, (float)n, grad_pred);
    else
        hipLaunchKernelGGL(k_l1_bwd_signs<false>, dim3((unsigned)nblk), dim3(kL1Threads), 0, st,
                           n, signs, pred, target, grad_out, (float)n, grad_pred);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_adam_step(int32_t num_groups, const gsx_adam_group* groups, float beta1, float beta2,
                  float eps, void* stream) {
    if (num_groups < 0 || num_groups > kAdamMaxGroups) return GSX_ERR_INVALID;
    if (num_groups > 0 && !groups) return GSX_ERR_INVALID;
    AdamArgs a{};
    int64_t blocks = 0;
    int count = 0;
    for (int i = 0; i < num_groups; ++i) {
        const gsx_adam_group& g = groups[i];
        if (g.n < 0) return GSX_ERR_INVALID;
        if (g.n == 0) continue;
        if (!g.param || !g.grad || !g.m || !g.v) return GSX_ERR_INVALID;
        a.p[count] = g.param;
        a.g[count] = g.grad;
        a.m[count] = g.m;
        a.v[count] = g.v;
        a.n[count] = g.n;
        a.lr[count] = g.lr;
        const uintptr_t any = (uintptr_t)g.param | (uintptr_t)g.grad | (uintptr_t)g.m |
                              (uintptr_t)g.v;
        a.vec[count] = (any & 15u) == 0;
        a.blk[count] = blocks;
        blocks += (g.n + kAdamPerBlock - 1) / kAdamPerBlock;
        ++count;
    }
    a.blk[count] = blocks;
    a.count = count;
    if (blocks == 0) return GSX_OK;
    if (blocks > 0x7fffffff) return GSX_ERR_TOO_LARGE;
    // (1 - b1) and (1 - b2) are formed in double and rounded once, as the
    // Python scalars of the reference reach the float32 arithmetic.
    const float omb1 = (float)(1.0 - (double)beta1), omb2 = (float)(1.0 - (double)beta2);
    hipLaunchKernelGGL(k_adam, dim3((unsigned)blocks), dim3(kAdamThreads), 0, (hipStream_t)stream, a,
                       beta1, omb1, beta2, omb2, eps);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_accum_screen_grads(int64_t n, const float* g_means2d, const float* radii, int32_t width,
                           int32_t height, float* grad_accum, float* grad_count,
                           int32_t grad_stride, void* stream) {
    if (n < 0 || width <= 0 || height <= 0) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!g_means2d || !radii || !grad_accum || !grad_count) return GSX_ERR_INVALID;
    if (((uintptr_t)g_means2d & 7u) != 0 || grad_stride < 0 || (grad_stride & 1) != 0)
        return GSX_ERR_INVALID;
    const unsigned blocks = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL(k_accum_screen_grads, dim3(blocks), dim3(256), 0, (hipStream_t)stream, n,
                       g_means2d, grad_stride > 0 ? (int)grad_stride : 2, radii,
                       (float)(width / 2.0), (float)(height / 2.0), grad_accum, grad_count);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // extern "C"
