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

constexpr int kSsT = 16;                  // output tile edge (16 x 16 threads)
constexpr int kSsThreads = kSsT * kSsT;
constexpr int kSsMaxR = 7;                // window radius up to 7 (15 taps)
constexpr int kSsMaxCh = 4;               // channels per launch

struct SsimWindow {
    float g[2 * kSsMaxR + 1];
};

template <int R>
struct SsimTile {
    static constexpr int kSpan = kSsT + 2 * R;
};

// Tile of this workgroup: linear ids go round-robin over the XCDs, and the
// remap gives each XCD a contiguous band of tiles, so the halo rows that
// neighbouring tiles share are fetched into one L2.
__device__ __forceinline__ void ssim_tile(int tiles_x, int& x0, int& y0) {
    const int t = (int)gsx::xcd_remap(blockIdx.x, gridDim.x);
    x0 = (t % tiles_x) * kSsT;
    y0 = (t / tiles_x) * kSsT;
}

// Loads channels [c0, c0 + CH) of the (16 + 2R)^2 window around the tile into
// dst[c][y][x], zero outside the image.  Consecutive threads read consecutive
// floats of the interleaved (H, W, C) rows.
template <int R, int CH>
__device__ __forceinline__ void load_halo(float (*dst)[SsimTile<R>::kSpan][SsimTile<R>::kSpan + 1],
                                          const float* __restrict__ src, int H, int W, int C,
                                          int c0, int x0, int y0) {
    constexpr int S = SsimTile<R>::kSpan;
    for (int i = threadIdx.x; i < S * S * CH; i += kSsThreads) {
        const int ly = i / (S * CH);
        const int rem = i - ly * (S * CH);
        const int lx = rem / CH, c = rem - lx * CH;
        const int gy = y0 - R + ly, gx = x0 - R + lx;
        float v = 0.0f;
        if (gy >= 0 && gy < H && gx >= 0 && gx < W) v = src[((int64_t)gy * W + gx) * C + c0 + c];
        dst[c][ly][lx] = v;
    }
}

template <int R, int CH>
__global__ __launch_bounds__(kSsThreads) void k_ssim_fwd(
    const float* __restrict__ pred, const float* __restrict__ tgt, int H, int W, int C, int c0,
    int tiles_x, SsimWindow win, float c1, float c2, float* __restrict__ maps,
    float* __restrict__ partials) {
    constexpr int S = SsimTile<R>::kSpan;
    constexpr int K = 2 * R + 1;
    __shared__ float s_p[CH][S][S + 1];
    __shared__ float s_t[CH][S][S + 1];
    __shared__ float s_h[5][S][kSsT + 1];
    __shared__ float s_red[2][kSsThreads / kWave];

    const int tid = threadIdx.x;
    const int tx = tid & (kSsT - 1), ty = tid / kSsT;
    int x0, y0;
    ssim_tile(tiles_x, x0, y0);
    const int x = x0 + tx, y = y0 + ty;
    const bool inside = x < W && y < H;
    const int64_t plane = (int64_t)H * W * C;
    const int64_t pix = ((int64_t)y * W + x) * C + c0;
    float l1 = 0.0f, ssum = 0.0f;

    load_halo<R, CH>(s_p, pred, H, W, C, c0, x0, y0);
    load_halo<R, CH>(s_t, tgt, H, W, C, c0, x0, y0);
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < CH; ++c) {
        for (int i = tid; i < S * kSsT; i += kSsThreads) {
            const int ly = i / kSsT, lx = i - ly * kSsT;
            float a = 0.0f, b = 0.0f, pp = 0.0f, tt = 0.0f, pt = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float w = win.g[k], p = s_p[c][ly][lx + k], t = s_t[c][ly][lx + k];
                a = fmaf(w, p, a);
                b = fmaf(w, t, b);
                pp = fmaf(w, p * p, pp);
                tt = fmaf(w, t * t, tt);
                pt = fmaf(w, p * t, pt);
            }
            s_h[0][ly][lx] = a;
            s_h[1][ly][lx] = b;
            s_h[2][ly][lx] = pp;
            s_h[3][ly][lx] = tt;
            s_h[4][ly][lx] = pt;
        }
        __syncthreads();
        float mp = 0.0f, mt = 0.0f, epp = 0.0f, ett = 0.0f, ept = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const float w = win.g[k];
            mp = fmaf(w, s_h[0][ty + k][tx], mp);
            mt = fmaf(w, s_h[1][ty + k][tx], mt);
            epp = fmaf(w, s_h[2][ty + k][tx], epp);
            ett = fmaf(w, s_h[3][ty + k][tx], ett);
            ept = fmaf(w, s_h[4][ty + k][tx], ept);
        }
        if (inside) {
            const float p = s_p[c][ty + R][tx + R], t = s_t[c][ty + R][tx + R];
            const float mpp = mp * mp, mtt = mt * mt, mpt = mp * mt;
            const float A = 2.0f * mpt + c1, B = mpp + mtt + c1;
            const float Cn = 2.0f * (ept - mpt) + c2, D = (epp - mpp) + (ett - mtt) + c2;
            const float cs = Cn / D, l = A / B;
            ssum += l * cs;
            l1 += fabsf(p - t);
            maps[pix + c] = 2.0f * (mt - l * mp) * cs / B + 2.0f * l * (mp * cs - mt) / D;
            maps[plane + pix + c] = -l * cs / D;
            maps[2 * plane + pix + c] = 2.0f * l / D;
        }
        __syncthreads();
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        l1 += __shfl_xor(l1, o, kWave);
        ssum += __shfl_xor(ssum, o, kWave);
    }
    if ((tid & (kWave - 1)) == 0) {
        s_red[0][tid / kWave] = l1;
        s_red[1][tid / kWave] = ssum;
    }
    __syncthreads();
    if (tid == 0) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int w = 0; w < kSsThreads / kWave; ++w) {
            a += s_red[0][w];
            b += s_red[1][w];
        }
        partials[2 * (int64_t)blockIdx.x] = a;
        partials[2 * (int64_t)blockIdx.x + 1] = b;
    }
}

// Sums the per-tile partials in a fixed order (double accumulators) and
// writes [mean |pred - target|, mean SSIM].
__global__ __launch_bounds__(256) void k_loss_reduce(const float* __restrict__ partials,
                                                     int64_t nblk, double inv_n,
                                                     float* __restrict__ out) {
    __shared__ double s[2][256];
    double a = 0.0, b = 0.0;
    for (int64_t i = threadIdx.x; i < nblk; i += 256) {
        a += (double)partials[2 * i];
        b += (double)partials[2 * i + 1];
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
        out[0] = (float)(s[0][0] * inv_n);
        out[1] = (float)(s[1][0] * inv_n);
    }
}

// grad_pred = g_l1 sign(p - t) / n + g_ssim (F(dmu) + 2 p F(dpp) + t F(dpt)) / n
template <int R, int CH>
__global__ __launch_bounds__(kSsThreads) void k_ssim_bwd(
    const float* __restrict__ pred, const float* __restrict__ tgt, int H, int W, int C, int c0,
    int tiles_x, SsimWindow win, const float* __restrict__ maps, const float* __restrict__ grad_in,
    float inv_n, float* __restrict__ grad) {
    constexpr int S = SsimTile<R>::kSpan;
    constexpr int K = 2 * R + 1;
    __shared__ float s_m[3][CH][S][S + 1];
    __shared__ float s_h[3][S][kSsT + 1];

    const int tid = threadIdx.x;
    const int tx = tid & (kSsT - 1), ty = tid / kSsT;
    int x0, y0;
    ssim_tile(tiles_x, x0, y0);
    const int x = x0 + tx, y = y0 + ty;
    const bool inside = x < W && y < H;
    const int64_t plane = (int64_t)H * W * C;
    const int64_t pix = ((int64_t)y * W + x) * C + c0;
    const float gl = grad_in[0] * inv_n, gs = grad_in[1] * inv_n;

#pragma unroll
    for (int q = 0; q < 3; ++q) load_halo<R, CH>(s_m[q], maps + q * plane, H, W, C, c0, x0, y0);
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < CH; ++c) {
        for (int i = tid; i < S * kSsT; i += kSsThreads) {
            const int ly = i / kSsT, lx = i - ly * kSsT;
            float a = 0.0f, b = 0.0f, d = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float w = win.g[k];
                a = fmaf(w, s_m[0][c][ly][lx + k], a);
                b = fmaf(w, s_m[1][c][ly][lx + k], b);
                d = fmaf(w, s_m[2][c][ly][lx + k], d);
            }
            s_h[0][ly][lx] = a;
            s_h[1][ly][lx] = b;
            s_h[2][ly][lx] = d;
        }
        __syncthreads();
        float fm = 0.0f, fpp = 0.0f, fpt = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const float w = win.g[k];
            fm = fmaf(w, s_h[0][ty + k][tx], fm);
            fpp = fmaf(w, s_h[1][ty + k][tx], fpp);
            fpt = fmaf(w, s_h[2][ty + k][tx], fpt);
        }
        if (inside) {
            const float p = pred[pix + c], t = tgt[pix + c];
            const float sgn = (float)((p > t) - (p < t));
            const float gss = fm + 2.0f * p * fpp + t * fpt;
            grad[pix + c] = fmaf(gs, gss, gl * sgn);
        }
        __syncthreads();
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
    m = b1 * m + omb1 * g;
    v = b2 * v + omb2 * (g * g);
    p = p - (lr * m) / (sqrtf(v) + eps);
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
__global__ __launch_bounds__(256) void k_accum_screen_grads(int64_t n,
                                                            const float2* __restrict__ g,
                                                            const float* __restrict__ radii,
                                                            float half_w, float half_h,
                                                            float* __restrict__ accum,
                                                            float* __restrict__ count) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float2 d = g[i];
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

int64_t photometric_blocks(int32_t H, int32_t W) {
    return (int64_t)((W + kSsT - 1) / kSsT) * ((H + kSsT - 1) / kSsT);
}

int64_t photometric_groups(int32_t C) { return (C + kSsMaxCh - 1) / kSsMaxCh; }

// ------------------------------------------------------------------ L1 --
// mean |pred - target| (image_metrics.py:13-14): each workgroup sums 4096
// elements (float4 loads) in double into its partial (k_loss_reduce adds
// the partials in a fixed order), and the gradient sign(pred - target) g/n
// in one elementwise pass.
constexpr int kL1Threads = 256, kL1Per = 16, kL1Block = kL1Threads * kL1Per;

template <bool VEC>
__global__ __launch_bounds__(kL1Threads) void k_l1_partial(int64_t n,
                                                           const float* __restrict__ p,
                                                           const float* __restrict__ t,
                                                           float* __restrict__ partials) {
    __shared__ double s[kL1Threads];
    const int64_t base = (int64_t)blockIdx.x * kL1Block;
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < kL1Per / 4; ++k) {
        const int64_t i = base + 4 * ((int64_t)k * kL1Threads + threadIdx.x);
        if (VEC && i + 3 < n) {
            const float4 a = *reinterpret_cast<const float4*>(p + i);
            const float4 b = *reinterpret_cast<const float4*>(t + i);
            acc += (double)fabsf(a.x - b.x) + (double)fabsf(a.y - b.y) +
                   (double)fabsf(a.z - b.z) + (double)fabsf(a.w - b.w);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (i + e < n) acc += (double)fabsf(p[i + e] - t[i + e]);
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
int l1_fwd_into(int64_t n, const float* pred, const float* target, float* partials, float* out,
                hipStream_t st) {
    const int64_t nblk = (n + kL1Block - 1) / kL1Block;
    const bool vec = (((uintptr_t)pred | (uintptr_t)target) & 15u) == 0;
    if (vec)
        hipLaunchKernelGGL(k_l1_partial<true>, dim3((unsigned)nblk), dim3(kL1Threads), 0, st, n,
                           pred, target, partials);
    else
        hipLaunchKernelGGL(k_l1_partial<false>, dim3((unsigned)nblk), dim3(kL1Threads), 0, st, n,
                           pred, target, partials);
    GSX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_loss_reduce, dim3(1), dim3(256), 0, st, (const float*)partials, nblk,
                       1.0 / (double)n, out);
    GSX_LAUNCH_CHECK();
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
    const int tiles_x = (width + kSsT - 1) / kSsT;
    const int64_t nblk = photometric_blocks(height, width);
    hipStream_t st = (hipStream_t)stream;
    for (int c0 = 0; c0 < channels; c0 += kSsMaxCh) {
        const int nc = std::min(kSsMaxCh, channels - c0);
        float* part = partials + 2 * (c0 / kSsMaxCh) * nblk;
        const int key = (window_size / 2) * 8 + nc;
        switch (key) {
#define GSX_SSIM_FWD(RR, CC)                                                                   \
    case RR * 8 + CC:                                                                          \
        hipLaunchKernelGGL((k_ssim_fwd<RR, CC>), dim3((unsigned)nblk), dim3(kSsThreads), 0, st, \
                           pred, target, height, width, channels, c0, tiles_x, win, c1, c2,     \
                           maps, part);                                                        \
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
    hipLaunchKernelGGL(k_loss_reduce, dim3(1), dim3(256), 0, st, partials,
                       photometric_groups(channels) * nblk, inv_n, out);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_photometric_bwd(int32_t height, int32_t width, int32_t channels, const float* pred,
                        const float* target, int32_t window_size, float sigma,
                        const void* workspace, int64_t workspace_bytes, const float* grad_out,
                        float* grad_pred, void* stream) {
    if (height <= 0 || width <= 0 || channels <= 0) return GSX_ERR_INVALID;
    if (!pred || !target || !workspace || !grad_out || !grad_pred) return GSX_ERR_INVALID;
    if ((int64_t)height * width * channels >= (int64_t(1) << 40)) return GSX_ERR_TOO_LARGE;
    SsimWindow win;
    if (!make_window(window_size, sigma, win)) return GSX_ERR_INVALID;
    if (workspace_bytes < gsx_photometric_workspace_bytes(height, width, channels))
        return GSX_ERR_WORKSPACE;
    const float inv_n = (float)(1.0 / ((double)height * width * channels));
    const int tiles_x = (width + kSsT - 1) / kSsT;
    const int64_t nblk = photometric_blocks(height, width);
    hipStream_t st = (hipStream_t)stream;
    const float* maps = (const float*)workspace;
    for (int c0 = 0; c0 < channels; c0 += kSsMaxCh) {
        const int nc = std::min(kSsMaxCh, channels - c0);
        const int key = (window_size / 2) * 8 + nc;
        switch (key) {
#define GSX_SSIM_BWD(RR, CC)                                                                   \
    case RR * 8 + CC:                                                                          \
        hipLaunchKernelGGL((k_ssim_bwd<RR, CC>), dim3((unsigned)nblk), dim3(kSsThreads), 0, st, \
                           pred, target, height, width, channels, c0, tiles_x, win, maps,       \
                           grad_out, inv_n, grad_pred);                                        \
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
    return l1_fwd_into(n, pred, target, (float*)workspace, out, (hipStream_t)stream);
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
    return l1_fwd_into(n, pred, target, partials, out, st);
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
                           int32_t height, float* grad_accum, float* grad_count, void* stream) {
    if (n < 0 || width <= 0 || height <= 0) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!g_means2d || !radii || !grad_accum || !grad_count) return GSX_ERR_INVALID;
    if (((uintptr_t)g_means2d & 7u) != 0) return GSX_ERR_INVALID;
    const unsigned blocks = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL(k_accum_screen_grads, dim3(blocks), dim3(256), 0, (hipStream_t)stream, n,
                       (const float2*)g_means2d, radii, (float)(width / 2.0),
                       (float)(height / 2.0), grad_accum, grad_count);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // extern "C"
