// raster.hip -- tile compositing (replaces gs_rasterize_forward,
// gs_rasterize_backward and gs_rasterize_depth, splatting/rasterize.py:28-290).
//
// One 256-lane workgroup (4 wave64) per 16x16 tile; wave w owns the 8x8
// pixel quadrant (w&1, w>>1).  The tile's depth-sorted Gaussians are staged
// through LDS in batches (two 16-byte records per Gaussian plus its
// channels, read as broadcasts).  While staging, each lane tests its
// Gaussian's alpha >= 1/255 ellipse (bounding box, float64, with a margin
// that covers the float32 rounding of the per-pixel power) against the four
// quadrants, and the workgroup publishes per quadrant a bit mask of the
// Gaussians that can touch it.  Each wave walks only its own set bits, in
// list order, prefetching the next record while it evaluates the current
// one.  Skipped pairs are exactly pairs whose alpha is below 1/255, which
// the reference also skips, so every output is unchanged.
//
// Forward: per-pixel front-to-back compositing as rasterize.py:60-96 (same
// skips, same termination before compositing the splat that would drop T
// below 1e-4), branch-free per pair; a wave stops once its 64 pixels have
// terminated and the workgroup stops loading once all 256 have.
// Backward: back-to-front replay (rasterize.py:147-220) from the largest
// n_contrib of each quadrant.  A pair's gradient terms are summed over the
// wave with DPP row operations; lane 63 stores the sums in the wave's own
// LDS slot for that Gaussian (no LDS atomics), and after the batch one lane
// per Gaussian adds the four waves' slots and issues one global atomic per
// (Gaussian, tile, component) -- the reference issues one per (pixel,
// Gaussian, component).
#include "gsx_device.h"

using namespace gsx;

namespace {

constexpr int kThreads = kTilePixels;
constexpr int kWaves = kThreads / kWave;  // 4 quadrant waves

// exp with the range handling of dexp done by selects instead of branches;
// identical results to dexp for every input.
__device__ __forceinline__ float dexp_sel(float x) {
    const float xc = fminf(fmaxf(x, -86.0f), 88.0f);
    const float k = rintf(xc * 1.44269504088896341f);
    float r = fmaf(k, -0.693145751953125f, xc);
    r = fmaf(k, -1.42860682030941723e-06f, r);
    float p = 1.98412698412698413e-04f;
    p = fmaf(p, r, 1.38888888888888889e-03f);
    p = fmaf(p, r, 8.33333333333333333e-03f);
    p = fmaf(p, r, 4.16666666666666667e-02f);
    p = fmaf(p, r, 1.66666666666666667e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    float e = ldexpf(p, (int)k);
    e = (x < -86.0f) ? 0.0f : e;
    e = (x > 88.0f) ? __builtin_huge_valf() : e;
    return (x != x) ? x : e;
}

// Power below which o * exp(power) < 1/255 for certain.  +inf when the
// opacity can never reach 1/255 (o <= 0 or tiny), -inf when no bound is safe
// (o NaN or +inf).
__device__ __forceinline__ float alpha_floor_power(float o) {
    if (o > 0.0f) {
        float L = -__logf(255.0f * o);  // ln(1 / (255 o))
        L = fminf(L, 200.0f);
        return L - (1e-3f + 1e-4f * fabsf(L));
    }
    if (o <= 0.0f) return __builtin_huge_valf();
    return -__builtin_huge_valf();
}

// Which of the tile's four 8x8 quadrants (bit q = quadrant (q&1, q>>1)) the
// pixels with alpha >= 1/255 of this Gaussian can lie in.  alpha >= 1/255
// needs q(d) = a dx^2 + 2 b dx dy + c dy^2 <= 2 ln(255 o); the bounding box
// of that ellipse has half-widths sqrt(2 tau c / det), sqrt(2 tau a / det).
// With b^2 < 0.999 a c the float32 evaluation of the power is within 7.2e-4
// relative of the exact value, so tau is inflated by 1% (+1e-3) and the box
// by 0.05 px.  Ill-conditioned, non-positive or non-finite conics get no
// culling (all four bits).
__device__ __forceinline__ uint32_t quadrant_mask(float x, float y, float4 c, int px0, int py0) {
    const float o = c.w;
    if (!(o >= 0.0039215f)) return (o == o) ? 0u : 0xFu;  // alpha < 1/255 everywhere
    const double A = c.x, B = c.y, C = c.z;
    const double det = A * C - B * B;
    if (!(A > 0.0 && C > 0.0 && det > 1e-3 * A * C)) return 0xFu;
    const double tau = log(255.0 * (double)o) * 1.01 + 1e-3;
    const double ex = sqrt(2.0 * tau * C / det) + 0.05;
    const double ey = sqrt(2.0 * tau * A / det) + 0.05;
    const double xd = x, yd = y;
    if (!(ex < 1e30 && ey < 1e30 && xd == xd && yd == yd)) return 0xFu;
    uint32_t m = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const double qx0 = px0 + (q & 1) * 8 + 0.5, qy0 = py0 + (q >> 1) * 8 + 0.5;
        const bool hit = (xd + ex >= qx0) && (xd - ex <= qx0 + 7.0) && (yd + ey >= qy0) &&
                         (yd - ey <= qy0 + 7.0);
        m |= hit ? (1u << q) : 0u;
    }
    return m;
}

template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK,
                                                       BANK_MASK, false));
}

// Sum over the 64 lanes of the wave; the total ends up in lane 63.
// quad_perm xor1, xor2, half-row mirror, row mirror, then the gfx9
// row_bcast15 / row_bcast31 steps fold the four rows.  All lanes must be
// active.
__device__ __forceinline__ float wave_total_lane63(float v) {
    v += dpp_f<0xB1, 0xF, 0xF>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E, 0xF, 0xF>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141, 0xF, 0xF>(v);  // row_half_mirror
    v += dpp_f<0x140, 0xF, 0xF>(v);  // row_mirror
    v += dpp_f<0x142, 0xA, 0xF>(v);  // row_bcast15 -> rows 1, 3
    v += dpp_f<0x143, 0xC, 0xF>(v);  // row_bcast31 -> rows 2, 3
    return v;
}

__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Clamp a tile's [start, end) to the id array so a malformed range can
// never read outside it.
__device__ __forceinline__ void tile_span(int2 rg, int64_t n_ids, int& start, int& num) {
    const int64_t s0 = rg.x < 0 ? 0 : (rg.x > n_ids ? n_ids : rg.x);
    const int64_t s1 = rg.y < s0 ? s0 : (rg.y > n_ids ? n_ids : rg.y);
    start = (int)s0;
    num = (int)(s1 - s0);
}

// Walk over the set bits of a quadrant's staged-Gaussian mask (NW 64-bit
// words in LDS), ascending or descending.  Only the current word is held
// (in scalar registers); the next word is read from LDS when it runs out.
struct BitWalkUp {
    const uint64_t* words;  // LDS
    int nw, w;
    uint64_t cur;
    __device__ __forceinline__ void init(const uint64_t* p, int n) {
        words = p;
        nw = n;
        w = 0;
        cur = uniform64(p[0]);
    }
    __device__ __forceinline__ int next() {
        while (cur == 0ull) {
            if (++w >= nw) return -1;
            cur = uniform64(words[w]);
        }
        const int b = __builtin_ctzll(cur);
        cur &= cur - 1ull;
        return w * kWave + b;
    }
};

struct BitWalkDown {
    const uint64_t* words;  // LDS
    int w;
    uint64_t cur;
    __device__ __forceinline__ void init(const uint64_t* p, int n) {
        words = p;
        w = n - 1;
        cur = uniform64(p[w]);
    }
    __device__ __forceinline__ int next() {
        while (cur == 0ull) {
            if (--w < 0) return -1;
            cur = uniform64(words[w]);
        }
        const int b = 63 - __builtin_clzll(cur);
        cur &= ~(1ull << b);
        return w * kWave + b;
    }
};

template <int CH>
__device__ __forceinline__ void stage_features(float4* dst, const float* f, int nc) {
    constexpr int F4 = (CH + 3) / 4;
#pragma unroll
    for (int k = 0; k < F4; ++k) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int ch = 4 * k + e;
            v[e] = (ch < CH && ch < nc) ? f[ch] : 0.0f;
        }
        dst[k] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

__device__ __forceinline__ float comp4(const float4& v, int e) {
    return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

template <int CH, bool DEPTH>
__global__ __launch_bounds__(kThreads) void k_raster_fwd(
    const float2* __restrict__ xy, const float4* __restrict__ co, const float* __restrict__ feat,
    int C, int c0, int nc, const float* __restrict__ depths, const int* __restrict__ ids,
    const int2* __restrict__ ranges, int64_t n, int64_t n_ids, const float* __restrict__ bg,
    int W, int H, int tiles_x, float* __restrict__ out, float* __restrict__ final_T,
    int* __restrict__ n_contrib, float* __restrict__ depth_out) {
    constexpr int F4 = (CH + 3) / 4;
    __shared__ float4 s_r0[kThreads];      // mean x, mean y, log-alpha bound, opacity
    __shared__ float4 s_r1[kThreads];      // conic a, b, c, depth
    __shared__ float4 s_f[kThreads][F4];   // channels, zero padded
    __shared__ uint64_t s_mask[kWaves][kWaves];  // [quadrant][loader wave]

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = (int)xcd_remap(blockIdx.x, gridDim.x);
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px0 = tx * kTile, py0 = ty * kTile;
    const int px = px0 + (wave & 1) * 8 + (lane & 7);
    const int py = py0 + (wave >> 1) * 8 + (lane >> 3);
    const bool inside = px < W && py < H;
    const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;

    int start, num;
    tile_span(ranges[tile], n_ids, start, num);

    float T = 1.0f, dacc = 0.0f;
    float acc[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) acc[k] = 0.0f;
    int last = 0;
    bool done = !inside;

    for (int base = 0; base < num; base += kThreads) {
        if (__syncthreads_count(done) == kThreads) break;
        const int k = base + tid;
        uint32_t qm = 0;
        if (k < num) {
            const int g = ids[start + k];
            if ((uint32_t)g < (uint64_t)n) {
                const float2 m = xy[g];
                const float4 c = co[g];
                s_r0[tid] = make_float4(m.x, m.y, alpha_floor_power(c.w), c.w);
                s_r1[tid] = make_float4(c.x, c.y, c.z, DEPTH ? depths[g] : 0.0f);
                stage_features<CH>(s_f[tid], feat + (int64_t)g * C + c0, nc);
                qm = quadrant_mask(m.x, m.y, c, px0, py0);
            }
        }
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
            const uint64_t b = __ballot((qm >> q) & 1u);
            if (lane == 0) s_mask[q][wave] = b;
        }
        __syncthreads();
        if (__ballot(!done) == 0ull) continue;
        BitWalkUp walk;
        walk.init(s_mask[wave], kWaves);
        int j = walk.next();
        if (j < 0) continue;
        float4 r0 = s_r0[j], r1 = s_r1[j];
        while (true) {
            const int jn = walk.next();
            float4 r0n = r0, r1n = r1;
            if (jn >= 0) {
                r0n = s_r0[jn];
                r1n = s_r1[jn];
            }
            const float dx = r0.x - pxf, dy = r0.y - pyf;
            const float power = -0.5f * (r1.x * dx * dx + r1.z * dy * dy) - r1.y * dx * dy;
            const bool live = !done && !(power > 0.0f) && !(power < r0.z);
            if (__ballot(live) != 0ull) {
                float4 fv[F4];
#pragma unroll
                for (int q = 0; q < F4; ++q) fv[q] = s_f[j][q];
                const float alpha = fminf(0.99f, r0.w * dexp_sel(power));
                const bool pass = live && !(alpha < 1.0f / 255.0f);
                const float next_T = T * (1.0f - alpha);
                const bool stop = pass && next_T < 1e-4f;
                const bool add = pass && !stop;
                const float w = alpha * T;
#pragma unroll
                for (int ch = 0; ch < CH; ++ch) {
                    const float a2 = acc[ch] + comp4(fv[ch >> 2], ch & 3) * w;
                    acc[ch] = add ? a2 : acc[ch];
                }
                if (DEPTH) {
                    const float d2 = dacc + r1.w * w;
                    dacc = add ? d2 : dacc;
                }
                T = add ? next_T : T;
                last = add ? base + j + 1 : last;
                done = done || stop;
                if (__ballot(!done) == 0ull) break;
            }
            if (jn < 0) break;
            j = jn;
            r0 = r0n;
            r1 = r1n;
        }
    }
    if (inside) {
        const int64_t pid = (int64_t)py * W + px;
        float* o = out + pid * C + c0;
#pragma unroll
        for (int ch = 0; ch < CH; ++ch)
            if (ch < nc) o[ch] = acc[ch] + T * (bg ? bg[c0 + ch] : 0.0f);
        if (c0 == 0) {
            final_T[pid] = T;
            n_contrib[pid] = last;
            if (DEPTH) {
                const float al = 1.0f - T;
                depth_out[pid] = al > 1e-6f ? dacc / al : 0.0f;
            }
        }
    }
}

template <int CH>
__global__ __launch_bounds__(kThreads) void k_raster_bwd(
    const float2* __restrict__ xy, const float4* __restrict__ co, const float* __restrict__ feat,
    int C, int c0, int nc, const int* __restrict__ ids, const int2* __restrict__ ranges,
    int64_t n, int64_t n_ids, const float* __restrict__ bg, int W, int H, int tiles_x,
    const float* __restrict__ final_T, const int* __restrict__ n_contrib,
    const float* __restrict__ grad_out, const float* __restrict__ grad_T,
    float* __restrict__ g_xy, float* __restrict__ g_conic, float* __restrict__ g_feat,
    float* __restrict__ g_opac) {
    constexpr int F4 = (CH + 3) / 4;
    constexpr int NV = CH + 6;             // dx, dy, conic a, b, c, opacity, channels
    constexpr int NV4 = (NV + 3) / 4;
    constexpr int BB = (CH <= 4) ? 128 : 64;  // Gaussians per batch (bounded by slot LDS)
    constexpr int NLW = BB / kWave;
    static_assert(NLW == 1 || NLW == 2, "the written-mask words are held as two scalars");
    __shared__ float4 s_r0[BB];
    __shared__ float4 s_r1[BB];
    __shared__ float4 s_f[BB][F4];
    __shared__ int s_id[BB];
    __shared__ float4 s_part[kWaves][BB][NV4];  // per-wave gradient sums per Gaussian
    __shared__ uint64_t s_mask[kWaves][NLW];
    __shared__ uint64_t s_wrote[kWaves][NLW];
    __shared__ int s_last[kWaves];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = (int)xcd_remap(blockIdx.x, gridDim.x);
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px0 = tx * kTile, py0 = ty * kTile;
    const int px = px0 + (wave & 1) * 8 + (lane & 7);
    const int py = py0 + (wave >> 1) * 8 + (lane >> 3);
    const bool inside = px < W && py < H;
    const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
    const int64_t pid = (int64_t)py * W + px;

    int start, num;
    tile_span(ranges[tile], n_ids, start, num);

    const float T_final = inside ? final_T[pid] : 1.0f;
    float T = T_final;
    const int last = inside ? n_contrib[pid] : 0;
    float gpix[CH];
    float bg_dot = 0.0f;
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) {
        gpix[ch] = (inside && ch < nc) ? grad_out[pid * C + c0 + ch] : 0.0f;
        if (ch < nc) bg_dot = bg_dot + (bg ? bg[c0 + ch] : 0.0f) * gpix[ch];
    }
    // The alpha output's cotangent enters once, with the first channel block.
    if (inside && c0 == 0 && grad_T) bg_dot = bg_dot + grad_T[pid];

    // Largest n_contrib of each quadrant: later list entries changed no pixel.
    {
        int m = last;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, kWave));
        if (lane == 0) s_last[wave] = m;
    }
    __syncthreads();
    int quad_last[kWaves];
#pragma unroll
    for (int q = 0; q < kWaves; ++q) quad_last[q] = s_last[q];
    const int max_last = max(max(quad_last[0], quad_last[1]), max(quad_last[2], quad_last[3]));
    const int n_batches = (max_last + BB - 1) / BB;

    float accum[CH], lastc[CH];
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) accum[ch] = lastc[ch] = 0.0f;
    float last_alpha = 0.0f;

    for (int b = n_batches - 1; b >= 0; --b) {
        __syncthreads();
        uint32_t qm = 0;
        if (tid < BB) {
            const int k = b * BB + tid;
            int gid = -1;
            if (k < num) {
                const int g = ids[start + k];
                if ((uint32_t)g < (uint64_t)n) {
                    gid = g;
                    const float2 m = xy[g];
                    const float4 c = co[g];
                    s_r0[tid] = make_float4(m.x, m.y, alpha_floor_power(c.w), c.w);
                    s_r1[tid] = make_float4(c.x, c.y, c.z, 0.0f);
                    stage_features<CH>(s_f[tid], feat + (int64_t)g * C + c0, nc);
                    qm = quadrant_mask(m.x, m.y, c, px0, py0);
#pragma unroll
                    for (int q = 0; q < kWaves; ++q)
                        if (k >= quad_last[q]) qm &= ~(1u << q);
                }
            }
            s_id[tid] = gid;
        }
        if (wave < NLW) {
#pragma unroll
            for (int q = 0; q < kWaves; ++q) {
                const uint64_t bq = __ballot((qm >> q) & 1u);
                if (lane == 0) s_mask[q][wave] = bq;
            }
        }
        __syncthreads();
        BitWalkDown walk;
        walk.init(s_mask[wave], NLW);
        uint64_t wrote0 = 0ull, wrote1 = 0ull;  // NLW <= 2
        int j = walk.next();
        float4 r0 = make_float4(0, 0, 0, 0), r1 = r0;
        if (j >= 0) {
            r0 = s_r0[j];
            r1 = s_r1[j];
        }
        while (j >= 0) {
            const int jn = walk.next();
            float4 r0n = r0, r1n = r1;
            if (jn >= 0) {
                r0n = s_r0[jn];
                r1n = s_r1[jn];
            }
            const int gj = b * BB + j;
            const float dx = r0.x - pxf, dy = r0.y - pyf;
            const float power = -0.5f * (r1.x * dx * dx + r1.z * dy * dy) - r1.y * dx * dy;
            bool ok = gj < last && !(power > 0.0f) && !(power < r0.z);
            if (__ballot(ok) != 0ull) {
                const float G = dexp_sel(power);
                const float alpha = fminf(0.99f, r0.w * G);
                ok = ok && !(alpha < 1.0f / 255.0f);
                if (__ballot(ok) != 0ull) {
                    float4 fv[F4];
#pragma unroll
                    for (int q = 0; q < F4; ++q) fv[q] = s_f[j][q];
                    const float Tn = T / (1.0f - alpha);
                    T = ok ? Tn : T;
                    const float aT = alpha * T;
                    float dl = 0.0f;
#pragma unroll
                    for (int ch = 0; ch < CH; ++ch) {
                        const float f = comp4(fv[ch >> 2], ch & 3);
                        const float an = last_alpha * lastc[ch] + (1.0f - last_alpha) * accum[ch];
                        accum[ch] = ok ? an : accum[ch];
                        lastc[ch] = ok ? f : lastc[ch];
                        dl = dl + (f - accum[ch]) * gpix[ch];
                    }
                    last_alpha = ok ? alpha : last_alpha;
                    float dL_dalpha = dl * T;
                    dL_dalpha += (-T_final / (1.0f - alpha)) * bg_dot;
                    const float dL_dG = r0.w * dL_dalpha;
                    const float gdx = G * dx, gdy = G * dy;
                    float v[4 * NV4];
                    v[0] = -(gdx * r1.x + gdy * r1.y) * dL_dG;
                    v[1] = -(gdy * r1.z + gdx * r1.y) * dL_dG;
                    v[2] = -0.5f * gdx * dx * dL_dG;
                    v[3] = -gdx * dy * dL_dG;
                    v[4] = -0.5f * gdy * dy * dL_dG;
                    v[5] = G * dL_dalpha;
#pragma unroll
                    for (int ch = 0; ch < CH; ++ch) v[6 + ch] = aT * gpix[ch];
#pragma unroll
                    for (int q = 0; q < NV; ++q) v[q] = wave_total_lane63(ok ? v[q] : 0.0f);
#pragma unroll
                    for (int q = NV; q < 4 * NV4; ++q) v[q] = 0.0f;
                    if (lane == 63) {
#pragma unroll
                        for (int q = 0; q < NV4; ++q)
                            s_part[wave][j][q] =
                                make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
                    }
                    if (j < kWave) wrote0 |= 1ull << j;
                    else wrote1 |= 1ull << (j - kWave);
                }
            }
            j = jn;
            r0 = r0n;
            r1 = r1n;
        }
        if (lane == 0) {
            s_wrote[wave][0] = wrote0;
            if (NLW > 1) s_wrote[wave][NLW - 1] = wrote1;
        }
        __syncthreads();
        if (tid < BB) {
            const int g = s_id[tid];
            float4 sum[NV4];
#pragma unroll
            for (int q = 0; q < NV4; ++q) sum[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            bool any = false;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                if ((s_wrote[w][tid >> 6] >> (tid & 63)) & 1ull) {
                    any = true;
#pragma unroll
                    for (int q = 0; q < NV4; ++q) {
                        const float4 p = s_part[w][tid][q];
                        sum[q].x += p.x;
                        sum[q].y += p.y;
                        sum[q].z += p.z;
                        sum[q].w += p.w;
                    }
                }
            }
            if (any && g >= 0) {
                float e[4 * NV4];
#pragma unroll
                for (int q = 0; q < NV4; ++q) {
                    e[4 * q] = sum[q].x;
                    e[4 * q + 1] = sum[q].y;
                    e[4 * q + 2] = sum[q].z;
                    e[4 * q + 3] = sum[q].w;
                }
                if (e[0] != 0.0f) atomicAdd(&g_xy[2 * g], e[0]);
                if (e[1] != 0.0f) atomicAdd(&g_xy[2 * g + 1], e[1]);
                if (e[2] != 0.0f) atomicAdd(&g_conic[3 * g], e[2]);
                if (e[3] != 0.0f) atomicAdd(&g_conic[3 * g + 1], e[3]);
                if (e[4] != 0.0f) atomicAdd(&g_conic[3 * g + 2], e[4]);
                if (e[5] != 0.0f) atomicAdd(&g_opac[g], e[5]);
#pragma unroll
                for (int ch = 0; ch < CH; ++ch)
                    if (ch < nc && e[6 + ch] != 0.0f)
                        atomicAdd(&g_feat[(int64_t)g * C + c0 + ch], e[6 + ch]);
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_zero_f32(float* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

int pick_ch(int nc) {
    if (nc <= 1) return 1;
    if (nc <= 2) return 2;
    if (nc <= 3) return 3;
    if (nc <= 4) return 4;
    if (nc <= 8) return 8;
    if (nc <= 16) return 16;
    return 32;
}
constexpr int kMaxChunk = 32;

template <int CH>
void launch_fwd(dim3 grid, hipStream_t st, bool depth, const float2* xy, const float4* co,
                const float* feat, int C, int c0, int nc, const float* depths, const int* ids,
                const int2* ranges, int64_t n, int64_t n_ids, const float* bg, int W, int H,
                int tiles_x, float* out, float* fT, int* ncon, float* dout) {
    if (depth)
        hipLaunchKernelGGL((k_raster_fwd<CH, true>), grid, dim3(kThreads), 0, st, xy, co, feat, C,
                           c0, nc, depths, ids, ranges, n, n_ids, bg, W, H, tiles_x, out, fT,
                           ncon, dout);
    else
        hipLaunchKernelGGL((k_raster_fwd<CH, false>), grid, dim3(kThreads), 0, st, xy, co, feat, C,
                           c0, nc, depths, ids, ranges, n, n_ids, bg, W, H, tiles_x, out, fT,
                           ncon, dout);
}

template <int CH>
void launch_bwd(dim3 grid, hipStream_t st, const float2* xy, const float4* co, const float* feat,
                int C, int c0, int nc, const int* ids, const int2* ranges, int64_t n,
                int64_t n_ids, const float* bg, int W, int H, int tiles_x, const float* fT,
                const int* ncon, const float* gout, const float* gT, float* gxy, float* gcon,
                float* gfeat, float* gop) {
    hipLaunchKernelGGL((k_raster_bwd<CH>), grid, dim3(kThreads), 0, st, xy, co, feat, C, c0, nc,
                       ids, ranges, n, n_ids, bg, W, H, tiles_x, fT, ncon, gout, gT, gxy, gcon,
                       gfeat, gop);
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline bool aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }

}  // namespace

extern "C" {

int gsx_raster_fwd(int64_t n, int32_t C, const float* means2d, const float* conic_opacity,
                   const float* features, const float* depths, const int32_t* sorted_ids,
                   int64_t num_ids, const int32_t* tile_ranges, const float* background,
                   int32_t width,
                   int32_t height, float* out, float* final_T, int32_t* n_contrib,
                   float* depth_out, void* stream) {
    if (n < 0 || num_ids < 0 || C <= 0 || width <= 0 || height <= 0) return GSX_ERR_INVALID;
    if (!tile_ranges || !out || !final_T || !n_contrib) return GSX_ERR_INVALID;
    if (n > 0 && (!means2d || !conic_opacity || !features)) return GSX_ERR_INVALID;
    if (num_ids > 0 && !sorted_ids) return GSX_ERR_INVALID;
    if (n == 0) num_ids = 0;
    if (depths && !depth_out) return GSX_ERR_INVALID;
    if (!aligned8(means2d) || !aligned16(conic_opacity) || !aligned8(tile_ranges))
        return GSX_ERR_INVALID;
    hipStream_t st = (hipStream_t)stream;
    const int tiles_x = (width + kTile - 1) / kTile;
    const int tiles_y = (height + kTile - 1) / kTile;
    const dim3 grid((unsigned)(tiles_x * tiles_y));
    for (int c0 = 0; c0 < C; c0 += kMaxChunk) {
        const int nc = (C - c0 < kMaxChunk) ? C - c0 : kMaxChunk;
        const bool depth = depths && c0 == 0;
        switch (pick_ch(nc)) {
#define GSX_FWD_CASE(V)                                                                          \
    case V:                                                                                      \
        launch_fwd<V>(grid, st, depth, (const float2*)means2d, (const float4*)conic_opacity,     \
                      features, C, c0, nc, depths, sorted_ids, (const int2*)tile_ranges, n,      \
                      num_ids, background, width, height, tiles_x, out, final_T, n_contrib,      \
                      depth_out);                                                                \
        break;
            GSX_FWD_CASE(1)
            GSX_FWD_CASE(2)
            GSX_FWD_CASE(3)
            GSX_FWD_CASE(4)
            GSX_FWD_CASE(8)
            GSX_FWD_CASE(16)
            GSX_FWD_CASE(32)
#undef GSX_FWD_CASE
            default:
                return GSX_ERR_INVALID;
        }
        GSX_LAUNCH_CHECK();
    }
    return GSX_OK;
}

int gsx_raster_bwd(int64_t n, int32_t C, const float* means2d, const float* conic_opacity,
                   const float* features, const int32_t* sorted_ids, int64_t num_ids,
                   const int32_t* tile_ranges,
                   const float* background, int32_t width, int32_t height, const float* final_T,
                   const int32_t* n_contrib, const float* grad_out, const float* grad_final_T,
                   float* g_means2d, float* g_conics, float* g_features, float* g_opacities,
                   void* stream) {
    if (n < 0 || num_ids < 0 || C <= 0 || width <= 0 || height <= 0) return GSX_ERR_INVALID;
    if (!tile_ranges || !final_T || !n_contrib || !grad_out) return GSX_ERR_INVALID;
    if (n > 0 && (!means2d || !conic_opacity || !features || !g_means2d || !g_conics ||
                  !g_features || !g_opacities))
        return GSX_ERR_INVALID;
    if (num_ids > 0 && !sorted_ids) return GSX_ERR_INVALID;
    if (!aligned8(means2d) || !aligned16(conic_opacity) || !aligned8(tile_ranges))
        return GSX_ERR_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (n == 0) return GSX_OK;
    auto zero = [&](float* p, int64_t cnt) {
        hipLaunchKernelGGL(k_zero_f32, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, st, p,
                           cnt);
    };
    zero(g_means2d, 2 * n);
    zero(g_conics, 3 * n);
    zero(g_features, (int64_t)C * n);
    zero(g_opacities, n);
    GSX_LAUNCH_CHECK();
    const int tiles_x = (width + kTile - 1) / kTile;
    const int tiles_y = (height + kTile - 1) / kTile;
    const dim3 grid((unsigned)(tiles_x * tiles_y));
    for (int c0 = 0; c0 < C; c0 += kMaxChunk) {
        const int nc = (C - c0 < kMaxChunk) ? C - c0 : kMaxChunk;
        switch (pick_ch(nc)) {
#define GSX_BWD_CASE(V)                                                                          \
    case V:                                                                                      \
        launch_bwd<V>(grid, st, (const float2*)means2d, (const float4*)conic_opacity, features,  \
                      C, c0, nc, sorted_ids, (const int2*)tile_ranges, n, num_ids, background,   \
                      width, height, tiles_x, final_T, n_contrib, grad_out, grad_final_T,        \
                      g_means2d, g_conics, g_features, g_opacities);                             \
        break;
            GSX_BWD_CASE(1)
            GSX_BWD_CASE(2)
            GSX_BWD_CASE(3)
            GSX_BWD_CASE(4)
            GSX_BWD_CASE(8)
            GSX_BWD_CASE(16)
            GSX_BWD_CASE(32)
#undef GSX_BWD_CASE
            default:
                return GSX_ERR_INVALID;
        }
        GSX_LAUNCH_CHECK();
    }
    return GSX_OK;
}

}  // extern "C"
