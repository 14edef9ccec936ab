// raster.hip -- tile compositing (replaces gs_rasterize_forward,
// gs_rasterize_backward and gs_rasterize_depth, splatting/rasterize.py:28-290).
//
// One 256-lane workgroup (4 wave64) per 16x16 tile; wave w owns the 8x8
// quadrant (w&1, w>>1).  Gaussians of the tile's depth-sorted list are
// staged through LDS 256 at a time (structure-of-arrays, broadcast reads).
//
// Forward: per-pixel front-to-back compositing exactly as rasterize.py:60-96
// (same skips, same termination before compositing the splat that would drop
// T below 1e-4).  Two shortcuts never change a result:
//   * a workgroup stops loading batches once every pixel has terminated
//     (__syncthreads_count), where the reference keeps loading;
//   * a per-Gaussian log-space bound skips the exp for pairs whose alpha is
//     provably below 1/255 (margin 1e-3 in log space, far above the exp and
//     log errors).
// Backward: back-to-front replay (rasterize.py:147-220) starting at the
// tile's largest n_contrib instead of the list end; the per-pair gradients
// are summed over the wave with DPP row operations, accumulated per
// Gaussian in LDS across the 4 waves, and flushed with one global atomic per
// (Gaussian, tile, component) instead of one per (pixel, Gaussian, component).
#include "gsx_device.h"

using namespace gsx;

namespace {

constexpr int kThreads = kTilePixels;

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

template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK,
                                                       BANK_MASK, false));
}

// Sum over the 64 lanes of the wave; the total ends up in lane 63.
// quad_perm xor1, xor2, half-row mirror, row mirror, then the gfx9
// row_bcast15 / row_bcast31 steps fold the four rows.
__device__ __forceinline__ float wave_total_lane63(float v) {
    v += dpp_f<0xB1, 0xF, 0xF>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E, 0xF, 0xF>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141, 0xF, 0xF>(v);  // row_half_mirror
    v += dpp_f<0x140, 0xF, 0xF>(v);  // row_mirror
    v += dpp_f<0x142, 0xA, 0xF>(v);  // row_bcast15 -> rows 1, 3
    v += dpp_f<0x143, 0xC, 0xF>(v);  // row_bcast31 -> rows 2, 3
    return v;
}

// Clamp a tile's [start, end) to the id array so a malformed range can
// never read outside it.
__device__ __forceinline__ void tile_span(int2 rg, int64_t n_ids, int& start, int& num) {
    const int64_t s0 = rg.x < 0 ? 0 : (rg.x > n_ids ? n_ids : rg.x);
    const int64_t s1 = rg.y < s0 ? s0 : (rg.y > n_ids ? n_ids : rg.y);
    start = (int)s0;
    num = (int)(s1 - s0);
}

// An id outside [0, N) stages a Gaussian with zero opacity: it never
// passes the alpha test and receives no gradient.
template <int CH>
__device__ __forceinline__ void load_empty(float4* s_xy, float4* s_co, float (*s_f)[kThreads],
                                           int tid) {
    s_xy[tid] = make_float4(0.0f, 0.0f, __builtin_huge_valf(), 0.0f);
    s_co[tid] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) s_f[ch][tid] = 0.0f;
}

template <int CH, bool DEPTH>
__global__ __launch_bounds__(kThreads) void k_raster_fwd(
    const float2* __restrict__ xy, const float4* __restrict__ co, const float* __restrict__ feat,
    int C, int c0, int nc, const float* __restrict__ depths, const int* __restrict__ ids,
    const int2* __restrict__ ranges, int64_t n, int64_t n_ids, const float* __restrict__ bg,
    int W, int H, int tiles_x, float* __restrict__ out, float* __restrict__ final_T,
    int* __restrict__ n_contrib, float* __restrict__ depth_out) {
    __shared__ float4 s_xy[kThreads];  // mean x, mean y, log-alpha bound, depth
    __shared__ float4 s_co[kThreads];  // conic a, b, c, opacity
    __shared__ float s_f[CH][kThreads];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = (int)xcd_remap(blockIdx.x, gridDim.x);
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px = tx * kTile + (wave & 1) * 8 + (lane & 7);
    const int py = ty * kTile + (wave >> 1) * 8 + (lane >> 3);
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
        if (k < num) {
            const int g = ids[start + k];
            if ((uint32_t)g < (uint64_t)n) {
                const float2 m = xy[g];
                const float4 c = co[g];
                s_xy[tid] = make_float4(m.x, m.y, alpha_floor_power(c.w), DEPTH ? depths[g] : 0.0f);
                s_co[tid] = c;
                const float* f = feat + (int64_t)g * C + c0;
#pragma unroll
                for (int ch = 0; ch < CH; ++ch) s_f[ch][tid] = (ch < nc) ? f[ch] : 0.0f;
            } else {
                load_empty<CH>(s_xy, s_co, s_f, tid);
            }
        }
        __syncthreads();
        if (!done) {
            const int bs = min(kThreads, num - base);
            for (int j = 0; j < bs; ++j) {
                const float4 a = s_xy[j];
                const float4 c = s_co[j];
                const float dx = a.x - pxf, dy = a.y - pyf;
                const float power = -0.5f * (c.x * dx * dx + c.z * dy * dy) - c.y * dx * dy;
                if (power > 0.0f || power < a.z) continue;
                const float alpha = fminf(0.99f, c.w * dexp(power));
                if (alpha < 1.0f / 255.0f) continue;
                const float next_T = T * (1.0f - alpha);
                if (next_T < 1e-4f) {
                    done = true;
                    break;
                }
                const float w = alpha * T;
#pragma unroll
                for (int ch = 0; ch < CH; ++ch) acc[ch] = acc[ch] + s_f[ch][j] * w;
                if (DEPTH) dacc = dacc + a.w * w;
                T = next_T;
                last = base + j + 1;
            }
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
    const float* __restrict__ final_T,
    const int* __restrict__ n_contrib, const float* __restrict__ grad_out,
    const float* __restrict__ grad_T, float* __restrict__ g_xy, float* __restrict__ g_conic,
    float* __restrict__ g_feat, float* __restrict__ g_opac) {
    constexpr int NV = CH + 6;          // dx, dy, conic a, b, c, opacity, channels
    constexpr int kAccStride = NV | 1;  // odd stride: conflict-free column reads
    __shared__ float4 s_xy[kThreads];
    __shared__ float4 s_co[kThreads];
    __shared__ float s_f[CH][kThreads];
    __shared__ int s_id[kThreads];
    __shared__ float s_acc[kThreads * kAccStride];
    __shared__ int s_max_last;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = (int)xcd_remap(blockIdx.x, gridDim.x);
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px = tx * kTile + (wave & 1) * 8 + (lane & 7);
    const int py = ty * kTile + (wave >> 1) * 8 + (lane >> 3);
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

    if (tid == 0) s_max_last = 0;
    __syncthreads();
    if (last > 0) atomicMax(&s_max_last, last);
    __syncthreads();
    const int n_batches = (s_max_last + kThreads - 1) / kThreads;

    float accum[CH], lastc[CH];
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) accum[ch] = lastc[ch] = 0.0f;
    float last_alpha = 0.0f;

    for (int b = n_batches - 1; b >= 0; --b) {
        __syncthreads();
        const int k = b * kThreads + tid;
        if (k < num) {
            const int g = ids[start + k];
            if ((uint32_t)g < (uint64_t)n) {
                s_id[tid] = g;
                const float2 m = xy[g];
                const float4 c = co[g];
                s_xy[tid] = make_float4(m.x, m.y, alpha_floor_power(c.w), 0.0f);
                s_co[tid] = c;
                const float* f = feat + (int64_t)g * C + c0;
#pragma unroll
                for (int ch = 0; ch < CH; ++ch) s_f[ch][tid] = (ch < nc) ? f[ch] : 0.0f;
            } else {
                s_id[tid] = -1;
                load_empty<CH>(s_xy, s_co, s_f, tid);
            }
        }
#pragma unroll
        for (int v = 0; v < NV; ++v) s_acc[tid * kAccStride + v] = 0.0f;
        __syncthreads();
        const int bs = min(kThreads, num - b * kThreads);
        for (int j = bs - 1; j >= 0; --j) {
            const int gj = b * kThreads + j;
            const float4 a = s_xy[j];
            const float4 c = s_co[j];
            const float dx = a.x - pxf, dy = a.y - pyf;
            const float power = -0.5f * (c.x * dx * dx + c.z * dy * dy) - c.y * dx * dy;
            bool ok = gj < last && !(power > 0.0f) && !(power < a.z);
            float G = 0.0f, alpha = 0.0f;
            if (ok) {
                G = dexp(power);
                alpha = fminf(0.99f, c.w * G);
                ok = !(alpha < 1.0f / 255.0f);
            }
            if (__ballot(ok) == 0ull) continue;
            float v[NV];
#pragma unroll
            for (int q = 0; q < NV; ++q) v[q] = 0.0f;
            if (ok) {
                T = T / (1.0f - alpha);
                const float aT = alpha * T;
                float dl = 0.0f;
#pragma unroll
                for (int ch = 0; ch < CH; ++ch) {
                    accum[ch] = last_alpha * lastc[ch] + (1.0f - last_alpha) * accum[ch];
                    const float f = s_f[ch][j];
                    lastc[ch] = f;
                    dl = dl + (f - accum[ch]) * gpix[ch];
                }
                last_alpha = alpha;
                float dL_dalpha = dl * T;
                dL_dalpha += (-T_final / (1.0f - alpha)) * bg_dot;
                const float dL_dG = c.w * dL_dalpha;
                const float gdx = G * dx, gdy = G * dy;
                v[0] = -(gdx * c.x + gdy * c.y) * dL_dG;
                v[1] = -(gdy * c.z + gdx * c.y) * dL_dG;
                v[2] = -0.5f * gdx * dx * dL_dG;
                v[3] = -gdx * dy * dL_dG;
                v[4] = -0.5f * gdy * dy * dL_dG;
                v[5] = G * dL_dalpha;
#pragma unroll
                for (int ch = 0; ch < CH; ++ch) v[6 + ch] = aT * gpix[ch];
            }
#pragma unroll
            for (int q = 0; q < NV; ++q) v[q] = wave_total_lane63(v[q]);
            if (lane == 63) {
#pragma unroll
                for (int q = 0; q < NV; ++q)
                    if (q < 6 + nc) atomicAdd(&s_acc[j * kAccStride + q], v[q]);
            }
        }
        __syncthreads();
        if (tid < bs && s_id[tid] >= 0) {
            const int g = s_id[tid];
            const float* e = &s_acc[tid * kAccStride];
            if (e[0] != 0.0f) atomicAdd(&g_xy[2 * g], e[0]);
            if (e[1] != 0.0f) atomicAdd(&g_xy[2 * g + 1], e[1]);
            if (e[2] != 0.0f) atomicAdd(&g_conic[3 * g], e[2]);
            if (e[3] != 0.0f) atomicAdd(&g_conic[3 * g + 1], e[3]);
            if (e[4] != 0.0f) atomicAdd(&g_conic[3 * g + 2], e[4]);
            if (e[5] != 0.0f) atomicAdd(&g_opac[g], e[5]);
#pragma unroll
            for (int ch = 0; ch < CH; ++ch)
                if (ch < nc && e[6 + ch] != 0.0f) atomicAdd(&g_feat[(int64_t)g * C + c0 + ch], e[6 + ch]);
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
