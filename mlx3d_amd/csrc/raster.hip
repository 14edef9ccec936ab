// raster.hip -- tile compositing (replaces gs_rasterize_forward,
// gs_rasterize_backward and gs_rasterize_depth, splatting/rasterize.py:28-290).
//
// One 256-lane workgroup (4 wave64) per 16x16 tile; wave w owns the 8x8
// pixel quadrant (w&1, w>>1).  The tile's depth-sorted Gaussians are staged
// through LDS in batches (two 16-byte records per Gaussian plus its
// channels, read as broadcasts).  While staging, each lane tests its
// Gaussian's alpha >= 1/255 ellipse against the four quadrants (exact
// minimum of the conic form over each quadrant's pixel centres, with a
// margin that covers the float32 rounding of the per-pixel power), and the
// workgroup publishes per quadrant a bit mask of the Gaussians that can
// touch it.  Each wave compacts its quadrant's bits into a list of record
// offsets and walks it in list order, reading each Gaussian's records while
// the previous one is evaluated.  Skipped pairs are exactly pairs whose
// alpha is below 1/255, which the reference also skips, so every output is
// unchanged.
//
// Forward: per-pixel front-to-back compositing as rasterize.py:60-96 (same
// skips, same termination before compositing the splat that would drop T
// below 1e-4), branch-free per pair; a wave stops once its 64 pixels have
// terminated and the workgroup stops loading once all 256 have.
// Backward: back-to-front replay (rasterize.py:147-220) from the largest
// n_contrib of each quadrant.  A pair's gradient terms are summed over the
// wave with cross-row swaps and DPP row operations (two Gaussians per
// reduction up to four channels); lane 15 of each row stores its share of
// the sums in the wave's own LDS slot for that Gaussian (no LDS atomics),
// and after the batch one lane per Gaussian adds the four waves' slots and
// issues one global atomic per (Gaussian, tile, component) -- the reference
// issues one per (pixel, Gaussian, component).
#include <algorithm>

#include "gsx_device.h"
#include "tile_order.h"

using namespace gsx;

namespace {

constexpr int kThreads = kTilePixels;
constexpr int kWaves = kThreads / kWave;  // 4 quadrant waves

// The compositing loops' exp (stands in for metal::exp at rasterize.py:80,
// 171), nine instructions: k = the integer nearest x log2 e from one fused
// multiply-add with the rounding constant 1.5 * 2^23 (j lies in
// [2^23, 2^24), where floats are spaced 1 apart, so j - 1.5 * 2^23 = k
// exactly); r = x - k ln2 with ln2 rounded to float32 (one multiply-add);
// e^r by the degree-5 polynomial p = 1 + r q(r) whose coefficients were
// fitted for least maximum relative error on |r| <= ln2/2; then 2^k p by
// one shift-and-add of j's encoding into p's (its low nine bits are
// k mod 2^9, so the shift adds k to the exponent field modulo 2^32; for x in
// [-86, 88] the result is normal and the add is the exact scaling).  At
// most 2.02 ulp from exp for x in [-6, 0] (every power that can pass the
// alpha test), 4.75 ulp on [-87, 0], and exp(0) = 1.  splat_exp_core is the
// sequence without range handling (callers that know x lies in [-86, 88]);
// splat_exp_sel adds it with selects: 0 below -86, +inf above 88, NaN
// unchanged.
__device__ __forceinline__ float splat_exp_core(float x) {
    const float j = fmaf(x, 1.44269504088896341f, 12582912.0f);
    const float k = j - 12582912.0f;
    const float r = fmaf(k, -0.693147182464599609375f, x);
    float q = 8.290260538610955e-03f;
    q = fmaf(q, r, 4.189814578274823e-02f);
    q = fmaf(q, r, 1.6667638172664237e-01f);
    q = fmaf(q, r, 4.9999147944277167e-01f);
    q = fmaf(q, r, 9.999997063356061e-01f);
    const float p = fmaf(q, r, 1.0f);
    return __uint_as_float(__float_as_uint(p) + (__float_as_uint(j) << 23));
}

__device__ __forceinline__ float splat_exp_sel(float x) {
    float e = splat_exp_core(fminf(fmaxf(x, -86.0f), 88.0f));
    e = (x < -86.0f) ? 0.0f : e;
    e = (x > 88.0f) ? __builtin_huge_valf() : e;
    return (x != x) ? x : e;
}

// rasterize.py:77-78, power = -0.5 (a dx^2 + c dy^2) - b dx dy, with the
// conic staged pre-scaled to (A, B, C) = (-a/2, -b, -c/2) (exact scalings)
// and factored as power = (A dx + B dy) dx + (C dy) dy: three products and
// two multiply-adds, five roundings whose error is at most
// 2 eps (|A| dx^2 + |B dx dy| + |C| dy^2) + eps |power| (eps = 2^-24).
__device__ __forceinline__ float splat_power(float A, float B, float C, float dx, float dy) {
    return fmaf(fmaf(B, dy, A * dx), dx, (C * dy) * dy);
}

// ln x from the hardware base-2 logarithm (about 1 ulp of log2 x, plus the
// rounding of the product): the culling bounds below carry margins of
// 1e-3 + 1e-4 |L| (alpha_floor_power) and 1% + 1e-3 (quadrant_mask), far
// above that error.  x must be a positive normal number.
__device__ __forceinline__ float ln_fast(float x) {
    return __builtin_amdgcn_logf(x) * 0.693147180559945309f;
}

// Power below which o * exp(power) < 1/255 for certain.  +inf when the
// opacity can never reach 1/255 (o <= 0 or tiny), -inf when no bound is safe
// (o NaN or +inf).
__device__ __forceinline__ float alpha_floor_power(float o) {
    if (o > 0.0f) {
        // ln(1 / (255 o)); below the normal range the bound is 200 anyway
        float L = 255.0f * o >= 1.17549435e-38f ? -ln_fast(255.0f * o) : 200.0f;
        L = fminf(L, 200.0f);
        return L - (1e-3f + 1e-4f * fabsf(L));
    }
    if (o <= 0.0f) return __builtin_huge_valf();
    return -__builtin_huge_valf();
}

// Which of the tile's four 8x8 quadrants (bit q = quadrant (q&1, q>>1)) the
// pixels with alpha >= 1/255 of this Gaussian can lie in.  alpha >= 1/255
// needs q(d) = a dx^2 + 2 b dx dy + c dy^2 <= 2 ln(255 o); a quadrant is
// kept when the minimum of q over its rectangle of pixel centres is within
// that bound: zero if the mean is inside, else the least of the four edge
// minima.  On a row dy = k, q = a (dx + b k / a)^2 + k^2 det / a, so the
// edge minimum is that expression at dx clamped to the edge (columns alike
// with a and c exchanged), and the eight edge lines are shared by the
// quadrants.  Float32 throughout: with det > 1e-3 a c every term carries a
// relative error below 1e-4, and with b^2 < 0.999 a c the float32
// evaluation of the power (splat_power) is within 4.8e-4 relative of the
// exact value, so tau is inflated by 1% (+1e-3); the float32 log of the
// bound and the <= 5 ulp of splat_exp add errors of ~1e-6, well inside
// that.  Ill-conditioned, non-positive or non-finite conics get no culling
// (all four bits).
__device__ __forceinline__ uint32_t quadrant_mask(float x, float y, float4 c, int px0, int py0) {
    const float o = c.w;
    if (!(o >= 0.0039215f)) return (o == o) ? 0u : 0xFu;  // alpha < 1/255 everywhere
    const float A = c.x, B = c.y, C = c.z;
    const float det = fmaf(A, C, -B * B);
    if (!(A > 0.0f && C > 0.0f && det > 1e-3f * A * C)) return 0xFu;
    const float t2 = 2.0f * fmaf(ln_fast(255.0f * o), 1.01f, 1e-3f);
    if (!(t2 < 1e30f && A < 1e30f && C < 1e30f && fabsf(x) < 1e30f && fabsf(y) < 1e30f))
        return 0xFu;
    const float ia = __builtin_amdgcn_rcpf(A), ic = __builtin_amdgcn_rcpf(C);
    const float ba = -B * ia, bc = -B * ic, da = det * ia, dc = det * ic;
    // pixel-centre offsets from the mean: columns [xl0, xl0 + 7] (left
    // quadrants) and [xl0 + 8, xl0 + 15] (right), rows likewise
    const float xl0 = ((float)px0 + 0.5f) - x, xl1 = xl0 + 7.0f;
    const float xr0 = xl0 + 8.0f, xr1 = xl0 + 15.0f;
    const float yt0 = ((float)py0 + 0.5f) - y, yt1 = yt0 + 7.0f;
    const float yb0 = yt0 + 8.0f, yb1 = yt0 + 15.0f;
    // minimum of q on row dy = k over dx in [lo, hi], and on columns
    auto row = [&](float k, float lo, float hi) {
        const float xs = ba * k, u = fminf(fmaxf(xs, lo), hi) - xs;
        return fmaf(A * u, u, k * k * da);
    };
    auto col = [&](float k, float lo, float hi) {
        const float ys = bc * k, u = fminf(fmaxf(ys, lo), hi) - ys;
        return fmaf(C * u, u, k * k * dc);
    };
    const bool inl = xl0 <= 0.0f && xl1 >= 0.0f, inr = xr0 <= 0.0f && xr1 >= 0.0f;
    const bool intp = yt0 <= 0.0f && yt1 >= 0.0f, inb = yb0 <= 0.0f && yb1 >= 0.0f;
    // With the mean outside a rectangle, q's minimum over it lies on an edge
    // whose outer side holds the mean (at a minimiser inside an edge the
    // gradient 2M(p - mean) points into the rectangle, so the mean lies
    // beyond that edge): of each quadrant's two rows and two columns only
    // the one nearer the mean can hold it, and the other edge of the pair
    // is an upper bound, so min(row edge, column edge) is the minimum.
    const float kt = yt1 < 0.0f ? yt1 : yt0, kb = yb1 < 0.0f ? yb1 : yb0;
    const float kl = xl1 < 0.0f ? xl1 : xl0, kr = xr1 < 0.0f ? xr1 : xr0;
    const float q0 = fminf(row(kt, xl0, xl1), col(kl, yt0, yt1));
    const float q1 = fminf(row(kt, xr0, xr1), col(kr, yt0, yt1));
    const float q2 = fminf(row(kb, xl0, xl1), col(kl, yb0, yb1));
    const float q3 = fminf(row(kb, xr0, xr1), col(kr, yb0, yb1));
    return ((inl && intp) || q0 <= t2 ? 1u : 0u) | ((inr && intp) || q1 <= t2 ? 2u : 0u) |
           ((inl && inb) || q2 <= t2 ? 4u : 0u) | ((inr && inb) || q3 <= t2 ? 8u : 0u);
}

// A staged Gaussian is "plain" when every quantity the per-pixel loop reads
// is finite and small enough that the float32 power is finite and, for a
// pixel that passes the alpha bound, within [-86, 0]: then exp needs no
// range handling and a zero weight leaves the accumulators unchanged.
//
// The conic must also be well conditioned, det > 1e-6 (a + c)^2 with
// a + c in [1e-12, 1e19), and then the float32 power (splat_power) is never
// positive, so the loops need no power > 0 test.  Its rounding error is at
// most eps (a dx^2 + c dy^2 + 2 |b dx dy|) <= 1.25 eps (a + c) |d|^2
// (eps = 2^-24, |b| < (a + c) / 2), while the exact value is at most
// -lambda_min |d|^2 / 2 with lambda_min >= det / (a + c) > 1e-6 (a + c) (the
// float32 det and trace lose far less than the factor 6.7 of margin).  A
// nonzero offset has |d| >= 2^-25 (pixel centres are >= 0.5 and the
// difference of two floats within a factor two of each other is exact), so
// the exact value stays above 4e-34 in magnitude, far from where the
// denormal rounding of the products (<= 2^-150 each) could matter; at d = 0
// the power is a signed zero.
template <int CH>
__device__ __forceinline__ bool plain_gaussian(float x, float y, float4 c, float thr,
                                               const float4* f) {
    const float tr = c.x + c.z, det = fmaf(c.x, c.z, -c.y * c.y);
    bool ok = fabsf(x) < 1e6f && fabsf(y) < 1e6f && tr >= 1e-12f && tr < 1e19f &&
              det > 1e-6f * (tr * tr) && c.w >= 0.0f && c.w < 1e30f && thr >= -86.0f;
    constexpr int F4 = (CH + 3) / 4;
#pragma unroll
    for (int k = 0; k < F4; ++k)
        ok = ok && fabsf(f[k].x) < 1e30f && fabsf(f[k].y) < 1e30f && fabsf(f[k].z) < 1e30f &&
             fabsf(f[k].w) < 1e30f;
    return ok;
}

template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK,
                                                       BANK_MASK, false));
}

// In-place v_permlane32_swap (upper 32 lanes of a[k] <-> lower 32 lanes of
// b[k]) and v_permlane16_swap (odd rows of a[k] <-> even rows of b[k]) for
// K register pairs, up to four per asm block.  Written as asm so the
// operands are swapped where they live (the builtins' two results made the
// register allocator copy both operands first); each block starts with
// s_nop 1, the two wait states a swap needs after a VALU write of its
// operands, since the compiler's hazard check cannot see into the asm (the
// swaps inside a block touch disjoint registers).
#define GSX_SWAP_BLOCK(OP, K, a, b)                                                          \
    do {                                                                                     \
        if constexpr (K >= 4) {                                                              \
            asm("s_nop 1\n\t" OP " %0, %1\n\t" OP " %2, %3\n\t" OP " %4, %5\n\t" OP " %6, %7" \
                : "+v"(a[0]), "+v"(b[0]), "+v"(a[1]), "+v"(b[1]), "+v"(a[2]), "+v"(b[2]),    \
                  "+v"(a[3]), "+v"(b[3]));                                                   \
        } else if constexpr (K == 3) {                                                       \
            asm("s_nop 1\n\t" OP " %0, %1\n\t" OP " %2, %3\n\t" OP " %4, %5"                \
                : "+v"(a[0]), "+v"(b[0]), "+v"(a[1]), "+v"(b[1]), "+v"(a[2]), "+v"(b[2]));   \
        } else if constexpr (K == 2) {                                                       \
            asm("s_nop 1\n\t" OP " %0, %1\n\t" OP " %2, %3"                                 \
                : "+v"(a[0]), "+v"(b[0]), "+v"(a[1]), "+v"(b[1]));                           \
        } else if constexpr (K == 1) {                                                       \
            asm("s_nop 1\n\t" OP " %0, %1" : "+v"(a[0]), "+v"(b[0]));                        \
        }                                                                                    \
    } while (0)

// The last two steps of a 16-lane row sum for K registers, up to four per
// asm block: t[k] += t[k] of the mirrored lane of its 8-lane half-row (DPP
// row_half_mirror), then += that of the mirrored lane of its row
// (row_mirror), after which every lane of a row holds the row's total.
// asm (volatile) so the adds are not sunk into the following one-lane store
// branch, where each would become a DPP move with a zero fill plus a
// separate add; s_nop 1 gives the two wait states a DPP read needs after a
// VALU write of its operand.
#define GSX_DPP_ADD(r, ctl) "v_add_f32_dpp " r ", " r ", " r " " ctl " row_mask:0xf bank_mask:0xf\n\t"
#define GSX_ROW_TAIL1(ctl) GSX_DPP_ADD("%0", ctl)
#define GSX_ROW_TAIL2(ctl) GSX_DPP_ADD("%0", ctl) GSX_DPP_ADD("%1", ctl)
#define GSX_ROW_TAIL3(ctl) GSX_DPP_ADD("%0", ctl) GSX_DPP_ADD("%1", ctl) GSX_DPP_ADD("%2", ctl)
#define GSX_ROW_TAIL4(ctl) \
    GSX_DPP_ADD("%0", ctl) GSX_DPP_ADD("%1", ctl) GSX_DPP_ADD("%2", ctl) GSX_DPP_ADD("%3", ctl)
#define GSX_ROW_TAIL(N)                                                                   \
    "s_nop 1\n\t" GSX_ROW_TAIL##N("row_half_mirror") "s_nop 1\n\t" GSX_ROW_TAIL##N("row_mirror")

template <int K>
__device__ __forceinline__ void row_tail_add(float (&t)[K]) {
    static_assert(K >= 1 && K <= 4, "one to four registers per block");
    if constexpr (K == 4) {
        asm volatile(GSX_ROW_TAIL(4) : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]));
    } else if constexpr (K == 3) {
        asm volatile(GSX_ROW_TAIL(3) : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]));
    } else if constexpr (K == 2) {
        asm volatile(GSX_ROW_TAIL(2) : "+v"(t[0]), "+v"(t[1]));
    } else {
        asm volatile(GSX_ROW_TAIL(1) : "+v"(t[0]));
    }
}

template <int K>
__device__ __forceinline__ void swap_rows32(float (&a)[K], float (&b)[K]) {
    GSX_SWAP_BLOCK("v_permlane32_swap_b32", K, a, b);
}
template <int K>
__device__ __forceinline__ void swap_rows16(float (&a)[K], float (&b)[K]) {
    GSX_SWAP_BLOCK("v_permlane16_swap_b32", K, a, b);
}

// Sums of NVP per-lane values (NVP a multiple of 4) over the 64 lanes of
// the wave, spread over the four 16-lane rows: afterwards every lane of row
// r holds in q[m] the total of value 4m + row_value(r).  Step 1 swaps the
// upper half of value 2k with the lower half of value 2k + 1 and adds, so
// each half carries one of the two values; step 2 does the same between
// rows; step 3 sums each row with four DPP steps.  NVP + NVP/2 + NVP
// exchanges/adds instead of 6 NVP for a separate 64-lane reduction of every
// value.  Values from index NZ on are known zeros: pairs of them skip their
// exchange.  All lanes must be active.
__device__ __forceinline__ int row_value(int row) { return ((row & 1) << 1) | (row >> 1); }

// Step 1 for value pairs K0..K1-1: h[k] = swap32-sum of v[2k], v[2k + 1]
// (values from NZ on are zeros), four pairs per asm block.
template <int K0, int K1, int NVP, int NZ>
__device__ __forceinline__ void reduce_step1(const float (&v)[NVP], float (&h)[NVP / 2]) {
    if constexpr (K0 < K1) {
        constexpr int N = (K1 - K0) < 4 ? (K1 - K0) : 4;
        float a[N], b[N];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            a[k] = v[2 * (K0 + k)];
            b[k] = 2 * (K0 + k) + 1 < NZ ? v[2 * (K0 + k) + 1] : 0.0f;
        }
        swap_rows32<N>(a, b);
#pragma unroll
        for (int k = 0; k < N; ++k) h[K0 + k] = a[k] + b[k];
        reduce_step1<K0 + N, K1, NVP, NZ>(v, h);
    }
}

// Step 2 alone for row groups M0..M1-1: q[m] = swap16-sum of h[2m],
// h[2m + 1] (the row's partial of value 4m + row_value(row)).
template <int M0, int M1, int NVP>
__device__ __forceinline__ void reduce_step2(const float (&h)[NVP / 2], float (&q)[NVP / 4]) {
    if constexpr (M0 < M1) {
        constexpr int N = (M1 - M0) < 4 ? (M1 - M0) : 4;
        float a[N], b[N];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            a[k] = h[2 * (M0 + k)];
            b[k] = h[2 * (M0 + k) + 1];
        }
        swap_rows16<N>(a, b);
#pragma unroll
        for (int k = 0; k < N; ++k) q[M0 + k] = a[k] + b[k];
        reduce_step2<M0 + N, M1, NVP>(h, q);
    }
}

// Steps 2 and 3 for row groups M0..M1-1: swap16-sum of h[2m], h[2m + 1],
// then the four DPP steps within each row.
template <int M0, int M1, int NVP>
__device__ __forceinline__ void reduce_step23(const float (&h)[NVP / 2], float (&q)[NVP / 4]) {
    if constexpr (M0 < M1) {
        constexpr int N = (M1 - M0) < 4 ? (M1 - M0) : 4;
        float a[N], b[N];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            a[k] = h[2 * (M0 + k)];
            b[k] = h[2 * (M0 + k) + 1];
        }
        swap_rows16<N>(a, b);
#pragma unroll
        for (int k = 0; k < N; ++k) {
            float t = a[k] + b[k];
            t += dpp_f<0xB1, 0xF, 0xF>(t);  // quad_perm [1,0,3,2]
            t += dpp_f<0x4E, 0xF, 0xF>(t);  // quad_perm [2,3,0,1]
            a[k] = t;
        }
        row_tail_add<N>(a);
#pragma unroll
        for (int k = 0; k < N; ++k) q[M0 + k] = a[k];
        reduce_step23<M0 + N, M1, NVP>(h, q);
    }
}

template <int NVP, int NZ = NVP>
__device__ __forceinline__ void wave_reduce_rows(const float (&v)[NVP], float (&q)[NVP / 4]) {
    static_assert(NVP % 4 == 0 && NZ <= NVP, "values come in groups of four");
    constexpr int K1 = (NZ + 1) / 2;  // value pairs with a non-zero member
    constexpr int K2 = (K1 + 1) / 2;  // row groups with a non-zero member
    float h[NVP / 2];
#pragma unroll
    for (int k = K1; k < NVP / 2; ++k) h[k] = 0.0f;
    reduce_step1<0, K1, NVP, NZ>(v, h);
#pragma unroll
    for (int m = K2; m < NVP / 4; ++m) q[m] = 0.0f;
    reduce_step23<0, K2, NVP>(h, q);
}

__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}


// Tile processing order.  Workgroups go round-robin over the 8 XCDs and a
// workgroup slot that frees takes the next workgroup of its XCD, so the
// kernel ends when the last XCD drains its share; tiles differ in work by
// 2-3x (crowded regions of the frame).  xcd_remap gives each XCD a
// contiguous band of tiles (neighbours share its L2: the same Gaussians'
// records).  With an order (k_tile_order) the bands stay contiguous, each
// XCD takes its band's heaviest tiles first (longest-processing-time-first
// list scheduling), and for the backward, whose per-tile work the forward
// recorded exactly, the bands are cut to equal work rather than equal tile
// counts, with up to twice the mean tiles per band: the backward then
// launches 16 ceil(T / 8) workgroups, those past a band's end exit at once.
// Ordering the whole frame instead, heaviest first regardless of bands,
// balanced as well but doubled the rasterizers' HBM traffic (1.05 GB per
// C3 backward instead of 0.47: neighbouring tiles on different XCDs).
// by_block: order is indexed by workgroup (the backward's layout), else by
// xcd_remap position; -1 = no tile.
__device__ __forceinline__ int tile_at(const int* order, uint32_t b, uint32_t nb, bool by_block) {
    if (!order) return (int)xcd_remap(b, nb);
    return order[by_block ? b : xcd_remap(b, nb)];
}

// The workgroup's largest contributor count (n_contrib) into work[tile]:
// the number of list entries the backward replays for the tile.  Every
// thread of the workgroup calls it.
__device__ __forceinline__ void store_tile_work(int* work, int tile, int last, int wave,
                                                int lane) {
    __shared__ int s_wmax[kWaves];
    int m = last;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, kWave));
    if (lane == 0) s_wmax[wave] = m;
    __syncthreads();
    if (wave == 0 && lane == 0)
        work[tile] = max(max(s_wmax[0], s_wmax[1]), max(s_wmax[2], s_wmax[3]));
}

// A quadrant wave's walk list: the staged Gaussians whose bit is set in the
// quadrant's NW mask words (loader wave lw, lane l <-> staged index
// 64 lw + l), compacted in LDS as 32-bit record byte offsets (16 x index)
// so the walk is a counted loop over uniform offsets.  Built by the wave
// itself after the workgroup barrier that publishes the masks; ascending
// index order (REV: descending).  list[cnt .. cnt + PADS - 1] are set to
// pad, a valid record offset, for the walks' look-ahead.  Returns cnt
// (uniform).
template <int NW, bool REV, int PADS = 2>
__device__ __forceinline__ int build_list(const uint64_t* words, uint32_t* list, int lane,
                                          int pad) {
    int total = 0;
    const uint64_t below = (1ull << lane) - 1ull;
    const uint64_t above = lane == 63 ? 0ull : ~((2ull << lane) - 1ull);
#pragma unroll
    for (int k = 0; k < NW; ++k) {
        const int lw = REV ? NW - 1 - k : k;
        const uint64_t m = uniform64(words[lw]);
        if ((m >> lane) & 1ull)
            list[total + __popcll(m & (REV ? above : below))] = (uint32_t)((lw * kWave + lane) * 16);
        total += __popcll(m);
    }
    if (lane < PADS) list[total + lane] = (uint32_t)pad;
    return total;
}

// The staged record at a byte offset from a list (16 x staged index).
__device__ __forceinline__ const float4& rec_at(const float4* base, int off) {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(base) + off);
}

template <int CH>
__device__ __forceinline__ void stage_features(float4* dst, const float* f, int nc) {
    constexpr int F4 = (CH + 3) / 4;
    float v[4 * F4];
    if (nc >= CH) {  // uniform: every channel, loads without branches
#pragma unroll
        for (int ch = 0; ch < 4 * F4; ++ch) v[ch] = ch < CH ? f[ch] : 0.0f;
    } else {
#pragma unroll
        for (int ch = 0; ch < 4 * F4; ++ch) v[ch] = (ch < CH && ch < nc) ? f[ch] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < F4; ++k) dst[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
}

__device__ __forceinline__ float comp4(const float4& v, int e) {
    return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

// One (pixel, Gaussian) step of the front-to-back loop (rasterize.py:74-87):
// lanes that do not composite keep their state.  PLAIN: the Gaussian passed
// plain_gaussian(), so its power is never positive and exp needs no range
// handling; the channel sums then run under the compositing lanes' exec
// mask (a branch that no lane takes is skipped).  Otherwise every update is
// a select.  The per-lane decisions are kept as wave masks (alive: the
// pixel has not stopped): a ballot of one comparison is that comparison's
// lane mask, the masks combine in scalar registers, and inverse_ballot
// hands one back to the lanes as a select condition, so none of it costs
// vector ALU work.
template <int CH, bool DEPTH, bool PLAIN>
__device__ __forceinline__ void fwd_pair(const float4& r0, const float4& r1,
                                         const float4 (&fv)[(CH + 3) / 4], int off,
                                         float pxf, float pyf, float& T, float* acc,
                                         float& dacc, int& last_off, uint64_t& alive) {
    const float dx = r0.x - pxf, dy = r0.y - pyf;
    const float power = splat_power(r1.x, r1.y, r1.z, dx, dy);
    const uint64_t live =
        PLAIN ? alive & __ballot(!(power < r0.z))
              : alive & __ballot(!(power > 0.0f)) & __ballot(!(power < r0.z));
    const float e = PLAIN ? splat_exp_core(power) : splat_exp_sel(power);
    const float alpha = fminf(0.99f, r0.w * e);
    const uint64_t pass = live & __ballot(!(alpha < 1.0f / 255.0f));
    const float next_T = T * (1.0f - alpha);
    const uint64_t lt = __ballot(next_T < 1e-4f);
    alive &= ~(pass & lt);  // the reference's early stop
    const bool add = __builtin_amdgcn_inverse_ballot_w64(pass & ~lt);
    // acc += rgb * (alpha * T) (rasterize.py:84) as one fused multiply-add,
    // the contraction Metal's default fast-math applies to the reference
    const float w = alpha * T;
    if (PLAIN) {
        T = add ? next_T : T;
        last_off = add ? off : last_off;
        if (add) {
            // keeps the sums a branch (the compiler would turn them into
            // selects) and w computed before it
            asm volatile("" ::"v"(w) : "memory");
#pragma unroll
            for (int ch = 0; ch < CH; ++ch) acc[ch] = fmaf(comp4(fv[ch >> 2], ch & 3), w, acc[ch]);
            if (DEPTH) dacc = fmaf(r1.w, w, dacc);
        }
        return;
    } else {
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
            const float a2 = fmaf(comp4(fv[ch >> 2], ch & 3), w, acc[ch]);
            acc[ch] = add ? a2 : acc[ch];
        }
        if (DEPTH) {
            const float d2 = fmaf(r1.w, w, dacc);
            dacc = add ? d2 : dacc;
        }
    }
    T = add ? next_T : T;
    last_off = add ? off : last_off;
}

// Front-to-back walk of one quadrant wave over its list, four Gaussians per
// round: each Gaussian's records (and, up to four channels, its channels)
// are read while the one before it is evaluated, and list entries two
// places ahead.  list[cnt .. cnt + 3] are the padding record, which no pixel
// takes, so a round may run past the list's end (a stale entry is read only
// as the next round's offsets and never used, since the round count ends
// first).  The wave stops once its 64 pixels have terminated.  last_off gets
// the offset of each pixel's last composited Gaussian of this batch.
template <int CH, bool DEPTH, bool PLAIN>
__device__ __forceinline__ void fwd_walk(const uint32_t* list, int cnt, const float4* s_r0,
                                         const float4* s_r1, const float4 (*s_f)[(CH + 3) / 4],
                                         float pxf, float pyf, float& T, float* acc, float& dacc,
                                         int& last_off, uint64_t& alive) {
    constexpr int F4 = (CH + 3) / 4;
    // more channels are read just before their pair (registers)
    constexpr bool kAhead = F4 == 1;
    if (cnt == 0) return;
    const float4* sf = &s_f[0][0];
    float4 fa[F4], fb[F4];
    auto feat = [&](float4 (&f)[F4], int off) {
#pragma unroll
        for (int q = 0; q < F4; ++q) f[q] = (&rec_at(sf, off * F4))[q];
    };
    auto pair = [&](const float4& r0, const float4& r1, float4 (&f)[F4], int off) {
        if (!kAhead) feat(f, off);
        fwd_pair<CH, DEPTH, PLAIN>(r0, r1, f, off, pxf, pyf, T, acc, dacc, last_off, alive);
    };
    int oa = list[0], ob = list[1];
    float4 a0 = rec_at(s_r0, oa), a1 = rec_at(s_r1, oa);
    if (kAhead) feat(fa, oa);
    for (int i = 0;; i += 4) {
        const int nc = list[i + 2], nd = list[i + 3];
        float4 b0 = rec_at(s_r0, ob), b1 = rec_at(s_r1, ob);
        if (kAhead) feat(fb, ob);
        pair(a0, a1, fa, oa);
        a0 = rec_at(s_r0, nc);
        a1 = rec_at(s_r1, nc);
        if (kAhead) feat(fa, nc);
        pair(b0, b1, fb, ob);
        const int na = list[i + 4], nb = list[i + 5];
        b0 = rec_at(s_r0, nd);
        b1 = rec_at(s_r1, nd);
        if (kAhead) feat(fb, nd);
        pair(a0, a1, fa, nc);
        a0 = rec_at(s_r0, na);
        a1 = rec_at(s_r1, na);
        if (kAhead) feat(fa, na);
        pair(b0, b1, fb, nd);
        if (alive == 0ull || i + 4 >= cnt) return;
        oa = na;
        ob = nb;
    }
}

// Occupancy targets that the compiler meets without spilling: seven waves
// per SIMD (<= 72 VGPRs) up to three channels (C3's forward 193.8 -> 190.4
// us against six), six up to four, five up to eight.
constexpr int fwd_min_waves(int ch) { return ch <= 3 ? 7 : (ch <= 4 ? 6 : (ch <= 8 ? 5 : 1)); }

template <int CH, bool DEPTH>
__global__ __launch_bounds__(kThreads, fwd_min_waves(CH)) void k_raster_fwd(
    const float2* __restrict__ xy, const float4* __restrict__ co, const float* __restrict__ feat,
    int C, int c0, int nc, const float* __restrict__ depths, const int* __restrict__ ids,
    const int2* __restrict__ ranges, int64_t n, int64_t n_ids, const float* __restrict__ bg,
    int W, int H, int tiles_x, float* __restrict__ out, float* __restrict__ final_T,
    int* __restrict__ n_contrib, float* __restrict__ depth_out, float* __restrict__ alpha_out,
    const int* __restrict__ order, int* __restrict__ work) {
    constexpr int F4 = (CH + 3) / 4;
    // entry kThreads of the records is the walk lists' padding: a record no
    // pixel can take (alpha bound +inf)
    __shared__ float4 s_r0[kThreads + 1];     // mean x, mean y, log-alpha bound, opacity
    __shared__ float4 s_r1[kThreads + 1];     // -a/2, -b, -c/2 (conic), depth
    __shared__ float4 s_f[kThreads + 1][F4];  // channels, zero padded
    __shared__ uint64_t s_mask[kWaves][kWaves];  // [quadrant][loader wave]
    __shared__ uint32_t s_list[kWaves][kThreads + 8];  // walk lists (+ look-ahead room)
    // one word per wave, written before a barrier and read by every thread
    // after it (a 16-byte read): some pixel of the wave still composites /
    // every Gaussian the wave staged is plain.  Each batch's reads come
    // before the next barrier, and the next batch writes only after it.
    __shared__ __align__(16) uint32_t s_alive[kWaves];
    __shared__ __align__(16) uint32_t s_plain[kWaves];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = __builtin_amdgcn_readfirstlane(tile_at(order, blockIdx.x, gridDim.x, false));
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
    uint64_t alive = __ballot(inside);  // the wave's pixels still compositing
    // the padding record (written before the first barrier)
    if (tid == 0) {
        s_r0[kThreads] = make_float4(0.0f, 0.0f, __builtin_huge_valf(), 0.0f);
        s_r1[kThreads] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int q = 0; q < F4; ++q) s_f[kThreads][q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }

    for (int base = 0; base < num; base += kThreads) {
        if (lane == 0) s_alive[wave] = alive != 0ull;
        __syncthreads();
        const uint4 al = *reinterpret_cast<const uint4*>(s_alive);
        if ((al.x | al.y | al.z | al.w) == 0u) break;  // all 256 pixels done
        const int k = base + tid;
        uint32_t qm = 0;
        bool plain = true;
        if (k < num) {
            const int g = ids[start + k];
            if ((uint32_t)g < (uint64_t)n) {
                // the record, depth and feature loads issue together
                const float2 m = xy[g];
                const float4 c = co[g];
                const float dz = DEPTH ? depths[g] : 0.0f;
                stage_features<CH>(s_f[tid], feat + (int64_t)g * C + c0, nc);
                const float thr = alpha_floor_power(c.w);
                s_r0[tid] = make_float4(m.x, m.y, thr, c.w);
                s_r1[tid] = make_float4(-0.5f * c.x, -c.y, -0.5f * c.z, dz);
                qm = quadrant_mask(m.x, m.y, c, px0, py0);
                plain = plain_gaussian<CH>(m.x, m.y, c, thr, s_f[tid]) && fabsf(dz) < 1e30f;
            }
        }
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
            const uint64_t b = __ballot((qm >> q) & 1u);
            if (lane == 0) s_mask[q][wave] = b;
        }
        const uint64_t np = __ballot(!plain);
        if (lane == 0) s_plain[wave] = np == 0ull;
        __syncthreads();
        const uint4 pl = *reinterpret_cast<const uint4*>(s_plain);
        const bool batch_plain = (pl.x & pl.y & pl.z & pl.w) != 0u;
        if (alive == 0ull) continue;
        const int cnt =
            build_list<kWaves, false, 4>(s_mask[wave], s_list[wave], lane, kThreads * 16);
        int last_off = -1;
        if (batch_plain)
            fwd_walk<CH, DEPTH, true>(s_list[wave], cnt, s_r0, s_r1, s_f, pxf, pyf, T, acc, dacc,
                                      last_off, alive);
        else
            fwd_walk<CH, DEPTH, false>(s_list[wave], cnt, s_r0, s_r1, s_f, pxf, pyf, T, acc,
                                       dacc, last_off, alive);
        if (last_off >= 0) last = base + (last_off >> 4) + 1;
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
            if (alpha_out) alpha_out[pid] = 1.0f - T;
            if (DEPTH) {
                const float al = 1.0f - T;
                depth_out[pid] = al > 1e-6f ? dacc / al : 0.0f;
            }
        }
    }
    if (work) store_tile_work(work, tile, last, wave, lane);
}

// Per-pixel state of the back-to-front replay.
//
// The reference (rasterize.py:170-195) carries per channel the recursively
// blended colour behind the current Gaussian, accum_c = S_c / T_after with
// S_c = sum over later contributors k of c_k alpha_k T_k, and forms
//   dL/dalpha_i = T_i sum_c g_c (c_i - accum_c) - T_final (bg . g) / (1 - alpha_i).
// Since T_i / T_after = 1 / (1 - alpha_i), the channel sum of g_c accum_c
// collapses into one scalar,
//   Q = T_final (bg . g) + sum over later contributors k of alpha_k T_k (c_k . g),
//   dL/dalpha_i = T_i (c_i . g) - Q / (1 - alpha_i),
// so a pixel holds its cotangent g (CH floats) and Q instead of 3 CH floats.
template <int CH>
struct BwdPixel {
    float T;  // transmittance in front of the current Gaussian
    float Q;
    int last;
    float gpix[CH];
};

// One (pixel, Gaussian) step of the back-to-front replay
// (rasterize.py:162-219).  Returns whether any lane of the wave contributes
// and writes each lane's values to out[S q + O] (all zeros when none does):
//   u = G dx dL/dalpha, w = G dy dL/dalpha, u dx, u dy, w dy, G dL/dalpha,
//   alpha T g_c
// (zero for lanes that do not contribute), whose wave sums the flush turns
// into the reference's means2d, conic, opacity and colour gradients (linear
// in these sums).  power, alpha and the skip tests repeat the forward's
// float32 arithmetic exactly (the replay must take the forward's
// decisions); the gradient arithmetic itself uses fused multiply-adds.  T is
// recovered with one reciprocal of (1 - alpha) per pair.  off is the
// Gaussian's record offset (16 x its staged index) and lim = 16 (n_contrib -
// batch base): the pixel's forward composited it only if off < lim.  PLAIN:
// inputs are finite, so a lane that does not contribute can run the same
// update with a zero weight.
template <int CH, bool PLAIN, int S = 1, int O = 0, int NW>
__device__ __forceinline__ bool bwd_values(const float4& r0, const float4& r1,
                                           const float4* __restrict__ fsrc, int off, int lim,
                                           float pxf, float pyf, BwdPixel<CH>& px,
                                           float (&out)[NW]) {
    static_assert(S * (CH + 5) + O < NW, "strided values fit the output array");
    constexpr int F4 = (CH + 3) / 4;
    constexpr int NV = CH + 6;
    const float dx = r0.x - pxf, dy = r0.y - pyf;
    const float power = splat_power(r1.x, r1.y, r1.z, dx, dy);
    // the wave-wide tests ballot each comparison on its own: a ballot of a
    // single comparison is its lane mask, one of a combined condition is
    // first materialised in a vector register
    // PLAIN: the power is never positive (plain_gaussian's conic bound)
    const bool c1 = off < lim, c2 = PLAIN || !(power > 0.0f), c3 = !(power < r0.z);
    bool ok = c1 && c2 && c3;
    const uint64_t m123 = PLAIN ? __ballot(c1) & __ballot(c3)
                                : __ballot(c1) & __ballot(c2) & __ballot(c3);
    if (m123 == 0ull) {
#pragma unroll
        for (int q = 0; q < NV; ++q) out[S * q + O] = 0.0f;
        return false;
    }
    // PLAIN: lanes that pass have power in [-86, 0]; the others' G is
    // replaced by zero below, whatever its value.
    const float G = PLAIN ? splat_exp_core(power) : splat_exp_sel(power);
    const float alpha = fminf(0.99f, r0.w * G);
    const bool c4 = !(alpha < 1.0f / 255.0f);
    ok = ok && c4;
    if ((m123 & __ballot(c4)) == 0ull) {
        // every output is written on every path, so callers hold no stale
        // values across iterations
#pragma unroll
        for (int q = 0; q < NV; ++q) out[S * q + O] = 0.0f;
        return false;
    }
    float4 fv[F4];
#pragma unroll
    for (int q = 0; q < F4; ++q) fv[q] = fsrc[q];
    float cg = 0.0f;  // c_i . g
    // ga = G dL/dalpha (the opacity factor of G dL/dG = o G dL/dalpha is
    // applied to the sums in the flush), aT = alpha T
    float ga, aT;
    if constexpr (PLAIN) {
        // a lane that does not contribute runs the update with G = alpha = 0:
        // its rcp is 1 (T, Q unchanged) and its dL/dalpha is finite, so
        // every value below is zero for it without further selects
        const float Gs = ok ? G : 0.0f;
        const float as = ok ? alpha : 0.0f;
        const float rcp = __builtin_amdgcn_rcpf(1.0f - as);
        px.T = px.T * rcp;
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) cg = fmaf(comp4(fv[ch >> 2], ch & 3), px.gpix[ch], cg);
        const float dL_dalpha = fmaf(cg, px.T, -(px.Q * rcp));
        aT = as * px.T;
        px.Q = fmaf(aT, cg, px.Q);
        ga = Gs * dL_dalpha;
    } else {
        const float rcp = __builtin_amdgcn_rcpf(1.0f - alpha);
        px.T = ok ? px.T * rcp : px.T;
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) cg = fmaf(comp4(fv[ch >> 2], ch & 3), px.gpix[ch], cg);
        float dL_dalpha = fmaf(cg, px.T, -(px.Q * rcp));
        dL_dalpha = ok ? dL_dalpha : 0.0f;
        aT = ok ? alpha * px.T : 0.0f;
        px.Q = ok ? fmaf(aT, cg, px.Q) : px.Q;
        ga = G * dL_dalpha;
    }
    const float u = ga * dx, w = ga * dy;
    float v[NV];
    v[0] = u;
    v[1] = w;
    v[2] = u * dx;
    v[3] = u * dy;
    v[4] = w * dy;
    v[5] = ga;
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) v[6 + ch] = aT * px.gpix[ch];
#pragma unroll
    for (int q = 0; q < NV; ++q) out[S * q + O] = (PLAIN || ok) ? v[q] : 0.0f;
    return true;
}

// A Gaussian's slot in the wave's LDS sums, from its record offset.
template <int CH>
__device__ __forceinline__ float* slot_at(float4 (*part)[((CH + 6) + 3) / 4], int off) {
    constexpr int NV4 = ((CH + 6) + 3) / 4;
    return reinterpret_cast<float*>(reinterpret_cast<char*>(part) + off * NV4);
}

// Wave sums of one Gaussian's values into its slot: row r of the wave ends
// with the totals of values 4m + row_value(r), which lane 15 of the row
// stores at those positions.
template <int CH>
__device__ __forceinline__ void bwd_reduce1(const float (&v)[CH + 6], int off,
                                            float4 (*part)[((CH + 6) + 3) / 4], int lane) {
    constexpr int NV = CH + 6;
    constexpr int NVP = 4 * ((NV + 3) / 4);
    float w[NVP];
#pragma unroll
    for (int q = 0; q < NVP; ++q) w[q] = q < NV ? v[q] : 0.0f;
    float tot[NVP / 4];
    wave_reduce_rows<NVP, NV>(w, tot);
    if ((lane & 15) == 15) {
        float* dst = slot_at<CH>(part, off) + row_value(lane >> 4);
#pragma unroll
        for (int m = 0; m < NVP / 4; ++m) dst[4 * m] = tot[m];
    }
}

// The same for two different Gaussians in one reduction (fewer padding
// values and shared exchange steps): value i of Gaussian a sits at 2i and of
// Gaussian b at 2i + 1 of the combined array, so the first exchange pairs
// a's and b's value i; rows with row_value 0 and 2 then finish a's values
// 2m and 2m + 1, rows with 1 and 3 b's, each stored at slot position
// 2m + (row_value >> 1).
template <int CH>
__device__ __forceinline__ void bwd_reduce2(float (&w)[4 * ((CH + 7) / 2)], int oa, int ob,
                                            float4 (*part)[((CH + 6) + 3) / 4], int lane) {
    constexpr int NV = CH + 6;
    constexpr int NH = (NV + 1) / 2;  // value pairs per Gaussian
    static_assert(2 * NH <= 4 * ((NV + 3) / 4), "a Gaussian's slot holds its padded pairs");
    constexpr int K1 = NV;            // value pairs with a non-zero member (of 2 NH)
    constexpr int K2 = (K1 + 1) / 2;  // row groups with a non-zero member
    float h[2 * NH];
#pragma unroll
    for (int k = K1; k < 2 * NH; ++k) h[k] = 0.0f;
    reduce_step1<0, K1, 4 * NH, 2 * NV>(w, h);
    // step 2 (swap16-sum between rows) as in wave_reduce_rows: a[m] holds in
    // row r the row's partial of value 4m + row_value(r)
    float a[NH];
#pragma unroll
    for (int m = K2; m < NH; ++m) a[m] = 0.0f;
    reduce_step2<0, K2, 4 * NH>(h, a);
    // Step 3 within the row with halving exchanges.  A: row_mirror pairs
    // a[2j], a[2j + 1] (lanes 8..15 keep the second); B: row_half_mirror
    // pairs those results (lanes with bit 2 set keep the second); then two
    // quad steps.  Afterwards d[k] holds the total of a[4k + 2 bit2 + bit3],
    // bl (nb odd) that of a[2 (nb - 1) + bit3] and c (NH odd) that of
    // a[NH - 1]: 3 instructions per exchanged pair instead of 2 per value
    // and step.
    const int l = lane & 15;
    const bool hi8 = (l & 8) != 0, hi4 = (l & 4) != 0;
    constexpr int NB = NH / 2, ND = NB / 2;
    float b[NB + 1];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const float x = hi8 ? a[2 * j + 1] : a[2 * j];
        const float y = hi8 ? a[2 * j] : a[2 * j + 1];
        b[j] = x + dpp_f<0x140, 0xF, 0xF>(y);  // row_mirror
    }
    float c = 0.0f;
    if constexpr (NH % 2 == 1) {
        c = a[NH - 1];
        c += dpp_f<0x140, 0xF, 0xF>(c);
        c += dpp_f<0x141, 0xF, 0xF>(c);  // row_half_mirror
    }
    float d[ND + 1];
#pragma unroll
    for (int k = 0; k < ND; ++k) {
        const float x = hi4 ? b[2 * k + 1] : b[2 * k];
        const float y = hi4 ? b[2 * k] : b[2 * k + 1];
        d[k] = x + dpp_f<0x141, 0xF, 0xF>(y);  // row_half_mirror
    }
    float bl = 0.0f;
    if constexpr (NB % 2 == 1) {
        bl = b[NB - 1];
        bl += dpp_f<0x141, 0xF, 0xF>(bl);
    }
    auto quad_sum = [](float t) {
        t += dpp_f<0xB1, 0xF, 0xF>(t);  // quad_perm [1,0,3,2]
        t += dpp_f<0x4E, 0xF, 0xF>(t);  // quad_perm [2,3,0,1]
        return t;
    };
#pragma unroll
    for (int k = 0; k < ND; ++k) d[k] = quad_sum(d[k]);
    if constexpr (NB % 2 == 1) bl = quad_sum(bl);
    if constexpr (NH % 2 == 1) c = quad_sum(c);
    // the sums complete before the stores' lane branches (the compiler would
    // move the last add into them and lose its DPP form)
#pragma unroll
    for (int k = 0; k < ND; ++k) asm volatile("" ::"v"(d[k]));
    if constexpr (NB % 2 == 1) asm volatile("" ::"v"(bl));
    if constexpr (NH % 2 == 1) asm volatile("" ::"v"(c));
    const int rv = row_value(lane >> 4);
    float* dst = slot_at<CH>(part, (rv & 1) ? ob : oa) + (rv >> 1);
    const int sel = (hi4 ? 2 : 0) + (hi8 ? 1 : 0);
    if ((l & 3) == 3) {
#pragma unroll
        for (int k = 0; k < ND; ++k) dst[2 * (4 * k + sel)] = d[k];
    }
    if constexpr (NB % 2 == 1) {
        if ((l & 7) == 7) dst[2 * (2 * (NB - 1) + (hi8 ? 1 : 0))] = bl;
    }
    if constexpr (NH % 2 == 1) {
        if (l == 15) dst[2 * (NH - 1)] = c;
    }
}

// Back-to-front walk of one quadrant wave over its list (descending staged
// index), records and list entries read ahead as in fwd_walk, one
// reduction per contributing Gaussian.
template <int CH, bool PLAIN>
__device__ __forceinline__ void bwd_walk1(const uint32_t* list, int cnt, int lim,
                                          const float4* s_r0, const float4* s_r1,
                                          const float4 (*s_f)[(CH + 3) / 4],
                                          float4 (*part)[((CH + 6) + 3) / 4], float pxf,
                                          float pyf, int lane, BwdPixel<CH>& px) {
    constexpr int F4 = (CH + 3) / 4;
    const float4* sf = &s_f[0][0];
    if (cnt <= 0) return;
    int oa = list[0], ob = list[1];
    float4 a0 = rec_at(s_r0, oa), a1 = rec_at(s_r1, oa);
    for (int i = 0;; i += 2) {
        const int na = list[i + 2];
        const float4 b0 = rec_at(s_r0, ob), b1 = rec_at(s_r1, ob);
        {
            float v[CH + 6];
            if (bwd_values<CH, PLAIN>(a0, a1, &rec_at(sf, oa * F4), oa, lim, pxf, pyf, px, v))
                bwd_reduce1<CH>(v, oa, part, lane);
        }
        if (i + 1 >= cnt) return;
        const int nb = list[i + 3];
        a0 = rec_at(s_r0, na);
        a1 = rec_at(s_r1, na);
        {
            float v[CH + 6];
            if (bwd_values<CH, PLAIN>(b0, b1, &rec_at(sf, ob * F4), ob, lim, pxf, pyf, px, v))
                bwd_reduce1<CH>(v, ob, part, lane);
        }
        if (i + 2 >= cnt) return;
        oa = na;
        ob = nb;
    }
}

// The same walk two Gaussians at a time, the pair sharing one reduction (a
// Gaussian without contributions enters it as zeros): their values are
// written interleaved, a's at even and b's at odd positions, which is the
// layout bwd_reduce2 sums.  b's records are read before a is evaluated and
// the next a's before b is.  An odd count pairs the last Gaussian with the
// padding record, which contributes nothing and owns a slot of its own.
template <int CH, bool PLAIN>
__device__ __forceinline__ void bwd_walk2(const uint32_t* list, int cnt, int lim,
                                          const float4* s_r0, const float4* s_r1,
                                          const float4 (*s_f)[(CH + 3) / 4],
                                          float4 (*part)[((CH + 6) + 3) / 4], float pxf,
                                          float pyf, int lane, BwdPixel<CH>& px) {
    constexpr int F4 = (CH + 3) / 4;
    constexpr int NV = CH + 6;
    constexpr int NW = 4 * ((NV + 1) / 2);
    const float4* sf = &s_f[0][0];
    int oa = list[0], ob = list[1];
    float4 a0 = rec_at(s_r0, oa), a1 = rec_at(s_r1, oa);
    for (int i = 0; i < cnt; i += 2) {
        const int na = list[i + 2], nb = list[i + 3];
        const float4 b0 = rec_at(s_r0, ob), b1 = rec_at(s_r1, ob);
        float w[NW];
#pragma unroll
        for (int q = 2 * NV; q < NW; ++q) w[q] = 0.0f;
        const bool ha = bwd_values<CH, PLAIN, 2, 0>(a0, a1, &rec_at(sf, oa * F4), oa, lim, pxf,
                                                    pyf, px, w);
        a0 = rec_at(s_r0, na);
        a1 = rec_at(s_r1, na);
        const bool hb = bwd_values<CH, PLAIN, 2, 1>(b0, b1, &rec_at(sf, ob * F4), ob, lim, pxf,
                                                    pyf, px, w);
        if (ha || hb) bwd_reduce2<CH>(w, oa, ob, part, lane);
        oa = na;
        ob = nb;
    }
}

// Paired reductions up to four channels (at most 20 values per pair); wider
// channel blocks reduce one Gaussian at a time, where padding is a small
// share and two value sets would not fit the register budget.
template <int CH, bool PLAIN>
__device__ __forceinline__ void bwd_walk(const uint32_t* list, int cnt, int lim,
                                         const float4* s_r0, const float4* s_r1,
                                         const float4 (*s_f)[(CH + 3) / 4],
                                         float4 (*part)[((CH + 6) + 3) / 4], float pxf, float pyf,
                                         int lane, BwdPixel<CH>& px) {
    if constexpr (CH <= 4)
        bwd_walk2<CH, PLAIN>(list, cnt, lim, s_r0, s_r1, s_f, part, pxf, pyf, lane, px);
    else
        bwd_walk1<CH, PLAIN>(list, cnt, lim, s_r0, s_r1, s_f, part, pxf, pyf, lane, px);
}

// Waves per SIMD the backward asks for (more waves hide LDS and ballot
// latencies): six at one and three channels (<= 80 VGPRs, 12-16 KB of LDS),
// five at two and four channels (which would spill at 80), four up to 16
// channels, three at 32; no instantiation spills (checked with
// -Rpass-analysis=kernel-resource-usage: ScratchSize 0 for every one).
constexpr int bwd_min_waves(int ch) {
    return (ch == 2 || ch == 4) ? 5 : (ch <= 4 ? 6 : (ch <= 16 ? 4 : 3));
}

template <int CH>
__global__ __launch_bounds__(kThreads, bwd_min_waves(CH)) void k_raster_bwd(
    const float2* __restrict__ xy, const float4* __restrict__ co, const float* __restrict__ feat,
    int C, int c0, int nc, const int* __restrict__ ids, const int2* __restrict__ ranges,
    int64_t n, int64_t n_ids, const float* __restrict__ bg, int W, int H, int tiles_x,
    const float* __restrict__ final_T, const int* __restrict__ n_contrib,
    const float* __restrict__ grad_out, const float* __restrict__ grad_T,
    float* __restrict__ g_xy, float* __restrict__ g_conic, float* __restrict__ g_feat,
    float* __restrict__ g_opac, int gstride, const int* __restrict__ order) {
    constexpr int F4 = (CH + 3) / 4;
    constexpr int NV = CH + 6;             // u, w, u dx, u dy, w dy, opacity term, channels
    constexpr int NV4 = (NV + 3) / 4;
    // Gaussians per batch: 64 keeps the slot LDS at 16 KB up to four
    // channels (more workgroups per CU; measured faster than 128)
    constexpr int BB = 64;
    constexpr int NLW = BB / kWave;  // mask words per quadrant
    // entry BB of the records and slots is the walk lists' padding: a record
    // no pixel can take (alpha bound +inf) whose slot the flush never reads
    __shared__ float4 s_r0[BB + 1];
    __shared__ float4 s_r1[BB + 1];  // -a/2, -b, -c/2 (conic), Gaussian id (int bits)
    __shared__ float4 s_f[BB + 1][F4];
    __shared__ float4 s_part[kWaves][BB + 1][NV4];  // per-wave gradient sums per Gaussian
    __shared__ uint64_t s_mask[kWaves][NLW];
    __shared__ uint32_t s_list[kWaves][BB + 4];  // walk lists (+ look-ahead room)
    __shared__ int s_last[kWaves];
    // per wave: every Gaussian it staged is plain (written before the staging
    // barrier, read by all after it; the loop-top barrier orders batches)
    __shared__ __align__(16) uint32_t s_plain[kWaves];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = __builtin_amdgcn_readfirstlane(tile_at(order, blockIdx.x, gridDim.x, true));
    if (tile < 0) return;  // past the end of this XCD's band
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px0 = tx * kTile, py0 = ty * kTile;
    const int px = px0 + (wave & 1) * 8 + (lane & 7);
    const int py = py0 + (wave >> 1) * 8 + (lane >> 3);
    const bool inside = px < W && py < H;
    const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
    const int64_t pid = (int64_t)py * W + px;

    int start, num;
    tile_span(ranges[tile], n_ids, start, num);

    BwdPixel<CH> st;
    // the pixel's loads issue together (clamped indices, masked after)
    const int64_t pidc = inside ? pid : 0;
    const float tf = final_T[pidc];
    const int nct = n_contrib[pidc];
    float gp[CH], bgv[CH];
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) {
        gp[ch] = grad_out[pidc * C + c0 + min(ch, nc - 1)];
        bgv[ch] = bg ? bg[c0 + min(ch, nc - 1)] : 0.0f;
    }
    const float gt = grad_T ? grad_T[pidc] : 0.0f;
    const float T_final = inside ? tf : 1.0f;
    st.T = T_final;
    st.last = inside ? nct : 0;
    float bg_dot = 0.0f;
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) {
        st.gpix[ch] = (inside && ch < nc) ? gp[ch] : 0.0f;
        if (ch < nc) bg_dot = bg_dot + bgv[ch] * st.gpix[ch];
    }
    // The alpha output's cotangent enters once, with the first channel block.
    if (inside && c0 == 0 && grad_T) bg_dot = bg_dot + gt;
    st.Q = T_final * bg_dot;

    // the padding record (written before the barrier below)
    if (tid == 0) {
        s_r0[BB] = make_float4(0.0f, 0.0f, __builtin_huge_valf(), 0.0f);
        s_r1[BB] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int q = 0; q < F4; ++q) s_f[BB][q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }

    // Largest n_contrib of each quadrant: later list entries changed no pixel.
    {
        int m = st.last;
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

    for (int b = n_batches - 1; b >= 0; --b) {
        __syncthreads();
        uint32_t qm = 0;
        bool plain = true;
        if (tid < BB) {
            const int k = b * BB + tid;
            float4 r1 = make_float4(0.0f, 0.0f, 0.0f, __int_as_float(-1));
            if (k < num) {
                const int g = ids[start + k];
                if ((uint32_t)g < (uint64_t)n) {
                    // the record and feature loads issue together
                    const float2 m = xy[g];
                    const float4 c = co[g];
                    stage_features<CH>(s_f[tid], feat + (int64_t)g * C + c0, nc);
                    const float thr = alpha_floor_power(c.w);
                    s_r0[tid] = make_float4(m.x, m.y, thr, c.w);
                    r1 = make_float4(-0.5f * c.x, -c.y, -0.5f * c.z, __int_as_float(g));
                    qm = quadrant_mask(m.x, m.y, c, px0, py0);
#pragma unroll
                    for (int q = 0; q < kWaves; ++q)
                        if (k >= quad_last[q]) qm &= ~(1u << q);
                    plain = plain_gaussian<CH>(m.x, m.y, c, thr, s_f[tid]);
                }
            }
            s_r1[tid] = r1;
        }
        if (wave < NLW) {
#pragma unroll
            for (int q = 0; q < kWaves; ++q) {
                const uint64_t bq = __ballot((qm >> q) & 1u);
                if (lane == 0) s_mask[q][wave] = bq;
            }
        }
        const uint64_t np = __ballot(!plain);
        if (lane == 0) s_plain[wave] = np == 0ull;
        __syncthreads();
        const uint4 pl = *reinterpret_cast<const uint4*>(s_plain);
        const bool batch_plain = (pl.x & pl.y & pl.z & pl.w) != 0u;
        // the wave's slots start at zero: Gaussians it does not walk, or
        // whose sums it does not store, then add nothing in the flush
        {
            float4* p = &s_part[wave][0][0];
#pragma unroll
            for (int k = 0; k < BB * NV4 / kWave; ++k)
                p[k * kWave + lane] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        const int cnt = build_list<NLW, true>(s_mask[wave], s_list[wave], lane, BB * 16);
        const int lim = 16 * max(0, min(st.last - b * BB, BB));
        if (batch_plain)
            bwd_walk<CH, true>(s_list[wave], cnt, lim, s_r0, s_r1, s_f, s_part[wave], pxf, pyf,
                               lane, st);
        else
            bwd_walk<CH, false>(s_list[wave], cnt, lim, s_r0, s_r1, s_f, s_part[wave], pxf, pyf,
                                lane, st);
        __syncthreads();
        // 1. one thread per Gaussian adds the four waves' slots and turns the
        //    sums into the reference's gradient components, kept in its own
        //    wave-0 slot
        if (tid < BB) {
            float4 sum[NV4];
#pragma unroll
            for (int q = 0; q < NV4; ++q) sum[q] = s_part[0][tid][q];
            // one wave's slot at a time (all four in flight would need
            // 4 NV4 float4 registers)
#pragma unroll 1
            for (int w = 1; w < kWaves; ++w) {
#pragma unroll
                for (int q = 0; q < NV4; ++q) {
                    const float4 p = s_part[w][tid][q];
                    sum[q].x += p.x;
                    sum[q].y += p.y;
                    sum[q].z += p.z;
                    sum[q].w += p.w;
                }
            }
            float e[4 * NV4];
#pragma unroll
            for (int q = 0; q < NV4; ++q) {
                e[4 * q] = sum[q].x;
                e[4 * q + 1] = sum[q].y;
                e[4 * q + 2] = sum[q].z;
                e[4 * q + 3] = sum[q].w;
            }
            // rasterize.py:197-218 in terms of the sums (dL/dG = o dL/dalpha);
            // the staged conic is (-a/2, -b, -c/2)
            const float4 c = s_r1[tid];
            const float o = s_r0[tid].w;
            float* fin = reinterpret_cast<float*>(s_part[0][tid]);
            fin[0] = o * (2.0f * c.x * e[0] + c.y * e[1]);
            fin[1] = o * (c.y * e[0] + 2.0f * c.z * e[1]);
            fin[2] = -0.5f * o * e[2];
            fin[3] = -o * e[3];
            fin[4] = -0.5f * o * e[4];
#pragma unroll
            for (int q = 5; q < NV; ++q) fin[q] = e[q];
        }
        __syncthreads();
        // 2. the global atomics, component-major across the lanes: a wave's
        //    atomic instruction covers about 64 / NV Gaussians.  With a
        //    gradient record (gstride > 0) each Gaussian's components are
        //    adjacent words of one record; with separate arrays each
        //    Gaussian touches one cache line per array
        for (int item = tid; item < BB * NV; item += kThreads) {
            const int j = item / NV, k = item - j * NV;
            const int g = __float_as_int(s_r1[j].w);
            const float v = reinterpret_cast<const float*>(s_part[0][j])[k];
            if (g < 0 || v == 0.0f || (k >= 6 && k - 6 >= nc)) continue;
            float* dst = gstride > 0 ? g_xy + (int64_t)gstride * g + (k < 6 ? k : c0 + k)
                       : k < 2 ? g_xy + 2 * (int64_t)g + k
                       : k < 5 ? g_conic + 3 * (int64_t)g + (k - 2)
                       : k == 5 ? g_opac + g
                                : g_feat + (int64_t)g * C + c0 + (k - 6);
            atomicAdd(dst, v);
        }
    }
}

// ------------------------------------------------- matrix-core backward --
// The backward for wide channel blocks (CH = 32) with its channel work on
// the matrix cores.  Per (Gaussian, pixel) pair the replay is the same VALU
// arithmetic as bwd_values -- every alpha / T / early-stop decision and the
// per-pixel running state are unchanged -- except that the two channel
// contractions come from v_mfma_f32_16x16x4_f32 products over groups of 16
// list entries:
//   A. cg[g][p] = sum_c f[g][c] g[p][c], (16 x 32) x (32 x 64), before the
//      group's replay (the features are staged; the pixels' cotangents are
//      held in registers in the B-operand layout for the whole walk), and
//   B. dL/dc[g][c] = sum over the wave's 64 pixels of aT[g][p] g[p][c],
//      (16 x 64) x (64 x 32), after it (aT = alpha T of each pair).
// One LDS tile per wave carries cg[g][p] to the replay, which overwrites
// entry (g, p) with aT[g][p] once read.  The replay itself produces only
// the six geometric values (u, w, u dx, u dy, w dy, G dL/dalpha), reduced
// across the wave as before.  Operand layouts (checked on the GPU):
// A[row = l % 16][k = l / 16], B[k = l / 16][col = l % 16]; the result's lane
// l holds rows 4 (l / 16) + i, column l % 16.  The features are staged
// channel-major (row stride 65) and the tile with row stride 68, so the
// operand reads and result writes of a wave hit distinct LDS banks.  The
// geometric sums of the four quadrant waves meet in one LDS slot per
// Gaussian through LDS float atomics (three per pair); product B's channel
// sums go straight to the gradient record with global float atomics, one
// instruction covering four Gaussians' 16 consecutive channels -- LDS
// float atomics for them (eight per group and lane) cost more than the
// whole global flush, and per-wave LDS slots instead (34 KB) cut the
// workgroups per CU from three to two, slower still.  The contractions add
// in a different order than the VALU path, so gradients agree with it to
// float32 rounding, not bitwise; no decision depends on them.
constexpr int kMxGroup = 16;   // Gaussians per matrix-core group
constexpr int kMxPad = 68;     // row stride (floats) of a wave's tile: 4 r + q bank spread
constexpr int kMxFPad = 65;    // row stride (floats) of the channel-major features
constexpr int kMxGeo = 6;      // geometric values per Gaussian
constexpr int kMxGeoStride = 8;   // slot stride (floats) of the geometric sums

// Where a Gaussian's feature gradients go: base + stride * id + offset + c
// for channels c < nc of the block.
struct MxFeatOut {
    float* base;
    int64_t stride;
    int offset;
    int nc;
};

typedef float mx_floatx4 __attribute__((ext_vector_type(4)));

struct MxPixel {
    float T;  // transmittance in front of the current Gaussian
    float Q;
    int last;
};

// The replay of one (pixel, Gaussian) pair given cg = c . g: the geometric
// values into v (zeros where the pixel does not composite the Gaussian) and
// alpha T into aT (zero likewise).  Returns whether any lane of the wave
// passes the first tests (v and aT are zero when it does not).
template <bool PLAIN>
__device__ __forceinline__ bool bwd_geo(const float4& r0, const float4& r1, float cg, int off,
                                        int lim, float pxf, float pyf, MxPixel& px,
                                        float (&v)[8], float& aT_out) {
    const float dx = r0.x - pxf, dy = r0.y - pyf;
    const float power = splat_power(r1.x, r1.y, r1.z, dx, dy);
    // PLAIN: the power is never positive (plain_gaussian's conic bound)
    const bool c1 = off < lim, c2 = PLAIN || !(power > 0.0f), c3 = !(power < r0.z);
    bool ok = c1 && c2 && c3;
    const uint64_t m123 = PLAIN ? __ballot(c1) & __ballot(c3)
                                : __ballot(c1) & __ballot(c2) & __ballot(c3);
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = 0.0f;
    aT_out = 0.0f;
    if (m123 == 0ull) return false;
    const float G = PLAIN ? splat_exp_core(power) : splat_exp_sel(power);
    const float alpha = fminf(0.99f, r0.w * G);
    const bool c4 = !(alpha < 1.0f / 255.0f);
    ok = ok && c4;
    if ((m123 & __ballot(c4)) == 0ull) return false;
    float ga, aT;
    if constexpr (PLAIN) {
        const float Gs = ok ? G : 0.0f;
        const float as = ok ? alpha : 0.0f;
        const float rcp = __builtin_amdgcn_rcpf(1.0f - as);
        px.T = px.T * rcp;
        const float dL_dalpha = fmaf(cg, px.T, -(px.Q * rcp));
        aT = as * px.T;
        px.Q = fmaf(aT, cg, px.Q);
        ga = Gs * dL_dalpha;
    } else {
        const float rcp = __builtin_amdgcn_rcpf(1.0f - alpha);
        px.T = ok ? px.T * rcp : px.T;
        float dL_dalpha = fmaf(cg, px.T, -(px.Q * rcp));
        dL_dalpha = ok ? dL_dalpha : 0.0f;
        aT = ok ? alpha * px.T : 0.0f;
        px.Q = ok ? fmaf(aT, cg, px.Q) : px.Q;
        ga = G * dL_dalpha;
    }
    const float u = ga * dx, w = ga * dy;
    v[0] = (PLAIN || ok) ? u : 0.0f;
    v[1] = (PLAIN || ok) ? w : 0.0f;
    v[2] = (PLAIN || ok) ? u * dx : 0.0f;
    v[3] = (PLAIN || ok) ? u * dy : 0.0f;
    v[4] = (PLAIN || ok) ? w * dy : 0.0f;
    v[5] = (PLAIN || ok) ? ga : 0.0f;
    aT_out = aT;  // zero for lanes that do not composite (PLAIN: as = 0)
    return true;
}

// The walk of one quadrant wave for the matrix-core backward: groups of up
// to 16 list entries (back to front): product A into the tile, the replay
// pair by pair, product B into the Gaussians' LDS slots.  gA[pb][ks] =
// g(pixel 16 pb + l % 16, channel 4 ks + l / 16); gB[ks][cb] = g(pixel
// 4 ks + l / 16, channel 16 cb + l % 16).
template <bool PLAIN>
__device__ __forceinline__ void bwd_walk_mx(const uint32_t* list, int cnt, int lim,
                                            const float4* s_r0, const float4* s_r1,
                                            const float* s_feat, int pad_slot,
                                            float (*sum)[kMxGeoStride], const MxFeatOut& fo,
                                            float (*tile)[kMxPad],
                                            const float (&gA)[4][8], const float (&gB)[16][2],
                                            float pxf, float pyf, int lane, MxPixel& px) {
#pragma unroll 1
    for (int i0 = 0; i0 < cnt; i0 += kMxGroup) {
        const int ng = min(kMxGroup, cnt - i0);
        // A: the features of entry l % 16 (the padding record's zeros past
        // the group), channels 4 ks + l / 16
        const int row = lane & 15;
        const int slot = row < ng ? (list[i0 + row] >> 4) : pad_slot;
        float fa[8];
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) fa[ks] = s_feat[(4 * ks + (lane >> 4)) * kMxFPad + slot];
#pragma unroll
        for (int pb = 0; pb < 4; ++pb) {
            mx_floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[ks], gA[pb][ks], acc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) tile[4 * (lane >> 4) + i][16 * pb + row] = acc[i];
        }
        // the wave's LDS accesses complete in order; the fence keeps the
        // compiler from moving the reads below above the writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        // the replay two entries at a time (a = j, b = j + 1; past the group
        // the padding record, which contributes nothing), their geometric
        // values interleaved (a's at even, b's at odd positions) into one
        // reduction, the next pair's records read before this pair is
        // evaluated
        const int pad = pad_slot * 16;
        int oa = 0 < ng ? list[i0] : pad, ob = 1 < ng ? list[i0 + 1] : pad;
        float4 a0 = rec_at(s_r0, oa), a1 = rec_at(s_r1, oa);
        float4 b0 = rec_at(s_r0, ob), b1 = rec_at(s_r1, ob);
        float cga = tile[0][lane], cgb = tile[1][lane];
#pragma unroll 1
        for (int j = 0; j < kMxGroup; j += 2) {
            const int na = j + 2 < ng ? list[i0 + j + 2] : pad;
            const int nb = j + 3 < ng ? list[i0 + j + 3] : pad;
            // the next pair's rows are not overwritten before they are read
            const float nca = j + 2 < kMxGroup ? tile[j + 2][lane] : 0.0f;
            const float ncb = j + 3 < kMxGroup ? tile[j + 3][lane] : 0.0f;
            float va[8], vb[8], aTa, aTb;
            const bool ha = bwd_geo<PLAIN>(a0, a1, cga, oa, lim, pxf, pyf, px, va, aTa);
            const bool hb = bwd_geo<PLAIN>(b0, b1, cgb, ob, lim, pxf, pyf, px, vb, aTb);
            tile[j][lane] = aTa;
            tile[j + 1][lane] = aTb;
            a0 = rec_at(s_r0, na);
            a1 = rec_at(s_r1, na);
            b0 = rec_at(s_r0, nb);
            b1 = rec_at(s_r1, nb);
            if (ha || hb) {
                float w[12], h[6], q[3];
#pragma unroll
                for (int k = 0; k < kMxGeo; ++k) {
                    w[2 * k] = va[k];
                    w[2 * k + 1] = vb[k];
                }
                reduce_step1<0, 6, 12, 12>(w, h);
                reduce_step2<0, 3, 12>(h, q);
                // within the row: q[0], q[1] exchanged by halving over
                // row_mirror (lanes 8..15 keep q[1]), q[2] summed whole;
                // rows with row_value 0 and 2 hold a's values 2m and 2m + 1,
                // rows with 1 and 3 b's
                const bool hi8 = (lane & 8) != 0;
                const float x = hi8 ? q[1] : q[0], y = hi8 ? q[0] : q[1];
                float b = x + dpp_f<0x140, 0xF, 0xF>(y);  // row_mirror
                float c = q[2] + dpp_f<0x140, 0xF, 0xF>(q[2]);
                b += dpp_f<0x141, 0xF, 0xF>(b);  // row_half_mirror
                c += dpp_f<0x141, 0xF, 0xF>(c);
                b += dpp_f<0xB1, 0xF, 0xF>(b);  // quad_perm [1,0,3,2]
                c += dpp_f<0xB1, 0xF, 0xF>(c);
                b += dpp_f<0x4E, 0xF, 0xF>(b);  // quad_perm [2,3,0,1]
                c += dpp_f<0x4E, 0xF, 0xF>(c);
                asm volatile("" ::"v"(b), "v"(c));
                const int rv = row_value(lane >> 4);
                float* dst = sum[((rv & 1) ? ob : oa) >> 4] + (rv >> 1);
                if ((lane & 7) == 7) atomicAdd(dst + (hi8 ? 2 : 0), b);
                if ((lane & 15) == 15) atomicAdd(dst + 4, c);
            }
            oa = na;
            ob = nb;
            cga = nca;
            cgb = ncb;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        mx_floatx4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
            const float a = tile[row][4 * ks + (lane >> 4)];
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, gB[ks][0], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, gB[ks][1], acc1, 0, 0, 0);
        }
        // lane l holds the sums of entries 4 (l / 16) + i, channels l % 16
        // and 16 + l % 16: added straight into the Gaussians' feature
        // gradients (one instruction covers four Gaussians' 16 consecutive
        // channels; zero sums are skipped)
        const uint4 gl = *reinterpret_cast<const uint4*>(list + i0 + 4 * (lane >> 4));
        const uint32_t gi[4] = {gl.x, gl.y, gl.z, gl.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = 4 * (lane >> 4) + i;
            if (g < ng) {
                const int gid = __float_as_int(s_r1[gi[i] >> 4].w);
                float* dst = fo.base + (int64_t)fo.stride * gid + fo.offset + row;
                if (acc0[i] != 0.0f && row < fo.nc) atomicAdd(dst, acc0[i]);
                if (acc1[i] != 0.0f && row + 16 < fo.nc) atomicAdd(dst + 16, acc1[i]);
            }
        }
        // the next group's product A overwrites the tile
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    }
}

template <int CH>
__global__ __launch_bounds__(kThreads, 3) void k_raster_bwd_mx(
    const float2* __restrict__ xy, const float4* __restrict__ co, const float* __restrict__ feat,
    int C, int c0, int nc, const int* __restrict__ ids, const int2* __restrict__ ranges,
    int64_t n, int64_t n_ids, const float* __restrict__ bg, int W, int H, int tiles_x,
    const float* __restrict__ final_T, const int* __restrict__ n_contrib,
    const float* __restrict__ grad_out, const float* __restrict__ grad_T,
    float* __restrict__ g_xy, float* __restrict__ g_conic, float* __restrict__ g_feat,
    float* __restrict__ g_opac, int gstride, const int* __restrict__ order) {
    static_assert(CH == 32, "the matrix-core backward covers 32-channel blocks");
    constexpr int F4 = CH / 4;
    constexpr int BB = 64;
    constexpr int NLW = BB / kWave;
    __shared__ float4 s_r0[BB + 1];
    __shared__ float4 s_r1[BB + 1];  // -a/2, -b, -c/2 (conic), Gaussian id (int bits)
    __shared__ float s_fT[CH * kMxFPad];              // features, channel-major (column BB: zeros)
    __shared__ float s_sum[BB + 1][kMxGeoStride];     // geometric sums over the waves
    __shared__ float s_tile[kWaves][kMxGroup][kMxPad];  // per-wave cg / aT tiles
    __shared__ uint64_t s_mask[kWaves][NLW];
    // walk lists; a group's 16 entries are read as four 16-byte pieces, so
    // each row has room for a whole group past the last entry
    __shared__ __align__(16) uint32_t s_list[kWaves][BB + kMxGroup];
    __shared__ int s_last[kWaves];
    __shared__ __align__(16) uint32_t s_plain[kWaves];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = __builtin_amdgcn_readfirstlane(tile_at(order, blockIdx.x, gridDim.x, true));
    if (tile < 0) return;  // past the end of this XCD's band
    // rows of CH channels at 16-byte aligned addresses: float4 loads
    const bool vec4 = nc >= CH && ((C | c0) & 3) == 0 && ((uintptr_t)feat & 15u) == 0;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px0 = tx * kTile, py0 = ty * kTile;
    const int qx0 = px0 + (wave & 1) * 8, qy0 = py0 + (wave >> 1) * 8;
    const int px = qx0 + (lane & 7);
    const int py = qy0 + (lane >> 3);
    const bool inside = px < W && py < H;
    const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
    const int64_t pid = (int64_t)py * W + px;

    int start, num;
    tile_span(ranges[tile], n_ids, start, num);

    MxPixel st;
    // the pixel's loads issue together (clamped indices, masked after)
    const int64_t pidc = inside ? pid : 0;
    const float tf = final_T[pidc];
    const int nct = n_contrib[pidc];
    const float gt = grad_T ? grad_T[pidc] : 0.0f;
    const float T_final = inside ? tf : 1.0f;
    st.T = T_final;
    st.last = inside ? nct : 0;
    float bg_dot = 0.0f;
    {
        float gp[CH], bgv[CH];
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
            gp[ch] = grad_out[pidc * C + c0 + min(ch, nc - 1)];
            bgv[ch] = bg ? bg[c0 + min(ch, nc - 1)] : 0.0f;
        }
#pragma unroll
        for (int ch = 0; ch < CH; ++ch)
            if (ch < nc) bg_dot = bg_dot + bgv[ch] * (inside ? gp[ch] : 0.0f);
    }
    if (inside && c0 == 0 && grad_T) bg_dot = bg_dot + gt;
    st.Q = T_final * bg_dot;
    // the quadrant's cotangents in the two B-operand layouts (pixel q of
    // the quadrant is (q % 8, q / 8))
    auto gval = [&](int q, int ch) {
        const int bx = qx0 + (q & 7), by = qy0 + (q >> 3);
        return (bx < W && by < H && ch < nc) ? grad_out[((int64_t)by * W + bx) * C + c0 + ch]
                                             : 0.0f;
    };
    float gA[4][8], gB[16][2];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) gA[pb][ks] = gval(16 * pb + (lane & 15), 4 * ks + (lane >> 4));
#pragma unroll
    for (int ks = 0; ks < 16; ++ks)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) gB[ks][cb] = gval(4 * ks + (lane >> 4), 16 * cb + (lane & 15));

    if (tid == 0) {
        s_r0[BB] = make_float4(0.0f, 0.0f, __builtin_huge_valf(), 0.0f);
        s_r1[BB] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if (tid < CH) s_fT[tid * kMxFPad + BB] = 0.0f;
    {
        int m = st.last;
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
    const MxFeatOut fout = gstride > 0 ? MxFeatOut{g_xy, gstride, kMxGeo + c0, nc}
                                       : MxFeatOut{g_feat, C, c0, nc};

    for (int b = n_batches - 1; b >= 0; --b) {
        __syncthreads();
        uint32_t qm = 0;
        bool plain = true;
        for (int k = tid; k < (BB + 1) * kMxGeoStride; k += kThreads) (&s_sum[0][0])[k] = 0.0f;
        if (tid < BB) {
            const int k = b * BB + tid;
            float4 r1 = make_float4(0.0f, 0.0f, 0.0f, __int_as_float(-1));
            if (k < num) {
                const int g = ids[start + k];
                if ((uint32_t)g < (uint64_t)n) {
                    const float2 m = xy[g];
                    const float4 c = co[g];
                    const float thr = alpha_floor_power(c.w);
                    s_r0[tid] = make_float4(m.x, m.y, thr, c.w);
                    r1 = make_float4(-0.5f * c.x, -c.y, -0.5f * c.z, __int_as_float(g));
                    qm = quadrant_mask(m.x, m.y, c, px0, py0);
#pragma unroll
                    for (int q = 0; q < kWaves; ++q)
                        if (k >= quad_last[q]) qm &= ~(1u << q);
                    plain = plain_gaussian<0>(m.x, m.y, c, thr, nullptr);
                }
            }
            s_r1[tid] = r1;
        }
        if (wave < NLW) {
#pragma unroll
            for (int q = 0; q < kWaves; ++q) {
                const uint64_t bq = __ballot((qm >> q) & 1u);
                if (lane == 0) s_mask[q][wave] = bq;
            }
        }
        // the features: every thread stages two of the batch's float4
        // pieces (the ids come from the records above), so no thread holds a
        // Gaussian's 32 channels beside the walk's cotangent registers
        __syncthreads();
        if (vec4) {
            // whole aligned rows: the 16-byte loads issue together (entries
            // without a Gaussian read row 0 and are dropped)
            constexpr int NIT = BB * F4 / kThreads;
            static_assert(BB * F4 % kThreads == 0, "whole rounds");
            int g[NIT];
            float4 v[NIT];
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int k = tid + it * kThreads, j = k / F4, q = k - j * F4;
                g[it] = __float_as_int(s_r1[j].w);
                const int64_t gi = g[it] >= 0 ? g[it] : 0;
                v[it] = *reinterpret_cast<const float4*>(feat + gi * C + c0 + 4 * q);
            }
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int k = tid + it * kThreads, j = k / F4, q = k - j * F4;
                if (g[it] >= 0) {
                    float* d = s_fT + (4 * q) * kMxFPad + j;
                    d[0] = v[it].x;
                    d[kMxFPad] = v[it].y;
                    d[2 * kMxFPad] = v[it].z;
                    d[3 * kMxFPad] = v[it].w;
                    plain = plain && fabsf(v[it].x) < 1e30f && fabsf(v[it].y) < 1e30f &&
                            fabsf(v[it].z) < 1e30f && fabsf(v[it].w) < 1e30f;
                }
            }
        } else
        for (int k = tid; k < BB * F4; k += kThreads) {
            const int j = k / F4, q = k - j * F4;
            const int g = __float_as_int(s_r1[j].w);
            if (g >= 0) {
                const float* f = feat + (int64_t)g * C + c0 + 4 * q;
                float4 v;
                v.x = 4 * q < nc ? f[0] : 0.0f;
                v.y = 4 * q + 1 < nc ? f[1] : 0.0f;
                v.z = 4 * q + 2 < nc ? f[2] : 0.0f;
                v.w = 4 * q + 3 < nc ? f[3] : 0.0f;
                float* d = s_fT + (4 * q) * kMxFPad + j;
                d[0] = v.x;
                d[kMxFPad] = v.y;
                d[2 * kMxFPad] = v.z;
                d[3 * kMxFPad] = v.w;
                plain = plain && fabsf(v.x) < 1e30f && fabsf(v.y) < 1e30f &&
                        fabsf(v.z) < 1e30f && fabsf(v.w) < 1e30f;
            }
        }
        const uint64_t np = __ballot(!plain);
        if (lane == 0) s_plain[wave] = np == 0ull;
        __syncthreads();
        const uint4 pl = *reinterpret_cast<const uint4*>(s_plain);
        const bool batch_plain = (pl.x & pl.y & pl.z & pl.w) != 0u;
        const int cnt = build_list<NLW, true>(s_mask[wave], s_list[wave], lane, BB * 16);
        const int lim = 16 * max(0, min(st.last - b * BB, BB));
        const float* sfeat = s_fT;
        if (batch_plain)
            bwd_walk_mx<true>(s_list[wave], cnt, lim, s_r0, s_r1, sfeat, BB, s_sum, fout,
                              s_tile[wave], gA, gB, pxf, pyf, lane, st);
        else
            bwd_walk_mx<false>(s_list[wave], cnt, lim, s_r0, s_r1, sfeat, BB, s_sum, fout,
                               s_tile[wave], gA, gB, pxf, pyf, lane, st);
        __syncthreads();
        // one thread per Gaussian turns the sums into the reference's
        // gradient components (rasterize.py:197-218 in terms of the sums)
        if (tid < BB) {
            float* e = s_sum[tid];
            const float4 c = s_r1[tid];
            const float o = s_r0[tid].w;
            const float e0 = e[0], e1 = e[1];
            e[0] = o * (2.0f * c.x * e0 + c.y * e1);
            e[1] = o * (c.y * e0 + 2.0f * c.z * e1);
            e[2] = -0.5f * o * e[2];
            e[3] = -o * e[3];
            e[4] = -0.5f * o * e[4];
        }
        __syncthreads();
        for (int item = tid; item < BB * kMxGeo; item += kThreads) {
            const int j = item / kMxGeo, k = item - j * kMxGeo;
            const int g = __float_as_int(s_r1[j].w);
            const float v = s_sum[j][k];
            if (g < 0 || v == 0.0f) continue;
            float* dst = gstride > 0 ? g_xy + (int64_t)gstride * g + k
                       : k < 2 ? g_xy + 2 * (int64_t)g + k
                       : k < 5 ? g_conic + 3 * (int64_t)g + (k - 2)
                                : g_opac + g;
            atomicAdd(dst, v);
        }
    }
}

// Matrix-core forward for 32-channel blocks.  The per-pixel loop keeps every
// decision of fwd_pair on the vector ALU (power, exp, alpha, the early stop,
// T, depth, the last contributor), so final_T, n_contrib, alpha and depth
// are the VALU path's bits; only the channel sums move.  For a group of 16
// list entries the replay writes each pair's weight w = alpha T (zero where
// the pixel does not composite) into a per-wave LDS tile, then
//   out[c][p] += sum over the group of f[g][c] w[g][p]
// runs as 32 v_mfma_f32_16x16x4_f32 (A = features, 16 channels x 4 entries;
// B = weights, 4 entries x 16 pixels; 2 channel blocks x 4 pixel blocks of
// accumulators).  Lane l holds channels 16 cb + 4 (l / 16) + i of quadrant
// pixel 16 pb + l % 16.  The features are staged row-major with a row
// stride of 48 floats (rows four slots apart share no bank window) and the
// tile with a row stride of 80 (the four rows one operand read touches hit
// disjoint banks).  The sums add in another order than the sequential
// multiply-adds of fwd_pair: channels agree with it to float32 rounding.
// Batches holding a non-finite (or |f| >= 1e30) feature add their groups on
// the vector ALU into the same accumulators, pair by pair in list order and
// only where w != 0, so 0 * inf never reaches a pixel that skipped the
// Gaussian.
constexpr int kMfBatch = 128;  // list entries staged per batch
constexpr int kMfFeat = 48;    // feature row stride (floats)
constexpr int kMfTile = 80;    // weight tile row stride (floats)

// One (pixel, Gaussian) step of fwd_pair without the channel sums: returns
// the weight the pixel gives the Gaussian (zero unless it composites).
template <bool DEPTH, bool PLAIN>
__device__ __forceinline__ float fwd_weight(const float4& r0, const float4& r1, int off,
                                            float pxf, float pyf, float& T, float& dacc,
                                            int& last_off, uint64_t& alive) {
    const float dx = r0.x - pxf, dy = r0.y - pyf;
    const float power = splat_power(r1.x, r1.y, r1.z, dx, dy);
    const uint64_t live =
        PLAIN ? alive & __ballot(!(power < r0.z))
              : alive & __ballot(!(power > 0.0f)) & __ballot(!(power < r0.z));
    const float e = PLAIN ? splat_exp_core(power) : splat_exp_sel(power);
    const float alpha = fminf(0.99f, r0.w * e);
    const uint64_t pass = live & __ballot(!(alpha < 1.0f / 255.0f));
    const float next_T = T * (1.0f - alpha);
    const uint64_t lt = __ballot(next_T < 1e-4f);
    alive &= ~(pass & lt);
    const bool add = __builtin_amdgcn_inverse_ballot_w64(pass & ~lt);
    const float w = alpha * T;
    const float wa = add ? w : 0.0f;
    if (DEPTH) {
        if (PLAIN) {
            dacc = fmaf(r1.w, wa, dacc);
        } else {
            const float d2 = fmaf(r1.w, w, dacc);
            dacc = add ? d2 : dacc;
        }
    }
    T = add ? next_T : T;
    last_off = add ? off : last_off;
    return wa;
}

// The walk of one quadrant wave for the matrix-core forward, in groups of
// 16 list entries: the replay (two entries per round, the next pair's
// records read before this pair is evaluated) fills the weight tile; rows
// past the entries replayed (the group's end, or the wave's early stop)
// are zero.  FINITE: every staged feature is finite and below 1e30.
template <bool DEPTH, bool PLAIN, bool FINITE>
__device__ __forceinline__ void fwd_walk_mx(const uint32_t* list, int cnt, const float4* s_r0,
                                            const float4* s_r1, const float* s_feat,
                                            int pad_slot, float (*tile)[kMfTile], float pxf,
                                            float pyf, int lane, float& T, float& dacc,
                                            int& last_off, uint64_t& alive,
                                            mx_floatx4 (&acc)[2][4]) {
    const int pad = pad_slot * 16;
    const int row = lane & 15, kq = lane >> 4;
#pragma unroll 1
    for (int i0 = 0; i0 < cnt; i0 += kMxGroup) {
        const int ng = min(kMxGroup, cnt - i0);
        int oa = list[i0], ob = 1 < ng ? list[i0 + 1] : pad;
        float4 a0 = rec_at(s_r0, oa), a1 = rec_at(s_r1, oa);
        int j = 0;
#pragma unroll 1
        while (j < ng) {
            const int na = j + 2 < ng ? list[i0 + j + 2] : pad;
            const int nb = j + 3 < ng ? list[i0 + j + 3] : pad;
            const float4 b0 = rec_at(s_r0, ob), b1 = rec_at(s_r1, ob);
            tile[j][lane] =
                fwd_weight<DEPTH, PLAIN>(a0, a1, oa, pxf, pyf, T, dacc, last_off, alive);
            a0 = rec_at(s_r0, na);
            a1 = rec_at(s_r1, na);
            tile[j + 1][lane] =
                fwd_weight<DEPTH, PLAIN>(b0, b1, ob, pxf, pyf, T, dacc, last_off, alive);
            oa = na;
            ob = nb;
            j += 2;
            if (alive == 0ull) break;
        }
#pragma unroll 1
        for (; j < kMxGroup; ++j) tile[j][lane] = 0.0f;
        // the wave's LDS accesses complete in order; the fence keeps the
        // compiler from moving the reads below above the writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        if constexpr (FINITE) {
#pragma unroll 1
            for (int ks = 0; ks < 4; ++ks) {
                const int r = 4 * ks + kq;
                const int slot = r < ng ? (list[i0 + r] >> 4) : pad_slot;
                const float fa0 = s_feat[slot * kMfFeat + row];
                const float fa1 = s_feat[slot * kMfFeat + 16 + row];
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) {
                    const float wb = tile[r][16 * pb + row];
                    acc[0][pb] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa0, wb, acc[0][pb], 0, 0, 0);
                    acc[1][pb] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa1, wb, acc[1][pb], 0, 0, 0);
                }
            }
        } else {
#pragma unroll 1
            for (int r = 0; r < ng; ++r) {
                const int slot = list[i0 + r] >> 4;
                float wv[4];
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) wv[pb] = tile[r][16 * pb + row];
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    const float4 f =
                        *reinterpret_cast<const float4*>(s_feat + slot * kMfFeat + 16 * cb + 4 * kq);
#pragma unroll
                    for (int pb = 0; pb < 4; ++pb) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float v = fmaf(comp4(f, i), wv[pb], acc[cb][pb][i]);
                            acc[cb][pb][i] = wv[pb] != 0.0f ? v : acc[cb][pb][i];
                        }
                    }
                }
            }
        }
        // the next group's replay overwrites the tile
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        if (alive == 0ull) return;
    }
}

template <bool DEPTH>
__global__ __launch_bounds__(kThreads, 3) void k_raster_fwd_mx(
    const float2* __restrict__ xy, const float4* __restrict__ co, const float* __restrict__ feat,
    int C, int c0, int nc, const float* __restrict__ depths, const int* __restrict__ ids,
    const int2* __restrict__ ranges, int64_t n, int64_t n_ids, const float* __restrict__ bg,
    int W, int H, int tiles_x, float* __restrict__ out, float* __restrict__ final_T,
    int* __restrict__ n_contrib, float* __restrict__ depth_out, float* __restrict__ alpha_out,
    const int* __restrict__ order, int* __restrict__ work) {
    constexpr int BB = kMfBatch;
    constexpr int NLW = BB / kWave;  // waves that stage records
    constexpr int F4 = 8;            // float4 pieces of a 32-channel row
    // entry BB of the records (and feature row BB, zeros) is the padding
    __shared__ float4 s_r0[BB + 1];  // mean x, mean y, log-alpha bound, opacity
    __shared__ float4 s_r1[BB + 1];  // -a/2, -b, -c/2 (conic), depth
    __shared__ __align__(16) float s_feat[(BB + 1) * kMfFeat];
    __shared__ float s_tile[kWaves][kMxGroup][kMfTile];
    __shared__ uint64_t s_mask[kWaves][NLW];
    __shared__ uint32_t s_list[kWaves][BB + 4];
    __shared__ __align__(16) uint32_t s_alive[kWaves];
    __shared__ __align__(16) uint32_t s_plain[kWaves];
    __shared__ __align__(16) uint32_t s_finite[kWaves];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = __builtin_amdgcn_readfirstlane(tile_at(order, blockIdx.x, gridDim.x, false));
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px0 = tx * kTile, py0 = ty * kTile;
    const int qx0 = px0 + (wave & 1) * 8, qy0 = py0 + (wave >> 1) * 8;
    const int px = qx0 + (lane & 7);
    const int py = qy0 + (lane >> 3);
    const bool inside = px < W && py < H;
    const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;

    int start, num;
    tile_span(ranges[tile], n_ids, start, num);

    float T = 1.0f, dacc = 0.0f;
    mx_floatx4 acc[2][4];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int pb = 0; pb < 4; ++pb) acc[cb][pb] = mx_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    int last = 0;
    uint64_t alive = __ballot(inside);
    if (tid == 0) {
        s_r0[BB] = make_float4(0.0f, 0.0f, __builtin_huge_valf(), 0.0f);
        s_r1[BB] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if (tid < kMfFeat) s_feat[BB * kMfFeat + tid] = 0.0f;
    // rows of 32 channels at 16-byte aligned addresses: float4 loads
    const bool vec4 = nc >= 4 * F4 && ((C | c0) & 3) == 0 && ((uintptr_t)feat & 15u) == 0;

    for (int base = 0; base < num; base += BB) {
        if (lane == 0) s_alive[wave] = alive != 0ull;
        __syncthreads();
        const uint4 al = *reinterpret_cast<const uint4*>(s_alive);
        if ((al.x | al.y | al.z | al.w) == 0u) break;  // all 256 pixels done
        uint32_t qm = 0;
        bool plain = true, finite = true;
        if (tid < BB) {
            const int k = base + tid;
            if (k < num) {
                const int g = ids[start + k];
                if ((uint32_t)g < (uint64_t)n) {
                    const float2 m = xy[g];
                    const float4 c = co[g];
                    const float thr = alpha_floor_power(c.w);
                    s_r0[tid] = make_float4(m.x, m.y, thr, c.w);
                    const float dz = DEPTH ? depths[g] : 0.0f;
                    s_r1[tid] = make_float4(-0.5f * c.x, -c.y, -0.5f * c.z, dz);
                    qm = quadrant_mask(m.x, m.y, c, px0, py0);
                    plain = plain_gaussian<0>(m.x, m.y, c, thr, nullptr) && fabsf(dz) < 1e30f;
                }
            }
        }
        // the features: thread t stages piece t % 8 of entries t / 8 + 32 i
        constexpr int NIT = BB * F4 / kThreads;
        if (vec4) {
            // whole aligned rows: the id loads, then the 16-byte feature
            // loads, each issued together (invalid entries read row 0 and
            // are dropped)
            int g[NIT];
            float4 v[NIT];
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int k = base + (tid >> 3) + (kThreads / F4) * it;
                g[it] = ids[start + min(k, num - 1)];
                if (k >= num) g[it] = -1;
            }
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int64_t gi = (uint32_t)g[it] < (uint64_t)n ? g[it] : 0;
                v[it] = *reinterpret_cast<const float4*>(feat + gi * C + c0 + 4 * (tid & 7));
            }
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                if ((uint32_t)g[it] < (uint64_t)n) {
                    const int j = (tid >> 3) + (kThreads / F4) * it;
                    *reinterpret_cast<float4*>(s_feat + j * kMfFeat + 4 * (tid & 7)) = v[it];
                    finite = finite && fabsf(v[it].x) < 1e30f && fabsf(v[it].y) < 1e30f &&
                             fabsf(v[it].z) < 1e30f && fabsf(v[it].w) < 1e30f;
                }
            }
        } else {
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int j = (tid >> 3) + (kThreads / F4) * it, q = tid & 7;
            const int k = base + j;
            if (k < num) {
                const int g = ids[start + k];
                if ((uint32_t)g < (uint64_t)n) {
                    const float* f = feat + (int64_t)g * C + c0 + 4 * q;
                    float4 v;
                    v.x = 4 * q < nc ? f[0] : 0.0f;
                    v.y = 4 * q + 1 < nc ? f[1] : 0.0f;
                    v.z = 4 * q + 2 < nc ? f[2] : 0.0f;
                    v.w = 4 * q + 3 < nc ? f[3] : 0.0f;
                    *reinterpret_cast<float4*>(s_feat + j * kMfFeat + 4 * q) = v;
                    finite = finite && fabsf(v.x) < 1e30f && fabsf(v.y) < 1e30f &&
                             fabsf(v.z) < 1e30f && fabsf(v.w) < 1e30f;
                }
            }
        }
        }
        if (wave < NLW) {
#pragma unroll
            for (int q = 0; q < kWaves; ++q) {
                const uint64_t b = __ballot((qm >> q) & 1u);
                if (lane == 0) s_mask[q][wave] = b;
            }
        }
        const uint64_t np = __ballot(!plain), nf = __ballot(!finite);
        if (lane == 0) {
            s_plain[wave] = np == 0ull;
            s_finite[wave] = nf == 0ull;
        }
        __syncthreads();
        const uint4 pl = *reinterpret_cast<const uint4*>(s_plain);
        const uint4 fi = *reinterpret_cast<const uint4*>(s_finite);
        const bool batch_plain = (pl.x & pl.y & pl.z & pl.w) != 0u;
        const bool batch_finite = (fi.x & fi.y & fi.z & fi.w) != 0u;
        if (alive == 0ull) continue;
        const int cnt = build_list<NLW, false>(s_mask[wave], s_list[wave], lane, BB * 16);
        int last_off = -1;
        if (batch_finite) {
            if (batch_plain)
                fwd_walk_mx<DEPTH, true, true>(s_list[wave], cnt, s_r0, s_r1, s_feat, BB,
                                               s_tile[wave], pxf, pyf, lane, T, dacc, last_off,
                                               alive, acc);
            else
                fwd_walk_mx<DEPTH, false, true>(s_list[wave], cnt, s_r0, s_r1, s_feat, BB,
                                                s_tile[wave], pxf, pyf, lane, T, dacc, last_off,
                                                alive, acc);
        } else {
            fwd_walk_mx<DEPTH, false, false>(s_list[wave], cnt, s_r0, s_r1, s_feat, BB,
                                             s_tile[wave], pxf, pyf, lane, T, dacc, last_off,
                                             alive, acc);
        }
        if (last_off >= 0) last = base + (last_off >> 4) + 1;
    }
    if (inside && c0 == 0) {
        const int64_t pid = (int64_t)py * W + px;
        final_T[pid] = T;
        n_contrib[pid] = last;
        if (alpha_out) alpha_out[pid] = 1.0f - T;
        if (DEPTH) {
            const float al = 1.0f - T;
            depth_out[pid] = al > 1e-6f ? dacc / al : 0.0f;
        }
    }
    if (work) store_tile_work(work, tile, last, wave, lane);
    // channel results: lane l holds quadrant pixel 16 pb + l % 16, channels
    // 16 cb + 4 (l / 16) + i; that pixel's T is lane (16 pb + l % 16)'s
    const int row = lane & 15, kq = lane >> 4;
    // whole 16-byte pieces when the block is 32 aligned channels
    const bool vec_out = nc == 32 && (C & 3) == 0 && (c0 & 3) == 0 &&
                         (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
        const int q = 16 * pb + row;
        const float Tq = __shfl(T, q, kWave);
        const int bx = qx0 + (q & 7), by = qy0 + (q >> 3);
        if (bx < W && by < H) {
            float* o = out + ((int64_t)by * W + bx) * C + c0;
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                const int ch0 = 16 * cb + 4 * kq;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    v[i] = acc[cb][pb][i] + Tq * (bg && ch0 + i < nc ? bg[c0 + ch0 + i] : 0.0f);
                if (vec_out) {
                    *reinterpret_cast<float4*>(o + ch0) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (ch0 + i < nc) o[ch0 + i] = v[i];
                }
            }
        }
    }
}

// One workgroup per band (the forward's order, or the backward's).
template <bool BWD>
__global__ __launch_bounds__(kOrderThreads) void k_tile_order(const int2* __restrict__ ranges,
                                                              const int* __restrict__ work,
                                                              int64_t n_ids, int tiles,
                                                              int* __restrict__ order) {
    __shared__ uint32_t s_order[tile_order_lds_words<kOrderThreads>()];
    tile_order_band<BWD>(blockIdx.x, ranges, work, n_ids, tiles, order, s_order);
}

// The gradient outputs to clear: one record (a, na floats, 16-byte aligned,
// na a multiple of 4) or four arrays.
struct ZeroGrads {
    float* p[4];
    int64_t n[4];
    bool record;
};

// The backward's prologue in one launch: workgroups [0, bands) build the
// backward's tile order from the forward's per-tile work (bands = 0 without
// one), the others clear the gradient outputs (a fill kernel rather than
// hipMemsetAsync, so the call can sit inside a captured graph).  The order's
// few long-lived workgroups run beside the clearing instead of after it.
__global__ __launch_bounds__(kOrderThreads) void k_bwd_prologue(ZeroGrads z, int bands,
                                                                const int* __restrict__ work,
                                                                int64_t n_ids, int tiles,
                                                                int* __restrict__ order) {
    __shared__ uint32_t s_order[tile_order_lds_words<kOrderThreads>()];
    if ((int)blockIdx.x < bands) {
        tile_order_band<true>(blockIdx.x, nullptr, work, n_ids, tiles, order, s_order);
        return;
    }
    const int64_t b = (int64_t)blockIdx.x - bands;
    const int64_t stride = ((int64_t)gridDim.x - bands) * kOrderThreads;
    if (z.record) {
        float4* a = reinterpret_cast<float4*>(z.p[0]);
        for (int64_t i = b * kOrderThreads + threadIdx.x; i < z.n[0] / 4; i += stride)
            a[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
        for (int64_t i = b * kOrderThreads + threadIdx.x; i < z.n[r]; i += stride) z.p[r][i] = 0.0f;
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
                int tiles_x, float* out, float* fT, int* ncon, float* dout, float* aout,
                const int* order, int* work) {
    if constexpr (CH == 32) {
        if (depth)
            hipLaunchKernelGGL((k_raster_fwd_mx<true>), grid, dim3(kThreads), 0, st, xy, co, feat,
                               C, c0, nc, depths, ids, ranges, n, n_ids, bg, W, H, tiles_x, out,
                               fT, ncon, dout, aout, order, work);
        else
            hipLaunchKernelGGL((k_raster_fwd_mx<false>), grid, dim3(kThreads), 0, st, xy, co,
                               feat, C, c0, nc, depths, ids, ranges, n, n_ids, bg, W, H, tiles_x,
                               out, fT, ncon, dout, aout, order, work);
    } else if (depth) {
        hipLaunchKernelGGL((k_raster_fwd<CH, true>), grid, dim3(kThreads), 0, st, xy, co, feat, C,
                           c0, nc, depths, ids, ranges, n, n_ids, bg, W, H, tiles_x, out, fT,
                           ncon, dout, aout, order, work);
    } else {
        hipLaunchKernelGGL((k_raster_fwd<CH, false>), grid, dim3(kThreads), 0, st, xy, co, feat, C,
                           c0, nc, depths, ids, ranges, n, n_ids, bg, W, H, tiles_x, out, fT,
                           ncon, dout, aout, order, work);
    }
}

template <int CH>
void launch_bwd(dim3 grid, hipStream_t st, const float2* xy, const float4* co, const float* feat,
                int C, int c0, int nc, const int* ids, const int2* ranges, int64_t n,
                int64_t n_ids, const float* bg, int W, int H, int tiles_x, const float* fT,
                const int* ncon, const float* gout, const float* gT, float* gxy, float* gcon,
                float* gfeat, float* gop, int gstride, const int* order) {
    if constexpr (CH == 32)
        hipLaunchKernelGGL((k_raster_bwd_mx<CH>), grid, dim3(kThreads), 0, st, xy, co, feat, C,
                           c0, nc, ids, ranges, n, n_ids, bg, W, H, tiles_x, fT, ncon, gout, gT,
                           gxy, gcon, gfeat, gop, gstride, order);
    else
        hipLaunchKernelGGL((k_raster_bwd<CH>), grid, dim3(kThreads), 0, st, xy, co, feat, C, c0,
                           nc, ids, ranges, n, n_ids, bg, W, H, tiles_x, fT, ncon, gout, gT, gxy,
                           gcon, gfeat, gop, gstride, order);
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
                   float* depth_out, float* alpha_out, int32_t* tile_order, int32_t order_ready,
                   void* stream) {
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
    const int tiles = tiles_x * tiles_y;
    // tile_order: [0, T) the bounds this call writes, [T, 2T) its order
    // (order_ready: gsx_bin_tiles_async wrote it for these ranges)
    int* const order = tile_order ? tile_order + tiles : nullptr;
    if (order && !order_ready) {
        hipLaunchKernelGGL(k_tile_order<false>, dim3(kOrderBands), dim3(kOrderThreads), 0, st,
                           (const int2*)tile_ranges, (const int*)nullptr, num_ids, tiles, order);
        GSX_LAUNCH_CHECK();
    }
    for (int c0 = 0; c0 < C; c0 += kMaxChunk) {
        const int nc = (C - c0 < kMaxChunk) ? C - c0 : kMaxChunk;
        const bool depth = depths && c0 == 0;
        int* work = (tile_order && c0 == 0) ? tile_order : nullptr;
        switch (pick_ch(nc)) {
#define GSX_FWD_CASE(V)                                                                          \
    case V:                                                                                      \
        launch_fwd<V>(grid, st, depth, (const float2*)means2d, (const float4*)conic_opacity,     \
                      features, C, c0, nc, depths, sorted_ids, (const int2*)tile_ranges, n,      \
                      num_ids, background, width, height, tiles_x, out, final_T, n_contrib,      \
                      depth_out, alpha_out, order, work);                                        \
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

int64_t gsx_tile_order_words(int32_t width, int32_t height) {
    if (width <= 0 || height <= 0) return 0;
    const int64_t tiles =
        (int64_t)((width + kTile - 1) / kTile) * (int64_t)((height + kTile - 1) / kTile);
    return tile_order_words(tiles);
}

int gsx_raster_bwd(int64_t n, int32_t C, const float* means2d, const float* conic_opacity,
                   const float* features, const int32_t* sorted_ids, int64_t num_ids,
                   const int32_t* tile_ranges,
                   const float* background, int32_t width, int32_t height, const float* final_T,
                   const int32_t* n_contrib, const float* grad_out, const float* grad_final_T,
                   float* g_means2d, float* g_conics, float* g_features, float* g_opacities,
                   int32_t grad_stride, int32_t* tile_order, void* stream) {
    if (n < 0 || num_ids < 0 || C <= 0 || width <= 0 || height <= 0) return GSX_ERR_INVALID;
    if (!tile_ranges || !final_T || !n_contrib || !grad_out) return GSX_ERR_INVALID;
    const bool rec = grad_stride > 0;
    if (grad_stride < 0 || (rec && (grad_stride % 4 != 0 || grad_stride < 6 + C ||
                                    !aligned16(g_means2d) || g_conics || g_features ||
                                    g_opacities)))
        return GSX_ERR_INVALID;
    if (n > 0 && (!means2d || !conic_opacity || !features || !g_means2d ||
                  (!rec && (!g_conics || !g_features || !g_opacities))))
        return GSX_ERR_INVALID;
    if (num_ids > 0 && !sorted_ids) return GSX_ERR_INVALID;
    if (!aligned8(means2d) || !aligned16(conic_opacity) || !aligned8(tile_ranges))
        return GSX_ERR_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (n == 0) return GSX_OK;
    const int tiles_x = (width + kTile - 1) / kTile;
    const int tiles_y = (height + kTile - 1) / kTile;
    const int tiles = tiles_x * tiles_y;
    // tile_order: [0, T) the forward's bounds, [T, T + 16 ceil(T / 8)) this
    // call's order, one entry per workgroup
    int* const order = tile_order ? tile_order + tiles : nullptr;
    const dim3 grid((unsigned)(order ? tile_order_words(tiles) - tiles : tiles));
    {
        // gradient clearing and the tile order in one launch
        ZeroGrads z{};
        z.record = rec;
        if (rec) {
            z.p[0] = g_means2d;
            z.n[0] = (int64_t)grad_stride * n;
        } else {
            z.p[0] = g_means2d;
            z.n[0] = 2 * n;
            z.p[1] = g_conics;
            z.n[1] = 3 * n;
            z.p[2] = g_features;
            z.n[2] = (int64_t)C * n;
            z.p[3] = g_opacities;
            z.n[3] = n;
        }
        const int64_t most = rec ? z.n[0] / 4 : std::max<int64_t>((int64_t)C, 3) * n;
        const int bands = order ? kOrderBands : 0;
        const unsigned blocks =
            (unsigned)std::min<int64_t>((most + kOrderThreads - 1) / kOrderThreads, 2048);
        hipLaunchKernelGGL(k_bwd_prologue, dim3(blocks + (unsigned)bands), dim3(kOrderThreads), 0,
                           st, z, bands, (const int*)tile_order, num_ids, tiles, order);
        GSX_LAUNCH_CHECK();
    }
    for (int c0 = 0; c0 < C; c0 += kMaxChunk) {
        const int nc = (C - c0 < kMaxChunk) ? C - c0 : kMaxChunk;
        switch (pick_ch(nc)) {
#define GSX_BWD_CASE(V)                                                                          \
    case V:                                                                                      \
        launch_bwd<V>(grid, st, (const float2*)means2d, (const float4*)conic_opacity, features,  \
                      C, c0, nc, sorted_ids, (const int2*)tile_ranges, n, num_ids, background,   \
                      width, height, tiles_x, final_T, n_contrib, grad_out, grad_final_T,        \
                      g_means2d, g_conics, g_features, g_opacities, grad_stride, order);         \
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
