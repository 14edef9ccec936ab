// binning.hip -- tile binning (replaces bin_gaussians, splatting/tiles.py:19-182).
//
// The reference builds key = tile*N + rank(depth) and argsorts it
// (tiles.py:166-172).  Here the same order is produced depth-first:
//   1. stable LSD radix sort of the N per-Gaussian depth keys (4 x 8 bits),
//      which orders Gaussians by (depth, index);
//   2. exclusive scan of the tile counts gathered in that order (the only
//      host readback: the duplicate total D);
//   3. emission of the D (tile, gaussian) pairs in depth order, one lane per
//      duplicate with a block-narrowed binary search (no long serial loops
//      for Gaussians spanning thousands of tiles);
//   4. stable LSD radix sort of the tile ids (ceil(log2 tiles)/8 passes),
//      so inside a tile the depth order of step 1 is kept;
//   5. [start, end) ranges from the sorted tile ids; empty tiles stay (0,0)
//      as the scatter-min/max of tiles.py:175-180 leaves them.
// Only 2 passes run over the D-sized arrays at 1080p (13 tile bits) instead
// of the 6 a 45-bit (tile, depth) key would need.
#include <algorithm>

#include "gsx_device.h"

using namespace gsx;

namespace {

constexpr int kThreads = 256;
constexpr int kItems = 16;
constexpr int kChunk = kThreads * kItems;  // 4096 elements per workgroup
constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// LDS index padded by one word per 32 so that a lane reading its 16
// consecutive elements hits 32 distinct banks across a half-wave.
__device__ __forceinline__ int pad(int i) { return i + (i >> 5); }
constexpr int kPadded = kChunk + kChunk / 32;

// Exclusive scan of the kChunk values in s (padded layout), plus `carry`.
// Returns the chunk total.  Every thread of the block must call it.
__device__ uint32_t block_scan_chunk(uint32_t* s, uint32_t* s_wave, uint32_t carry) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t v[kItems];
    uint32_t sum = 0;
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        v[k] = s[pad(tid * kItems + k)];
        sum += v[k];
    }
    const uint32_t incl = wave_incl_scan(sum);
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    uint32_t wave_off = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        const uint32_t t = s_wave[w];
        if (w < wave) wave_off += t;
        total += t;
    }
    uint32_t run = carry + wave_off + incl - sum;
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        s[pad(tid * kItems + k)] = run;
        run += v[k];
    }
    __syncthreads();
    return total;
}

__device__ __forceinline__ uint32_t block_sum(uint32_t v, uint32_t* s_wave) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == 0) s_wave[wave] = v;
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) t += s_wave[w];
    return t;
}

// Phase 1 of the reduce-then-scan: per-chunk sums.  `gather` (optional)
// reads in[gather[i]] instead of in[i].
__global__ __launch_bounds__(kThreads) void k_scan_reduce(const uint32_t* __restrict__ in,
                                                          const uint32_t* __restrict__ gather,
                                                          int64_t n, uint32_t* __restrict__ partials) {
    __shared__ uint32_t s_wave[kThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kChunk;
    uint32_t s = 0;
#pragma unroll 4
    for (int k = 0; k < kItems; ++k) {
        const int64_t i = base + k * kThreads + threadIdx.x;
        if (i < n) s += gather ? in[gather[i]] : in[i];
    }
    const uint32_t t = block_sum(s, s_wave);
    if (threadIdx.x == 0) partials[blockIdx.x] = t;
}

// Phase 2: one workgroup scans the partials (exclusive, in place), chunk by
// chunk; the grand total goes to total_out[0] and, if given, total_out2[0].
__global__ __launch_bounds__(kThreads) void k_scan_partials(uint32_t* __restrict__ partials,
                                                            int64_t nparts,
                                                            uint32_t* __restrict__ total_out,
                                                            uint32_t* __restrict__ total_out2) {
    __shared__ uint32_t s[kPadded];
    __shared__ uint32_t s_wave[kThreads / 64];
    uint32_t carry = 0;
    for (int64_t base = 0; base < nparts; base += kChunk) {
#pragma unroll 4
        for (int k = 0; k < kItems; ++k) {
            const int idx = k * kThreads + threadIdx.x;
            const int64_t i = base + idx;
            s[pad(idx)] = (i < nparts) ? partials[i] : 0u;
        }
        __syncthreads();
        carry += block_scan_chunk(s, s_wave, carry) ;
        // block_scan_chunk returned the chunk total; carry now includes it.
#pragma unroll 4
        for (int k = 0; k < kItems; ++k) {
            const int idx = k * kThreads + threadIdx.x;
            const int64_t i = base + idx;
            if (i < nparts) partials[i] = s[pad(idx)];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        total_out[0] = carry;
        if (total_out2) total_out2[0] = carry;
    }
}

// Phase 3: each chunk scanned with its carry-in.  In-place (out == in) is
// allowed: a chunk is fully read into LDS before it is written.
__global__ __launch_bounds__(kThreads) void k_scan_down(const uint32_t* in,
                                                        const uint32_t* __restrict__ gather,
                                                        int64_t n,
                                                        const uint32_t* __restrict__ partials,
                                                        uint32_t* out) {
    __shared__ uint32_t s[kPadded];
    __shared__ uint32_t s_wave[kThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kChunk;
#pragma unroll 4
    for (int k = 0; k < kItems; ++k) {
        const int idx = k * kThreads + threadIdx.x;
        const int64_t i = base + idx;
        s[pad(idx)] = (i < n) ? (gather ? in[gather[i]] : in[i]) : 0u;
    }
    __syncthreads();
    block_scan_chunk(s, s_wave, partials[blockIdx.x]);
#pragma unroll 4
    for (int k = 0; k < kItems; ++k) {
        const int idx = k * kThreads + threadIdx.x;
        const int64_t i = base + idx;
        if (i < n) out[i] = s[pad(idx)];
    }
}

// Lanes of the wave (among `valid` ones) holding the same 8-bit digit.
__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool valid) {
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bb = __ballot(bit);
        m &= bit ? bb : ~bb;
    }
    return valid ? m : 0ull;
}

// Digit histogram of one 4096-key chunk -> hist[digit * nblocks + block].
// Element order inside a chunk: wave w owns [w*1024, (w+1)*1024), round r
// covers 64 consecutive keys -- the same order the scatter ranks in.
__global__ __launch_bounds__(kThreads) void k_radix_hist(const uint32_t* __restrict__ keys,
                                                         int64_t n, int shift,
                                                         uint32_t* __restrict__ hist,
                                                         int64_t nblocks) {
    __shared__ uint32_t s_h[kThreads / 64][kRadix];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s_h[w][tid] = 0u;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kChunk + wave * (kChunk / 4);
    const uint64_t lt = (1ull << lane) - 1ull;
    for (int r = 0; r < kItems; ++r) {
        const int64_t i = base + r * 64 + lane;
        const bool valid = i < n;
        const uint32_t d = valid ? (keys[i] >> shift) & (kRadix - 1) : 0u;
        const uint64_t m = match_digit(d, valid);
        if (valid && (m & lt) == 0ull) s_h[wave][d] += (uint32_t)__popcll(m);
    }
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) t += s_h[w][tid];
    hist[(int64_t)tid * nblocks + blockIdx.x] = t;
}

// Stable scatter of one chunk by digit using the scanned histogram.
// vals_in == nullptr means "values are the element indices".
__global__ __launch_bounds__(kThreads) void k_radix_scatter(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n,
    int shift, const uint32_t* __restrict__ hist_scanned, int64_t nblocks,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out) {
    __shared__ uint32_t s_cnt[kThreads / 64][kRadix];
    __shared__ uint32_t s_base[kRadix];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s_cnt[w][tid] = 0u;
    s_base[tid] = hist_scanned[(int64_t)tid * nblocks + blockIdx.x];
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kChunk + wave * (kChunk / 4);
    const uint64_t lt = (1ull << lane) - 1ull;
    uint32_t key[kItems], val[kItems], rank[kItems];
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
        const int64_t i = base + r * 64 + lane;
        const bool valid = i < n;
        key[r] = valid ? keys_in[i] : 0u;
        val[r] = valid ? (vals_in ? vals_in[i] : (uint32_t)i) : 0u;
        const uint32_t d = (key[r] >> shift) & (kRadix - 1);
        const uint64_t m = match_digit(d, valid);
        const uint32_t before = s_cnt[wave][d];
        rank[r] = before + (uint32_t)__popcll(m & lt);
        if (valid && (m & lt) == 0ull) s_cnt[wave][d] = before + (uint32_t)__popcll(m);
    }
    __syncthreads();
    {
        uint32_t run = 0;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) {
            const uint32_t c = s_cnt[w][tid];
            s_cnt[w][tid] = run;
            run += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
        const int64_t i = base + r * 64 + lane;
        if (i < n) {
            const uint32_t d = (key[r] >> shift) & (kRadix - 1);
            const uint32_t pos = s_base[d] + s_cnt[wave][d] + rank[r];
            if (pos < (uint64_t)n) {  // always true for a consistent histogram
                keys_out[pos] = key[r];
                vals_out[pos] = val[r];
            }
        }
    }
}

// Largest i in [lo, hi] with offs[i] <= d (offs non-decreasing,
// offs[hi + 1] > d guaranteed by the caller).
__device__ __forceinline__ int64_t find_owner(const uint32_t* __restrict__ offs, int64_t lo,
                                              int64_t hi, uint32_t d) {
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (offs[mid] <= d) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

constexpr int kEmitItems = 4;
constexpr int kEmitChunk = kThreads * kEmitItems;

// One lane per duplicate: duplicate d belongs to the depth-ordered Gaussian
// whose [offs[i], offs[i+1]) contains d; its tile is the (d - offs[i])-th
// cell of the Gaussian's tile rectangle in row-major order (tiles.py:85-89).
__global__ __launch_bounds__(kThreads) void k_emit(int64_t nd, int64_t n,
                                                   const uint32_t* __restrict__ offs,
                                                   const uint32_t* __restrict__ gids,
                                                   const uint2* __restrict__ rects, int tiles_x,
                                                   uint32_t* __restrict__ keys_out,
                                                   uint32_t* __restrict__ vals_out) {
    __shared__ int64_t s_range[2];
    const int64_t d0 = (int64_t)blockIdx.x * kEmitChunk;
    if (threadIdx.x < 2) {
        const int64_t dq = threadIdx.x == 0 ? d0 : min(d0 + kEmitChunk - 1, nd - 1);
        s_range[threadIdx.x] = find_owner(offs, 0, n - 1, (uint32_t)dq);
    }
    __syncthreads();
    const int64_t lo = s_range[0], hi = s_range[1];
#pragma unroll
    for (int k = 0; k < kEmitItems; ++k) {
        const int64_t d = d0 + k * kThreads + threadIdx.x;
        if (d >= nd) break;
        const int64_t i = find_owner(offs, lo, hi, (uint32_t)d);
        const uint32_t g = gids[i];
        const uint32_t local = (uint32_t)d - offs[i];
        const uint2 r = rects[g];
        const uint32_t w = r.y & 0xFFFFu;
        const uint32_t tx = (r.x & 0xFFFFu) + local % w;
        const uint32_t ty = (r.x >> 16) + local / w;
        keys_out[d] = ty * (uint32_t)tiles_x + tx;
        vals_out[d] = g;
    }
}

__global__ __launch_bounds__(kThreads) void k_fill_u32(uint32_t* __restrict__ p, int64_t n,
                                                       uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ __launch_bounds__(kThreads) void k_tile_ranges(int64_t nd,
                                                          const uint32_t* __restrict__ tiles,
                                                          int64_t num_tiles,
                                                          int2* __restrict__ ranges) {
    const int64_t d = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (d >= nd) return;
    const uint32_t t = tiles[d];
    if (t >= (uint64_t)num_tiles) return;
    if (d == 0 || tiles[d - 1] != t) ranges[t].x = (int)d;
    if (d == nd - 1 || tiles[d + 1] != t) ranges[t].y = (int)(d + 1);
}

// ------------------------------------------------------------ host side --
struct Layout {
    size_t dk0, dk1, dv0, dv1, offs, tk0, tk1, tv, hist, parts, misc, total;
};

inline size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

Layout make_layout(int64_t n, int64_t cap) {
    Layout L{};
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = align_up(o + bytes);
        return at;
    };
    const size_t nn = (size_t)(n > 0 ? n : 1), cc = (size_t)(cap > 0 ? cap : 1);
    const int64_t nb = ceil_div(std::max<int64_t>(std::max<int64_t>(n, cap), 1), kChunk);
    const int64_t scan_len = std::max<int64_t>(nb * kRadix, n + 1);
    L.dk0 = take(4 * nn);
    L.dk1 = take(4 * nn);
    L.dv0 = take(4 * nn);
    L.dv1 = take(4 * nn);
    L.offs = take(4 * (nn + 1));
    L.tk0 = take(4 * cc);
    L.tk1 = take(4 * cc);
    L.tv = take(4 * cc);
    L.hist = take(4 * (size_t)(nb * kRadix));
    L.parts = take(4 * (size_t)(ceil_div(scan_len, kChunk) + 1));
    L.misc = take(4 * 16);
    L.total = o;
    return L;
}

template <typename T>
inline T* at(void* ws, size_t off) {
    return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

int scan_exclusive(const uint32_t* in, const uint32_t* gather, int64_t len, uint32_t* out,
                   uint32_t* partials, uint32_t* total, uint32_t* total2, hipStream_t st) {
    const int64_t nparts = ceil_div(len, kChunk);
    hipLaunchKernelGGL(k_scan_reduce, dim3((unsigned)nparts), dim3(kThreads), 0, st, in, gather,
                       len, partials);
    hipLaunchKernelGGL(k_scan_partials, dim3(1), dim3(kThreads), 0, st, partials, nparts, total,
                       total2);
    hipLaunchKernelGGL(k_scan_down, dim3((unsigned)nparts), dim3(kThreads), 0, st, in, gather, len,
                       partials, out);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int radix_pass(const uint32_t* kin, const uint32_t* vin, int64_t count, int shift,
               uint32_t* kout, uint32_t* vout, uint32_t* hist, uint32_t* parts, uint32_t* misc,
               hipStream_t st) {
    const int64_t nb = ceil_div(count, kChunk);
    hipLaunchKernelGGL(k_radix_hist, dim3((unsigned)nb), dim3(kThreads), 0, st, kin, count, shift,
                       hist, nb);
    GSX_LAUNCH_CHECK();
    const int rc = scan_exclusive(hist, nullptr, nb * kRadix, hist, parts, misc + 8, nullptr, st);
    if (rc != GSX_OK) return rc;
    hipLaunchKernelGGL(k_radix_scatter, dim3((unsigned)nb), dim3(kThreads), 0, st, kin, vin, count,
                       shift, hist, nb, kout, vout);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

inline int bits_for(int64_t count) {
    int b = 0;
    while ((int64_t(1) << b) < count) ++b;
    return b;
}

}  // namespace

extern "C" {

int64_t gsx_bin_workspace_bytes(int64_t n, int64_t capacity, int32_t num_tiles) {
    (void)num_tiles;
    if (n < 0 || capacity < 0) return -1;
    return (int64_t)make_layout(n, capacity).total;
}

int gsx_bin_sort(int64_t n, const uint32_t* tile_counts, const uint32_t* depth_keys,
                 const uint32_t* tile_rects, int32_t width, int32_t height, void* workspace,
                 int64_t workspace_bytes, int64_t capacity, int32_t* sorted_ids,
                 int32_t* tile_ranges, int64_t* num_dups, void* stream) {
    if (n < 0 || width <= 0 || height <= 0 || capacity < 0 || !num_dups || !tile_ranges)
        return GSX_ERR_INVALID;
    if (n > 0x7FFFFFFF) return GSX_ERR_TOO_LARGE;
    hipStream_t st = (hipStream_t)stream;
    const int tiles_x = (width + kTile - 1) / kTile;
    const int tiles_y = (height + kTile - 1) / kTile;
    const int64_t T = (int64_t)tiles_x * tiles_y;
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)ceil_div(2 * T, kThreads)), dim3(kThreads), 0, st,
                       (uint32_t*)tile_ranges, 2 * T, 0u);
    GSX_LAUNCH_CHECK();
    if (n == 0) {
        *num_dups = 0;
        return GSX_OK;
    }
    if (!tile_counts || !depth_keys || !tile_rects || !workspace) return GSX_ERR_INVALID;
    const Layout L = make_layout(n, capacity);
    if (workspace_bytes < (int64_t)L.total) return GSX_ERR_WORKSPACE;
    void* ws = workspace;
    uint32_t* hist = at<uint32_t>(ws, L.hist);
    uint32_t* parts = at<uint32_t>(ws, L.parts);
    uint32_t* misc = at<uint32_t>(ws, L.misc);

    // 1. stable sort of the Gaussians by depth key (index order breaks ties)
    const uint32_t* kin = depth_keys;
    const uint32_t* vin = nullptr;
    uint32_t* kbuf[2] = {at<uint32_t>(ws, L.dk0), at<uint32_t>(ws, L.dk1)};
    uint32_t* vbuf[2] = {at<uint32_t>(ws, L.dv0), at<uint32_t>(ws, L.dv1)};
    for (int p = 0; p < 4; ++p) {
        const int rc = radix_pass(kin, vin, n, p * kRadixBits, kbuf[p & 1], vbuf[p & 1], hist,
                                  parts, misc, st);
        if (rc != GSX_OK) return rc;
        kin = kbuf[p & 1];
        vin = vbuf[p & 1];
    }
    const uint32_t* gids = vin;

    // 2. duplicate offsets in depth order; D = total
    uint32_t* offs = at<uint32_t>(ws, L.offs);
    int rc = scan_exclusive(tile_counts, gids, n, offs, parts, misc, offs + n, st);
    if (rc != GSX_OK) return rc;
    uint32_t D32 = 0;
    if (hipMemcpyAsync(&D32, misc, sizeof(uint32_t), hipMemcpyDeviceToHost, st) != hipSuccess)
        return GSX_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return GSX_ERR_HIP;
    const int64_t D = (int64_t)D32;
    *num_dups = D;
    if (D > 0x7FFFFFFF) return GSX_ERR_TOO_LARGE;
    if (D > capacity) return 1;
    if (D == 0) return GSX_OK;
    if (!sorted_ids) return GSX_ERR_INVALID;

    // 3. emit, 4. sort by tile so the final values land in sorted_ids
    const int passes = (bits_for(T) + kRadixBits - 1) / kRadixBits;
    uint32_t* tk[2] = {at<uint32_t>(ws, L.tk0), at<uint32_t>(ws, L.tk1)};
    uint32_t* tv[2] = {(uint32_t*)sorted_ids, at<uint32_t>(ws, L.tv)};
    int cur = (passes % 2 == 0) ? 0 : 1;
    hipLaunchKernelGGL(k_emit, dim3((unsigned)ceil_div(D, kEmitChunk)), dim3(kThreads), 0, st, D, n,
                       offs, gids, (const uint2*)tile_rects, tiles_x, tk[cur], tv[cur]);
    GSX_LAUNCH_CHECK();
    for (int p = 0; p < passes; ++p) {
        rc = radix_pass(tk[cur], tv[cur], D, p * kRadixBits, tk[cur ^ 1], tv[cur ^ 1], hist, parts,
                        misc, st);
        if (rc != GSX_OK) return rc;
        cur ^= 1;
    }
    // 5. ranges
    hipLaunchKernelGGL(k_tile_ranges, dim3((unsigned)ceil_div(D, kThreads)), dim3(kThreads), 0, st,
                       D, tk[cur], T, (int2*)tile_ranges);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // extern "C"
