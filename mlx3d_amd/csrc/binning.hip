// binning.hip -- tile binning (replaces bin_gaussians, splatting/tiles.py:19-182).
//
// The reference builds key = tile*N + rank(depth) and argsorts it
// (tiles.py:166-172).  Here the same order is produced depth-first:
//   1. stable LSD radix sort of the N per-Gaussian depth keys (4 x 8 bits),
//      which orders Gaussians by (depth, index);
//   2. exclusive scan of the tile counts in that order -> duplicate offsets
//      and the duplicate count D (kept on the device);
//   3. emission of the (tile, gaussian) pairs, balanced by duplicates: each
//      workgroup owns 4096 consecutive duplicates, finds the Gaussians that
//      own them with a cooperative search, stages those Gaussians in LDS and
//      expands their tile rectangles (row-major, tiles.py:85-89).  It also
//      histograms the tile-id digits for step 4;
//   4. stable LSD radix sort of the tile ids (ceil(log2 tiles)/8 passes), so
//      inside a tile the depth order of step 1 is kept;
//   5. [start, end) ranges from the sorted tile ids; empty tiles stay (0,0)
//      as the scatter-min/max of tiles.py:175-180 leaves them.
// Radix passes are single-kernel "onesweep" passes (Adinets & Merrill,
// 2022): digit histograms come from an earlier read, each pass ranks a chunk
// with wave-level multi-split, publishes its digit counts and finds its
// global offsets by decoupled look-back (Merrill & Garland, 2016), then
// writes the chunk through LDS in digit order so the global stores are
// runs of consecutive addresses.  The scan of step 2 uses the same
// look-back.  Chunks are claimed through an atomic counter, so a chunk only
// waits for chunks that are already running; each wait is bounded and
// raises an error flag instead of spinning forever.  No host round trip
// splits the pipeline: later steps size themselves from the device-side D.
#include <algorithm>

#include "gsx_device.h"

using namespace gsx;

namespace {

constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kMaxPasses = 4;
// depth sort: 512 threads x 8 keys per chunk; tile sort: 512 x 14 (the
// largest chunk at which two workgroups fit a CU: 124 VGPRs, 65 KB of LDS;
// measured against 1024 x 12 at one per CU: 48.5 vs 53.0 us per pass at C3,
// 276 vs 287 us at C4; 512 x 13, 15 and 16 slower)
constexpr int kDepthThreads = 512, kDepthItems = 8;
constexpr int kTileThreads = 512, kTileItems = 14;
// depth histogram: 256 threads x hist_items(n) keys (short serial chains
// per thread for small n, fewer workgroups and global histogram atomics for
// large n; measured: 4 keys 6.1 us at 100k keys, 8 keys 13.1 us at 1M, 16
// keys 14.4 / 16.0 us)
constexpr int kHistThreads = 256;
__host__ __device__ inline int hist_items(int64_t n) { return n <= (int64_t(1) << 18) ? 4 : 8; }
// count scan: 1024 threads x 4 Gaussians; emission: 1024 threads x 4 duplicates
constexpr int kScanThreads = 1024, kScanItems = 4, kScanChunk = kScanThreads * kScanItems;
constexpr int kEmitThreads = 1024, kEmitItems = 4, kEmitDups = kEmitThreads * kEmitItems;
// Global digit histograms are kept in kHistCopies copies (workgroup b adds
// into copy b % kHistCopies): same-address device atomics serialize, so one
// shared copy would cost a serialized update per workgroup per bin.
constexpr int kHistCopies = 16;
constexpr int kHistStride = kMaxPasses * kRadix;  // words between copies

// Look-back status word: 2 flag bits | 30-bit count.
constexpr uint32_t kFlagAgg = 1u << 30;
constexpr uint32_t kFlagInc = 2u << 30;
constexpr uint32_t kCountMask = (1u << 30) - 1u;
constexpr uint32_t kSpinLimit = 1u << 16;

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Status words are read and written with relaxed device-scope atomics.
// Each word carries everything a waiting chunk needs (flag + count), and the
// scattered keys are only read by the next kernel, so no acquire/release
// ordering is required -- on this GPU an agent-scope release or acquire
// would write back or invalidate the XCD's whole L2 on every publish/poll.
__device__ __forceinline__ uint32_t status_load(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void status_store(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exclusive prefix of one counter column for chunk `chunk`: sums earlier
// chunks' published counts, walking back until an inclusive one.  Statuses
// are read kLookWindow at a time so a long walk costs few round trips.
// Chunk 0 always publishes inclusive, so the walk ends; an unpublished
// predecessor is polled at most kSpinLimit times, then the error flag is
// raised.
constexpr int kLookWindow = 8;
__device__ __forceinline__ uint32_t look_back(const uint32_t* status, int64_t chunk, int stride,
                                              int col, uint32_t* err) {
    uint32_t prefix = 0;
    uint32_t spins = 0;
    int64_t c = chunk - 1;
    while (c >= 0) {
        uint32_t s[kLookWindow];
#pragma unroll
        for (int k = 0; k < kLookWindow; ++k)  // before chunk 0: an inclusive zero
            s[k] = c - k >= 0 ? status_load(status + (c - k) * stride + col) : kFlagInc;
        int used = 0;
        bool done = false, stalled = false;
#pragma unroll
        for (int k = 0; k < kLookWindow; ++k) {
            if (done || stalled) continue;
            const uint32_t flag = s[k] & ~kCountMask;
            if (flag == 0u) {
                stalled = true;
                continue;
            }
            prefix += s[k] & kCountMask;
            ++used;
            done = flag == kFlagInc;
        }
        if (done) break;
        c -= used;
        if (stalled) {
            if (++spins > kSpinLimit) {
                atomicOr(err, GSX_BIN_ERR_LOOKBACK);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    return prefix;
}

// min(n_host, *n_dev) when the live length is only known on the device.
__device__ __forceinline__ int64_t live_count(int64_t n_host, const uint32_t* n_dev) {
    if (!n_dev) return n_host;
    const int64_t d = (int64_t)*n_dev;
    return d < n_host ? d : n_host;
}

// Lanes of the wave (among `valid` ones) holding the same digit, whose
// significant bits are the low `nbits` (<= 8, uniform; the others are zero
// in every key).  Per bit, the lanes whose bit differs from this lane's are
// the ballot XOR this lane's bit replicated (a sign-extended bit field), and
// the differing masks are OR-ed: four to five 32-bit operations per bit
// instead of selecting between the ballot and its complement in 64 bits.
__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool valid, int nbits) {
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
        if (b >= nbits) break;
        const int s = __builtin_amdgcn_sbfe((int)d, b, 1);  // 0 or -1
        const uint64_t bb = __ballot(s != 0);
        lo |= (uint32_t)bb ^ (uint32_t)s;
        hi |= (uint32_t)(bb >> 32) ^ (uint32_t)s;
    }
    const uint64_t same = ~(((uint64_t)hi << 32) | lo) & __ballot(valid);
    return valid ? same : 0ull;
}

// LDS histogram add of one digit per valid lane.  Lanes sharing the digit
// of the first valid lane are folded into one add (the common case for
// high digits, which are nearly constant across a wave); the rest add 1.
__device__ __forceinline__ void hist_add(uint32_t* s_h, uint32_t d, bool valid) {
    const uint64_t act = __ballot(valid);
    if (act == 0ull) return;
    const int leader = __ffsll((unsigned long long)act) - 1;
    const uint32_t first = __builtin_amdgcn_readlane(d, leader);
    const uint64_t same = __ballot(valid && d == first);
    if (!valid) return;
    if (d != first) atomicAdd(&s_h[d], 1u);
    else if ((int)(threadIdx.x & 63) == leader) atomicAdd(&s_h[d], (uint32_t)__popcll(same));
}

// Exclusive scan over the workgroup; *total gets the sum.  Every thread
// must call it; s_w holds THREADS/64 words.
template <int THREADS>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* s_w, uint32_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t incl = wave_incl_scan(v);
    if (lane == 63) s_w[wave] = incl;
    __syncthreads();
    uint32_t off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < THREADS / 64; ++w) {
        const uint32_t t = s_w[w];
        if (w < wave) off += t;
        tot += t;
    }
    *total = tot;
    return off + incl - v;
}

// The same for two values at once (one barrier); s_w holds 2*THREADS/64 words.
template <int THREADS>
__device__ __forceinline__ void block_excl_scan2(uint32_t a, uint32_t b, uint32_t* s_w,
                                                 uint32_t* ea, uint32_t* eb) {
    constexpr int kW = THREADS / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t ia = wave_incl_scan(a), ib = wave_incl_scan(b);
    if (lane == 63) {
        s_w[wave] = ia;
        s_w[kW + wave] = ib;
    }
    __syncthreads();
    uint32_t oa = 0, ob = 0;
#pragma unroll
    for (int w = 0; w < kW; ++w)
        if (w < wave) {
            oa += s_w[w];
            ob += s_w[kW + w];
        }
    *ea = oa + ia - a;
    *eb = ob + ib - b;
}

// Largest o in [0, n) with offs[o] <= x (offs non-decreasing, offs[0] <= x),
// found by the whole workgroup: each round probes THREADS evenly spaced
// positions and keeps the interval after the last probe <= x.
template <int THREADS>
__device__ __forceinline__ int64_t block_find_owner(const uint32_t* __restrict__ offs, int64_t n,
                                                    uint32_t x) {
    int64_t a = 0, b = n;
    while (b - a > 1) {
        const int64_t step = ceil_div(b - a, THREADS);
        const int64_t p = a + (int64_t)threadIdx.x * step;
        const bool le = p < b && offs[p] <= x;
        const int cnt = __syncthreads_count(le);  // probes are monotone; p = a always counts
        a += (int64_t)(cnt - 1) * step;
        b = min(a + step, b);
    }
    return a;
}

constexpr int kZeroRanges = 5;
struct ZeroRanges {
    uint32_t* p[kZeroRanges];
    int64_t n[kZeroRanges];
};

__global__ __launch_bounds__(256) void k_zero_ranges(ZeroRanges z) {
    const int64_t stride = (int64_t)gridDim.x * 256;
#pragma unroll
    for (int r = 0; r < kZeroRanges; ++r)
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < z.n[r]; i += stride)
            z.p[r][i] = 0u;
}

// Digit histograms of the 4 bytes of every depth key from one read, added
// into copy blockIdx % kHistCopies of hist[copy][pass][digit], and the sum
// of the tile counts (the number of duplicates emission will write) added
// to *total, with the overflow bit once it passes kCountMask.
__global__ __launch_bounds__(kHistThreads) void k_depth_hist(const uint32_t* __restrict__ keys,
                                                             const uint32_t* __restrict__ counts,
                                                             int64_t n,
                                                             uint32_t* __restrict__ hist,
                                                             uint32_t* __restrict__ total,
                                                             uint32_t* __restrict__ err) {
    __shared__ uint32_t s_h[kMaxPasses][kRadix];
    __shared__ uint64_t s_sum[kHistThreads / 64];
    const int tid = threadIdx.x, wave = tid >> 6;
    const int items = hist_items(n);  // as the host sized the grid
    for (int k = tid; k < kMaxPasses * kRadix; k += kHistThreads) (&s_h[0][0])[k] = 0u;
    __syncthreads();
    const int64_t base =
        (int64_t)blockIdx.x * (kHistThreads * items) + wave * (64 * items);
    uint64_t sum = 0;
    for (int r = 0; r < items; ++r) {
        const int64_t i = base + r * 64 + (tid & 63);
        const bool valid = i < n;
        const uint32_t key = valid ? keys[i] : 0u;
        sum += valid ? counts[i] : 0u;
#pragma unroll
        for (int p = 0; p < kMaxPasses; ++p)
            hist_add(s_h[p], (key >> (p * kRadixBits)) & (kRadix - 1), valid);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if ((tid & 63) == 0) s_sum[wave] = sum;
    __syncthreads();
    if (tid == 0) {
        uint64_t t = 0;
#pragma unroll
        for (int w = 0; w < kHistThreads / 64; ++w) t += s_sum[w];
        if (t > 0) {
            // each add is at most 2^30, so the word cannot wrap before the
            // bit is set
            const uint32_t add = (uint32_t)(t > kCountMask ? kCountMask + 1u : t);
            const uint32_t old = atomicAdd(total, add);
            if ((uint64_t)old + add > kCountMask) atomicOr(err, GSX_BIN_ERR_OVERFLOW);
        }
    }
    uint32_t* h = hist + (blockIdx.x % kHistCopies) * kHistStride;
    for (int k = tid; k < kMaxPasses * kRadix; k += kHistThreads) {
        const uint32_t v = (&s_h[0][0])[k];
        if (v) atomicAdd(&h[k], v);
    }
}

// One stable LSD pass over the 8 bits at `shift`.  Chunk c (claimed in
// launch order) holds keys [c * chunk, (c + 1) * chunk); wave w of it owns
// a contiguous slice, ranked round by round, so the order is stable.  The
// chunk is regrouped by digit in LDS, then written out: element j of the
// regrouped chunk goes to global_base[digit] + j - chunk_base[digit].
// `hist` points at this pass's histogram in copy 0.  vals_in == nullptr
// means "values are the element indices".
template <int THREADS, int ITEMS>
__global__ __launch_bounds__(THREADS) void k_onesweep(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n_host,
    const uint32_t* __restrict__ n_dev, int shift, int nbits, const uint32_t* __restrict__ hist,
    uint32_t* __restrict__ status, uint32_t* __restrict__ counter,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out, uint32_t* __restrict__ err) {
    constexpr int kWaves = THREADS / 64;
    constexpr int kChunk = THREADS * ITEMS;
    static_assert(THREADS >= kRadix, "one thread per digit");
    __shared__ uint32_t s_cnt[kWaves][kRadix];
    __shared__ uint32_t s_dexcl[kRadix];
    __shared__ uint32_t s_shift[kRadix];
    __shared__ uint32_t s_w[2 * kWaves];
    __shared__ uint32_t s_key[kChunk], s_val[kChunk];
    __shared__ uint32_t s_chunk;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t n = live_count(n_host, n_dev);
    // The first ceil(n / chunk) workgroups claim exactly the live chunks;
    // the rest leave without claiming, so no live chunk waits on them.
    if ((int64_t)blockIdx.x * kChunk >= n) return;
    if (tid == 0) s_chunk = atomicAdd(counter, 1u);
    for (int k = tid; k < kWaves * kRadix; k += THREADS) (&s_cnt[0][0])[k] = 0u;
    uint32_t dsum = 0;
    if (tid < kRadix) {
#pragma unroll 4
        for (int c = 0; c < kHistCopies; ++c) dsum += hist[c * kHistStride + tid];
    }
    __syncthreads();
    const int64_t chunk = s_chunk;
    const int64_t base = chunk * kChunk + wave * (64 * ITEMS);
    const uint64_t lt = (1ull << lane) - 1ull;
    uint32_t key[ITEMS], val[ITEMS], rank[ITEMS];
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        const int64_t i = base + r * 64 + lane;
        key[r] = i < n ? keys_in[i] : 0u;
        val[r] = i < n ? (vals_in ? vals_in[i] : (uint32_t)i) : 0u;
    }
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        const bool valid = base + r * 64 + lane < n;
        const uint32_t d = (key[r] >> shift) & (kRadix - 1);
        const uint64_t m = match_digit(d, valid, nbits);
        const uint32_t before = s_cnt[wave][d];
        rank[r] = before + (uint32_t)__popcll(m & lt);
        if (valid && (m & lt) == 0ull) s_cnt[wave][d] = before + (uint32_t)__popcll(m);
    }
    __syncthreads();
    uint32_t local = 0;
    uint32_t* st = status + chunk * kRadix + tid;
    if (tid < kRadix) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t c = s_cnt[w][tid];
            s_cnt[w][tid] = local;
            local += c;
        }
        status_store(st, (chunk == 0 ? kFlagInc : kFlagAgg) | local);
    }
    // in-chunk digit offsets and global digit bases
    uint32_t dexcl, dbase;
    block_excl_scan2<THREADS>(local, dsum, s_w, &dexcl, &dbase);
    if (tid < kRadix) s_dexcl[tid] = dexcl;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        if (base + r * 64 + lane < n) {
            const uint32_t d = (key[r] >> shift) & (kRadix - 1);
            const uint32_t j = s_dexcl[d] + s_cnt[wave][d] + rank[r];
            s_key[j] = key[r];
            s_val[j] = val[r];
        }
    }
    if (tid < kRadix) {
        uint32_t prefix = 0;
        if (chunk > 0) {
            prefix = look_back(status, chunk, kRadix, tid, err);
            status_store(st, kFlagInc | ((prefix + local) & kCountMask));
        }
        s_shift[tid] = dbase + prefix - dexcl;  // modular: + j >= dexcl below
    }
    __syncthreads();
    const int cnt = (int)min<int64_t>(kChunk, n - chunk * kChunk);
    for (int j = tid; j < cnt; j += THREADS) {
        const uint32_t k = s_key[j];
        const uint32_t pos = s_shift[(k >> shift) & (kRadix - 1)] + (uint32_t)j;
        if (pos < (uint64_t)n) {  // always true for a consistent histogram
            keys_out[pos] = k;
            vals_out[pos] = s_val[j];
        }
    }
}

// Exclusive scan of the tile counts in depth order: offs[i] = sum of the
// counts of depth-ordered Gaussians 0..i-1, offs[n] = D, *d_total = D; and
// owner[b] for every emission workgroup b that has duplicates: the
// depth-ordered Gaussian that owns its first duplicate b * kEmitDups.
__global__ __launch_bounds__(kScanThreads) void k_count_scan(
    int64_t n, const uint32_t* __restrict__ counts, const uint32_t* __restrict__ gids,
    uint32_t* __restrict__ status, uint32_t* __restrict__ counter, uint32_t* __restrict__ offs,
    uint32_t* __restrict__ owner, int64_t n_owner, uint32_t* __restrict__ d_total,
    uint32_t* __restrict__ err, uint32_t* __restrict__ clear, int64_t n_clear) {
    __shared__ uint32_t s_w[kScanThreads / 64];
    __shared__ uint32_t s_chunk, s_prefix;
    const int tid = threadIdx.x;
    // the tile passes' look-back status words start at zero (they run after
    // this kernel and emission)
    for (int64_t k = (int64_t)blockIdx.x * kScanThreads + tid; k < n_clear;
         k += (int64_t)gridDim.x * kScanThreads)
        clear[k] = 0u;
    if (tid == 0) s_chunk = atomicAdd(counter, 1u);
    __syncthreads();
    const int64_t chunk = s_chunk;
    const int64_t nchunks = ceil_div(n, kScanChunk);
    if (chunk >= nchunks) return;  // not reached: the grid has exactly nchunks workgroups
    const int64_t i0 = chunk * kScanChunk + (int64_t)tid * kScanItems;
    uint32_t c[kScanItems];
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) c[j] = i0 + j < n ? counts[gids[i0 + j]] : 0u;
    uint32_t total;
    uint32_t csum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) csum += c[j];
    const uint32_t excl = block_excl_scan<kScanThreads>(csum, s_w, &total);
    if (tid == 0) {
        uint32_t prefix = 0;
        uint32_t* st = status + chunk;
        if (total > kCountMask) atomicOr(err, GSX_BIN_ERR_OVERFLOW);
        if (chunk == 0) {
            status_store(st, kFlagInc | (total & kCountMask));
        } else {
            status_store(st, kFlagAgg | (total & kCountMask));
            prefix = look_back(status, chunk, 1, 0, err);
            if ((uint64_t)prefix + total > kCountMask) atomicOr(err, GSX_BIN_ERR_OVERFLOW);
            status_store(st, kFlagInc | ((prefix + total) & kCountMask));
        }
        s_prefix = prefix;
        if (chunk == nchunks - 1) {
            *d_total = prefix + total;
            offs[n] = prefix + total;
        }
    }
    __syncthreads();
    uint32_t run = s_prefix + excl;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        if (i0 + j < n) {
            offs[i0 + j] = run;
            // owner[b] = the Gaussian whose duplicates include b * kEmitDups
            for (int64_t b = ceil_div((int64_t)run, kEmitDups);
                 b * kEmitDups < (int64_t)run + c[j] && b < n_owner; ++b)
                owner[b] = (uint32_t)(i0 + j);
        }
        run += c[j];
    }
}

// refine_tiles (tiles.py:91-146): keep a (tile, Gaussian) duplicate only if
// the minimum of q(d) = a dx^2 + 2 b dx dy + c dy^2 over the tile's
// continuous rectangle (clipped to the image) is <= 12 -- the least of the
// four corners and the four clipped edge minimisers, zero when the mean is
// inside.  float32 in the reference's evaluation order.
__device__ __forceinline__ float refine_q(float a, float b, float c, float dx, float dy) {
    return (a * dx * dx + 2.0f * b * dx * dy) + c * dy * dy;
}

__device__ __forceinline__ bool refine_keep(uint32_t tx, uint32_t ty, int W, int H, float gx,
                                            float gy, float a, float b, float c) {
    const float x0 = (float)(tx * kTile), y0 = (float)(ty * kTile);
    const float x1 = (float)min((int)(tx + 1) * kTile, W);
    const float y1 = (float)min((int)(ty + 1) * kTile, H);
    const float dxl = x0 - gx, dxr = x1 - gx, dyb = y0 - gy, dyt = y1 - gy;
    if (dxl <= 0.0f && dxr >= 0.0f && dyb <= 0.0f && dyt >= 0.0f) return true;
    const float dy_l = fminf(fmaxf(-(b / c) * dxl, dyb), dyt);
    const float dy_r = fminf(fmaxf(-(b / c) * dxr, dyb), dyt);
    const float dx_b = fminf(fmaxf(-(b / a) * dyb, dxl), dxr);
    const float dx_t = fminf(fmaxf(-(b / a) * dyt, dxl), dxr);
    float q = refine_q(a, b, c, dxl, dyb);
    q = fminf(q, refine_q(a, b, c, dxl, dyt));
    q = fminf(q, refine_q(a, b, c, dxr, dyb));
    q = fminf(q, refine_q(a, b, c, dxr, dyt));
    q = fminf(q, refine_q(a, b, c, dxl, dy_l));
    q = fminf(q, refine_q(a, b, c, dxr, dy_r));
    q = fminf(q, refine_q(a, b, c, dx_b, dyb));
    q = fminf(q, refine_q(a, b, c, dx_t, dyt));
    return q <= 12.0f;
}

// Duplicate emission, kEmitDups duplicates per workgroup (of the
// min(D, cap) that fit the output).  Duplicate d belongs to the
// depth-ordered Gaussian o with offs[o] <= d < offs[o + 1]; its tile is the
// (d - offs[o])-th cell of o's tile rectangle in row-major order.  The
// owners of a workgroup's duplicates form a contiguous range, staged in LDS
// when it fits (always, unless zero-count Gaussians sit between owners);
// otherwise each duplicate searches offs directly.  With conics given,
// duplicates refine_tiles rejects get the tile id `sentinel` (= the tile
// count, so they sort after every tile and the range pass ignores them) and
// are counted into *dropped.  The digit histograms of the emitted tile ids
// (passes x 256) go into copy blockIdx % kHistCopies of tile_hist.
__global__ __launch_bounds__(kEmitThreads) void k_emit(
    int64_t n, int64_t cap, const uint32_t* __restrict__ d_total,
    const uint32_t* __restrict__ offs, const uint32_t* __restrict__ owner,
    const uint32_t* __restrict__ gids,
    const uint2* __restrict__ rects, int tiles_x, int passes, const float2* __restrict__ xy,
    const float* __restrict__ con, int64_t cstride, int W, int H, uint32_t sentinel,
    uint32_t* __restrict__ dropped, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, uint32_t* __restrict__ tile_hist) {
    __shared__ uint32_t s_off[kEmitDups];
    __shared__ uint2 s_rect[kEmitDups];
    __shared__ uint32_t s_gid[kEmitDups];
    __shared__ uint32_t s_h[kMaxPasses][kRadix];
    __shared__ uint32_t s_drop;
    const int tid = threadIdx.x;
    const int64_t nd = live_count(cap, d_total);
    const int64_t d0 = (int64_t)blockIdx.x * kEmitDups;
    if (d0 >= nd) return;
    const int64_t d1 = min(d0 + kEmitDups, nd);
    for (int k = tid; k < kMaxPasses * kRadix; k += kEmitThreads) (&s_h[0][0])[k] = 0u;
    if (tid == 0) s_drop = 0u;
    // owner of the first duplicate, and a bound on the owner of the last:
    // the next workgroup's first owner, or a search for the last workgroup
    const int64_t lo = owner[blockIdx.x];
    const int64_t hi = d1 < nd ? (int64_t)owner[blockIdx.x + 1]
                               : block_find_owner<kEmitThreads>(offs, n, (uint32_t)(d1 - 1));
    const int64_t w = hi - lo + 1;
    const bool staged = w <= kEmitDups;  // uniform
    if (staged) {
        for (int k = tid; k < w; k += kEmitThreads) {
            const uint32_t g = gids[lo + k];
            s_off[k] = offs[lo + k];
            s_gid[k] = g;
            s_rect[k] = rects[g];
        }
    }
    __syncthreads();
    const int64_t dd = d0 + (int64_t)tid * kEmitItems;
    uint32_t t[kEmitItems], g[kEmitItems];
    uint32_t ndrop = 0;
    if (dd < d1) {
        // owner of dd, then walk forward for the following duplicates
        int64_t o;
        if (staged) {
            int a = 0, b = (int)w - 1;
            while (a < b) {
                const int mid = (a + b + 1) >> 1;
                if (s_off[mid] <= (uint32_t)dd) a = mid;
                else b = mid - 1;
            }
            o = a;
        } else {
            int64_t a = lo, b = hi;
            while (a < b) {
                const int64_t mid = (a + b + 1) >> 1;
                if (offs[mid] <= (uint32_t)dd) a = mid;
                else b = mid - 1;
            }
            o = a;
        }
#pragma unroll
        for (int j = 0; j < kEmitItems; ++j) {
            const uint32_t d = (uint32_t)(dd + j);
            uint32_t off;
            uint2 r;
            if (staged) {
                while (o + 1 < w && s_off[o + 1] <= d) ++o;
                off = s_off[o];
                r = s_rect[o];
                g[j] = s_gid[o];
            } else {
                while (o + 1 <= hi && offs[o + 1] <= d) ++o;
                off = offs[o];
                g[j] = gids[o];
                r = rects[g[j]];
            }
            const uint32_t local = d - off;
            const uint32_t rw = r.y & 0xFFFFu;
            const uint32_t tx = (r.x & 0xFFFFu) + local % rw;
            const uint32_t ty = (r.x >> 16) + local / rw;
            t[j] = ty * (uint32_t)tiles_x + tx;
            if (con && (int64_t)d < d1) {
                const float2 m = xy[g[j]];
                const float* cg = con + (int64_t)g[j] * cstride;
                if (!refine_keep(tx, ty, W, H, m.x, m.y, cg[0], cg[1], cg[2])) {
                    t[j] = sentinel;
                    ++ndrop;
                }
            }
        }
        if (dd + kEmitItems <= d1) {
            *reinterpret_cast<uint4*>(keys_out + dd) = make_uint4(t[0], t[1], t[2], t[3]);
            *reinterpret_cast<uint4*>(vals_out + dd) = make_uint4(g[0], g[1], g[2], g[3]);
        } else {
            for (int j = 0; j < kEmitItems; ++j)
                if (dd + j < d1) {
                    keys_out[dd + j] = t[j];
                    vals_out[dd + j] = g[j];
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < kEmitItems; ++j) t[j] = 0u;
    }
#pragma unroll
    for (int j = 0; j < kEmitItems; ++j)
        for (int p = 0; p < passes; ++p)
            hist_add(s_h[p], (t[j] >> (p * kRadixBits)) & (kRadix - 1), dd + j < d1);
    if (con) {
        const uint32_t wsum = wave_incl_scan(ndrop);
        if ((tid & 63) == 63 && wsum) atomicAdd(&s_drop, wsum);
    }
    __syncthreads();
    uint32_t* h = tile_hist + (blockIdx.x % kHistCopies) * kHistStride;
    for (int k = tid; k < passes * kRadix; k += kEmitThreads) {
        const uint32_t v = (&s_h[0][0])[k];
        if (v) atomicAdd(&h[k], v);
    }
    if (tid == 0 && s_drop) atomicAdd(dropped, s_drop);
}

// Tile ranges from the sorted tile ids, 4 ids per thread: a tile starts
// where the id differs from its predecessor and ends where it differs from
// its successor.
__global__ __launch_bounds__(256) void k_tile_ranges(int64_t cap,
                                                     const uint32_t* __restrict__ nd_dev,
                                                     const uint32_t* __restrict__ tiles,
                                                     int64_t num_tiles,
                                                     int2* __restrict__ ranges) {
    const int64_t nd = live_count(cap, nd_dev);
    const int64_t d0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (d0 >= nd) return;
    uint32_t t[6];  // t[0] = predecessor, t[1..4] = own ids, t[5] = successor
    if (d0 + 4 <= nd) {
        const uint4 v = *reinterpret_cast<const uint4*>(tiles + d0);
        t[1] = v.x; t[2] = v.y; t[3] = v.z; t[4] = v.w;
    } else {
        for (int j = 0; j < 4; ++j) t[1 + j] = d0 + j < nd ? tiles[d0 + j] : 0xFFFFFFFFu;
    }
    t[0] = d0 > 0 ? tiles[d0 - 1] : 0xFFFFFFFFu;
    t[5] = d0 + 4 < nd ? tiles[d0 + 4] : 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t d = d0 + j;
        const uint32_t cur = t[1 + j];
        if (d >= nd || cur >= (uint64_t)num_tiles) continue;
        if (d == 0 || t[j] != cur) ranges[cur].x = (int)d;
        if (d == nd - 1 || t[2 + j] != cur) ranges[cur].y = (int)(d + 1);
    }
}

// ------------------------------------------------------------ host side --
inline int bits_for(int64_t count) {
    int b = 0;
    while ((int64_t(1) << b) < count) ++b;
    return b;
}

inline int passes_for(int64_t max_key) {
    return (bits_for(std::max<int64_t>(max_key, 1)) + kRadixBits - 1) / kRadixBits;
}

// misc words: [0..3] depth-pass chunk counters, [4..7] tile-pass counters,
// [8] emit counter, [12..15] status words of gsx_bin_sort, then the digit
// histogram copies of the depth sort and of the tile sort.
constexpr int kMiscCounters = 16;
constexpr int kSyncStatusWord = 12;
constexpr int kMiscWords = kMiscCounters + 2 * kHistCopies * kHistStride;

// Workspace of the depth phase (sized by n alone) and of the tile phase
// (sized by the duplicate capacity); gsx_bin_sort(_async) places the tile
// part right after the depth part of one workspace.
struct DepthLayout {
    size_t dk0, dk1, dv0, dv1, offs, status, misc, total;
    int64_t depth_chunks, scan_chunks, hist_blocks, status_words;
};
struct TileLayout {
    size_t owner, tk0, tk1, tv, status, total;
    int64_t tile_chunks, emit_blocks, status_words;
    int tile_passes;
};

inline size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

struct Taker {
    size_t o = 0;
    size_t operator()(size_t bytes) {
        const size_t at = o;
        o = align_up(o + bytes);
        return at;
    }
};

DepthLayout make_depth_layout(int64_t n) {
    DepthLayout L{};
    Taker take;
    const size_t nn = (size_t)std::max<int64_t>(n, 1);
    L.depth_chunks = ceil_div((int64_t)nn, kDepthThreads * kDepthItems);
    L.scan_chunks = ceil_div((int64_t)nn, kScanChunk);
    L.hist_blocks = ceil_div((int64_t)nn, kHistThreads * hist_items(n));
    L.status_words = 4 * L.depth_chunks * kRadix + L.scan_chunks;
    L.dk0 = take(4 * nn);
    L.dk1 = take(4 * nn);
    L.dv0 = take(4 * nn);
    L.dv1 = take(4 * nn);
    L.offs = take(4 * (nn + 1));
    L.status = take(4 * (size_t)L.status_words);
    L.misc = take(4 * (size_t)kMiscWords);
    L.total = take.o;
    return L;
}

TileLayout make_tile_layout(int64_t cap, int64_t num_tiles) {
    TileLayout L{};
    Taker take;
    const size_t cc = (size_t)std::max<int64_t>(cap, 1);
    L.tile_chunks = ceil_div((int64_t)cc, kTileThreads * kTileItems);
    L.emit_blocks = ceil_div((int64_t)cc, kEmitDups);
    // room for the refine_tiles sentinel id (= num_tiles)
    L.tile_passes = passes_for(num_tiles + 1);
    L.status_words = (int64_t)L.tile_passes * L.tile_chunks * kRadix;
    L.owner = take(4 * (size_t)L.emit_blocks);
    L.tk0 = take(4 * cc);
    L.tk1 = take(4 * cc);
    L.tv = take(4 * cc);
    L.status = take(4 * (size_t)L.status_words);
    L.total = take.o;
    return L;
}

template <typename T>
inline T* at(void* ws, size_t off) {
    return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

inline unsigned grid_for(int64_t n, int64_t per) {
    return (unsigned)std::max<int64_t>(1, ceil_div(n, per));
}

int zero(ZeroRanges z, hipStream_t st) {
    int64_t most = 0;
    for (int r = 0; r < kZeroRanges; ++r) {
        if (!z.p[r]) z.n[r] = 0;
        most = std::max(most, z.n[r]);
    }
    if (most == 0) return GSX_OK;
    const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(most, 256), 4096);
    hipLaunchKernelGGL(k_zero_ranges, dim3(grid), dim3(256), 0, st, z);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int check_args(int64_t n, int32_t width, int32_t height, int64_t capacity) {
    if (n < 0 || width <= 0 || height <= 0 || capacity < 0) return GSX_ERR_INVALID;
    if (width > 0xFFFF * kTile || height > 0xFFFF * kTile) return GSX_ERR_INVALID;
    if (n > (int64_t)kCountMask || capacity > (int64_t)kCountMask) return GSX_ERR_TOO_LARGE;
    return GSX_OK;
}

int count_phase(int64_t n, const uint32_t* tile_counts, const uint32_t* depth_keys,
                int32_t width, int32_t height, void* depth_ws, int64_t depth_ws_bytes,
                int32_t* tile_ranges, uint32_t* bin_status, bool clear_errors,
                hipStream_t st) {
    int rc = check_args(n, width, height, 0);
    if (rc != GSX_OK) return rc;
    if (!tile_ranges || !bin_status) return GSX_ERR_INVALID;
    if (n > 0 && (!tile_counts || !depth_keys || !depth_ws)) return GSX_ERR_INVALID;
    const int64_t T = (int64_t)((width + kTile - 1) / kTile) * ((height + kTile - 1) / kTile);
    const DepthLayout L = make_depth_layout(n);
    if (n > 0 && depth_ws_bytes < (int64_t)L.total) return GSX_ERR_WORKSPACE;
    uint32_t* status = n > 0 ? at<uint32_t>(depth_ws, L.status) : nullptr;
    uint32_t* misc = n > 0 ? at<uint32_t>(depth_ws, L.misc) : nullptr;
    // ranges, the bin_status counts (and, when asked, its error bits),
    // look-back status words, counters and histograms all start at zero
    rc = zero(ZeroRanges{{(uint32_t*)tile_ranges, bin_status + (clear_errors ? 0 : 2),
                          bin_status, status, misc},
                         {2 * T, clear_errors ? 4 : 2, 1, L.status_words, kMiscWords}},
              st);
    if (rc != GSX_OK || n == 0) return rc;
    // digit histograms of the depth keys; the tile counts summed into
    // bin_status[3]
    hipLaunchKernelGGL(k_depth_hist, dim3((unsigned)L.hist_blocks), dim3(kHistThreads), 0, st,
                       depth_keys, tile_counts, n, misc + kMiscCounters, bin_status + 3,
                       bin_status + 1);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // namespace

extern "C" {

int64_t gsx_bin_depth_workspace_bytes(int64_t n) {
    if (n < 0) return -1;
    return (int64_t)make_depth_layout(n).total;
}

int64_t gsx_bin_tile_workspace_bytes(int64_t capacity, int32_t num_tiles) {
    if (capacity < 0 || num_tiles <= 0) return -1;
    return (int64_t)make_tile_layout(capacity, num_tiles).total;
}

int64_t gsx_bin_workspace_bytes(int64_t n, int64_t capacity, int32_t num_tiles) {
    if (n < 0 || capacity < 0 || num_tiles <= 0) return -1;
    return (int64_t)(make_depth_layout(n).total + make_tile_layout(capacity, num_tiles).total);
}

int gsx_bin_count_async(int64_t n, const uint32_t* tile_counts, const uint32_t* depth_keys,
                        int32_t width, int32_t height, void* depth_ws, int64_t depth_ws_bytes,
                        int32_t* tile_ranges, uint32_t* bin_status, void* stream) {
    return count_phase(n, tile_counts, depth_keys, width, height, depth_ws, depth_ws_bytes,
                       tile_ranges, bin_status, false, (hipStream_t)stream);
}

int gsx_bin_depth_async(int64_t n, const uint32_t* depth_keys, void* depth_ws,
                        int64_t depth_ws_bytes, uint32_t* bin_status, void* stream) {
    if (n < 0 || n > (int64_t)kCountMask) return n < 0 ? GSX_ERR_INVALID : GSX_ERR_TOO_LARGE;
    if (!bin_status) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!depth_keys || !depth_ws) return GSX_ERR_INVALID;
    hipStream_t st = (hipStream_t)stream;
    const DepthLayout L = make_depth_layout(n);
    if (depth_ws_bytes < (int64_t)L.total) return GSX_ERR_WORKSPACE;
    uint32_t* status = at<uint32_t>(depth_ws, L.status);
    uint32_t* misc = at<uint32_t>(depth_ws, L.misc);
    uint32_t* depth_hist = misc + kMiscCounters;
    // stable sort of the Gaussians by depth key (index order breaks ties)
    const uint32_t* kin = depth_keys;
    const uint32_t* vin = nullptr;
    uint32_t* kbuf[2] = {at<uint32_t>(depth_ws, L.dk0), at<uint32_t>(depth_ws, L.dk1)};
    uint32_t* vbuf[2] = {at<uint32_t>(depth_ws, L.dv0), at<uint32_t>(depth_ws, L.dv1)};
    for (int p = 0; p < 4; ++p) {
        hipLaunchKernelGGL((k_onesweep<kDepthThreads, kDepthItems>), dim3((unsigned)L.depth_chunks),
                           dim3(kDepthThreads), 0, st, kin, vin, n, (const uint32_t*)nullptr,
                           p * kRadixBits, kRadixBits, depth_hist + p * kRadix,
                           status + (size_t)p * L.depth_chunks * kRadix, misc + p, kbuf[p & 1],
                           vbuf[p & 1], bin_status + 1);
        kin = kbuf[p & 1];
        vin = vbuf[p & 1];
    }
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_bin_tiles_async(int64_t n, const uint32_t* tile_counts, const uint32_t* tile_rects,
                        const float* means2d, const float* conics, int64_t conic_stride,
                        int32_t width, int32_t height, void* depth_ws, int64_t depth_ws_bytes,
                        void* tile_ws, int64_t tile_ws_bytes, int64_t capacity,
                        int32_t* sorted_ids, int32_t* tile_ranges, uint32_t* bin_status,
                        void* stream) {
    int rc = check_args(n, width, height, capacity);
    if (rc != GSX_OK) return rc;
    if (!tile_ranges || !bin_status) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;  // the depth phase cleared the ranges and status
    if (!tile_counts || !tile_rects || !depth_ws || !tile_ws) return GSX_ERR_INVALID;
    const bool refine = conics != nullptr;
    if (refine && (!means2d || ((uintptr_t)means2d & 7u) != 0u || conic_stride < 3))
        return GSX_ERR_INVALID;
    if (capacity > 0 && (!sorted_ids || ((uintptr_t)sorted_ids & 15u) != 0u))
        return GSX_ERR_INVALID;  // emission stores 4 ids at a time
    hipStream_t st = (hipStream_t)stream;
    const int tiles_x = (width + kTile - 1) / kTile;
    const int tiles_y = (height + kTile - 1) / kTile;
    const int64_t T = (int64_t)tiles_x * tiles_y;
    const DepthLayout D = make_depth_layout(n);
    const TileLayout L = make_tile_layout(capacity, T);
    if (depth_ws_bytes < (int64_t)D.total || tile_ws_bytes < (int64_t)L.total)
        return GSX_ERR_WORKSPACE;
    uint32_t* misc = at<uint32_t>(depth_ws, D.misc);
    uint32_t* d_total = bin_status;
    uint32_t* err = bin_status + 1;
    uint32_t* dropped = bin_status + 2;
    uint32_t* tile_hist = misc + kMiscCounters + kHistCopies * kHistStride;
    const uint32_t* gids = at<uint32_t>(depth_ws, D.dv1);  // after the four depth passes

    // scan of the counts in depth order (it also clears the tile passes'
    // status words); emission (+ tile digit histograms) into the buffers
    // from which the tile passes end in sorted_ids; tile sort over the
    // device-side D; ranges
    const int passes = refine ? L.tile_passes : passes_for(T);
    // significant bits of the tile ids (the refine_tiles sentinel T included)
    const int tile_bits = bits_for(std::max<int64_t>(refine ? T + 1 : T, 1));
    uint32_t* tk[2] = {at<uint32_t>(tile_ws, L.tk0), at<uint32_t>(tile_ws, L.tk1)};
    uint32_t* tv[2] = {(uint32_t*)sorted_ids, at<uint32_t>(tile_ws, L.tv)};
    int cur = passes & 1;
    uint32_t* tstatus = at<uint32_t>(tile_ws, L.status);
    uint32_t* sstatus = at<uint32_t>(depth_ws, D.status) + (size_t)4 * D.depth_chunks * kRadix;
    uint32_t* offs = at<uint32_t>(depth_ws, D.offs);
    uint32_t* owner = at<uint32_t>(tile_ws, L.owner);
    hipLaunchKernelGGL(k_count_scan, dim3((unsigned)D.scan_chunks), dim3(kScanThreads), 0, st, n,
                       tile_counts, gids, sstatus, misc + 8, offs, owner, L.emit_blocks, d_total,
                       err, tstatus, L.status_words);
    GSX_LAUNCH_CHECK();
    if (capacity == 0) return GSX_OK;
    hipLaunchKernelGGL(k_emit, dim3((unsigned)L.emit_blocks), dim3(kEmitThreads), 0, st, n,
                       capacity, (const uint32_t*)d_total, (const uint32_t*)offs,
                       (const uint32_t*)owner, gids,
                       (const uint2*)tile_rects, tiles_x, passes, (const float2*)means2d,
                       conics, conic_stride, (int)width, (int)height, (uint32_t)T, dropped,
                       tk[cur], tv[cur], tile_hist);
    GSX_LAUNCH_CHECK();
    for (int p = 0; p < passes; ++p) {
        hipLaunchKernelGGL((k_onesweep<kTileThreads, kTileItems>), dim3((unsigned)L.tile_chunks),
                           dim3(kTileThreads), 0, st, tk[cur], tv[cur], capacity,
                           (const uint32_t*)d_total, p * kRadixBits,
                           std::min(kRadixBits, tile_bits - p * kRadixBits), tile_hist + p * kRadix,
                           tstatus + (size_t)p * L.tile_chunks * kRadix, misc + 4 + p,
                           tk[cur ^ 1], tv[cur ^ 1], err);
        cur ^= 1;
    }
    GSX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_tile_ranges, dim3(grid_for(capacity, 1024)), dim3(256), 0, st, capacity,
                       (const uint32_t*)d_total, tk[cur], T, (int2*)tile_ranges);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_bin_sort_async(int64_t n, const uint32_t* tile_counts, const uint32_t* depth_keys,
                       const uint32_t* tile_rects, const float* means2d, const float* conics,
                       int64_t conic_stride, int32_t width, int32_t height, void* workspace,
                       int64_t workspace_bytes, int64_t capacity, int32_t* sorted_ids,
                       int32_t* tile_ranges, uint32_t* bin_status, void* stream) {
    int rc = check_args(n, width, height, capacity);
    if (rc != GSX_OK) return rc;
    if (!tile_ranges || !bin_status) return GSX_ERR_INVALID;
    if (n > 0 && (!tile_counts || !depth_keys || !tile_rects || !workspace)) return GSX_ERR_INVALID;
    const int64_t T = (int64_t)((width + kTile - 1) / kTile) * ((height + kTile - 1) / kTile);
    const int64_t dbytes = (int64_t)make_depth_layout(n).total;
    const int64_t tbytes = (int64_t)make_tile_layout(capacity, T).total;
    if (n > 0 && workspace_bytes < dbytes + tbytes) return GSX_ERR_WORKSPACE;
    rc = count_phase(n, tile_counts, depth_keys, width, height, workspace, dbytes, tile_ranges,
                     bin_status, true, (hipStream_t)stream);
    if (rc != GSX_OK || n == 0) return rc;
    rc = gsx_bin_depth_async(n, depth_keys, workspace, dbytes, bin_status, stream);
    if (rc != GSX_OK) return rc;
    return gsx_bin_tiles_async(n, tile_counts, tile_rects, means2d, conics, conic_stride, width,
                               height, workspace, dbytes, static_cast<char*>(workspace) + dbytes,
                               tbytes, capacity, sorted_ids, tile_ranges, bin_status, stream);
}

int gsx_bin_status_check(const uint32_t* host_status, int64_t capacity, int64_t* num_dups) {
    if (!host_status || !num_dups) return GSX_ERR_INVALID;
    const int64_t emitted = (int64_t)host_status[0];
    *num_dups = emitted;
    if (host_status[1] & GSX_BIN_ERR_OVERFLOW) return GSX_ERR_TOO_LARGE;
    if (host_status[1] != 0u) return GSX_ERR_DEVICE;
    if (emitted > capacity) return 1;
    *num_dups = emitted - (int64_t)host_status[2];  // refine_tiles drops sort last
    return GSX_OK;
}

int gsx_bin_sort(int64_t n, const uint32_t* tile_counts, const uint32_t* depth_keys,
                 const uint32_t* tile_rects, const float* means2d, const float* conics,
                 int64_t conic_stride, int32_t width, int32_t height, void* workspace,
                 int64_t workspace_bytes, int64_t capacity, int32_t* sorted_ids,
                 int32_t* tile_ranges, int64_t* num_dups, void* stream) {
    if (!num_dups) return GSX_ERR_INVALID;
    *num_dups = 0;
    int rc = check_args(n, width, height, capacity);
    if (rc != GSX_OK) return rc;
    if (!tile_ranges) return GSX_ERR_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (n == 0) {
        const int64_t T = (int64_t)((width + kTile - 1) / kTile) * ((height + kTile - 1) / kTile);
        return zero(ZeroRanges{{(uint32_t*)tile_ranges, nullptr, nullptr, nullptr}, {2 * T, 0, 0, 0}},
                    st);
    }
    if (!workspace) return GSX_ERR_INVALID;
    const int tiles_x = (width + kTile - 1) / kTile;
    const int tiles_y = (height + kTile - 1) / kTile;
    const int64_t need = gsx_bin_workspace_bytes(n, capacity, tiles_x * tiles_y);
    if (workspace_bytes < need) return GSX_ERR_WORKSPACE;
    // the status words sit in the workspace's counter block, past the counters
    // the pipeline uses (it clears the whole block before the first kernel)
    uint32_t* bs = at<uint32_t>(workspace, make_depth_layout(n).misc) + kSyncStatusWord;
    rc = gsx_bin_sort_async(n, tile_counts, depth_keys, tile_rects, means2d, conics,
                            conic_stride, width, height, workspace, workspace_bytes, capacity,
                            sorted_ids, tile_ranges, bs, stream);
    if (rc != GSX_OK) return rc;
    uint32_t host[4] = {0u, 0u, 0u, 0u};
    if (hipMemcpyAsync(host, bs, sizeof(host), hipMemcpyDeviceToHost, st) != hipSuccess)
        return GSX_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return GSX_ERR_HIP;
    return gsx_bin_status_check(host, capacity, num_dups);
}

}  // extern "C"
