// binning.hip -- tile binning (replaces bin_gaussians, splatting/tiles.py:19-182).
//
// The reference builds key = tile*N + rank(depth) and argsorts it
// (tiles.py:166-172).  Here the same order -- tile, then depth, then index --
// is produced depth-first:
//
//   count phase  one read of the N depth keys: the digit histograms of the
//                depth sort, the duplicate count D = sum of the tile counts,
//                and, per tile row, the number of Gaussians whose rectangle
//                covers it and the duplicates they put in it (row
//                histograms, as range adds of +-1 / +-w at the rectangle's
//                first and one-past-last row).
//   depth sort   stable LSD radix sort of the N depth keys in passes of 9,
//                9, 9 and 5 bits; the renderer's keys are relative to the
//                camera's near plane (zero for Gaussians that are not
//                binned), so for every depth below 2^27 float32 ulps past
//                znear (z < ~650 for znear = 0.01) the top pass finds one
//                digit and is skipped on the device.
//   tile phase   (images up to 256 x 256 tiles, refine_tiles off)
//     row scan     exclusive scan of the rectangles' heights in depth order:
//                  each Gaussian's first "row entry" (one per tile row it
//                  covers); the row plan (per-row bases and segment counts)
//                  from the row histograms.
//     row emit     each workgroup expands 4096 row entries of depth-ordered
//                  Gaussians and places them stably by tile row (wave
//                  multi-split ranking, decoupled look-back over the rows),
//                  with each entry's offset in its row's duplicate sequence
//                  (a second look-back column of width sums).
//     seg count    a row's duplicates (its entries expanded left to right,
//                  in depth order) are cut into 2048-duplicate segments;
//                  per segment and tile column, the number of duplicates.
//     tile scan    per row: exclusive prefix over the row's segments of each
//                  column's counts, the tile totals, the tile ranges
//                  [start, start + count) (empty tiles (0,0), as the
//                  scatter-min/max of tiles.py:175-180 leaves them) and each
//                  (segment, column)'s first output position.
//     place        each segment ranks its duplicates by column (stable, in
//                  duplicate order) and writes the Gaussian ids at their
//                  final positions, regrouped in LDS so stores are runs.
//                  No sort pass over the D duplicates is left.
//   tile phase   (larger images or refine_tiles: the general path)
//     count scan of the tile counts in depth order, emission of (tile, id)
//     pairs balanced by duplicates (with the refine_tiles test), stable LSD
//     radix sort of the tile ids, ranges from the sorted ids.
//
// Radix passes are single-kernel "onesweep" passes (Adinets & Merrill,
// 2022): digit histograms come from an earlier read, each pass ranks a chunk
// with wave-level multi-split, publishes its digit counts and finds its
// global offsets by decoupled look-back (Merrill & Garland, 2016), then
// writes the chunk through LDS in digit order so the global stores are runs
// of consecutive addresses.  A chunk is its workgroup's index: workgroups
// are dispatched in index order (round robin over the XCDs, in order on
// each), so the lowest unfinished chunk is always running or next to start
// and only waits for finished chunks -- no claim counter (a same-address
// atomic per workgroup, microseconds under contention) is needed.  Each
// wait is bounded and raises an error flag instead of spinning forever,
// which also covers a dispatcher that did otherwise.  (The general path's
// count scan still claims its chunks through a counter.)
//
// Host status without stream copies: when the caller passes pinned host
// memory, the first depth pass (its workgroup 0, which starts after the
// count phase has finished) writes the status words there as
// (sequence << 32 | word), and so does the last kernel of the tile phase;
// the host polls that memory instead of enqueueing a device-to-host copy
// and an event behind the kernels.
#include <algorithm>
#include <cstring>

#include "gsx_device.h"
#include "tile_order.h"

using namespace gsx;

namespace {

// ------------------------------------------------------------ constants --
constexpr int kRadixBits = 8;  // tile-id passes of the general path
constexpr int kRadix = 1 << kRadixBits;
constexpr int kMaxTilePasses = 4;
// depth sort: 9 + 9 + 9 + 5 bits, 512 threads x 8 keys per chunk
constexpr int kDepthBits = 9;
constexpr int kDepthRadix = 1 << kDepthBits;
constexpr int kDepthPasses = 4;
constexpr int kDepthTopShift = 3 * kDepthBits;       // 27
constexpr int kDepthTopBits = 32 - kDepthTopShift;   // 5
constexpr int kDepthThreads = 512, kDepthItems = 8;
constexpr int kDepthChunk = kDepthThreads * kDepthItems;
// words between histogram copies, pass p at p * kDepthRadix
constexpr int kDepthHistStride = kDepthPasses * kDepthRadix;
// tile sort (general path): 512 x 14 (the largest chunk at which two
// workgroups fit a CU: 124 VGPRs, 65 KB of LDS)
constexpr int kTileThreads = 512, kTileItems = 14;
constexpr int kTileHistStride = kMaxTilePasses * kRadix;
// count phase: 1024 threads x 4 keys (245 workgroups per million keys, so
// every CU takes one)
constexpr int kHistThreads = 1024, kHistItems = 4;
// count / row scans: 1024 threads x 4 Gaussians; emission, row emission,
// segments: 1024 threads x 4
constexpr int kScanThreads = 1024, kScanItems = 4, kScanChunk = kScanThreads * kScanItems;
constexpr int kEmitThreads = 1024, kEmitItems = 4, kEmitDups = kEmitThreads * kEmitItems;
constexpr int kRowChunk = kEmitDups;  // row entries per row-emission workgroup
// placement: 512 threads x 4 duplicates per segment (four workgroups per
// CU: 38 KB of LDS each)
constexpr int kPlaceThreads = 512;
constexpr int kSegDups = kPlaceThreads * kEmitItems;  // duplicates per placement segment
// fast tile path limits: tile rows and columns fit an 8-bit digit
constexpr int kMaxFastTiles = 256;
constexpr int kRowWords = kMaxFastTiles + 1;  // one row histogram (diff form)
// Global histograms are kept in kHistCopies copies (workgroup b adds into
// copy b % kHistCopies): same-address device atomics serialize, so one
// shared copy would cost a serialized update per workgroup per bin.
constexpr int kHistCopies = 16;

// Look-back status word: 2 flag bits | 30-bit count.
constexpr uint32_t kFlagAgg = 1u << 30;
constexpr uint32_t kFlagInc = 2u << 30;
constexpr uint32_t kCountMask = (1u << 30) - 1u;
constexpr uint32_t kSpinLimit = 1u << 16;
constexpr int kStatusWords = 8;  // bin_status words

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Row plan of the fast tile path, written by the row scan's workgroup 0.
struct RowPlan {
    uint32_t rowcnt[kMaxFastTiles];   // Gaussians covering row y
    uint32_t rowdup[kMaxFastTiles];   // duplicates in row y
    uint32_t rowbase[kRowWords];      // first row entry of row y
    uint32_t rowstart[kRowWords];     // first output position of row y
    uint32_t segbase[kRowWords];      // first segment of row y
    uint32_t entries, dups, segments; // totals
    uint32_t pad;
};

// Host status target of one call: the device status words and the pinned
// host words they are copied to, tagged with `seq`.
struct Publish {
    const uint32_t* words;
    unsigned long long* host;
    uint32_t seq;
};

// The words were written by earlier kernels of the stream (a kernel
// boundary makes them visible), so plain loads fetch all eight in one
// round trip.
__device__ __forceinline__ void publish(const Publish& p) {
    uint32_t v[kStatusWords];
#pragma unroll
    for (int k = 0; k < kStatusWords; ++k) v[k] = p.words[k];
#pragma unroll
    for (int k = 0; k < kStatusWords; ++k)
        __hip_atomic_store(p.host + k, ((unsigned long long)p.seq << 32) | v[k], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    __threadfence_system();
}

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

// Two-level look-back for many chunks per column.  Chunks are grouped in
// blocks of kLookBlock; besides its status word (aggregate, then inclusive
// prefix) every chunk writes its aggregate once more into `aggs`, and the
// last chunk of each block publishes the block's status in `bstat`: the sum
// of the block's aggregates as soon as they are all published, then the
// inclusive prefix through the block.  A chunk walks its own block's
// predecessors, then the block statuses, so the prefix of chunk c needs
// about c / (8 kLookBlock) rounds instead of c / 8 when all chunks publish
// together (an inclusive prefix otherwise spreads 8 chunks per round).  The
// in-block reads take the whole block at once (one round trip).
constexpr int kLookBlock = 16;

// Prefix of the column over chunks [base, chunk) of the chunk's block
// (base = its first chunk), stopping at the nearest inclusive one; *done
// when one was found (or the block is the first).
__device__ __forceinline__ uint32_t look_back_in_block(const uint32_t* status, int64_t chunk,
                                                       int stride, int col, uint32_t* err,
                                                       bool* done) {
    const int64_t base = chunk - chunk % kLookBlock;
    uint32_t prefix = 0;
    uint32_t spins = 0;
    int64_t c = chunk - 1;
    *done = base == 0 && chunk == 0;
    while (c >= base) {
        uint32_t s[kLookBlock];
#pragma unroll
        for (int k = 0; k < kLookBlock; ++k)
            s[k] = c - k >= base ? status_load(status + (c - k) * stride + col) : 0u;
        int used = 0;
        bool stalled = false, found = false;
#pragma unroll
        for (int k = 0; k < kLookBlock; ++k) {
            if (found || stalled || c - k < base) continue;
            const uint32_t flag = s[k] & ~kCountMask;
            if (flag == 0u) {
                stalled = true;
                continue;
            }
            prefix += s[k] & kCountMask;
            ++used;
            found = flag == kFlagInc;
        }
        if (found) {
            *done = true;
            break;
        }
        c -= used;
        if (stalled) {
            if (++spins > kSpinLimit) {
                atomicOr(err, GSX_BIN_ERR_LOOKBACK);
                *done = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    // chunk 0 is inclusive: a walk in the first block always ends there
    if (base == 0) *done = true;
    return prefix;
}

// The aggregate of the last chunk's block: its own count plus the
// aggregates the block's other chunks wrote into `aggs` (polled until all
// are there, bounded as above).
__device__ __forceinline__ uint32_t block_aggregate(const uint32_t* aggs, int64_t chunk,
                                                    int stride, int col, uint32_t own,
                                                    uint32_t* err) {
    const int64_t base = chunk - chunk % kLookBlock;
    uint32_t sum = own;
    uint32_t spins = 0;
    for (int64_t c = base; c < chunk;) {
        uint32_t s[kLookBlock];
#pragma unroll
        for (int k = 0; k < kLookBlock; ++k)
            s[k] = c + k < chunk ? status_load(aggs + (c + k) * stride + col) : kFlagAgg;
        int got = 0;
        bool stalled = false;
#pragma unroll
        for (int k = 0; k < kLookBlock; ++k) {
            if (stalled || c + k >= chunk) continue;
            if ((s[k] & ~kCountMask) == 0u) {
                stalled = true;
                continue;
            }
            sum += s[k] & kCountMask;
            ++got;
        }
        c += got;
        if (stalled) {
            if (++spins > kSpinLimit) {
                atomicOr(err, GSX_BIN_ERR_LOOKBACK);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    return sum;
}

// The same for a single counter column (stride 1, column 0), walked by one
// whole wave: each round reads the 64 statuses before the current position
// at once (lane l: chunk c - l) and adds them up to the nearest inclusive
// one, stopping before the first unpublished one (polled again, bounded as
// above).  A lone thread's 8-status window needs ~n/8 round trips for the
// n-th chunk when all chunks start together; the wave needs ~n/64.  Every
// lane of the wave calls it; the result is uniform.
__device__ __forceinline__ uint32_t wave_look_back(const uint32_t* status, int64_t chunk,
                                                   uint32_t* err) {
    const int lane = lane_id();
    uint32_t prefix = 0;
    uint32_t spins = 0;
    int64_t c = chunk - 1;
    while (c >= 0) {
        const int64_t idx = c - lane;  // before chunk 0: an inclusive zero
        const uint32_t s = idx >= 0 ? status_load(status + idx) : kFlagInc;
        const uint32_t flag = s & ~kCountMask;
        const uint64_t pend = __ballot(flag == 0u);
        const uint64_t inc = __ballot(flag == kFlagInc);
        const int first_pend = pend ? __ffsll((unsigned long long)pend) - 1 : kWave;
        const int first_inc = inc ? __ffsll((unsigned long long)inc) - 1 : kWave;
        const bool done = first_inc < first_pend;
        const int take = done ? first_inc + 1 : first_pend;  // lanes [0, take)
        uint32_t v = lane < take ? (s & kCountMask) : 0u;
#pragma unroll
        for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
        prefix += v;
        if (done) break;
        c -= take;
        if (take == 0) {
            if (++spins > kSpinLimit) {
                if (lane == 0) atomicOr(err, GSX_BIN_ERR_LOOKBACK);
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
// significant bits are the low `nbits` (<= BITS, uniform; the others are
// zero in every key).  Per bit, the lanes whose bit differs from this lane's
// are the ballot XOR this lane's bit replicated (a sign-extended bit field),
// and the differing masks are OR-ed: four to five 32-bit operations per bit
// instead of selecting between the ballot and its complement in 64 bits.
template <int BITS>
__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool valid, int nbits) {
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int b = 0; b < BITS; ++b) {
        if (b < nbits) {
            const int s = __builtin_amdgcn_sbfe((int)d, b, 1);  // 0 or -1
            const uint64_t bb = __ballot(s != 0);
            lo |= (uint32_t)bb ^ (uint32_t)s;
            hi |= (uint32_t)(bb >> 32) ^ (uint32_t)s;
        }
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
// must call it; s_w holds THREADS/64 words and is free again on return
// only after the caller's next barrier.
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

// Whether the depth sort's top pass runs: it is skipped (an identity
// permutation) when one of its digits holds all n keys.  Every kernel that
// depends on it takes the same decision from the same histogram; every
// thread of the workgroup must call it.
__device__ __forceinline__ bool top_pass_runs(const uint32_t* __restrict__ depth_hist,
                                              int64_t n) {
    const uint32_t* h = depth_hist + (kDepthPasses - 1) * kDepthRadix;
    bool whole = false;
    const int d = threadIdx.x;
    if (d < (1 << kDepthTopBits)) {
        uint32_t s = 0;
#pragma unroll
        for (int c = 0; c < kHistCopies; ++c) s += h[c * kDepthHistStride + d];
        whole = (int64_t)s == n;
    }
    return !__syncthreads_or(whole);
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

// ------------------------------------------------------------ count phase --
// Digit histograms of the depth keys (10, 10, 10, 2 bits) from one read,
// added into copy blockIdx % kHistCopies; the sum of the tile counts (the
// duplicates) added to status[3] (with the overflow bit past kCountMask)
// and the sum of the rectangle heights (the row entries) to status[4]; with
// rows > 0 the row histograms in difference form: row_diff[copy][0][y] gets
// +1 at each binned Gaussian's first row and -1 one past its last,
// row_diff[copy][1][y] the same weighted by the rectangle's width.  The
// workgroup counts rows in eight LDS copies (lane % 8): the lanes of a
// spatially sorted table share rows, and same-address LDS atomics of a wave
// serialize.
__global__ __launch_bounds__(kHistThreads) void k_depth_hist(
    const uint32_t* __restrict__ keys, const uint32_t* __restrict__ counts,
    const uint2* __restrict__ rects, int64_t n, int rows, uint32_t* __restrict__ hist,
    uint32_t* __restrict__ row_diff, uint32_t* __restrict__ status) {
    constexpr int kHistBins = 3 * kDepthRadix + (1 << kDepthTopBits);
    __shared__ uint32_t s_h[kHistBins];
    constexpr int kRowCopies = 8;
    __shared__ uint32_t s_rows[kRowCopies][2][kRowWords];
    __shared__ uint64_t s_sum[2][kHistThreads / 64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int k = tid; k < kHistBins; k += kHistThreads) s_h[k] = 0u;
    for (int k = tid; k < kRowCopies * 2 * kRowWords; k += kHistThreads) (&s_rows[0][0][0])[k] = 0u;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * (kHistThreads * kHistItems) + wave * (64 * kHistItems);
    uint64_t sum = 0, hsum = 0;
    // every load issued before the histogram work (clamped indices, n >= 1)
    uint32_t kk[kHistItems], cc[kHistItems];
    uint2 rr[kHistItems];
#pragma unroll
    for (int r = 0; r < kHistItems; ++r) {
        const int64_t i = min(base + r * 64 + lane, n - 1);
        kk[r] = keys[i];
        cc[r] = counts[i];
        rr[r] = rects[i];
    }
#pragma unroll
    for (int r = 0; r < kHistItems; ++r) {
        const int64_t i = base + r * 64 + lane;
        const bool valid = i < n;
        const uint32_t key = valid ? kk[r] : 0u;
        const uint32_t cnt = valid ? cc[r] : 0u;
        sum += cnt;
        if (cnt) {
            const uint2 rc = rr[r];
            const uint32_t h = rc.y >> 16;
            hsum += h;
            if (rows > 0 && (rc.x >> 16) + h <= (uint32_t)rows) {
                const uint32_t y0 = rc.x >> 16, w = rc.y & 0xFFFFu;
                uint32_t (*sr)[kRowWords] = s_rows[lane & (kRowCopies - 1)];
                atomicAdd(&sr[0][y0], 1u);
                atomicAdd(&sr[0][y0 + h], 0xFFFFFFFFu);
                atomicAdd(&sr[1][y0], w);
                atomicAdd(&sr[1][y0 + h], 0u - w);
            }
        }
#pragma unroll
        for (int p = 0; p < 3; ++p)
            hist_add(s_h + p * kDepthRadix, (key >> (p * kDepthBits)) & (kDepthRadix - 1), valid);
        hist_add(s_h + 3 * kDepthRadix, key >> kDepthTopShift, valid);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        sum += __shfl_xor(sum, o, 64);
        hsum += __shfl_xor(hsum, o, 64);
    }
    if (lane == 0) {
        s_sum[0][wave] = sum;
        s_sum[1][wave] = hsum;
    }
    __syncthreads();
    if (tid < 2) {
        uint64_t t = 0;
#pragma unroll
        for (int w = 0; w < kHistThreads / 64; ++w) t += s_sum[tid][w];
        if (t > 0) {
            // each add is at most 2^30, so the word cannot wrap before the
            // overflow bit is set
            uint32_t* word = status + (tid == 0 ? 3 : 4);
            const uint32_t add = (uint32_t)(t > kCountMask ? kCountMask + 1u : t);
            const uint32_t old = atomicAdd(word, add);
            if ((uint64_t)old + add > kCountMask) atomicOr(status + 1, GSX_BIN_ERR_OVERFLOW);
        }
    }
    const int copy = blockIdx.x % kHistCopies;
    uint32_t* h = hist + copy * kDepthHistStride;
    for (int k = tid; k < kHistBins; k += kHistThreads) {
        const uint32_t v = s_h[k];
        if (v) atomicAdd(&h[k], v);
    }
    if (rows > 0) {
        uint32_t* rd = row_diff + copy * 2 * kRowWords;
        for (int k = tid; k < 2 * kRowWords; k += kHistThreads) {
            uint32_t v = 0u;
#pragma unroll
            for (int c = 0; c < kRowCopies; ++c) v += (&s_rows[c][0][0])[k];
            if (v) atomicAdd(&rd[k], v);
        }
    }
}

// ------------------------------------------------------------ radix pass --
// One stable LSD pass over the BITS-bit digit at `shift` (`nbits`
// significant).  Chunk c (workgroup c) holds keys
// [c * chunk, (c + 1) * chunk); wave w of it owns a contiguous slice, ranked
// round by round, so the order is stable.  The chunk is regrouped by digit
// in LDS, then written out: element j of the regrouped chunk goes to
// global_base[digit] + j - chunk_base[digit].  `hist` points at this pass's
// histogram in copy 0 (copies hist_stride words apart).  vals_in == nullptr
// means "values are the element indices".  With skip_constant, a pass whose
// digit is the same for all n keys returns at once (its output buffers are
// not written).  With route_hist (the depth histograms), the output goes to
// (keys_alt, vals_alt) when the depth sort's top pass will be skipped, so
// the sorted order always ends in the same buffers.  With pub.host,
// workgroup 0 copies the status words to the host first.
template <int THREADS, int ITEMS, int BITS>
__global__ __launch_bounds__(THREADS) void k_onesweep(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n_host,
    const uint32_t* __restrict__ n_dev, int shift, int nbits, const uint32_t* __restrict__ hist,
    int hist_stride, bool skip_constant, uint32_t* __restrict__ status,
    uint32_t* __restrict__ aggs, uint32_t* __restrict__ bstat, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, uint32_t* __restrict__ err, Publish pub,
    const uint32_t* __restrict__ route_hist, uint32_t* __restrict__ keys_alt,
    uint32_t* __restrict__ vals_alt) {
    constexpr int kWaves = THREADS / 64;
    constexpr int kChunk = THREADS * ITEMS;
    constexpr int kR = 1 << BITS;
    constexpr int kBPT = kR > THREADS ? kR / THREADS : 1;  // digits per thread
    static_assert(kR <= THREADS || kR % THREADS == 0, "digits split evenly over threads");
    __shared__ uint32_t s_cnt[kWaves][kR];
    __shared__ uint32_t s_dexcl[kR];
    __shared__ uint32_t s_shift[kR];
    __shared__ uint32_t s_w[2 * kWaves];
    __shared__ uint32_t s_key[kChunk], s_val[kChunk];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (pub.host && blockIdx.x == 0 && tid == 0) publish(pub);
    const int64_t n = live_count(n_host, n_dev);
    // The first ceil(n / chunk) workgroups are the live chunks; the rest
    // leave at once.
    if ((int64_t)blockIdx.x * kChunk >= n) return;
    // digit totals over the histogram copies (the copies' loads issue
    // together, one round trip)
    uint32_t dsum[kBPT];
    auto digit_totals = [&]() {
#pragma unroll
        for (int k = 0; k < kBPT; ++k) {
            const int b = tid * kBPT + k;
            uint32_t s = 0;
            if (b < kR) {
                uint32_t v[kHistCopies];
#pragma unroll
                for (int c = 0; c < kHistCopies; ++c) v[c] = hist[c * hist_stride + b];
#pragma unroll
                for (int c = 0; c < kHistCopies; ++c) s += v[c];
            }
            dsum[k] = s;
        }
    };
    if (skip_constant) {
        digit_totals();
        bool whole = false;
#pragma unroll
        for (int k = 0; k < kBPT; ++k) whole |= (int64_t)dsum[k] == n;
        if (__syncthreads_or(whole)) return;  // identity permutation
    }
    for (int k = tid; k < kWaves * kR; k += THREADS) (&s_cnt[0][0])[k] = 0u;
    const int64_t chunk = blockIdx.x;
    const int64_t base = chunk * kChunk + wave * (64 * ITEMS);
    const uint64_t lt = (1ull << lane) - 1ull;
    uint32_t key[ITEMS], val[ITEMS], rank[ITEMS];
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        const int64_t i = base + r * 64 + lane;
        key[r] = i < n ? keys_in[i] : 0u;
        val[r] = i < n ? (vals_in ? vals_in[i] : (uint32_t)i) : 0u;
    }
    // without the skip test the totals are first needed after the ranking:
    // their loads go out behind the keys'
    if (!skip_constant) digit_totals();
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        const bool valid = base + r * 64 + lane < n;
        const uint32_t d = (key[r] >> shift) & (kR - 1);
        const uint64_t m = match_digit<BITS>(d, valid, nbits);
        const uint32_t before = s_cnt[wave][d];
        rank[r] = before + (uint32_t)__popcll(m & lt);
        if (valid && (m & lt) == 0ull) s_cnt[wave][d] = before + (uint32_t)__popcll(m);
    }
    __syncthreads();
    uint32_t local[kBPT];
    uint32_t lsum = 0, dtot = 0;
#pragma unroll
    for (int k = 0; k < kBPT; ++k) {
        const int b = tid * kBPT + k;
        uint32_t acc = 0;
        if (b < kR) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const uint32_t c = s_cnt[w][b];
                s_cnt[w][b] = acc;
                acc += c;
            }
            // a digit no key of the pass holds (zero in the histogram) is
            // never looked up: no status, no look-back
            if (dsum[k] != 0u) {
                status_store(status + chunk * kR + b, (chunk == 0 ? kFlagInc : kFlagAgg) | acc);
                if (bstat) status_store(aggs + chunk * kR + b, kFlagAgg | acc);
            }
        }
        local[k] = acc;
        lsum += acc;
        dtot += dsum[k];
    }
    // in-chunk digit offsets and global digit bases
    uint32_t dexcl0, dbase0;
    block_excl_scan2<THREADS>(lsum, dtot, s_w, &dexcl0, &dbase0);
    uint32_t dexcl[kBPT], dbase[kBPT];
#pragma unroll
    for (int k = 0; k < kBPT; ++k) {
        dexcl[k] = dexcl0;
        dbase[k] = dbase0;
        dexcl0 += local[k];
        dbase0 += dsum[k];
        const int b = tid * kBPT + k;
        if (b < kR) s_dexcl[b] = dexcl[k];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        if (base + r * 64 + lane < n) {
            const uint32_t d = (key[r] >> shift) & (kR - 1);
            const uint32_t j = s_dexcl[d] + s_cnt[wave][d] + rank[r];
            s_key[j] = key[r];
            s_val[j] = val[r];
        }
    }
#pragma unroll
    for (int k = 0; k < kBPT; ++k) {
        const int b = tid * kBPT + k;
        if (b < kR) {
            uint32_t prefix = 0;
            if (dsum[k] != 0u && bstat) {
                // two levels: the block's last chunk publishes the block's
                // aggregate first, its inclusive prefix after the walk
                const int64_t blk = chunk / kLookBlock;
                const bool last = chunk % kLookBlock == kLookBlock - 1;
                if (last)
                    status_store(bstat + blk * kR + b,
                                 (blk == 0 ? kFlagInc : kFlagAgg) |
                                     (block_aggregate(aggs, chunk, kR, b, local[k], err) &
                                      kCountMask));
                bool done;
                prefix = look_back_in_block(status, chunk, kR, b, err, &done);
                if (!done) prefix += look_back(bstat, blk, kR, b, err);
                if (chunk > 0)
                    status_store(status + chunk * kR + b,
                                 kFlagInc | ((prefix + local[k]) & kCountMask));
                if (last && blk > 0)
                    status_store(bstat + blk * kR + b,
                                 kFlagInc | ((prefix + local[k]) & kCountMask));
            } else if (chunk > 0 && dsum[k] != 0u) {
                prefix = look_back(status, chunk, kR, b, err);
                status_store(status + chunk * kR + b, kFlagInc | ((prefix + local[k]) & kCountMask));
            }
            s_shift[b] = dbase[k] + prefix - dexcl[k];  // modular: + j >= dexcl below
        }
    }
    __syncthreads();
    const int cnt = (int)min<int64_t>(kChunk, n - chunk * kChunk);
    if (route_hist && !top_pass_runs(route_hist, n)) {  // uniform (all threads call it)
        keys_out = keys_alt;
        vals_out = vals_alt;
    }
    for (int j = tid; j < cnt; j += THREADS) {
        const uint32_t k = s_key[j];
        const uint32_t pos = s_shift[(k >> shift) & (kR - 1)] + (uint32_t)j;
        if (pos < (uint64_t)n) {  // always true for a consistent histogram
            keys_out[pos] = k;
            vals_out[pos] = s_val[j];
        }
    }
}

// ------------------------------------------------------- fast tile phase --
// The row plan (workgroup-wide; every thread calls it): row histograms from
// their difference form (summed over the copies, then prefix-summed over
// the rows), then the exclusive scans of the row entries, the duplicates
// and the segments; the row of every segment; status[0] = D.
__device__ __forceinline__ void row_plan(const uint32_t* __restrict__ row_diff, int tiles_y,
                                         RowPlan* __restrict__ plan,
                                         uint32_t* __restrict__ segrow, int64_t max_segs,
                                         uint32_t* __restrict__ status, uint32_t* s_w) {
    const int tid = threadIdx.x;
    uint32_t dc = 0, dw = 0;
    if (tid < tiles_y) {  // the 32 loads issued together
#pragma unroll
        for (int c = 0; c < kHistCopies; ++c) {
            dc += row_diff[c * 2 * kRowWords + tid];
            dw += row_diff[c * 2 * kRowWords + kRowWords + tid];
        }
    }
    uint32_t tot;
    const uint32_t cnt = block_excl_scan<kScanThreads>(dc, s_w, &tot) + dc;
    __syncthreads();
    const uint32_t dup = block_excl_scan<kScanThreads>(dw, s_w, &tot) + dw;
    __syncthreads();
    const uint32_t segs = tid < tiles_y ? (uint32_t)ceil_div(dup, kSegDups) : 0u;
    uint32_t ent_tot, dup_tot, seg_tot;
    const uint32_t eb = block_excl_scan<kScanThreads>(tid < tiles_y ? cnt : 0u, s_w, &ent_tot);
    __syncthreads();
    const uint32_t db = block_excl_scan<kScanThreads>(tid < tiles_y ? dup : 0u, s_w, &dup_tot);
    __syncthreads();
    const uint32_t sb = block_excl_scan<kScanThreads>(segs, s_w, &seg_tot);
    __shared__ uint32_t s_sb[kMaxFastTiles + 1];  // segment base of each row
    if (tid < tiles_y) {
        plan->rowcnt[tid] = cnt;
        plan->rowdup[tid] = dup;
        s_sb[tid] = sb;
    }
    if (tid == 0) s_sb[tiles_y] = seg_tot;
    __syncthreads();
    // the row of every segment, spread over the workgroup: the last row
    // whose segment base is <= k (rows without segments share a base with
    // the next row, so the search takes the last of equal bases)
    for (uint32_t k = tid; k < seg_tot && (int64_t)k < max_segs; k += kScanThreads) {
        int lo = 0, hi = tiles_y - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_sb[mid] <= k) lo = mid;
            else hi = mid - 1;
        }
        segrow[k] = (uint32_t)lo;
    }
    if (tid <= tiles_y) {
        plan->rowbase[tid] = eb;
        plan->rowstart[tid] = db;
        plan->segbase[tid] = sb;
    }
    if (tid == 0) {
        plan->entries = ent_tot;
        plan->dups = dup_tot;
        plan->segments = seg_tot;
        status[0] = dup_tot;
    }
}

// Exclusive scan of the rectangles' heights (row entries) in depth order:
// roffs[i] = row entries of depth-ordered Gaussians 0..i-1, roffs[n] = the
// total; owner[b] for every row-emission workgroup b that has entries: the
// depth-ordered Gaussian that owns entry b * kRowChunk.  (Rectangles of
// Gaussians with a zero count are (0, 0): height 0.)  The grid has one
// workgroup more than chunks: the last one writes the row plan from the row
// histograms (the count phase's, so it starts at once, beside the scan),
// the row of every segment (segrow) and status[0] = D; the row emission,
// launched after this kernel, is its first reader.
__global__ __launch_bounds__(kScanThreads) void k_row_scan(
    int64_t n, const uint2* __restrict__ rects, const uint32_t* __restrict__ gids,
    uint32_t* __restrict__ sstatus, uint32_t* __restrict__ roffs, uint32_t* __restrict__ prect,
    uint32_t* __restrict__ owner, int64_t n_owner, uint32_t* __restrict__ status,
    uint32_t* __restrict__ clear, int64_t n_clear, const uint32_t* __restrict__ row_diff,
    int tiles_y, RowPlan* __restrict__ plan, uint32_t* __restrict__ segrow, int64_t max_segs) {
    __shared__ uint32_t s_w[kScanThreads / 64];
    __shared__ uint32_t s_prefix;
    const int tid = threadIdx.x;
    uint32_t* err = status + 1;
    // the row emission's look-back status words start at zero (those of
    // the chunks the row entries -- status[4], final since the count
    // phase -- will use)
    const int64_t used = min<int64_t>(n_clear, ceil_div((int64_t)status[4], kRowChunk) *
                                                   (2 * kMaxFastTiles));
    for (int64_t k = (int64_t)blockIdx.x * kScanThreads + tid; k < used;
         k += (int64_t)gridDim.x * kScanThreads)
        clear[k] = 0u;
    const int64_t nchunks = ceil_div(n, kScanChunk);
    if (blockIdx.x == gridDim.x - 1) {  // the row plan's workgroup
        row_plan(row_diff, tiles_y, plan, segrow, max_segs, status, s_w);
        return;
    }
    const int64_t chunk = blockIdx.x;  // the other workgroups are exactly nchunks
    if (chunk < nchunks) {
        const int64_t i0 = chunk * kScanChunk + (int64_t)tid * kScanItems;
        // clamped indices, so the id loads and then the rectangle loads
        // issue together (n >= 1 here); items past n count zero
        uint32_t g[kScanItems], c[kScanItems];
        uint2 rc[kScanItems];
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) g[j] = gids[min(i0 + j, n - 1)];
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) rc[j] = rects[g[j]];
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) {
            c[j] = i0 + j < n ? rc[j].y >> 16 : 0u;
            // the rectangle packed into one word for the row emission:
            // x0 | y0 << 8 | (w - 1) << 16 (every field below 256)
            if (i0 + j < n)
                prect[i0 + j] = (rc[j].x & 0xFFu) | (((rc[j].x >> 16) & 0xFFu) << 8) |
                                ((((rc[j].y & 0xFFFFu) - 1u) & 0xFFu) << 16);
        }
        uint32_t total;
        uint32_t csum = 0;
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) csum += c[j];
        const uint32_t excl = block_excl_scan<kScanThreads>(csum, s_w, &total);
        if (tid < kWave) {  // wave 0 walks the look-back
            uint32_t prefix = 0;
            uint32_t* st = sstatus + chunk;
            if (chunk == 0) {
                if (tid == 0) status_store(st, kFlagInc | (total & kCountMask));
            } else {
                if (tid == 0) status_store(st, kFlagAgg | (total & kCountMask));
                prefix = wave_look_back(sstatus, chunk, err);
                if (tid == 0) status_store(st, kFlagInc | ((prefix + total) & kCountMask));
            }
            if (tid == 0) {
                s_prefix = prefix;
                if (chunk == nchunks - 1) roffs[n] = prefix + total;
            }
        }
        __syncthreads();
        uint32_t run = s_prefix + excl;
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) {
            if (i0 + j < n) {
                roffs[i0 + j] = run;
                for (int64_t b = ceil_div((int64_t)run, kRowChunk);
                     b * kRowChunk < (int64_t)run + c[j] && b < n_owner; ++b)
                    owner[b] = (uint32_t)(i0 + j);
            }
            run += c[j];
        }
    }
}

// Row emission: 4096 row entries per workgroup (of the plan's total, which
// the caller's capacity must cover, or nothing is written).  Entry r belongs
// to the depth-ordered Gaussian o with roffs[o] <= r < roffs[o + 1] and is
// its (r - roffs[o])-th row.  Entries are ranked by row (stable), placed at
// rowbase[row] + (earlier chunks' entries of that row, by look-back) + rank,
// and written as the Gaussian id, the packed column span (x0 | (w - 1) << 8)
// and the entry's first duplicate within its row's duplicate sequence (the
// widths of the row's earlier entries, a second look-back column).  The
// entry holding a segment's first duplicate records itself in segk0.
// Two workgroups per CU (eight waves per SIMD: at most 64 VGPRs), so all
// 512 chunk slots are resident at once.
__global__ __launch_bounds__(kEmitThreads, 8) void k_row_emit(
    int64_t n, int64_t cap, const uint32_t* __restrict__ roffs, const uint32_t* __restrict__ owner,
    const uint32_t* __restrict__ gids, const uint32_t* __restrict__ prect,
    const RowPlan* __restrict__ plan, int tiles_y, uint32_t* __restrict__ rstatus,
    uint32_t* __restrict__ e_gid, uint32_t* __restrict__ e_pack,
    uint32_t* __restrict__ e_doff, uint32_t* __restrict__ segk0, int64_t max_segs,
    uint32_t* __restrict__ err) {
    constexpr int kWaves = kEmitThreads / 64;
    constexpr int kCols = 2 * kMaxFastTiles;  // count and width-sum columns
    // staging (offset, id, packed rectangle per owner) and the slot owners;
    // after the ranking the first three blocks hold the regrouped (id, pack,
    // width prefix) per entry
    __shared__ uint32_t s_buf[3 * kRowChunk];
    __shared__ uint16_t s_own[kRowChunk];
    __shared__ uint32_t s_cnt[kWaves][kMaxFastTiles];
    __shared__ uint32_t s_dexcl[kMaxFastTiles + 1];
    __shared__ uint32_t s_local[kMaxFastTiles];
    __shared__ uint32_t s_shift[kMaxFastTiles], s_wshift[kMaxFastTiles];
    __shared__ uint32_t s_row[kMaxFastTiles];  // rowbase
    __shared__ uint32_t s_seg[kMaxFastTiles];  // segbase
    __shared__ uint32_t s_w[2 * kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the duplicates (and so the row entries) do not fit: nothing is written
    if ((int64_t)plan->dups > cap || (int64_t)plan->entries > cap) return;
    const int64_t nr = (int64_t)plan->entries;
    const int64_t chunk = blockIdx.x;
    const int64_t r0 = chunk * kRowChunk;
    if (r0 >= nr) return;
    const int64_t r1 = min<int64_t>(r0 + kRowChunk, nr);
    // owner of the first entry, and a bound on the owner of the last (the
    // loads issue beside the plan's)
    const int64_t lo = owner[chunk];
    const int64_t hi = r1 < nr ? (int64_t)owner[chunk + 1]
                               : block_find_owner<kEmitThreads>(roffs, n, (uint32_t)(r1 - 1));
    for (int k = tid; k < kWaves * kMaxFastTiles; k += kEmitThreads) (&s_cnt[0][0])[k] = 0u;
    if (tid < kMaxFastTiles) {
        s_row[tid] = tid < tiles_y ? plan->rowbase[tid] : 0u;
        s_seg[tid] = tid < tiles_y ? plan->segbase[tid] : 0u;
    }
    __syncthreads();
    const int64_t wo = hi - lo + 1;
    const bool staged = wo <= kRowChunk;  // uniform
    // a rectangle of the fast path packs into one word: x0 | y0 << 8 |
    // (w - 1) << 16 (every field below 256)
    uint32_t* s_off = s_buf;
    uint32_t* s_gid = s_buf + kRowChunk;
    uint32_t* s_rect = s_buf + 2 * kRowChunk;
    if (staged) {
        // slot owners: staged owner k holds the chunk's entries
        // [max(roffs[k], r0), min(roffs[k + 1], r1)) (its height from the
        // next offset; roffs has n + 1 words); the spans are disjoint and
        // cover the chunk, so each slot is written once
        for (int k = tid; k < wo; k += kEmitThreads) {
            const uint32_t g = gids[lo + k];
            const uint32_t off = roffs[lo + k];
            const uint32_t end = roffs[lo + k + 1];
            s_off[k] = off;
            s_gid[k] = g;
            s_rect[k] = prect[lo + k];
            for (uint32_t x = max(off, (uint32_t)r0); x < min(end, (uint32_t)r1); ++x)
                s_own[x - (uint32_t)r0] = (uint16_t)k;
        }
    }
    __syncthreads();
    // item r of a thread is entry r0 + wave * 256 + r * 64 + lane (the
    // ranking order)
    const int64_t base = r0 + wave * (64 * kEmitItems);
    const uint64_t lt = (1ull << lane) - 1ull;
    const int ybits = 32 - __builtin_clz((uint32_t)max(tiles_y - 1, 1));
    uint32_t yy[kEmitItems], gg[kEmitItems], pk[kEmitItems], rank[kEmitItems];
#pragma unroll
    for (int r = 0; r < kEmitItems; ++r) {
        const int64_t e = base + r * 64 + lane;
        yy[r] = 0u;
        gg[r] = 0u;
        pk[r] = 0u;
        if (e < r1) {
            uint32_t off, g, rc;
            if (staged) {
                const uint32_t o = s_own[e - r0];
                off = s_off[o];
                g = s_gid[o];
                rc = s_rect[o];
            } else {
                int64_t a = lo, b = hi;
                while (a < b) {
                    const int64_t mid = (a + b + 1) >> 1;
                    if (roffs[mid] <= (uint32_t)e) a = mid;
                    else b = mid - 1;
                }
                off = roffs[a];
                g = gids[a];
                rc = prect[a];
            }
            yy[r] = (((rc >> 8) & 0xFFu) + ((uint32_t)e - off)) & 0xFFu;
            gg[r] = g;
            pk[r] = (rc & 0xFFu) | (((rc >> 16) & 0xFFu) << 8);
        }
    }
#pragma unroll
    for (int r = 0; r < kEmitItems; ++r) {
        const bool valid = base + r * 64 + lane < r1;
        const uint64_t m = match_digit<8>(yy[r], valid, ybits);
        const uint32_t before = s_cnt[wave][yy[r]];
        rank[r] = before + (uint32_t)__popcll(m & lt);
        if (valid && (m & lt) == 0ull) s_cnt[wave][yy[r]] = before + (uint32_t)__popcll(m);
    }
    __syncthreads();  // the staging words are free from here on
    uint32_t local = 0;
    if (tid < kMaxFastTiles) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t c = s_cnt[w][tid];
            s_cnt[w][tid] = local;
            local += c;
        }
        s_local[tid] = local;
    }
    uint32_t tot;
    const uint32_t dexcl = block_excl_scan<kEmitThreads>(tid < kMaxFastTiles ? local : 0u, s_w, &tot);
    if (tid < kMaxFastTiles) s_dexcl[tid] = dexcl;
    if (tid == 0) s_dexcl[kMaxFastTiles] = tot;
    __syncthreads();
    uint32_t* q_gid = s_buf;
    uint32_t* q_pack = s_buf + kRowChunk;
    uint32_t* q_wpre = s_buf + 2 * kRowChunk;
#pragma unroll
    for (int r = 0; r < kEmitItems; ++r) {
        if (base + r * 64 + lane < r1) {
            const uint32_t j = s_dexcl[yy[r]] + s_cnt[wave][yy[r]] + rank[r];
            q_gid[j] = gg[r];
            q_pack[j] = pk[r] | (yy[r] << 16);
            q_wpre[j] = ((pk[r] >> 8) & 0xFFu) + 1u;  // the width
        }
    }
    __syncthreads();
    // exclusive prefix of the widths over the regrouped chunk (4 per thread)
    const int cnt = (int)(r1 - r0);
    uint32_t wv[4], ws = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int j = tid * 4 + k;
        wv[k] = j < cnt ? q_wpre[j] : 0u;
        ws += wv[k];
    }
    uint32_t wtot;
    uint32_t wrun = block_excl_scan<kEmitThreads>(ws, s_w, &wtot);
    __syncthreads();  // every thread has read its widths
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        q_wpre[tid * 4 + k] = wrun;
        wrun += wv[k];
    }
    __syncthreads();
    // publish this chunk's per-row entry counts (columns 0..255) and width
    // sums (columns 256..511), then look back over earlier chunks
    uint32_t* st = rstatus + chunk * kCols;
    uint32_t mine = 0;
    int col = -1;
    if (tid < kMaxFastTiles) {
        col = tid;
        mine = s_local[tid];
    } else if (tid < 2 * kMaxFastTiles) {
        const int y = tid - kMaxFastTiles;
        const uint32_t a = s_dexcl[y], b = s_dexcl[y + 1];
        const uint32_t pa = a < (uint32_t)cnt ? q_wpre[a] : wtot;
        const uint32_t pb = b < (uint32_t)cnt ? q_wpre[b] : wtot;
        col = tid;
        mine = pb - pa;
    }
    if (col >= 0) {
        uint32_t prefix = 0;
        if (chunk == 0) {
            status_store(st + col, kFlagInc | mine);
        } else {
            status_store(st + col, kFlagAgg | mine);
            prefix = look_back(rstatus, chunk, kCols, col, err);
            status_store(st + col, kFlagInc | ((prefix + mine) & kCountMask));
        }
        if (tid < kMaxFastTiles) {
            s_shift[tid] = s_row[tid] + prefix - s_dexcl[tid];
        } else {
            const int y = tid - kMaxFastTiles;
            const uint32_t a = s_dexcl[y];
            const uint32_t pa = a < (uint32_t)cnt ? q_wpre[a] : wtot;
            s_wshift[y] = prefix - pa;
        }
    }
    __syncthreads();
    for (int j = tid; j < cnt; j += kEmitThreads) {
        const uint32_t p = q_pack[j];
        const uint32_t y = p >> 16;
        const uint32_t pos = s_shift[y] + (uint32_t)j;
        if (pos < (uint64_t)nr) {  // always true for a consistent plan
            const uint32_t doff = s_wshift[y] + q_wpre[j];
            const uint32_t w = ((p >> 8) & 0xFFu) + 1u;
            e_gid[pos] = q_gid[j];
            e_pack[pos] = p & 0xFFFFu;
            e_doff[pos] = doff;
            // the segments whose first duplicate this entry holds
            for (uint32_t sgi = (uint32_t)ceil_div(doff, kSegDups); sgi * kSegDups < doff + w; ++sgi) {
                const int64_t b = (int64_t)s_seg[y] + sgi;
                if (b < max_segs) segk0[b] = pos - s_row[y];
            }
        }
    }
}

// The segment of a fast-path workgroup: its row y, its first duplicate a
// and end e within the row's duplicate sequence, the row's entries
// [rb, rb + rc) and the segment's entries [k0, k1) within them (k0 holds
// duplicate a; entries from k1 - 1 on may start at or after e and are
// skipped).  Returns false for workgroups past the last segment.
struct Segment {
    uint32_t a, e, rb, k0, k1;
    int y;
};

__device__ __forceinline__ bool find_segment(const RowPlan* __restrict__ plan,
                                             const uint32_t* __restrict__ segrow,
                                             const uint32_t* __restrict__ segk0, int64_t b,
                                             Segment& s) {
    if (b >= (int64_t)plan->segments) return false;
    const int y = (int)segrow[b];
    const uint32_t sb = plan->segbase[y], se = plan->segbase[y + 1];
    const uint32_t rc = plan->rowcnt[y];
    s.y = y;
    s.a = (uint32_t)(b - sb) * kSegDups;
    s.e = min(s.a + (uint32_t)kSegDups, plan->rowdup[y]);
    s.rb = plan->rowbase[y];
    s.k0 = segk0[b];
    s.k1 = (uint32_t)(b + 1) < se ? min(segk0[b + 1] + 1u, rc) : rc;
    return true;
}

// Per segment and tile column: the number of its duplicates (range adds
// over the columns its entries' clipped spans cover, then a prefix sum).
// One thread per column.
__global__ __launch_bounds__(kMaxFastTiles) void k_seg_count(
    int64_t cap, const RowPlan* __restrict__ plan, const uint32_t* __restrict__ segrow,
    const uint32_t* __restrict__ segk0, int tiles_x, const uint32_t* __restrict__ e_pack,
    const uint32_t* __restrict__ e_doff, uint32_t* __restrict__ sc) {
    __shared__ uint32_t s_diff[kMaxFastTiles + 1];
    __shared__ uint32_t s_w[kMaxFastTiles / 64];
    const int tid = threadIdx.x;
    if ((int64_t)plan->dups > cap) return;
    Segment sg;
    if (!find_segment(plan, segrow, segk0, blockIdx.x, sg)) return;
    s_diff[tid] = 0u;
    if (tid == 0) s_diff[kMaxFastTiles] = 0u;
    __syncthreads();
    // four entries per thread per round, their loads issued together
    // (clamped to the segment's last entry, masked after)
    constexpr int kBatch = 4;
    for (uint32_t k0 = sg.k0 + tid; k0 < sg.k1; k0 += kBatch * kMaxFastTiles) {
        uint32_t dv[kBatch], pv[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const uint32_t k = min(k0 + i * kMaxFastTiles, sg.k1 - 1u);
            dv[i] = e_doff[sg.rb + k];
            pv[i] = e_pack[sg.rb + k];
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const uint32_t doff = dv[i];
            if (k0 + i * kMaxFastTiles >= sg.k1 || doff >= sg.e) continue;
            const uint32_t p = pv[i];
            const uint32_t x0 = p & 0xFFu, w = ((p >> 8) & 0xFFu) + 1u;
            const uint32_t from = max(sg.a, doff) - doff;
            const uint32_t to = min(sg.e, doff + w) - doff;
            atomicAdd(&s_diff[min(x0 + from, (uint32_t)kMaxFastTiles)], 1u);
            atomicAdd(&s_diff[min(x0 + to, (uint32_t)kMaxFastTiles)], 0xFFFFFFFFu);
        }
    }
    __syncthreads();
    uint32_t tot;
    const uint32_t v = s_diff[tid];
    const uint32_t incl = block_excl_scan<kMaxFastTiles>(v, s_w, &tot) + v;
    if (tid < tiles_x) sc[(int64_t)blockIdx.x * kMaxFastTiles + tid] = incl;
}

// Per tile row (one workgroup; four threads per column, each over a
// quarter of the row's segments): exclusive prefix of each column's counts
// over the row's segments, the tile totals and their exclusive scan along
// the row from the row's first output position, the tile ranges, and
// sc[segment][x] = the segment's first output position for column x.
constexpr int kScanParts = 4;
__global__ __launch_bounds__(kScanParts * kMaxFastTiles) void k_tile_scan(
    int64_t cap, const RowPlan* __restrict__ plan, int tiles_x, uint32_t* __restrict__ sc,
    int2* __restrict__ ranges) {
    constexpr int kBatch = 8;
    __shared__ uint32_t s_part[kScanParts][kMaxFastTiles];
    __shared__ uint32_t s_start[kMaxFastTiles];
    __shared__ uint32_t s_w[kScanParts * kMaxFastTiles / 64];
    const int tid = threadIdx.x;
    const int x = tid % kMaxFastTiles, q = tid / kMaxFastTiles;
    if ((int64_t)plan->dups > cap) return;  // ranges stay zero
    const int y = blockIdx.x;
    const uint32_t r0 = plan->segbase[y], r1 = plan->segbase[y + 1];
    const uint32_t per = (r1 - r0 + kScanParts - 1) / kScanParts;
    const uint32_t s0 = min(r0 + q * per, r1), s1 = min(s0 + per, r1);
    const bool col = x < tiles_x;
    uint32_t sum = 0;
    if (col) {
        for (uint32_t s = s0; s < s1; s += kBatch) {
            uint32_t v[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k)  // clamped: the loads issue together
                v[k] = sc[(int64_t)min(s + k, s1 - 1u) * kMaxFastTiles + x];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) sum += s + k < s1 ? v[k] : 0u;
        }
    }
    s_part[q][x] = sum;
    __syncthreads();
    uint32_t total = 0, before = 0;
#pragma unroll
    for (int k = 0; k < kScanParts; ++k) {
        const uint32_t t = s_part[k][x];
        if (k < q) before += t;
        total += t;
    }
    uint32_t tot;
    const uint32_t ex = block_excl_scan<kScanParts * kMaxFastTiles>(
        q == 0 && col ? total : 0u, s_w, &tot);
    if (q == 0) {
        const uint32_t start = plan->rowstart[y] + ex;
        s_start[x] = start;
        if (col)
            ranges[(int64_t)y * tiles_x + x] =
                total ? make_int2((int)start, (int)(start + total)) : make_int2(0, 0);
    }
    __syncthreads();
    if (col) {
        uint32_t run = s_start[x] + before;
        for (uint32_t s = s0; s < s1; s += kBatch) {
            uint32_t v[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k)
                v[k] = s + k < s1 ? sc[(int64_t)min(s + k, s1 - 1u) * kMaxFastTiles + x] : 0u;
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const uint32_t t = v[k];
                v[k] = run;
                run += t;
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k)
                if (s + k < s1) sc[(int64_t)(s + k) * kMaxFastTiles + x] = v[k];
        }
    }
}

// Placement: each segment's duplicates (the row's entries expanded left to
// right, in entry order) are ranked by column, stably in duplicate order,
// and written at sc[segment][column] + (earlier duplicates of that column
// in the segment).  Duplicate i of the segment is item i of the ranking
// order (wave-contiguous slices, rounds of 64 lanes); its entry, the staged
// entry whose span holds i, is written into the segment's slots by the
// entry itself.  With pub.host, workgroup 0 copies the status words to
// the host first (every earlier kernel of the binning has finished).
// The forward rasterizer's tile order where no placement launch computes it
// (the general path, no duplicates): one workgroup per band.
__global__ __launch_bounds__(kOrderThreads) void k_fwd_order(const int2* __restrict__ ranges,
                                                             int64_t n_ids, int tiles,
                                                             int* __restrict__ order) {
    __shared__ uint32_t s_order[tile_order_lds_words<kOrderThreads>()];
    tile_order_band<false>(blockIdx.x, ranges, nullptr, n_ids, tiles, order, s_order);
}

__global__ __launch_bounds__(kPlaceThreads) void k_place(
    int64_t cap, const RowPlan* __restrict__ plan, const uint32_t* __restrict__ segrow,
    const uint32_t* __restrict__ segk0, int tiles_x, const uint32_t* __restrict__ e_gid,
    const uint32_t* __restrict__ e_pack, const uint32_t* __restrict__ e_doff,
    const uint32_t* __restrict__ sc, int32_t* __restrict__ ids, Publish pub, int bands,
    const int2* __restrict__ ranges, int tiles, int* __restrict__ order) {
    constexpr int kWaves = kPlaceThreads / 64;
    __shared__ uint32_t s_ent[3 * kSegDups];   // staged (doff, gid, pack); then (pos, gid)
    static_assert(3 * kSegDups >= tile_order_lds_words<kPlaceThreads>(), "order scratch fits");
    __shared__ uint16_t s_own[kSegDups];
    __shared__ uint32_t s_cnt[kWaves][kMaxFastTiles];
    __shared__ uint32_t s_base[kMaxFastTiles];
    __shared__ uint32_t s_dexcl[kMaxFastTiles];
    __shared__ uint32_t s_w[kPlaceThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (pub.host && blockIdx.x == 0 && tid == 0) publish(pub);
    if ((int)blockIdx.x < bands) {
        // the forward rasterizer's tile order (k_tile_order's), band
        // blockIdx.x, beside the placement: the ranges are final (zero when
        // the duplicates overflowed, which still gives a valid order)
        tile_order_band<false, kPlaceThreads>(blockIdx.x, ranges, nullptr, cap, tiles, order,
                                              s_ent);
        return;
    }
    const uint32_t seg = blockIdx.x - (uint32_t)bands;
    if ((int64_t)plan->dups > cap) return;
    Segment sg;
    if (!find_segment(plan, segrow, segk0, seg, sg)) return;
    const int ne = (int)min(sg.k1 - sg.k0, (uint32_t)kSegDups);
    uint32_t* s_doff = s_ent;
    uint32_t* s_gid = s_ent + kSegDups;
    uint32_t* s_pack = s_ent + 2 * kSegDups;
    for (int k = tid; k < kWaves * kMaxFastTiles; k += kPlaceThreads) (&s_cnt[0][0])[k] = 0u;
    if (tid < tiles_x) s_base[tid] = sc[(int64_t)seg * kMaxFastTiles + tid];
    for (int k = tid; k < ne; k += kPlaceThreads) {
        const uint32_t e = sg.rb + sg.k0 + (uint32_t)k;
        const uint32_t doff = e_doff[e];
        const uint32_t pack = e_pack[e];
        s_doff[k] = doff;
        s_gid[k] = e_gid[e];
        s_pack[k] = pack;
        // slot owners: entry k holds the segment's duplicates
        // [max(doff, a), min(doff + w, e)) (k = 0 starts at or before a; an
        // entry starting at or after e, the candidate past the segment,
        // holds none); the spans are disjoint and cover the segment
        const uint32_t end = min(doff + ((pack >> 8) & 0xFFu) + 1u, sg.e);
        for (uint32_t x = max(doff, sg.a); x < end; ++x) s_own[x - sg.a] = (uint16_t)k;
    }
    __syncthreads();
    const uint32_t nd = sg.e - sg.a;
    const int xbits = 32 - __builtin_clz((uint32_t)max(tiles_x - 1, 1));
    const int base = wave * (64 * kEmitItems);
    const uint64_t lt = (1ull << lane) - 1ull;
    uint32_t xx[kEmitItems], gg[kEmitItems], rank[kEmitItems];
#pragma unroll
    for (int r = 0; r < kEmitItems; ++r) {
        const uint32_t i = (uint32_t)(base + r * 64 + lane);
        xx[r] = 0u;
        gg[r] = 0u;
        if (i < nd) {
            const uint32_t o = s_own[i];
            xx[r] = ((s_pack[o] & 0xFFu) + (sg.a + i - s_doff[o])) & 0xFFu;
            gg[r] = s_gid[o];
        }
    }
#pragma unroll
    for (int r = 0; r < kEmitItems; ++r) {
        const bool valid = (uint32_t)(base + r * 64 + lane) < nd;
        const uint64_t m = match_digit<8>(xx[r], valid, xbits);
        const uint32_t before = s_cnt[wave][xx[r]];
        rank[r] = before + (uint32_t)__popcll(m & lt);
        if (valid && (m & lt) == 0ull) s_cnt[wave][xx[r]] = before + (uint32_t)__popcll(m);
    }
    __syncthreads();  // the staged entries are free from here on
    uint32_t local = 0;
    if (tid < kMaxFastTiles) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t c = s_cnt[w][tid];
            s_cnt[w][tid] = local;
            local += c;
        }
    }
    uint32_t tot;
    const uint32_t dexcl = block_excl_scan<kPlaceThreads>(tid < kMaxFastTiles ? local : 0u, s_w, &tot);
    if (tid < kMaxFastTiles) s_dexcl[tid] = dexcl;
    __syncthreads();
    uint32_t* q_pos = s_ent;
    uint32_t* q_gid = s_ent + kSegDups;
#pragma unroll
    for (int r = 0; r < kEmitItems; ++r) {
        if ((uint32_t)(base + r * 64 + lane) < nd) {
            const uint32_t x = xx[r];
            const uint32_t within = s_cnt[wave][x] + rank[r];
            const uint32_t j = s_dexcl[x] + within;
            q_pos[j] = s_base[x] + within;
            q_gid[j] = gg[r];
        }
    }
    __syncthreads();
    for (uint32_t j = tid; j < nd; j += kPlaceThreads) {
        const uint32_t pos = q_pos[j];
        if (pos < (uint64_t)cap) ids[pos] = (int32_t)q_gid[j];  // always true for a consistent plan
    }
}

// ------------------------------------------------------ general tile phase --
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
    if (tid < kWave) {  // wave 0 walks the look-back
        uint32_t prefix = 0;
        uint32_t* st = status + chunk;
        if (tid == 0 && total > kCountMask) atomicOr(err, GSX_BIN_ERR_OVERFLOW);
        if (chunk == 0) {
            if (tid == 0) status_store(st, kFlagInc | (total & kCountMask));
        } else {
            if (tid == 0) status_store(st, kFlagAgg | (total & kCountMask));
            prefix = wave_look_back(status, chunk, err);
            if (tid == 0) {
                if ((uint64_t)prefix + total > kCountMask) atomicOr(err, GSX_BIN_ERR_OVERFLOW);
                status_store(st, kFlagInc | ((prefix + total) & kCountMask));
            }
        }
        if (tid == 0) {
            s_prefix = prefix;
            if (chunk == nchunks - 1) {
                *d_total = prefix + total;
                offs[n] = prefix + total;
            }
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
    __shared__ uint32_t s_h[kMaxTilePasses][kRadix];
    __shared__ uint32_t s_drop;
    const int tid = threadIdx.x;
    const int64_t nd = live_count(cap, d_total);
    const int64_t d0 = (int64_t)blockIdx.x * kEmitDups;
    if (d0 >= nd) return;
    const int64_t d1 = min(d0 + kEmitDups, nd);
    for (int k = tid; k < kMaxTilePasses * kRadix; k += kEmitThreads) (&s_h[0][0])[k] = 0u;
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
    uint32_t* h = tile_hist + (blockIdx.x % kHistCopies) * kTileHistStride;
    for (int k = tid; k < passes * kRadix; k += kEmitThreads) {
        const uint32_t v = (&s_h[0][0])[k];
        if (v) atomicAdd(&h[k], v);
    }
    if (tid == 0 && s_drop) atomicAdd(dropped, s_drop);
}

// Tile ranges from the sorted tile ids, 4 ids per thread: a tile starts
// where the id differs from its predecessor and ends where it differs from
// its successor.  With pub.host, workgroup 0 copies the status words to the
// host first (the tile passes, the last writers of error bits, are done).
__global__ __launch_bounds__(256) void k_tile_ranges(int64_t cap,
                                                     const uint32_t* __restrict__ nd_dev,
                                                     const uint32_t* __restrict__ tiles,
                                                     int64_t num_tiles,
                                                     int2* __restrict__ ranges, Publish pub) {
    if (pub.host && blockIdx.x == 0 && threadIdx.x == 0) publish(pub);
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

// Copies the status words to the host (for a tile phase that launches no
// other kernel).
__global__ void k_publish(Publish pub) {
    if (threadIdx.x == 0) publish(pub);
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

inline int tiles_x_of(int32_t width) { return (width + kTile - 1) / kTile; }
inline int tiles_y_of(int32_t height) { return (height + kTile - 1) / kTile; }

// The row-placement tile phase: tile rows and columns fit 8-bit digits and
// refine_tiles (which drops duplicates after emission) is off.
inline bool fast_tiles(int tiles_x, int tiles_y) {
    return tiles_x <= kMaxFastTiles && tiles_y <= kMaxFastTiles;
}

// misc words: [8] the count scan's chunk counter ([0..7], [9..15] unused),
// [16..23] the status words of gsx_bin_sort, then the histogram copies of
// the depth sort, of the tile sort and the row histograms.
constexpr int kSyncStatusWord = 16;
constexpr int kMiscHead = 32;
constexpr int64_t kMiscDepthHist = kMiscHead;
constexpr int64_t kMiscTileHist = kMiscDepthHist + (int64_t)kHistCopies * kDepthHistStride;
constexpr int64_t kMiscRowDiff = kMiscTileHist + (int64_t)kHistCopies * kTileHistStride;
constexpr int64_t kMiscWords = kMiscRowDiff + (int64_t)kHistCopies * 2 * kRowWords;

// Workspace of the depth phase (sized by n alone) and of the tile phase
// (sized by the duplicate capacity); gsx_bin_sort(_async) places the tile
// part right after the depth part of one workspace.
struct DepthLayout {
    size_t dk[3], dv[3], offs, status, misc, plan, total;
    int64_t depth_chunks, scan_chunks, hist_blocks, status_words;
};
struct TileLayout {
    // general path
    size_t owner, tk0, tk1, tv, status;
    int64_t tile_chunks, emit_blocks, status_words;
    int tile_passes;
    // row-placement path
    size_t e_gid, e_pack, e_doff, rstatus, sc, segrow, segk0;
    int64_t row_chunks, segments, rstatus_words;
    size_t total;
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

// Look-back words of one depth pass over `chunks` chunks and `radix`
// digits: the statuses, the aggregates and the block statuses.
inline int64_t depth_pass_words(int64_t chunks, int radix) {
    return (2 * chunks + ceil_div(chunks, kLookBlock)) * radix;
}
inline int64_t depth_status_words(int64_t chunks) {
    return 3 * depth_pass_words(chunks, kDepthRadix) + depth_pass_words(chunks, 1 << kDepthTopBits);
}

DepthLayout make_depth_layout(int64_t n) {
    DepthLayout L{};
    Taker take;
    const size_t nn = (size_t)std::max<int64_t>(n, 1);
    L.depth_chunks = ceil_div((int64_t)nn, kDepthChunk);
    L.scan_chunks = ceil_div((int64_t)nn, kScanChunk);
    L.hist_blocks = ceil_div((int64_t)nn, kHistThreads * kHistItems);
    L.status_words = depth_status_words(L.depth_chunks) + L.scan_chunks;
    for (int k = 0; k < 3; ++k) {
        L.dk[k] = take(4 * nn);
        L.dv[k] = take(4 * nn);
    }
    L.offs = take(4 * (nn + 1));
    L.status = take(4 * (size_t)L.status_words);
    L.misc = take(4 * (size_t)kMiscWords);
    L.plan = take(sizeof(RowPlan));
    L.total = take.o;
    return L;
}

TileLayout make_tile_layout(int64_t cap, int64_t num_tiles) {
    TileLayout L{};
    const size_t cc = (size_t)std::max<int64_t>(cap, 1);
    {
        Taker take;
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
    }
    {
        // the row entries are at most the duplicates (each binned Gaussian
        // has at least one column per row), the segments at most one per
        // kSegDups duplicates plus one partial per row
        Taker take;
        L.row_chunks = ceil_div((int64_t)cc, kRowChunk);
        L.segments = ceil_div((int64_t)cc, kSegDups) + kMaxFastTiles;
        L.rstatus_words = L.row_chunks * 2 * kMaxFastTiles;
        take(4 * (size_t)L.row_chunks);  // owner, as in the general path
        L.e_gid = take(4 * cc);
        L.e_pack = take(4 * cc);
        L.e_doff = take(4 * cc);
        L.rstatus = take(4 * (size_t)L.rstatus_words);
        L.sc = take(4 * (size_t)L.segments * kMaxFastTiles);
        L.segrow = take(4 * (size_t)L.segments);
        L.segk0 = take(4 * (size_t)L.segments);
        L.total = std::max(L.total, take.o);
    }
    return L;
}

template <typename T>
inline T* at(void* ws, size_t off) {
    return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

inline unsigned grid_for(int64_t n, int64_t per) {
    return (unsigned)std::max<int64_t>(1, ceil_div(n, per));
}

inline Publish make_publish(const uint32_t* words, uint64_t* host, uint32_t seq) {
    return Publish{words, reinterpret_cast<unsigned long long*>(host), seq};
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
                const uint32_t* tile_rects, int32_t width, int32_t height, void* depth_ws,
                int64_t depth_ws_bytes, int32_t* tile_ranges, uint32_t* bin_status,
                bool clear_errors, hipStream_t st) {
    int rc = check_args(n, width, height, 0);
    if (rc != GSX_OK) return rc;
    if (!tile_ranges || !bin_status) return GSX_ERR_INVALID;
    if (n > 0 && (!tile_counts || !depth_keys || !tile_rects || !depth_ws))
        return GSX_ERR_INVALID;
    const int tx = tiles_x_of(width), ty = tiles_y_of(height);
    const int64_t T = (int64_t)tx * ty;
    const DepthLayout L = make_depth_layout(n);
    if (n > 0 && depth_ws_bytes < (int64_t)L.total) return GSX_ERR_WORKSPACE;
    uint32_t* status = n > 0 ? at<uint32_t>(depth_ws, L.status) : nullptr;
    uint32_t* misc = n > 0 ? at<uint32_t>(depth_ws, L.misc) : nullptr;
    // ranges, the bin_status words (and, when asked, its error bits),
    // look-back status words, counters and histograms all start at zero
    rc = zero(ZeroRanges{{(uint32_t*)tile_ranges, bin_status + (clear_errors ? 0 : 2), bin_status,
                          status, misc},
                         {2 * T, clear_errors ? kStatusWords : kStatusWords - 2, 1,
                          L.status_words, kMiscWords}},
              st);
    if (rc != GSX_OK || n == 0) return rc;
    // digit histograms of the depth keys; the tile counts summed into
    // bin_status[3], the rectangle heights into bin_status[4]; the row
    // histograms of the row-placement path
    hipLaunchKernelGGL(k_depth_hist, dim3((unsigned)L.hist_blocks), dim3(kHistThreads), 0, st,
                       depth_keys, tile_counts, (const uint2*)tile_rects, n,
                       fast_tiles(tx, ty) ? ty : 0, misc + kMiscDepthHist, misc + kMiscRowDiff,
                       bin_status);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int depth_phase(int64_t n, const uint32_t* depth_keys, void* depth_ws, int64_t depth_ws_bytes,
                uint32_t* bin_status, uint64_t* host_status, uint32_t seq, hipStream_t st) {
    if (n < 0 || n > (int64_t)kCountMask) return n < 0 ? GSX_ERR_INVALID : GSX_ERR_TOO_LARGE;
    if (!bin_status) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!depth_keys || !depth_ws) return GSX_ERR_INVALID;
    const DepthLayout L = make_depth_layout(n);
    if (depth_ws_bytes < (int64_t)L.total) return GSX_ERR_WORKSPACE;
    uint32_t* status = at<uint32_t>(depth_ws, L.status);
    uint32_t* misc = at<uint32_t>(depth_ws, L.misc);
    const uint32_t* hist = misc + kMiscDepthHist;
    // stable sort of the Gaussians by depth key (index order breaks ties):
    // buffers A -> B -> A -> C, or A -> B -> C when the top pass is skipped
    // (the third pass then writes C itself); the sorted ids end in C's values
    uint32_t* dk[3] = {at<uint32_t>(depth_ws, L.dk[0]), at<uint32_t>(depth_ws, L.dk[1]),
                       at<uint32_t>(depth_ws, L.dk[2])};
    uint32_t* dv[3] = {at<uint32_t>(depth_ws, L.dv[0]), at<uint32_t>(depth_ws, L.dv[1]),
                       at<uint32_t>(depth_ws, L.dv[2])};
    const Publish none{nullptr, nullptr, 0};
    const Publish pub = host_status ? make_publish(bin_status, host_status, seq) : none;
    const unsigned grid = (unsigned)L.depth_chunks;
    // per pass: statuses, aggregates, block statuses (depth_pass_words)
    const size_t per_pass = (size_t)depth_pass_words(L.depth_chunks, kDepthRadix);
    const size_t chunk_words = (size_t)L.depth_chunks * kDepthRadix;
    const uint32_t* nil = nullptr;
    uint32_t* no = nullptr;
    auto pass10 = [&](int p, const uint32_t* kin, const uint32_t* vin, uint32_t* ko,
                      uint32_t* vo, const Publish& pb, const uint32_t* route, uint32_t* ka,
                      uint32_t* va) {
        hipLaunchKernelGGL((k_onesweep<kDepthThreads, kDepthItems, kDepthBits>), dim3(grid),
                           dim3(kDepthThreads), 0, st, kin, vin, n, nil, p * kDepthBits,
                           kDepthBits, hist + p * kDepthRadix, kDepthHistStride, false,
                           status + p * per_pass, status + p * per_pass + chunk_words,
                           status + p * per_pass + 2 * chunk_words, ko, vo, bin_status + 1, pb,
                           route,
                           ka, va);
    };
    pass10(0, depth_keys, nil, dk[0], dv[0], pub, nil, no, no);
    pass10(1, dk[0], dv[0], dk[1], dv[1], none, nil, no, no);
    // the third pass writes A when the top pass runs, C when it is skipped
    pass10(2, dk[1], dv[1], dk[0], dv[0], none, hist, dk[2], dv[2]);
    hipLaunchKernelGGL((k_onesweep<kDepthThreads, kDepthItems, kDepthTopBits>), dim3(grid),
                       dim3(kDepthThreads), 0, st, dk[0], dv[0], n, nil, kDepthTopShift,
                       kDepthTopBits, hist + 3 * kDepthRadix, kDepthHistStride, true,
                       status + 3 * per_pass,
                       status + 3 * per_pass + (size_t)L.depth_chunks * (1 << kDepthTopBits),
                       status + 3 * per_pass + 2 * (size_t)L.depth_chunks * (1 << kDepthTopBits),
                       dk[2], dv[2], bin_status + 1, none, nil,
                       no, no);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int tiles_phase(int64_t n, const uint32_t* tile_counts, const uint32_t* tile_rects,
                const float* means2d, const float* conics, int64_t conic_stride, int32_t width,
                int32_t height, void* depth_ws, int64_t depth_ws_bytes, void* tile_ws,
                int64_t tile_ws_bytes, int64_t capacity, int32_t* sorted_ids,
                int32_t* tile_ranges, uint32_t* bin_status, uint64_t* host_status, uint32_t seq,
                int32_t* tile_order, hipStream_t st) {
    int rc = check_args(n, width, height, capacity);
    if (rc != GSX_OK) return rc;
    if (!tile_ranges || !bin_status) return GSX_ERR_INVALID;
    // the forward rasterizer's order, when asked: [T, T + T) of tile_order
    const int64_t tiles = (int64_t)tiles_x_of(width) * tiles_y_of(height);
    int* const order = tile_order ? tile_order + tiles : nullptr;
    auto order_alone = [&]() {
        if (order)
            hipLaunchKernelGGL(k_fwd_order, dim3(kOrderBands), dim3(kOrderThreads), 0, st,
                               (const int2*)tile_ranges, capacity, (int)tiles, order);
    };
    if (n == 0) {  // the count phase cleared the ranges and status
        order_alone();
        GSX_LAUNCH_CHECK();
        return GSX_OK;
    }
    if (!tile_counts || !tile_rects || !depth_ws || !tile_ws) return GSX_ERR_INVALID;
    const bool refine = conics != nullptr;
    if (refine && (!means2d || ((uintptr_t)means2d & 7u) != 0u || conic_stride < 3))
        return GSX_ERR_INVALID;
    if (capacity > 0 && (!sorted_ids || ((uintptr_t)sorted_ids & 15u) != 0u))
        return GSX_ERR_INVALID;  // emission stores 4 ids at a time
    const int tiles_x = tiles_x_of(width);
    const int tiles_y = tiles_y_of(height);
    const int64_t T = (int64_t)tiles_x * tiles_y;
    const DepthLayout D = make_depth_layout(n);
    const TileLayout L = make_tile_layout(capacity, T);
    if (depth_ws_bytes < (int64_t)D.total || tile_ws_bytes < (int64_t)L.total)
        return GSX_ERR_WORKSPACE;
    uint32_t* misc = at<uint32_t>(depth_ws, D.misc);
    uint32_t* err = bin_status + 1;
    const uint32_t* gids = at<uint32_t>(depth_ws, D.dv[2]);  // the depth sort's order
    uint32_t* offs = at<uint32_t>(depth_ws, D.offs);
    uint32_t* sstatus = at<uint32_t>(depth_ws, D.status) + depth_status_words(D.depth_chunks);
    uint32_t* owner = at<uint32_t>(tile_ws, 0);
    const Publish none{nullptr, nullptr, 0};
    const Publish pub = host_status ? make_publish(bin_status, host_status, seq) : none;

    if (!refine && fast_tiles(tiles_x, tiles_y)) {
        // row scan (+ row plan, D into bin_status[0]); row emission;
        // segment counts; per-row tile scan (ranges); placement
        RowPlan* plan = at<RowPlan>(depth_ws, D.plan);
        // the rectangles in depth order, packed (the depth sort's first key
        // buffer is free once the sort has ended)
        uint32_t* prect = at<uint32_t>(depth_ws, D.dk[0]);
        uint32_t* rstatus = at<uint32_t>(tile_ws, L.rstatus);
        uint32_t* e_gid = at<uint32_t>(tile_ws, L.e_gid);
        uint32_t* e_pack = at<uint32_t>(tile_ws, L.e_pack);
        uint32_t* e_doff = at<uint32_t>(tile_ws, L.e_doff);
        uint32_t* sc = at<uint32_t>(tile_ws, L.sc);
        uint32_t* segrow = at<uint32_t>(tile_ws, L.segrow);
        uint32_t* segk0 = at<uint32_t>(tile_ws, L.segk0);
        hipLaunchKernelGGL(k_row_scan, dim3((unsigned)D.scan_chunks + 1u), dim3(kScanThreads), 0, st,
                           n, (const uint2*)tile_rects, gids, sstatus, offs, prect, owner,
                           L.row_chunks, bin_status, rstatus, L.rstatus_words,
                           (const uint32_t*)(misc + kMiscRowDiff), tiles_y, plan, segrow,
                           L.segments);
        GSX_LAUNCH_CHECK();
        if (capacity == 0) {
            if (pub.host) hipLaunchKernelGGL(k_publish, dim3(1), dim3(64), 0, st, pub);
            order_alone();
            GSX_LAUNCH_CHECK();
            return GSX_OK;
        }
        hipLaunchKernelGGL(k_row_emit, dim3((unsigned)L.row_chunks), dim3(kEmitThreads), 0, st,
                           n, capacity, (const uint32_t*)offs, (const uint32_t*)owner, gids,
                           (const uint32_t*)prect, (const RowPlan*)plan, tiles_y, rstatus,
                           e_gid, e_pack, e_doff, segk0, L.segments, err);
        hipLaunchKernelGGL(k_seg_count, dim3((unsigned)L.segments), dim3(kMaxFastTiles), 0, st,
                           capacity, (const RowPlan*)plan, (const uint32_t*)segrow,
                           (const uint32_t*)segk0, tiles_x, (const uint32_t*)e_pack,
                           (const uint32_t*)e_doff, sc);
        hipLaunchKernelGGL(k_tile_scan, dim3((unsigned)tiles_y), dim3(kScanParts * kMaxFastTiles),
                           0, st,
                           capacity, (const RowPlan*)plan, tiles_x, sc, (int2*)tile_ranges);
        // the first kOrderBands workgroups build the forward's tile order
        const int bands = order ? kOrderBands : 0;
        hipLaunchKernelGGL(k_place, dim3((unsigned)L.segments + (unsigned)bands),
                           dim3(kPlaceThreads), 0, st, capacity, (const RowPlan*)plan,
                           (const uint32_t*)segrow, (const uint32_t*)segk0, tiles_x,
                           (const uint32_t*)e_gid, (const uint32_t*)e_pack,
                           (const uint32_t*)e_doff, (const uint32_t*)sc, sorted_ids, pub, bands,
                           (const int2*)tile_ranges, (int)T, order);
        GSX_LAUNCH_CHECK();
        return GSX_OK;
    }

    // general path: scan of the counts in depth order (it also clears the
    // tile passes' status words); emission (+ tile digit histograms) into
    // the buffers from which the tile passes end in sorted_ids; tile sort
    // over the device-side D; ranges
    uint32_t* d_total = bin_status;
    uint32_t* dropped = bin_status + 2;
    uint32_t* tile_hist = misc + kMiscTileHist;
    const int passes = refine ? L.tile_passes : passes_for(T);
    // significant bits of the tile ids (the refine_tiles sentinel T included)
    const int tile_bits = bits_for(std::max<int64_t>(refine ? T + 1 : T, 1));
    uint32_t* tk[2] = {at<uint32_t>(tile_ws, L.tk0), at<uint32_t>(tile_ws, L.tk1)};
    uint32_t* tv[2] = {(uint32_t*)sorted_ids, at<uint32_t>(tile_ws, L.tv)};
    int cur = passes & 1;
    uint32_t* tstatus = at<uint32_t>(tile_ws, L.status);
    hipLaunchKernelGGL(k_count_scan, dim3((unsigned)D.scan_chunks), dim3(kScanThreads), 0, st, n,
                       tile_counts, gids, sstatus, misc + 8, offs, owner, L.emit_blocks, d_total,
                       err, tstatus, L.status_words);
    GSX_LAUNCH_CHECK();
    if (capacity == 0) {
        if (pub.host) hipLaunchKernelGGL(k_publish, dim3(1), dim3(64), 0, st, pub);
        order_alone();
        GSX_LAUNCH_CHECK();
        return GSX_OK;
    }
    hipLaunchKernelGGL(k_emit, dim3((unsigned)L.emit_blocks), dim3(kEmitThreads), 0, st, n,
                       capacity, (const uint32_t*)d_total, (const uint32_t*)offs,
                       (const uint32_t*)owner, gids, (const uint2*)tile_rects, tiles_x, passes,
                       (const float2*)means2d, conics, conic_stride, (int)width, (int)height,
                       (uint32_t)T, dropped, tk[cur], tv[cur], tile_hist);
    GSX_LAUNCH_CHECK();
    const Publish nopub{nullptr, nullptr, 0};
    for (int p = 0; p < passes; ++p) {
        hipLaunchKernelGGL((k_onesweep<kTileThreads, kTileItems, kRadixBits>),
                           dim3((unsigned)L.tile_chunks), dim3(kTileThreads), 0, st, tk[cur],
                           tv[cur], capacity, (const uint32_t*)d_total, p * kRadixBits,
                           std::min(kRadixBits, tile_bits - p * kRadixBits),
                           tile_hist + p * kRadix, kTileHistStride, false,
                           tstatus + (size_t)p * L.tile_chunks * kRadix, (uint32_t*)nullptr,
                           (uint32_t*)nullptr, tk[cur ^ 1], tv[cur ^ 1], err, nopub,
                           (const uint32_t*)nullptr,
                           (uint32_t*)nullptr, (uint32_t*)nullptr);
        cur ^= 1;
    }
    GSX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_tile_ranges, dim3(grid_for(capacity, 1024)), dim3(256), 0, st, capacity,
                       (const uint32_t*)d_total, tk[cur], T, (int2*)tile_ranges, pub);
    order_alone();
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
                        const uint32_t* tile_rects, int32_t width, int32_t height,
                        void* depth_ws, int64_t depth_ws_bytes, int32_t* tile_ranges,
                        uint32_t* bin_status, void* stream) {
    return count_phase(n, tile_counts, depth_keys, tile_rects, width, height, depth_ws,
                       depth_ws_bytes, tile_ranges, bin_status, false, (hipStream_t)stream);
}

int gsx_bin_depth_async(int64_t n, const uint32_t* depth_keys, void* depth_ws,
                        int64_t depth_ws_bytes, uint32_t* bin_status, uint64_t* host_status,
                        uint32_t seq, void* stream) {
    return depth_phase(n, depth_keys, depth_ws, depth_ws_bytes, bin_status, host_status, seq,
                       (hipStream_t)stream);
}

int gsx_bin_tiles_async(int64_t n, const uint32_t* tile_counts, const uint32_t* tile_rects,
                        const float* means2d, const float* conics, int64_t conic_stride,
                        int32_t width, int32_t height, void* depth_ws, int64_t depth_ws_bytes,
                        void* tile_ws, int64_t tile_ws_bytes, int64_t capacity,
                        int32_t* sorted_ids, int32_t* tile_ranges, uint32_t* bin_status,
                        uint64_t* host_status, uint32_t seq, int32_t* tile_order, void* stream) {
    return tiles_phase(n, tile_counts, tile_rects, means2d, conics, conic_stride, width, height,
                       depth_ws, depth_ws_bytes, tile_ws, tile_ws_bytes, capacity, sorted_ids,
                       tile_ranges, bin_status, host_status, seq, tile_order,
                       (hipStream_t)stream);
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
    const int64_t T = (int64_t)tiles_x_of(width) * tiles_y_of(height);
    const int64_t dbytes = (int64_t)make_depth_layout(n).total;
    const int64_t tbytes = (int64_t)make_tile_layout(capacity, T).total;
    if (n > 0 && workspace_bytes < dbytes + tbytes) return GSX_ERR_WORKSPACE;
    rc = count_phase(n, tile_counts, depth_keys, tile_rects, width, height, workspace, dbytes,
                     tile_ranges, bin_status, true, (hipStream_t)stream);
    if (rc != GSX_OK || n == 0) return rc;
    rc = depth_phase(n, depth_keys, workspace, dbytes, bin_status, nullptr, 0,
                     (hipStream_t)stream);
    if (rc != GSX_OK) return rc;
    return tiles_phase(n, tile_counts, tile_rects, means2d, conics, conic_stride, width, height,
                       workspace, dbytes, static_cast<char*>(workspace) + dbytes, tbytes,
                       capacity, sorted_ids, tile_ranges, bin_status, nullptr, 0, nullptr,
                       (hipStream_t)stream);
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
        const int64_t T = (int64_t)tiles_x_of(width) * tiles_y_of(height);
        return zero(ZeroRanges{{(uint32_t*)tile_ranges, nullptr, nullptr, nullptr, nullptr},
                               {2 * T, 0, 0, 0, 0}},
                    st);
    }
    if (!workspace) return GSX_ERR_INVALID;
    const int64_t need =
        gsx_bin_workspace_bytes(n, capacity, tiles_x_of(width) * tiles_y_of(height));
    if (workspace_bytes < need) return GSX_ERR_WORKSPACE;
    // the status words sit in the workspace's counter block, past the counters
    // the pipeline uses (it clears the whole block before the first kernel)
    uint32_t* bs = at<uint32_t>(workspace, make_depth_layout(n).misc) + kSyncStatusWord;
    rc = gsx_bin_sort_async(n, tile_counts, depth_keys, tile_rects, means2d, conics,
                            conic_stride, width, height, workspace, workspace_bytes, capacity,
                            sorted_ids, tile_ranges, bs, stream);
    if (rc != GSX_OK) return rc;
    uint32_t host[kStatusWords] = {};
    if (hipMemcpyAsync(host, bs, sizeof(host), hipMemcpyDeviceToHost, st) != hipSuccess)
        return GSX_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return GSX_ERR_HIP;
    return gsx_bin_status_check(host, capacity, num_dups);
}

int gsx_host_status_alloc(uint64_t** words) {
    if (!words) return GSX_ERR_INVALID;
    *words = nullptr;
    void* p = nullptr;
    if (hipHostMalloc(&p, 2 * kStatusWords * sizeof(uint64_t),
                      hipHostMallocCoherent | hipHostMallocMapped | hipHostMallocPortable) !=
        hipSuccess)
        return GSX_ERR_HIP;
    // kernels write the words through the same address (unified addressing)
    void* dp = nullptr;
    if (hipHostGetDevicePointer(&dp, p, 0) != hipSuccess || dp != p) {
        (void)hipHostFree(p);
        return GSX_ERR_HIP;
    }
    memset(p, 0, 2 * kStatusWords * sizeof(uint64_t));
    *words = static_cast<uint64_t*>(p);
    return GSX_OK;
}

int gsx_host_status_free(uint64_t* words) {
    if (!words) return GSX_OK;
    return hipHostFree(words) == hipSuccess ? GSX_OK : GSX_ERR_HIP;
}

}  // extern "C"
