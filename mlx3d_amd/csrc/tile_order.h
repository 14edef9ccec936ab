// Tile processing order of the rasterizers, shared by the rasterizer (its
// own order kernels) and the binning (which computes the forward's order
// beside its placement): the work estimate buckets, the band layout and the
// per-band counting sort.  Device code only; no host symbols.
#pragma once

#include "gsx_device.h"

namespace gsx {
// Clamp a tile's [start, end) to the id array so a malformed range can
// never read outside it.
__device__ __forceinline__ void tile_span(int2 rg, int64_t n_ids, int& start, int& num) {
    const int64_t s0 = rg.x < 0 ? 0 : (rg.x > n_ids ? n_ids : rg.x);
    const int64_t s1 = rg.y < s0 ? s0 : (rg.y > n_ids ? n_ids : rg.y);
    start = (int)s0;
    num = (int)(s1 - s0);
}

// The tile order for tile_at: one workgroup per band (XCD) x.  Each tile
// gets a band and a work estimate; band x's workgroup lists its tiles by
// descending quarter-octave bucket of the estimate (4 log2(w + 1), 64
// buckets) with a counting sort.  Forward (BWD false): the estimate is the
// list length (ranges), the bands are xcd_remap's (equal tile counts), and
// tile t lands at order[band start + its rank in the band].  Backward: the
// estimate is the contributor bound the forward stored (work, the entries
// the backward replays); up to 16384 tiles the bands are cut at equal
// shares of sum(min(w, 2^16) + 16) (the 16 stands for a tile's fixed cost;
// every workgroup computes the same cuts from the whole frame), each
// capped at cap = 2 ceil(T / 8) tiles, and tile t lands at
// order[8 rank + band], so workgroup b = 8 i + x (XCD x) takes band x's
// i-th tile; band x's other entries of the 8 cap hold -1.  The sort is
// stable (tiles of one bucket keep their raster order) and uses no LDS
// atomics (same-address lanes of one would serialize).  Every tile is
// placed exactly once, whatever the estimates hold.
constexpr int kOrderThreads = 1024;
constexpr int kOrderItems = 16;   // tiles per thread of the band cut, read at once
constexpr int kOrderBuckets = 64;
constexpr int kOrderBands = 8;
constexpr int kOrderBalanced = kOrderThreads * kOrderItems;     // most tiles cut by work

__device__ __forceinline__ int order_bucket(int w) {
    const uint32_t v = (uint32_t)max(w, 0) + 1u;
    const int e = 31 - __clz(v);
    const int frac = e >= 2 ? (int)((v >> (e - 2)) & 3u) : (int)((v << (2 - e)) & 3u);
    return kOrderBuckets - 1 - min(kOrderBuckets - 1, 4 * e + frac);  // heaviest first
}

// Words of a tile-order buffer for T tiles: T bounds, then 16 ceil(T / 8)
// order entries.
__host__ __device__ inline int64_t tile_order_words(int64_t tiles) {
    return tiles + 16 * ((tiles + kOrderBands - 1) / kOrderBands);
}

// LDS words tile_order_band needs from its caller at THREADS threads.
constexpr int kBandItems = 4;
template <int THREADS>
constexpr int tile_order_lds_words() {
    return kOrderBuckets * kBandItems * (THREADS / kWave) + THREADS / kWave + kOrderBands + 1;
}

// Band `band`'s order by the workgroup of THREADS threads (the backward's
// band cuts need kOrderThreads); lds holds tile_order_lds_words<THREADS>()
// words of the caller's shared memory.
template <bool BWD, int THREADS = kOrderThreads>
__device__ __forceinline__ void tile_order_band(int band, const int2* __restrict__ ranges,
                                                const int* __restrict__ work, int64_t n_ids,
                                                int tiles, int* __restrict__ order,
                                                uint32_t* lds) {
    static_assert(!BWD || THREADS == kOrderThreads, "the band cuts assume kOrderThreads");
    static_assert(THREADS % kWave == 0 && THREADS <= kOrderThreads, "whole waves");
    uint32_t* s_cnt = lds;  // [bucket][item][wave] counts, then their scan
    uint32_t* s_w = lds + kOrderBuckets * kBandItems * (THREADS / kWave);
    int* s_start = reinterpret_cast<int*>(s_w + THREADS / kWave);  // first tile of each band
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int cap = 2 * ((tiles + kOrderBands - 1) / kOrderBands);
    auto estimate = [&](int t) {
        if constexpr (BWD) {
            return work[t];
        } else {
            int start, num;
            tile_span(ranges[t], n_ids, start, num);
            return num;
        }
    };
    // equal-count bands (xcd_remap's ranges)
    const int q = tiles / kOrderBands, r = tiles % kOrderBands;
    if (tid <= kOrderBands)
        s_start[tid] = tid < r ? tid * (q + 1) : r * (q + 1) + (tid - r) * q;
    if (BWD)  // this band's unused entries say "no tile"
        for (int i = tid; i < cap; i += THREADS) order[kOrderBands * i + band] = -1;
    for (int k = tid; k < kOrderBuckets * kBandItems * (THREADS / kWave); k += THREADS)
        s_cnt[k] = 0u;
    if (BWD && tiles <= kOrderBalanced) {
        // bands of equal work: exclusive prefix of the weights over the
        // tiles in raster order (thread tid: tiles 16 tid .. 16 tid + 15)
        int w[kOrderItems];
#pragma unroll
        for (int k = 0; k < kOrderItems; ++k)
            w[k] = work[min(tid * kOrderItems + k, tiles - 1)];
        uint32_t v[kOrderItems], sum = 0;
#pragma unroll
        for (int k = 0; k < kOrderItems; ++k) {
            const int t = tid * kOrderItems + k;
            v[k] = t < tiles ? (uint32_t)min(max(w[k], 0), 1 << 16) + 16u : 0u;
            sum += v[k];
        }
        const uint32_t incl = wave_incl_scan(sum);
        if (lane == kWave - 1) s_w[wave] = incl;
        __syncthreads();
        if (tid > 0 && tid <= kOrderBands) s_start[tid] = tiles;
        uint32_t pe = incl - sum, total = 0;
#pragma unroll
        for (int x = 0; x < THREADS / kWave; ++x) {
            if (x < wave) pe += s_w[x];
            total += s_w[x];
        }
        __syncthreads();
        // band of tile t: floor(8 pe / total); the first tile of each band
        // (the smallest t with that band) recorded with atomicMin
        int prev = -1;
#pragma unroll
        for (int k = 0; k < kOrderItems; ++k) {
            const int t = tid * kOrderItems + k;
            if (t < tiles) {
                const int x = (int)min<uint64_t>(kOrderBands - 1,
                                                 (uint64_t)pe * kOrderBands / max(total, 1u));
                if (x != prev && x > 0) atomicMin(&s_start[x], t);
                prev = x;
            }
            pe += v[k];
        }
        __syncthreads();
        if (tid == 0) {
            // empty bands start where the next one does; then every band
            // holds at most cap tiles (the cuts move forward, then back)
            int b[kOrderBands + 1];
#pragma unroll
            for (int x = 1; x < kOrderBands; ++x) b[x] = s_start[x];
            b[0] = 0;
            b[kOrderBands] = tiles;
#pragma unroll
            for (int x = kOrderBands - 1; x > 0; --x) b[x] = min(b[x], b[x + 1]);
#pragma unroll
            for (int x = 1; x < kOrderBands; ++x) b[x] = min(b[x], b[x - 1] + cap);
#pragma unroll
            for (int x = kOrderBands - 1; x > 0; --x) b[x] = max(b[x], b[x + 1] - cap);
#pragma unroll
            for (int x = 0; x <= kOrderBands; ++x) s_start[x] = b[x];
        }
    }
    __syncthreads();
    const int lo = s_start[band], hi = s_start[band + 1];
    // this band's tiles: item k of thread tid is tile lo + k * 1024 + tid, so
    // tile order is (k, wave, lane) order.  A stable counting sort: per
    // item, the lanes of the wave holding the same bucket (ballots over its
    // six bits) give the rank within the wave; counts per (bucket, item,
    // wave), scanned in that order, give each wave's start.  Within a
    // bucket the tiles keep their raster order, so neighbouring tiles of
    // similar work run close together in time and share the XCD's L2.
    // Bands of more than kBandItems * 1024 tiles are placed in rounds, each
    // round sorted on its own (the rounds in raster order).
    for (int r0 = lo; r0 < hi; r0 += kBandItems * THREADS) {
        int bk[kBandItems], est[kBandItems];
        uint32_t rk[kBandItems];
#pragma unroll
        for (int k = 0; k < kBandItems; ++k)  // clamped: the loads issue together
            est[k] = estimate(min(r0 + k * THREADS + tid, hi - 1));
#pragma unroll
        for (int k = 0; k < kBandItems; ++k) {
            const int t = r0 + k * THREADS + tid;
            bk[k] = t < hi ? order_bucket(est[k]) : -1;
        }
#pragma unroll
        for (int k = 0; k < kBandItems; ++k) {
            const bool valid = bk[k] >= 0;
            uint64_t m = __ballot(valid);
#pragma unroll
            for (int b = 0; b < 6; ++b) {
                const bool bit = (bk[k] >> b) & 1;
                const uint64_t ones = __ballot(bit);
                m &= bit ? ones : ~ones;
            }
            rk[k] = (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
            // the lowest lane of each bucket group writes the group's count
            if (valid && rk[k] == 0u)
                s_cnt[(bk[k] * kBandItems + k) * (THREADS / kWave) + wave] =
                    (uint32_t)__popcll(m);
        }
        __syncthreads();
        {
            // exclusive scan of the (bucket, item, wave) counts, 4 per thread
            uint32_t c[kBandItems], sum = 0;
#pragma unroll
            for (int k = 0; k < kBandItems; ++k) {
                c[k] = s_cnt[tid * kBandItems + k];
                sum += c[k];
            }
            const uint32_t incl = wave_incl_scan(sum);
            if (lane == kWave - 1) s_w[wave] = incl;
            __syncthreads();
            uint32_t base = incl - sum;
            for (int x = 0; x < wave; ++x) base += s_w[x];
#pragma unroll
            for (int k = 0; k < kBandItems; ++k) {
                s_cnt[tid * kBandItems + k] = base;
                base += c[k];
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kBandItems; ++k) {
            if (bk[k] < 0) continue;
            const int t = r0 + k * THREADS + tid;
            const int rank = (int)(s_cnt[(bk[k] * kBandItems + k) * (THREADS / kWave) + wave] +
                                   rk[k]) + (r0 - lo);
            order[BWD ? kOrderBands * rank + band : lo + rank] = t;
        }
        __syncthreads();
        // counters back to zero for the next round
        for (int k = tid; k < kOrderBuckets * kBandItems * (THREADS / kWave);
             k += THREADS)
            s_cnt[k] = 0u;
        __syncthreads();
    }
}

}  // namespace gsx
