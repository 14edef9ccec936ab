// density.hip -- Gaussian-table edits of training on the device: the
// nearest-neighbour scale initialisation of GaussianModel.from_points
// (splatting/model.py:37-106), adaptive density control (densify_and_prune,
// model.py:406-480) and MCMC relocation (relocate_mcmc, model.py:482-531).
//
// Design.  A Gaussian table is a set of float32 (N, w) tensors -- the six
// parameter groups and, in training, their Adam moments -- described by a
// gsx_row_table.  Every edit is a row map applied to all of them in one
// launch:
//   densify  classify each row (keep / clone / split) -> per-block counts
//            -> one-workgroup scan of the block counts (the host reads the
//            three totals to size the new table and draw the split samples)
//            -> emit: each source row writes its kept copy, clone and split
//            pair at positions from the block prefix plus an in-block scan;
//            moments follow kept rows and are zero in new rows.
//   relocate gather the k source rows (with the relocation edits) into a
//            staging buffer, then write them over the k destination rows
//            and clear the destinations' moments (two launches, so a row
//            that is both a source and a destination is read before it is
//            overwritten).
// The kNN kernel gives each lane one query point and streams the reference
// points through LDS, keeping the K nearest (distance, index) pairs sorted
// in registers.
#include <hip/hip_runtime.h>

#include <cmath>

#include "gsx.h"
#include "gsx_device.h"

using namespace gsx;

namespace {

constexpr int kKnnThreads = 256;
constexpr int kKnnMaxK = 8;

// K nearest reference points of each query (squared distance as the sum of
// the three squared differences, ties to the lower index), then the mean of
// the K - 1 nearest after skipping a self hit (first distance <= 1e-12), or
// of the first K - 1 otherwise, clamped at 1e-8 (model.py:81-89), written as
// the isotropic log-scale log(sqrt(mean)), capped at log_cap.
template <int K>
__global__ __launch_bounds__(kKnnThreads) void k_knn_log_scale(
    int64_t nq, const float* __restrict__ q, int64_t nr, const float* __restrict__ r,
    float log_cap, float* __restrict__ out) {
    __shared__ float s_x[kKnnThreads], s_y[kKnnThreads], s_z[kKnnThreads];
    const int64_t i = (int64_t)blockIdx.x * kKnnThreads + threadIdx.x;
    const bool live = i < nq;
    const float qx = live ? q[3 * i] : 0.0f;
    const float qy = live ? q[3 * i + 1] : 0.0f;
    const float qz = live ? q[3 * i + 2] : 0.0f;
    float bd[K];
    int64_t bi[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        bd[k] = __builtin_huge_valf();
        bi[k] = INT64_MAX;
    }
    for (int64_t base = 0; base < nr; base += kKnnThreads) {
        __syncthreads();
        const int64_t j = base + threadIdx.x;
        if (j < nr) {
            s_x[threadIdx.x] = r[3 * j];
            s_y[threadIdx.x] = r[3 * j + 1];
            s_z[threadIdx.x] = r[3 * j + 2];
        }
        __syncthreads();
        const int cnt = (int)min<int64_t>(kKnnThreads, nr - base);
        for (int t = 0; t < cnt; ++t) {
            const float dx = qx - s_x[t], dy = qy - s_y[t], dz = qz - s_z[t];
            const float d = dx * dx + dy * dy + dz * dz;
            const int64_t idx = base + t;
            // insertion into the sorted list; equal distances keep index order
            // because indices arrive in increasing order
            if (!(d < bd[K - 1])) continue;
            float cd = d;
            int64_t ci = idx;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                if (cd < bd[k]) {
                    const float td = bd[k];
                    const int64_t ti = bi[k];
                    bd[k] = cd;
                    bi[k] = ci;
                    cd = td;
                    ci = ti;
                }
            }
        }
    }
    if (!live) return;
    // the reference clamps each distance at 0 (knn.py); the sum of squares is >= 0
    const bool self_hit = bd[0] <= 1e-12f;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < K - 1; ++k) s = s + (self_hit ? bd[k + 1] : bd[k]);
    const float mean = fmaxf(s / (float)(K - 1), 1e-8f);
    out[i] = fminf(logf(sqrtf(mean)), log_cap);
}

// ----------------------------------------------------------- densify --
constexpr int kRowThreads = 256;
constexpr uint8_t kKeep = 1, kClone = 2, kSplit = 4;

__device__ __forceinline__ float sigmoid_clipped(float o) {
    const float c = fminf(fmaxf(o, -50.0f), 50.0f);
    return 1.0f / (1.0f + expf(-c));
}

// Row classes of densify_and_prune (model.py:427-465) and per-block counts
// (kept, cloned, split) of each 256-row block.
__global__ __launch_bounds__(kRowThreads) void k_density_classify(
    int64_t n, const float* __restrict__ log_scales, const float* __restrict__ logit_opac,
    const float* __restrict__ acc, const float* __restrict__ cnt, float grad_threshold,
    float dense, float prune_scale, float min_opacity, uint8_t* __restrict__ cls,
    uint32_t* __restrict__ block_counts) {
    __shared__ uint32_t s_c[3][kRowThreads / kWave];
    const int64_t i = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
    uint8_t c = 0;
    if (i < n) {
        const float avg = acc[i] / fmaxf(cnt[i], 1.0f);
        const float s0 = expf(log_scales[3 * i]), s1 = expf(log_scales[3 * i + 1]);
        const float s2 = expf(log_scales[3 * i + 2]);
        const float smax = fmaxf(fmaxf(s0, s1), s2);
        const bool high = avg > grad_threshold;
        const bool clone = high && smax <= dense;
        const bool split = high && smax > dense;
        const bool prune = sigmoid_clipped(logit_opac[i]) < min_opacity || split ||
                           smax > prune_scale;
        c = (prune ? 0 : kKeep) | (clone ? kClone : 0) | (split ? kSplit : 0);
        cls[i] = c;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t k = __popcll(__ballot(c & kKeep)), cl = __popcll(__ballot(c & kClone)),
                   sp = __popcll(__ballot(c & kSplit));
    if (lane == 0) {
        s_c[0][wave] = k;
        s_c[1][wave] = cl;
        s_c[2][wave] = sp;
    }
    __syncthreads();
    if (threadIdx.x < 3) {
        uint32_t t = 0;
#pragma unroll
        for (int w = 0; w < kRowThreads / kWave; ++w) t += s_c[threadIdx.x][w];
        block_counts[3 * (int64_t)blockIdx.x + threadIdx.x] = t;
    }
}

// Exclusive prefix of the per-block counts, in place, by one workgroup
// (1024 threads, blocks in rounds of 1024), and the three totals.
__global__ __launch_bounds__(1024) void k_density_scan(int64_t nblk,
                                                       uint32_t* __restrict__ block_counts,
                                                       uint32_t* __restrict__ totals) {
    __shared__ uint32_t s_w[3][16];
    __shared__ uint32_t s_carry[3];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < 3) s_carry[tid] = 0;
    for (int64_t b0 = 0; b0 < nblk; b0 += 1024) {
        __syncthreads();
        const int64_t b = b0 + tid;
        uint32_t v[3], incl[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            v[c] = b < nblk ? block_counts[3 * b + c] : 0u;
            incl[c] = wave_incl_scan(v[c]);
            if (lane == 63) s_w[c][wave] = incl[c];
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            uint32_t off = s_carry[c], tot = 0;
            for (int w = 0; w < 16; ++w) {
                if (w < wave) off += s_w[c][w];
                tot += s_w[c][w];
            }
            if (b < nblk) block_counts[3 * b + c] = off + incl[c] - v[c];
            __syncthreads();
            if (tid == 0) s_carry[c] += tot;
        }
    }
    __syncthreads();
    if (tid < 3) totals[tid] = s_carry[tid];
}

// Relocation scores (model.py:497-512): target = 2 - sigmoid(o) for
// underused rows (sigmoid(o) < min_opacity or never seen), -sigmoid(o)
// otherwise; source = the average screen gradient; *under += the number of
// underused rows.
__global__ __launch_bounds__(kRowThreads) void k_relocate_scores(
    int64_t n, const float* __restrict__ acc, const float* __restrict__ cnt,
    const float* __restrict__ logit_opac, float min_opacity, float* __restrict__ target,
    float* __restrict__ source, uint32_t* __restrict__ under) {
    const int64_t i = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
    bool u = false;
    if (i < n) {
        const float o = 1.0f / (1.0f + expf(-logit_opac[i]));
        const float c = cnt[i];
        u = o < min_opacity || c <= 0.0f;
        target[i] = u ? 2.0f - o : -o;
        source[i] = acc[i] / fmaxf(c, 1.0f);
    }
    const uint64_t b = __ballot(u);
    if ((threadIdx.x & 63) == 0 && b) atomicAdd(under, (uint32_t)__popcll(b));
}

struct RowTable {
    int count;
    int width[GSX_TABLE_MAX];
    int role[GSX_TABLE_MAX];
    const float* src[GSX_TABLE_MAX];
    float* dst[GSX_TABLE_MAX];
};

__device__ __forceinline__ void copy_row(const float* __restrict__ s, float* __restrict__ d,
                                         int w) {
    for (int k = 0; k < w; ++k) d[k] = s[k];
}

// Rotation matrix of a unit quaternion (w, x, y, z), float32, the
// rotations.py:30-49 expression.
__device__ __forceinline__ void quat_rot(float w, float x, float y, float z, float* R) {
    R[0] = 1.0f - 2.0f * (y * y + z * z);
    R[1] = 2.0f * (x * y - w * z);
    R[2] = 2.0f * (x * z + w * y);
    R[3] = 2.0f * (x * y + w * z);
    R[4] = 1.0f - 2.0f * (x * x + z * z);
    R[5] = 2.0f * (y * z - w * x);
    R[6] = 2.0f * (x * z - w * y);
    R[7] = 2.0f * (y * z + w * x);
    R[8] = 1.0f - 2.0f * (x * x + y * y);
}

__device__ __forceinline__ void normalize4(float& w, float& x, float& y, float& z) {
    const float nrm = sqrtf(w * w + x * x + y * y + z * z);
    w = w / nrm;
    x = x / nrm;
    y = y / nrm;
    z = z / nrm;
}

// Writes every source row's outputs: kept copy at kept[i], clone at
// K + clone[i], split pair at K + C + 2 split[i] + {0, 1}.  A split row's
// mean moves by R(q) (s * xi) with xi the caller's standard-normal sample
// (float64, as drawn) and s = exp(log-scale), formed in double and rounded
// once (model.py:436-452); its log-scales drop by log 1.6.  Moment tensors
// are zero in every new row.
__global__ __launch_bounds__(kRowThreads) void k_density_emit(
    int64_t n, const uint8_t* __restrict__ cls, const uint32_t* __restrict__ block_prefix,
    const uint32_t* __restrict__ totals, RowTable tab, int means_col, int scales_col,
    int quats_col, const double* __restrict__ samples, float log_shrink) {
    __shared__ uint32_t s_w[3][kRowThreads / kWave];
    const int64_t i = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint8_t c = i < n ? cls[i] : 0;
    uint32_t flag[3] = {(uint32_t)(c & kKeep), (uint32_t)((c >> 1) & 1), (uint32_t)((c >> 2) & 1)};
    uint32_t incl[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        incl[k] = wave_incl_scan(flag[k]);
        if (lane == 63) s_w[k][wave] = incl[k];
    }
    __syncthreads();
    if (i >= n || c == 0) return;
    uint32_t pos[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        uint32_t off = block_prefix[3 * (int64_t)blockIdx.x + k];
        for (int w = 0; w < wave; ++w) off += s_w[k][w];
        pos[k] = off + incl[k] - flag[k];
    }
    const int64_t kept = totals[0], cloned = totals[1];
    const int64_t rows[4] = {(c & kKeep) ? (int64_t)pos[0] : -1,
                             (c & kClone) ? kept + pos[1] : -1,
                             (c & kSplit) ? kept + cloned + 2 * (int64_t)pos[2] : -1,
                             (c & kSplit) ? kept + cloned + 2 * (int64_t)pos[2] + 1 : -1};
    for (int t = 0; t < tab.count; ++t) {
        const int w = tab.width[t];
        const float* s = tab.src[t] + i * w;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (rows[r] < 0) continue;
            float* d = tab.dst[t] + rows[r] * w;
            if (tab.role[t] == GSX_ROW_MOMENT && r > 0) {
                for (int k = 0; k < w; ++k) d[k] = 0.0f;
            } else if (r >= 2 && t == scales_col) {
                for (int k = 0; k < w; ++k) d[k] = s[k] - log_shrink;
            } else if (r >= 2 && t == means_col) {
                const float* qs = tab.src[quats_col] + i * 4;
                float qw = qs[0], qx = qs[1], qy = qs[2], qz = qs[3];
                normalize4(qw, qx, qy, qz);  // model.py:441 normalises
                normalize4(qw, qx, qy, qz);  // and quaternion_to_matrix again
                float R[9];
                quat_rot(qw, qx, qy, qz, R);
                const float* ls = tab.src[scales_col] + i * 3;
                const double* xi = samples + 3 * (2 * (int64_t)pos[2] + (r - 2));
                double v[3];
#pragma unroll
                for (int a = 0; a < 3; ++a) v[a] = xi[a] * (double)expf(ls[a]);
#pragma unroll
                for (int a = 0; a < 3; ++a) {
                    const double off = (double)R[3 * a] * v[0] + (double)R[3 * a + 1] * v[1] +
                                       (double)R[3 * a + 2] * v[2];
                    d[a] = s[a] + (float)off;
                }
            } else {
                copy_row(s, d, w);
            }
        }
    }
}

// ---------------------------------------------------------- relocate --
// Staged row j = source row src[j] with the relocation edits (model.py:
// 517-529): means + noise * exp(log-scale) * jitter, opacity logit reset,
// log-scales - shrink.  Staging packs the tables' rows back to back.
__global__ __launch_bounds__(kRowThreads) void k_relocate_gather(
    int64_t k, const int64_t* __restrict__ src, RowTable tab, int means_col, int scales_col,
    int opac_col, const float* __restrict__ noise, float jitter, float reset_logit,
    float log_shrink, int row_width, float* __restrict__ staging) {
    const int64_t j = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
    if (j >= k) return;
    const int64_t i = src[j];
    float* out = staging + j * row_width;
    for (int t = 0; t < tab.count; ++t) {
        const int w = tab.width[t];
        if (tab.role[t] == GSX_ROW_MOMENT) continue;
        const float* s = tab.src[t] + i * w;
        if (t == means_col) {
            const float* ls = tab.src[scales_col] + i * 3;
            for (int a = 0; a < w; ++a)
                out[a] = s[a] + noise[3 * j + a] * expf(ls[a]) * jitter;
        } else if (t == opac_col) {
            for (int a = 0; a < w; ++a) out[a] = reset_logit;
        } else if (t == scales_col) {
            for (int a = 0; a < w; ++a) out[a] = s[a] - log_shrink;
        } else {
            copy_row(s, out, w);
        }
        out += w;
    }
}

// Destination row dst[j] = old + (staged - old), the rounding of the
// reference's scatter-add arr.at[dst].add(values - arr[dst]); moments of the
// destination rows become zero (old + (-old)).
__global__ __launch_bounds__(kRowThreads) void k_relocate_scatter(
    int64_t k, const int64_t* __restrict__ dst, RowTable tab, int row_width,
    const float* __restrict__ staging) {
    const int64_t j = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
    if (j >= k) return;
    const int64_t i = dst[j];
    const float* in = staging + j * row_width;
    for (int t = 0; t < tab.count; ++t) {
        const int w = tab.width[t];
        float* d = tab.dst[t] + i * w;
        if (tab.role[t] == GSX_ROW_MOMENT) {
            for (int a = 0; a < w; ++a) d[a] = 0.0f;
            continue;
        }
        for (int a = 0; a < w; ++a) d[a] = d[a] + (in[a] - d[a]);
        in += w;
    }
}

bool load_table(const gsx_row_table* t, RowTable& out, bool in_place) {
    if (!t || t->count <= 0 || t->count > GSX_TABLE_MAX) return false;
    out.count = t->count;
    for (int k = 0; k < t->count; ++k) {
        if (t->width[k] <= 0 || !t->src[k] || !t->dst[k]) return false;
        if (t->role[k] != GSX_ROW_PARAM && t->role[k] != GSX_ROW_MOMENT) return false;
        if (in_place && t->src[k] != t->dst[k]) return false;
        out.width[k] = t->width[k];
        out.role[k] = t->role[k];
        out.src[k] = t->src[k];
        out.dst[k] = t->dst[k];
    }
    for (int k = t->count; k < GSX_TABLE_MAX; ++k) {
        out.width[k] = 0;
        out.role[k] = 0;
        out.src[k] = nullptr;
        out.dst[k] = nullptr;
    }
    return true;
}

bool col_ok(const RowTable& t, int col, int width) {
    return col >= 0 && col < t.count && t.width[col] == width && t.role[col] == GSX_ROW_PARAM;
}

inline unsigned blocks_for(int64_t n, int threads) {
    return (unsigned)((n + threads - 1) / threads);
}

}  // namespace

extern "C" {

int gsx_knn_log_scale(int64_t n_query, const float* query, int64_t n_ref, const float* ref,
                      int32_t k, float log_cap, float* log_scale, void* stream) {
    if (n_query < 0 || n_ref < 0 || k < 2 || k > kKnnMaxK || k > n_ref) return GSX_ERR_INVALID;
    if (n_query == 0) return GSX_OK;
    if (!query || !ref || !log_scale) return GSX_ERR_INVALID;
    if (n_query > ((int64_t)1 << 40)) return GSX_ERR_TOO_LARGE;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(blocks_for(n_query, kKnnThreads));
    switch (k) {
#define GSX_KNN(K)                                                                             \
    case K:                                                                                    \
        hipLaunchKernelGGL(k_knn_log_scale<K>, grid, dim3(kKnnThreads), 0, st, n_query, query, \
                           n_ref, ref, log_cap, log_scale);                                    \
        break;
        GSX_KNN(2) GSX_KNN(3) GSX_KNN(4) GSX_KNN(5) GSX_KNN(6) GSX_KNN(7) GSX_KNN(8)
#undef GSX_KNN
        default:
            return GSX_ERR_INVALID;
    }
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int64_t gsx_density_workspace_bytes(int64_t n) {
    if (n < 0) return GSX_ERR_INVALID;
    const int64_t nblk = (n + kRowThreads - 1) / kRowThreads;
    return 256 + ((n + 255) / 256) * 256 + 3 * 4 * nblk;
}

int gsx_density_classify(int64_t n, const float* log_scales, const float* logit_opacities,
                         const float* grad_accum, const float* grad_count,
                         float grad_threshold, float dense_scale, float prune_scale,
                         float min_opacity, void* workspace, int64_t workspace_bytes,
                         uint32_t* totals, void* stream) {
    if (n <= 0 || !log_scales || !logit_opacities || !grad_accum || !grad_count || !workspace ||
        !totals)
        return GSX_ERR_INVALID;
    if (n > 0x3FFFFFFF) return GSX_ERR_TOO_LARGE;
    if (workspace_bytes < gsx_density_workspace_bytes(n)) return GSX_ERR_WORKSPACE;
    hipStream_t st = (hipStream_t)stream;
    uint8_t* cls = (uint8_t*)workspace;
    uint32_t* counts = (uint32_t*)((char*)workspace + ((n + 255) / 256) * 256);
    const int64_t nblk = blocks_for(n, kRowThreads);
    hipLaunchKernelGGL(k_density_classify, dim3((unsigned)nblk), dim3(kRowThreads), 0, st, n,
                       log_scales, logit_opacities, grad_accum, grad_count, grad_threshold,
                       dense_scale, prune_scale, min_opacity, cls, counts);
    GSX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_density_scan, dim3(1), dim3(1024), 0, st, nblk, counts, totals);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_density_emit(int64_t n, const void* workspace, int64_t workspace_bytes,
                     const uint32_t* totals, const gsx_row_table* table, int32_t means_col,
                     int32_t scales_col, int32_t quats_col, const double* split_samples,
                     float log_shrink, void* stream) {
    RowTable tab;
    if (n <= 0 || !workspace || !totals || !load_table(table, tab, false)) return GSX_ERR_INVALID;
    if (!col_ok(tab, means_col, 3) || !col_ok(tab, scales_col, 3) || !col_ok(tab, quats_col, 4))
        return GSX_ERR_INVALID;
    if (workspace_bytes < gsx_density_workspace_bytes(n)) return GSX_ERR_WORKSPACE;
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* cls = (const uint8_t*)workspace;
    const uint32_t* prefix =
        (const uint32_t*)((const char*)workspace + ((n + 255) / 256) * 256);
    hipLaunchKernelGGL(k_density_emit, dim3(blocks_for(n, kRowThreads)), dim3(kRowThreads), 0, st,
                       n, cls, prefix, totals, tab, means_col, scales_col, quats_col,
                       split_samples, log_shrink);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_relocate_scores(int64_t n, const float* grad_accum, const float* grad_count,
                        const float* logit_opacities, float min_opacity, float* target_score,
                        float* source_score, uint32_t* under_count, void* stream) {
    if (n < 0) return GSX_ERR_INVALID;
    if (n == 0) return GSX_OK;
    if (!grad_accum || !grad_count || !logit_opacities || !target_score || !source_score ||
        !under_count)
        return GSX_ERR_INVALID;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_relocate_scores, dim3(blocks_for(n, kRowThreads)), dim3(kRowThreads), 0,
                       st, n, grad_accum, grad_count, logit_opacities, min_opacity, target_score,
                       source_score, under_count);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

int gsx_density_relocate(int64_t k, const int64_t* src_rows, const int64_t* dst_rows,
                         const gsx_row_table* table, int32_t means_col, int32_t scales_col,
                         int32_t opac_col, const float* noise, float jitter, float reset_logit,
                         float log_shrink, float* staging, int64_t staging_floats,
                         void* stream) {
    RowTable tab;
    if (k < 0 || !load_table(table, tab, true)) return GSX_ERR_INVALID;
    if (k == 0) return GSX_OK;
    if (!src_rows || !dst_rows || !noise || !staging) return GSX_ERR_INVALID;
    if (!col_ok(tab, means_col, 3) || !col_ok(tab, scales_col, 3) || !col_ok(tab, opac_col, 1))
        return GSX_ERR_INVALID;
    int row_width = 0;
    for (int t = 0; t < tab.count; ++t)
        if (tab.role[t] == GSX_ROW_PARAM) row_width += tab.width[t];
    if (staging_floats < k * row_width) return GSX_ERR_WORKSPACE;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(blocks_for(k, kRowThreads));
    hipLaunchKernelGGL(k_relocate_gather, grid, dim3(kRowThreads), 0, st, k, src_rows, tab,
                       means_col, scales_col, opac_col, noise, jitter, reset_logit, log_shrink,
                       row_width, staging);
    GSX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_relocate_scatter, grid, dim3(kRowThreads), 0, st, k, dst_rows, tab,
                       row_width, (const float*)staging);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // extern "C"
