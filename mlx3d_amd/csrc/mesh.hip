// mesh.hip -- hard z-buffer triangle visibility on the shared tile binning
// (renderer/rasterizer.py:29-87, the mesh consumer of bin_gaussians).
//
// One 256-thread workgroup per 16x16 tile; the tile's faces (sorted by tile,
// then centroid depth) are staged through LDS 256 at a time as screen-space
// vertices (6 floats) and camera depths (3 floats), and every pixel keeps the
// nearest face whose barycentrics (same float32 operations as the
// reference) are all >= -1e-5 and whose interpolated depth exceeds znear.
// Ties keep the earlier face in list order.

#include <hip/hip_runtime.h>

#include "gsx.h"
#include "gsx_device.h"

namespace {

constexpr int kMeshThreads = 256;
constexpr int kMeshBatch = 256;

__global__ __launch_bounds__(kMeshThreads) void k_mesh_raster(
    int64_t n_faces, const float* __restrict__ tri_xy, const float* __restrict__ tri_z,
    const int32_t* __restrict__ ids, const int2* __restrict__ ranges, int64_t n_ids, int W,
    int H, int tiles_x, float znear, int32_t* __restrict__ pix_to_face,
    float* __restrict__ zbuf) {
    __shared__ float s_xy[kMeshBatch][6];
    __shared__ float s_z[kMeshBatch][3];
    __shared__ int s_f[kMeshBatch];

    const int tile = (int)gsx::xcd_remap(blockIdx.x, gridDim.x);
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int lx = threadIdx.x & 15, ly = threadIdx.x >> 4;
    const int px = tx * gsx::kTile + lx, py = ty * gsx::kTile + ly;
    const bool inside = px < W && py < H;
    const float cx = (float)px + 0.5f, cy = (float)py + 0.5f;

    // tile_span-style clamping: a malformed range cannot read out of bounds
    int2 r = ranges[tile];
    int64_t start = r.x < 0 ? 0 : r.x, end = r.y;
    if (end > n_ids) end = n_ids;
    if (end < start) end = start;

    int best_f = -1;
    float best_z = 1e30f;
    for (int64_t b = start; b < end; b += kMeshBatch) {
        const int cnt = (int)((end - b) < kMeshBatch ? (end - b) : kMeshBatch);
        __syncthreads();
        if ((int)threadIdx.x < cnt) {
            const int f = ids[b + threadIdx.x];
            const bool ok = (uint32_t)f < (uint64_t)n_faces;
            s_f[threadIdx.x] = ok ? f : -1;
#pragma unroll
            for (int k = 0; k < 6; ++k) s_xy[threadIdx.x][k] = ok ? tri_xy[6 * (int64_t)f + k] : 0.0f;
#pragma unroll
            for (int k = 0; k < 3; ++k) s_z[threadIdx.x][k] = ok ? tri_z[3 * (int64_t)f + k] : 0.0f;
        }
        __syncthreads();
        for (int j = 0; j < cnt; ++j) {
            const int f = s_f[j];
            if (f < 0) continue;
            const float ax = s_xy[j][0], ay = s_xy[j][1], bx = s_xy[j][2], by = s_xy[j][3];
            const float ccx = s_xy[j][4], ccy = s_xy[j][5];
            const float denom = (by - ccy) * (ax - ccx) + (ccx - bx) * (ay - ccy);
            if (fabsf(denom) < 1e-12f) continue;
            const float l0 = ((by - ccy) * (cx - ccx) + (ccx - bx) * (cy - ccy)) / denom;
            const float l1 = ((ccy - ay) * (cx - ccx) + (ax - ccx) * (cy - ccy)) / denom;
            const float l2 = 1.0f - l0 - l1;
            if (l0 < -1e-5f || l1 < -1e-5f || l2 < -1e-5f) continue;
            const float z = l0 * s_z[j][0] + l1 * s_z[j][1] + l2 * s_z[j][2];
            if (z <= znear) continue;
            if (z < best_z) {
                best_z = z;
                best_f = f;
            }
        }
    }
    if (inside) {
        const int64_t idx = (int64_t)py * W + px;
        pix_to_face[idx] = best_f;
        zbuf[idx] = best_f >= 0 ? best_z : 0.0f;
    }
}

}  // namespace

extern "C" {

int gsx_mesh_raster(int64_t n_faces, const float* tri_xy, const float* tri_z,
                    const int32_t* sorted_ids, int64_t num_ids, const int32_t* tile_ranges,
                    int32_t width, int32_t height, float znear, int32_t* pix_to_face,
                    float* zbuf, void* stream) {
    if (n_faces < 0 || num_ids < 0 || width <= 0 || height <= 0) return GSX_ERR_INVALID;
    if (!tile_ranges || !pix_to_face || !zbuf) return GSX_ERR_INVALID;
    if (n_faces > 0 && (!tri_xy || !tri_z)) return GSX_ERR_INVALID;
    if (num_ids > 0 && !sorted_ids) return GSX_ERR_INVALID;
    if (((uintptr_t)tile_ranges & 7u) != 0) return GSX_ERR_INVALID;
    if (n_faces == 0) num_ids = 0;
    const int tiles_x = (width + gsx::kTile - 1) / gsx::kTile;
    const int tiles_y = (height + gsx::kTile - 1) / gsx::kTile;
    hipLaunchKernelGGL(k_mesh_raster, dim3((unsigned)(tiles_x * tiles_y)), dim3(kMeshThreads), 0,
                       (hipStream_t)stream, n_faces, tri_xy, tri_z, sorted_ids,
                       (const int2*)tile_ranges, num_ids, width, height, tiles_x, znear,
                       pix_to_face, zbuf);
    GSX_LAUNCH_CHECK();
    return GSX_OK;
}

}  // extern "C"
