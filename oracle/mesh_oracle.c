/*
 * mesh_oracle.c -- CPU restatement of the hard z-buffer mesh rasterizer
 * kernel (renderer/rasterizer.py:29-87).  TEST INFRASTRUCTURE ONLY (the
 * checker of tests/); nothing in the product package links, loads or calls
 * it.  Float32, each operation rounded once (-ffp-contract=off), in the
 * reference kernel's operation order.
 */
#include <math.h>
#include <stdint.h>

#include "gsx_oracle.h"

static int clamp_threads(int n) { return n > 0 ? n : 1; }

void orc_mesh_raster(int64_t n_faces, const float* tri_xy, const float* tri_z,
                     const int32_t* sorted_ids, const int32_t* tile_ranges, int width,
                     int height, float znear, int32_t* pix_to_face, float* zbuf,
                     int nthreads) {
    const int tiles_x = (width + 15) / 16;
#pragma omp parallel for num_threads(clamp_threads(nthreads)) schedule(static)
    for (int64_t pid = 0; pid < (int64_t)width * height; ++pid) {
        const int px = (int)(pid % width), py = (int)(pid / width);
        const int tile = (py / 16) * tiles_x + px / 16;
        const float cx = (float)px + 0.5f, cy = (float)py + 0.5f;
        int best_f = -1;
        float best_z = 1e30f;
        for (int32_t k = tile_ranges[2 * tile]; k < tile_ranges[2 * tile + 1]; ++k) {
            const int f = sorted_ids[k];
            if (f < 0 || f >= n_faces) continue;
            const float* t = tri_xy + 6 * (int64_t)f;
            const float ax = t[0], ay = t[1], bx = t[2], by = t[3], ccx = t[4], ccy = t[5];
            /* rasterizer.py:63-73 */
            const float denom = (by - ccy) * (ax - ccx) + (ccx - bx) * (ay - ccy);
            if (fabsf(denom) < 1e-12f) continue;
            const float l0 = ((by - ccy) * (cx - ccx) + (ccx - bx) * (cy - ccy)) / denom;
            const float l1 = ((ccy - ay) * (cx - ccx) + (ax - ccx) * (cy - ccy)) / denom;
            const float l2 = 1.0f - l0 - l1;
            if (l0 < -1e-5f || l1 < -1e-5f || l2 < -1e-5f) continue;
            const float* zz = tri_z + 3 * (int64_t)f;
            const float z = l0 * zz[0] + l1 * zz[1] + l2 * zz[2];
            if (z <= znear) continue;
            if (z < best_z) {
                best_z = z;
                best_f = f;
            }
        }
        pix_to_face[pid] = best_f;                  /* rasterizer.py:76-80 */
        zbuf[pid] = best_f >= 0 ? best_z : 0.0f;
    }
}
