// ct_warm.h — device side of the decode GEMMs' weight read-ahead (CtWarmSet).
#pragma once
#include <stdio.h>
#include <stdlib.h>
#include "ct_dev.h"
#include "ct_launch.h"

// Read-ahead workgroup j of XCD x: reads the tiles of the GEMM workgroups
// i = x + 8 j, x + 8 (j + rows), ... of each listed GEMM.  GEMM workgroup i
// runs on XCD i % 8; the caller places this workgroup on XCD x, so the tiles
// land in the L2 that GEMM workgroup reads them from.
template <int NT>
__device__ __forceinline__ void ct_warm_tiles(const CtWarmSet &ws, int x, int j) {
    unsigned acc = 0;
    for (int t = 0; t < ws.n; t++) {
        const CtWarm w = ws.t[t];
        const int G = w.gx * w.gy;
        for (int i = x + 8 * j; i < G; i += 8 * ws.rows) {
            const int cx = w.heads ? ct_qkv_col(i / w.gy) : i / w.gy, ks = i % w.gy;
            for (int c = 0; c < w.cb; c++) {
                const uint4 *p = reinterpret_cast<const uint4 *>(
                    w.W + ((((long)cx * w.cb + c) * w.nsteps + (long)ks * w.per) << 9));
#pragma unroll 8
                for (int e = threadIdx.x; e < w.per * 64; e += NT) {
                    const uint4 v = p[e];
                    acc ^= v.x ^ v.y ^ v.z ^ v.w;
                }
            }
        }
    }
    if (acc == ws.magic) ws.sink[threadIdx.x] = acc;
}

// Host-side check of a read-ahead set; returns the extra rows it needs.
static inline int ct_warm_rows(const CtWarmSet *ws, const char *who) {
    if (!ws || ws->n == 0) return 0;
    bool ok = ws->n > 0 && ws->n <= 4 && ws->rows >= 1 && ws->rows <= 128 && ws->sink;
    for (int t = 0; ok && t < ws->n; t++)
        ok = ws->t[t].gx >= 0 && ws->t[t].gy >= 1 && ws->t[t].cb >= 1 && ws->t[t].per >= 1 &&
             ws->t[t].per * ws->t[t].gy <= ws->t[t].nsteps &&
             (ws->t[t].gx == 0 || ws->t[t].W) && ((uintptr_t)ws->t[t].W & 15) == 0;
    if (!ok) {
        fprintf(stderr, "%s: read-ahead needs 1..4 tiled GEMMs, 1..128 rows and a sink\n", who);
        exit(1);
    }
    return ws->rows;
}
