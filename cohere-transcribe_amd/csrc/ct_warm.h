// ct_warm.h — device side of the decode GEMMs' weight read-ahead (CtWarmSet).
#pragma once
#include <stdio.h>
#include <stdlib.h>
#include "ct_dev.h"
#include "ct_launch.h"

// Read-ahead workgroup j of XCD x.  The GEMM workgroups on XCD x are
// i = x + 8 k (GEMM workgroup i runs on XCD i % 8), each reading cb column
// blocks of per tiles; this workgroup reads the units (k, c) numbered
// u = k * cb + c = j, j + rows, j + 2 rows, ...  Dealing 16-column units
// rather than whole GEMM workgroups keeps each read-ahead workgroup's share
// the same whatever columns per workgroup the GEMM takes.  The caller places
// this workgroup on XCD x, so the tiles land in the L2 the GEMM reads them from.
template <int NT>
__device__ __forceinline__ void ct_warm_tiles(const CtWarmSet &ws, int x, int j) {
    unsigned acc = 0;
    for (int t = 0; t < ws.n; t++) {
        const CtWarm w = ws.t[t];
        const int U = (w.gx * w.gy - x + 7) / 8 * w.cb;      // units on XCD x
        for (int u = j; u < U; u += ws.rows) {
            const int i = x + 8 * (u / w.cb), c = u % w.cb;
            const int cx = w.heads ? ct_qkv_col(i / w.gy, w.cb) : i / w.gy, ks = i % w.gy;
            const uint4 *p = reinterpret_cast<const uint4 *>(
                w.W + ((((long)cx * w.cb + c) * w.nsteps + (long)ks * w.per) << 9));
#pragma unroll 8
            for (int e = threadIdx.x; e < w.per * 64; e += NT) {
                const uint4 v = p[e];
                acc ^= v.x ^ v.y ^ v.z ^ v.w;
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
