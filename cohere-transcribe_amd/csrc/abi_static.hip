// abi_static.hip — device scratch for backend_rel_pos_mhsa_noalloc.
//
// The relative-position MHSA of one clip needs Q, K, V (T rows each), the
// position projection P (2T - 1 rows) and the attention output O (T rows):
// (6T - 1) x ENC_D floats, which backend_rel_pos_mhsa takes from the
// caller's workspace.  For callers that cannot allocate, the same work runs
// over a file-scope device array sized for the longest clip the reference
// batches unchunked (30 s, transcribe.c:894: T = 376 frames), 11.5 MB per
// device, held until the process ends.
// Host code never passes the array's name to a kernel: its device address
// is looked up once per device (ct_static_init, from backend_init with the
// device current) and kept per device.
#include <hip/hip_runtime.h>

#include "../../include/model_types.h"
#include "ct_launch.h"
#include <stdio.h>
#include <stdlib.h>

#define CT_STATIC_DEVICES 8

static_assert(CT_MHSA_SCRATCH_FLOATS(1) == (size_t)5 * ENC_D, "row width");
static __device__ __align__(256) float scratch[CT_MHSA_SCRATCH_FLOATS(CT_STATIC_MHSA_MAX_T)];

static float *g_scratch[CT_STATIC_DEVICES];

extern "C" void ct_static_init(int dev) {
    if (dev < 0 || dev >= CT_STATIC_DEVICES) {
        fprintf(stderr, "ct_static_init: device %d out of range\n", dev);
        exit(1);
    }
    if (g_scratch[dev]) return;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        fprintf(stderr, "ct_static_init: hipGetSymbolAddress failed on device %d: %s\n", dev,
                hipGetErrorString(e));
        exit(1);
    }
    g_scratch[dev] = (float *)p;
}

extern "C" size_t ct_static_scratch_floats(void) { return sizeof(scratch) / sizeof(float); }

extern "C" float *ct_static_scratch(int dev) {
    return (dev >= 0 && dev < CT_STATIC_DEVICES) ? g_scratch[dev] : nullptr;
}
