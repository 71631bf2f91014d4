// phase_handoff.hip — what it costs to hand one decode phase's output to the
// next: a kernel boundary inside a HIP graph, against one kernel whose two
// phases meet at device-scope ready counters.  A benchmark for the decode
// step's launch structure; not part of the library.
//
// Shape (a decode GEMM pair at a 64-slot step): 256 workgroups of 512 threads,
// one per CU.  Each phase streams a 16-KB weight tile per workgroup from HBM
// (4 MB a phase; 16 weight sets rotate so the tiles are not in any cache).  A
// phase-1 workgroup writes a 1-KB piece of a 256-KB output; a phase-2
// workgroup reads a 64-KB quarter of it, as a 16-row group reads its
// activations (16 rows x 1024 columns x hi + lo bf16).
//
//   two launches  phase1 then phase2, plain stores and loads.
//   xcd counters  one kernel.  A producer writes its piece with 16-byte
//                 device-coherent stores (sc1), waits for them, and adds 1 to
//                 the counter of its workgroup group (workgroup id mod 8, 8
//                 counters 256 bytes apart).  It then issues its phase-2 weight
//                 loads, lanes 0..7 poll the 8 counters, and it reads its
//                 quarter with 16-byte device-coherent loads.
//   one counter   the same with a single counter that all 256 producers add to.
//   acquire       plain stores, a release add on the single counter, an
//                 acquire fence after the wait (the L2 write-back and
//                 invalidate), plain loads.
//
// Counters grow across the iterations of a graph (iteration i waits for
// (i + 1) x producers), so no reset runs between iterations; a fill kernel
// clears them before each replay.  Every wait is bounded: a wait that gives up
// sets a flag, the kernel finishes, and the program exits 1.  Every variant's
// output must equal the two-launch output bit for bit (exit 1 otherwise).
//
//   phase_handoff            graph replays, per-iteration times
//   phase_handoff --eager    the same launches without graphs, for a kernel trace
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define CHK(x)                                                                               \
    do {                                                                                     \
        hipError_t e_ = (x);                                                                 \
        if (e_ != hipSuccess) {                                                              \
            fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);   \
            exit(1);                                                                         \
        }                                                                                    \
    } while (0)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int NWG = 256, NT = 512;
constexpr int TILE = 1024;                 // 16-byte pieces of weight per workgroup and phase (16 KB)
constexpr int PIECE = 64;                  // 16-byte pieces a producer writes (1 KB)
constexpr int OUT = NWG * PIECE;           // 16384 pieces = 256 KB
constexpr int QUARTER = OUT / 4;           // what a consumer reads (64 KB)
constexpr int GROUPS = 8, CSTRIDE = 64;    // counters: one per workgroup group, 256 bytes apart
constexpr long SPIN = 1 << 16;             // bounded wait
constexpr int ITER = 200, ROT = 16;

enum Variant { TWO = 0, XCD = 1, ONE = 2, ACQ = 3, NVAR = 4 };
static const char *vname[NVAR] = {"two launches", "xcd counters", "one counter", "acquire"};

__device__ __forceinline__ u32x4 stream_tile(const u32x4 *w) {
    u32x4 v[TILE / NT], acc = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < TILE / NT; i++) v[i] = __builtin_nontemporal_load(w + threadIdx.x + NT * i);
#pragma unroll
    for (int i = 0; i < TILE / NT; i++) acc ^= v[i];
    return acc;
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rsrc(const f32x4 *O) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<f32x4 *>(O), 0, OUT * 16, 0x00020000);
}
__device__ __forceinline__ f32x4 piece_of(u32x4 a) {
    const float f = (float)(a.x ^ a.y ^ a.z ^ a.w);
    return f32x4{f, f + 1.f, f + 2.f, (float)threadIdx.x};
}
// sc1 = bit 4 of the buffer instructions' cache-policy operand on gfx950
constexpr int SC1 = 16;
template <bool COHERENT> __device__ __forceinline__ float read_quarter(const f32x4 *O) {
    const int base = (blockIdx.x & 3) * QUARTER;
    float x = 0.f;
#pragma unroll 8
    for (int j = 0; j < QUARTER / NT; j++) {
        const int i = base + threadIdx.x + NT * j;
        const f32x4 v = COHERENT ? __builtin_amdgcn_raw_buffer_load_b128(out_rsrc(O), i * 16, 0, SC1) : O[i];
        x += v.x + v.y + v.z + v.w;
    }
    return x;
}

__global__ __launch_bounds__(NT) void phase1(const u32x4 *W, f32x4 *O) {
    const u32x4 a = stream_tile(W + (long)blockIdx.x * TILE);
    if (threadIdx.x < PIECE) O[blockIdx.x * PIECE + threadIdx.x] = piece_of(a);
}
__global__ __launch_bounds__(NT) void phase2(const u32x4 *W, const f32x4 *O, float *R) {
    const u32x4 b = stream_tile(W + (long)(NWG + blockIdx.x) * TILE);
    R[blockIdx.x * NT + threadIdx.x] = read_quarter<false>(O) + (float)(b.x ^ b.w);
}

template <int V>
__global__ __launch_bounds__(NT) void fused(const u32x4 *W, f32x4 *O, float *R, int *cnt, int iter, int *flag) {
    const u32x4 a = stream_tile(W + (long)blockIdx.x * TILE);
    if (threadIdx.x < PIECE) {
        const int i = blockIdx.x * PIECE + threadIdx.x;
        if (V == ACQ) O[i] = piece_of(a);
        else __builtin_amdgcn_raw_buffer_store_b128(piece_of(a), out_rsrc(O), i * 16, 0, SC1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (V == ACQ) {
            __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            __builtin_amdgcn_s_waitcnt(0);       // this wave's stores (all of the piece) are done
            __hip_atomic_fetch_add(V == XCD ? cnt + (blockIdx.x % GROUPS) * CSTRIDE : cnt, 1,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // phase 2's weight loads are in flight during the wait
    u32x4 v[TILE / NT];
    const u32x4 *w2 = W + (long)(NWG + blockIdx.x) * TILE;
#pragma unroll
    for (int i = 0; i < TILE / NT; i++) v[i] = __builtin_nontemporal_load(w2 + threadIdx.x + NT * i);
    const int pollers = V == XCD ? GROUPS : 1;
    if ((int)threadIdx.x < pollers) {
        const int *c = V == XCD ? cnt + threadIdx.x * CSTRIDE : cnt;
        const int want = (iter + 1) * (V == XCD ? NWG / GROUPS : NWG);
        long k = 0;
        while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < want && k < SPIN) {
            __builtin_amdgcn_s_sleep(1);
            k++;
        }
        if (k >= SPIN) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (V == ACQ) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    u32x4 b = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < TILE / NT; i++) b ^= v[i];
    R[blockIdx.x * NT + threadIdx.x] = read_quarter<V != ACQ>(O) + (float)(b.x ^ b.w);
}
__global__ void clear_counters(int *cnt) {
    for (int i = threadIdx.x; i < GROUPS * CSTRIDE; i += blockDim.x) cnt[i] = 0;
}

static u32x4 *W;
static f32x4 *O;
static float *R;
static int *cnt, *flag;
static const size_t WSET = (size_t)2 * NWG * TILE * sizeof(u32x4);   // both phases' tiles
static const u32x4 *wset(int i) { return (const u32x4 *)((const char *)W + WSET * (i % ROT)); }

static void enqueue(int var, int iters, hipStream_t st) {
    hipLaunchKernelGGL(clear_counters, dim3(1), dim3(256), 0, st, cnt);
    for (int i = 0; i < iters; i++) {
        if (var == TWO) {
            hipLaunchKernelGGL(phase1, dim3(NWG), dim3(NT), 0, st, wset(i), O);
            hipLaunchKernelGGL(phase2, dim3(NWG), dim3(NT), 0, st, wset(i), O, R);
        } else if (var == XCD) {
            hipLaunchKernelGGL(fused<XCD>, dim3(NWG), dim3(NT), 0, st, wset(i), O, R, cnt, i, flag);
        } else if (var == ONE) {
            hipLaunchKernelGGL(fused<ONE>, dim3(NWG), dim3(NT), 0, st, wset(i), O, R, cnt, i, flag);
        } else {
            hipLaunchKernelGGL(fused<ACQ>, dim3(NWG), dim3(NT), 0, st, wset(i), O, R, cnt, i, flag);
        }
    }
    CHK(hipGetLastError());
}

static int cmpd(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return x < y ? -1 : x > y;
}

int main(int argc, char **argv) {
    const bool eager = argc > 1 && !strcmp(argv[1], "--eager");
    hipDeviceProp_t p;
    CHK(hipGetDeviceProperties(&p, 0));
    printf("device %s, %d CUs; %s\n", p.gcnArchName, p.multiProcessorCount, eager ? "eager launches" : "graph replays");
    fflush(stdout);
    // one workgroup per CU must fit at once, or a wait could outlast its producers
    if (p.multiProcessorCount < NWG) {
        printf("needs %d CUs\n", NWG);
        return 1;
    }
    CHK(hipMalloc(&W, WSET * ROT));
    CHK(hipMalloc(&O, (size_t)OUT * 16));
    CHK(hipMalloc(&R, (size_t)NWG * NT * 4));
    CHK(hipMalloc(&cnt, GROUPS * CSTRIDE * 4));
    CHK(hipMalloc(&flag, 4));
    {
        // deterministic, varied weights
        uint32_t *h = (uint32_t *)malloc(WSET * ROT);
        uint32_t s = 12345u;
        for (size_t i = 0; i < WSET * ROT / 4; i++) h[i] = s = s * 1664525u + 1013904223u;
        CHK(hipMemcpy(W, h, WSET * ROT, hipMemcpyHostToDevice));
        free(h);
    }
    CHK(hipMemset(O, 0, (size_t)OUT * 16));
    CHK(hipMemset(flag, 0, 4));
    hipStream_t st;
    CHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    hipEvent_t e0, e1;
    CHK(hipEventCreate(&e0));
    CHK(hipEventCreate(&e1));

    // outputs of one iteration of every variant, against the two-launch output
    static float ref[NWG * NT], got[NWG * NT];
    int bad = 0;
    for (int v = 0; v < NVAR; v++) {
        CHK(hipMemset(O, 0, (size_t)OUT * 16));
        enqueue(v, 1, st);
        CHK(hipMemcpyAsync(v ? got : ref, R, sizeof ref, hipMemcpyDeviceToHost, st));
        CHK(hipStreamSynchronize(st));
        if (v && memcmp(ref, got, sizeof ref)) {
            printf("%s: output differs from two launches\n", vname[v]);
            bad = 1;
        }
    }

    double us[NVAR];
    for (int v = 0; v < NVAR; v++) {
        hipGraphExec_t ge = nullptr;
        if (!eager) {
            hipGraph_t g;
            CHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            enqueue(v, ITER, st);
            CHK(hipStreamEndCapture(st, &g));
            CHK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            CHK(hipGraphDestroy(g));
        }
        double t[5];
        for (int r = 0; r < 5; r++) {
            float ms;
            CHK(hipEventRecord(e0, st));
            if (eager) enqueue(v, ITER, st);
            else CHK(hipGraphLaunch(ge, st));
            CHK(hipEventRecord(e1, st));
            CHK(hipEventSynchronize(e1));
            CHK(hipEventElapsedTime(&ms, e0, e1));
            t[r] = ms * 1e3 / ITER;
        }
        qsort(t, 5, sizeof t[0], cmpd);
        us[v] = t[2];
        if (ge) CHK(hipGraphExecDestroy(ge));
        printf("%-13s %6.2f us per phase pair (median of 5 runs of %d)\n", vname[v], us[v], ITER);
        fflush(stdout);
    }
    int timeouts = 0;
    CHK(hipMemcpy(&timeouts, flag, 4, hipMemcpyDeviceToHost));
    printf("hand-off in one kernel minus a kernel boundary: xcd counters %+.2f us, one counter %+.2f us, "
           "acquire %+.2f us; waits given up: %d; outputs %s\n",
           us[XCD] - us[TWO], us[ONE] - us[TWO], us[ACQ] - us[TWO], timeouts, bad ? "DIFFER" : "equal");
    return bad || timeouts ? 1 : 0;
}
