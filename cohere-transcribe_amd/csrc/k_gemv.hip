// k_gemv.hip — the decode step's GEMMs: one row per KV slot (M <= a few
// hundred), weights streamed once per step.
//
// Activations arrive pre-split (hi + lo bf16) in frag layout, so every load
// a lane issues is one contiguous 16-byte piece of a 1-KB run: no strided row
// reads, no split arithmetic in the GEMM.  A workgroup of 8 wavefronts owns
// 16*CB output columns, one 64-row block and one K-slice of 256*SPW columns;
// wavefront w takes K-steps w, w+8, ... of the slice and issues all of its
// loads before the first MFMA.  The 8 wave tiles are summed in LDS in wave
// order.  With ksplit > 1 the slice sums are written as partial rows and the
// consumer (the next LayerNorm, or the attention's query load) adds them in
// slice order.  The split is a function of (N, K) only, so a row's bits never
// depend on how many rows the step has.
//
// Semantics per output: backends/cpu/backend.c:124-182 (y = x W^T + b, ReLU,
// fmadd), with x = hi + lo exactly representable to 2^-17 relative.
#include "ct_dev.h"
#include "ct_launch.h"
#include "../../include/model_types.h"
#include <stdio.h>
#include <stdlib.h>

namespace {

constexpr int GV_WAVES = 8;
// Launch order: K-slices vary fastest (grid x), so with 8 K-slices each XCD
// (its own L2) serves one slice and fetches only that slice's activations;
// column blocks follow (grid y), a QKV launch's dealt head by head over the
// XCDs (ct_qkv_col) so that head h's blocks run where the attention's head-h
// workgroups read them.

template <int CB, int SPW>
__global__ __launch_bounds__(64 * GV_WAVES) void gemv_kernel(CtGemv g) {
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int r = lane & 15, kg = lane >> 4;
    const int pos = blockIdx.y;
    const int c0 = (g.out == CT_GV_QKV ? ct_qkv_col(pos) : pos) * 16 * CB;
    const int ks = blockIdx.x, z = blockIdx.z, m0 = z * 64;
    const int nsteps = g.K >> 5;
    const int s0 = ks * (GV_WAVES * SPW);
    int nrb = min(4, (g.M - m0 + 15) >> 4);
    if (g.m_active && m0 > 0) {
        // rows past the first block may be unused spare rows this step
        const int ma = *g.m_active;
        if (m0 >= ma) return;
        nrb = min(nrb, (ma - m0 + 15) >> 4);
    }
    const uint16_t *ablk = g.A + ((long)z * nsteps << 12);
    u16x8 ah[SPW][4], al[SPW][4], wv[SPW][CB];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int st = s0 + w + GV_WAVES * j;
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            if (rb < nrb) {
                const uint16_t *p = ablk + ((long)(st * 4 + rb) << 10) + lane * 8;
                ah[j][rb] = *reinterpret_cast<const u16x8 *>(p);
                al[j][rb] = *reinterpret_cast<const u16x8 *>(p + 512);
            } else {
                ah[j][rb] = al[j][rb] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
            wv[j][cb] = *reinterpret_cast<const u16x8 *>(
                g.wtile ? g.W + ((((long)(c0 >> 4) + cb) * nsteps + st) << 9) + lane * 8
                        : g.W + (long)(c0 + cb * 16 + r) * g.K + st * 32 + kg * 8);
    }
    f32x4 acc[4][CB];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++) acc[rb][cb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < SPW; j++)
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            if (rb >= nrb) break;
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                const bf16x8 b = as_bf16x8(wv[j][cb]);
                acc[rb][cb] = mfma16(as_bf16x8(ah[j][rb]), b, acc[rb][cb]);
                acc[rb][cb] = mfma16(as_bf16x8(al[j][rb]), b, acc[rb][cb]);
            }
        }
    __shared__ float part[GV_WAVES][64][16 * CB + 1];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int j = 0; j < 4; j++) part[w][rb * 16 + kg * 4 + j][cb * 16 + r] = acc[rb][cb][j];
    __syncthreads();

    if (g.out == CT_GV_FRAG) {
        // one thread per (row, 8 consecutive columns): a 16-byte piece per plane
        for (int e = tid; e < 64 * 2 * CB; e += 64 * GV_WAVES) {
            const int row = e / (2 * CB), grp = e % (2 * CB), m = m0 + row;
            if (m >= g.M) continue;
            u16x8 hv, lv;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int cc = grp * 8 + i;
                float s = part[0][row][cc];
#pragma unroll
                for (int ww = 1; ww < GV_WAVES; ww++) s += part[ww][row][cc];
                if (g.bias) s += bf2f(g.bias[c0 + cc]);
                if (g.relu) s = s > 0.0f ? s : 0.0f;
                uint16_t hh, ll;
                split_bf16(s, hh, ll);
                hv[i] = hh; lv[i] = ll;
            }
            const long o = ct_frag_off(m, c0 + grp * 8, g.N);
            *reinterpret_cast<u16x8 *>(g.F + o) = hv;
            *reinterpret_cast<u16x8 *>(g.F + o + 512) = lv;
        }
        return;
    }
    for (int e = tid; e < 64 * 16 * CB; e += 64 * GV_WAVES) {
        const int row = e / (16 * CB), cc = e % (16 * CB), m = m0 + row, col = c0 + cc;
        if (m >= g.M) continue;
        float s = part[0][row][cc];
#pragma unroll
        for (int ww = 1; ww < GV_WAVES; ww++) s += part[ww][row][cc];
        if (g.out == CT_GV_PARTIAL) {
            g.Y[((long)ks * g.M + m) * g.N + col] = s;
            continue;
        }
        if (g.bias) s += bf2f(g.bias[col]);
        if (g.relu) s = s > 0.0f ? s : 0.0f;
        if (g.out == CT_GV_DENSE || col < DEC_D) {
            g.Y[(long)m * g.ldy + col] = s;
            continue;
        }
        const long ro = g.rowoff[m];
        if (ro < 0) continue;
        const int seg = col / DEC_D, c = col - seg * DEC_D;
        const long off = ro + (long)(c >> 7) * g.hstride + (c & 127);
        void *base = seg == 1 ? g.kc : g.vc;
        if (g.kv_bf16) reinterpret_cast<uint16_t *>(base)[off] = f2bf(s);
        else reinterpret_cast<float *>(base)[off] = s;
    }
}

// The weight reads of gemv_kernel alone (tiled weights): the same grid, and
// workgroup (x, y, z) reads the same 1 KB tiles as the GEMM's workgroup, one
// 16-byte piece per lane, wave w taking tiles w, w + 8, ... with four loads
// in flight; no activations, no MFMAs.  The XOR of what a workgroup read
// goes to sink[linear workgroup id] so the loads are not removed.  A floor
// for the GEMM's duration at its grid, for benchmarking.
template <int CB>
__global__ __launch_bounds__(64 * GV_WAVES) void read_floor_kernel(CtGemv g, int ksplit, float *sink) {
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int pos = blockIdx.y;
    const int cbk = (g.out == CT_GV_QKV ? ct_qkv_col(pos) : pos) * CB;
    const int ks = blockIdx.x;
    const int nsteps = g.K >> 5, per = nsteps / ksplit, s0 = ks * per;
    const int ntile = CB * per;
    u16x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int t0 = w; t0 < ntile; t0 += 4 * GV_WAVES) {
        u16x8 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t = min(t0 + u * GV_WAVES, ntile - 1);
            const int cb = t / per, st = s0 + t % per;
            v[u] = *reinterpret_cast<const u16x8 *>(g.W + ((((long)cbk + cb) * nsteps + st) << 9) + lane * 8);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) x ^= v[u];
    }
    __shared__ unsigned red[GV_WAVES];
    unsigned r = (unsigned)x[0] ^ x[1] ^ x[2] ^ x[3] ^ x[4] ^ x[5] ^ x[6] ^ x[7];
    r = wave_xor(r);
    if (lane == 0) red[w] = r;
    __syncthreads();
    if (tid == 0) {
        unsigned a = 0;
#pragma unroll
        for (int i = 0; i < GV_WAVES; i++) a ^= red[i];
        const long b = ((long)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
        sink[b] = __uint_as_float(a);
    }
}

// One thread per 16-byte piece of the tiled weight.
__global__ __launch_bounds__(256) void tile_w_kernel(const uint16_t *W, uint16_t *Wt, int N, int K) {
    const long piece = blockIdx.x * 256L + threadIdx.x, pieces = (long)N * K / 8;
    if (piece >= pieces) return;
    const int lane = (int)(piece & 63);
    const long tile = piece >> 6;
    const int nsteps = K >> 5, st = (int)(tile % nsteps), rb = (int)(tile / nsteps);
    const int n = rb * 16 + (lane & 15), k = st * 32 + (lane >> 4) * 8;
    *reinterpret_cast<u16x8 *>(Wt + piece * 8) = *reinterpret_cast<const u16x8 *>(W + (long)n * K + k);
}

[[noreturn]] void gv_fatal(const char *msg, const CtGemv *g) {
    fprintf(stderr, "ctk_gemv: %s (M=%d N=%d K=%d ksplit=%d out=%d)\n", msg, g->M, g->N, g->K,
            g->ksplit, g->out);
    exit(1);
}

}  // namespace

extern "C" void ctk_tile_w(const uint16_t *W, uint16_t *Wt, int N, int K, hipStream_t s) {
    if (N % 16 || K % 32 || ((uintptr_t)W & 15) || ((uintptr_t)Wt & 15)) {
        fprintf(stderr, "ctk_tile_w: needs N %% 16 == 0, K %% 32 == 0 and 16-byte aligned buffers\n");
        exit(1);
    }
    const long pieces = (long)N * K / 8;
    hipLaunchKernelGGL(tile_w_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, s, W, Wt, N, K);
}

extern "C" int ctk_gemv_sizeof(void) { return (int)sizeof(CtGemv); }
extern "C" int ctk_warmset_sizeof(void) { return (int)sizeof(CtWarmSet); }

extern "C" int ctk_gemv_ksplit(int N, int K) {
    if (N <= DEC_D && K == DEC_D) return 4;       // 256-column slices, one K-step per wave
    if (N <= DEC_D && K == DEC_FF) return 8;      // 512-column slices
    return 1;
}

// columns per workgroup: 64 for the LM head; 32 for the long-K projection
// (its 512-column K-slices leave 256 workgroups); else 16
static int gv_cb(int N, int K) { return (N >= 8192 && N % 64 == 0) ? 4 : (K >= 4096 && N % 32 == 0) ? 2 : 1; }

extern "C" long ctk_gemv_read_floor_blocks(const CtGemv *g) {
    const int ksplit = g->ksplit < 1 ? 1 : g->ksplit, cb = gv_cb(g->N, g->K);
    return (long)ksplit * (g->N / (16 * cb)) * ((g->M + 63) / 64);
}

extern "C" void ctk_gemv_read_floor(const CtGemv *g, float *sink, hipStream_t s) {
    if (g->M <= 0) return;
    const int ksplit = g->ksplit < 1 ? 1 : g->ksplit, cb = gv_cb(g->N, g->K);
    if (!g->wtile || g->K % (256 * ksplit) != 0 || g->N % (16 * cb) != 0 || ((uintptr_t)g->W & 15))
        gv_fatal("read floor needs tiled, 16-byte aligned weights of a supported shape", g);
    const dim3 grid(ksplit, g->N / (16 * cb),
                    (g->M + 63) / 64);
    if (cb == 1) hipLaunchKernelGGL(read_floor_kernel<1>, grid, dim3(64 * GV_WAVES), 0, s, *g, ksplit, sink);
    else if (cb == 2) hipLaunchKernelGGL(read_floor_kernel<2>, grid, dim3(64 * GV_WAVES), 0, s, *g, ksplit, sink);
    else hipLaunchKernelGGL(read_floor_kernel<4>, grid, dim3(64 * GV_WAVES), 0, s, *g, ksplit, sink);
}


extern "C" void ctk_gemv_warm(const CtGemv *g, CtWarm *w) {
    const int ksplit = g->ksplit < 1 ? 1 : g->ksplit, cb = gv_cb(g->N, g->K);
    w->W = g->W;
    w->gx = g->wtile ? g->N / (16 * cb) : 0;
    w->gy = ksplit; w->cb = cb;
    w->per = g->K / ksplit / 32; w->nsteps = g->K / 32;
    w->heads = g->out == CT_GV_QKV;
}

extern "C" void ctk_gemv(const CtGemv *g, hipStream_t s) {
    if (g->M <= 0) return;
    const int ksplit = g->ksplit < 1 ? 1 : g->ksplit;
    if (g->K % (256 * ksplit) != 0 || g->N % 16 != 0) gv_fatal("unsupported shape", g);
    if (ksplit > 1 && g->out != CT_GV_PARTIAL) gv_fatal("a K split needs partial output", g);
    if (g->out == CT_GV_QKV && g->N != 3 * DEC_D) gv_fatal("QKV output needs N = 3*DEC_D", g);
    if (((uintptr_t)g->A & 15) || ((uintptr_t)g->W & 15) ||
        (g->out == CT_GV_FRAG && ((uintptr_t)g->F & 15)))
        gv_fatal("operands must be 16-byte aligned", g);
    const int spw = g->K / ksplit / 256;
    const int cb = gv_cb(g->N, g->K);
    const dim3 grid(ksplit, g->N / (16 * cb),
                    (g->M + 63) / 64);
    const dim3 block(64 * GV_WAVES);
#define GV_CASE(CB, SPW)                                                          \
    if (cb == CB && spw == SPW) {                                                 \
        hipLaunchKernelGGL((gemv_kernel<CB, SPW>), grid, block, 0, s, *g);        \
        return;                                                                   \
    }
    GV_CASE(1, 1) GV_CASE(1, 2) GV_CASE(1, 4) GV_CASE(2, 1) GV_CASE(2, 2) GV_CASE(2, 4)
    GV_CASE(4, 1) GV_CASE(4, 2) GV_CASE(4, 4)
#undef GV_CASE
    gv_fatal("no kernel for this K slice", g);
}
