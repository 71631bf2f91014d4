// k_gemv.hip — the decode step's GEMMs: one row per KV slot (M <= a few
// hundred), weights streamed once per step.
//
// Activations arrive pre-split (hi + lo bf16) in frag layout, so every load
// a lane issues is one contiguous 16-byte piece of a 1-KB run: no strided row
// reads, no split arithmetic in the GEMM.  A workgroup of 8 wavefronts owns
// 16*CB output columns, 16*RB rows and one K-slice of 256*SPW columns;
// wavefront w takes K-steps w, w+8, ... of the slice and issues all of its
// loads before the first MFMA.  The 8 wave tiles are summed in LDS in wave
// order.  With ksplit > 1 the slice sums are written as partial rows and the
// consumer (the next LayerNorm, or the attention's query load) adds them in
// slice order.  The split is a function of (N, K) only, and every tiling
// gives an element the same MFMA sequence (its K-steps in order, hi then lo,
// then the wave sum), so a row's bits never depend on how many rows the step
// has or on the tiling chosen for them.
//
// Two fused forms: the residual projection (CT_GV_RESID) adds its sums into
// the residual rows and leaves per-block LayerNorm statistics, and a GEMM with
// CtGemv.X normalises those rows itself instead of reading frag activations.
//
// Semantics per output: backends/cpu/backend.c:124-182 (y = x W^T + b, ReLU,
// fmadd), with x = hi + lo exactly representable to 2^-17 relative.
#include "ct_dev.h"
#include "ct_launch.h"
#include "ct_warm.h"
#include "../../include/model_types.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

namespace {

constexpr int GV_WAVES = 8;
// Launch order: K-slices vary fastest (grid x), so with 8 K-slices each XCD
// (its own L2) serves one slice and fetches only that slice's activations;
// column blocks follow (grid y), a QKV launch's dealt head by head over the
// XCDs (ct_qkv_col) so that head h's blocks run where the attention's head-h
// workgroups read them; row groups come last (grid z), and since a launch's
// K-slices x column blocks are a multiple of 8, every row group of a column
// block runs on the same XCD and finds its weight tiles in that L2.

// Sum over each 32-lane half of a wavefront, every lane getting the same
// bits: rotations by 8, 4, 2 and 1 within each 16-lane row (DPP row_ror, no
// LDS round trip), then the two rows swapped (ds_swizzle, XOR 16 within 32
// lanes).  At every step the two lanes being combined hold equal values in
// the step before, so each lane adds the same two numbers.
template <int N>
__device__ __forceinline__ float row_ror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}
__device__ __forceinline__ float half_wave_sum(float v) {
    v += row_ror<8>(v);
    v += row_ror<4>(v);
    v += row_ror<2>(v);
    v += row_ror<1>(v);
    return v + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}

// FOLD: the GEMM consumes LayerNorm(h) without a normalised copy of h.  With
// LN(h)_k = (h_k - mu) * rstd * w_k + b_k (backends/cpu/backend.c layernorm,
// eps 1e-5), a product row is
//     y_n = sum_k LN(h)_k W_nk + bias_n = rstd * (s_n - mu * c1_n) + c2_n,
//     s_n = sum_k (h_k w_k) W_nk,  c1_n = sum_k w_k W_nk,  c2_n = sum_k b_k W_nk + bias_n,
// so A is frag(h * w) (written by the residual projection that produced h),
// c1 / c2 are per-column constants (ctk_fold_cols), and each row's (mu, rstd)
// merges the producer's 32 per-block (mean, squared deviations) pairs in a
// fixed order (Chan et al.'s pairwise update with equal block sizes: mean of
// the means, then the blocks' sums plus 32 (mean_b - mean)^2 each).
template <int CB, int SPW, int RB, bool FOLD>
__global__ __launch_bounds__(64 * GV_WAVES) void gemv_kernel(CtGemv g) {
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int r = lane & 15, kg = lane >> 4;
    const int pos = blockIdx.y;
    const int c0 = (g.out == CT_GV_QKV ? ct_qkv_col(pos, CB) : pos) * 16 * CB;
    const int ks = blockIdx.x, q0 = blockIdx.z * RB, m0 = q0 * 16;   // first 16-row block, row
    const int nsteps = g.K >> 5;
    const int s0 = ks * (GV_WAVES * SPW);
    int nrb = min(RB, (g.M - m0 + 15) >> 4);
    if (g.m_active && m0 >= 64) {
        // rows past the first 64 may be unused spare rows this step
        const int ma = *g.m_active;
        if (m0 >= ma) return;
        nrb = min(nrb, (ma - m0 + 15) >> 4);
    }
    const bool resid = CB == 2 && RB == 1 && g.out == CT_GV_RESID;
    float2 lst[FOLD ? RB : 1];
    float h_in = 0.0f, b_in = 0.0f, fw = 0.0f;
    if (FOLD) {
        // this thread's block statistics first, so their wait leaves the row loads in flight
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            const int m = min(m0 + 16 * rb + (tid >> 5), g.M - 1);
            lst[rb] = reinterpret_cast<const float2 *>(g.lnstat)[(long)m * CT_LN_BLOCKS + (tid & 31)];
        }
    }
    // the folded LayerNorm's column constants of the columns this thread
    // finishes (its column is the same in every epilogue round: 512 threads
    // are a multiple of the tile width), loaded before the MFMAs
    constexpr int NFC = FOLD ? 8 : 1;
    float fc1[NFC], fc2[NFC];
    if (FOLD) {
        if (g.out == CT_GV_FRAG) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int col = c0 + (tid % (2 * CB)) * 8 + i;
                fc1[i] = g.fold_c1[col];
                fc2[i] = g.fold_c2[col];
            }
        } else {
            fc1[0] = g.fold_c1[c0 + tid % (16 * CB)];
            fc2[0] = g.fold_c2[c0 + tid % (16 * CB)];
        }
    }
    if (resid) {
        // the residual row element, bias and next LayerNorm gain this thread's epilogue needs
        const int m = m0 + (tid >> 5), col = c0 + (tid & 31);
        if (m < g.M) h_in = g.Y[(long)m * g.ldy + col];
        if (g.bias) b_in = bf2f(g.bias[col]);
        if (g.F) fw = bf2f(g.fold_w[col]);
    }
    // every load before the first MFMA: wavefront w takes K-steps w, w + 8, ...
    u16x8 ah[SPW][RB], al[SPW][RB], wv[SPW][CB];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int st = s0 + w + GV_WAVES * j;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            if (rb < nrb) {
                // frag layout: per 64 rows and K-step, four 16-row pieces of 1 KB hi + 1 KB lo
                const int q = q0 + rb;
                const uint16_t *p = g.A + ((((long)(q >> 2) * nsteps + st) * 4 + (q & 3)) << 10) + lane * 8;
                ah[j][rb] = *reinterpret_cast<const u16x8 *>(p);
                al[j][rb] = *reinterpret_cast<const u16x8 *>(p + 512);
            } else {
                ah[j][rb] = al[j][rb] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
            // non-temporal: a launch's weight tiles are dead after it, so they do not
            // displace tiles the read-ahead brought in for the next GEMMs
            wv[j][cb] = __builtin_nontemporal_load(reinterpret_cast<const u16x8 *>(
                g.wtile ? g.W + ((((long)(c0 >> 4) + cb) * nsteps + st) << 9) + lane * 8
                        : g.W + (long)(c0 + cb * 16 + r) * g.K + st * 32 + kg * 8));
    }
    __shared__ float2 lnrow[FOLD ? 16 * RB : 1];
    if (FOLD) {
        // half-wavefront h holds row h's 32 blocks (512 threads = 16 rows x 32 blocks)
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            const float mu = half_wave_sum(lst[rb].x) / (float)CT_LN_BLOCKS;
            const float d = lst[rb].x - mu;
            const float m2 = half_wave_sum(lst[rb].y + (float)(DEC_D / CT_LN_BLOCKS) * d * d);
            if ((tid & 31) == 0)
                lnrow[16 * rb + (tid >> 5)] = make_float2(mu, 1.0f / sqrtf(m2 / (float)DEC_D + 1e-5f));
        }
    }
    f32x4 acc[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++) acc[rb][cb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < SPW; j++)
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            if (rb >= nrb) break;
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                const bf16x8 b = as_bf16x8(wv[j][cb]);
                acc[rb][cb] = mfma16(as_bf16x8(ah[j][rb]), b, acc[rb][cb]);
                acc[rb][cb] = mfma16(as_bf16x8(al[j][rb]), b, acc[rb][cb]);
            }
        }
    __shared__ float part[GV_WAVES][16 * RB][16 * CB + 1];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int j = 0; j < 4; j++) part[w][rb * 16 + kg * 4 + j][cb * 16 + r] = acc[rb][cb][j];
    __syncthreads();

    // bias, or the folded LayerNorm's row correction and column constants
    // (fc1 / fc2 entry i)
    auto finish = [&](float s, int row, int col, int i) {
        if (FOLD) {
            const float2 mr = lnrow[row];
            return mr.y * (s - mr.x * fc1[i]) + fc2[i];
        }
        return g.bias ? s + bf2f(g.bias[col]) : s;
    };

    if (resid) {
        // thread: row m0 + tid / 32, column c0 + tid % 32; a half-wavefront holds
        // one row of this 32-column block
        const int row = tid >> 5, cc = tid & 31, m = m0 + row, col = c0 + cc;
        const bool ok = m < g.M && row < 16 * nrb;
        float s = part[0][row][cc];
#pragma unroll
        for (int ww = 1; ww < GV_WAVES; ww++) s += part[ww][row][cc];
        float x = 0.0f;
        if (ok) {
            x = h_in + (s + b_in);
            g.Y[(long)m * g.ldy + col] = x;
        }
        const float mean = half_wave_sum(x) / 32.0f;
        const float d = x - mean;
        const float m2 = half_wave_sum(d * d);
        if (ok && cc == 0)
            reinterpret_cast<float2 *>(g.lnstat)[(long)m * CT_LN_BLOCKS + (col >> 5)] = make_float2(mean, m2);
        if (g.F) {
            // frag(h * w) for the next GEMM's folded LayerNorm: lane cc of a
            // half-wavefront gathers columns cc..cc+7 of its row by lane
            // exchange, and every eighth lane stores the 16-byte pieces
            uint16_t hh, ll;
            // the product rounded on its own (no contraction into the split's subtraction)
            split_bf16(mul_rn(x, fw), hh, ll);
            const int v = (int)((uint32_t)hh | ((uint32_t)ll << 16));
            u16x8 hv, lv;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t u = (uint32_t)__shfl(v, (lane & ~7) + i);
                hv[i] = (uint16_t)(u & 0xFFFFu);
                lv[i] = (uint16_t)(u >> 16);
            }
            if (ok && (cc & 7) == 0) {
                const long o = ct_frag_off(m, col, DEC_D);
                *reinterpret_cast<u16x8 *>(g.F + o) = hv;
                *reinterpret_cast<u16x8 *>(g.F + o + 512) = lv;
            }
        }
        return;
    }
    if (g.out == CT_GV_FRAG) {
        // one thread per (row, 8 consecutive columns): a 16-byte piece per plane
        for (int e = tid; e < 16 * RB * 2 * CB; e += 64 * GV_WAVES) {
            const int row = e / (2 * CB), grp = e % (2 * CB), m = m0 + row;
            if (m >= g.M) continue;
            u16x8 hv, lv;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int cc = grp * 8 + i;
                float s = part[0][row][cc];
#pragma unroll
                for (int ww = 1; ww < GV_WAVES; ww++) s += part[ww][row][cc];
                s = finish(s, row, c0 + cc, i);
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
    for (int e = tid; e < 16 * RB * 16 * CB; e += 64 * GV_WAVES) {
        const int row = e / (16 * CB), cc = e % (16 * CB), m = m0 + row, col = c0 + cc;
        if (m >= g.M) continue;
        float s = part[0][row][cc];
#pragma unroll
        for (int ww = 1; ww < GV_WAVES; ww++) s += part[ww][row][cc];
        if (g.out == CT_GV_PARTIAL) {
            g.Y[((long)ks * g.M + m) * g.N + col] = s;
            continue;
        }
        s = finish(s, row, col, 0);
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
    const int cbk = (g.out == CT_GV_QKV ? ct_qkv_col(pos, CB) : pos) * CB;
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

// One thread per output column n of W[N][K] (row-major bf16): c1[n] =
// sum_k w_k W_nk, c2[n] = sum_k b_k W_nk + bias_n, in double, k in order.
__global__ __launch_bounds__(256) void fold_cols_kernel(const uint16_t *W, const uint16_t *w,
                                                        const uint16_t *b, const uint16_t *bias, int N,
                                                        int K, float *c1, float *c2) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    double s1 = 0.0, s2 = 0.0;
    const uint16_t *row = W + (long)n * K;
    for (int k = 0; k < K; k++) {
        const double x = (double)bf2f(row[k]);
        s1 += (double)bf2f(w[k]) * x;
        s2 += (double)bf2f(b[k]) * x;
    }
    if (bias) s2 += (double)bf2f(bias[n]);
    c1[n] = (float)s1;
    c2[n] = (float)s2;
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

extern "C" void ctk_fold_cols(const uint16_t *W, const uint16_t *w, const uint16_t *b, const uint16_t *bias,
                              int N, int K, float *c1, float *c2, hipStream_t s) {
    if (N <= 0 || K <= 0 || !W || !w || !b || !c1 || !c2) {
        fprintf(stderr, "ctk_fold_cols: needs W, w, b, c1, c2 and N, K > 0\n");
        exit(1);
    }
    hipLaunchKernelGGL(fold_cols_kernel, dim3((N + 255) / 256), dim3(256), 0, s, W, w, b, bias, N, K, c1, c2);
}

extern "C" int ctk_gemv_sizeof(void) { return (int)sizeof(CtGemv); }
extern "C" int ctk_warmset_sizeof(void) { return (int)sizeof(CtWarmSet); }

extern "C" int ctk_gemv_ksplit(int N, int K) {
    if (N <= DEC_D && K == DEC_D) return 2;       // 512-column slices, two K-steps per wave
    if (N <= DEC_D && K == DEC_FF) return 8;      // 512-column slices
    return 1;
}

// Tiling: 16-column blocks (cb) and 16-row blocks (rb) per workgroup.  A
// workgroup pulls 16*rb*K*4 bytes of activations and 16*cb*K*2 of weights
// through its CU's L2 port (≈ 64 B/clk), so the all-rows, 16-column tile
// moved 8x more activation than weight bytes.  Measured over M = 16..80,
// weights streamed from HBM and resident in L2: one row block per workgroup
// and 32 columns take 15-25% off the 64-row launches, 64 columns for the
// long-K projection and (above 32 rows, weights in L2 as the decode step's
// read-ahead leaves them) for the wide ones; 16 columns stay best for the
// wide projections at M <= 16, and the LM head (32 MB of weights, 256
// workgroups) keeps all rows and 64 columns.
// The residual projection always takes 32 columns and one row block (its
// epilogue holds a row's 32-column block in a half-wavefront; K = DEC_D).
static void gv_tile(int N, int K, int M, int out, int *cb, int *rb) {
    if (out == CT_GV_RESID) { *cb = 2; *rb = 1; return; }
    if (N >= 8192 && N % 64 == 0) { *cb = 4; *rb = 4; return; }
    *rb = 1;
    if (K >= 4096) *cb = N % 64 == 0 && M > 16 ? 4 : N % 32 == 0 ? 2 : 1;
    else if (N > DEC_D && N % 64 == 0 && M > 32) *cb = 4;
    else *cb = N % 32 == 0 && (M > 16 || N <= DEC_D) ? 2 : 1;
}

extern "C" long ctk_gemv_read_floor_blocks(const CtGemv *g) {
    const int ksplit = g->ksplit < 1 ? 1 : g->ksplit;
    int cb, rb;
    gv_tile(g->N, g->K, g->M, g->out, &cb, &rb);
    return (long)ksplit * (g->N / (16 * cb)) * ((g->M + 16 * rb - 1) / (16 * rb));
}

extern "C" void ctk_gemv_read_floor(const CtGemv *g, float *sink, hipStream_t s) {
    if (g->M <= 0) return;
    const int ksplit = g->ksplit < 1 ? 1 : g->ksplit;
    int cb, rb;
    gv_tile(g->N, g->K, g->M, g->out, &cb, &rb);
    if (!g->wtile || g->K % (256 * ksplit) != 0 || g->N % (16 * cb) != 0 || ((uintptr_t)g->W & 15))
        gv_fatal("read floor needs tiled, 16-byte aligned weights of a supported shape", g);
    const dim3 grid(ksplit, g->N / (16 * cb), (g->M + 16 * rb - 1) / (16 * rb));
    if (cb == 1) hipLaunchKernelGGL(read_floor_kernel<1>, grid, dim3(64 * GV_WAVES), 0, s, *g, ksplit, sink);
    else if (cb == 2) hipLaunchKernelGGL(read_floor_kernel<2>, grid, dim3(64 * GV_WAVES), 0, s, *g, ksplit, sink);
    else hipLaunchKernelGGL(read_floor_kernel<4>, grid, dim3(64 * GV_WAVES), 0, s, *g, ksplit, sink);
}


extern "C" void ctk_gemv_warm(const CtGemv *g, CtWarm *w) {
    const int ksplit = g->ksplit < 1 ? 1 : g->ksplit;
    int cb, rb;
    gv_tile(g->N, g->K, g->M, g->out, &cb, &rb);
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
    int cb, rb;
    gv_tile(g->N, g->K, g->M, g->out, &cb, &rb);
    const bool fold = g->fold_c1 != NULL;
    if (g->out == CT_GV_RESID &&
        (g->N != DEC_D || g->K != DEC_D || ksplit != 1 || !g->lnstat || ((uintptr_t)g->lnstat & 7) ||
         (g->F && (!g->fold_w || ((uintptr_t)g->F & 15)))))
        gv_fatal("residual output needs N = K = DEC_D, no K split, an 8-byte aligned lnstat, and with F "
                 "a 16-byte aligned F and its LayerNorm gain fold_w", g);
    if (fold && (g->K != DEC_D || !g->fold_c2 || !g->lnstat || ((uintptr_t)g->lnstat & 7) ||
                 g->out == CT_GV_PARTIAL || g->out == CT_GV_RESID))
        gv_fatal("a folded LayerNorm needs K = DEC_D, c1, c2 and lnstat, and a dense, frag or QKV output", g);
    const dim3 grid(ksplit, g->N / (16 * cb), (g->M + 16 * rb - 1) / (16 * rb));
    const dim3 block(64 * GV_WAVES);
#define GV_CASE(CB, SPW, RB)                                                                \
    if (cb == CB && spw == SPW && rb == RB && !fold) {                                      \
        hipLaunchKernelGGL((gemv_kernel<CB, SPW, RB, false>), grid, block, 0, s, *g);       \
        return;                                                                             \
    }
#define GV_FOLD(CB, RB)                                                                     \
    if (cb == CB && spw == 4 && rb == RB && fold) {                                         \
        hipLaunchKernelGGL((gemv_kernel<CB, 4, RB, true>), grid, block, 0, s, *g);          \
        return;                                                                             \
    }
    GV_CASE(1, 1, 1) GV_CASE(1, 2, 1) GV_CASE(1, 4, 1) GV_CASE(2, 1, 1) GV_CASE(2, 2, 1) GV_CASE(2, 4, 1)
    GV_CASE(4, 1, 1) GV_CASE(4, 2, 1) GV_CASE(4, 4, 1) GV_CASE(4, 1, 4) GV_CASE(4, 2, 4) GV_CASE(4, 4, 4)
    GV_FOLD(1, 1) GV_FOLD(2, 1) GV_FOLD(4, 1)
#undef GV_CASE
#undef GV_FOLD
    gv_fatal("no kernel for this K slice", g);
}
