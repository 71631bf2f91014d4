// k_gemm.hip — Y = epi(A W^T + b) on gfx950 bf16 MFMA.
//
// A is fp32 (activations), W is bf16 (the model's weights, exact).  Each A
// element is split into hi + lo bf16 terms and both are multiplied by the
// weight on v_mfma_f32_16x16x32_bf16 with fp32 accumulation, so the product
// carries ~16 significant activation bits (error <= 2^-17 relative) instead of
// bf16's 8.  Weights are read exactly once per output tile.
//
// Batch invariance: every tile shape runs the same per-element sequence
// (K-steps of 32 in order, hi then lo), so a row's result never depends on
// M, on the tile shape chosen for M, or on the other rows.
//
// Reference semantics: backends/cpu/backend.c:124-182 (linear, silu, relu,
// fmadd), 300-311 (GLU), 398-408 / 466-476 (KV-cache row scatter).
#include "ct_dev.h"
#include "ct_launch.h"
#include <stdio.h>
#include <stdlib.h>

namespace {

template <int RB, bool VEC>
__device__ __forceinline__ void load_a(const CtGemm &g, int m0, int kk, int r, float (&a)[RB][8]) {
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int m = m0 + rb * 16 + r;
        if (VEC) {
            if (m < g.M && kk < g.K) {
                const float4 *p = reinterpret_cast<const float4 *>(g.A + (long)m * g.lda + kk);
                const float4 x0 = p[0], x1 = p[1];
                a[rb][0] = x0.x; a[rb][1] = x0.y; a[rb][2] = x0.z; a[rb][3] = x0.w;
                a[rb][4] = x1.x; a[rb][5] = x1.y; a[rb][6] = x1.z; a[rb][7] = x1.w;
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) a[rb][j] = 0.0f;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++)
                a[rb][j] = (m < g.M && kk + j < g.K) ? g.A[(long)m * g.lda + kk + j] : 0.0f;
        }
    }
}

template <bool VEC>
__device__ __forceinline__ u16x8 load_w(const CtGemm &g, int n, int kk) {
    u16x8 w;
    if (VEC) {
        if (n < g.N && kk < g.K) w = *reinterpret_cast<const u16x8 *>(g.W + (long)n * g.K + kk);
        else w = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) w[j] = (n < g.N && kk + j < g.K) ? g.W[(long)n * g.K + kk + j] : 0;
    }
    return w;
}

// Writes one finished output element (bias already added) through the
// configured epilogue: segmented (dense / head-major KV scatter), row scatter
// (KV-cache append), or dense with SiLU / ReLU / fused residual.
__device__ __forceinline__ void store_out(const CtGemm &g, int m, int col, float s) {
    if (g.nseg > 0) {
        const int si = col / g.seg_w, c = col - si * g.seg_w;
        const CtSeg &sg = g.seg[si];
        if (sg.mode == CT_OUT_DENSE) {
            reinterpret_cast<float *>(sg.base)[(long)m * sg.ld + c] = s;
        } else {
            const long ro = sg.rowoff[m];
            if (ro < 0) return;
            const long off = ro + (long)(c >> 7) * sg.hstride + (c & 127);
            if (sg.mode == CT_OUT_HEADS_BF16) reinterpret_cast<uint16_t *>(sg.base)[off] = f2bf(s);
            else reinterpret_cast<float *>(sg.base)[off] = s;
        }
        return;
    }
    long yrow = m;
    if (g.row_len) {
        const int len = g.row_len[(long)m * g.row_len_step];
        if (len <= 0) return;          // no slot to write
        yrow = (long)m * g.row_stride + len - 1;
    }
    float *y = g.Y + yrow * g.ldy + col;
    if (g.epi == CT_EPI_SILU) *y = s / (1.0f + expf(-s));
    else if (g.epi == CT_EPI_RELU) *y = s > 0.0f ? s : 0.0f;
    else if (g.epi == CT_EPI_FMADD) *y += g.scale * s;
    else *y = s;
}

// ---------------------------------------------------------------------------
// Decoder-class GEMM (weights with K = 1024, or K = 4096 -> 1024): few rows
// (one per decode slot), weight-stream bound.  A workgroup owns 16*CB output
// columns and up to 64 rows; its DSPLIT wavefronts take contiguous K ranges,
// issue all of their loads early, and the DSPLIT partial tiles are summed in
// LDS in wave order.  The split depends only on K, never on M, so a row's
// result is the same for any number of rows.
// ---------------------------------------------------------------------------
constexpr int DSPLIT = 8;

template <int CB>
__global__ __launch_bounds__(64 * DSPLIT) void gemm_dec_kernel(CtGemm g) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15, kg = lane >> 4;
    const int c0 = blockIdx.x * 16 * CB;
    const int m0 = blockIdx.y * 64;
    const int nrb = min(4, (g.M - m0 + 15) / 16);
    const int kper = g.K / DSPLIT;
    const int kbeg = w * kper;
    f32x4 acc[4][CB];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++) acc[rb][cb] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const float *arow[4];
#pragma unroll
    for (int rb = 0; rb < 4; rb++) {
        const int m = m0 + rb * 16 + r;
        arow[rb] = (m < g.M) ? g.A + (long)m * g.lda : nullptr;
    }
    const uint16_t *wrow[CB];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        const int n = c0 + cb * 16 + r;
        wrow[cb] = (n < g.N) ? g.W + (long)n * g.K : nullptr;
    }
    for (int k0 = kbeg; k0 < kbeg + kper; k0 += 64) {
        // two K-steps of loads in flight
        float4 a[2][4][2];
        u16x8 wv[2][CB];
#pragma unroll
        for (int st = 0; st < 2; st++) {
            const int kk = k0 + st * 32 + kg * 8;
            const bool ok = kk < kbeg + kper;
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                if (ok && rb < nrb && arow[rb]) {
                    const float4 *p = reinterpret_cast<const float4 *>(arow[rb] + kk);
                    a[st][rb][0] = p[0]; a[st][rb][1] = p[1];
                } else {
                    a[st][rb][0] = a[st][rb][1] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
#pragma unroll
            for (int cb = 0; cb < CB; cb++)
                wv[st][cb] = (ok && wrow[cb]) ? *reinterpret_cast<const u16x8 *>(wrow[cb] + kk)
                                              : (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int st = 0; st < 2; st++) {
            if (k0 + st * 32 >= kbeg + kper) break;
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                if (rb >= nrb) break;
                const float x[8] = {a[st][rb][0].x, a[st][rb][0].y, a[st][rb][0].z, a[st][rb][0].w,
                                    a[st][rb][1].x, a[st][rb][1].y, a[st][rb][1].z, a[st][rb][1].w};
                u16x8 hi, lo;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    uint16_t h, l;
                    split_bf16(x[j], h, l);
                    hi[j] = h; lo[j] = l;
                }
                const bf16x8 ah = as_bf16x8(hi), al = as_bf16x8(lo);
#pragma unroll
                for (int cb = 0; cb < CB; cb++) {
                    const bf16x8 bw = as_bf16x8(wv[st][cb]);
                    acc[rb][cb] = mfma16(ah, bw, acc[rb][cb]);
                    acc[rb][cb] = mfma16(al, bw, acc[rb][cb]);
                }
            }
        }
    }
    __shared__ float part[DSPLIT][64][16 * CB + 1];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int j = 0; j < 4; j++) part[w][rb * 16 + kg * 4 + j][cb * 16 + r] = acc[rb][cb][j];
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 16 * CB; e += 64 * DSPLIT) {
        const int row = e / (16 * CB), cc = e % (16 * CB);
        const int m = m0 + row, col = c0 + cc;
        if (m >= g.M || col >= g.N) continue;
        if (g.row_mask && !g.row_mask[m]) continue;
        float s = part[0][row][cc];
#pragma unroll
        for (int ww = 1; ww < DSPLIT; ww++) s += part[ww][row][cc];
        if (g.bias) s += bf2f(g.bias[col]);
        store_out(g, m, col, s);
    }
}

// One wavefront computes a (16*RB) x (16*CB) tile.  In GLU mode the first CB/2
// column blocks are the "a" half and the last CB/2 the gate half (+glu_half).
template <int RB, int CB, bool VEC, bool GLU, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void gemm_kernel(CtGemm g, int n_mt, int n_tiles) {
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x * WAVES + (threadIdx.x >> 6);
    if (tile >= n_tiles) return;
    const int tm = tile % n_mt, tn = tile / n_mt;
    const int r = lane & 15, kg = lane >> 4;
    const int m0 = tm * 16 * RB;
    constexpr int CO = GLU ? CB / 2 : CB;          // output column blocks
    const int c0 = tn * 16 * CO;

    int ncol[CB];
#pragma unroll
    for (int cb = 0; cb < CB; cb++)
        ncol[cb] = GLU ? (cb < CO ? c0 + cb * 16 + r : g.glu_half + c0 + (cb - CO) * 16 + r)
                       : c0 + cb * 16 + r;
    const int nlim = GLU ? 2 * g.glu_half : g.N;

    f32x4 acc[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++) acc[rb][cb] = (f32x4){0.f, 0.f, 0.f, 0.f};

    float a_cur[RB][8];
    u16x8 w_cur[CB];
    load_a<RB, VEC>(g, m0, kg * 8, r, a_cur);
#pragma unroll
    for (int cb = 0; cb < CB; cb++) w_cur[cb] = (ncol[cb] < nlim) ? load_w<VEC>(g, ncol[cb], kg * 8) : (u16x8){0,0,0,0,0,0,0,0};

    for (int k0 = 0; k0 < g.K; k0 += 32) {
        float a_nxt[RB][8];
        u16x8 w_nxt[CB];
        const bool more = k0 + 32 < g.K;
        if (more) {
            load_a<RB, VEC>(g, m0, k0 + 32 + kg * 8, r, a_nxt);
#pragma unroll
            for (int cb = 0; cb < CB; cb++)
                w_nxt[cb] = (ncol[cb] < nlim) ? load_w<VEC>(g, ncol[cb], k0 + 32 + kg * 8) : (u16x8){0,0,0,0,0,0,0,0};
        }
        bf16x8 bw[CB];
#pragma unroll
        for (int cb = 0; cb < CB; cb++) bw[cb] = as_bf16x8(w_cur[cb]);
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            u16x8 hi, lo;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint16_t h, l;
                split_bf16(a_cur[rb][j], h, l);
                hi[j] = h; lo[j] = l;
            }
            const bf16x8 ah = as_bf16x8(hi), al = as_bf16x8(lo);
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                acc[rb][cb] = mfma16(ah, bw[cb], acc[rb][cb]);
                acc[rb][cb] = mfma16(al, bw[cb], acc[rb][cb]);
            }
        }
        if (more) {
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
#pragma unroll
                for (int j = 0; j < 8; j++) a_cur[rb][j] = a_nxt[rb][j];
#pragma unroll
            for (int cb = 0; cb < CB; cb++) w_cur[cb] = w_nxt[cb];
        }
    }

    // Epilogue.  Lane (r, kg) holds rows 4*kg + j, column r of each 16x16 block.
#pragma unroll
    for (int cb = 0; cb < CO; cb++) {
        const int col = c0 + cb * 16 + r;
        const int nout = GLU ? g.glu_half : g.N;
        if (col >= nout) continue;
        const float ba = g.bias ? bf2f(g.bias[ncol[cb]]) : 0.0f;
        const float bg = (GLU && g.bias) ? bf2f(g.bias[ncol[cb + (GLU ? CO : 0)]]) : 0.0f;
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int m = m0 + rb * 16 + kg * 4 + j;
                if (m >= g.M) continue;
                if (g.row_mask && !g.row_mask[m]) continue;
                const float s = acc[rb][cb][j] + ba;
                if (GLU) {
                    const float gt = acc[rb][cb + (GLU ? CO : 0)][j] + bg;
                    g.Y[(long)m * g.ldy + col] = s / (1.0f + expf(-gt));
                } else {
                    store_out(g, m, col, s);
                }
            }
    }
}

template <int RB, int CB, bool VEC, bool GLU, int WAVES>
void launch(const CtGemm &g, hipStream_t s) {
    const int n_mt = (g.M + 16 * RB - 1) / (16 * RB);
    const int cols = GLU ? g.glu_half : g.N;
    const int co = GLU ? CB / 2 : CB;
    const int n_nt = (cols + 16 * co - 1) / (16 * co);
    const int n_tiles = n_mt * n_nt;
    const int blocks = (n_tiles + WAVES - 1) / WAVES;
    hipLaunchKernelGGL((gemm_kernel<RB, CB, VEC, GLU, WAVES>), dim3(blocks), dim3(64 * WAVES), 0, s,
                       g, n_mt, n_tiles);
}

template <bool VEC, bool GLU>
void dispatch(const CtGemm &g, hipStream_t s) {
    if constexpr (GLU) {
        if (g.M <= 16) launch<1, 4, VEC, GLU, 1>(g, s);
        else if (g.M <= 64) launch<2, 4, VEC, GLU, 2>(g, s);
        else launch<4, 4, VEC, GLU, 4>(g, s);
    } else {
    // Small M (decode): one row-block group per wave, narrow columns, one
    // wave per workgroup so the weight stream spreads over many CUs.
    if (g.M <= 16) launch<1, 1, VEC, GLU, 1>(g, s);
    else if (g.M <= 32) launch<2, 1, VEC, GLU, 1>(g, s);
    else if (g.M <= 64) launch<4, 1, VEC, GLU, 1>(g, s);
    else launch<4, 4, VEC, GLU, 4>(g, s);
    }
}

}  // namespace

// Shapes of the decoder's weights: K = DEC_D, or the FFN down projection
// (K = DEC_FF, N = DEC_D).  They always take the split-K kernel.
static bool decoder_class(const CtGemm *g) {
    return g->epi != CT_EPI_GLU && (g->K == 1024 || (g->K == 4096 && g->N == 1024));
}

extern "C" void ctk_gemm(const CtGemm *g, hipStream_t s) {
    if (g->M <= 0 || g->N <= 0) return;
    if (g->epi == CT_EPI_GLU && g->N != 2 * g->glu_half) {
        fprintf(stderr, "ctk_gemm: GLU needs N == 2*glu_half\n");
        exit(1);
    }
    const bool vec = (g->K % 8 == 0) && (g->lda % 4 == 0) &&
                     (((uintptr_t)g->A & 15) == 0) && (((uintptr_t)g->W & 15) == 0);
    const bool glu = g->epi == CT_EPI_GLU;
    if (vec && decoder_class(g)) {
        const int cb = g->N >= 4096 ? 2 : 1;
        const dim3 grid((g->N + 16 * cb - 1) / (16 * cb), (g->M + 63) / 64);
        if (cb == 2) hipLaunchKernelGGL(gemm_dec_kernel<2>, grid, dim3(64 * DSPLIT), 0, s, *g);
        else hipLaunchKernelGGL(gemm_dec_kernel<1>, grid, dim3(64 * DSPLIT), 0, s, *g);
        return;
    }
    if (vec) { if (glu) dispatch<true, true>(*g, s); else dispatch<true, false>(*g, s); }
    else     { if (glu) dispatch<false, true>(*g, s); else dispatch<false, false>(*g, s); }
}
