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
        } else if (sg.mode == CT_OUT_SPLIT) {
            float v = s;
            if (g.epi == CT_EPI_SILU) v = s * sigmoid_hw(s);
            else if (g.epi == CT_EPI_RELU) v = s > 0.0f ? s : 0.0f;
            uint16_t h, l;
            split_bf16(v, h, l);
            reinterpret_cast<uint16_t *>(sg.base)[(long)m * sg.ld + c] = h;
            if (sg.base_lo) reinterpret_cast<uint16_t *>(sg.base_lo)[(long)m * sg.ld + c] = l;
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
    if (g.epi == CT_EPI_SILU) *y = s * sigmoid_hw(s);
    else if (g.epi == CT_EPI_RELU) *y = s > 0.0f ? s : 0.0f;
    else if (g.epi == CT_EPI_FMADD) *y += g.scale * s;
    else *y = s;
}

// Eight consecutive columns col..col+7 of row m (same segment, same head),
// with the bias already added: the 16-byte-store form of store_out.
__device__ __forceinline__ void act8(const CtGemm &g, float (&v)[8]) {
    if (g.epi == CT_EPI_SILU) {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = v[i] * sigmoid_hw(v[i]);
    } else if (g.epi == CT_EPI_RELU) {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = v[i] > 0.0f ? v[i] : 0.0f;
    }
}

// As store_out: the activation applies to plain rows and to SPLIT segments;
// DENSE and HEADS segments store the sum as it is.
__device__ __forceinline__ void store_out8(const CtGemm &g, int m, int col, float (&v)[8]) {
    float *yf = nullptr;
    uint16_t *yb = nullptr;
    if (g.nseg > 0) {
        const int si = col / g.seg_w, c = col - si * g.seg_w;
        const CtSeg &sg = g.seg[si];
        if (sg.mode == CT_OUT_SPLIT) {
            act8(g, v);
            u16x8 h8, l8;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint16_t h, l;
                split_bf16(v[i], h, l);
                h8[i] = h; l8[i] = l;
            }
            *reinterpret_cast<u16x8 *>(reinterpret_cast<uint16_t *>(sg.base) + (long)m * sg.ld + c) = h8;
            if (sg.base_lo)
                *reinterpret_cast<u16x8 *>(reinterpret_cast<uint16_t *>(sg.base_lo) + (long)m * sg.ld + c) = l8;
            return;
        }
        if (sg.mode == CT_OUT_DENSE) {
            yf = reinterpret_cast<float *>(sg.base) + (long)m * sg.ld + c;
        } else {
            const long ro = sg.rowoff[m];
            if (ro < 0) return;
            const long off = ro + (long)(c >> 7) * sg.hstride + (c & 127);
            if (sg.mode == CT_OUT_HEADS_BF16) yb = reinterpret_cast<uint16_t *>(sg.base) + off;
            else yf = reinterpret_cast<float *>(sg.base) + off;
        }
    } else {
        long yrow = m;
        if (g.row_len) {
            const int len = g.row_len[(long)m * g.row_len_step];
            if (len <= 0) return;
            yrow = (long)m * g.row_stride + len - 1;
        }
        yf = g.Y + yrow * g.ldy + col;
        act8(g, v);
    }
    if (yb) {
        u16x8 b8;
#pragma unroll
        for (int i = 0; i < 8; i++) b8[i] = f2bf(v[i]);
        *reinterpret_cast<u16x8 *>(yb) = b8;
        return;
    }
    float4 *y4 = reinterpret_cast<float4 *>(yf);
    if (g.nseg == 0 && g.epi == CT_EPI_FMADD) {
        float4 a = y4[0], b = y4[1];
        a.x += g.scale * v[0]; a.y += g.scale * v[1]; a.z += g.scale * v[2]; a.w += g.scale * v[3];
        b.x += g.scale * v[4]; b.y += g.scale * v[5]; b.z += g.scale * v[6]; b.w += g.scale * v[7];
        y4[0] = a; y4[1] = b;
        return;
    }
    y4[0] = make_float4(v[0], v[1], v[2], v[3]);
    y4[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ---------------------------------------------------------------------------
// Decoder-class GEMM (weights with K = 1024, or K = 4096 -> 1024): few rows
// (one per decode slot), weight-stream bound.  A workgroup owns 16*CB output
// columns and up to 64 rows; its DSPLIT wavefronts take contiguous K ranges,
// issue all of their loads early, and the DSPLIT partial tiles are summed in
// LDS in wave order.  The split depends only on K, never on M, so a row's
// result is the same for any number of rows.
// ---------------------------------------------------------------------------
#ifndef CT_DEC_SPLIT
#define CT_DEC_SPLIT 8
#endif
constexpr int DSPLIT = CT_DEC_SPLIT;

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

// ---------------------------------------------------------------------------
// Encoder-class GEMM (many rows): 128x128 output tile per 256-thread
// workgroup, K in steps of 32, double-buffered LDS.  Each stage loads the A
// tile (128x32 fp32, 64 contiguous bytes per thread), splits it to hi/lo
// bf16 into LDS, and stages the W tile (128x32 bf16); every wave then runs a
// 64x64 sub-tile as 4x4 MFMA 16x16x32 tiles, hi then lo, per K-step.  Tiles
// are numbered so that consecutive workgroups of one XCD (blockIdx % 8) share
// an A row block and read it from that XCD's L2.  Per element the sequence is
// the same as the small-M kernels (K-steps in order, hi then lo), so results
// do not depend on which of them ran.
// ---------------------------------------------------------------------------
constexpr int BT = 128, BK = 32, LDP = BK + 8;   // LDS row pitch 80 B (conflict-free b128 reads)

template <bool GLU>
__global__ __launch_bounds__(256) void gemm_big_kernel(CtGemm g, int n_mt, int n_nt, int vepi) {
    // one LDS block: [A hi x2][A lo x2][W x2] stage buffers; the GLU epilogue
    // reuses its first 32 KB
    __shared__ __attribute__((aligned(16))) uint16_t smem[6 * BT * LDP];
    uint16_t (*sAh)[BT * LDP] = reinterpret_cast<uint16_t (*)[BT * LDP]>(smem);
    uint16_t (*sAl)[BT * LDP] = reinterpret_cast<uint16_t (*)[BT * LDP]>(smem + 2 * BT * LDP);
    uint16_t (*sW)[BT * LDP] = reinterpret_cast<uint16_t (*)[BT * LDP]>(smem + 4 * BT * LDP);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, kg = lane >> 4;
    // XCD-aware tile order: workgroup b runs on XCD b % 8; give each XCD a
    // contiguous range of tiles, row-block major.
    const int nt = n_mt * n_nt;
    const int per = (nt + 7) / 8;
    const int xcd = blockIdx.x % 8, loc = blockIdx.x / 8;
    const int tile = xcd * per + loc;
    if (tile >= nt) return;
    const int tm = tile / n_nt, tn = tile % n_nt;
    const int m0 = tm * BT;
    const int c0 = tn * (GLU ? BT / 2 : BT);          // first output column
    // loader mapping: thread -> row tid/2, 16 consecutive k at (tid%2)*16
    const int lr = tid >> 1, lk = (tid & 1) * 16;
    const int am = m0 + lr;
    const float *arow = am < g.M ? g.A + (long)am * g.lda : nullptr;
    int wn;
    if (GLU) wn = lr < 64 ? c0 + lr : g.glu_half + c0 + (lr - 64);
    else wn = c0 + lr;
    const int nlim = GLU ? 2 * g.glu_half : g.N;
    const uint16_t *wrow = wn < nlim ? g.W + (long)wn * g.K : nullptr;

    float4 pa[4];
    u16x8 pw[2];
    auto gload = [&](int k0) {
        if (arow) {
            const float4 *p = reinterpret_cast<const float4 *>(arow + k0 + lk);
            pa[0] = p[0]; pa[1] = p[1]; pa[2] = p[2]; pa[3] = p[3];
        } else {
            pa[0] = pa[1] = pa[2] = pa[3] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (wrow) {
            const u16x8 *q = reinterpret_cast<const u16x8 *>(wrow + k0 + lk);
            pw[0] = q[0]; pw[1] = q[1];
        } else {
            pw[0] = pw[1] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
        }
    };
    auto lstore = [&](int buf) {
        const float x[16] = {pa[0].x, pa[0].y, pa[0].z, pa[0].w, pa[1].x, pa[1].y, pa[1].z, pa[1].w,
                             pa[2].x, pa[2].y, pa[2].z, pa[2].w, pa[3].x, pa[3].y, pa[3].z, pa[3].w};
        u16x8 h0, h1, l0, l1;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint16_t h, l;
            split_bf16(x[j], h, l); h0[j] = h; l0[j] = l;
            split_bf16(x[j + 8], h, l); h1[j] = h; l1[j] = l;
        }
        u16x8 *ah = reinterpret_cast<u16x8 *>(&sAh[buf][lr * LDP + lk]);
        u16x8 *al = reinterpret_cast<u16x8 *>(&sAl[buf][lr * LDP + lk]);
        u16x8 *ww = reinterpret_cast<u16x8 *>(&sW[buf][lr * LDP + lk]);
        ah[0] = h0; ah[1] = h1; al[0] = l0; al[1] = l1; ww[0] = pw[0]; ww[1] = pw[1];
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int wm = (wv >> 1) * 64, wnn = (wv & 1) * 64;   // wave sub-tile origin

    gload(0);
    lstore(0);
    __syncthreads();
    const int nk = g.K / BK;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        bf16x8 bfr[4];
#pragma unroll
        for (int cb = 0; cb < 4; cb++)
            bfr[cb] = as_bf16x8(*reinterpret_cast<const u16x8 *>(&sW[cur][(wnn + cb * 16 + r) * LDP + kg * 8]));
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            const int row = (wm + rb * 16 + r) * LDP + kg * 8;
            const bf16x8 ah = as_bf16x8(*reinterpret_cast<const u16x8 *>(&sAh[cur][row]));
            const bf16x8 al = as_bf16x8(*reinterpret_cast<const u16x8 *>(&sAl[cur][row]));
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                acc[rb][cb] = mfma16(ah, bfr[cb], acc[rb][cb]);
                acc[rb][cb] = mfma16(al, bfr[cb], acc[rb][cb]);
            }
        }
        if (kt + 1 < nk) {
            lstore(cur ^ 1);
            __syncthreads();
        }
    }

    // epilogue: wave sub-tile rows wm + rb*16 + 4*kg + j, columns wnn + cb*16 + r
    if (GLU) {
        // local columns [0,64) are the value half, [64,128) the gate half:
        // waves with wnn == 0 hold values, wnn == 64 gates -> pair via LDS.
        __syncthreads();
        float *sx = reinterpret_cast<float *>(smem);   // 128 x 64 floats = 32 KB of the 60 KB block
        if (wnn == 64) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int cb = 0; cb < 4; cb++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        sx[(wm + rb * 16 + kg * 4 + j) * 64 + cb * 16 + r] = acc[rb][cb][j];
        }
        __syncthreads();
        if (wnn == 0) {
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                const int col = c0 + cb * 16 + r;
                if (col >= g.glu_half) continue;
                const float ba = g.bias ? bf2f(g.bias[col]) : 0.0f;
                const float bg = g.bias ? bf2f(g.bias[g.glu_half + col]) : 0.0f;
#pragma unroll
                for (int rb = 0; rb < 4; rb++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int lrow = wm + rb * 16 + kg * 4 + j, m = m0 + lrow;
                        if (m >= g.M) continue;
                        const float a = acc[rb][cb][j] + ba;
                        const float gt = sx[lrow * 64 + cb * 16 + r] + bg;
                        g.Y[(long)m * g.ldy + col] = a * sigmoid_hw(gt);
                    }
            }
        }
        return;
    }
    // epilogue in two 64-row halves through LDS (32 KB each): each thread
    // finishes 8 consecutive columns of a row (16-byte stores when vepi)
    __syncthreads();
    float *sc = reinterpret_cast<float *>(smem);
#pragma unroll
    for (int half = 0; half < 2; half++) {
        if ((wm >> 6) == half) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int cb = 0; cb < 4; cb++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int row = rb * 16 + kg * 4 + j;
                        sc[row * BT + ((wnn + cb * 16 + r) ^ (((row >> 2) & 3) << 4))] = acc[rb][cb][j];
                    }
        }
        __syncthreads();
        for (int it = tid; it < 64 * (BT / 8); it += 256) {
            const int row = it / (BT / 8), g8 = it % (BT / 8);
            const int m = m0 + 64 * half + row, col = c0 + g8 * 8;
            if (m >= g.M || col >= g.N) continue;
            if (g.row_mask && !g.row_mask[m]) continue;
            const float4 *pv = reinterpret_cast<const float4 *>(sc + row * BT + ((g8 * 8) ^ (((row >> 2) & 3) << 4)));
            const float4 v0 = pv[0], v1 = pv[1];
            float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            if (vepi) {
                if (g.bias) {
                    const u16x8 b8 = *reinterpret_cast<const u16x8 *>(g.bias + col);
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] += bf2f(b8[i]);
                }
                store_out8(g, m, col, v);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (col + i < g.N) store_out(g, m, col + i, v[i] + (g.bias ? bf2f(g.bias[col + i]) : 0.0f));
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Pre-split encoder GEMM: A arrives as two bf16 planes (hi, lo) written by the
// producing kernel, so all three operands stream straight from HBM/L2 into
// LDS with gfx950 global_load_lds_dwordx4 (no register staging) through a
// ring of SST stages, one barrier per stage.  Tile 128 (rows) x 256 (weight
// columns): A is the doubled operand, so the tile is wide in N.  BK = 32 (one
// MFMA K-step) per stage; 8 waves, each a 64x64 sub-tile (4x4 MFMA 16x16x32,
// hi then lo).  LDS rows are 64 B; 16-B chunk c of row R sits at chunk
// c ^ ((R >> 2) & 3), which makes the 16-lane fragment reads conflict-free.
// Tiles run in groups of SGM row blocks (all column tiles of a group before
// the next), each XCD taking a contiguous range, so a group's A rows and the
// W columns in use stay in that XCD's L2.
// Per element: K-steps in order, hi then lo (as every other GEMM kernel).
// Single-pass form (LO = false, no lo plane): A is bf16 (hi) alone, one MFMA
// per K-step and fragment, two thirds of the DMA bytes, and a deeper ring.
// ---------------------------------------------------------------------------
constexpr int SBM = 128, SBN = 256, SBK = 32, SST = 4, SGM = 4;
// rows from which the 256-row tile kernel takes pre-split GEMMs
#ifndef CT_SPLIT256_MIN_M
#define CT_SPLIT256_MIN_M 1024
#endif
constexpr int S_A = SBM * SBK, S_W = SBN * SBK;       // elements per operand tile
template <bool LO> struct SplitCfg {
    static constexpr int STAGE = (LO ? 2 : 1) * S_A + S_W;   // Ahi, (Alo,) W
    static constexpr int PER_WAVE = STAGE / 512 / 8;          // 1-KB DMA instructions (4, 3)
    static constexpr int STAGES = LO ? SST : 5;               // 128 KB, 120 KB of LDS
};

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// One 16-byte-per-lane DMA from global memory into the wave's LDS range,
// issued from inline assembly.  The compiler counts the builtin form's
// (__builtin_amdgcn_global_load_lds) LDS write as an LDS event of unknown
// order (it is not: the hardware's lgkmcnt does not wait for the DMA's data),
// so with the builtin in a loop every first use of an LDS fragment waits for
// all LDS reads in flight.  Issued here, the DMA is invisible to that bookkeeping and the
// fragment reads get in-order waits; the DMA itself is waited for explicitly
// (vmcnt) before the barrier that publishes a stage.  M0 takes the wave's LDS
// destination; one wait state separates its write from the load.  M0 is a
// register the compiler reserves (an asm clobber of it is ignored): the kernels
// that use this helper have no other instruction that reads M0 (no LDS-DMA
// builtin, no register-indexed moves), so nothing relies on its old value.
__device__ __forceinline__ void lds_dma16_asm(const void *g, uint16_t *lds_wave_base) {
    const unsigned l = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_ptr_t)lds_wave_base);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(l) : "memory");
}

// 16-byte chunk c of a 64-byte LDS row R sits at chunk swz(R, c).  The 16 rows
// a fragment read touches then cover every bank once whether the LDS serves
// 16 lanes over 64 banks or 8 lanes over 32 banks per cycle.
__device__ __forceinline__ int swz(int R, int c) { return c ^ (((R >> 1) ^ (R >> 2)) & 3); }

// The vector epilogue of a tile staged in LDS as fp32 rows of SBN floats
// (16-column groups XOR-swizzled by row).  A thread finishes the 8 columns
// col..col+7 (one segment, one head, col < N; local group g8) of NI rows 16
// apart.  What is constant for the thread (bias, segment) is set up once per
// tile (Epi8), and every global load the rows need (row mask, cache row
// offset, the FMADD residual) is issued before the first store, so their
// latencies overlap instead of adding up row after row.  Per element the
// arithmetic is store_out8's.
struct Epi8 {
    float b[8];
    int mode;               // CtSeg mode, or -1 for plain rows (nseg == 0)
    void *base, *base_lo;
    long ld;
    const long *rowoff;
    long off;               // column offset in a row (HEADS: head block + column)
};

__device__ __forceinline__ Epi8 epi8_setup(const CtGemm &g, int col) {
    Epi8 e;
    if (g.bias) {
        const u16x8 b8 = *reinterpret_cast<const u16x8 *>(g.bias + col);
#pragma unroll
        for (int i = 0; i < 8; i++) e.b[i] = bf2f(b8[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) e.b[i] = 0.0f;
    }
    if (g.nseg > 0) {
        const int si = col / g.seg_w, c = col - si * g.seg_w;
        const CtSeg &sg = g.seg[si];
        e.mode = sg.mode; e.base = sg.base; e.base_lo = sg.base_lo; e.ld = sg.ld; e.rowoff = sg.rowoff;
        e.off = (sg.mode == CT_OUT_DENSE || sg.mode == CT_OUT_SPLIT) ? c : (long)(c >> 7) * sg.hstride + (c & 127);
    } else {
        e.mode = -1; e.base = g.Y; e.base_lo = nullptr; e.ld = g.ldy; e.rowoff = nullptr; e.off = col;
    }
    return e;
}

template <int NI>
__device__ __forceinline__ void epi8_rows_any(const CtGemm &g, const Epi8 &e, const float *sc, int lr0, int m0, int g8);

// Local rows lr0 + 16*i (i < NI) of the staged tile sc = output rows m0 + those.
template <int NI>
__device__ __forceinline__ void epi8_rows(const CtGemm &g, const Epi8 &e, const float *sc, int lr0, int m0, int g8) {
    if (!g.row_mask && (e.mode == CT_OUT_SPLIT || e.mode == CT_OUT_DENSE ||
                        (e.mode < 0 && g.epi != CT_EPI_FMADD))) {
        // rows that only store (bf16 planes, dense fp32 segments, plain rows
        // with their activation): every row's staged sums are read first,
        // then each row is finished and stored straight through, the store
        // predicated on the row being in range, so no branch stands between
        // one row's LDS reads and the next row's
        float4 a[NI], b[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int row = lr0 + 16 * i;
            const float4 *pv = reinterpret_cast<const float4 *>(sc + row * SBN + ((g8 * 8) ^ (((row >> 2) & 3) << 4)));
            a[i] = pv[0]; b[i] = pv[1];
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int m = m0 + lr0 + 16 * i;
            const long o = (long)m * e.ld + e.off;
            float v[8] = {a[i].x, a[i].y, a[i].z, a[i].w, b[i].x, b[i].y, b[i].z, b[i].w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] += e.b[j];
            if (e.mode == CT_OUT_SPLIT) {
                act8(g, v);
                u16x8 h8;
#pragma unroll
                for (int j = 0; j < 8; j++) h8[j] = f2bf(v[j]);
                if (m < g.M) *reinterpret_cast<u16x8 *>(reinterpret_cast<uint16_t *>(e.base) + o) = h8;
                if (e.base_lo) {
                    // lo = the rounding remainder, as split_bf16
                    u16x8 l8;
#pragma unroll
                    for (int j = 0; j < 8; j++) l8[j] = f2bf(v[j] - bf2f(h8[j]));
                    if (m < g.M) *reinterpret_cast<u16x8 *>(reinterpret_cast<uint16_t *>(e.base_lo) + o) = l8;
                }
            } else {
                if (e.mode < 0) act8(g, v);      // plain rows take the activation; DENSE segments do not
                float4 *y4 = reinterpret_cast<float4 *>(reinterpret_cast<float *>(e.base) + o);
                if (m < g.M) {
                    y4[0] = make_float4(v[0], v[1], v[2], v[3]);
                    y4[1] = make_float4(v[4], v[5], v[6], v[7]);
                }
            }
        }
    } else if (!g.row_mask && e.mode < 0 && g.epi == CT_EPI_FMADD) {
        // y += scale * (sum + bias) on plain fp32 rows: every row's residual
        // load goes out first, then the rows straight through
        float4 y0[NI], y1[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int m = m0 + lr0 + 16 * i;
            if (m < g.M) {
                const float4 *y4 = reinterpret_cast<const float4 *>(reinterpret_cast<float *>(e.base) + (long)m * e.ld + e.off);
                y0[i] = y4[0]; y1[i] = y4[1];
            } else {
                y0[i] = y1[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int row = lr0 + 16 * i, m = m0 + row;
            const float4 *pv = reinterpret_cast<const float4 *>(sc + row * SBN + ((g8 * 8) ^ (((row >> 2) & 3) << 4)));
            const float4 a = pv[0], b = pv[1];
            float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] += e.b[j];
            float4 p = y0[i], q = y1[i];
            p.x += g.scale * v[0]; p.y += g.scale * v[1]; p.z += g.scale * v[2]; p.w += g.scale * v[3];
            q.x += g.scale * v[4]; q.y += g.scale * v[5]; q.z += g.scale * v[6]; q.w += g.scale * v[7];
            float4 *y4 = reinterpret_cast<float4 *>(reinterpret_cast<float *>(e.base) + (long)m * e.ld + e.off);
            if (m < g.M) { y4[0] = p; y4[1] = q; }
        }
    } else {
        epi8_rows_any<NI>(g, e, sc, lr0, m0, g8);
    }
}

// The general form of epi8_rows (row masks, cache rows by head), row by row.
template <int NI>
__device__ __forceinline__ void epi8_rows_any(const CtGemm &g, const Epi8 &e, const float *sc, int lr0, int m0, int g8) {
    const bool fmadd = e.mode < 0 && g.epi == CT_EPI_FMADD;
    const bool heads = e.mode == CT_OUT_HEADS_F32 || e.mode == CT_OUT_HEADS_BF16;
    bool ok[NI];
    long ro[NI];
    float4 y0[NI], y1[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int m = m0 + lr0 + 16 * i;
        ok[i] = m < g.M && (!g.row_mask || g.row_mask[m] != 0);
        ro[i] = heads && ok[i] ? e.rowoff[m] : 0;
        if (fmadd && ok[i]) {
            const float4 *y4 = reinterpret_cast<const float4 *>(reinterpret_cast<float *>(e.base) + (long)m * e.ld + e.off);
            y0[i] = y4[0]; y1[i] = y4[1];
        } else {
            y0[i] = y1[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int row = lr0 + 16 * i, m = m0 + row;
        if (!ok[i] || ro[i] < 0) continue;
        const float4 *pv = reinterpret_cast<const float4 *>(sc + row * SBN + ((g8 * 8) ^ (((row >> 2) & 3) << 4)));
        const float4 v0 = pv[0], v1 = pv[1];
        float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] += e.b[j];
        if (heads) {
            const long o = ro[i] + e.off;
            if (e.mode == CT_OUT_HEADS_BF16) {
                u16x8 b8;
#pragma unroll
                for (int j = 0; j < 8; j++) b8[j] = f2bf(v[j]);
                *reinterpret_cast<u16x8 *>(reinterpret_cast<uint16_t *>(e.base) + o) = b8;
            } else {
                float4 *y4 = reinterpret_cast<float4 *>(reinterpret_cast<float *>(e.base) + o);
                y4[0] = make_float4(v[0], v[1], v[2], v[3]);
                y4[1] = make_float4(v[4], v[5], v[6], v[7]);
            }
            continue;
        }
        if (e.mode == CT_OUT_SPLIT) {
            act8(g, v);
            u16x8 h8;
#pragma unroll
            for (int j = 0; j < 8; j++) h8[j] = f2bf(v[j]);
            *reinterpret_cast<u16x8 *>(reinterpret_cast<uint16_t *>(e.base) + (long)m * e.ld + e.off) = h8;
            if (e.base_lo) {
                // lo = the rounding remainder, as split_bf16
                u16x8 l8;
#pragma unroll
                for (int j = 0; j < 8; j++) l8[j] = f2bf(v[j] - bf2f(h8[j]));
                *reinterpret_cast<u16x8 *>(reinterpret_cast<uint16_t *>(e.base_lo) + (long)m * e.ld + e.off) = l8;
            }
            continue;
        }
        if (e.mode < 0) act8(g, v);      // plain rows take the activation; DENSE segments do not
        float4 *y4 = reinterpret_cast<float4 *>(reinterpret_cast<float *>(e.base) + (long)m * e.ld + e.off);
        if (fmadd) {
            float4 a = y0[i], b = y1[i];
            a.x += g.scale * v[0]; a.y += g.scale * v[1]; a.z += g.scale * v[2]; a.w += g.scale * v[3];
            b.x += g.scale * v[4]; b.y += g.scale * v[5]; b.z += g.scale * v[6]; b.w += g.scale * v[7];
            y4[0] = a; y4[1] = b;
        } else {
            y4[0] = make_float4(v[0], v[1], v[2], v[3]);
            y4[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
}

template <bool GLU, bool LO>
__global__ __launch_bounds__(512) void gemm_split_kernel(CtGemm g, int n_mt, int n_nt, int vepi) {
    constexpr int STAGE_ELEMS = SplitCfg<LO>::STAGE, S_PER_WAVE = SplitCfg<LO>::PER_WAVE;
    constexpr int NST = SplitCfg<LO>::STAGES;
    // the ring, and the epilogue's 128 x 256 fp32 tile after it
    constexpr int SMEM = NST * STAGE_ELEMS > SBM * SBN * 2 ? NST * STAGE_ELEMS : SBM * SBN * 2;
    __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, kg = lane >> 4;
    const int nt = n_mt * n_nt;
    const int per = (nt + 7) / 8;
    const int t = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (t >= nt) return;
    // grouped order: SGM row blocks x all column tiles per group, row fastest
    const int gsize = SGM * n_nt;
    const int grp = t / gsize, rem = t % gsize;
    const int gm = min(SGM, n_mt - grp * SGM);
    const int tn = rem / gm, tm = grp * SGM + rem % gm;
    const int m0 = tm * SBM;
    const int c0 = tn * (GLU ? SBN / 2 : SBN);
    const int nlim = GLU ? 2 * g.glu_half : g.N;

    // DMA plan: instruction i covers 16 rows x 64 B of one operand tile:
    // i < 8 A-hi, then (LO) i < 16 A-lo, then W.  Lane L lands at row
    // 16*(i%8 or (i-NA)) + L/4, chunk slot L%4, fetching global chunk
    // swz(row, L%4).  Wave wv issues i = wv + 8*j.
    constexpr int NA = LO ? 16 : 8;                      // A instructions per stage
    const uint16_t *src[S_PER_WAVE];
    int dst[S_PER_WAVE];
#pragma unroll
    for (int j = 0; j < S_PER_WAVE; j++) {
        const int i = wv + 8 * j;
        const int Rl = lane >> 2, ch = lane & 3;
        if (i < NA) {
            const int R = (i & 7) * 16 + Rl;
            const int m = min(m0 + R, g.M - 1);            // rows >= M are never stored
            src[j] = (i < 8 ? g.Ahi : g.Alo) + (long)m * g.lda + swz(R, ch) * 8;
            dst[j] = (i < 8 ? 0 : S_A) + (i & 7) * 16 * SBK;
        } else {
            const int R = (i - NA) * 16 + Rl;
            int n = GLU ? (R < SBN / 2 ? c0 + R : g.glu_half + c0 + R - SBN / 2) : c0 + R;
            n = min(n, nlim - 1);
            src[j] = g.W + (long)n * g.K + swz(R, ch) * 8;
            dst[j] = (LO ? 2 : 1) * S_A + (i - NA) * 16 * SBK;
        }
    }
    // DMA instruction j of stage kt (inline assembly: the builtin makes the
    // compiler wait for all LDS traffic before every fragment read)
    auto issue1 = [&](int kt, int j) {
        lds_dma16_asm(src[j] + kt * SBK, smem + (kt % NST) * STAGE_ELEMS + dst[j]);
    };
    auto issue = [&](int kt) {
#pragma unroll
        for (int j = 0; j < S_PER_WAVE; j++) issue1(kt, j);
    };
    static_assert(S_PER_WAVE <= 4, "at most one refill DMA instruction per MFMA row group");

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int wm = (wv >> 2) * 64, wn = (wv & 3) * 64;
    const int nk = g.K / SBK;
#pragma unroll
    for (int p = 0; p < NST - 1; p++)
        if (p < nk) issue(p);
    for (int kt = 0; kt < nk; kt++) {
        // wait for this wave's part of stage kt; younger stages stay in flight
        const int younger = min(nk - 1 - kt, NST - 2);
        if (younger >= 3) __builtin_amdgcn_s_waitcnt(((3 * S_PER_WAVE) & 0xF) | (0x7 << 4) | (0xF << 8));
        else if (younger == 2) __builtin_amdgcn_s_waitcnt(((2 * S_PER_WAVE) & 0xF) | (0x7 << 4) | (0xF << 8));
        else if (younger == 1) __builtin_amdgcn_s_waitcnt((S_PER_WAVE & 0xF) | (0x7 << 4) | (0xF << 8));
        else __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));
        __builtin_amdgcn_s_barrier();            // stage kt landed for every wave, and every
        asm volatile("" ::: "memory");           // wave is done reading stage kt-1
        // the refill of the freed slot (stage kt + NST - 1) goes out one DMA
        // instruction per MFMA row group, after that group's fragment reads,
        // rather than all at once ahead of the first MFMA
        const bool refill = kt + NST - 1 < nk;
        const uint16_t *st = smem + (kt % NST) * STAGE_ELEMS;
        const uint16_t *sAh = st, *sAl = st + S_A, *sW = st + (LO ? 2 : 1) * S_A;
        bf16x8 bfr[4];
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            const int R = wn + cb * 16 + r;
            bfr[cb] = as_bf16x8(*reinterpret_cast<const u16x8 *>(sW + R * SBK + swz(R, kg) * 8));
        }
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            const int R = wm + rb * 16 + r;
            const int off = R * SBK + swz(R, kg) * 8;
            const bf16x8 ah = as_bf16x8(*reinterpret_cast<const u16x8 *>(sAh + off));
            bf16x8 al;
            if (LO) al = as_bf16x8(*reinterpret_cast<const u16x8 *>(sAl + off));
            if (refill && rb < S_PER_WAVE) issue1(kt + NST - 1, rb);
            __builtin_amdgcn_sched_barrier(0);
            if (LO) {
#pragma unroll
                for (int cb = 0; cb < 4; cb++) {
                    acc[rb][cb] = mfma16(ah, bfr[cb], acc[rb][cb]);
                    acc[rb][cb] = mfma16(al, bfr[cb], acc[rb][cb]);
                }
            } else {
#pragma unroll
                for (int cb = 0; cb < 4; cb++) acc[rb][cb] = mfma16(ah, bfr[cb], acc[rb][cb]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    if (GLU) {
        // local columns [0,128) are values (waves wn < 128), [128,256) gates
        float *sx = reinterpret_cast<float *>(smem);     // 128 x 128 floats = 64 KB
        if (wn >= 128) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int cb = 0; cb < 4; cb++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        sx[(wm + rb * 16 + kg * 4 + j) * 128 + (wn - 128) + cb * 16 + r] = acc[rb][cb][j];
        }
        __syncthreads();
        if (wn < 128) {
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                const int lc = wn + cb * 16 + r, col = c0 + lc;
                if (col >= g.glu_half) continue;
                const float ba = g.bias ? bf2f(g.bias[col]) : 0.0f;
                const float bg = g.bias ? bf2f(g.bias[g.glu_half + col]) : 0.0f;
#pragma unroll
                for (int rb = 0; rb < 4; rb++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int lrow = wm + rb * 16 + kg * 4 + j, m = m0 + lrow;
                        if (m >= g.M) continue;
                        const float a = acc[rb][cb][j] + ba;
                        const float gt = sx[lrow * 128 + lc] + bg;
                        g.Y[(long)m * g.ldy + col] = a * sigmoid_hw(gt);
                    }
            }
        }
        return;
    }
    // Epilogue: the 128 x 256 fp32 tile goes through the (now idle) LDS ring,
    // then each thread finishes 8 consecutive columns of a row and writes them
    // as 16-byte pieces (when vepi allows), 32 threads per 1-KB row run.  Column
    // groups of 16 are XOR-swizzled by row so the fragment writes spread over
    // all banks.
    float *sc = reinterpret_cast<float *>(smem);
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int cb = 0; cb < 4; cb++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int row = wm + rb * 16 + kg * 4 + j;
                const int col = (wn + cb * 16 + r) ^ (((row >> 2) & 3) << 4);
                sc[row * SBN + col] = acc[rb][cb][j];
            }
    __syncthreads();
    if (vepi == 2) {
        // thread tid finishes columns 8*(tid%32).. of rows tid/32 + 16*i
        const int g8 = tid & 31, col = c0 + g8 * 8;
        if (col < g.N) {
            const Epi8 e = epi8_setup(g, col);
            epi8_rows<SBM / 16>(g, e, sc, tid >> 5, m0, g8);
        }
        return;
    }
    for (int it = tid; it < SBM * (SBN / 8); it += 512) {
        const int row = it / (SBN / 8), g8 = it % (SBN / 8);
        const int m = m0 + row, col = c0 + g8 * 8;
        if (m >= g.M || col >= g.N) continue;
        if (g.row_mask && !g.row_mask[m]) continue;
        const float4 *pv = reinterpret_cast<const float4 *>(sc + row * SBN + ((g8 * 8) ^ (((row >> 2) & 3) << 4)));
        const float4 v0 = pv[0], v1 = pv[1];
        float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        if (g.bias) {
            if (vepi) {
                const u16x8 b8 = *reinterpret_cast<const u16x8 *>(g.bias + col);
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] += bf2f(b8[i]);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] += col + i < g.N ? bf2f(g.bias[col + i]) : 0.0f;
            }
        }
        if (vepi) {
            store_out8(g, m, col, v);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (col + i < g.N) store_out(g, m, col + i, v[i]);
        }
    }
}

// ---------------------------------------------------------------------------
// The same pre-split GEMM with 256 x 256 tiles for many-row problems: 8 waves
// as 4 (rows) x 2 (columns), each a 64 x 128 sub-tile (4 x 8 MFMA 16x16x32,
// hi then lo), so a K-step reads 16 fragments from LDS for 64 MFMAs (the
// 128-row tile reads 12 for 32) and one barrier covers twice the work.
// 3-stage ring of 48 KB (A hi, A lo: 256 x 32 each; W: 256 x 32), 6 DMA
// instructions per wave per stage.  Per element the sequence is unchanged.
// ---------------------------------------------------------------------------
constexpr int TBM = 256;
constexpr int T_A = TBM * SBK;
template <bool LO> struct Split256Cfg {
    static constexpr int STAGE = (LO ? 2 : 1) * T_A + S_W;    // 48 KB, 32 KB
    static constexpr int PER_WAVE = STAGE / 512 / 8;          // 6, 4
    static constexpr int STAGES = LO ? 3 : 4;                 // 144 KB, 128 KB of LDS
};

// GLU: the tile's 256 weight rows are 128 value columns c0.. and their 128
// gate columns glu_half + c0..; waves with wn = 128 hold the gates and hand
// them to the value waves through LDS (as gemm_split_kernel<true, LO> does).
template <bool GLU>
__global__ __launch_bounds__(512) void gemm_split256_kernel(CtGemm g, int n_mt, int n_nt, int vepi) {
    constexpr bool LO = true;
    constexpr int T_STAGE = Split256Cfg<LO>::STAGE, T_PER_WAVE = Split256Cfg<LO>::PER_WAVE;
    constexpr int TST = Split256Cfg<LO>::STAGES;
    __shared__ __attribute__((aligned(16))) uint16_t smem[TST * T_STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, kg = lane >> 4;
    const int nt = n_mt * n_nt;
    const int per = (nt + 7) / 8;
    const int t = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (t >= nt) return;
    const int gsize = SGM * n_nt;
    const int grp = t / gsize, rem = t % gsize;
    const int gm = min(SGM, n_mt - grp * SGM);
    const int tn = rem / gm, tm = grp * SGM + rem % gm;
    const int m0 = tm * TBM, c0 = tn * (GLU ? SBN / 2 : SBN);
    const int nlim = GLU ? 2 * g.glu_half : g.N;

    // instruction i = wv + 8*j: i < 16 A-hi rows 16i.., then (LO) i < 32
    // A-lo, then W
    constexpr int NA = LO ? 32 : 16;
    const uint16_t *src[T_PER_WAVE];
    int dst[T_PER_WAVE];
#pragma unroll
    for (int j = 0; j < T_PER_WAVE; j++) {
        const int i = wv + 8 * j;
        const int Rl = lane >> 2, ch = lane & 3;
        if (i < NA) {
            const int R = (i & 15) * 16 + Rl;
            const int m = min(m0 + R, g.M - 1);
            src[j] = (i < 16 ? g.Ahi : g.Alo) + (long)m * g.lda + swz(R, ch) * 8;
            dst[j] = (i < 16 ? 0 : T_A) + (i & 15) * 16 * SBK;
        } else {
            const int R = (i - NA) * 16 + Rl;
            const int n = min(GLU ? (R < SBN / 2 ? c0 + R : g.glu_half + c0 + R - SBN / 2) : c0 + R, nlim - 1);
            src[j] = g.W + (long)n * g.K + swz(R, ch) * 8;
            dst[j] = (LO ? 2 : 1) * T_A + (i - NA) * 16 * SBK;
        }
    }
    // the DMA from inline assembly (lds_dma16_asm: this kernel has no other
    // M0 reader), so the fragment reads get exact LDS waits
    auto issue = [&](int kt) {
        uint16_t *stage = smem + (kt % TST) * T_STAGE;
#pragma unroll
        for (int j = 0; j < T_PER_WAVE; j++) lds_dma16_asm(src[j] + kt * SBK, stage + dst[j]);
    };
    // DMA instruction j of stage kt
    static_assert(T_PER_WAVE == 6, "the refill is spread 2, 2, 1, 1 over the row groups");
    auto issue1 = [&](int kt, int j) {
        lds_dma16_asm(src[j] + kt * SBK, smem + (kt % TST) * T_STAGE + dst[j]);
    };

    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int wm = (wv >> 1) * 64, wn = (wv & 1) * 128;
    const int nk = g.K / SBK;
#pragma unroll
    for (int p = 0; p < TST - 1; p++)
        if (p < nk) issue(p);
    for (int kt = 0; kt < nk; kt++) {
        // this wave's part of stage kt landed; younger stages stay in flight
        const int younger = min(nk - 1 - kt, TST - 2);
        if (younger >= 2) __builtin_amdgcn_s_waitcnt(((2 * T_PER_WAVE) & 0xF) | (0x7 << 4) | (0xF << 8));
        else if (younger == 1) __builtin_amdgcn_s_waitcnt((T_PER_WAVE & 0xF) | (0x7 << 4) | (0xF << 8));
        else __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // the refill of the freed slot (stage kt + TST - 1) goes out beside the
        // MFMAs: 2, 2, 1 and 1 DMA instructions after the row groups' reads
        const bool refill = kt + TST - 1 < nk;
        const uint16_t *st = smem + (kt % TST) * T_STAGE;
        const uint16_t *sAh = st, *sAl = st + T_A, *sW = st + (LO ? 2 : 1) * T_A;
        bf16x8 bfr[8];
#pragma unroll
        for (int cb = 0; cb < 8; cb++) {
            const int R = wn + cb * 16 + r;
            bfr[cb] = as_bf16x8(*reinterpret_cast<const u16x8 *>(sW + R * SBK + swz(R, kg) * 8));
        }
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            const int R = wm + rb * 16 + r;
            const int off = R * SBK + swz(R, kg) * 8;
            const bf16x8 ah = as_bf16x8(*reinterpret_cast<const u16x8 *>(sAh + off));
            const bf16x8 al = as_bf16x8(*reinterpret_cast<const u16x8 *>(sAl + off));
            if (refill) {
                if (rb < 2) {
                    issue1(kt + TST - 1, 2 * rb);
                    issue1(kt + TST - 1, 2 * rb + 1);
                } else {
                    issue1(kt + TST - 1, 2 + rb);
                }
            }
#pragma unroll
            for (int cb = 0; cb < 8; cb++) {
                acc[rb][cb] = mfma16(ah, bfr[cb], acc[rb][cb]);
                acc[rb][cb] = mfma16(al, bfr[cb], acc[rb][cb]);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    if (GLU) {
        // value column lc (< 128) of row m: (s + b) * sigmoid(gate s + gate b)
        float *sx = reinterpret_cast<float *>(smem);     // 256 x 128 gate sums = 128 KB
        if (wn >= SBN / 2) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int cb = 0; cb < 8; cb++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        sx[(wm + rb * 16 + kg * 4 + j) * (SBN / 2) + cb * 16 + r] = acc[rb][cb][j];
        }
        __syncthreads();
        if (wn < SBN / 2) {
#pragma unroll
            for (int cb = 0; cb < 8; cb++) {
                const int lc = cb * 16 + r, col = c0 + lc;
                if (col >= g.glu_half) continue;
                const float ba = g.bias ? bf2f(g.bias[col]) : 0.0f;
                const float bg = g.bias ? bf2f(g.bias[g.glu_half + col]) : 0.0f;
#pragma unroll
                for (int rb = 0; rb < 4; rb++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int lrow = wm + rb * 16 + kg * 4 + j, m = m0 + lrow;
                        if (m >= g.M) continue;
                        const float a = acc[rb][cb][j] + ba;
                        const float gt = sx[lrow * (SBN / 2) + lc] + bg;
                        g.Y[(long)m * g.ldy + col] = a * sigmoid_hw(gt);
                    }
            }
        }
        return;
    }
    // epilogue in two 128-row halves through the LDS ring (128 KB each); rows
    // finish 8 columns per thread (16-byte stores when vepi allows)
    float *sc = reinterpret_cast<float *>(smem);
    const int eg8 = tid & 31, ecol = c0 + eg8 * 8;
    Epi8 ep;
    if (vepi == 2 && ecol < g.N) ep = epi8_setup(g, ecol);
    for (int half = 0; half < 2; half++) {
        if ((wm >> 7) == half) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int cb = 0; cb < 8; cb++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int row = wm - 128 * half + rb * 16 + kg * 4 + j;
                        const int col = (wn + cb * 16 + r) ^ (((row >> 2) & 3) << 4);
                        sc[row * SBN + col] = acc[rb][cb][j];
                    }
        }
        __syncthreads();
        if (vepi == 2) {
            if (ecol < g.N) {
                // two batches of four rows: the other half's accumulators are still live
                epi8_rows<4>(g, ep, sc, tid >> 5, m0 + 128 * half, eg8);
                epi8_rows<4>(g, ep, sc, (tid >> 5) + 64, m0 + 128 * half, eg8);
            }
            __syncthreads();
            continue;
        }
        for (int it = tid; it < 128 * (SBN / 8); it += 512) {
            const int row = it / (SBN / 8), g8 = it % (SBN / 8);
            const int m = m0 + 128 * half + row, col = c0 + g8 * 8;
            if (m >= g.M || col >= g.N) continue;
            if (g.row_mask && !g.row_mask[m]) continue;
            const float4 *pv = reinterpret_cast<const float4 *>(sc + row * SBN + ((g8 * 8) ^ (((row >> 2) & 3) << 4)));
            const float4 v0 = pv[0], v1 = pv[1];
            float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            if (g.bias) {
                if (vepi) {
                    const u16x8 b8 = *reinterpret_cast<const u16x8 *>(g.bias + col);
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] += bf2f(b8[i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] += col + i < g.N ? bf2f(g.bias[col + i]) : 0.0f;
                }
            }
            if (vepi) {
                store_out8(g, m, col, v);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (col + i < g.N) store_out(g, m, col + i, v[i]);
            }
        }
        __syncthreads();
    }
}


// ---------------------------------------------------------------------------
// The 256 x 256 tile, single-pass form (A is bf16 alone: one MFMA per K-step
// and fragment; 4-stage ring of 32 KB, 4 DMA instructions per wave per stage),
// software-pipelined: the W fragments of K-step kt + 1 are read while the
// MFMAs of step kt run (two register sets), and each 16-row A fragment one
// row block ahead of its MFMAs, so LDS latency sits under the MFMAs.  Stage
// kt + 1 is made readable (its DMA waited for, one barrier) at the top of step
// kt, which also frees the slot of stage kt - 1 for the next DMA.  The number
// of K-steps must be even (K % 64 == 0): the last pair is peeled so that no
// LDS read sits under a branch.  Per element the MFMA sequence is unchanged.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void gemm_split256_sp_kernel(CtGemm g, int n_mt, int n_nt, int vepi) {
    constexpr int T_STAGE = Split256Cfg<false>::STAGE, T_PER_WAVE = Split256Cfg<false>::PER_WAVE;
    constexpr int TST = Split256Cfg<false>::STAGES;
    static_assert(TST >= 3, "the ring needs a landed stage, a stage in use and a free slot");
    __shared__ __attribute__((aligned(16))) uint16_t smem[TST * T_STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, kg = lane >> 4;
    const int nt = n_mt * n_nt;
    const int per = (nt + 7) / 8;
    const int t = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (t >= nt) return;
    const int gsize = SGM * n_nt;
    const int grp = t / gsize, rem = t % gsize;
    const int gm = min(SGM, n_mt - grp * SGM);
    const int tn = rem / gm, tm = grp * SGM + rem % gm;
    const int m0 = tm * TBM, c0 = tn * SBN;

    // instruction i = wv + 8*j: i < 16 A rows 16i.., then W
    const uint16_t *src[T_PER_WAVE];
    int dst[T_PER_WAVE];
#pragma unroll
    for (int j = 0; j < T_PER_WAVE; j++) {
        const int i = wv + 8 * j;
        const int Rl = lane >> 2, ch = lane & 3;
        if (i < 16) {
            const int R = i * 16 + Rl;
            const int m = min(m0 + R, g.M - 1);
            src[j] = g.Ahi + (long)m * g.lda + swz(R, ch) * 8;
            dst[j] = i * 16 * SBK;
        } else {
            const int R = (i - 16) * 16 + Rl;
            const int n = min(c0 + R, g.N - 1);
            src[j] = g.W + (long)n * g.K + swz(R, ch) * 8;
            dst[j] = T_A + (i - 16) * 16 * SBK;
        }
    }
    auto issue = [&](int kt) {
        uint16_t *stage = smem + (kt % TST) * T_STAGE;
#pragma unroll
        for (int j = 0; j < T_PER_WAVE; j++) lds_dma16_asm(src[j] + kt * SBK, stage + dst[j]);
    };
    // DMA instruction j of stage kt
    static_assert(T_PER_WAVE == 4, "one DMA instruction per MFMA row group");
    auto issue1 = [&](int kt, int j) {
        lds_dma16_asm(src[j] + kt * SBK, smem + (kt % TST) * T_STAGE + dst[j]);
    };
    const int wm = (wv >> 1) * 64, wn = (wv & 1) * 128;
    // fragment offsets within a stage: rows of one fragment share the swizzle
    const int aoff = (wm + r) * SBK + swz(r, kg) * 8;
    const int boff = T_A + (wn + r) * SBK + swz(r, kg) * 8;
    // W fragments of a stage (8) double-buffered across steps; A fragments of
    // a 16-row block read one block ahead (the last block's successor is
    // block 0 of the next stage)
    struct BFr { bf16x8 v[8]; };
    struct AFr { bf16x8 h; };
    auto read_b = [&](int kt, BFr &f) {
        const uint16_t *st = smem + (kt % TST) * T_STAGE;
#pragma unroll
        for (int cb = 0; cb < 8; cb++)
            f.v[cb] = as_bf16x8(*reinterpret_cast<const u16x8 *>(st + boff + cb * 16 * SBK));
    };
    // W fragments c0, c0 + 1 of step kt
    auto read_b2 = [&](int kt, int c0, BFr &f) {
        const uint16_t *st = smem + (kt % TST) * T_STAGE;
#pragma unroll
        for (int cb = c0; cb < c0 + 2; cb++)
            f.v[cb] = as_bf16x8(*reinterpret_cast<const u16x8 *>(st + boff + cb * 16 * SBK));
    };
    auto read_a = [&](int kt, int rb, AFr &f) {
        const uint16_t *st = smem + (kt % TST) * T_STAGE + aoff + rb * 16 * SBK;
        f.h = as_bf16x8(*reinterpret_cast<const u16x8 *>(st));
    };
    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    auto mma_row = [&](int rb, const AFr &a, const BFr &b) {
#pragma unroll
        for (int cb = 0; cb < 8; cb++) acc[rb][cb] = mfma16(a.h, b.v[cb], acc[rb][cb]);
    };
    // vmcnt(n * T_PER_WAVE): this wave's DMA of all but the n youngest stages landed
    auto wait_stages = [&](int n) {
        if (n >= 2) __builtin_amdgcn_s_waitcnt(((2 * T_PER_WAVE) & 0xF) | (0x7 << 4) | (0xF << 8));
        else if (n == 1) __builtin_amdgcn_s_waitcnt((T_PER_WAVE & 0xF) | (0x7 << 4) | (0xF << 8));
        else __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));
    };
    static_assert(TST - 3 <= 2 && 2 * T_PER_WAVE <= 15, "wait_stages covers at most two younger stages");
    const int nk = g.K / SBK;
#pragma unroll
    for (int p = 0; p < TST - 1; p++)
        if (p < nk) issue(p);
    wait_stages(min(nk - 1, TST - 2));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    BFr b0, b1;
    AFr a0, a1;
    read_b(0, b0);
    read_a(0, 0, a0);
    // step kt (kt + 1 < nk): make stage kt + 1 readable and refill the freed
    // slot, read W of kt + 1, then the row blocks of kt, each MFMA group with
    // the next block's A read in flight.  No branch around the reads, so each
    // wait leaves the younger reads in flight.
    auto step = [&](int kt, const BFr &bc, BFr &bn) {
        wait_stages(min(nk - 2 - kt, TST - 3));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // the refill of the freed slot (stage kt + TST - 1) goes out one DMA
        // instruction per MFMA group; LDS reads complete in issue order, so
        // each group's A fragment is read ahead of the two W fragments of
        // step kt + 1 that ride under the same group: its wait leaves them in
        // flight
        const bool refill = kt + TST - 1 < nk;
        read_a(kt, 1, a1);
        read_b2(kt + 1, 0, bn);
        if (refill) issue1(kt + TST - 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        mma_row(0, a0, bc);
        __builtin_amdgcn_sched_barrier(0);
        read_a(kt, 2, a0);
        read_b2(kt + 1, 2, bn);
        if (refill) issue1(kt + TST - 1, 1);
        __builtin_amdgcn_sched_barrier(0);
        mma_row(1, a1, bc);
        __builtin_amdgcn_sched_barrier(0);
        read_a(kt, 3, a1);
        read_b2(kt + 1, 4, bn);
        if (refill) issue1(kt + TST - 1, 2);
        __builtin_amdgcn_sched_barrier(0);
        mma_row(2, a0, bc);
        __builtin_amdgcn_sched_barrier(0);
        read_a(kt + 1, 0, a0);
        read_b2(kt + 1, 6, bn);
        if (refill) issue1(kt + TST - 1, 3);
        __builtin_amdgcn_sched_barrier(0);
        mma_row(3, a1, bc);
        __builtin_amdgcn_sched_barrier(0);
    };
    // the last step: no next stage
    auto last = [&](int kt, const BFr &bc) {
        read_a(kt, 1, a1);
        mma_row(0, a0, bc);
        read_a(kt, 2, a0);
        mma_row(1, a1, bc);
        read_a(kt, 3, a1);
        mma_row(2, a0, bc);
        mma_row(3, a1, bc);
    };
    // nk is even (the launch checks K % 64 == 0): the last pair is peeled
    for (int kt = 0; kt + 2 < nk; kt += 2) {
        step(kt, b0, b1);
        step(kt + 1, b1, b0);
    }
    step(nk - 2, b0, b1);
    last(nk - 1, b1);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    float *sc = reinterpret_cast<float *>(smem);
    const int eg8 = tid & 31, ecol = c0 + eg8 * 8;
    Epi8 ep;
    if (vepi == 2 && ecol < g.N) ep = epi8_setup(g, ecol);
    for (int half = 0; half < 2; half++) {
        if ((wm >> 7) == half) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int cb = 0; cb < 8; cb++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int row = wm - 128 * half + rb * 16 + kg * 4 + j;
                        const int col = (wn + cb * 16 + r) ^ (((row >> 2) & 3) << 4);
                        sc[row * SBN + col] = acc[rb][cb][j];
                    }
        }
        __syncthreads();
        if (vepi == 2) {
            if (ecol < g.N) {
                // two batches of four rows: the other half's accumulators are still live
                epi8_rows<4>(g, ep, sc, tid >> 5, m0 + 128 * half, eg8);
                epi8_rows<4>(g, ep, sc, (tid >> 5) + 64, m0 + 128 * half, eg8);
            }
            __syncthreads();
            continue;
        }
        for (int it = tid; it < 128 * (SBN / 8); it += 512) {
            const int row = it / (SBN / 8), g8 = it % (SBN / 8);
            const int m = m0 + 128 * half + row, col = c0 + g8 * 8;
            if (m >= g.M || col >= g.N) continue;
            if (g.row_mask && !g.row_mask[m]) continue;
            const float4 *pv = reinterpret_cast<const float4 *>(sc + row * SBN + ((g8 * 8) ^ (((row >> 2) & 3) << 4)));
            const float4 v0 = pv[0], v1 = pv[1];
            float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            if (g.bias) {
                if (vepi) {
                    const u16x8 b8 = *reinterpret_cast<const u16x8 *>(g.bias + col);
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] += bf2f(b8[i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] += col + i < g.N ? bf2f(g.bias[col + i]) : 0.0f;
                }
            }
            if (vepi) {
                store_out8(g, m, col, v);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (col + i < g.N) store_out(g, m, col + i, v[i]);
            }
        }
        __syncthreads();
    }
}

__global__ void split_kernel(uint16_t *hi, uint16_t *lo, const float *x, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint16_t h, l;
    split_bf16(x[i], h, l);
    hi[i] = h;
    lo[i] = l;
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
                    g.Y[(long)m * g.ldy + col] = s * sigmoid_hw(gt);
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

// The 16-byte epilogue needs 8-column groups that stay inside one segment
// (and one 128-column head) and 16-byte aligned destinations.
static int vector_epilogue_ok(const CtGemm *g) {
    if (g->N % 8 || ((uintptr_t)g->bias & 15)) return 0;
    if (g->nseg == 0) return ((uintptr_t)g->Y % 16 == 0) && g->ldy % 4 == 0;
    if (g->seg_w % 8) return 0;
    for (int i = 0; i < g->nseg; i++) {
        const CtSeg *sg = &g->seg[i];
        if (sg->mode == CT_OUT_SPLIT) {
            if (((uintptr_t)sg->base & 15) || ((uintptr_t)sg->base_lo & 15) || sg->ld % 8) return 0;
        } else if (sg->mode == CT_OUT_DENSE) {
            if (((uintptr_t)sg->base & 15) || sg->ld % 4) return 0;
        } else {
            const int el = sg->mode == CT_OUT_HEADS_BF16 ? 8 : 4;   /* elements per 16 B */
            if (((uintptr_t)sg->base & 15) || sg->hstride % el) return 0;
        }
    }
    return 1;
}

// Tile choice of the pre-split kernels, for tests: 0 follows the tile-count
// model below; 128 or 256 takes that tile wherever it applies (the two give
// the same bits: the same per-element MFMA sequence).
static int g_force_tile = 0;
extern "C" void ctk_gemm_force_tile(int rows) { g_force_tile = rows; }
extern "C" int ctk_gemm_sizeof(void) { return (int)sizeof(CtGemm); }

// Tile-count model for the two pre-split kernels: a 256-row tile costs about
// 1.74 128-row tiles (measured), and tiles run in rounds over the CUs.
static int prefer_256(int M, int n_nt) {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
    }
    const long t128 = (long)((M + SBM - 1) / SBM) * n_nt, t256 = (long)((M + TBM - 1) / TBM) * n_nt;
    const double r128 = (double)((t128 + cus - 1) / cus), r256 = (double)((t256 + cus - 1) / cus);
    return r256 * 1.74 < r128;
}

extern "C" void ctk_gemm(const CtGemm *g, hipStream_t s) {
    if (g->M <= 0 || g->N <= 0) return;
    if (g->epi == CT_EPI_GLU && g->N != 2 * g->glu_half) {
        fprintf(stderr, "ctk_gemm: GLU needs N == 2*glu_half\n");
        exit(1);
    }
    if (g->Ahi) {
        // pre-split activations: the DMA kernel (needs K % 32 == 0, 16-B aligned rows)
        if (!(g->K % SBK == 0 && g->lda % 8 == 0 && ((uintptr_t)g->Ahi & 15) == 0 &&
              ((uintptr_t)g->Alo & 15) == 0 && ((uintptr_t)g->W & 15) == 0)) {
            fprintf(stderr, "ctk_gemm: pre-split A needs K %% 32 == 0 and 16-byte aligned rows\n");
            exit(1);
        }
        const bool glu = g->epi == CT_EPI_GLU;
        const int n_mt = (g->M + SBM - 1) / SBM;
        const int n_nt = glu ? (g->glu_half + SBN / 2 - 1) / (SBN / 2) : (g->N + SBN - 1) / SBN;
        const int nt = n_mt * n_nt, per = (nt + 7) / 8;
        // 2: the batched vector epilogue (no row scatter), 1: vector stores, 0: scalar
        const int vepi = vector_epilogue_ok(g) ? (g->row_len ? 1 : 2) : 0;
        const bool lo = g->Alo != NULL;     /* no lo plane: single-pass bf16 A */
        const bool t256 = g_force_tile ? g_force_tile == 256
                                       : g->M >= CT_SPLIT256_MIN_M && prefer_256(g->M, n_nt);
        if (t256 && (glu ? lo : (lo || g->K % 64 == 0))) {
            const int n_mt2 = (g->M + TBM - 1) / TBM, nt2 = n_mt2 * n_nt, per2 = (nt2 + 7) / 8;
            if (glu) hipLaunchKernelGGL(gemm_split256_kernel<true>, dim3(per2 * 8), dim3(512), 0, s, *g, n_mt2, n_nt, 0);
            else if (lo) hipLaunchKernelGGL(gemm_split256_kernel<false>, dim3(per2 * 8), dim3(512), 0, s, *g, n_mt2, n_nt, vepi);
            else hipLaunchKernelGGL(gemm_split256_sp_kernel, dim3(per2 * 8), dim3(512), 0, s, *g, n_mt2, n_nt, vepi);
            return;
        }
        if (glu && lo) hipLaunchKernelGGL((gemm_split_kernel<true, true>), dim3(per * 8), dim3(512), 0, s, *g, n_mt, n_nt, 0);
        else if (glu) hipLaunchKernelGGL((gemm_split_kernel<true, false>), dim3(per * 8), dim3(512), 0, s, *g, n_mt, n_nt, 0);
        else if (lo) hipLaunchKernelGGL((gemm_split_kernel<false, true>), dim3(per * 8), dim3(512), 0, s, *g, n_mt, n_nt, vepi);
        else hipLaunchKernelGGL((gemm_split_kernel<false, false>), dim3(per * 8), dim3(512), 0, s, *g, n_mt, n_nt, vepi);
        return;
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
    if (vec && g->K % BK == 0 && g->M > 64) {
        // same per-element MFMA sequence as the small-M kernels: bit-identical rows
        const int n_mt = (g->M + BT - 1) / BT;
        const int n_nt = glu ? (g->glu_half + BT / 2 - 1) / (BT / 2) : (g->N + BT - 1) / BT;
        const int nt = n_mt * n_nt, per = (nt + 7) / 8;
        const int blocks = per * 8;
        if (glu) hipLaunchKernelGGL(gemm_big_kernel<true>, dim3(blocks), dim3(256), 0, s, *g, n_mt, n_nt, 0);
        else hipLaunchKernelGGL(gemm_big_kernel<false>, dim3(blocks), dim3(256), 0, s, *g, n_mt, n_nt,
                                vector_epilogue_ok(g));
        return;
    }
    if (vec) { if (glu) dispatch<true, true>(*g, s); else dispatch<true, false>(*g, s); }
    else     { if (glu) dispatch<false, true>(*g, s); else dispatch<false, false>(*g, s); }
}

extern "C" void ctk_split(uint16_t *hi, uint16_t *lo, const float *x, long n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(split_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, hi, lo, x, n);
}
