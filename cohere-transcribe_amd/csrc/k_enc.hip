// k_enc.hip — Conformer encoder kernels other than the GEMMs: the relative-
// position attention core, the depthwise-conv/BN/SiLU stage of the conv
// module, and the convolutional subsampling front-end.
//
// Activations are position-major ([t][channel]) everywhere so the pointwise
// convolutions are plain GEMMs.
#include "ct_dev.h"
#include "ct_launch.h"
#include "../../include/model_types.h"
#include <stdio.h>
#include <stdlib.h>

namespace {

// ---------------------------------------------------------------------------
// Relative-position attention core (backends/cpu/backend.c:262-296) on fp32
// MFMA (v_mfma_f32_16x16x4f32: exact fp32 products, fp32 sums).
// Workgroup = 16 query rows x one head, 4 waves.  S[q][k] = ((Q_q+u).K_k)*s +
// ((Q_q+v).P_{k+T-1-q})*s with s = 1/sqrt(160), softmax over k, then S V.
//   A: 16 x 16 score tiles over the keys (waves take tiles w, w+4, ...);
//   B: 16 x 16 tiles over the window of T+15 P rows the block needs; window
//      row j of query i is key j + i - 15, so each product lands on exactly
//      one score and is added there;
//   softmax per row in LDS; C: O = S V as 10 tiles of 16 head dimensions.
// MFMA lanes: A[i][k] from lane 16k + i, B[k][j] from lane 16k + j, result
// D[4(l/16) + r][l%16] in lane l.  Scores live in LDS, row stride ldS.
// Rows of Q, K, P, V must be 16-byte aligned (the launchers check).
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int RQ = 16;                // query rows per workgroup
constexpr int RKS = ENC_DK / 4;       // 40 MFMA K-steps over the head dimension

template <bool PACKED>
__global__ __launch_bounds__(256) void relpos_attn_kernel(float *O, const float *Q, const float *K,
                                                          const float *V, const float *P,
                                                          const uint16_t *pbu, const uint16_t *pbv,
                                                          int T_arg, int T_max, const int *seq_off,
                                                          const int *seq_T, const int *blk_seq,
                                                          const int *blk_q0, int ldS,
                                                          uint16_t *Oh, uint16_t *Ol) {
    extern __shared__ float S[];      // [RQ][ldS]
    // Dispatch order: workgroup L = x + y * gridDim.x runs on XCD L mod 8, so
    // L is taken as (block L / 8, head L mod 8): every block of head h runs on
    // XCD h, in block order, and a clip-head's consecutive query blocks share
    // that XCD's L2 for its K, P and V rows.
    const int lin = blockIdx.x + blockIdx.y * gridDim.x;
    const int bi = lin / ENC_H, h = lin % ENC_H;
    int T, q0;
    long off = 0;
    if (PACKED) {
        const int sq = blk_seq[bi];
        q0 = blk_q0[bi];
        T = seq_T[sq];
        off = seq_off[sq];
        P += (long)(T_max - T) * ENC_D;     // this clip's window of the T_max table
    } else {
        T = T_arg;
        q0 = bi * RQ;
    }
    Q += off * ENC_D; K += off * ENC_D; V += off * ENC_D;
    // the output goes to O, or split hi/lo to the planes Oh/Ol
    if (Oh) { Oh += off * ENC_D; Ol += off * ENC_D; }
    else O += off * ENC_D;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lk = lane >> 4;
    const int nq = min(RQ, T - q0);
    const long hc = (long)h * ENC_DK;
    const float sc = 1.0f / sqrtf((float)ENC_DK);

    // The MFMA K index of step st = 4c + e in lane group lk is head dim
    // 16c + 4lk + e: a float4 load c of row li takes dims [16c, 16c + 16) of
    // the row across the 4 lane groups, one 64-byte segment.  (With a 160-
    // byte run per lane, each segment is requested by 4 successive loads and
    // the L1 does not keep it between them: twice the L1 -> L2 requests.)
    // A fragments of Q+u and Q+v: row li.
    float au[RKS], av[RKS];
    {
        const bool ok = li < nq;
        const float4 *qp = reinterpret_cast<const float4 *>(Q + (long)(q0 + li) * ENC_D + hc + 4 * lk);
#pragma unroll
        for (int c = 0; c < RKS / 4; c++) {
            const float4 x = ok ? qp[4 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
            const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int st = 4 * c + e, d = 16 * c + 4 * lk + e;
                au[st] = xs[e] + bf2f(pbu[hc + d]);
                av[st] = xs[e] + bf2f(pbv[hc + d]);
            }
        }
    }
    // A: content scores
    const int nkt = (T + 15) / 16;
    for (int kt = w; kt < nkt; kt += 4) {
        const int key = kt * 16 + li;
        const bool ok = key < T;
        const float4 *kp = reinterpret_cast<const float4 *>(K + (long)key * ENC_D + hc + 4 * lk);
        float b[RKS];
#pragma unroll
        for (int c = 0; c < RKS / 4; c++) {
            const float4 x = ok ? kp[4 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
            b[4 * c] = x.x; b[4 * c + 1] = x.y; b[4 * c + 2] = x.z; b[4 * c + 3] = x.w;
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < RKS; st++) acc = mfma4(au[st], b[st], acc);
        if (ok) {
#pragma unroll
            for (int j = 0; j < 4; j++) S[(4 * lk + j) * ldS + key] = acc[j] * sc;
        }
    }
    __syncthreads();
    // B: position scores over window rows p = plo + win, win in [0, T+15)
    const int plo = T - 1 - (q0 + RQ - 1);
    const int nwt = (T + RQ - 1 + 15) / 16;
    for (int wt = w; wt < nwt; wt += 4) {
        const int win = wt * 16 + li, p = plo + win;
        const bool ok = win < T + RQ - 1 && p >= 0 && p <= 2 * T - 2;
        const float4 *pp = reinterpret_cast<const float4 *>(P + (long)p * ENC_D + hc + 4 * lk);
        float b[RKS];
#pragma unroll
        for (int c = 0; c < RKS / 4; c++) {
            const float4 x = ok ? pp[4 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
            b[4 * c] = x.x; b[4 * c + 1] = x.y; b[4 * c + 2] = x.z; b[4 * c + 3] = x.w;
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < RKS; st++) acc = mfma4(av[st], b[st], acc);
        // column li of the tile is window row win; query i = 4*lk + j reads
        // it as key win + i - 15
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int qi = 4 * lk + j, k = win + qi - (RQ - 1);
            if (ok && qi < nq && k >= 0 && k < T) S[qi * ldS + k] += acc[j] * sc;
        }
    }
    __syncthreads();
    // softmax per row (backends/cpu/backend.c:67-73)
    for (int qi = w; qi < nq; qi += 4) {
        float *row = S + qi * ldS;
        float mx = -INFINITY;
        for (int k = lane; k < T; k += 64) mx = fmaxf(mx, row[k]);
        mx = wave_max(mx);
        float sum = 0.0f;
        // e^(s - max) as 2^((s - max) log2 e) on the hardware exp2
        for (int k = lane; k < T; k += 64) {
            const float e = __builtin_amdgcn_exp2f((row[k] - mx) * 1.4426950408889634f);
            row[k] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        for (int k = lane; k < T; k += 64) row[k] /= sum;
    }
    __syncthreads();
    // C: O = S V, 10 tiles of 16 dimensions, keys in steps of 4
    for (int dt = w; dt < ENC_DK / 16; dt += 4) {
        const int d = dt * 16 + li;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const float *vp = V + hc + d;
        const float *sr = S + (li < nq ? li : 0) * ldS;
        int k0 = 0;
        for (; k0 + 32 <= T; k0 += 32) {
            float a[8], bv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int k = k0 + 4 * u + lk;
                a[u] = sr[k];
                bv[u] = vp[(long)k * ENC_D];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) acc = mfma4(a[u], bv[u], acc);
        }
        if (k0 < T) {
            // the last T - k0 < 32 keys: every load of the batch goes out before
            // the first MFMA (one round trip instead of one per step of 4
            // keys); the MFMAs are the same steps as one at a time
            float a[8], bv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int k = k0 + 4 * u + lk;
                a[u] = k < T ? sr[k] : 0.0f;
                bv[u] = k < T ? vp[(long)k * ENC_D] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (k0 + 4 * u < T) acc = mfma4(a[u], bv[u], acc);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int qi = 4 * lk + j;
            if (qi >= nq) continue;
            const long o = (long)(q0 + qi) * ENC_D + hc + d;
            if (Oh) {
                uint16_t hh, ll;
                split_bf16(acc[j], hh, ll);
                Oh[o] = hh;
                Ol[o] = ll;
            } else {
                O[o] = acc[j];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Depthwise conv (k = 9, zero padding 4 inside the sequence) + inference
// BatchNorm + SiLU (backends/cpu/backend.c:312-334).
// ---------------------------------------------------------------------------
// One thread per 8 consecutive channels of DW_RB consecutive rows: the
// DW_RB + 8 input rows the taps reach are read once (16-byte pieces) and kept
// in registers, so each input row is fetched about twice instead of once per
// tap.  The arithmetic per element is the scalar form's (taps in order, taps
// outside the row's sequence skipped, then BN and SiLU).
constexpr int DW_RB = 8;
__global__ __launch_bounds__(256) void dwconv_bn_silu_kernel(float *out, uint16_t *out_hi, uint16_t *out_lo,
                                                             const float *in, int M, const int *row_start,
                                                             const int *row_len, const uint16_t *dww,
                                                             const uint16_t *dwb, const uint16_t *bnw,
                                                             const uint16_t *bnb, const uint16_t *bnm,
                                                             const uint16_t *bnv) {
    constexpr int G = ENC_D / 8, HALO = (ENC_CK - 1) / 2, NX = DW_RB + ENC_CK - 1;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int nrb = (M + DW_RB - 1) / DW_RB;
    if (i >= (long)nrb * G) return;
    const int r0 = (int)(i / G) * DW_RB, c0 = (int)(i % G) * 8;
    // input rows r0 - 4 .. r0 + DW_RB + 3 of these 8 channels (zero outside [0, M))
    float x[NX][8];
#pragma unroll
    for (int j = 0; j < NX; j++) {
        const int rr = r0 - HALO + j;
        if (rr >= 0 && rr < M) {
            const float4 *p = reinterpret_cast<const float4 *>(in + (long)rr * ENC_D + c0);
            const float4 x0 = p[0], x1 = p[1];
            x[j][0] = x0.x; x[j][1] = x0.y; x[j][2] = x0.z; x[j][3] = x0.w;
            x[j][4] = x1.x; x[j][5] = x1.y; x[j][6] = x1.z; x[j][7] = x1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) x[j][e] = 0.0f;
        }
    }
    // taps of the 8 channels: dww[c][k] for c0 <= c < c0 + 8, 72 contiguous values
    uint16_t wk[8 * ENC_CK];
#pragma unroll
    for (int v = 0; v < ENC_CK; v++) {
        const u16x8 w8 = *reinterpret_cast<const u16x8 *>(dww + c0 * ENC_CK + 8 * v);
#pragma unroll
        for (int e = 0; e < 8; e++) wk[8 * v + e] = w8[e];
    }
    const u16x8 b8 = *reinterpret_cast<const u16x8 *>(dwb + c0);
    const u16x8 m8 = *reinterpret_cast<const u16x8 *>(bnm + c0), v8 = *reinterpret_cast<const u16x8 *>(bnv + c0);
    const u16x8 w8 = *reinterpret_cast<const u16x8 *>(bnw + c0), bb8 = *reinterpret_cast<const u16x8 *>(bnb + c0);
#pragma unroll
    for (int rb = 0; rb < DW_RB; rb++) {
        const int r = r0 + rb;
        if (r >= M) break;
        const int st = row_start ? row_start[r] : 0;       // this row's sequence: [st, st + T)
        const int T = row_len ? row_len[r] : M;
        const int t = r - st;
        float s[8];
#pragma unroll
        for (int e = 0; e < 8; e++) s[e] = bf2f(b8[e]);
#pragma unroll
        for (int k = 0; k < ENC_CK; k++) {
            const int ti = t - HALO + k;
            if (ti < 0 || ti >= T) continue;
            // input row st + ti = r - HALO + k is x[rb + k]
#pragma unroll
            for (int e = 0; e < 8; e++) s[e] += bf2f(wk[e * ENC_CK + k]) * x[rb + k][e];
        }
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float v = (s[e] - bf2f(m8[e])) / sqrtf(bf2f(v8[e]) + 1e-5f) * bf2f(w8[e]) + bf2f(bb8[e]);
            o[e] = v * sigmoid_hw(v);
        }
        const long oi = (long)r * ENC_D + c0;
        if (out_hi) {
            u16x8 h8, l8;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                uint16_t hh, ll;
                split_bf16(o[e], hh, ll);
                h8[e] = hh; l8[e] = ll;
            }
            *reinterpret_cast<u16x8 *>(out_hi + oi) = h8;
            *reinterpret_cast<u16x8 *>(out_lo + oi) = l8;
        } else {
            float4 *y = reinterpret_cast<float4 *>(out + oi);
            y[0] = make_float4(o[0], o[1], o[2], o[3]);
            y[1] = make_float4(o[4], o[5], o[6], o[7]);
        }
    }
}

// ---------------------------------------------------------------------------
// Subsampling (backends/cpu/backend.c:188-229).
// conv0: 3x3 stride 2 pad 1, 1 -> 256 channels, + ReLU, over the image
// img[t][m] = mel[m*stride + t]; output [T1][64][256].
// ---------------------------------------------------------------------------
__global__ void sub_conv0_kernel(float *out, const float *mel, int T_mel, int stride,
                                 const uint16_t *w, const uint16_t *b) {
    const int T1 = (T_mel + 1) / 2;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T1 * 64 * SUB_CH) return;
    const int oc = (int)(i % SUB_CH);
    const int ow = (int)((i / SUB_CH) % 64);
    const int oh = (int)(i / (SUB_CH * 64));
    float s = bf2f(b[oc]);
#pragma unroll
    for (int kh = 0; kh < 3; kh++) {
        const int ih = oh * 2 - 1 + kh;
        if (ih < 0 || ih >= T_mel) continue;
#pragma unroll
        for (int kw = 0; kw < 3; kw++) {
            const int iw = ow * 2 - 1 + kw;
            if (iw < 0 || iw >= N_MELS) continue;
            s += mel[(long)iw * stride + ih] * bf2f(w[oc * 9 + kh * 3 + kw]);
        }
    }
    out[i] = s > 0.0f ? s : 0.0f;
}

// Depthwise 3x3 stride 2 pad 1 over [H][Wd][256] -> [(H+1)/2][(Wd+1)/2][256].
__global__ void sub_dwconv_kernel(float *out, const float *in, int H, int Wd,
                                  const uint16_t *w, const uint16_t *b) {
    const int Ho = (H + 1) / 2, Wo = (Wd + 1) / 2;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)Ho * Wo * SUB_CH) return;
    const int c = (int)(i % SUB_CH);
    const int ow = (int)((i / SUB_CH) % Wo);
    const int oh = (int)(i / ((long)SUB_CH * Wo));
    float s = bf2f(b[c]);
#pragma unroll
    for (int kh = 0; kh < 3; kh++) {
        const int ih = oh * 2 - 1 + kh;
        if (ih < 0 || ih >= H) continue;
#pragma unroll
        for (int kw = 0; kw < 3; kw++) {
            const int iw = ow * 2 - 1 + kw;
            if (iw < 0 || iw >= Wd) continue;
            s += in[((long)ih * Wd + iw) * SUB_CH + c] * bf2f(w[c * 9 + kh * 3 + kw]);
        }
    }
    out[i] = s;
}

// Request of packed row tau: the r with off[r] <= tau < off[r + 1] (off has
// n + 1 ascending entries, off[0] = 0).
__device__ __forceinline__ int packed_owner(const int *off, int n, int tau) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= tau) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// The first two subsampling stages fused, over several requests packed
// along time: conv 3x3 stride 2 (1 -> 256 channels, ReLU) then depthwise
// 3x3 stride 2, without storing the conv output.  Workgroup = one output row
// tau of the depthwise stage (request r, row oh = tau - o2[r]), thread =
// channel c, looping over the 32 output columns.  The 7 mel frames the row
// needs (4*oh - 3 .. 4*oh + 3, all 128 bins) are staged in LDS; each conv
// value a depthwise tap needs is recomputed from them (9 products), in the
// same order and with the same skips as sub_conv0 then sub_dwconv, so the
// result is bit-identical to running the two stages
// (backends/cpu/backend.c:201-221).  The output is written split hi/lo for
// the pointwise GEMM that reads it.
constexpr int C0D_FRAMES = 7;
__global__ __launch_bounds__(256) void sub_conv0_dw_packed_kernel(uint16_t *out_hi, uint16_t *out_lo,
                                                                  const float *mel,
                                                                  const int *o1, const int *o2,
                                                                  const int *tmel, const int *moff, int n,
                                                                  const uint16_t *w0, const uint16_t *b0,
                                                                  const uint16_t *wd, const uint16_t *bd) {
    __shared__ float sm[C0D_FRAMES][N_MELS];
    const int tau = blockIdx.x, c = threadIdx.x;
    const int r = packed_owner(o2, n, tau);
    const int oh = tau - o2[r], H1 = o1[r + 1] - o1[r], T_mel = tmel[r];
    const float *m = mel + moff[r];
    const int f0 = 4 * oh - 3;                 // first mel frame of the window
    for (int e = c; e < C0D_FRAMES * N_MELS; e += 256) {
        const int fr = e / N_MELS, bin = e % N_MELS, ih0 = f0 + fr;
        sm[fr][bin] = (ih0 >= 0 && ih0 < T_mel) ? m[(long)bin * T_mel + ih0] : 0.0f;
    }
    float k0[9], kd[9];
#pragma unroll
    for (int k = 0; k < 9; k++) { k0[k] = bf2f(w0[c * 9 + k]); kd[k] = bf2f(wd[c * 9 + k]); }
    const float bias0 = bf2f(b0[c]), biasd = bf2f(bd[c]);
    __syncthreads();
    const long orow = (long)tau * 32 * SUB_CH + c;
    for (int ow = 0; ow < 32; ow++) {
        float acc = biasd;
#pragma unroll
        for (int kh2 = 0; kh2 < 3; kh2++) {
            const int ih1 = oh * 2 - 1 + kh2;
            if (ih1 < 0 || ih1 >= H1) continue;
#pragma unroll
            for (int kw2 = 0; kw2 < 3; kw2++) {
                const int iw1 = ow * 2 - 1 + kw2;
                if (iw1 < 0 || iw1 >= 64) continue;
                // conv value at (ih1, iw1, c)
                float x = bias0;
#pragma unroll
                for (int kh = 0; kh < 3; kh++) {
                    const int ih0 = ih1 * 2 - 1 + kh;
                    if (ih0 < 0 || ih0 >= T_mel) continue;
#pragma unroll
                    for (int kw = 0; kw < 3; kw++) {
                        const int iw0 = iw1 * 2 - 1 + kw;
                        if (iw0 < 0 || iw0 >= N_MELS) continue;
                        x += sm[ih0 - f0][iw0] * k0[kh * 3 + kw];
                    }
                }
                x = x > 0.0f ? x : 0.0f;
                acc += x * kd[kh2 * 3 + kw2];
            }
        }
        uint16_t hh, ll;
        split_bf16(acc, hh, ll);
        out_hi[orow + (long)ow * SUB_CH] = hh;
        out_lo[orow + (long)ow * SUB_CH] = ll;
    }
}

// sub_dwconv_kernel over several requests, written split hi/lo for the
// pointwise GEMM: request r's input rows oin[r] .. oin[r + 1] of
// [sum H][Wd][256], output rows oout[r] .. oout[r + 1] of
// [sum (H+1)/2][(Wd+1)/2][256].  Workgroup = one output row, thread =
// channel, looping over the output columns; each sum is the scalar form's
// (taps in order, skips at the edges).
__global__ __launch_bounds__(256) void sub_dw_split_packed_kernel(uint16_t *out_hi, uint16_t *out_lo,
                                                                  const float *in, const int *oin,
                                                                  const int *oout, int n, int Wd,
                                                                  const uint16_t *w, const uint16_t *b) {
    const int Wo = (Wd + 1) / 2;
    const int tau = blockIdx.x, c = threadIdx.x;
    const int r = packed_owner(oout, n, tau);
    const int oh = tau - oout[r], H = oin[r + 1] - oin[r];
    const float *x = in + (long)oin[r] * Wd * SUB_CH + c;
    float k[9];
#pragma unroll
    for (int j = 0; j < 9; j++) k[j] = bf2f(w[c * 9 + j]);
    const float bias = bf2f(b[c]);
    for (int ow = 0; ow < Wo; ow++) {
        float s = bias;
#pragma unroll
        for (int kh = 0; kh < 3; kh++) {
            const int ih = oh * 2 - 1 + kh;
            if (ih < 0 || ih >= H) continue;
#pragma unroll
            for (int kw = 0; kw < 3; kw++) {
                const int iw = ow * 2 - 1 + kw;
                if (iw < 0 || iw >= Wd) continue;
                s += x[((long)ih * Wd + iw) * SUB_CH] * k[kh * 3 + kw];
            }
        }
        uint16_t hh, ll;
        split_bf16(s, hh, ll);
        const long o = ((long)tau * Wo + ow) * SUB_CH + c;
        out_hi[o] = hh;
        out_lo[o] = ll;
    }
}

// [T][16][256] -> [T][ch*16 + f] (backends/cpu/backend.c:222-226).
__global__ void sub_flatten_kernel(float *out, const float *in, int T) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * 16 * SUB_CH) return;
    const int f = (int)(i % 16);
    const int c = (int)((i / 16) % SUB_CH);
    const long t = i / (16 * SUB_CH);
    out[i] = in[(t * 16 + f) * SUB_CH + c];
}

// The same flatten, written as hi/lo bf16 planes for the pre-split GEMM.
__global__ void sub_flatten_split_kernel(uint16_t *hi, uint16_t *lo, const float *in, int T) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * 16 * SUB_CH) return;
    const int f = (int)(i % 16);
    const int c = (int)((i / 16) % SUB_CH);
    const long t = i / (16 * SUB_CH);
    uint16_t h, l;
    split_bf16(in[(t * 16 + f) * SUB_CH + c], h, l);
    hi[i] = h;
    lo[i] = l;
}

inline unsigned nblk(long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

// The 8-channel form reads every operand in 16-byte pieces.
static void dw_check(const float *out, const uint16_t *out_hi, const float *in, const uint16_t *dww,
                     const uint16_t *dwb, const uint16_t *bnw, const uint16_t *bnb,
                     const uint16_t *bnm, const uint16_t *bnv) {
    const uintptr_t a = (uintptr_t)out | (uintptr_t)out_hi | (uintptr_t)in | (uintptr_t)dww |
                        (uintptr_t)dwb | (uintptr_t)bnw | (uintptr_t)bnb | (uintptr_t)bnm | (uintptr_t)bnv;
    if (a & 15) {
        fprintf(stderr, "dwconv: activations and parameters must be 16-byte aligned\n");
        exit(1);
    }
}

static int relpos_qb(int) { return RQ; }

// Score rows of ldS floats: T rounded up to 16, plus 4 so that 16 rows x 4
// columns of a fragment read fall in distinct banks.
static int relpos_lds(int max_T, size_t *bytes) {
    const int ldS = (max_T + 15) / 16 * 16 + 4;
    *bytes = (size_t)RQ * ldS * sizeof(float);
    return ldS;
}

template <bool PACKED>
static void relpos_allow_lds(size_t bytes) {
    static size_t allowed = 64 * 1024;
    if (bytes <= allowed) return;
    if (hipFuncSetAttribute((const void *)relpos_attn_kernel<PACKED>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) {
        fprintf(stderr, "relpos_attn: cannot reserve %zu bytes of LDS\n", bytes);
        exit(1);
    }
    allowed = bytes;
}

extern "C" void ctk_relpos_attn(float *O, const float *Q, const float *K, const float *V,
                                const float *P, const uint16_t *pbu, const uint16_t *pbv,
                                int T, hipStream_t s) {
    if (T <= 0) return;
    if (T > 2048) {
        fprintf(stderr, "ctk_relpos_attn: T=%d exceeds the supported 2048 frames\n", T);
        exit(1);
    }
    if (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V | (uintptr_t)P) & 15) {
        fprintf(stderr, "ctk_relpos_attn: Q, K, V and P must be 16-byte aligned\n");
        exit(1);
    }
    size_t lds;
    const int ldS = relpos_lds(T, &lds);
    relpos_allow_lds<false>(lds);
    const dim3 grid((T + RQ - 1) / RQ, ENC_H);
    hipLaunchKernelGGL((relpos_attn_kernel<false>), grid, dim3(256), lds, s,
                       O, Q, K, V, P, pbu, pbv, T, T, nullptr, nullptr, nullptr, nullptr, ldS,
                       nullptr, nullptr);
}

extern "C" int ctk_relpos_plan(int *blk_seq, int *blk_q0, const int *seq_T, int n_seq) {
    int mx = 0;
    for (int i = 0; i < n_seq; i++) mx = seq_T[i] > mx ? seq_T[i] : mx;
    const int qb = relpos_qb(mx);
    int n = 0;
    for (int i = 0; i < n_seq; i++)
        for (int q0 = 0; q0 < seq_T[i]; q0 += qb) {
            if (blk_seq) { blk_seq[n] = i; blk_q0[n] = q0; }
            n++;
        }
    return n;
}

extern "C" void ctk_relpos_attn_packed(float *O, uint16_t *Oh, uint16_t *Ol, const float *Q,
                                       const float *K, const float *V, const float *P, int T_max,
                                       const uint16_t *pbu, const uint16_t *pbv, const int *seq_off,
                                       const int *seq_T, const int *blk_seq, const int *blk_q0,
                                       int n_blk, int max_T, hipStream_t s) {
    if (n_blk <= 0) return;
    if (max_T > 2048) {
        fprintf(stderr, "ctk_relpos_attn_packed: T=%d exceeds the supported 2048 frames\n", max_T);
        exit(1);
    }
    if (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V | (uintptr_t)P) & 15) {
        fprintf(stderr, "ctk_relpos_attn: Q, K, V and P must be 16-byte aligned\n");
        exit(1);
    }
    if (!O == !Oh || !Oh != !Ol) {
        fprintf(stderr, "ctk_relpos_attn_packed: give either O or both planes Oh, Ol\n");
        exit(1);
    }
    size_t lds;
    const int ldS = relpos_lds(max_T, &lds);
    relpos_allow_lds<true>(lds);
    const dim3 grid(n_blk, ENC_H);
    hipLaunchKernelGGL((relpos_attn_kernel<true>), grid, dim3(256), lds, s,
                       O, Q, K, V, P, pbu, pbv, 0, T_max, seq_off, seq_T, blk_seq, blk_q0, ldS, Oh, Ol);
}

extern "C" void ctk_dwconv_bn_silu(float *out, const float *in, int T, const uint16_t *dww,
                                   const uint16_t *dwb, const uint16_t *bnw, const uint16_t *bnb,
                                   const uint16_t *bnm, const uint16_t *bnv, hipStream_t s) {
    if (T <= 0) return;
    dw_check(out, nullptr, in, dww, dwb, bnw, bnb, bnm, bnv);
    hipLaunchKernelGGL(dwconv_bn_silu_kernel, dim3(nblk((long)((T + DW_RB - 1) / DW_RB) * (ENC_D / 8))), dim3(256), 0, s,
                       out, nullptr, nullptr, in, T, nullptr, nullptr, dww, dwb, bnw, bnb, bnm, bnv);
}

extern "C" void ctk_dwconv_bn_silu_packed(uint16_t *out_hi, uint16_t *out_lo, const float *in, int M,
                                          const int *row_start, const int *row_len,
                                          const uint16_t *dww, const uint16_t *dwb,
                                          const uint16_t *bnw, const uint16_t *bnb,
                                          const uint16_t *bnm, const uint16_t *bnv, hipStream_t s) {
    if (M <= 0) return;
    dw_check(nullptr, out_hi, in, dww, dwb, bnw, bnb, bnm, bnv);
    if ((uintptr_t)out_lo & 15) { fprintf(stderr, "dwconv: outputs must be 16-byte aligned\n"); exit(1); }
    hipLaunchKernelGGL(dwconv_bn_silu_kernel, dim3(nblk((long)((M + DW_RB - 1) / DW_RB) * (ENC_D / 8))), dim3(256), 0, s,
                       nullptr, out_hi, out_lo, in, M, row_start, row_len, dww, dwb, bnw, bnb, bnm, bnv);
}

extern "C" void ctk_sub_conv0(float *out, const float *mel, int T_mel, int stride,
                              const uint16_t *w, const uint16_t *b, hipStream_t s) {
    const long n = (long)((T_mel + 1) / 2) * 64 * SUB_CH;
    if (n <= 0) return;
    hipLaunchKernelGGL(sub_conv0_kernel, dim3(nblk(n)), dim3(256), 0, s, out, mel, T_mel, stride, w, b);
}

extern "C" void ctk_sub_dwconv(float *out, const float *in, int H, int Wd,
                               const uint16_t *w, const uint16_t *b, hipStream_t s) {
    const long n = (long)((H + 1) / 2) * ((Wd + 1) / 2) * SUB_CH;
    if (n <= 0) return;
    hipLaunchKernelGGL(sub_dwconv_kernel, dim3(nblk(n)), dim3(256), 0, s, out, in, H, Wd, w, b);
}

extern "C" void ctk_sub_conv0_dw_packed(uint16_t *out_hi, uint16_t *out_lo, const float *mel, const int *o1,
                                        const int *o2,
                                        const int *tmel, const int *moff, int n, int rows2,
                                        const uint16_t *w0, const uint16_t *b0, const uint16_t *wd,
                                        const uint16_t *bd, hipStream_t s) {
    if (rows2 <= 0 || n <= 0) return;
    hipLaunchKernelGGL(sub_conv0_dw_packed_kernel, dim3(rows2), dim3(256), 0, s, out_hi, out_lo, mel, o1, o2,
                       tmel, moff, n, w0, b0, wd, bd);
}

extern "C" void ctk_sub_dw_split_packed(uint16_t *out_hi, uint16_t *out_lo, const float *in, const int *oin,
                                        const int *oout, int n, int rows_out, int Wd, const uint16_t *w,
                                        const uint16_t *b, hipStream_t s) {
    if (rows_out <= 0 || n <= 0) return;
    hipLaunchKernelGGL(sub_dw_split_packed_kernel, dim3(rows_out), dim3(256), 0, s, out_hi, out_lo, in, oin, oout,
                       n, Wd, w, b);
}

extern "C" void ctk_sub_flatten_split(uint16_t *hi, uint16_t *lo, const float *in, int T, hipStream_t s) {
    const long n = (long)T * 16 * SUB_CH;
    if (n <= 0) return;
    hipLaunchKernelGGL(sub_flatten_split_kernel, dim3(nblk(n)), dim3(256), 0, s, hi, lo, in, T);
}

extern "C" void ctk_sub_flatten(float *out, const float *in, int T, hipStream_t s) {
    const long n = (long)T * 16 * SUB_CH;
    if (n <= 0) return;
    hipLaunchKernelGGL(sub_flatten_kernel, dim3(nblk(n)), dim3(256), 0, s, out, in, T);
}
