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
// Relative-position attention core (backends/cpu/backend.c:262-296).
// Workgroup = QB query rows x one head.  S[q][k] = ((Q_q+u).K_k)*s +
// ((Q_q+v).P_{k+T-1-q})*s with s = 1/sqrt(160), softmax over k, then S V.
// Phase A walks keys, phase B walks the P window (T+QB-1 rows); each score
// receives exactly one term from each phase.
// ---------------------------------------------------------------------------
template <int QB, bool PACKED>
__global__ __launch_bounds__(256) void relpos_attn_kernel(float *O, const float *Q, const float *K,
                                                          const float *V, const float *P,
                                                          const uint16_t *pbu, const uint16_t *pbv,
                                                          int T_arg, int T_max, const int *seq_off,
                                                          const int *seq_T, const int *blk_seq,
                                                          const int *blk_q0) {
    extern __shared__ float smem[];
    int T, q0;
    long off = 0;
    if (PACKED) {
        const int sq = blk_seq[blockIdx.x];
        q0 = blk_q0[blockIdx.x];
        T = seq_T[sq];
        off = seq_off[sq];
        P += (long)(T_max - T) * ENC_D;     // this clip's window of the T_max table
    } else {
        T = T_arg;
        q0 = blockIdx.x * QB;
    }
    Q += off * ENC_D; K += off * ENC_D; V += off * ENC_D; O += off * ENC_D;
    float *qu = smem;                         // [QB][160]
    float *qv = qu + QB * ENC_DK;             // [QB][160]
    float *S = qv + QB * ENC_DK;              // [QB][T]
    const int h = blockIdx.y, tid = threadIdx.x;
    const int nq = min(QB, T - q0);
    const float sc = 1.0f / sqrtf((float)ENC_DK);
    for (int i = tid; i < QB * ENC_DK; i += 256) {
        const int qi = i / ENC_DK, d = i % ENC_DK;
        const float x = qi < nq ? Q[(long)(q0 + qi) * ENC_D + h * ENC_DK + d] : 0.0f;
        qu[i] = x + bf2f(pbu[h * ENC_DK + d]);
        qv[i] = x + bf2f(pbv[h * ENC_DK + d]);
    }
    __syncthreads();
    // phase A: content term
    for (int k = tid; k < T; k += 256) {
        const float *kr = K + (long)k * ENC_D + h * ENC_DK;
        float acc[QB];
#pragma unroll
        for (int qi = 0; qi < QB; qi++) acc[qi] = 0.0f;
        for (int d = 0; d < ENC_DK; d++) {
            const float kd = kr[d];
#pragma unroll
            for (int qi = 0; qi < QB; qi++) acc[qi] += qu[qi * ENC_DK + d] * kd;
        }
#pragma unroll
        for (int qi = 0; qi < QB; qi++) S[qi * T + k] = acc[qi] * sc;
    }
    __syncthreads();
    // phase B: position term over the window of P rows this query block uses
    const int plo = T - 1 - (q0 + QB - 1);
    const int nwin = T + QB - 1;
    for (int w = tid; w < nwin; w += 256) {
        const int p = plo + w;
        if (p < 0 || p > 2 * T - 2) continue;
        const float *pr = P + (long)p * ENC_D + h * ENC_DK;
        float acc[QB];
#pragma unroll
        for (int qi = 0; qi < QB; qi++) acc[qi] = 0.0f;
        for (int d = 0; d < ENC_DK; d++) {
            const float pd = pr[d];
#pragma unroll
            for (int qi = 0; qi < QB; qi++) acc[qi] += qv[qi * ENC_DK + d] * pd;
        }
#pragma unroll
        for (int qi = 0; qi < QB; qi++) {
            const int k = p - (T - 1) + q0 + qi;
            if (qi < nq && k >= 0 && k < T) S[qi * T + k] += acc[qi] * sc;
        }
    }
    __syncthreads();
    // softmax per row (backends/cpu/backend.c:67-73)
    const int wv = tid >> 6, lane = tid & 63;
    for (int qi = wv; qi < nq; qi += 4) {
        float *row = S + qi * T;
        float mx = -INFINITY;
        for (int k = lane; k < T; k += 64) mx = fmaxf(mx, row[k]);
        mx = wave_max(mx);
        float sum = 0.0f;
        for (int k = lane; k < T; k += 64) { const float e = expf(row[k] - mx); row[k] = e; sum += e; }
        sum = wave_sum(sum);
        for (int k = lane; k < T; k += 64) row[k] /= sum;
    }
    __syncthreads();
    if (tid < ENC_DK) {
        const int d = tid;
        float acc[QB];
#pragma unroll
        for (int qi = 0; qi < QB; qi++) acc[qi] = 0.0f;
        for (int k = 0; k < T; k++) {
            const float v = V[(long)k * ENC_D + h * ENC_DK + d];
#pragma unroll
            for (int qi = 0; qi < QB; qi++) acc[qi] += S[qi * T + k] * v;
        }
        for (int qi = 0; qi < nq; qi++) O[(long)(q0 + qi) * ENC_D + h * ENC_DK + d] = acc[qi];
    }
}

// ---------------------------------------------------------------------------
// Depthwise conv (k = 9, zero padding 4 inside the sequence) + inference
// BatchNorm + SiLU (backends/cpu/backend.c:312-334).
// ---------------------------------------------------------------------------
__global__ void dwconv_bn_silu_kernel(float *out, uint16_t *out_hi, uint16_t *out_lo,
                                      const float *in, int M, const int *row_start,
                                      const int *row_len, const uint16_t *dww,
                                      const uint16_t *dwb, const uint16_t *bnw, const uint16_t *bnb,
                                      const uint16_t *bnm, const uint16_t *bnv) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)M * ENC_D) return;
    const int r = (int)(i / ENC_D), c = (int)(i % ENC_D);
    const int st = row_start ? row_start[r] : 0;       // this row's sequence: [st, st + T)
    const int T = row_len ? row_len[r] : M;
    const int t = r - st;
    float s = bf2f(dwb[c]);
#pragma unroll
    for (int k = 0; k < ENC_CK; k++) {
        const int ti = t - (ENC_CK - 1) / 2 + k;
        if (ti < 0 || ti >= T) continue;
        s += bf2f(dww[c * ENC_CK + k]) * in[(long)(st + ti) * ENC_D + c];
    }
    const float v = (s - bf2f(bnm[c])) / sqrtf(bf2f(bnv[c]) + 1e-5f) * bf2f(bnw[c]) + bf2f(bnb[c]);
    const float o = v / (1.0f + expf(-v));
    if (out_hi) {
        uint16_t h, l;
        split_bf16(o, h, l);
        out_hi[i] = h;
        out_lo[i] = l;
    } else {
        out[i] = o;
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

static int relpos_qb(int max_T) { return max_T <= 512 ? 16 : 4; }

extern "C" void ctk_relpos_attn(float *O, const float *Q, const float *K, const float *V,
                                const float *P, const uint16_t *pbu, const uint16_t *pbv,
                                int T, hipStream_t s) {
    if (T <= 0) return;
    if (T > 2048) {
        fprintf(stderr, "ctk_relpos_attn: T=%d exceeds the supported 2048 frames\n", T);
        exit(1);
    }
    const int qb = relpos_qb(T);
    const size_t lds = (2 * qb * ENC_DK + qb * (size_t)T) * sizeof(float);
    const dim3 grid((T + qb - 1) / qb, ENC_H);
    if (qb == 16)
        hipLaunchKernelGGL((relpos_attn_kernel<16, false>), grid, dim3(256), lds, s,
                           O, Q, K, V, P, pbu, pbv, T, T, nullptr, nullptr, nullptr, nullptr);
    else
        hipLaunchKernelGGL((relpos_attn_kernel<4, false>), grid, dim3(256), lds, s,
                           O, Q, K, V, P, pbu, pbv, T, T, nullptr, nullptr, nullptr, nullptr);
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

extern "C" void ctk_relpos_attn_packed(float *O, const float *Q, const float *K, const float *V,
                                       const float *P, int T_max, const uint16_t *pbu,
                                       const uint16_t *pbv, const int *seq_off, const int *seq_T,
                                       const int *blk_seq, const int *blk_q0, int n_blk, int max_T,
                                       hipStream_t s) {
    if (n_blk <= 0) return;
    if (max_T > 2048) {
        fprintf(stderr, "ctk_relpos_attn_packed: T=%d exceeds the supported 2048 frames\n", max_T);
        exit(1);
    }
    const int qb = relpos_qb(max_T);
    const size_t lds = (2 * qb * ENC_DK + qb * (size_t)max_T) * sizeof(float);
    const dim3 grid(n_blk, ENC_H);
    if (qb == 16)
        hipLaunchKernelGGL((relpos_attn_kernel<16, true>), grid, dim3(256), lds, s,
                           O, Q, K, V, P, pbu, pbv, 0, T_max, seq_off, seq_T, blk_seq, blk_q0);
    else
        hipLaunchKernelGGL((relpos_attn_kernel<4, true>), grid, dim3(256), lds, s,
                           O, Q, K, V, P, pbu, pbv, 0, T_max, seq_off, seq_T, blk_seq, blk_q0);
}

extern "C" void ctk_dwconv_bn_silu(float *out, const float *in, int T, const uint16_t *dww,
                                   const uint16_t *dwb, const uint16_t *bnw, const uint16_t *bnb,
                                   const uint16_t *bnm, const uint16_t *bnv, hipStream_t s) {
    if (T <= 0) return;
    hipLaunchKernelGGL(dwconv_bn_silu_kernel, dim3(nblk((long)T * ENC_D)), dim3(256), 0, s,
                       out, nullptr, nullptr, in, T, nullptr, nullptr, dww, dwb, bnw, bnb, bnm, bnv);
}

extern "C" void ctk_dwconv_bn_silu_packed(uint16_t *out_hi, uint16_t *out_lo, const float *in, int M,
                                          const int *row_start, const int *row_len,
                                          const uint16_t *dww, const uint16_t *dwb,
                                          const uint16_t *bnw, const uint16_t *bnb,
                                          const uint16_t *bnm, const uint16_t *bnv, hipStream_t s) {
    if (M <= 0) return;
    hipLaunchKernelGGL(dwconv_bn_silu_kernel, dim3(nblk((long)M * ENC_D)), dim3(256), 0, s,
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
