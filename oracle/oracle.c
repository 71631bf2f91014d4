/* oracle.c — CPU fp32 restatement of the reference path (checker only).
 *
 * Test infrastructure: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this.  The HIP backend never calls
 * into it.
 *
 * Restates backends/cpu/backend.c (kernel-boundary functions), model.h
 * (encoder / decoder graph, batch semantics) and transcribe.c:45-214 (mel).
 * Each output element is one sequential fp32 accumulation in the reference's
 * order; OpenMP only distributes independent outputs.
 */
#include "oracle.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

#define EOS_ID 3

static void *xmalloc(size_t n) {
    void *p = malloc(n ? n : 1);
    if (!p) { fputs("oracle: out of memory\n", stderr); exit(1); }
    return p;
}

/* Round-to-nearest-even fp32 -> bf16 -> fp32 (used for the bf16-KV mode). */
static float round_bf16(float x) {
    uint32_t u; memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return x;     /* inf / nan untouched */
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r; memcpy(&r, &u, 4);
    return r;
}

/* In-place rounding of n values (exported for the rounding-mode test). */
void orc_round_bf16_n(float *x, long n) {
    for (long i = 0; i < n; i++) x[i] = round_bf16(x[i]);
}

/* ------------------------------------------------------------------ */
/* Kernel-boundary functions                                           */
/* ------------------------------------------------------------------ */

/* backends/cpu/backend.c:109-122 */
void orc_layernorm(float *dst, const float *src, const uint16_t *w, const uint16_t *b,
                   int T, int D) {
    #pragma omp parallel for if (T >= 16)
    for (int t = 0; t < T; t++) {
        const float *x = src + (size_t)t * D;
        float *y = dst + (size_t)t * D;
        float mu = 0.0f;
        for (int d = 0; d < D; d++) mu += x[d];
        mu /= D;
        float ss = 0.0f;
        for (int d = 0; d < D; d++) { float c = x[d] - mu; ss += c * c; }
        float r = 1.0f / sqrtf(ss / D + 1e-5f);
        for (int d = 0; d < D; d++) y[d] = (x[d] - mu) * r * bf16(w[d]) + bf16(b[d]);
    }
}

/* One output of the linear family: bias first, then k = 0..in_d-1
 * (backends/cpu/backend.c:130-134). */
static inline float dot_bf16(const float *x, const uint16_t *wrow, const uint16_t *b,
                             int j, int in_d) {
    float s = b ? bf16(b[j]) : 0.0f;
    for (int k = 0; k < in_d; k++) s += x[k] * bf16(wrow[k]);
    return s;
}

enum { EPI_NONE, EPI_SILU, EPI_RELU, EPI_FMADD };

static void linear_epi(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                       int T, int in_d, int out_d, int epi, float scale) {
    long work = (long)T * out_d * in_d;
    #pragma omp parallel for collapse(2) if (work > (1L << 20))
    for (int t = 0; t < T; t++)
        for (int j = 0; j < out_d; j++) {
            float s = dot_bf16(x + (size_t)t * in_d, W + (size_t)j * in_d, b, j, in_d);
            float *o = y + (size_t)t * out_d + j;
            switch (epi) {
            case EPI_SILU:  *o = s / (1.0f + expf(-s)); break;   /* cpu:149 */
            case EPI_RELU:  *o = s > 0.0f ? s : 0.0f; break;      /* cpu:164 */
            case EPI_FMADD: *o += scale * s; break;               /* cpu:179 */
            default:        *o = s;
            }
        }
}

/* backends/cpu/backend.c:124-137 */
void orc_linear(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                int T, int in_d, int out_d) {
    linear_epi(y, x, W, b, T, in_d, out_d, EPI_NONE, 0.0f);
}
/* backends/cpu/backend.c:139-152 */
void orc_linear_silu(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                     int T, int in_d, int out_d) {
    linear_epi(y, x, W, b, T, in_d, out_d, EPI_SILU, 0.0f);
}
/* backends/cpu/backend.c:154-167 */
void orc_linear_relu(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                     int T, int in_d, int out_d) {
    linear_epi(y, x, W, b, T, in_d, out_d, EPI_RELU, 0.0f);
}
/* backends/cpu/backend.c:169-182 */
void orc_linear_fmadd(float *acc, float scale, const float *x, const uint16_t *W,
                      const uint16_t *b, int T, int in_d, int out_d) {
    linear_epi(acc, x, W, b, T, in_d, out_d, EPI_FMADD, scale);
}

/* backends/cpu/backend.c:184-186 */
void orc_add_inplace(float *dst, const float *src, int n) {
    for (int i = 0; i < n; i++) dst[i] += src[i];
}

/* Grouped 2-D convolution, zero padding, accumulation order ic, kh, kw after
 * the bias (backends/cpu/backend.c:75-103).  Layouts are [c][h][w]. */
static void conv2d_ref(float *out, const float *in, const uint16_t *Wt, const uint16_t *bias,
                       int in_c, int in_h, int in_w, int out_c, int kh_n, int kw_n,
                       int stride, int pad, int groups) {
    const int oh_n = (in_h + 2 * pad - kh_n) / stride + 1;
    const int ow_n = (in_w + 2 * pad - kw_n) / stride + 1;
    const int icg = in_c / groups, ocg = out_c / groups;
    #pragma omp parallel for collapse(2)
    for (int oc = 0; oc < out_c; oc++)
        for (int oh = 0; oh < oh_n; oh++) {
            const int g = oc / ocg;
            for (int ow = 0; ow < ow_n; ow++) {
                float s = bias ? bf16(bias[oc]) : 0.0f;
                for (int ic = 0; ic < icg; ic++) {
                    const int icl = g * icg + ic;
                    for (int kh = 0; kh < kh_n; kh++) {
                        const int ih = oh * stride - pad + kh;
                        if (ih < 0 || ih >= in_h) continue;
                        for (int kw = 0; kw < kw_n; kw++) {
                            const int iw = ow * stride - pad + kw;
                            if (iw < 0 || iw >= in_w) continue;
                            s += in[(size_t)icl * in_h * in_w + (size_t)ih * in_w + iw]
                               * bf16(Wt[((size_t)oc * icg + ic) * kh_n * kw_n + kh * kw_n + kw]);
                        }
                    }
                }
                out[(size_t)oc * oh_n * ow_n + (size_t)oh * ow_n + ow] = s;
            }
        }
}

static void relu_n(float *x, size_t n) {
    for (size_t i = 0; i < n; i++) if (x[i] < 0.0f) x[i] = 0.0f;
}

size_t orc_subsampling_work_floats(int T_mel) {
    (void)T_mel;
    return 0;    /* the oracle allocates its own buffers */
}

/* backends/cpu/backend.c:188-229: conv(1->256,3x3,s2)+ReLU, dw 3x3 s2, pw+ReLU,
 * dw 3x3 s2, pw+ReLU, flatten (t, ch*16+f), linear 4096->1280. */
void orc_encoder_subsampling(const float *mel, int T_mel, int T_mel_stride,
                             float *x_enc, int T_enc, float *work, const Weights *W) {
    (void)work;
    const int T1 = (T_mel + 1) / 2, T2 = (T1 + 1) / 2;
    float *img = xmalloc((size_t)T_mel * N_MELS * sizeof(float));
    for (int t = 0; t < T_mel; t++)
        for (int m = 0; m < N_MELS; m++)
            img[(size_t)t * N_MELS + m] = mel[(size_t)m * T_mel_stride + t];
    float *a = xmalloc((size_t)SUB_CH * T1 * 64 * sizeof(float));
    float *bb = xmalloc((size_t)SUB_CH * T1 * 64 * sizeof(float));
    conv2d_ref(a, img, W->s0w, W->s0b, 1, T_mel, N_MELS, SUB_CH, 3, 3, 2, 1, 1);
    relu_n(a, (size_t)SUB_CH * T1 * 64);
    conv2d_ref(bb, a, W->s2w, W->s2b, SUB_CH, T1, 64, SUB_CH, 3, 3, 2, 1, SUB_CH);
    conv2d_ref(a, bb, W->s3w, W->s3b, SUB_CH, T2, 32, SUB_CH, 1, 1, 1, 0, 1);
    relu_n(a, (size_t)SUB_CH * T2 * 32);
    conv2d_ref(bb, a, W->s5w, W->s5b, SUB_CH, T2, 32, SUB_CH, 3, 3, 2, 1, SUB_CH);
    conv2d_ref(a, bb, W->s6w, W->s6b, SUB_CH, T_enc, 16, SUB_CH, 1, 1, 1, 0, 1);
    relu_n(a, (size_t)SUB_CH * T_enc * 16);
    float *flat = xmalloc((size_t)T_enc * SUB_CH * 16 * sizeof(float));
    for (int t = 0; t < T_enc; t++)
        for (int c = 0; c < SUB_CH; c++)
            for (int f = 0; f < 16; f++)
                flat[(size_t)t * SUB_CH * 16 + c * 16 + f] = a[(size_t)c * T_enc * 16 + t * 16 + f];
    orc_linear(x_enc, flat, W->sow, W->sob, T_enc, SUB_CH * 16, ENC_D);
    free(img); free(a); free(bb); free(flat);
}

/* backends/cpu/backend.c:231-242; same fp32 expression order. */
void orc_make_rel_pos_emb(float *pe, int T) {
    const int L = 2 * T - 1;
    const float ln1e4 = logf(10000.0f);
    for (int p = 0; p < L; p++) {
        const float pos = (float)(T - 1 - p);
        for (int k = 0; k < ENC_D / 2; k++) {
            const float dt = expf(-(float)(2 * k) * ln1e4 / ENC_D);
            pe[(size_t)p * ENC_D + 2 * k]     = sinf(pos * dt);
            pe[(size_t)p * ENC_D + 2 * k + 1] = cosf(pos * dt);
        }
    }
}

/* backends/cpu/backend.c:67-73 */
static void softmax_row(float *x, int n) {
    float m = x[0];
    for (int i = 1; i < n; i++) if (x[i] > m) m = x[i];
    float s = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - m); s += x[i]; }
    for (int i = 0; i < n; i++) x[i] /= s;
}

size_t orc_mhsa_work_floats(int T) { (void)T; return 0; }

/* backends/cpu/backend.c:244-298: Transformer-XL style relative-position
 * attention.  score(q,k) = ((Q_q+u).K_k)*s + ((Q_q+v).P_{k+T-1-q})*s,
 * s = 1/sqrt(160); softmax over k; P = pos_emb Wp^T (no bias). */
void orc_rel_pos_mhsa(float *x, const float *pos_emb, int T, const ELayer *L, float *work) {
    (void)work;
    const int PL = 2 * T - 1;
    float *Q = xmalloc((size_t)T * ENC_D * sizeof(float));
    float *K = xmalloc((size_t)T * ENC_D * sizeof(float));
    float *V = xmalloc((size_t)T * ENC_D * sizeof(float));
    float *P = xmalloc((size_t)PL * ENC_D * sizeof(float));
    float *O = xmalloc((size_t)T * ENC_D * sizeof(float));
    orc_linear(Q, x, L->sa_qw, L->sa_qb, T, ENC_D, ENC_D);
    orc_linear(K, x, L->sa_kw, L->sa_kb, T, ENC_D, ENC_D);
    orc_linear(V, x, L->sa_vw, L->sa_vb, T, ENC_D, ENC_D);
    orc_linear(P, pos_emb, L->sa_pw, NULL, PL, ENC_D, ENC_D);
    const float sc = 1.0f / sqrtf((float)ENC_DK);
    #pragma omp parallel for collapse(2)
    for (int h = 0; h < ENC_H; h++)
        for (int q = 0; q < T; q++) {
            float *row = xmalloc((size_t)T * sizeof(float));
            const int o = h * ENC_DK;
            for (int k = 0; k < T; k++) {
                float ac = 0.0f;
                for (int d = 0; d < ENC_DK; d++)
                    ac += (Q[(size_t)q * ENC_D + o + d] + bf16(L->sa_pbu[o + d]))
                        * K[(size_t)k * ENC_D + o + d];
                row[k] = ac * sc;
            }
            for (int k = 0; k < T; k++) {
                const int p = k + T - 1 - q;
                float bd = 0.0f;
                for (int d = 0; d < ENC_DK; d++)
                    bd += (Q[(size_t)q * ENC_D + o + d] + bf16(L->sa_pbv[o + d]))
                        * P[(size_t)p * ENC_D + o + d];
                row[k] += bd * sc;
            }
            softmax_row(row, T);
            for (int d = 0; d < ENC_DK; d++) {
                float s = 0.0f;
                for (int k = 0; k < T; k++) s += row[k] * V[(size_t)k * ENC_D + o + d];
                O[(size_t)q * ENC_D + o + d] = s;
            }
            free(row);
        }
    orc_linear(x, O, L->sa_ow, L->sa_ob, T, ENC_D, ENC_D);
    free(Q); free(K); free(V); free(P); free(O);
}

size_t orc_conv_work_floats(int T) { (void)T; return 0; }

/* backends/cpu/backend.c:300-337: pw1 (1280->2560) -> GLU a*sigmoid(b) ->
 * depthwise k=9 zero-padded inside the sequence -> BN(running stats) -> SiLU
 * -> pw2 (1280->1280).  x updated in place. */
void orc_conformer_conv(float *x, int T, const ELayer *L, float *work) {
    (void)work;
    float *pw = xmalloc((size_t)T * 2 * ENC_D * sizeof(float));
    float *g = xmalloc((size_t)T * ENC_D * sizeof(float));
    float *dw = xmalloc((size_t)T * ENC_D * sizeof(float));
    orc_linear(pw, x, L->cv_pw1w, L->cv_pw1b, T, ENC_D, 2 * ENC_D);
    for (int t = 0; t < T; t++)
        for (int c = 0; c < ENC_D; c++) {
            const float a = pw[(size_t)t * 2 * ENC_D + c];
            const float z = pw[(size_t)t * 2 * ENC_D + c + ENC_D];
            g[(size_t)t * ENC_D + c] = a / (1.0f + expf(-z));
        }
    const int half = (ENC_CK - 1) / 2;
    for (int t = 0; t < T; t++)
        for (int c = 0; c < ENC_D; c++) {
            float s = bf16(L->cv_dwb[c]);
            for (int k = 0; k < ENC_CK; k++) {
                const int ti = t - half + k;
                if (ti < 0 || ti >= T) continue;
                s += bf16(L->cv_dww[c * ENC_CK + k]) * g[(size_t)ti * ENC_D + c];
            }
            float v = (s - bf16(L->cv_bnmean[c])) / sqrtf(bf16(L->cv_bnvar[c]) + 1e-5f)
                    * bf16(L->cv_bnw[c]) + bf16(L->cv_bnb[c]);
            dw[(size_t)t * ENC_D + c] = v / (1.0f + expf(-v));
        }
    orc_linear(x, dw, L->cv_pw2w, L->cv_pw2b, T, ENC_D, ENC_D);
    free(pw); free(g); free(dw);
}

/* backends/cpu/backend.c:339-360: per head, scores*1/sqrt(128) + mask,
 * softmax, weighted sum of V.  Rows are DEC_D wide, head h at h*DEC_DK. */
void orc_sdp_attn(float *out, const float *q, const float *k, const float *v,
                  const float *mask, int T_q, int T_k, float *work) {
    (void)work;
    const float sc = 1.0f / sqrtf((float)DEC_DK);
    #pragma omp parallel for collapse(2) if ((long)T_q * T_k > 4096)
    for (int h = 0; h < DEC_H; h++)
        for (int qi = 0; qi < T_q; qi++) {
            float *row = xmalloc((size_t)T_k * sizeof(float));
            const int o = h * DEC_DK;
            for (int ki = 0; ki < T_k; ki++) {
                float s = 0.0f;
                for (int d = 0; d < DEC_DK; d++)
                    s += q[(size_t)qi * DEC_D + o + d] * k[(size_t)ki * DEC_D + o + d];
                row[ki] = s * sc + (mask ? mask[(size_t)qi * T_k + ki] : 0.0f);
            }
            softmax_row(row, T_k);
            for (int d = 0; d < DEC_DK; d++) {
                float s = 0.0f;
                for (int ki = 0; ki < T_k; ki++) s += row[ki] * v[(size_t)ki * DEC_D + o + d];
                out[(size_t)qi * DEC_D + o + d] = s;
            }
            free(row);
        }
}

/* backends/cpu/backend.c:362-371 */
void orc_embed(float *h, const int *tokens, int S, int pos_start,
               const uint16_t *etw, const uint16_t *epw,
               const uint16_t *elnw, const uint16_t *elnb) {
    for (int t = 0; t < S; t++)
        for (int d = 0; d < DEC_D; d++)
            h[(size_t)t * DEC_D + d] = bf16(etw[(size_t)tokens[t] * DEC_D + d])
                                     + bf16(epw[(size_t)(pos_start + t) * DEC_D + d]);
    orc_layernorm(h, h, elnw, elnb, S, DEC_D);
}

/* backends/cpu/backend.c:373-377 */
void orc_fill_causal_mask(float *mask, int S) {
    for (int i = 0; i < S; i++)
        for (int j = 0; j < S; j++)
            mask[(size_t)i * S + j] = (j > i) ? -1e9f : 0.0f;
}

/* backends/cpu/backend.c:379-387 */
void orc_lm_head(float *logits, const float *last, const uint16_t *etw, const uint16_t *hdb) {
    #pragma omp parallel for
    for (int v = 0; v < VOCAB; v++) {
        float s = bf16(hdb[v]);
        const uint16_t *e = etw + (size_t)v * DEC_D;
        for (int d = 0; d < DEC_D; d++) s += last[d] * bf16(e[d]);
        logits[v] = s;
    }
}

/* backends/cpu/backend.c:446-456 (strict '>', first maximum wins). */
int orc_argmax(const float *x, int n, int skip) {
    int best = (skip == 0) ? 1 : 0;
    float bv = x[best];
    for (int i = best + 1; i < n; i++) {
        if (i == skip) continue;
        if (x[i] > bv) { bv = x[i]; best = i; }
    }
    return best;
}

/* ------------------------------------------------------------------ */
/* Graph level                                                         */
/* ------------------------------------------------------------------ */

/* transcribe.c:268-271 */
int orc_T_enc(int T_mel) {
    const int t1 = (T_mel + 1) / 2, t2 = (t1 + 1) / 2;
    return (t2 + 1) / 2;
}
int orc_T_mel(int n_samples) { return 1 + n_samples / HOP_LEN; }

/* Single-pass precision mode of the encoder FFN projections: the inputs of
 * both FFN linears (the LayerNorm output and the SiLU output) are rounded to
 * bf16 before the fp32 dot products.  Off by default (the reference's fp32
 * arithmetic); not part of the reference. */
static int g_enc_ffn_bf16 = 0;
void orc_set_enc_ffn_bf16(int on) { g_enc_ffn_bf16 = on != 0; }

static void ffn_half(float *x, float *ln, float *mid, int T, const uint16_t *lnw,
                     const uint16_t *lnb, const uint16_t *w1, const uint16_t *b1,
                     const uint16_t *w2, const uint16_t *b2) {
    orc_layernorm(ln, x, lnw, lnb, T, ENC_D);
    if (g_enc_ffn_bf16) orc_round_bf16_n(ln, (long)T * ENC_D);
    orc_linear_silu(mid, ln, w1, b1, T, ENC_D, ENC_FF);
    if (g_enc_ffn_bf16) orc_round_bf16_n(mid, (long)T * ENC_FF);
    orc_linear_fmadd(x, 0.5f, mid, w2, b2, T, ENC_FF, ENC_D);
}

/* model.h:276-314: FFN/2, MHSA, conv module, FFN/2, final LN. */
void orc_conformer_layer(float *x, const float *pos_emb, int T, const ELayer *L, float *work) {
    (void)work;
    float *ln = xmalloc((size_t)T * ENC_D * sizeof(float));
    float *mid = xmalloc((size_t)T * ENC_FF * sizeof(float));
    ffn_half(x, ln, mid, T, L->ff1_lnw, L->ff1_lnb, L->ff1_w1, L->ff1_b1, L->ff1_w2, L->ff1_b2);

    orc_layernorm(ln, x, L->sa_lnw, L->sa_lnb, T, ENC_D);
    orc_rel_pos_mhsa(ln, pos_emb, T, L, NULL);
    orc_add_inplace(x, ln, T * ENC_D);

    orc_layernorm(ln, x, L->cv_lnw, L->cv_lnb, T, ENC_D);
    orc_conformer_conv(ln, T, L, NULL);
    orc_add_inplace(x, ln, T * ENC_D);

    ffn_half(x, ln, mid, T, L->ff2_lnw, L->ff2_lnb, L->ff2_w1, L->ff2_b1, L->ff2_w2, L->ff2_b2);

    orc_layernorm(x, x, L->out_lnw, L->out_lnb, T, ENC_D);
    free(ln); free(mid);
}

/* model.h:319-344 (single item) and 573-609 (batch item: same per-item math,
 * pos_emb shifted from the T_max table; identical values). */
void orc_encoder_forward(const float *mel, int T_mel, int T_mel_stride,
                         const Weights *W, float *x_enc_out, float *enc_h) {
    const int T = orc_T_enc(T_mel);
    float *x = x_enc_out ? x_enc_out : xmalloc((size_t)T * ENC_D * sizeof(float));
    float *pe = xmalloc((size_t)(2 * T - 1) * ENC_D * sizeof(float));
    orc_encoder_subsampling(mel, T_mel, T_mel_stride, x, T, NULL, W);
    orc_make_rel_pos_emb(pe, T);
    for (int l = 0; l < ENC_N; l++) orc_conformer_layer(x, pe, T, &W->enc[l], NULL);
    orc_linear(enc_h, x, W->prw, W->prb, T, ENC_D, DEC_D);
    free(pe);
    if (!x_enc_out) free(x);
}

/* model.h:349-364 / 620-635 */
void orc_cross_kv(const float *enc_h, int T_enc, const Weights *W, float *ca_k, float *ca_v) {
    for (int l = 0; l < DEC_N; l++) {
        orc_linear(ca_k + (size_t)l * T_enc * DEC_D, enc_h, W->dec[l].ca_kw, W->dec[l].ca_kb,
                   T_enc, DEC_D, DEC_D);
        orc_linear(ca_v + (size_t)l * T_enc * DEC_D, enc_h, W->dec[l].ca_vw, W->dec[l].ca_vb,
                   T_enc, DEC_D, DEC_D);
    }
}

void orc_seq_init(OrcSeq *s, const float *ca_k, const float *ca_v, int T_enc, int kv_bf16) {
    const size_t n = (size_t)DEC_N * MAX_SEQ * DEC_D;
    s->sk = xmalloc(n * sizeof(float));
    s->sv = xmalloc(n * sizeof(float));
    s->T_enc = T_enc;
    s->S = 0;
    s->kv_bf16 = kv_bf16;
    if (kv_bf16) {
        const size_t m = (size_t)DEC_N * T_enc * DEC_D;
        float *k = xmalloc(m * sizeof(float)), *v = xmalloc(m * sizeof(float));
        for (size_t i = 0; i < m; i++) { k[i] = round_bf16(ca_k[i]); v[i] = round_bf16(ca_v[i]); }
        s->ck = k; s->cv = v;
    } else {
        s->ck = ca_k; s->cv = ca_v;
    }
}

void orc_seq_free(OrcSeq *s) {
    free(s->sk); free(s->sv);
    if (s->kv_bf16) { free((void *)s->ck); free((void *)s->cv); }
    memset(s, 0, sizeof *s);
}

/* model.h:376-409 (decoder_layer) + 461-503 (decoder_step), generalised to
 * n new rows appended after s->S cached ones (causal mask over the new
 * rows only, -1e9 as backends/cpu/backend.c:373-377). */
void orc_seq_step(OrcSeq *s, const Weights *W, const int *tokens, int n,
                  float *logits, float *h_last) {
    const int S0 = s->S, S1 = S0 + n;
    if (S1 > MAX_SEQ) { fputs("oracle: sequence exceeds MAX_SEQ\n", stderr); exit(1); }
    float *h = xmalloc((size_t)n * DEC_D * sizeof(float));
    float *ln = xmalloc((size_t)n * DEC_D * sizeof(float));
    float *q = xmalloc((size_t)n * DEC_D * sizeof(float));
    float *at = xmalloc((size_t)n * DEC_D * sizeof(float));
    float *mid = xmalloc((size_t)n * DEC_FF * sizeof(float));
    float *mask = NULL;
    if (n > 1) {
        mask = xmalloc((size_t)n * S1 * sizeof(float));
        for (int i = 0; i < n; i++)
            for (int j = 0; j < S1; j++)
                mask[(size_t)i * S1 + j] = (j > S0 + i) ? -1e9f : 0.0f;
    }
    orc_embed(h, tokens, n, S0, W->etw, W->epw, W->elnw, W->elnb);
    for (int l = 0; l < DEC_N; l++) {
        const DLayer *L = &W->dec[l];
        float *kc = s->sk + (size_t)l * MAX_SEQ * DEC_D;
        float *vc = s->sv + (size_t)l * MAX_SEQ * DEC_D;
        orc_layernorm(ln, h, L->sa_lnw, L->sa_lnb, n, DEC_D);
        orc_linear(q, ln, L->sa_qw, L->sa_qb, n, DEC_D, DEC_D);
        orc_linear(kc + (size_t)S0 * DEC_D, ln, L->sa_kw, L->sa_kb, n, DEC_D, DEC_D);
        orc_linear(vc + (size_t)S0 * DEC_D, ln, L->sa_vw, L->sa_vb, n, DEC_D, DEC_D);
        if (s->kv_bf16)
            for (size_t i = (size_t)S0 * DEC_D; i < (size_t)S1 * DEC_D; i++) {
                kc[i] = round_bf16(kc[i]); vc[i] = round_bf16(vc[i]);
            }
        orc_sdp_attn(at, q, kc, vc, mask, n, S1, NULL);
        orc_linear_fmadd(h, 1.0f, at, L->sa_ow, L->sa_ob, n, DEC_D, DEC_D);

        orc_layernorm(ln, h, L->ca_lnw, L->ca_lnb, n, DEC_D);
        orc_linear(q, ln, L->ca_qw, L->ca_qb, n, DEC_D, DEC_D);
        orc_sdp_attn(at, q, s->ck + (size_t)l * s->T_enc * DEC_D,
                     s->cv + (size_t)l * s->T_enc * DEC_D, NULL, n, s->T_enc, NULL);
        orc_linear_fmadd(h, 1.0f, at, L->ca_ow, L->ca_ob, n, DEC_D, DEC_D);

        orc_layernorm(ln, h, L->ffn_lnw, L->ffn_lnb, n, DEC_D);
        orc_linear_relu(mid, ln, L->ffn_w1, L->ffn_b1, n, DEC_D, DEC_FF);
        orc_linear_fmadd(h, 1.0f, mid, L->ffn_w2, L->ffn_b2, n, DEC_FF, DEC_D);
    }
    float *last = h + (size_t)(n - 1) * DEC_D;
    orc_layernorm(last, last, W->dlnw, W->dlnb, 1, DEC_D);
    if (h_last) memcpy(h_last, last, DEC_D * sizeof(float));
    if (logits) orc_lm_head(logits, last, W->etw, W->hdb);
    s->S = S1;
    free(h); free(ln); free(q); free(at); free(mid); free(mask);
}

/* transcribe.c:264-390 (single) and 572-808 (batch: per item identical). */
int orc_transcribe(const Weights *W, const float *mel, int T_mel, int T_mel_stride,
                   const int *prompt, int n_prompt, int limit,
                   int suppress_eos, int force_eos, int kv_bf16,
                   int *tokens_out, float *logits_out, float *enc_h_out) {
    const int T = orc_T_enc(T_mel);
    float *eh = enc_h_out ? enc_h_out : xmalloc((size_t)T * DEC_D * sizeof(float));
    orc_encoder_forward(mel, T_mel, T_mel_stride, W, NULL, eh);
    const size_t m = (size_t)DEC_N * T * DEC_D;
    float *ck = xmalloc(m * sizeof(float)), *cv = xmalloc(m * sizeof(float));
    orc_cross_kv(eh, T, W, ck, cv);
    OrcSeq s;
    orc_seq_init(&s, ck, cv, T, kv_bf16);
    float *lg = xmalloc(VOCAB * sizeof(float));
    orc_seq_step(&s, W, prompt, n_prompt, lg, NULL);
    int ng = 0;
    for (;;) {
        int tok;
        if (force_eos && ng == limit - 1) tok = EOS_ID;
        else tok = orc_argmax(lg, VOCAB, suppress_eos ? EOS_ID : -1);
        if (logits_out) memcpy(logits_out + (size_t)ng * VOCAB, lg, VOCAB * sizeof(float));
        tokens_out[ng++] = tok;
        if (tok == EOS_ID && !suppress_eos) break;
        if (ng >= limit || s.S >= MAX_SEQ) break;
        orc_seq_step(&s, W, &tok, 1, lg, NULL);
    }
    orc_seq_free(&s);
    free(lg); free(ck); free(cv);
    if (!enc_h_out) free(eh);
    return ng;
}

/* ------------------------------------------------------------------ */
/* Log-mel front-end (transcribe.c:45-214)                             */
/* ------------------------------------------------------------------ */

static double slaney_hz_to_mel(double f) {
    const double fsp = 200.0 / 3.0, brk = 1000.0, brk_mel = brk / fsp;
    const double step = log(6.4) / 27.0;
    return f < brk ? f / fsp : brk_mel + log(f / brk) / step;
}
static double slaney_mel_to_hz(double m) {
    const double fsp = 200.0 / 3.0, brk = 1000.0, brk_mel = brk / fsp;
    const double step = log(6.4) / 27.0;
    return m < brk_mel ? fsp * m : brk * exp(step * (m - brk_mel));
}

/* transcribe.c:51-93: Slaney-normalised triangular filters, 0-8 kHz. */
void orc_mel_filterbank(float *fb) {
    double hz[N_MELS + 2], gap[N_MELS + 1];
    const double lo = slaney_hz_to_mel(0.0), hi = slaney_hz_to_mel(SR / 2.0);
    for (int i = 0; i < N_MELS + 2; i++) hz[i] = slaney_mel_to_hz(lo + (hi - lo) * i / (N_MELS + 1));
    for (int i = 0; i < N_MELS + 1; i++) gap[i] = hz[i + 1] - hz[i];
    for (int m = 0; m < N_MELS; m++) {
        const double norm = 2.0 / (hz[m + 2] - hz[m]);
        for (int i = 0; i < N_BINS; i++) {
            const double f = (SR / 2.0) * i / (N_BINS - 1);
            const double up = (f - hz[m]) / gap[m];
            const double dn = (hz[m + 2] - f) / gap[m + 1];
            const double w = up < dn ? up : dn;
            fb[m * N_BINS + i] = (float)(w > 0.0 ? w * norm : 0.0);
        }
    }
}

/* transcribe.c:95-122: in-place iterative radix-2 FFT with a rotated
 * twiddle per butterfly group. */
static void fft512(float *re, float *im) {
    const int n = N_FFT;
    for (int i = 1, j = 0; i < n; i++) {
        int bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) {
            float t = re[i]; re[i] = re[j]; re[j] = t;
            t = im[i]; im[i] = im[j]; im[j] = t;
        }
    }
    for (int len = 2; len <= n; len <<= 1) {
        const float ang = -2.0f * (float)M_PI / len;
        const float wr = cosf(ang), wi = sinf(ang);
        const int half = len / 2;
        for (int i = 0; i < n; i += len) {
            float cr = 1.0f, ci = 0.0f;
            for (int k = 0; k < half; k++) {
                const float ur = re[i + k], ui = im[i + k];
                const float vr = re[i + k + half] * cr - im[i + k + half] * ci;
                const float vi = re[i + k + half] * ci + im[i + k + half] * cr;
                re[i + k] = ur + vr; im[i + k] = ui + vi;
                re[i + k + half] = ur - vr; im[i + k + half] = ui - vi;
                const float nc = cr * wr - ci * wi;
                ci = cr * wi + ci * wr;
                cr = nc;
            }
        }
    }
}

/* transcribe.c:177-214: zero-pad 200 each side, pre-emphasis 0.97, Hann(400)
 * frames every 160 samples into a 512-point FFT, power, mel, log(x+2^-24),
 * per-bin mean/std normalisation with var/(T-1). */
void orc_compute_mel(const float *samples, int n, float *mel) {
    const int T = orc_T_mel(n);
    const int pad = WIN_LEN / 2, np = n + 2 * pad;
    float *s = calloc((size_t)np, sizeof(float));
    float *fb = xmalloc((size_t)N_MELS * N_BINS * sizeof(float));
    float win[WIN_LEN];
    if (!s) { fputs("oracle: out of memory\n", stderr); exit(1); }
    memcpy(s + pad, samples, (size_t)n * sizeof(float));
    for (int i = np - 1; i > 0; i--) s[i] -= 0.97f * s[i - 1];
    for (int i = 0; i < WIN_LEN; i++)
        win[i] = 0.5f * (1.0f - cosf(2.0f * (float)M_PI * i / (WIN_LEN - 1)));
    orc_mel_filterbank(fb);
    #pragma omp parallel for
    for (int t = 0; t < T; t++) {
        float re[N_FFT], im[N_FFT], ps[N_BINS];
        const int off = t * HOP_LEN;
        for (int i = 0; i < N_FFT; i++) re[i] = im[i] = 0.0f;
        for (int i = 0; i < WIN_LEN && off + i < np; i++) re[i] = s[off + i] * win[i];
        fft512(re, im);
        for (int i = 0; i < N_BINS; i++) ps[i] = re[i] * re[i] + im[i] * im[i];
        for (int m = 0; m < N_MELS; m++) {
            float acc = 0.0f;
            for (int i = 0; i < N_BINS; i++) acc += fb[m * N_BINS + i] * ps[i];
            mel[(size_t)m * T + t] = acc;
        }
    }
    const float guard = powf(2.0f, -24.0f);
    for (int m = 0; m < N_MELS; m++) {
        float *row = mel + (size_t)m * T;
        float mu = 0.0f, var = 0.0f;
        for (int t = 0; t < T; t++) { row[t] = logf(row[t] + guard); mu += row[t]; }
        mu /= T;
        for (int t = 0; t < T; t++) { const float d = row[t] - mu; var += d * d; }
        var /= (T - 1);
        const float r = 1.0f / sqrtf(var + 1e-5f);
        for (int t = 0; t < T; t++) row[t] = (row[t] - mu) * r;
    }
    free(s); free(fb);
}

/* ------------------------------------------------------------------ */
/* Long-audio chunking                                                 */
/* ------------------------------------------------------------------ */

/* transcribe.c:397-404: RMS of each 10 ms frame, one sequential fp32 sum of
 * squares (the reference's -O3 -march=native build contracts it to FMA). */
static void orc_frame_rms(const float *x, int n_frames, float *rms) {
    for (int f = 0; f < n_frames; f++) {
        float sum = 0.0f;
        for (int i = 0; i < HOP_LEN; i++) sum = fmaf(x[f * HOP_LEN + i], x[f * HOP_LEN + i], sum);
        rms[f] = sqrtf(sum / HOP_LEN);
    }
}

/* transcribe.c:406-421: histogram of RMS in 1024 buckets of width 1/1024;
 * the first bucket b at which the cumulative count reaches n_frames/20 gives
 * the threshold (b/1024)*10 (+20 dB). */
static float orc_auto_threshold(const float *rms, int n_frames) {
    int *hist = calloc(1024, sizeof(int));
    for (int f = 0; f < n_frames; f++) {
        int b = (int)(rms[f] * 1024);
        if (b > 1023) b = 1023;
        hist[b]++;
    }
    const int target = n_frames / 20;
    float t = 1.0f;
    int cum = 0;
    for (int b = 0; b < 1024; b++) {
        cum += hist[b];
        if (cum >= target) { t = ((float)b / 1024) * 10.0f; break; }
    }
    free(hist);
    return t;
}

/* transcribe.c:429-446: a quiet run [s, f) of at least
 * (int)(dur*SR/HOP_LEN) frames that is followed by a loud frame f yields the
 * cut ((s + f)/2)*HOP_LEN; a run reaching the end yields nothing. */
static int orc_find_cuts(const float *rms, int n_frames, float thresh, float dur, int *cuts, int cap) {
    const int min_frames = (int)(dur * SR / HOP_LEN);
    int n = 0, quiet = 0, s = 0;
    for (int f = 0; f < n_frames; f++) {
        if (rms[f] < thresh) {
            if (!quiet) { quiet = 1; s = f; }
        } else if (quiet) {
            if (f - s >= min_frames && n < cap) cuts[n++] = ((s + f) / 2) * HOP_LEN;
            quiet = 0;
        }
    }
    return n;
}

/* transcribe.c:456-465: keep cut i when it lies at least target_samp samples
 * after the previously kept cut (the start counts as kept at 0). */
static int orc_keep_cuts(int *cuts, int n, int target_samp) {
    int kept = 0, prev = 0;
    for (int i = 0; i < n; i++)
        if (cuts[i] - prev >= target_samp) { prev = cuts[i]; cuts[kept++] = prev; }
    return kept;
}

/* transcribe.c:486-533: threshold (auto, or 10^(dB/20)), cuts, targets,
 * then the chunks between consecutive cuts, skipping empty ones. */
int orc_chunk_bounds(const float *samples, int n_samples, float silence_db, float silence_dur,
                     float target_sec, int *bounds, int cap) {
    const int n_frames = n_samples / HOP_LEN;
    float *rms = xmalloc((size_t)n_frames * sizeof(float));
    orc_frame_rms(samples, n_frames, rms);
    const float thresh = isnan(silence_db) ? orc_auto_threshold(rms, n_frames)
                                           : powf(10.0f, silence_db / 20.0f);
    int *cuts = xmalloc(4096 * sizeof(int));
    int n = orc_find_cuts(rms, n_frames, thresh, silence_dur, cuts, 4096);
    free(rms);
    n = orc_keep_cuts(cuts, n, (int)(target_sec * SR));
    int nb = 0, start = 0;
    for (int c = 0; c <= n; c++) {
        const int end = c < n ? cuts[c] : n_samples;
        if (end <= start) { start = end; continue; }
        if (nb < cap) { bounds[2 * nb] = start; bounds[2 * nb + 1] = end; nb++; }
        start = end;
    }
    free(cuts);
    return nb;
}
