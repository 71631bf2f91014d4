/* synth.c — seeded synthetic weights and audio (see synth.h).
 *
 * Tensor names, shapes and the on-disk order follow the reference converter:
 * names convert.py:61-154, access order convert.py:161-190 (subsampling,
 * encoder layers field by field, projection, all cross-attention K/V, decoder
 * embedding, decoder layers, final norm + head bias), compact JSON header
 * convert.py:217 padded with spaces to a multiple of 8 (convert.py:219-220).
 * The tied LM-head weight that the host never loads (model.h:224) is not
 * emitted.
 */
#include "synth.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <pthread.h>
#include <unistd.h>

/* ---------------- counter-based generator ---------------- */

/* splitmix64 finaliser (Steele, Lea, Flood 2014). */
static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
uint64_t ct_hash64(uint64_t key, uint64_t i) {
    return mix64(key + 0x9E3779B97F4A7C15ULL * (i + 1));
}

/* Inverse standard-normal CDF: Acklam's rational approximation refined by one
 * Halley step on erfc (relative error far below bf16 resolution). */
static double inv_norm(double p) {
    static const double a[6] = {-3.969683028665376e+01, 2.209460984245205e+02,
        -2.759285104469687e+02, 1.383577518672690e+02, -3.066479806614716e+01,
        2.506628277459239e+00};
    static const double b[5] = {-5.447609879822406e+01, 1.615858368580409e+02,
        -1.556989798598866e+02, 6.680131188771972e+01, -1.328068155288572e+01};
    static const double c[6] = {-7.784894002430293e-03, -3.223964580411365e-01,
        -2.400758277161838e+00, -2.549732539343734e+00, 4.374664141464968e+00,
        2.938163982698783e+00};
    static const double d[4] = {7.784695709041462e-03, 3.224671290700398e-01,
        2.445134137142996e+00, 3.754408661907416e+00};
    const double lo = 0.02425;
    double x;
    if (p < lo) {
        const double q = sqrt(-2.0 * log(p));
        x = (((((c[0]*q + c[1])*q + c[2])*q + c[3])*q + c[4])*q + c[5]) /
            ((((d[0]*q + d[1])*q + d[2])*q + d[3])*q + 1.0);
    } else if (p <= 1.0 - lo) {
        const double q = p - 0.5, r = q * q;
        x = (((((a[0]*r + a[1])*r + a[2])*r + a[3])*r + a[4])*r + a[5]) * q /
            (((((b[0]*r + b[1])*r + b[2])*r + b[3])*r + b[4])*r + 1.0);
    } else {
        const double q = sqrt(-2.0 * log(1.0 - p));
        x = -(((((c[0]*q + c[1])*q + c[2])*q + c[3])*q + c[4])*q + c[5]) /
             ((((d[0]*q + d[1])*q + d[2])*q + d[3])*q + 1.0);
    }
    const double e = 0.5 * erfc(-x / sqrt(2.0)) - p;
    const double u = e * sqrt(2.0 * M_PI) * exp(x * x / 2.0);
    return x - u / (1.0 + x * u / 2.0);
}

/* 65536 equiprobable quantiles of N(0,1). */
static float g_qtab[65536];
static pthread_once_t g_qonce = PTHREAD_ONCE_INIT;
static void qtab_init(void) {
    for (int i = 0; i < 65536; i++) g_qtab[i] = (float)inv_norm((i + 0.5) / 65536.0);
}
float ct_normal16(uint64_t h) {
    pthread_once(&g_qonce, qtab_init);
    return g_qtab[h >> 48];
}

static inline uint16_t to_bf16_rne(float x) {
    uint32_t u; memcpy(&u, &x, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* ---------------- tensor table ---------------- */

enum { K_NORMAL, K_ONES, K_ZEROS, K_BIAS, K_GAIN, K_VAR };
/* K_BIAS/K_GAIN/K_VAR are zeros/ones/ones in the spec variant and perturbed in
 * the perturbed variant. */

typedef struct {
    char name[96];
    int kind;
    int nd;
    int shape[3];
    size_t elems;
    size_t off;           /* byte offset inside the data section */
} TInfo;

#define MAX_T 2200
static TInfo g_tab[MAX_T];
static int g_nt = 0;
static size_t g_data_bytes = 0;
static pthread_once_t g_tonce = PTHREAD_ONCE_INIT;

static void add_t(const char *name, int kind, int nd, int s0, int s1, int s2) {
    TInfo *t = &g_tab[g_nt++];
    snprintf(t->name, sizeof t->name, "%s", name);
    t->kind = kind; t->nd = nd;
    t->shape[0] = s0; t->shape[1] = s1; t->shape[2] = s2;
    t->elems = (size_t)s0 * (nd > 1 ? s1 : 1) * (nd > 2 ? s2 : 1);
    t->off = g_data_bytes;
    g_data_bytes += t->elems * 2;
}

static const char *ENC_PFX = "encoder.layers.";
static const char *DEC_PFX = "transf_decoder._decoder.layers.";

static void add_enc_layer(int i) {
    char n[96];
#define E(sfx, kind, nd, a, b, c) do { snprintf(n, sizeof n, "%s%d.%s", ENC_PFX, i, sfx); \
    add_t(n, kind, nd, a, b, c); } while (0)
    E("norm_feed_forward1.weight", K_GAIN, 1, ENC_D, 0, 0);
    E("norm_feed_forward1.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("feed_forward1.linear1.weight", K_NORMAL, 2, ENC_FF, ENC_D, 0);
    E("feed_forward1.linear1.bias", K_BIAS, 1, ENC_FF, 0, 0);
    E("feed_forward1.linear2.weight", K_NORMAL, 2, ENC_D, ENC_FF, 0);
    E("feed_forward1.linear2.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("norm_self_att.weight", K_GAIN, 1, ENC_D, 0, 0);
    E("norm_self_att.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("self_attn.linear_q.weight", K_NORMAL, 2, ENC_D, ENC_D, 0);
    E("self_attn.linear_q.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("self_attn.linear_k.weight", K_NORMAL, 2, ENC_D, ENC_D, 0);
    E("self_attn.linear_k.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("self_attn.linear_v.weight", K_NORMAL, 2, ENC_D, ENC_D, 0);
    E("self_attn.linear_v.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("self_attn.linear_pos.weight", K_NORMAL, 2, ENC_D, ENC_D, 0);
    E("self_attn.pos_bias_u", K_NORMAL, 2, ENC_H, ENC_DK, 0);
    E("self_attn.pos_bias_v", K_NORMAL, 2, ENC_H, ENC_DK, 0);
    E("self_attn.linear_out.weight", K_NORMAL, 2, ENC_D, ENC_D, 0);
    E("self_attn.linear_out.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("norm_conv.weight", K_GAIN, 1, ENC_D, 0, 0);
    E("norm_conv.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("conv.pointwise_conv1.weight", K_NORMAL, 3, 2 * ENC_D, ENC_D, 1);
    E("conv.pointwise_conv1.bias", K_BIAS, 1, 2 * ENC_D, 0, 0);
    E("conv.depthwise_conv.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("conv.depthwise_conv.weight", K_NORMAL, 3, ENC_D, 1, ENC_CK);
    E("conv.batch_norm.running_mean", K_BIAS, 1, ENC_D, 0, 0);
    E("conv.batch_norm.running_var", K_VAR, 1, ENC_D, 0, 0);
    E("conv.batch_norm.weight", K_GAIN, 1, ENC_D, 0, 0);
    E("conv.batch_norm.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("conv.pointwise_conv2.weight", K_NORMAL, 3, ENC_D, ENC_D, 1);
    E("conv.pointwise_conv2.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("norm_feed_forward2.weight", K_GAIN, 1, ENC_D, 0, 0);
    E("norm_feed_forward2.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("feed_forward2.linear1.weight", K_NORMAL, 2, ENC_FF, ENC_D, 0);
    E("feed_forward2.linear1.bias", K_BIAS, 1, ENC_FF, 0, 0);
    E("feed_forward2.linear2.weight", K_NORMAL, 2, ENC_D, ENC_FF, 0);
    E("feed_forward2.linear2.bias", K_BIAS, 1, ENC_D, 0, 0);
    E("norm_out.weight", K_GAIN, 1, ENC_D, 0, 0);
    E("norm_out.bias", K_BIAS, 1, ENC_D, 0, 0);
#undef E
}

static void add_dec(int i, const char *sfx, int kind, int nd, int a, int b) {
    char n[96];
    snprintf(n, sizeof n, "%s%d.%s", DEC_PFX, i, sfx);
    add_t(n, kind, nd, a, b, 0);
}

static void table_init(void) {
    add_t("encoder.pre_encode.conv.0.weight", K_NORMAL, 3, SUB_CH, 1, 9);
    add_t("encoder.pre_encode.conv.0.bias", K_BIAS, 1, SUB_CH, 0, 0);
    add_t("encoder.pre_encode.conv.2.weight", K_NORMAL, 3, SUB_CH, 1, 9);
    add_t("encoder.pre_encode.conv.2.bias", K_BIAS, 1, SUB_CH, 0, 0);
    add_t("encoder.pre_encode.conv.3.weight", K_NORMAL, 2, SUB_CH, SUB_CH, 0);
    add_t("encoder.pre_encode.conv.3.bias", K_BIAS, 1, SUB_CH, 0, 0);
    add_t("encoder.pre_encode.conv.5.weight", K_NORMAL, 3, SUB_CH, 1, 9);
    add_t("encoder.pre_encode.conv.5.bias", K_BIAS, 1, SUB_CH, 0, 0);
    add_t("encoder.pre_encode.conv.6.weight", K_NORMAL, 2, SUB_CH, SUB_CH, 0);
    add_t("encoder.pre_encode.conv.6.bias", K_BIAS, 1, SUB_CH, 0, 0);
    add_t("encoder.pre_encode.out.weight", K_NORMAL, 2, ENC_D, SUB_CH * 16, 0);
    add_t("encoder.pre_encode.out.bias", K_BIAS, 1, ENC_D, 0, 0);
    for (int i = 0; i < ENC_N; i++) add_enc_layer(i);
    add_t("encoder_decoder_proj.weight", K_NORMAL, 2, DEC_D, ENC_D, 0);
    add_t("encoder_decoder_proj.bias", K_BIAS, 1, DEC_D, 0, 0);
    for (int i = 0; i < DEC_N; i++) {
        add_dec(i, "second_sub_layer.key_net.weight", K_NORMAL, 2, DEC_D, DEC_D);
        add_dec(i, "second_sub_layer.key_net.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "second_sub_layer.value_net.weight", K_NORMAL, 2, DEC_D, DEC_D);
        add_dec(i, "second_sub_layer.value_net.bias", K_BIAS, 1, DEC_D, 0);
    }
    add_t("transf_decoder._embedding.token_embedding.weight", K_NORMAL, 2, VOCAB, DEC_D, 0);
    add_t("transf_decoder._embedding.position_embedding.pos_enc", K_NORMAL, 2, MAX_SEQ, DEC_D, 0);
    add_t("transf_decoder._embedding.layer_norm.weight", K_GAIN, 1, DEC_D, 0, 0);
    add_t("transf_decoder._embedding.layer_norm.bias", K_BIAS, 1, DEC_D, 0, 0);
    for (int i = 0; i < DEC_N; i++) {
        add_dec(i, "layer_norm_1.weight", K_GAIN, 1, DEC_D, 0);
        add_dec(i, "layer_norm_1.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "first_sub_layer.query_net.weight", K_NORMAL, 2, DEC_D, DEC_D);
        add_dec(i, "first_sub_layer.query_net.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "first_sub_layer.key_net.weight", K_NORMAL, 2, DEC_D, DEC_D);
        add_dec(i, "first_sub_layer.key_net.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "first_sub_layer.value_net.weight", K_NORMAL, 2, DEC_D, DEC_D);
        add_dec(i, "first_sub_layer.value_net.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "first_sub_layer.out_projection.weight", K_NORMAL, 2, DEC_D, DEC_D);
        add_dec(i, "first_sub_layer.out_projection.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "layer_norm_2.weight", K_GAIN, 1, DEC_D, 0);
        add_dec(i, "layer_norm_2.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "second_sub_layer.query_net.weight", K_NORMAL, 2, DEC_D, DEC_D);
        add_dec(i, "second_sub_layer.query_net.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "second_sub_layer.out_projection.weight", K_NORMAL, 2, DEC_D, DEC_D);
        add_dec(i, "second_sub_layer.out_projection.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "layer_norm_3.weight", K_GAIN, 1, DEC_D, 0);
        add_dec(i, "layer_norm_3.bias", K_BIAS, 1, DEC_D, 0);
        add_dec(i, "third_sub_layer.dense_in.weight", K_NORMAL, 2, DEC_FF, DEC_D);
        add_dec(i, "third_sub_layer.dense_in.bias", K_BIAS, 1, DEC_FF, 0);
        add_dec(i, "third_sub_layer.dense_out.weight", K_NORMAL, 2, DEC_D, DEC_FF);
        add_dec(i, "third_sub_layer.dense_out.bias", K_BIAS, 1, DEC_D, 0);
    }
    add_t("transf_decoder._decoder.final_layer_norm.weight", K_GAIN, 1, DEC_D, 0, 0);
    add_t("transf_decoder._decoder.final_layer_norm.bias", K_BIAS, 1, DEC_D, 0, 0);
    add_t("log_softmax.mlp.layer0.bias", K_BIAS, 1, VOCAB, 0, 0);
}

int ct_synth_tensor_count(void) {
    pthread_once(&g_tonce, table_init);
    return g_nt;
}

/* Serialises the JSON header (unpadded) into out (may be NULL); returns length. */
static size_t header_json(char *out, size_t cap) {
    size_t n = 0;
    char tmp[512];
#define PUT(s) do { size_t l_ = strlen(s); if (out && n + l_ <= cap) memcpy(out + n, s, l_); n += l_; } while (0)
    PUT("{");
    for (int i = 0; i < g_nt; i++) {
        const TInfo *t = &g_tab[i];
        char shp[64];
        if (t->nd == 1) snprintf(shp, sizeof shp, "[%d]", t->shape[0]);
        else if (t->nd == 2) snprintf(shp, sizeof shp, "[%d,%d]", t->shape[0], t->shape[1]);
        else snprintf(shp, sizeof shp, "[%d,%d,%d]", t->shape[0], t->shape[1], t->shape[2]);
        snprintf(tmp, sizeof tmp, "%s\"%s\":{\"dtype\":\"BF16\",\"shape\":%s,\"data_offsets\":[%zu,%zu]}",
                 i ? "," : "", t->name, shp, t->off, t->off + t->elems * 2);
        PUT(tmp);
    }
    PUT("}");
#undef PUT
    return n;
}

static size_t header_padded(void) {
    const size_t h = header_json(NULL, 0);
    return h + (8 - h % 8) % 8;
}

size_t ct_synth_file_bytes(void) {
    pthread_once(&g_tonce, table_init);
    return 8 + header_padded() + g_data_bytes;
}

typedef struct {
    uint8_t *data;
    uint64_t seed;
    int variant, tid, nthr;
} FillArg;

static uint16_t gen_value(const TInfo *t, int variant, uint64_t key, size_t i) {
    const float z = ct_normal16(ct_hash64(key, i));
    switch (t->kind) {
    case K_NORMAL:
        if ((variant == 2 || variant == 3) && !strncmp(t->name, DEC_PFX, strlen(DEC_PFX)))
            return to_bf16_rne((variant == 2 ? 0.12f : 0.08f) * z);
        return to_bf16_rne(0.02f * z);
    case K_ONES:   return to_bf16_rne(1.0f);
    case K_ZEROS:  return 0;
    case K_BIAS:   return variant == 1 ? to_bf16_rne(0.02f * z) : 0;
    case K_GAIN:   return to_bf16_rne(variant == 1 ? 1.0f + 0.02f * z : 1.0f);
    case K_VAR:    return to_bf16_rne(variant == 1 ? 1.0f + fabsf(0.1f * z) : 1.0f);
    }
    return 0;
}

/* Work is split into fixed 1 Mi-element chunks over all tensors; each value
 * depends only on (seed, tensor index, element index). */
#define CHUNK ((size_t)1 << 20)
static void *fill_worker(void *p) {
    FillArg *a = (FillArg *)p;
    size_t chunk_id = 0;
    for (int ti = 0; ti < g_nt; ti++) {
        const TInfo *t = &g_tab[ti];
        const uint64_t key = mix64(a->seed * 0xD1B54A32D192ED03ULL + (uint64_t)ti * 0x8CB92BA72F3D8DD7ULL);
        uint16_t *dst = (uint16_t *)(a->data + t->off);
        for (size_t c0 = 0; c0 < t->elems; c0 += CHUNK, chunk_id++) {
            if ((int)(chunk_id % (size_t)a->nthr) != a->tid) continue;
            const size_t c1 = c0 + CHUNK < t->elems ? c0 + CHUNK : t->elems;
            for (size_t i = c0; i < c1; i++) {
                const uint16_t v = gen_value(t, a->variant, key, i);
                memcpy(dst + i, &v, 2);
            }
        }
    }
    return NULL;
}

int ct_synth_weights(uint8_t *buf, size_t cap, uint64_t seed, int variant, int nthreads) {
    pthread_once(&g_tonce, table_init);
    pthread_once(&g_qonce, qtab_init);
    const size_t hp = header_padded();
    if (cap < 8 + hp + g_data_bytes) return -1;
    const uint64_t hl = hp;
    memcpy(buf, &hl, 8);
    const size_t h = header_json((char *)buf + 8, hp);
    memset(buf + 8 + h, ' ', hp - h);
    if (nthreads <= 0) {
        const long c = sysconf(_SC_NPROCESSORS_ONLN);
        nthreads = c > 0 ? (int)c : 1;
    }
    if (nthreads > 64) nthreads = 64;
    pthread_t th[64];
    FillArg args[64];
    for (int i = 0; i < nthreads; i++) {
        args[i] = (FillArg){buf + 8 + hp, seed, variant, i, nthreads};
        pthread_create(&th[i], NULL, fill_worker, &args[i]);
    }
    for (int i = 0; i < nthreads; i++) pthread_join(th[i], NULL);
    return 0;
}

/* ---------------- binding (safetensors header lookup) ---------------- */

/* Finds "name": at a key position (preceded by '{' or ',') and reads its
 * data_offsets.  Returns 0 on success. */
static int find_tensor(const char *hdr, size_t hlen, const char *name, size_t *s, size_t *e) {
    char key[128];
    const size_t kl = (size_t)snprintf(key, sizeof key, "\"%s\":", name);
    for (size_t i = 1; i + kl <= hlen; i++) {
        if ((hdr[i - 1] != '{' && hdr[i - 1] != ',') || memcmp(hdr + i, key, kl) != 0) continue;
        const char *p = hdr + i + kl;
        const char *end = hdr + hlen;
        const char *d = NULL;
        for (const char *q = p; q + 14 <= end; q++)
            if (!memcmp(q, "\"data_offsets\"", 14)) { d = q; break; }
        if (!d) return -1;
        while (d < end && *d != '[') d++;
        if (d >= end) return -1;
        unsigned long long a, b;
        if (sscanf(d + 1, " %llu , %llu", &a, &b) != 2 || b < a) return -1;
        *s = (size_t)a; *e = (size_t)b;
        return 0;
    }
    return -1;
}

int ct_weights_bind(const uint8_t *image, size_t size, Weights *W,
                    const uint8_t **data, size_t *data_bytes) {
    if (size < 8) return -1;
    uint64_t hl; memcpy(&hl, image, 8);
    if (8 + hl > size) return -1;
    const char *hdr = (const char *)image + 8;
    const uint8_t *base = image + 8 + hl;
    const size_t dbytes = size - 8 - hl;
    int bad = 0;
    char n[160];
#define GET(dst, nm) do { size_t s_, e_; \
        if (find_tensor(hdr, hl, nm, &s_, &e_) || e_ > dbytes) { \
            fprintf(stderr, "weights: tensor not found: %s\n", nm); bad = 1; (dst) = NULL; } \
        else (dst) = (const uint16_t *)(base + s_); } while (0)
    GET(W->s0w, "encoder.pre_encode.conv.0.weight"); GET(W->s0b, "encoder.pre_encode.conv.0.bias");
    GET(W->s2w, "encoder.pre_encode.conv.2.weight"); GET(W->s2b, "encoder.pre_encode.conv.2.bias");
    GET(W->s3w, "encoder.pre_encode.conv.3.weight"); GET(W->s3b, "encoder.pre_encode.conv.3.bias");
    GET(W->s5w, "encoder.pre_encode.conv.5.weight"); GET(W->s5b, "encoder.pre_encode.conv.5.bias");
    GET(W->s6w, "encoder.pre_encode.conv.6.weight"); GET(W->s6b, "encoder.pre_encode.conv.6.bias");
    GET(W->sow, "encoder.pre_encode.out.weight");    GET(W->sob, "encoder.pre_encode.out.bias");
    for (int i = 0; i < ENC_N; i++) {
        ELayer *L = &W->enc[i];
#define EG(f, s) do { snprintf(n, sizeof n, "%s%d.%s", ENC_PFX, i, s); GET(L->f, n); } while (0)
        EG(ff1_lnw, "norm_feed_forward1.weight"); EG(ff1_lnb, "norm_feed_forward1.bias");
        EG(ff1_w1, "feed_forward1.linear1.weight"); EG(ff1_b1, "feed_forward1.linear1.bias");
        EG(ff1_w2, "feed_forward1.linear2.weight"); EG(ff1_b2, "feed_forward1.linear2.bias");
        EG(sa_lnw, "norm_self_att.weight"); EG(sa_lnb, "norm_self_att.bias");
        EG(sa_qw, "self_attn.linear_q.weight"); EG(sa_qb, "self_attn.linear_q.bias");
        EG(sa_kw, "self_attn.linear_k.weight"); EG(sa_kb, "self_attn.linear_k.bias");
        EG(sa_vw, "self_attn.linear_v.weight"); EG(sa_vb, "self_attn.linear_v.bias");
        EG(sa_pw, "self_attn.linear_pos.weight");
        EG(sa_ow, "self_attn.linear_out.weight"); EG(sa_ob, "self_attn.linear_out.bias");
        EG(sa_pbu, "self_attn.pos_bias_u"); EG(sa_pbv, "self_attn.pos_bias_v");
        EG(cv_lnw, "norm_conv.weight"); EG(cv_lnb, "norm_conv.bias");
        EG(cv_pw1w, "conv.pointwise_conv1.weight"); EG(cv_pw1b, "conv.pointwise_conv1.bias");
        EG(cv_dww, "conv.depthwise_conv.weight"); EG(cv_dwb, "conv.depthwise_conv.bias");
        EG(cv_bnw, "conv.batch_norm.weight"); EG(cv_bnb, "conv.batch_norm.bias");
        EG(cv_bnmean, "conv.batch_norm.running_mean"); EG(cv_bnvar, "conv.batch_norm.running_var");
        EG(cv_pw2w, "conv.pointwise_conv2.weight"); EG(cv_pw2b, "conv.pointwise_conv2.bias");
        EG(ff2_lnw, "norm_feed_forward2.weight"); EG(ff2_lnb, "norm_feed_forward2.bias");
        EG(ff2_w1, "feed_forward2.linear1.weight"); EG(ff2_b1, "feed_forward2.linear1.bias");
        EG(ff2_w2, "feed_forward2.linear2.weight"); EG(ff2_b2, "feed_forward2.linear2.bias");
        EG(out_lnw, "norm_out.weight"); EG(out_lnb, "norm_out.bias");
#undef EG
    }
    GET(W->prw, "encoder_decoder_proj.weight"); GET(W->prb, "encoder_decoder_proj.bias");
    GET(W->etw, "transf_decoder._embedding.token_embedding.weight");
    GET(W->epw, "transf_decoder._embedding.position_embedding.pos_enc");
    GET(W->elnw, "transf_decoder._embedding.layer_norm.weight");
    GET(W->elnb, "transf_decoder._embedding.layer_norm.bias");
    for (int i = 0; i < DEC_N; i++) {
        DLayer *L = &W->dec[i];
#define DG(f, s) do { snprintf(n, sizeof n, "%s%d.%s", DEC_PFX, i, s); GET(L->f, n); } while (0)
        DG(sa_lnw, "layer_norm_1.weight"); DG(sa_lnb, "layer_norm_1.bias");
        DG(sa_qw, "first_sub_layer.query_net.weight"); DG(sa_qb, "first_sub_layer.query_net.bias");
        DG(sa_kw, "first_sub_layer.key_net.weight"); DG(sa_kb, "first_sub_layer.key_net.bias");
        DG(sa_vw, "first_sub_layer.value_net.weight"); DG(sa_vb, "first_sub_layer.value_net.bias");
        DG(sa_ow, "first_sub_layer.out_projection.weight"); DG(sa_ob, "first_sub_layer.out_projection.bias");
        DG(ca_lnw, "layer_norm_2.weight"); DG(ca_lnb, "layer_norm_2.bias");
        DG(ca_qw, "second_sub_layer.query_net.weight"); DG(ca_qb, "second_sub_layer.query_net.bias");
        DG(ca_kw, "second_sub_layer.key_net.weight"); DG(ca_kb, "second_sub_layer.key_net.bias");
        DG(ca_vw, "second_sub_layer.value_net.weight"); DG(ca_vb, "second_sub_layer.value_net.bias");
        DG(ca_ow, "second_sub_layer.out_projection.weight"); DG(ca_ob, "second_sub_layer.out_projection.bias");
        DG(ffn_lnw, "layer_norm_3.weight"); DG(ffn_lnb, "layer_norm_3.bias");
        DG(ffn_w1, "third_sub_layer.dense_in.weight"); DG(ffn_b1, "third_sub_layer.dense_in.bias");
        DG(ffn_w2, "third_sub_layer.dense_out.weight"); DG(ffn_b2, "third_sub_layer.dense_out.bias");
#undef DG
    }
    GET(W->dlnw, "transf_decoder._decoder.final_layer_norm.weight");
    GET(W->dlnb, "transf_decoder._decoder.final_layer_norm.bias");
    GET(W->hdb, "log_softmax.mlp.layer0.bias");
#undef GET
    if (data) *data = base;
    if (data_bytes) *data_bytes = dbytes;
    return bad ? -1 : 0;
}

/* ---------------- audio ---------------- */

static inline double unit53(uint64_t h) { return (double)(h >> 11) * (1.0 / 9007199254740992.0); }

void ct_synth_audio(float *out, int n, uint64_t seed) {
    const uint64_t key = mix64(seed ^ 0xA0761D6478BD642FULL);
    double f[5], ph[5], amp[5];
    for (int i = 0; i < 5; i++) {
        f[i] = 100.0 + 3900.0 * unit53(ct_hash64(key, 3 * i));
        ph[i] = 2.0 * M_PI * unit53(ct_hash64(key, 3 * i + 1));
        amp[i] = 0.1 * unit53(ct_hash64(key, 3 * i + 2));
    }
    const uint64_t nkey = mix64(key + 1);
    for (int t = 0; t < n; t++) {
        double v = 0.0;
        for (int i = 0; i < 5; i++) v += amp[i] * sin(2.0 * M_PI * f[i] * t / SR + ph[i]);
        /* Box-Muller on two 53-bit uniforms; u1 in (0, 1]. */
        const double u1 = 1.0 - unit53(ct_hash64(nkey, 2 * (uint64_t)t));
        const double u2 = unit53(ct_hash64(nkey, 2 * (uint64_t)t + 1));
        v += 0.01 * sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2);
        out[t] = (float)v;
    }
}
