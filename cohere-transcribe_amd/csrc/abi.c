/* abi.c — the 40 backend.h functions for MI355X, in C.
 *
 * Host-side glue only: device memory, streams, graph capture/replay, weight
 * pointer translation and the per-thread decode latches.  All arithmetic runs
 * in the gfx950 kernels behind ct_launch.h.
 *
 * Contract followed (reference file:line):
 *  - per-thread stream, arena and small device arrays; the weight blob is
 *    per device and read-only (backends/cuda/backend.cu:38-58, 108-159);
 *  - compute calls take HOST weight pointers and translate them by offset
 *    into the device copy of the blob (backends/cuda/backend.cu:95-99);
 *  - arena grows, never shrinks, and a new allocation drops cached graphs
 *    (backends/cuda/backend.cu:165-184);
 *  - graphs are cached under (tag, T, S, B, arena) and end_capture runs the
 *    captured region once (backends/cuda/backend.cu:802-860);
 *  - S latched by embed_decode_batch, T_enc by upload_T_enc
 *    (backends/cpu/backend.c:425-500).
 * Errors print and exit(1), as every reference backend does.
 */
#include "../../include/backend.h"
#include "ct_launch.h"
#include "ct_abi_state.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* Process-wide state: one read-only weight blob per device.           */
/* ------------------------------------------------------------------ */
static void *g_blob[CT_MAX_DEVICES];        /* blob start on each device          */
static void *g_blob_alloc[CT_MAX_DEVICES];  /* the allocation it sits in          */
static float *g_inv_freq[CT_MAX_DEVICES];
static const uint8_t *g_host_base;
static size_t g_blob_bytes;
static int g_ndev;
static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;

_Thread_local CtThread ct_t = {.dev = -1};

void ct_fatal(const char *what, const char *file, int line) {
    fprintf(stderr, "hip backend: %s (%s:%d)\n", what, file, line);
    exit(1);
}

void ct_hip_check(hipError_t e, const char *expr, const char *file, int line) {
    if (e != hipSuccess) {
        fprintf(stderr, "HIP error %s: %s (%s:%d)\n", hipGetErrorString(e), expr, file, line);
        exit(1);
    }
}

const void *ct_dev_w(const void *host_ptr) {
    if (!host_ptr) return NULL;
    if (!g_host_base || ct_t.dev < 0 || !g_blob[ct_t.dev])
        CT_FATAL("weight pointer used before backend_weights_upload_blob/backend_init "
                 "(build the host with -DBACKEND_CUDA so transcribe.c uploads the blob)");
    const uint8_t *p = (const uint8_t *)host_ptr;
    if (p < g_host_base || p >= g_host_base + g_blob_bytes)
        CT_FATAL("weight pointer outside the uploaded blob");
    return (const uint8_t *)g_blob[ct_t.dev] + (p - g_host_base);
}

const float *ct_inv_freq(void) { return g_inv_freq[ct_t.dev]; }

static void require_init(void) {
    if (ct_t.dev < 0) CT_FATAL("backend used on a thread that has not called backend_init");
}

/* ------------------------------------------------------------------ */
/* Lifecycle                                                           */
/* ------------------------------------------------------------------ */
int backend_num_devices(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n > CT_MAX_DEVICES ? CT_MAX_DEVICES : n;
}

void backend_weights_upload_blob(const void *host_base, size_t bytes) {
    int n = backend_num_devices();
    if (n <= 0) CT_FATAL("no HIP device");
    pthread_mutex_lock(&g_lock);
    g_host_base = (const uint8_t *)host_base;
    g_blob_bytes = bytes;
    /* A safetensors blob (8-byte header length, then a JSON header padded to
     * 8 bytes, convert.py:217-220) is placed so that its data section starts
     * 16-byte aligned on the device: every tensor of the model is a multiple
     * of 16 bytes, so all of them can then be read in 16-byte pieces. */
    size_t shift = 0;
    if (bytes > 9) {
        uint64_t hlen = 0;
        memcpy(&hlen, host_base, 8);
        if (hlen < bytes - 8 && ((const char *)host_base)[8] == '{') shift = (16 - (8 + hlen) % 16) % 16;
    }
    for (int d = 0; d < n; d++) {
        CHK(hipSetDevice(d));
        if (g_blob_alloc[d]) CHK(hipFree(g_blob_alloc[d]));
        CHK(hipMalloc(&g_blob_alloc[d], bytes + 16));
        g_blob[d] = (char *)g_blob_alloc[d] + shift;
        CHK(hipMemcpy(g_blob[d], host_base, bytes, hipMemcpyHostToDevice));
    }
    g_ndev = n;
    pthread_mutex_unlock(&g_lock);
}

void *backend_device_ptr(const void *host_ptr) { return (void *)ct_dev_w(host_ptr); }

void backend_init(int device_id) {
    if (device_id < 0 || device_id >= CT_MAX_DEVICES) CT_FATAL("device id out of range");
    CHK(hipSetDevice(device_id));
    ct_t.dev = device_id;
    CHK(hipStreamCreate(&ct_t.stream));
    CHK(hipMalloc((void **)&ct_t.d_tokens, MAX_SEQ * sizeof(int)));
    CHK(hipMalloc((void **)&ct_t.d_S, sizeof(int)));
    CHK(hipMalloc((void **)&ct_t.d_S_batch, CT_MAX_BATCH * sizeof(int)));
    CHK(hipMalloc((void **)&ct_t.d_T_enc, CT_MAX_BATCH * sizeof(int)));
    CHK(hipMalloc((void **)&ct_t.d_active, CT_MAX_BATCH * sizeof(int)));
    CHK(hipMalloc((void **)&ct_t.d_out, CT_MAX_BATCH * sizeof(int)));
    CHK(hipHostMalloc((void **)&ct_t.h_stage, (4 * CT_MAX_BATCH + MAX_SEQ) * sizeof(int), 0));
    pthread_mutex_lock(&g_lock);
    if (!g_inv_freq[device_id]) {
        /* w_k = exp(-2k ln(1e4) / ENC_D) in the reference's fp32 expression
         * order (backends/cpu/backend.c:233-237), computed with the host libm. */
        float w[ENC_D / 2];
        const float l = logf(10000.0f);
        for (int k = 0; k < ENC_D / 2; k++) w[k] = expf(-(float)(2 * k) * l / ENC_D);
        CHK(hipMalloc((void **)&g_inv_freq[device_id], sizeof w));
        CHK(hipMemcpy(g_inv_freq[device_id], w, sizeof w, hipMemcpyHostToDevice));
    }
    ct_static_init(device_id);
    pthread_mutex_unlock(&g_lock);
}

static void graphs_drop(void) {
    for (int i = 0; i < ct_t.n_graphs; i++) {
        hipGraphExecDestroy(ct_t.graphs[i].exec);
        hipGraphDestroy(ct_t.graphs[i].graph);
    }
    ct_t.n_graphs = 0;
}

void backend_thread_cleanup(void) {
    if (ct_t.dev < 0) return;
    CHK(hipSetDevice(ct_t.dev));
    CHK(hipStreamSynchronize(ct_t.stream));
    graphs_drop();
    free(ct_t.graphs);
    ct_t.graphs = NULL;
    ct_t.graph_cap = 0;
    if (ct_t.arena) CHK(hipFree(ct_t.arena));
    CHK(hipFree(ct_t.d_tokens));
    CHK(hipFree(ct_t.d_S));
    CHK(hipFree(ct_t.d_S_batch));
    CHK(hipFree(ct_t.d_T_enc));
    CHK(hipFree(ct_t.d_active));
    CHK(hipFree(ct_t.d_out));
    CHK(hipHostFree(ct_t.h_stage));
    CHK(hipStreamDestroy(ct_t.stream));
    memset(&ct_t, 0, sizeof ct_t);
    ct_t.dev = -1;
}

void backend_destroy(void) {
    backend_thread_cleanup();
    pthread_mutex_lock(&g_lock);
    for (int d = 0; d < CT_MAX_DEVICES; d++) {
        if (g_blob[d] || g_inv_freq[d]) CHK(hipSetDevice(d));
        if (g_blob_alloc[d]) { CHK(hipFree(g_blob_alloc[d])); g_blob_alloc[d] = NULL; g_blob[d] = NULL; }
        if (g_inv_freq[d]) { CHK(hipFree(g_inv_freq[d])); g_inv_freq[d] = NULL; }
    }
    g_ndev = 0;
    g_host_base = NULL;
    g_blob_bytes = 0;
    pthread_mutex_unlock(&g_lock);
}

/* ------------------------------------------------------------------ */
/* Memory                                                              */
/* ------------------------------------------------------------------ */
float *backend_arena_alloc(size_t floats) {
    if (floats > ((size_t)1 << 40)) CT_FATAL("backend_arena_alloc: request above 2^40 floats");
    require_init();
    const size_t need = (floats ? floats : 1) * sizeof(float);
    if (ct_t.arena) graphs_drop();
    if (need > ct_t.arena_bytes) {
        if (ct_t.arena) {
            CHK(hipStreamSynchronize(ct_t.stream));
            CHK(hipFree(ct_t.arena));
        }
        CHK(hipMalloc((void **)&ct_t.arena, need));
        ct_t.arena_bytes = need;
    }
    return ct_t.arena;
}

void backend_arena_free(float *arena) {
    (void)arena;
    require_init();
    CHK(hipStreamSynchronize(ct_t.stream));
}

void backend_htod(float *dev_dst, const float *host_src, size_t floats) {
    require_init();
    CHK(hipMemcpyAsync(dev_dst, host_src, floats * sizeof(float), hipMemcpyHostToDevice, ct_t.stream));
    CHK(hipStreamSynchronize(ct_t.stream));
}

void backend_dtoh(void *host_dst, const void *dev_src, size_t bytes) {
    require_init();
    CHK(hipMemcpyAsync(host_dst, dev_src, bytes, hipMemcpyDeviceToHost, ct_t.stream));
    CHK(hipStreamSynchronize(ct_t.stream));
}

/* Copies n host ints to a device array through pinned staging; the staging
 * slot is private to the call site and the copy completes before return. */
static void put_ints(int *dst, const int *src, int n, int slot) {
    if (n <= 0) return;
    if (n > CT_MAX_BATCH && slot != 4) CT_FATAL("batch larger than 256");
    int *stage = ct_t.h_stage + slot * CT_MAX_BATCH;
    memcpy(stage, src, (size_t)n * sizeof(int));
    CHK(hipMemcpyAsync(dst, stage, (size_t)n * sizeof(int), hipMemcpyHostToDevice, ct_t.stream));
}

static int capturing(void) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    CHK(hipStreamIsCapturing(ct_t.stream, &st));
    return st != hipStreamCaptureStatusNone;
}

/* ------------------------------------------------------------------ */
/* Dense ops                                                           */
/* ------------------------------------------------------------------ */
void backend_layernorm(float *dst, const float *src, const uint16_t *w, const uint16_t *b,
                       int T, int D) {
    require_init();
    ctk_layernorm(dst, src, CT_W(w), CT_W(b), T, D, ct_t.stream);
}

static void linear_epi(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                       int T, int in_d, int out_d, int epi, float scale) {
    require_init();
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.A = x; g.lda = in_d; g.W = CT_W(W); g.bias = CT_W(b);
    g.Y = y; g.ldy = out_d; g.M = T; g.N = out_d; g.K = in_d;
    g.epi = epi; g.scale = scale;
    ctk_gemm(&g, ct_t.stream);
}

void backend_linear(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                    int T, int in_d, int out_d) {
    linear_epi(y, x, W, b, T, in_d, out_d, CT_EPI_STORE, 0.0f);
}
void backend_linear_silu(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                         int T, int in_d, int out_d) {
    linear_epi(y, x, W, b, T, in_d, out_d, CT_EPI_SILU, 0.0f);
}
void backend_linear_relu(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                         int T, int in_d, int out_d) {
    linear_epi(y, x, W, b, T, in_d, out_d, CT_EPI_RELU, 0.0f);
}
void backend_linear_fmadd(float *acc, float scale, const float *x, const uint16_t *W,
                          const uint16_t *b, int T, int in_d, int out_d) {
    linear_epi(acc, x, W, b, T, in_d, out_d, CT_EPI_FMADD, scale);
}

void backend_add_inplace(float *dst, const float *src, int n) {
    require_init();
    ctk_add(dst, src, n, ct_t.stream);
}

/* ------------------------------------------------------------------ */
/* Encoder                                                             */
/* ------------------------------------------------------------------ */
void backend_encoder_subsampling(const float *mel, int T_mel, int T_mel_stride,
                                 float *x_enc, int T_enc, float *work, const Weights *W) {
    require_init();
    /* Scratch plan inside the caller's SUB_CH*(T1*64 + T2*32) floats
     * (transcribe.c:282-283): region A = [0, B0), region B = [B0, B0+B1). */
    const int T1 = (T_mel + 1) / 2, T2 = (T1 + 1) / 2;
    float *ra = work, *rb = work + (size_t)SUB_CH * T1 * 64;
    hipStream_t s = ct_t.stream;
    ctk_sub_conv0(ra, mel, T_mel, T_mel_stride, CT_W(W->s0w), CT_W(W->s0b), s);
    ctk_sub_dwconv(rb, ra, T1, 64, CT_W(W->s2w), CT_W(W->s2b), s);
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.A = rb; g.lda = SUB_CH; g.W = CT_W(W->s3w); g.bias = CT_W(W->s3b);
    g.Y = ra; g.ldy = SUB_CH; g.M = T2 * 32; g.N = SUB_CH; g.K = SUB_CH; g.epi = CT_EPI_RELU;
    ctk_gemm(&g, s);
    ctk_sub_dwconv(rb, ra, T2, 32, CT_W(W->s5w), CT_W(W->s5b), s);
    g.A = rb; g.W = CT_W(W->s6w); g.bias = CT_W(W->s6b); g.Y = ra; g.M = T_enc * 16;
    ctk_gemm(&g, s);
    ctk_sub_flatten(rb, ra, T_enc, s);
    memset(&g, 0, sizeof g);
    g.A = rb; g.lda = SUB_CH * 16; g.W = CT_W(W->sow); g.bias = CT_W(W->sob);
    g.Y = x_enc; g.ldy = ENC_D; g.M = T_enc; g.N = ENC_D; g.K = SUB_CH * 16; g.epi = CT_EPI_STORE;
    ctk_gemm(&g, s);
}

void backend_make_rel_pos_emb(float *pe, int T) {
    require_init();
    ctk_rel_pos_emb(pe, T, ct_inv_freq(), ct_t.stream);
}

void backend_rel_pos_mhsa(float *x, const float *pos_emb, int T, const ELayer *L, float *work) {
    require_init();
    /* Scratch: Q, K, V (T rows), P (2T-1 rows), O (T rows), i.e.
     * CT_MHSA_SCRATCH_FLOATS(T) = (6T-1)*ENC_D floats, within the
     * (5T-1)*ENC_D + max(T(3T-1), 2T*ENC_D) >= (7T-1)*ENC_D floats the host
     * provides (transcribe.c:286-293). */
    const size_t TD = (size_t)T * ENC_D;
    float *Q = work, *K = Q + TD, *V = K + TD, *P = V + TD, *O = P + (size_t)(2 * T - 1) * ENC_D;
    const float *Xs[4] = {x, x, x, pos_emb};
    float *Ys[4] = {Q, K, V, P};
    const uint16_t *Ws[4] = {L->sa_qw, L->sa_kw, L->sa_vw, L->sa_pw};
    const uint16_t *Bs[4] = {L->sa_qb, L->sa_kb, L->sa_vb, NULL};
    for (int i = 0; i < 4; i++)
        backend_linear(Ys[i], Xs[i], Ws[i], Bs[i], i == 3 ? 2 * T - 1 : T, ENC_D, ENC_D);
    ctk_relpos_attn(O, Q, K, V, P, CT_W(L->sa_pbu), CT_W(L->sa_pbv), T, ct_t.stream);
    backend_linear(x, O, L->sa_ow, L->sa_ob, T, ENC_D, ENC_D);
}

void backend_rel_pos_mhsa_noalloc(float *x, const float *pos_emb, int T, const ELayer *L) {
    if (T < 1 || T > CT_STATIC_MHSA_MAX_T) {
        fprintf(stderr, "hip backend: backend_rel_pos_mhsa_noalloc: T=%d outside [1, %d] frames "
                        "(its scratch holds a 30 s clip; use backend_rel_pos_mhsa with a workspace)\n",
                T, CT_STATIC_MHSA_MAX_T);
        exit(1);
    }
    require_init();
    float *work = ct_static_scratch(ct_t.dev);
    if (!work) CT_FATAL("backend_rel_pos_mhsa_noalloc: device scratch not set up");
    if (CT_MHSA_SCRATCH_FLOATS(T) > ct_static_scratch_floats())
        CT_FATAL("backend_rel_pos_mhsa_noalloc: scratch smaller than the layout");
    backend_rel_pos_mhsa(x, pos_emb, T, L, work);
}

void backend_conformer_conv(float *x, int T, const ELayer *L, float *work) {
    require_init();
    float *glu = work, *dw = work + (size_t)T * ENC_D;
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.A = x; g.lda = ENC_D; g.W = CT_W(L->cv_pw1w); g.bias = CT_W(L->cv_pw1b);
    g.Y = glu; g.ldy = ENC_D; g.M = T; g.N = 2 * ENC_D; g.K = ENC_D;
    g.epi = CT_EPI_GLU; g.glu_half = ENC_D;
    ctk_gemm(&g, ct_t.stream);
    ctk_dwconv_bn_silu(dw, glu, T, CT_W(L->cv_dww), CT_W(L->cv_dwb), CT_W(L->cv_bnw),
                       CT_W(L->cv_bnb), CT_W(L->cv_bnmean), CT_W(L->cv_bnvar), ct_t.stream);
    backend_linear(x, dw, L->cv_pw2w, L->cv_pw2b, T, ENC_D, ENC_D);
}

/* ------------------------------------------------------------------ */
/* Decoder (prefill / single)                                          */
/* ------------------------------------------------------------------ */
static void attn_common(CtAttn *a, float *out, const float *Q) {
    memset(a, 0, sizeof *a);
    a->out = out; a->Q = Q;
    a->q_sb = DEC_D; a->q_st = DEC_D;
    a->kv_st = DEC_D; a->kv_sh = DEC_DK;
    a->H = DEC_H;
    a->scale = 1.0f / sqrtf((float)DEC_DK);
}

void backend_sdp_attn(float *out, const float *q, const float *k, const float *v,
                      const float *mask, int T_q, int T_k, float *work) {
    (void)work;
    require_init();
    CtAttn a;
    attn_common(&a, out, q);
    a.K = k; a.V = v; a.len_const = T_k; a.mask = mask; a.T_q = T_q; a.B = 1;
    ctk_attn(&a, ct_t.stream);
}

void backend_embed(float *h, const int *tokens, int S, int pos_start,
                   const uint16_t *etw, const uint16_t *epw,
                   const uint16_t *elnw, const uint16_t *elnb) {
    if (S < 0 || S > MAX_SEQ) CT_FATAL("embed: S outside [0, MAX_SEQ]");
    require_init();
    /* Inside a captured region the tokens must already be staged
     * (backend_upload_tokens, model.h:466); outside, stage them here. */
    if (!capturing() && tokens) {
        put_ints(ct_t.d_tokens, tokens, S, 4);
        CHK(hipStreamSynchronize(ct_t.stream));
    }
    ctk_embed_ln(h, ct_t.d_tokens, S, pos_start, NULL, NULL, CT_W(etw), CT_W(epw),
                 CT_W(elnw), CT_W(elnb), ct_t.stream);
}

void backend_fill_causal_mask(float *mask, int S) {
    require_init();
    ctk_causal_mask(mask, S, ct_t.stream);
}

void backend_lm_head(float *logits_out, const float *last, const uint16_t *etw, const uint16_t *hdb) {
    linear_epi(logits_out, last, etw, hdb, 1, DEC_D, VOCAB, CT_EPI_STORE, 0.0f);
}

/* ------------------------------------------------------------------ */
/* Graphs                                                              */
/* ------------------------------------------------------------------ */
void backend_upload_tokens(const int *host_tokens, int S) {
    if (S < 0 || S > MAX_SEQ) CT_FATAL("upload_tokens: S outside [0, MAX_SEQ]");
    require_init();
    put_ints(ct_t.d_tokens, host_tokens, S, 4);
    CHK(hipStreamSynchronize(ct_t.stream));
}

static CtGraph *graph_find(int tag, int T, int S, int B) {
    for (int i = 0; i < ct_t.n_graphs; i++) {
        CtGraph *e = &ct_t.graphs[i];
        if (e->tag == tag && e->T == T && e->S == S && e->B == B && e->arena == ct_t.arena) return e;
    }
    return NULL;
}

int backend_graph_replay(int tag, int T_enc, int S, int B) {
    require_init();
    CtGraph *e = graph_find(tag, T_enc, S, B);
    if (!e) return 0;
    CHK(hipGraphLaunch(e->exec, ct_t.stream));
    CHK(hipStreamSynchronize(ct_t.stream));
    return 1;
}

void backend_graph_begin_capture(int tag) {
    require_init();
    (void)tag;
    CHK(hipStreamBeginCapture(ct_t.stream, hipStreamCaptureModeThreadLocal));
}

void backend_graph_end_capture(int tag, int T_enc, int S, int B) {
    require_init();
    hipGraph_t graph;
    hipGraphExec_t exec;
    CHK(hipStreamEndCapture(ct_t.stream, &graph));
    CHK(hipGraphInstantiate(&exec, graph, NULL, NULL, 0));
    CHK(hipGraphLaunch(exec, ct_t.stream));
    CHK(hipStreamSynchronize(ct_t.stream));
    if (ct_t.n_graphs >= CT_GRAPH_CAP) {
        hipGraphExecDestroy(exec);
        hipGraphDestroy(graph);
        return;
    }
    if (ct_t.n_graphs == ct_t.graph_cap) {
        const int cap = ct_t.graph_cap ? 2 * ct_t.graph_cap : 16;
        CtGraph *ng = realloc(ct_t.graphs, (size_t)cap * sizeof *ng);
        if (!ng) CT_FATAL("out of host memory");
        ct_t.graphs = ng;
        ct_t.graph_cap = cap;
    }
    ct_t.graphs[ct_t.n_graphs++] = (CtGraph){tag, T_enc, S, B, ct_t.arena, graph, exec};
}

/* ------------------------------------------------------------------ */
/* Device-side counter, batch = 1                                      */
/* ------------------------------------------------------------------ */
void backend_decode_set_S(int n) {
    require_init();
    put_ints(ct_t.d_S, &n, 1, 0);
    CHK(hipStreamSynchronize(ct_t.stream));
}

void backend_decode_inc_S(void) {
    require_init();
    ctk_inc(ct_t.d_S, ct_t.stream);
}

void backend_linear_to_kvcache(float *cache, const float *x, const uint16_t *W, const uint16_t *b,
                               int in_d, int out_d) {
    require_init();
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.A = x; g.lda = in_d; g.W = CT_W(W); g.bias = CT_W(b);
    g.Y = cache; g.ldy = out_d; g.M = 1; g.N = out_d; g.K = in_d; g.epi = CT_EPI_STORE;
    g.row_len = ct_t.d_S; g.row_len_step = 0; g.row_stride = 0;
    ctk_gemm(&g, ct_t.stream);
}

void backend_sdp_attn_devS(float *out, const float *q, const float *k, const float *v, float *work) {
    (void)work;
    require_init();
    CtAttn a;
    attn_common(&a, out, q);
    a.K = k; a.V = v; a.lens = ct_t.d_S; a.T_q = 1; a.B = 1;
    ctk_attn(&a, ct_t.stream);
}

void backend_embed_decode(float *h, const uint16_t *etw, const uint16_t *epw,
                          const uint16_t *elnw, const uint16_t *elnb) {
    require_init();
    ctk_embed_ln(h, ct_t.d_tokens, 1, 0, ct_t.d_S, NULL, CT_W(etw), CT_W(epw),
                 CT_W(elnw), CT_W(elnb), ct_t.stream);
}

/* ------------------------------------------------------------------ */
/* Batched decode step                                                 */
/* ------------------------------------------------------------------ */
static void check_batch(int B) {
    if (B < 0 || B > CT_MAX_BATCH) CT_FATAL("batch size outside [0, 256]");
}

void backend_embed_decode_batch(float *h, const int *tokens, const int *S_dev, const int *active,
                                int B, const uint16_t *etw, const uint16_t *epw,
                                const uint16_t *elnw, const uint16_t *elnb) {
    check_batch(B);
    require_init();
    put_ints(ct_t.d_out, tokens, B, 0);
    put_ints(ct_t.d_S_batch, S_dev, B, 1);
    put_ints(ct_t.d_active, active, B, 2);
    ctk_embed_ln(h, ct_t.d_out, B, 0, ct_t.d_S_batch, ct_t.d_active, CT_W(etw), CT_W(epw),
                 CT_W(elnw), CT_W(elnb), ct_t.stream);
    CHK(hipStreamSynchronize(ct_t.stream));
}

void backend_lm_head_batch(float *logits, const float *h, const uint16_t *etw, const uint16_t *hdb,
                           const int *active, int B) {
    check_batch(B);
    require_init();
    put_ints(ct_t.d_active, active, B, 2);
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.A = h; g.lda = DEC_D; g.W = CT_W(etw); g.bias = CT_W(hdb);
    g.Y = logits; g.ldy = VOCAB; g.M = B; g.N = VOCAB; g.K = DEC_D; g.epi = CT_EPI_STORE;
    g.row_mask = ct_t.d_active;
    ctk_gemm(&g, ct_t.stream);
    CHK(hipStreamSynchronize(ct_t.stream));
}

void backend_argmax_batch(int *out, const float *logits, const int *active, int B) {
    check_batch(B);
    require_init();
    put_ints(ct_t.d_active, active, B, 2);
    ctk_argmax(ct_t.d_out, logits, B, VOCAB, ct_t.d_active, ct_t.stream);
    int *res = ct_t.h_stage + 3 * CT_MAX_BATCH;
    CHK(hipMemcpyAsync(res, ct_t.d_out, (size_t)B * sizeof(int), hipMemcpyDeviceToHost, ct_t.stream));
    CHK(hipStreamSynchronize(ct_t.stream));
    for (int b = 0; b < B; b++)
        if (active[b]) out[b] = res[b];
}

void backend_upload_T_enc(const int *T_enc, int B) {
    check_batch(B);
    require_init();
    put_ints(ct_t.d_T_enc, T_enc, B, 3);
    CHK(hipStreamSynchronize(ct_t.stream));
}

void backend_linear_to_kvcache_batch(float *cache, const float *x, const uint16_t *W,
                                     const uint16_t *b, int B, int cache_seq_stride,
                                     int in_d, int out_d) {
    check_batch(B);
    require_init();
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.A = x; g.lda = in_d; g.W = CT_W(W); g.bias = CT_W(b);
    g.Y = cache; g.ldy = out_d; g.M = B; g.N = out_d; g.K = in_d; g.epi = CT_EPI_STORE;
    g.row_len = ct_t.d_S_batch; g.row_len_step = 1; g.row_stride = cache_seq_stride;
    ctk_gemm(&g, ct_t.stream);
}

static void batch_attn(float *out, const float *Q, const float *K, const float *V,
                       int T_k_stride, int B, const int *lens) {
    check_batch(B);
    require_init();
    CtAttn a;
    attn_common(&a, out, Q);
    a.K = K; a.V = V; a.kv_sb = (long)T_k_stride * DEC_D;
    a.lens = lens; a.lens_step = 1; a.T_q = 1; a.B = B;
    ctk_attn(&a, ct_t.stream);
}

void backend_sdp_attn_batch_decode_sa(float *out, const float *Q, const float *K, const float *V,
                                      int T_k_stride, int B, float *work) {
    (void)work;
    batch_attn(out, Q, K, V, T_k_stride, B, ct_t.d_S_batch);
}

void backend_sdp_attn_batch_decode_ca(float *out, const float *Q, const float *K, const float *V,
                                      int T_k_stride, int B, float *work) {
    (void)work;
    batch_attn(out, Q, K, V, T_k_stride, B, ct_t.d_T_enc);
}
