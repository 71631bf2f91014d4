/* backend.h — the 40-function compute-backend ABI, as exported by the MI355X
 * HIP backend (libct_hip.so).
 *
 * Every prototype below replaces the declaration at the cited line of the
 * reference's backends/backend.h; names, argument order and meaning are the
 * ABI and are kept identical so the unmodified host (transcribe.c, model.h,
 * tests/test_kernels.c) links against this backend.  Contract notes that the
 * reference leaves implicit are stated here.
 *
 * Conventions (all functions):
 *  - Activations are fp32 device pointers carved by the caller out of the
 *    arena returned by backend_arena_alloc.
 *  - Weight pointers are bf16 and point INTO THE HOST blob passed to
 *    backend_weights_upload_blob; the backend translates them by offset.
 *    A non-NULL weight pointer outside that blob is a fatal error.
 *  - Host arrays (tokens, S_dev, active, T_enc, argmax out) are host memory.
 *  - Compute calls are asynchronous on the calling thread's stream; htod,
 *    dtoh, arena_free and argmax_batch synchronise.
 *  - All mutable state is thread-local: each thread calls backend_init(dev)
 *    and, before exiting, backend_thread_cleanup().
 *  - Errors print a message to stderr and exit(1); nothing returns codes.
 */
#ifndef CT_BACKEND_H
#define CT_BACKEND_H

#include "model_types.h"
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Lifecycle (backends/backend.h:20-30) ---- */
void  backend_init(int device_id);                        /* backend.h:20 */
void  backend_destroy(void);                              /* backend.h:21 */
int   backend_num_devices(void);                          /* backend.h:25 */
void  backend_thread_cleanup(void);                       /* backend.h:30 */

/* ---- Weights and memory (backends/backend.h:34-46) ---- */
void  backend_weights_upload_blob(const void *host_base, size_t bytes);  /* :34 */
void *backend_device_ptr(const void *host_ptr);           /* backend.h:38 */
float *backend_arena_alloc(size_t floats);                /* backend.h:41 */
void   backend_arena_free(float *arena);                  /* backend.h:42 */
void backend_htod(float *dev_dst, const float *host_src, size_t floats);  /* :45 */
void backend_dtoh(void *host_dst, const void *dev_src, size_t bytes);     /* :46 */

/* ---- Dense ops (backends/backend.h:52-67) ---- */
void backend_layernorm(float *dst, const float *src,
                       const uint16_t *w, const uint16_t *b, int T, int D);     /* :52 */
void backend_linear(float *y, const float *x,
                    const uint16_t *W, const uint16_t *b, int T, int in_d, int out_d); /* :56 */
void backend_linear_silu(float *y, const float *x,
                         const uint16_t *W, const uint16_t *b, int T, int in_d, int out_d); /* :58 */
void backend_linear_relu(float *y, const float *x,
                         const uint16_t *W, const uint16_t *b, int T, int in_d, int out_d); /* :60 */
/* acc[t] += scale * (W x[t] + b) */
void backend_linear_fmadd(float *acc, float scale, const float *x,
                          const uint16_t *W, const uint16_t *b, int T, int in_d, int out_d); /* :63 */
void backend_add_inplace(float *dst, const float *src, int n);                   /* :67 */

/* ---- Encoder (backends/backend.h:72-86) ---- */
/* mel is (N_MELS, T_mel) with row stride T_mel_stride; writes x_enc (T_enc, ENC_D). */
void backend_encoder_subsampling(const float *mel, int T_mel, int T_mel_stride,
                                 float *x_enc, int T_enc, float *work,
                                 const Weights *W);                               /* :72 */
/* (2T-1, ENC_D) sinusoid table, row p is relative position T-1-p. */
void backend_make_rel_pos_emb(float *pe, int T);                                 /* :77 */
/* x (T, ENC_D) in place: x <- MHSA_relpos(x). */
void backend_rel_pos_mhsa(float *x, const float *pos_emb,
                          int T, const ELayer *L, float *work);                  /* :81 */
/* x (T, ENC_D) in place: pw1 -> GLU -> depthwise(9) -> BN -> SiLU -> pw2. */
void backend_conformer_conv(float *x, int T, const ELayer *L, float *work);     /* :86 */

/* ---- Decoder, prefill / single (backends/backend.h:90-106) ---- */
void backend_sdp_attn(float *out, const float *q, const float *k, const float *v,
                      const float *mask, int T_q, int T_k, float *work);          /* :90 */
void backend_embed(float *h, const int *tokens, int S, int pos_start,
                   const uint16_t *etw, const uint16_t *epw,
                   const uint16_t *elnw, const uint16_t *elnb);                  /* :96 */
void backend_fill_causal_mask(float *mask, int S);                               /* :101 */
void backend_lm_head(float *logits_out, const float *last,
                     const uint16_t *etw, const uint16_t *hdb);                  /* :105 */

/* ---- Graph capture / replay (backends/backend.h:113-138) ---- */
#define GRAPH_TAG_ENCODER    0
#define GRAPH_TAG_PRECOMPUTE 1
#define GRAPH_TAG_DECODER    2
void backend_upload_tokens(const int *host_tokens, int S);                       /* :121 */
/* Replays the graph cached under (tag, T_enc, S, B, current arena); returns 1
 * if one ran, 0 if the caller must run and capture the region. */
int  backend_graph_replay(int tag, int T_enc, int S, int B);                     /* :128 */
void backend_graph_begin_capture(int tag);                                       /* :133 */
/* Instantiates, caches and launches the captured region once. */
void backend_graph_end_capture(int tag, int T_enc, int S, int B);               /* :138 */

/* ---- Device-side sequence counter, batch = 1 (backends/backend.h:147-175) ---- */
void backend_decode_set_S(int n);                                                /* :147 */
void backend_decode_inc_S(void);                                                 /* :152 */
/* cache[(*S - 1) * out_d + j] = (W x + b)[j] */
void backend_linear_to_kvcache(float *cache, const float *x,
                               const uint16_t *W, const uint16_t *b,
                               int in_d, int out_d);                             /* :159 */
/* T_q = 1, T_k = *S, no mask. */
void backend_sdp_attn_devS(float *out, const float *q,
                           const float *k, const float *v, float *work);         /* :166 */
/* Embeds the staged token at position *S - 1, then layer-norms. */
void backend_embed_decode(float *h,
                          const uint16_t *etw, const uint16_t *epw,
                          const uint16_t *elnw, const uint16_t *elnb);           /* :173 */

/* ---- Batched decode step (backends/backend.h:185-228) ---- */
/* Latches S_dev[0..B) as the per-item self-attention lengths used by
 * linear_to_kvcache_batch and sdp_attn_batch_decode_sa.  Rows of inactive
 * items are left unchanged. */
void backend_embed_decode_batch(float *h, const int *tokens,
                                const int *S_dev, const int *active, int B,
                                const uint16_t *etw, const uint16_t *epw,
                                const uint16_t *elnw, const uint16_t *elnb);     /* :185 */
void backend_lm_head_batch(float *logits, const float *h,
                           const uint16_t *etw, const uint16_t *hdb,
                           const int *active, int B);                            /* :192 */
/* First index of the maximum (ties -> lowest id) for each active row; out[b]
 * of inactive rows is left unchanged. */
void backend_argmax_batch(int *out, const float *logits,
                          const int *active, int B);                             /* :198 */
void backend_upload_T_enc(const int *T_enc, int B);                              /* :207 */
void backend_linear_to_kvcache_batch(float *cache, const float *x,
                                     const uint16_t *W, const uint16_t *b,
                                     int B, int cache_seq_stride,
                                     int in_d, int out_d);                       /* :214 */
void backend_sdp_attn_batch_decode_sa(float *out, const float *Q,
                                      const float *K, const float *V,
                                      int T_k_stride, int B, float *work);       /* :223 */
void backend_sdp_attn_batch_decode_ca(float *out, const float *Q,
                                      const float *K, const float *V,
                                      int T_k_stride, int B, float *work);       /* :226 */

/* ---- Beyond the reference ABI ------------------------------------------ */
/* backend_rel_pos_mhsa without the workspace argument, for callers that
 * cannot allocate device memory (code under graph capture, serving loops,
 * harnesses that forbid allocation).  It has no counterpart in the
 * reference.  Its scratch (Q, K, V, P, O: (6T - 1) x ENC_D floats) is a
 * static device array of 11.5 MB per device, held until the process ends,
 * so T must be at most 376 frames (a 30 s clip); larger T prints an error
 * and exits.  Allocates nothing.  Every call on one device uses the same
 * scratch: calls that overlap on one device (other threads, other streams)
 * race.  Same results, bit for bit, as backend_rel_pos_mhsa. */
void backend_rel_pos_mhsa_noalloc(float *x, const float *pos_emb, int T, const ELayer *L);

#ifdef __cplusplus
}
#endif

#endif /* CT_BACKEND_H */
