/* oracle.h — CPU fp32 restatement of the reference's CPU backend and host
 * graph, used ONLY as the checker by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py.  Nothing in the product links it.
 *
 * Every function cites the reference lines it restates.  Loop order (one
 * sequential fp32 accumulation per output element, bias first) follows the
 * reference so that results agree with the compiled reference to rounding.
 * OpenMP only splits independent output elements, so results do not depend
 * on the thread count.
 */
#ifndef CT_ORACLE_H
#define CT_ORACLE_H

#include "../include/model_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernel-boundary functions (backends/cpu/backend.c) ---- */
void orc_layernorm(float *dst, const float *src, const uint16_t *w, const uint16_t *b,
                   int T, int D);
void orc_linear(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                int T, int in_d, int out_d);
void orc_linear_silu(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                     int T, int in_d, int out_d);
void orc_linear_relu(float *y, const float *x, const uint16_t *W, const uint16_t *b,
                     int T, int in_d, int out_d);
void orc_linear_fmadd(float *acc, float scale, const float *x, const uint16_t *W,
                      const uint16_t *b, int T, int in_d, int out_d);
void orc_add_inplace(float *dst, const float *src, int n);
size_t orc_subsampling_work_floats(int T_mel);
void orc_encoder_subsampling(const float *mel, int T_mel, int T_mel_stride,
                             float *x_enc, int T_enc, float *work, const Weights *W);
void orc_make_rel_pos_emb(float *pe, int T);
size_t orc_mhsa_work_floats(int T);
void orc_rel_pos_mhsa(float *x, const float *pos_emb, int T, const ELayer *L, float *work);
size_t orc_conv_work_floats(int T);
void orc_conformer_conv(float *x, int T, const ELayer *L, float *work);
void orc_sdp_attn(float *out, const float *q, const float *k, const float *v,
                  const float *mask, int T_q, int T_k, float *work);
void orc_embed(float *h, const int *tokens, int S, int pos_start,
               const uint16_t *etw, const uint16_t *epw,
               const uint16_t *elnw, const uint16_t *elnb);
void orc_fill_causal_mask(float *mask, int S);
void orc_lm_head(float *logits, const float *last, const uint16_t *etw, const uint16_t *hdb);
/* First index of the maximum over n values; with skip >= 0 that index is
 * excluded (EOS suppression).  Strict '>' as backends/cpu/backend.c:450-454. */
int  orc_argmax(const float *x, int n, int skip);

/* ---- graph level (model.h) ---- */
int  orc_T_enc(int T_mel);
void orc_conformer_layer(float *x, const float *pos_emb, int T, const ELayer *L, float *work);
/* 1: round the inputs of the encoder FFN linears to bf16 (the single-pass
 * precision mode of the HIP encoder); 0 (default): fp32 as the reference. */
void orc_set_enc_ffn_bf16(int on);
/* mel (N_MELS, T_mel) with row stride T_mel_stride -> enc_h (T_enc, DEC_D). */
void orc_encoder_forward(const float *mel, int T_mel, int T_mel_stride,
                         const Weights *W, float *x_enc_out, float *enc_h);
/* ca_k / ca_v: [DEC_N][T_enc][DEC_D]. */
void orc_cross_kv(const float *enc_h, int T_enc, const Weights *W, float *ca_k, float *ca_v);

/* Decode-state of one sequence: self K/V caches [DEC_N][MAX_SEQ][DEC_D] and
 * the cross K/V from orc_cross_kv. */
typedef struct {
    float *sk, *sv;           /* self caches, owned */
    const float *ck, *cv;     /* cross K/V, borrowed */
    int T_enc;
    int S;                    /* tokens already in the self cache */
    int kv_bf16;              /* round K/V to bf16 when cached (bf16-KV mode) */
} OrcSeq;
void orc_round_bf16_n(float *x, long n);
void orc_seq_init(OrcSeq *s, const float *ca_k, const float *ca_v, int T_enc, int kv_bf16);
void orc_seq_free(OrcSeq *s);
/* Feeds S_q new tokens at positions s->S .. s->S+S_q-1 through the decoder
 * (model.h:376-409 / 461-503), causal within the new rows, then writes the
 * logits of the LAST new row.  h_last (DEC_D) receives the final-LN hidden. */
void orc_seq_step(OrcSeq *s, const Weights *W, const int *tokens, int S_q,
                  float *logits, float *h_last);

/* Whole request: encoder, cross K/V, prompt prefill, greedy decode.
 * Policy: at most `limit` generated tokens; suppress_eos excludes EOS from the
 * argmax; force_eos makes token number `limit` EOS; without either the loop
 * stops at EOS (transcribe.c:789).  Returns the number generated.
 * logits_out (optional): [limit][VOCAB] per generated token. */
int  orc_transcribe(const Weights *W, const float *mel, int T_mel, int T_mel_stride,
                    const int *prompt, int n_prompt, int limit,
                    int suppress_eos, int force_eos, int kv_bf16,
                    int *tokens_out, float *logits_out, float *enc_h_out);

/* ---- host front-end (transcribe.c:45-214) ---- */
int  orc_T_mel(int n_samples);
void orc_compute_mel(const float *samples, int n, float *mel /* N_MELS x T_mel */);
void orc_mel_filterbank(float *fb /* N_MELS x N_BINS */);

/* ---- long-audio chunking (transcribe.c:397-535) ---- */
/* Chunk i is samples [bounds[2i], bounds[2i+1]); returns the chunk count
 * (at most cap).  silence_db NAN: automatic threshold. */
int  orc_chunk_bounds(const float *samples, int n_samples, float silence_db, float silence_dur,
                      float target_sec, int *bounds, int cap);

#ifdef __cplusplus
}
#endif
#endif
