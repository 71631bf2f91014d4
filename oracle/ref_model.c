/* ref_model.c — harness around the reference's own host graph (model.h).
 *
 * Compiled by oracle/Makefile together with the reference sources where they
 * lie.  Linked with the reference CPU backend it writes golden fixtures
 * (oracle/_ref/libref_model.so); linked with this repository's HIP backend
 * (oracle/_ref/libref_model_hip.so) it is the unmodified reference host
 * driving the drop-in backend through the 40-function ABI.
 *
 * All buffers come from backend_arena_alloc and move with backend_htod /
 * backend_dtoh, as in transcribe.c, so the same code drives a host or a device
 * backend.  The drivers follow transcribe_chunk (transcribe.c:264-390) and
 * transcribe_batch (transcribe.c:572-808) but take mel spectrograms directly
 * (no ffmpeg) and add the forced-length policy the benchmark configurations
 * use: EOS can be excluded from the argmax and token number `limit` can be
 * forced to EOS.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int verbose = 0;
#include "model.h"

#define EOS_ID TOK_EOS

void ref_set_weights(const Weights *w) { memcpy(&W, w, sizeof W); }

static int T_enc_of(int T_mel) {
    const int a = (T_mel + 1) / 2, b = (a + 1) / 2;
    return (b + 1) / 2;
}

/* Scratch sized as transcribe.c:274-304 computes it. */
static size_t work_floats(int T_mel) {
    const size_t T1 = (T_mel + 1) / 2, T2 = (T1 + 1) / 2, T = T_enc_of(T_mel);
    const size_t sub = (size_t)SUB_CH * (T1 * 64 + T2 * 32);
    const size_t sc = T * (3 * T - 1), at = 2 * T * ENC_D;
    const size_t mh = T * ENC_FF + T * ENC_D + (5 * T - 1) * ENC_D + (sc > at ? sc : at);
    const size_t cv = T * (ENC_FF + 4 * ENC_D);
    const size_t dec = (size_t)5 * MAX_SEQ * DEC_D + (size_t)MAX_SEQ * MAX_SEQ;
    size_t w = sub;
    if (mh > w) w = mh;
    if (cv > w) w = cv;
    if (dec > w) w = dec;
    return w;
}

/* per thread, as transcribe.c's workers each hold their own backend state */
static _Thread_local float *g_base;
static _Thread_local size_t g_off, g_cap;
static void arena_begin(size_t floats) {
    g_base = backend_arena_alloc(floats);
    g_cap = floats;
    g_off = 0;
}
static float *take(size_t n) {
    n = (n + 63) & ~(size_t)63;
    if (g_off + n > g_cap) { fputs("ref harness: arena too small\n", stderr); exit(1); }
    float *p = g_base + g_off;
    g_off += n;
    return p;
}

static int pick(const float *dev_logits, int suppress) {
    float *lg = malloc(VOCAB * sizeof(float));
    backend_dtoh(lg, dev_logits, VOCAB * sizeof(float));
    int best = -1;
    float bv = 0.0f;
    for (int v = 0; v < VOCAB; v++) {
        if (suppress && v == EOS_ID) continue;
        if (best < 0 || lg[v] > bv) { bv = lg[v]; best = v; }
    }
    free(lg);
    return best;
}

void ref_encoder(const float *mel, int T_mel, float *enc_h_out) {
    const int T = T_enc_of(T_mel);
    arena_begin((size_t)N_MELS * T_mel + (size_t)T * ENC_D + (size_t)(2 * T - 1) * ENC_D
                + (size_t)T * DEC_D + work_floats(T_mel) + 4096);
    float *m = take((size_t)N_MELS * T_mel), *x = take((size_t)T * ENC_D);
    float *pe = take((size_t)(2 * T - 1) * ENC_D), *eh = take((size_t)T * DEC_D);
    float *work = take(work_floats(T_mel));
    backend_htod(m, mel, (size_t)N_MELS * T_mel);
    encoder_forward(m, T_mel, x, T, pe, eh, work);
    backend_dtoh(enc_h_out, eh, (size_t)T * DEC_D * sizeof(float));
    backend_arena_free(g_base);
}

/* Single-sequence path (transcribe_chunk).  Returns tokens generated.
 * logits_out (optional): [limit][VOCAB]; enc_h_out (optional): [T_enc][DEC_D]. */
int ref_transcribe_single(const float *mel, int T_mel, const int *prompt, int n_prompt,
                          int limit, int suppress, int force, int *tokens_out,
                          float *logits_out, float *enc_h_out) {
    const int T = T_enc_of(T_mel);
    arena_begin((size_t)N_MELS * T_mel + (size_t)T * ENC_D + (size_t)(2 * T - 1) * ENC_D
                + (size_t)T * DEC_D + 2 * (size_t)DEC_N * T * DEC_D
                + 2 * (size_t)DEC_N * MAX_SEQ * DEC_D + 2 * (size_t)MAX_SEQ * DEC_D
                + (size_t)MAX_SEQ * MAX_SEQ + work_floats(T_mel) + 65536);
    float *m = take((size_t)N_MELS * T_mel), *x = take((size_t)T * ENC_D);
    float *pe = take((size_t)(2 * T - 1) * ENC_D), *eh = take((size_t)T * DEC_D);
    float *ck[DEC_N], *cv[DEC_N], *sk[DEC_N], *sv[DEC_N];
    for (int l = 0; l < DEC_N; l++) { ck[l] = take((size_t)T * DEC_D); cv[l] = take((size_t)T * DEC_D); }
    for (int l = 0; l < DEC_N; l++) { sk[l] = take((size_t)MAX_SEQ * DEC_D); sv[l] = take((size_t)MAX_SEQ * DEC_D); }
    float *h = take((size_t)MAX_SEQ * DEC_D), *mask = take((size_t)MAX_SEQ * MAX_SEQ);
    float *work = take(work_floats(T_mel));
    backend_htod(m, mel, (size_t)N_MELS * T_mel);
    encoder_forward(m, T_mel, x, T, pe, eh, work);
    if (enc_h_out) backend_dtoh(enc_h_out, eh, (size_t)T * DEC_D * sizeof(float));
    precompute_ca_kv(eh, T_mel, T, ck, cv);
    int toks[MAX_SEQ], S = 0, ng = 0;
    for (int i = 0; i < n_prompt; i++) toks[S++] = prompt[i];
    backend_decode_set_S(S);
    for (;;) {
        int id;
        if (ng == 0) id = decoder_step(toks, S, S, T_mel, T, ck, cv, sk, sv, h, mask, work);
        else id = decoder_step_decode(toks[S - 1], T_mel, T, ck, cv, sk, sv, h, work);
        /* the logits are at work[0 .. VOCAB) (model.h:466, 518) */
        if (logits_out) backend_dtoh(logits_out + (size_t)ng * VOCAB, work, VOCAB * sizeof(float));
        if (force && ng == limit - 1) id = EOS_ID;
        else if (suppress && id == EOS_ID) id = pick(work, 1);
        toks[S++] = id;
        tokens_out[ng++] = id;
        if (id == EOS_ID && !suppress) break;
        if (ng >= limit || S >= MAX_SEQ) break;
    }
    backend_arena_free(g_base);
    return ng;
}

/* Batched ragged path (transcribe_batch, count > 1).
 * mel_batch: host [B][N_MELS][T_mel_max]; tokens_out: [B][max_limit];
 * n_out[b]: tokens generated; enc_h_out (optional): [B][T_enc_max][DEC_D]. */
void ref_transcribe_batch(const float *mel_batch, int B, const int *T_mel, int T_mel_max,
                          const int *prompt, int n_prompt, const int *limit,
                          int suppress, int force, int max_limit,
                          int *tokens_out, int *n_out, float *enc_h_out) {
    int *Te = malloc(B * sizeof(int));
    for (int b = 0; b < B; b++) Te[b] = T_enc_of(T_mel[b]);
    const int TeM = T_enc_of(T_mel_max);
    const size_t wk = work_floats(T_mel_max) + (size_t)B * (3 * DEC_D + DEC_H * MAX_SEQ);
    arena_begin((size_t)B * N_MELS * T_mel_max + (size_t)B * TeM * ENC_D
                + (size_t)(2 * TeM - 1) * ENC_D + (size_t)B * TeM * DEC_D
                + 2 * (size_t)DEC_N * B * TeM * DEC_D + 2 * (size_t)DEC_N * B * MAX_SEQ * DEC_D
                + (size_t)MAX_SEQ * DEC_D + (size_t)MAX_SEQ * MAX_SEQ
                + (size_t)B * VOCAB + (size_t)B * DEC_D + wk + 65536);
    float *mb = take((size_t)B * N_MELS * T_mel_max), *x = take((size_t)B * TeM * ENC_D);
    float *pe = take((size_t)(2 * TeM - 1) * ENC_D), *eh = take((size_t)B * TeM * DEC_D);
    float *ck[DEC_N], *cv[DEC_N], *sk[DEC_N], *sv[DEC_N];
    for (int l = 0; l < DEC_N; l++) { ck[l] = take((size_t)B * TeM * DEC_D); cv[l] = take((size_t)B * TeM * DEC_D); }
    for (int l = 0; l < DEC_N; l++) { sk[l] = take((size_t)B * MAX_SEQ * DEC_D); sv[l] = take((size_t)B * MAX_SEQ * DEC_D); }
    float *h = take((size_t)MAX_SEQ * DEC_D), *mask = take((size_t)MAX_SEQ * MAX_SEQ);
    float *lgb = take((size_t)B * VOCAB), *hb = take((size_t)B * DEC_D), *work = take(wk);
    backend_htod(mb, mel_batch, (size_t)B * N_MELS * T_mel_max);
    encoder_forward_batch(mb, B, T_mel_max, T_mel, Te, TeM, x, pe, eh, work);
    if (enc_h_out) backend_dtoh(enc_h_out, eh, (size_t)B * TeM * DEC_D * sizeof(float));
    precompute_ca_kv_batch(eh, B, Te, TeM, ck, cv);
    int *toks = malloc((size_t)B * MAX_SEQ * sizeof(int));
    int *S = malloc(B * sizeof(int)), *Sd = malloc(B * sizeof(int)), *act = malloc(B * sizeof(int));
    int *cur = malloc(B * sizeof(int)), *nxt = malloc(B * sizeof(int));
    for (int b = 0; b < B; b++) {
        int *tb = toks + (size_t)b * MAX_SEQ;
        for (int i = 0; i < n_prompt; i++) tb[i] = prompt[i];
        S[b] = n_prompt;
        float *ckb[DEC_N], *cvb[DEC_N], *skb[DEC_N], *svb[DEC_N];
        for (int l = 0; l < DEC_N; l++) {
            ckb[l] = ck[l] + (size_t)b * TeM * DEC_D; cvb[l] = cv[l] + (size_t)b * TeM * DEC_D;
            skb[l] = sk[l] + (size_t)b * MAX_SEQ * DEC_D; svb[l] = sv[l] + (size_t)b * MAX_SEQ * DEC_D;
        }
        backend_decode_set_S(n_prompt);
        int id = decoder_step(tb, S[b], S[b], T_mel[b] + (b + 1) * 100000, Te[b],
                              ckb, cvb, skb, svb, h, mask, work);
        if (force && limit[b] == 1) id = EOS_ID;
        else if (suppress && id == EOS_ID) id = pick(work, 1);
        tb[S[b]++] = id;
        tokens_out[(size_t)b * max_limit] = id;
        n_out[b] = 1;
    }
    backend_upload_T_enc(Te, B);
    int n_act = 0;
    for (int b = 0; b < B; b++) {
        const int last = toks[(size_t)b * MAX_SEQ + S[b] - 1];
        act[b] = !(last == EOS_ID && !suppress) && n_out[b] < limit[b] && S[b] < MAX_SEQ;
        n_act += act[b];
        Sd[b] = S[b] - 1;
    }
    while (n_act > 0) {
        for (int b = 0; b < B; b++) cur[b] = act[b] ? toks[(size_t)b * MAX_SEQ + S[b] - 1] : 0;
        for (int b = 0; b < B; b++) if (act[b]) Sd[b]++;
        decoder_step_decode_batch(cur, Sd, act, TeM, ck, cv, sk, sv, hb, lgb, work, B, nxt);
        for (int b = 0; b < B; b++) {
            if (!act[b]) continue;
            int id = nxt[b];
            if (force && n_out[b] == limit[b] - 1) id = EOS_ID;
            else if (suppress && id == EOS_ID) id = pick(lgb + (size_t)b * VOCAB, 1);
            toks[(size_t)b * MAX_SEQ + S[b]++] = id;
            tokens_out[(size_t)b * max_limit + n_out[b]++] = id;
            if ((id == EOS_ID && !suppress) || n_out[b] >= limit[b] || S[b] >= MAX_SEQ) {
                act[b] = 0; n_act--;
            }
        }
    }
    backend_arena_free(g_base);
    free(toks); free(S); free(Sd); free(act); free(cur); free(nxt); free(Te);
}

/* ------------------------------------------------------------------ */
/* Timing support for the CPU baseline: pieces of the reference's own  */
/* host graph, run on whatever backend this file is linked with.       */
/* ------------------------------------------------------------------ */

/* n_layers Conformer layers (model.h conformer_layer, layers 0..n-1) over
 * T frames: x_io [T][ENC_D] in, out. */
void ref_encoder_layers(float *x_io, int T, int n_layers) {
    const int T_mel = 8 * T;           /* any T_mel whose T_enc is T sizes the scratch */
    arena_begin((size_t)T * ENC_D + (size_t)(2 * T - 1) * ENC_D + work_floats(T_mel) + 4096);
    float *x = take((size_t)T * ENC_D), *pe = take((size_t)(2 * T - 1) * ENC_D);
    float *work = take(work_floats(T_mel));
    backend_htod(x, x_io, (size_t)T * ENC_D);
    backend_make_rel_pos_emb(pe, T);
    for (int l = 0; l < n_layers; l++) conformer_layer(x, pe, T, &W.enc[l % ENC_N], work);
    backend_dtoh(x_io, x, (size_t)T * ENC_D * sizeof(float));
    backend_arena_free(g_base);
}

/* n_steps single-sequence decode steps (model.h decoder_step_decode) from
 * S0 tokens already in the self caches, over T_enc frames of cross K/V; the
 * caches hold a fixed pattern.  Returns the last token id. */
int ref_decode_steps(int T_enc, int S0, int n_steps) {
    const int T_mel = 8 * T_enc;
    arena_begin(2 * (size_t)DEC_N * T_enc * DEC_D + 2 * (size_t)DEC_N * MAX_SEQ * DEC_D
                + (size_t)MAX_SEQ * DEC_D + work_floats(T_mel) + 65536);
    float *ck[DEC_N], *cv[DEC_N], *sk[DEC_N], *sv[DEC_N];
    for (int l = 0; l < DEC_N; l++) { ck[l] = take((size_t)T_enc * DEC_D); cv[l] = take((size_t)T_enc * DEC_D); }
    for (int l = 0; l < DEC_N; l++) { sk[l] = take((size_t)MAX_SEQ * DEC_D); sv[l] = take((size_t)MAX_SEQ * DEC_D); }
    float *h = take((size_t)MAX_SEQ * DEC_D), *work = take(work_floats(T_mel));
    const size_t nfill = (size_t)(MAX_SEQ > T_enc ? MAX_SEQ : T_enc) * DEC_D;
    float *pat = malloc(nfill * sizeof(float));
    for (size_t i = 0; i < nfill; i++) pat[i] = (float)((int)(i * 2654435761u >> 20) % 201 - 100) * 1e-3f;
    for (int l = 0; l < DEC_N; l++) {
        backend_htod(ck[l], pat, (size_t)T_enc * DEC_D);
        backend_htod(cv[l], pat, (size_t)T_enc * DEC_D);
        backend_htod(sk[l], pat, (size_t)MAX_SEQ * DEC_D);
        backend_htod(sv[l], pat, (size_t)MAX_SEQ * DEC_D);
    }
    free(pat);
    backend_decode_set_S(S0);
    int id = 100;
    for (int i = 0; i < n_steps; i++) id = decoder_step_decode(id, T_mel, T_enc, ck, cv, sk, sv, h, work);
    backend_arena_free(g_base);
    return id;
}
