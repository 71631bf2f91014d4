/* engine.c — the hipb_* decode engine (include/hipb.h), host side.
 *
 * Owns the device state of a continuous-batching transcription run: the
 * request pool (encoder output, cross-attention K/V per request), the slot
 * table and self-attention KV caches per slot, activations for one step over
 * all slots, and a captured hipGraph of that step.  A step is
 *   eng_begin -> embed+LN -> 8 x [LN, QKV GEMM (+KV append), self attention,
 *   out-proj (+residual), LN, Q GEMM, cross attention, out-proj (+residual),
 *   LN, FFN up (ReLU), FFN down (+residual)] -> LN -> LM head -> eng_end,
 * the per-item loop of model.h:666-744 with every slot processed at once.
 * The encoder runs packed: all frames of a batch of requests form the rows
 * of one GEMM (model.h:573-635 per item, here M = sum of frames).
 */
#include "../../include/backend.h"
#include "../../include/hipb.h"
#include "ct_abi_state.h"
#include "ct_engine.h"
#include "ct_launch.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

typedef struct {
    float *mel;          /* host copy until encoded (mel requests) ...        */
    float *pcm;          /* ... or the 16 kHz samples (PCM requests) ...      */
    const float *dpcm;   /* ... or samples already in device memory          */
    int n;               /* samples of a PCM request                          */
    int T_mel, T_enc;
    int chained;         /* admitted only after its predecessor chunk ends    */
    int entry;           /* encoder-state entry once encoded, else -1         */
    int limit;           /* token budget                                      */
    int done;            /* seen retired by the host (recycle)                */
    /* results copied to the host when its request-ring slot was reused */
    int collected, n_out;
    int *out;
    float *score;
} HostReq;

struct HipbEngine {
    HipbConfig cfg;
    Weights W;
    hipStream_t s;
    int dev;
    int esz;             /* KV element size */
    CtEngDev d;
    /* repacked weights: [Wq;Wk;Wv] per layer, [Wk;Wv] cross per layer */
    uint16_t *wqkv, *bqkv, *wckv, *bckv;
    /* encoder self-attention [Wq;Wk;Wv] (3*ENC_D x ENC_D) and biases per
     * layer: one GEMM launch for the three projections */
    uint16_t *ew_qkv, *eb_qkv;
    /* decode-GEMM weights in the tile layout (ctk_tile_w), one allocation:
     * per layer [Wq;Wk;Wv], Wo, Wq_cross, Wo_cross, W_ffn1, W_ffn2; then the
     * tied LM head */
    uint16_t *wtile;
    const uint16_t *wt_qkv[DEC_N], *wt_o[DEC_N], *wt_cq[DEC_N], *wt_co[DEC_N], *wt_f1[DEC_N],
        *wt_f2[DEC_N], *wt_lm;
    /* caches */
    void *kself, *vself;       /* [L][slots][H][kv_rows][128] */
    void *kcross, *vcross;     /* [L][entries][H][tmax][128] */
    float *enc_pool;           /* encoder outputs, [entries][tmax][DEC_D] */
    /* encoder-state entries (cross K/V + encoder output, max_requests of
     * them): a FIFO of free ones (free_ent[i % entries] for i in
     * [free_head, free_tail)), the request holding each, and the retired
     * requests already recycled; the encoder thread of hipb_process takes
     * entries while the decode loop returns them, under mu/cv */
    int *free_ent, *ent_owner;
    long free_head, free_tail;
    int ret_seen;
    int *h_ret;                /* pinned: retired ids read back */
    pthread_mutex_t mu;
    pthread_cond_t cv;
    atomic_int n_assigned;     /* requests [0, n_assigned) have entries */
    atomic_int stop;           /* hipb_process ends: the encoder thread quits its wait */
    /* step activations: h residual rows (fp32); lnf/attf/midf the decode
     * GEMMs' inputs in frag layout (lnf holds h * w, the input of the next
     * GEMM with its LayerNorm folded in, or the final LayerNorm's output);
     * parts the FFN down projection's K-slice partial sums; lnstat the rows'
     * statistics per 32-column block, left with lnf for that GEMM */
    float *h, *q, *parts, *logits, *lnstat;
    /* folded LayerNorms: per layer the c1 / c2 column constants of the QKV,
     * cross-query and FFN-up GEMMs (ctk_fold_cols) */
    float *fold;
    const float *fc_qkv[DEC_N][2], *fc_cq[DEC_N][2], *fc_f1[DEC_N][2];
    int M;                     /* rows of the step being launched */
    /* decode GEMMs whose weight tiles the next attention launch reads ahead
     * into the L2 their workgroups will read from */
    CtWarmSet warm;
    unsigned *warm_sink;
    /* hipb_bench_read_floor: decode GEMM launches replaced by their weight
     * reads alone, one value per workgroup to floor_sink */
    int bench_floor;
    float *floor_sink;
    long floor_cap;
    /* encoder side: its stream (the engine stream, or a second stream while
     * hipb_process overlaps encoding with decoding), pinned staging of its
     * own, and the host count of requests published to the fresh queue */
    hipStream_t s2, enc_s;
    int *h_enc;
    int fq_count;
    int proc_batch;            /* encoder batch frames of hipb_process */
    int batch_frames;          /* encoder batch frames of the last hipb_encode */
    atomic_int enc_done;       /* the encoder thread has published every batch */
    atomic_int published;      /* encoded watermark last published (q[7]) */
    /* test support (hipb_test_hold_encoder): after publishing hold_batches
     * batches the encoder thread waits until the decode loop has seen
     * hold_finished requests finish */
    int hold_batches, hold_finished, hold_expired;
    atomic_int seen_finished;
    uint16_t *lnf, *attf, *midf;
    /* encoder workspace (lazy) */
    int enc_cap;               /* frames */
    int sub_cap;               /* subsampling scratch floats */
    int *e_subtab;             /* packed subsampling group tables */
    float *ex, *eln, *emid, *eq, *ek, *ev, *eo, *eg, *edw, *epe, *esub, *emel;
    /* relative-position projections of every layer for clips of up to tmax
     * frames, [ENC_N][2 tmax - 1][ENC_D], built once: a clip of T frames
     * reads rows tmax - T .. tmax + T - 2 */
    float *ep_all;
    uint16_t *eln_h, *eln_l, *emid_h, *emid_l, *eo_h, *eo_l, *edw_h, *edw_l;  /* pre-split GEMM inputs */
    size_t emel_cap;
    int *e_row_start, *e_row_len, *e_seq_off, *e_seq_T, *e_blk_seq, *e_blk_q0;
    int *e_dstrow;             /* encoder-output row of each packed row */
    long *e_rowoff;
    /* requests: host records grow with submissions; device fields live in
     * rings of `ring` slots (id & (ring - 1)) */
    HostReq *req;
    int req_cap, ring;
    int n_req, n_enc;          /* submitted; encoded (the first n_enc of order) */
    int *order;                /* [req_cap] encode order: ids by position      */
    int n_pub;                 /* publications so far (q[7])                   */
    int *d_pairs;              /* device staging of (id, entry) pairs          */
    int *h_tmp;                /* pinned staging */
    /* request fields as submitted (pinned): length, limit, flags, prompt
     * length, successor, then the prompts; requests [meta_lo, n_req) are
     * not on the device yet (flush_meta) */
    int *h_meta;
    int meta_lo;
    /* graph */
    hipGraph_t graph[2];       /* [0] slots rows, [1] with the spare prompt rows */
    hipGraphExec_t exec[2];
    int have_graph[2];
    int eager;           /* HIPB_EAGER=1: launch steps without a graph */
    int read_ahead;      /* HIPB_READ_AHEAD=0: no weight read-ahead rows */
    int bench_mode;
    int bench_gemm_M;    /* rows seeded by hipb_bench_encoder_gemm */
    /* log-mel front-end */
    CtMelTables mel_tab;
    float *d_hann, *d_twr, *d_twi, *d_fb;
    int *d_fb_lo, *d_fb_hi;
    float *epcm;
    size_t epcm_cap;
    CtMelClip *e_clips;
    int *e_frame_clip;
    int clips_cap, frames_cap;
};

#define ECHK(x) ct_hip_check((x), #x, __FILE__, __LINE__)
#define CT_META_FIELDS 7   /* request fields mirrored on the host (meta_field) */

static void *dmalloc(size_t bytes) {
    void *p = NULL;
    ECHK(hipMalloc(&p, bytes ? bytes : 16));
    return p;
}

static const uint16_t *DW(const void *p) { return (const uint16_t *)ct_dev_w(p); }

static void gemm(HipbEngine *e, const float *A, int M, int K, const uint16_t *Wh, const uint16_t *bh,
                 float *Y, int N, int epi, float scale, const int *row_mask) {
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.A = A; g.lda = K; g.W = DW(Wh); g.bias = DW(bh);
    g.Y = Y; g.ldy = N; g.M = M; g.N = N; g.K = K; g.epi = epi; g.scale = scale;
    g.row_mask = row_mask;
    ctk_gemm(&g, e->enc_s);
}

/* Slaney mel scale and the librosa-style filterbank the reference builds in
 * transcribe.c:51-93 (fmin 0, fmax 8 kHz, area-normalised triangles). */
static double hz_mel(double f) {
    const double sp = 200.0 / 3.0, brk = 1000.0, step = log(6.4) / 27.0;
    return f < brk ? f / sp : brk / sp + log(f / brk) / step;
}
static double mel_hz(double m) {
    const double sp = 200.0 / 3.0, brk = 1000.0, step = log(6.4) / 27.0;
    return m < brk / sp ? sp * m : brk * exp(step * (m - brk / sp));
}

static void mel_tables_init(HipbEngine *e) {
    float hann[WIN_LEN], twr[N_FFT / 2], twi[N_FFT / 2];
    static float fb[N_MELS * N_BINS];
    int lo[N_MELS], hi[N_MELS];
    /* Hann window in the reference's fp32 expression (transcribe.c:47-49) */
    for (int i = 0; i < WIN_LEN; i++)
        hann[i] = 0.5f * (1.0f - cosf(2.0f * (float)M_PI * i / (WIN_LEN - 1)));
    for (int k = 0; k < N_FFT / 2; k++) {
        twr[k] = (float)cos(2.0 * M_PI * k / N_FFT);
        twi[k] = (float)-sin(2.0 * M_PI * k / N_FFT);
    }
    double pts[N_MELS + 2];
    const double m0 = hz_mel(0.0), m1 = hz_mel(SR / 2.0);
    for (int i = 0; i < N_MELS + 2; i++) pts[i] = mel_hz(m0 + (m1 - m0) * i / (N_MELS + 1));
    for (int m = 0; m < N_MELS; m++) {
        const double norm = 2.0 / (pts[m + 2] - pts[m]);
        lo[m] = N_BINS; hi[m] = 0;
        for (int i = 0; i < N_BINS; i++) {
            const double f = (SR / 2.0) * i / (N_BINS - 1);
            const double up = (f - pts[m]) / (pts[m + 1] - pts[m]);
            const double dn = (pts[m + 2] - f) / (pts[m + 2] - pts[m + 1]);
            const double w = up < dn ? up : dn;
            fb[m * N_BINS + i] = (float)(w > 0.0 ? w * norm : 0.0);
            if (fb[m * N_BINS + i] != 0.0f) { if (i < lo[m]) lo[m] = i; hi[m] = i + 1; }
        }
        if (hi[m] < lo[m]) { lo[m] = 0; hi[m] = 0; }
    }
    e->d_hann = dmalloc(sizeof hann);
    e->d_twr = dmalloc(sizeof twr);
    e->d_twi = dmalloc(sizeof twi);
    e->d_fb = dmalloc(sizeof fb);
    e->d_fb_lo = dmalloc(sizeof lo);
    e->d_fb_hi = dmalloc(sizeof hi);
    ECHK(hipMemcpy(e->d_hann, hann, sizeof hann, hipMemcpyHostToDevice));
    ECHK(hipMemcpy(e->d_twr, twr, sizeof twr, hipMemcpyHostToDevice));
    ECHK(hipMemcpy(e->d_twi, twi, sizeof twi, hipMemcpyHostToDevice));
    ECHK(hipMemcpy(e->d_fb, fb, sizeof fb, hipMemcpyHostToDevice));
    ECHK(hipMemcpy(e->d_fb_lo, lo, sizeof lo, hipMemcpyHostToDevice));
    ECHK(hipMemcpy(e->d_fb_hi, hi, sizeof hi, hipMemcpyHostToDevice));
    e->mel_tab = (CtMelTables){e->d_hann, e->d_twr, e->d_twi, e->d_fb, e->d_fb_lo, e->d_fb_hi};
}

/* GEMM whose activations come pre-split (hi, lo bf16 planes). */
static void gemm_sp(HipbEngine *e, const uint16_t *Ah, const uint16_t *Al, int M, int K,
                    const uint16_t *Wh, const uint16_t *bh, float *Y, int N, int epi, float scale) {
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.Ahi = Ah; g.Alo = Al; g.lda = K; g.W = DW(Wh); g.bias = DW(bh);
    g.Y = Y; g.ldy = N; g.M = M; g.N = N; g.K = K; g.epi = epi; g.scale = scale;
    ctk_gemm(&g, e->enc_s);
}

/* FFN up projection with SiLU, written pre-split for the down projection. */
static void gemm_sp_silu_split(HipbEngine *e, const uint16_t *Ah, const uint16_t *Al, int M,
                               const uint16_t *Wh, const uint16_t *bh, uint16_t *Oh, uint16_t *Ol) {
    CtGemm g;
    memset(&g, 0, sizeof g);
    g.Ahi = Ah; g.Alo = Al; g.lda = ENC_D; g.W = DW(Wh); g.bias = DW(bh);
    g.M = M; g.N = ENC_FF; g.K = ENC_D; g.epi = CT_EPI_SILU;
    g.nseg = 1; g.seg_w = ENC_FF;
    g.seg[0].mode = CT_OUT_SPLIT; g.seg[0].base = Oh; g.seg[0].base_lo = Ol; g.seg[0].ld = ENC_FF;
    ctk_gemm(&g, e->enc_s);
}

HipbEngine *hipb_create(const HipbConfig *cfg, const Weights *W) {
    if (ct_t.dev < 0) CT_FATAL("hipb_create: call backend_init first");
    if (cfg->slots < 1 || cfg->slots > CT_MAX_BATCH) CT_FATAL("hipb_create: slots outside [1, 256]");
    if (cfg->max_frames < 1 || cfg->max_frames > 2048) CT_FATAL("hipb_create: max_frames outside [1, 2048]");
    if (cfg->max_requests < 1) CT_FATAL("hipb_create: max_requests < 1");
    if (cfg->max_tokens < 0 || cfg->max_tokens > MAX_SEQ) CT_FATAL("hipb_create: max_tokens outside [0, MAX_SEQ]");
    HipbEngine *e = calloc(1, sizeof *e);
    if (!e) CT_FATAL("out of host memory");
    e->cfg = *cfg;
    e->W = *W;
    e->s = ct_t.stream;
    ECHK(hipStreamCreate(&e->s2));   /* the encoder's stream in hipb_process */
    e->enc_s = e->s;
    e->dev = ct_t.dev;
    e->esz = cfg->kv_bf16 ? 2 : 4;
    const int S = cfg->slots, R = cfg->max_requests;
    const int tmax = (cfg->max_frames + 7) / 8 * 8;
    CtEngDev *d = &e->d;
    /* request ring: at least 4 entries' worth of requests outstanding, and
     * room for the retirements of 8 steps over all slots 4 times over (the
     * host reads the retirement ring at least every ring / 4 of them) */
    int ring = 1024;
    {
        /* HIPB_RING_MIN (a power of two >= 16): a smaller lower bound, so that
         * tests reach the ring's wraparound with few requests */
        const char *rmin = getenv("HIPB_RING_MIN");
        if (rmin && rmin[0]) {
            ring = atoi(rmin);
            if (ring < 16 || (ring & (ring - 1))) CT_FATAL("hipb_create: HIPB_RING_MIN must be a power of two >= 16");
        }
    }
    while (ring < 4 * R || ring < 32 * S) ring <<= 1;
    e->ring = ring;
    d->ring_mask = ring - 1;
    if (cfg->prefill_rows < 0 || cfg->prefill_rows > CT_MAX_BATCH)
        CT_FATAL("hipb_create: prefill_rows outside [0, 256]");
    const int NR = S + cfg->prefill_rows;   /* step rows */
    d->slots = S; d->max_req = R; d->tmax = tmax; d->rows = NR;
    d->smax = cfg->max_tokens > 0 ? cfg->max_tokens : MAX_SEQ;
    d->kv_rows = d->smax + CT_KV_PAD;
    d->slot_req = dmalloc(S * sizeof(int));
    d->slot_S = dmalloc(S * sizeof(int));
    d->slot_np = dmalloc(S * sizeof(int));
    d->slot_T = dmalloc(S * sizeof(int));
    d->slot_flags = dmalloc(S * sizeof(int));
    d->slot_lim = dmalloc(S * sizeof(int));
    d->slot_ng = dmalloc(S * sizeof(int));
    d->slot_tok = dmalloc(S * sizeof(int));
    d->slot_ent = dmalloc(S * sizeof(int));
    d->act = dmalloc(NR * sizeof(int));
    d->tok = dmalloc(NR * sizeof(int));
    d->pos_len = dmalloc(NR * sizeof(int));
    d->cross_len = dmalloc(NR * sizeof(int));
    d->cross_idx = dmalloc(NR * sizeof(int));
    d->row_slot = dmalloc(NR * sizeof(int));
    d->rank_self = dmalloc(NR * sizeof(int));
    d->rank_cross = dmalloc(NR * sizeof(int));
    e->warm_sink = dmalloc(1024);
    d->kv_rowoff = dmalloc(NR * sizeof(long));
    d->req_T = dmalloc(ring * sizeof(int));
    d->req_limit = dmalloc(ring * sizeof(int));
    d->req_flags = dmalloc(ring * sizeof(int));
    d->req_np = dmalloc(ring * sizeof(int));
    d->req_ngen = dmalloc(ring * sizeof(int));
    d->req_entry = dmalloc(ring * sizeof(int));
    d->req_prompt = dmalloc((size_t)ring * CT_PROMPT_MAX * sizeof(int));
    d->req_out = dmalloc((size_t)ring * d->smax * sizeof(int));
    d->req_score = dmalloc((size_t)ring * d->smax * sizeof(float));
    d->q = dmalloc(CT_Q_WORDS * sizeof(int));
    d->fq = dmalloc(ring * sizeof(int));
    d->req_next = dmalloc(ring * sizeof(int));
    d->rq = dmalloc(ring * sizeof(int));
    d->ret = dmalloc(ring * sizeof(int));
    d->pend = dmalloc(S * sizeof(int));
    ECHK(hipMemsetAsync(d->slot_req, 0xff, S * sizeof(int), e->s));   /* -1: free */
    ECHK(hipMemsetAsync(d->slot_S, 0, S * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->slot_ent, 0, S * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->req_ngen, 0, ring * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->q, 0, CT_Q_WORDS * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->req_next, 0xff, ring * sizeof(int), e->s));   /* -1: no successor */
    ECHK(hipMemsetAsync(d->pend, 0xff, S * sizeof(int), e->s));

    /* repack [Wq;Wk;Wv] and cross [Wk;Wv] contiguously (device to device) */
    const size_t wsz = (size_t)DEC_D * DEC_D * 2, bsz = (size_t)DEC_D * 2;
    e->wqkv = dmalloc(DEC_N * 3 * wsz);
    e->bqkv = dmalloc(DEC_N * 3 * bsz);
    e->wckv = dmalloc(DEC_N * 2 * wsz);
    e->bckv = dmalloc(DEC_N * 2 * bsz);
    for (int l = 0; l < DEC_N; l++) {
        const DLayer *L = &W->dec[l];
        const uint16_t *ws[3] = {L->sa_qw, L->sa_kw, L->sa_vw}, *bs[3] = {L->sa_qb, L->sa_kb, L->sa_vb};
        for (int i = 0; i < 3; i++) {
            ECHK(hipMemcpyAsync((char *)e->wqkv + (3 * l + i) * wsz, DW(ws[i]), wsz, hipMemcpyDeviceToDevice, e->s));
            ECHK(hipMemcpyAsync((char *)e->bqkv + (3 * l + i) * bsz, DW(bs[i]), bsz, hipMemcpyDeviceToDevice, e->s));
        }
        ECHK(hipMemcpyAsync((char *)e->wckv + (2 * l) * wsz, DW(L->ca_kw), wsz, hipMemcpyDeviceToDevice, e->s));
        ECHK(hipMemcpyAsync((char *)e->wckv + (2 * l + 1) * wsz, DW(L->ca_vw), wsz, hipMemcpyDeviceToDevice, e->s));
        ECHK(hipMemcpyAsync((char *)e->bckv + (2 * l) * bsz, DW(L->ca_kb), bsz, hipMemcpyDeviceToDevice, e->s));
        ECHK(hipMemcpyAsync((char *)e->bckv + (2 * l + 1) * bsz, DW(L->ca_vb), bsz, hipMemcpyDeviceToDevice, e->s));
    }
    {
        const size_t ewsz = (size_t)ENC_D * ENC_D * 2, ebsz = (size_t)ENC_D * 2;
        e->ew_qkv = dmalloc(ENC_N * 3 * ewsz);
        e->eb_qkv = dmalloc(ENC_N * 3 * ebsz);
        for (int l = 0; l < ENC_N; l++) {
            const ELayer *L = &W->enc[l];
            const uint16_t *ws[3] = {L->sa_qw, L->sa_kw, L->sa_vw}, *bs[3] = {L->sa_qb, L->sa_kb, L->sa_vb};
            for (int i = 0; i < 3; i++) {
                ECHK(hipMemcpyAsync((char *)e->ew_qkv + (3 * l + i) * ewsz, DW(ws[i]), ewsz,
                                    hipMemcpyDeviceToDevice, e->s));
                ECHK(hipMemcpyAsync((char *)e->eb_qkv + (3 * l + i) * ebsz, DW(bs[i]), ebsz,
                                    hipMemcpyDeviceToDevice, e->s));
            }
        }
    }
    {
        const size_t DD = (size_t)DEC_D * DEC_D, per = 3 * DD + 3 * DD + 2 * (size_t)DEC_FF * DEC_D;
        e->wtile = dmalloc((DEC_N * per + (size_t)VOCAB * DEC_D) * 2);
        uint16_t *p = e->wtile;
        for (int l = 0; l < DEC_N; l++) {
            const DLayer *L = &W->dec[l];
            ctk_tile_w(e->wqkv + 3 * l * DD, p, 3 * DEC_D, DEC_D, e->s); e->wt_qkv[l] = p; p += 3 * DD;
            ctk_tile_w(DW(L->sa_ow), p, DEC_D, DEC_D, e->s); e->wt_o[l] = p; p += DD;
            ctk_tile_w(DW(L->ca_qw), p, DEC_D, DEC_D, e->s); e->wt_cq[l] = p; p += DD;
            ctk_tile_w(DW(L->ca_ow), p, DEC_D, DEC_D, e->s); e->wt_co[l] = p; p += DD;
            ctk_tile_w(DW(L->ffn_w1), p, DEC_FF, DEC_D, e->s); e->wt_f1[l] = p; p += (size_t)DEC_FF * DEC_D;
            ctk_tile_w(DW(L->ffn_w2), p, DEC_D, DEC_FF, e->s); e->wt_f2[l] = p; p += (size_t)DEC_FF * DEC_D;
        }
        ctk_tile_w(DW(W->etw), p, VOCAB, DEC_D, e->s);
        e->wt_lm = p;
    }
    {
        /* column constants of the GEMMs whose LayerNorm is folded in */
        const size_t per = 2 * (3 * DEC_D + DEC_D + DEC_FF);
        e->fold = dmalloc(DEC_N * per * sizeof(float));
        float *p = e->fold;
        for (int l = 0; l < DEC_N; l++) {
            const DLayer *L = &W->dec[l];
            ctk_fold_cols(e->wqkv + (size_t)3 * l * DEC_D * DEC_D, DW(L->sa_lnw), DW(L->sa_lnb),
                          e->bqkv + (size_t)3 * l * DEC_D, 3 * DEC_D, DEC_D, p, p + 3 * DEC_D, e->s);
            e->fc_qkv[l][0] = p; e->fc_qkv[l][1] = p + 3 * DEC_D; p += 6 * DEC_D;
            ctk_fold_cols(DW(L->ca_qw), DW(L->ca_lnw), DW(L->ca_lnb), DW(L->ca_qb), DEC_D, DEC_D, p,
                          p + DEC_D, e->s);
            e->fc_cq[l][0] = p; e->fc_cq[l][1] = p + DEC_D; p += 2 * DEC_D;
            ctk_fold_cols(DW(L->ffn_w1), DW(L->ffn_lnw), DW(L->ffn_lnb), DW(L->ffn_b1), DEC_FF, DEC_D, p,
                          p + DEC_FF, e->s);
            e->fc_f1[l][0] = p; e->fc_f1[l][1] = p + DEC_FF; p += 2 * DEC_FF;
        }
    }
    const size_t self_el = (size_t)DEC_N * S * DEC_H * d->kv_rows * DEC_DK;
    const size_t cross_el = (size_t)DEC_N * R * DEC_H * tmax * DEC_DK;
    e->kself = dmalloc(self_el * e->esz);
    e->vself = dmalloc(self_el * e->esz);
    e->kcross = dmalloc(cross_el * e->esz);
    e->vcross = dmalloc(cross_el * e->esz);
    e->enc_pool = dmalloc((size_t)R * tmax * DEC_D * sizeof(float));
    e->h = dmalloc((size_t)NR * DEC_D * 4);
    e->q = dmalloc((size_t)NR * DEC_D * 4);
    e->parts = dmalloc((size_t)ctk_gemv_ksplit(DEC_D, DEC_FF) * NR * DEC_D * 4);
    e->midf = dmalloc(ct_frag_elems(NR, DEC_FF) * 2);
    e->lnf = dmalloc(ct_frag_elems(NR, DEC_D) * 2);
    e->attf = dmalloc(ct_frag_elems(NR, DEC_D) * 2);
    e->logits = dmalloc((size_t)S * VOCAB * 4);
    e->lnstat = dmalloc((size_t)NR * CT_LN_BLOCKS * 2 * 4);
    ECHK(hipMemsetAsync(e->h, 0, (size_t)NR * DEC_D * 4, e->s));
    ECHK(hipMemsetAsync(e->lnstat, 0, (size_t)NR * CT_LN_BLOCKS * 2 * 4, e->s));
    ECHK(hipMemsetAsync(d->act, 0, NR * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->tok, 0, NR * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->pos_len, 0, NR * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->cross_len, 0, NR * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->cross_idx, 0, NR * sizeof(int), e->s));
    ECHK(hipMemsetAsync(d->row_slot, 0, NR * sizeof(int), e->s));
    {
        /* identity until a step ranks the rows */
        int *ident = malloc((size_t)NR * sizeof(int));
        if (!ident) CT_FATAL("out of host memory");
        for (int i = 0; i < NR; i++) ident[i] = i;
        ECHK(hipMemcpy(d->rank_self, ident, NR * sizeof(int), hipMemcpyHostToDevice));
        ECHK(hipMemcpy(d->rank_cross, ident, NR * sizeof(int), hipMemcpyHostToDevice));
        free(ident);
    }
    ECHK(hipMemsetAsync(d->kv_rowoff, 0xff, NR * sizeof(long), e->s));
    e->M = S;
    e->req_cap = R;
    e->req = calloc(R, sizeof(HostReq));
    e->order = malloc((size_t)R * sizeof(int));
    e->d_pairs = dmalloc((size_t)2 * R * sizeof(int));
    if (cfg->admit_order < 0 || cfg->admit_order > 1) CT_FATAL("hipb_create: admit_order outside [0, 1]");
    if (cfg->enc_ffn_bf16 < 0 || cfg->enc_ffn_bf16 > 1) CT_FATAL("hipb_create: enc_ffn_bf16 outside [0, 1]");
    e->free_ent = malloc((size_t)R * sizeof(int));
    e->ent_owner = malloc((size_t)R * sizeof(int));
    if (!e->req || !e->order || !e->free_ent || !e->ent_owner) CT_FATAL("out of host memory");
    for (int i = 0; i < R; i++) { e->free_ent[i] = i; e->ent_owner[i] = -1; }
    e->free_head = 0;
    e->free_tail = R;
    pthread_mutex_init(&e->mu, NULL);
    pthread_cond_init(&e->cv, NULL);
    const char *eg = getenv("HIPB_EAGER");
    e->eager = eg && eg[0] == '1';
    /* scheduling knobs (the results are the same bits either way) */
    const char *rm = getenv("HIPB_RANK_MIN_ROWS"), *ra = getenv("HIPB_READ_AHEAD");
    d->rank_min = rm && rm[0] ? atoi(rm) : CT_RANK_MIN_ROWS;
    e->read_ahead = !(ra && ra[0] == '0');
    mel_tables_init(e);
    ECHK(hipHostMalloc((void **)&e->h_tmp, (size_t)(R + 8) * (MAX_SEQ + 8) * sizeof(int), 0));
    ECHK(hipHostMalloc((void **)&e->h_meta, (size_t)ring * (CT_META_FIELDS + CT_PROMPT_MAX) * sizeof(int), 0));
    ECHK(hipHostMalloc((void **)&e->h_ret, (size_t)ring * sizeof(int), 0));
    /* per batch (at most R requests): subsampling group tables (<= 10 R
     * ints), queue words, published ids, their entries */
    ECHK(hipHostMalloc((void **)&e->h_enc, (size_t)(13 * R + 64) * sizeof(int), 0));
    ECHK(hipStreamSynchronize(e->s));
    return e;
}

void hipb_destroy(HipbEngine *e) {
    if (!e) return;
    ECHK(hipStreamSynchronize(e->s));
    for (int w = 0; w < 2; w++)
        if (e->have_graph[w]) { hipGraphExecDestroy(e->exec[w]); hipGraphDestroy(e->graph[w]); }
    void *ptrs[] = {e->d.slot_req, e->d.slot_S, e->d.slot_np, e->d.slot_T, e->d.slot_flags,
                    e->d.slot_lim, e->d.slot_ng, e->d.slot_tok, e->d.slot_ent, e->d.act, e->d.tok, e->d.pos_len,
                    e->d.cross_len, e->d.req_entry, e->d.ret, e->e_dstrow, e->d_pairs,
                    e->d.row_slot, e->d.rank_self, e->d.rank_cross, e->warm_sink,
                    e->d.cross_idx, e->d.kv_rowoff, e->d.req_T, e->d.req_limit, e->d.req_flags,
                    e->d.req_np, e->d.req_ngen, e->d.req_prompt, e->d.req_out, e->d.req_score, e->d.q,
                    e->d.req_next, e->d.rq, e->d.pend, e->d.fq,
                    e->wqkv, e->bqkv, e->wckv, e->bckv, e->ew_qkv, e->eb_qkv, e->wtile, e->kself, e->vself, e->kcross, e->vcross,
                    e->enc_pool, e->h, e->q, e->parts, e->fold, e->lnf, e->attf, e->midf, e->logits, e->lnstat,
                    e->ex, e->eln, e->emid, e->eq, e->ek, e->ev, e->eo, e->eg, e->edw, e->epe, e->ep_all,
                    e->esub, e->emel, e->e_subtab, e->e_row_start, e->e_row_len, e->e_seq_off, e->e_seq_T,
                    e->e_blk_seq, e->e_blk_q0, e->e_rowoff, e->d_hann, e->d_twr, e->d_twi, e->d_fb,
                    e->d_fb_lo, e->d_fb_hi, e->epcm, e->e_clips, e->e_frame_clip,
                    e->eln_h, e->eln_l, e->emid_h, e->emid_l, e->eo_h, e->eo_l, e->edw_h, e->edw_l,
                    e->floor_sink};
    for (size_t i = 0; i < sizeof ptrs / sizeof ptrs[0]; i++)
        if (ptrs[i]) ECHK(hipFree(ptrs[i]));
    for (int r = 0; r < e->n_req; r++) {
        free(e->req[r].mel); free(e->req[r].pcm); free(e->req[r].out); free(e->req[r].score);
    }
    free(e->req);
    free(e->order);
    free(e->free_ent);
    free(e->ent_owner);
    pthread_mutex_destroy(&e->mu);
    pthread_cond_destroy(&e->cv);
    ECHK(hipHostFree(e->h_tmp));
    ECHK(hipHostFree(e->h_meta));
    ECHK(hipHostFree(e->h_ret));
    ECHK(hipHostFree(e->h_enc));
    ECHK(hipStreamDestroy(e->s2));
    free(e);
}

void *hipb_stream(HipbEngine *e) { return (void *)e->s; }

void hipb_reset(HipbEngine *e) {
    ECHK(hipStreamSynchronize(e->s));
    for (int r = 0; r < e->n_req; r++) {
        free(e->req[r].mel); free(e->req[r].pcm); free(e->req[r].out); free(e->req[r].score);
        memset(&e->req[r], 0, sizeof e->req[r]);
    }
    e->n_req = e->n_enc = 0;
    atomic_store(&e->n_assigned, 0);
    e->meta_lo = 0;
    e->fq_count = 0;
    e->n_pub = 0;
    e->ret_seen = 0;
    for (int i = 0; i < e->d.max_req; i++) { e->free_ent[i] = i; e->ent_owner[i] = -1; }
    e->free_head = 0;
    e->free_tail = e->d.max_req;
    atomic_store(&e->published, 0);
    e->bench_mode = 0;
    ECHK(hipMemsetAsync(e->d.slot_req, 0xff, e->d.slots * sizeof(int), e->s));
    ECHK(hipMemsetAsync(e->d.slot_S, 0, e->d.slots * sizeof(int), e->s));
    ECHK(hipMemsetAsync(e->d.req_ngen, 0, e->ring * sizeof(int), e->s));
    ECHK(hipMemsetAsync(e->d.q, 0, CT_Q_WORDS * sizeof(int), e->s));
    ECHK(hipMemsetAsync(e->d.req_next, 0xff, e->ring * sizeof(int), e->s));
    ECHK(hipMemsetAsync(e->d.pend, 0xff, e->d.slots * sizeof(int), e->s));
    ECHK(hipStreamSynchronize(e->s));
}

/* ------------------------------------------------------------------ */
/* Requests and the packed encoder                                     */
/* ------------------------------------------------------------------ */
static int t_enc_of(int T_mel) {
    const int a = (T_mel + 1) / 2, b = (a + 1) / 2;
    return (b + 1) / 2;
}

static int submit_common(HipbEngine *e, int T_mel, const int *prompt, int n_prompt, int limit,
                         int flags);

/* Host mirror of the request ring: field f (0 length, 1 limit, 2 flags,
 * 3 prompt length, 4 successor, 5 tokens generated = 0, 6 encoder entry =
 * -1 until published) at ring slot i, then the prompts. */
static int *meta_field(HipbEngine *e, int f) { return e->h_meta + (size_t)f * e->ring; }
static int *meta_prompt(HipbEngine *e, int r) {
    return e->h_meta + (size_t)CT_META_FIELDS * e->ring + (size_t)(r & (e->ring - 1)) * CT_PROMPT_MAX;
}

/* Copies `width` ints per request for the ids [lo, lo + n) from the host
 * ring `src` into the device ring `dst`, on stream s (at most two pieces:
 * the ids' slots wrap around once at most, n <= ring). */
static void ring_put(HipbEngine *e, int *dst, const int *src, int lo, int n, int width, hipStream_t s) {
    const int mask = e->ring - 1, a = lo & mask, n1 = n < e->ring - a ? n : e->ring - a;
    ECHK(hipMemcpyAsync(dst + (size_t)a * width, src + (size_t)a * width, (size_t)n1 * width * sizeof(int),
                        hipMemcpyHostToDevice, s));
    if (n > n1)
        ECHK(hipMemcpyAsync(dst, src, (size_t)(n - n1) * width * sizeof(int), hipMemcpyHostToDevice, s));
}

/* Uploads the fields of the requests submitted since the last upload to
 * their ring slots, on the engine stream: ahead of every step that could
 * admit them (the device edits a chained request's prompt only after its
 * predecessor, uploaded with it, has decoded). */
static void flush_meta(HipbEngine *e) {
    const int lo = e->meta_lo, n = e->n_req - lo;
    if (n <= 0) return;
    int *const dst[CT_META_FIELDS] = {e->d.req_T, e->d.req_limit, e->d.req_flags, e->d.req_np,
                                      e->d.req_next, e->d.req_ngen, e->d.req_entry};
    for (int f = 0; f < CT_META_FIELDS; f++) ring_put(e, dst[f], meta_field(e, f), lo, n, 1, e->s);
    ring_put(e, e->d.req_prompt, e->h_meta + (size_t)CT_META_FIELDS * e->ring, lo, n, CT_PROMPT_MAX, e->s);
    e->meta_lo = e->n_req;
}

int hipb_submit(HipbEngine *e, const float *mel, int T_mel, const int *prompt, int n_prompt,
                int limit, int flags) {
    const int r = submit_common(e, T_mel, prompt, n_prompt, limit, flags);
    HostReq *q = &e->req[r];
    q->mel = malloc((size_t)N_MELS * T_mel * sizeof(float));
    if (!q->mel) CT_FATAL("out of host memory");
    memcpy(q->mel, mel, (size_t)N_MELS * T_mel * sizeof(float));
    return r;
}

int hipb_submit_pcm(HipbEngine *e, const float *pcm, int n_samples, const int *prompt, int n_prompt,
                    int limit, int flags) {
    if (n_samples < HOP_LEN) CT_FATAL("hipb_submit_pcm: clip shorter than one hop (160 samples)");
    const int r = submit_common(e, 1 + n_samples / HOP_LEN, prompt, n_prompt, limit, flags);
    HostReq *q = &e->req[r];
    q->pcm = malloc((size_t)n_samples * sizeof(float));
    if (!q->pcm) CT_FATAL("out of host memory");
    memcpy(q->pcm, pcm, (size_t)n_samples * sizeof(float));
    q->n = n_samples;
    return r;
}

int hipb_submit_pcm_chunked(HipbEngine *e, const float *pcm, int n_samples, const int *prompt,
                            int n_prompt, int limit, int flags, float silence_db, float silence_dur,
                            float target_sec, int *first_req) {
    if (n_prompt < 2) CT_FATAL("hipb_submit_pcm_chunked: the prompt needs at least 2 ids (pre + post)");
    if (n_prompt + CT_CARRY_MAX + limit > e->d.smax)
        CT_FATAL("hipb_submit_pcm_chunked: prompt + 64 carried ids + limit exceeds the engine's max_tokens");
    const int cap = n_samples / HOP_LEN + 1;
    int *b = malloc((size_t)2 * cap * sizeof(int));
    if (!b) CT_FATAL("out of host memory");
    const int nc = hipb_chunk_bounds(pcm, n_samples, silence_db, silence_dur, target_sec, b, cap);
    const int r0 = e->n_req;
    for (int c = 0; c < nc; c++) {
        const int r = hipb_submit_pcm(e, pcm + b[2 * c], b[2 * c + 1] - b[2 * c], prompt, n_prompt,
                                      limit, flags);
        e->req[r].chained = c > 0;
    }
    free(b);
    /* link chunk c to chunk c + 1 */
    for (int c = 0; c + 1 < nc; c++) meta_field(e, 4)[(r0 + c) & (e->ring - 1)] = r0 + c + 1;
    if (first_req) *first_req = r0;
    return nc;
}

int hipb_submit_pcm_device(HipbEngine *e, const float *dev_pcm, int n_samples, const int *prompt,
                           int n_prompt, int limit, int flags) {
    if (n_samples < HOP_LEN) CT_FATAL("hipb_submit_pcm_device: clip shorter than one hop (160 samples)");
    const int r = submit_common(e, 1 + n_samples / HOP_LEN, prompt, n_prompt, limit, flags);
    e->req[r].dpcm = dev_pcm;
    e->req[r].n = n_samples;
    return r;
}

static void read_queue(HipbEngine *e, int *q);
static void recycle(HipbEngine *e, int finished);

/* Copies a finished request's tokens and scores from its ring slot to the
 * host (before the slot is reused). */
static void collect(HipbEngine *e, int r) {
    HostReq *q = &e->req[r];
    if (q->collected) return;
    const size_t slot = (size_t)(r & (e->ring - 1));
    int n = 0;
    ECHK(hipStreamSynchronize(e->s));
    ECHK(hipMemcpy(&n, e->d.req_ngen + slot, sizeof(int), hipMemcpyDeviceToHost));
    q->out = malloc((size_t)(n > 0 ? n : 1) * sizeof(int));
    q->score = malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!q->out || !q->score) CT_FATAL("out of host memory");
    if (n > 0) {
        ECHK(hipMemcpy(q->out, e->d.req_out + slot * e->d.smax, n * sizeof(int), hipMemcpyDeviceToHost));
        ECHK(hipMemcpy(q->score, e->d.req_score + slot * e->d.smax, n * sizeof(float), hipMemcpyDeviceToHost));
    }
    q->n_out = n;
    q->collected = 1;
}

/* Request r takes ring slot r & (ring - 1): the slot's previous request,
 * r - ring, must have finished; its results move to the host first. */
static void ring_slot_take(HipbEngine *e, int r) {
    if (r < e->ring) return;
    HostReq *o = &e->req[r - e->ring];
    if (o->collected) return;
    if (!o->done) {
        int q[CT_Q_WORDS];
        read_queue(e, q);
        recycle(e, q[2]);
    }
    if (!o->done)
        CT_FATAL("hipb_submit: more requests outstanding than the request ring holds (4 x max_requests, "
                 "at least 1024): run the submitted ones first");
    collect(e, r - e->ring);
}

static int submit_common(HipbEngine *e, int T_mel, const int *prompt, int n_prompt, int limit,
                         int flags) {
    if (e->bench_mode) CT_FATAL("hipb_submit: engine is in microbenchmark mode");
    if (n_prompt < 1 || n_prompt > CT_PROMPT_SUBMIT_MAX) CT_FATAL("hipb_submit: prompt length outside [1, 16]");
    if (limit < 1) CT_FATAL("hipb_submit: limit < 1");
    if (n_prompt + limit > e->d.smax) CT_FATAL("hipb_submit: prompt + limit exceeds the engine's max_tokens");
    const int Te = t_enc_of(T_mel);
    if (T_mel < 1 || Te > e->d.tmax || Te > e->cfg.max_frames) CT_FATAL("hipb_submit: clip longer than max_frames");
    if (e->n_req == e->req_cap) {
        const int nc = 2 * e->req_cap;
        HostReq *nr = realloc(e->req, (size_t)nc * sizeof(HostReq));
        if (!nr) CT_FATAL("out of host memory");
        memset(nr + e->req_cap, 0, (size_t)(nc - e->req_cap) * sizeof(HostReq));
        e->req = nr;
        int *no = realloc(e->order, (size_t)nc * sizeof(int));
        if (!no) CT_FATAL("out of host memory");
        e->order = no;
        e->req_cap = nc;
    }
    const int r = e->n_req;
    ring_slot_take(e, r);
    e->n_req++;
    HostReq *q = &e->req[r];
    memset(q, 0, sizeof *q);
    q->T_mel = T_mel;
    q->T_enc = Te;
    q->entry = -1;
    q->limit = limit;
    e->order[r] = r;
    /* the ring slot's mirror entries were last uploaded for request
     * r - ring, which has finished, so no upload is still reading them */
    const int rs = r & (e->ring - 1);
    meta_field(e, 0)[rs] = Te;
    meta_field(e, 1)[rs] = limit;
    meta_field(e, 2)[rs] = flags;
    meta_field(e, 3)[rs] = n_prompt;
    meta_field(e, 4)[rs] = -1;
    meta_field(e, 5)[rs] = 0;
    meta_field(e, 6)[rs] = -1;
    int *pp = meta_prompt(e, r);
    memset(pp, 0, sizeof(int) * CT_PROMPT_MAX);
    memcpy(pp, prompt, (size_t)n_prompt * sizeof(int));
    return r;
}

int hipb_req_frames(HipbEngine *e, int req) {
    return (req >= 0 && req < e->n_req) ? e->req[req].T_enc : 0;
}

/* Subsampling scratch (floats) at least this large: 80 Mi floats (320 MB)
 * hold the stage buffers of about 5 minutes of audio, packed. */
#define CT_SUB_PACK_FLOATS (80 << 20)

static void enc_reserve(HipbEngine *e, int frames, int max_tmel) {
    const int T1 = (max_tmel + 1) / 2, T2 = (T1 + 1) / 2;
    /* one request's stage buffers, and at least CT_SUB_PACK_FLOATS so that
     * several requests' subsampling runs packed */
    int sub = SUB_CH * (T1 * 64 + T2 * 32);
    if (sub < CT_SUB_PACK_FLOATS) sub = CT_SUB_PACK_FLOATS;
    if (frames <= e->enc_cap && sub <= e->sub_cap) return;
    ECHK(hipStreamSynchronize(e->enc_s));
    float **bufs[] = {&e->ex, &e->eln, &e->emid, &e->eq, &e->ek, &e->ev, &e->eo, &e->eg, &e->edw};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++)
        if (*bufs[i]) { ECHK(hipFree(*bufs[i])); *bufs[i] = NULL; }
    uint16_t **hb[] = {&e->eln_h, &e->eln_l, &e->emid_h, &e->emid_l, &e->eo_h, &e->eo_l, &e->edw_h, &e->edw_l};
    for (size_t i = 0; i < sizeof hb / sizeof hb[0]; i++)
        if (*hb[i]) { ECHK(hipFree(*hb[i])); *hb[i] = NULL; }
    int **ib[] = {&e->e_row_start, &e->e_row_len, &e->e_seq_off, &e->e_seq_T, &e->e_blk_seq, &e->e_blk_q0};
    for (size_t i = 0; i < sizeof ib / sizeof ib[0]; i++)
        if (*ib[i]) { ECHK(hipFree(*ib[i])); *ib[i] = NULL; }
    if (e->e_rowoff) ECHK(hipFree(e->e_rowoff));
    if (e->e_subtab) ECHK(hipFree(e->e_subtab));
    if (e->esub) ECHK(hipFree(e->esub));
    const int M = frames > e->enc_cap ? frames : e->enc_cap;
    const size_t rows = (size_t)M;
    e->ex = dmalloc(rows * ENC_D * 4);
    e->eln = NULL;
    e->emid = NULL;
    e->eln_h = dmalloc(rows * ENC_D * 2);
    e->eln_l = dmalloc(rows * ENC_D * 2);
    e->emid_h = dmalloc(rows * ENC_FF * 2);
    e->emid_l = dmalloc(rows * ENC_FF * 2);
    e->eo_h = dmalloc(rows * ENC_D * 2);
    e->eo_l = dmalloc(rows * ENC_D * 2);
    e->edw_h = dmalloc(rows * ENC_D * 2);
    e->edw_l = dmalloc(rows * ENC_D * 2);
    e->eq = dmalloc(rows * ENC_D * 4);
    e->ek = dmalloc(rows * ENC_D * 4);
    e->ev = dmalloc(rows * ENC_D * 4);
    e->eo = dmalloc(rows * ENC_D * 4);
    e->eg = dmalloc(rows * ENC_D * 4);
    e->edw = NULL;
    e->e_row_start = dmalloc(rows * sizeof(int));
    if (e->e_dstrow) ECHK(hipFree(e->e_dstrow));
    e->e_dstrow = dmalloc(rows * sizeof(int));
    e->e_row_len = dmalloc(rows * sizeof(int));
    e->e_rowoff = dmalloc(rows * sizeof(long));
    /* at most M sequences (one frame each) and M query blocks */
    e->e_seq_off = dmalloc(rows * sizeof(int));
    e->e_seq_T = dmalloc(rows * sizeof(int));
    e->e_blk_seq = dmalloc(rows * sizeof(int));
    e->e_blk_q0 = dmalloc(rows * sizeof(int));
    /* subsampling group tables: 5 (n + 1) ints per group, at most n groups */
    e->e_subtab = dmalloc((size_t)10 * (rows + 1) * sizeof(int));
    const int sc = sub > e->sub_cap ? sub : e->sub_cap;
    e->esub = dmalloc((size_t)sc * 4);
    e->enc_cap = M;
    e->sub_cap = sc;
}

/* Grows the mel, PCM and clip-table buffers for the batch ids[0..n). */
static void batch_buffers(HipbEngine *e, const int *ids, int n) {
    size_t mel_need = 0, pcm_need = 0;
    int nclip = 0, nfr = 0;
    for (int i = 0; i < n; i++) {
        const int r = ids[i];
        mel_need += (size_t)N_MELS * e->req[r].T_mel;
        if (e->req[r].pcm || e->req[r].dpcm) {
            if (e->req[r].pcm) pcm_need += e->req[r].n;
            nclip++;
            nfr += e->req[r].T_mel;
        }
    }
    if (mel_need > e->emel_cap) {
        if (e->emel) ECHK(hipFree(e->emel));
        e->emel = dmalloc(mel_need * 4);
        e->emel_cap = mel_need;
    }
    if (pcm_need > e->epcm_cap) {
        if (e->epcm) ECHK(hipFree(e->epcm));
        e->epcm = dmalloc(pcm_need * 4);
        e->epcm_cap = pcm_need;
    }
    if (nclip > e->clips_cap) {
        if (e->e_clips) ECHK(hipFree(e->e_clips));
        e->e_clips = dmalloc((size_t)nclip * sizeof(CtMelClip));
        e->clips_cap = nclip;
    }
    if (nfr > e->frames_cap) {
        if (e->e_frame_clip) ECHK(hipFree(e->e_frame_clip));
        e->e_frame_clip = dmalloc((size_t)nfr * sizeof(int));
        e->frames_cap = nfr;
    }
}

/* The position projections P_l = pos_emb W_pos_l of every layer, for the
 * engine's longest clip (tmax frames).  Row p holds relative distance
 * tmax - 1 - p, so any shorter clip's window is a contiguous slice and its
 * rows equal those a table built for that clip would hold (the GEMM's rows
 * do not depend on the row count). */
static void pos_tables(HipbEngine *e) {
    if (e->ep_all) return;
    const int rows = 2 * e->d.tmax - 1;
    e->epe = dmalloc((size_t)rows * ENC_D * 4);
    e->ep_all = dmalloc((size_t)ENC_N * rows * ENC_D * 4);
    ctk_rel_pos_emb(e->epe, e->d.tmax, ct_inv_freq(), e->enc_s);
    for (int l = 0; l < ENC_N; l++)
        gemm(e, e->epe, rows, ENC_D, e->W.enc[l].sa_pw, NULL, e->ep_all + (size_t)l * rows * ENC_D, ENC_D,
             CT_EPI_STORE, 0, NULL);
}

/* Encodes the requests ids[0..n) as one packed batch. */
static void encode_batch(HipbEngine *e, const int *ids, int n) {
    int M = 0, tmel_max = 0, T_max = 0;
    for (int i = 0; i < n; i++) {
        const int r = ids[i];
        M += e->req[r].T_enc;
        if (e->req[r].T_mel > tmel_max) tmel_max = e->req[r].T_mel;
        if (e->req[r].T_enc > T_max) T_max = e->req[r].T_enc;
    }
    enc_reserve(e, M, tmel_max);
    hipStream_t s = e->enc_s;
    /* host-side row tables */
    int *row_start = malloc(M * sizeof(int)), *row_len = malloc(M * sizeof(int));
    int *dstrow = malloc(M * sizeof(int));
    long *rowoff = malloc(M * sizeof(long));
    int *seq_off = malloc(n * sizeof(int)), *seq_T = malloc(n * sizeof(int));
    int off = 0;
    for (int i = 0; i < n; i++) {
        const int r = ids[i], T = e->req[r].T_enc, ent = e->req[r].entry;
        if (ent < 0) CT_FATAL("encode: request without an encoder entry");
        seq_off[i] = off;
        seq_T[i] = T;
        for (int t = 0; t < T; t++) {
            row_start[off + t] = off;
            row_len[off + t] = T;
            dstrow[off + t] = ent * e->d.tmax + t;
            rowoff[off + t] = ((long)ent * DEC_H * e->d.tmax + t) * DEC_DK;
        }
        off += T;
    }
    const int nblk = ctk_relpos_plan(NULL, NULL, seq_T, n);
    int *blk_seq = malloc(nblk * sizeof(int)), *blk_q0 = malloc(nblk * sizeof(int));
    ctk_relpos_plan(blk_seq, blk_q0, seq_T, n);
    if (nblk > e->enc_cap) CT_FATAL("encode: query-block table larger than the workspace");
    ECHK(hipMemcpyAsync(e->e_row_start, row_start, M * sizeof(int), hipMemcpyHostToDevice, s));
    ECHK(hipMemcpyAsync(e->e_row_len, row_len, M * sizeof(int), hipMemcpyHostToDevice, s));
    ECHK(hipMemcpyAsync(e->e_dstrow, dstrow, M * sizeof(int), hipMemcpyHostToDevice, s));
    ECHK(hipMemcpyAsync(e->e_rowoff, rowoff, M * sizeof(long), hipMemcpyHostToDevice, s));
    ECHK(hipMemcpyAsync(e->e_seq_off, seq_off, n * sizeof(int), hipMemcpyHostToDevice, s));
    ECHK(hipMemcpyAsync(e->e_seq_T, seq_T, n * sizeof(int), hipMemcpyHostToDevice, s));
    ECHK(hipMemcpyAsync(e->e_blk_seq, blk_seq, nblk * sizeof(int), hipMemcpyHostToDevice, s));
    ECHK(hipMemcpyAsync(e->e_blk_q0, blk_q0, nblk * sizeof(int), hipMemcpyHostToDevice, s));

    /* mel for every request of the batch, then the subsampling */
    batch_buffers(e, ids, n);
    /* log-mel on the GPU for PCM requests, uploaded mel otherwise */
    {
        int nclip = 0, nfr = 0;
        for (int i = 0; i < n; i++)
            if (e->req[ids[i]].pcm || e->req[ids[i]].dpcm) {
                nclip++;
                nfr += e->req[ids[i]].T_mel;
            }
        if (nclip) {
            CtMelClip *cl = malloc(nclip * sizeof *cl);
            int *fc = malloc(nfr * sizeof(int));
            size_t po = 0, mo = 0;
            int ci = 0, fo = 0;
            for (int i = 0; i < n; i++) {
                HostReq *q = &e->req[ids[i]];
                if (q->pcm || q->dpcm) {
                    const float *src = q->dpcm;
                    if (q->pcm) {
                        ECHK(hipMemcpyAsync(e->epcm + po, q->pcm, (size_t)q->n * 4, hipMemcpyHostToDevice, s));
                        src = e->epcm + po;
                        po += q->n;
                    }
                    cl[ci] = (CtMelClip){src, q->n, (long)mo, q->T_mel, fo};
                    for (int t = 0; t < q->T_mel; t++) fc[fo + t] = ci;
                    fo += q->T_mel; ci++;
                }
                mo += (size_t)N_MELS * q->T_mel;
            }
            ECHK(hipMemcpyAsync(e->e_clips, cl, nclip * sizeof *cl, hipMemcpyHostToDevice, s));
            ECHK(hipMemcpyAsync(e->e_frame_clip, fc, nfr * sizeof(int), hipMemcpyHostToDevice, s));
            ctk_mel(e->emel, e->e_clips, nclip, e->e_frame_clip, nfr, &e->mel_tab, s);
            ECHK(hipStreamSynchronize(s));
            free(cl); free(fc);
        }
    }
    size_t moff = 0;
    const Weights *W = &e->W;
    int *mel_off = malloc(n * sizeof(int));
    for (int i = 0; i < n; i++) {
        HostReq *q = &e->req[ids[i]];
        mel_off[i] = (int)moff;
        if (q->mel)
            ECHK(hipMemcpyAsync(e->emel + moff, q->mel, (size_t)N_MELS * q->T_mel * 4, hipMemcpyHostToDevice, s));
        moff += (size_t)N_MELS * q->T_mel;
    }
    /* subsampling over groups of requests packed along time, each group as
     * large as the scratch allows: conv0 + depthwise -> rb (split), pointwise
     * -> ra, depthwise -> rb (split), pointwise -> ra (ra and rb each hold the
     * group's first-stage output, [sum T2][32][256] floats or its two bf16
     * planes), then the flattened frames go
     * pre-split into the packed rows (the FFN planes are free until layer 0)
     * for one projection GEMM.  The group tables (row offsets of the three
     * stages, mel lengths and offsets) are staged in distinct parts of the
     * pinned buffer, so no group overwrites one still to be copied. */
    int *tab_h = e->h_enc, *tab_d = e->e_subtab;
    for (int g0 = 0; g0 < n;) {
        long s2 = 0;
        int g1 = g0;
        while (g1 < n) {
            const int tm = e->req[ids[g1]].T_mel, T1 = (tm + 1) / 2, T2 = (T1 + 1) / 2;
            const long b = (long)T2 * 32 * SUB_CH;
            if (g1 > g0 && 2 * (s2 + b) > e->sub_cap) break;
            s2 += b; g1++;
        }
        const int ng = g1 - g0, L = ng + 1;
        int *o1 = tab_h, *o2 = o1 + L, *o3 = o2 + L, *tm = o3 + L, *mo = tm + L;
        o1[0] = o2[0] = o3[0] = 0;
        for (int j = 0; j < ng; j++) {
            const HostReq *q = &e->req[ids[g0 + j]];
            const int T1 = (q->T_mel + 1) / 2, T2 = (T1 + 1) / 2;
            o1[j + 1] = o1[j] + T1;
            o2[j + 1] = o2[j] + T2;
            o3[j + 1] = o3[j] + q->T_enc;
            tm[j] = q->T_mel;
            mo[j] = mel_off[g0 + j];
        }
        ECHK(hipMemcpyAsync(tab_d, tab_h, (size_t)5 * L * sizeof(int), hipMemcpyHostToDevice, s));
        const int *d1 = tab_d, *d2 = d1 + L, *d3 = d2 + L, *dtm = d3 + L, *dmo = dtm + L;
        float *ra = e->esub;
        uint16_t *rb_h = (uint16_t *)(e->esub + s2), *rb_l = rb_h + s2;
        ctk_sub_conv0_dw_packed(rb_h, rb_l, e->emel, d1, d2, dtm, dmo, ng, o2[ng], DW(W->s0w), DW(W->s0b),
                                DW(W->s2w), DW(W->s2b), s);
        gemm_sp(e, rb_h, rb_l, o2[ng] * 32, SUB_CH, W->s3w, W->s3b, ra, SUB_CH, CT_EPI_RELU, 0);
        ctk_sub_dw_split_packed(rb_h, rb_l, ra, d2, d3, ng, o3[ng], 32, DW(W->s5w), DW(W->s5b), s);
        gemm_sp(e, rb_h, rb_l, o3[ng] * 16, SUB_CH, W->s6w, W->s6b, ra, SUB_CH, CT_EPI_RELU, 0);
        ctk_sub_flatten_split(e->emid_h + (size_t)seq_off[g0] * SUB_CH * 16,
                              e->emid_l + (size_t)seq_off[g0] * SUB_CH * 16, ra, o3[ng], s);
        tab_h += 5 * L;
        tab_d += 5 * L;
        g0 = g1;
    }
    free(mel_off);
    gemm_sp(e, e->emid_h, e->emid_l, M, SUB_CH * 16, W->sow, W->sob, e->ex, ENC_D, CT_EPI_STORE, 0);
    pos_tables(e);
    const long pos_rows = 2L * e->d.tmax - 1;
    /* the FFN projections in single-pass bf16 when configured: their inputs
     * (the LayerNorm and the SiLU outputs) as the hi plane alone */
    uint16_t *const ffl = e->cfg.enc_ffn_bf16 ? NULL : e->eln_l, *const ffm = e->cfg.enc_ffn_bf16 ? NULL : e->emid_l;
    for (int l = 0; l < ENC_N; l++) {
        const ELayer *L = &W->enc[l];
        /* x += 0.5 FFN1(LN x); past layer 0 the LayerNorm ran with the
         * previous layer's output norm */
        if (l == 0) ctk_layernorm_split(e->eln_h, ffl, e->ex, DW(L->ff1_lnw), DW(L->ff1_lnb), M, ENC_D, s);
        gemm_sp_silu_split(e, e->eln_h, ffl, M, L->ff1_w1, L->ff1_b1, e->emid_h, ffm);
        gemm_sp(e, e->emid_h, ffm, M, ENC_FF, L->ff1_w2, L->ff1_b2, e->ex, ENC_D, CT_EPI_FMADD, 0.5f);
        /* x += MHSA(LN x) */
        ctk_layernorm_split(e->eln_h, e->eln_l, e->ex, DW(L->sa_lnw), DW(L->sa_lnb), M, ENC_D, s);
        {
            /* Q, K, V in one launch: columns [0, 1280) to eq, then ek, ev */
            CtGemm g;
            memset(&g, 0, sizeof g);
            g.Ahi = e->eln_h; g.Alo = e->eln_l; g.lda = ENC_D;
            g.W = e->ew_qkv + (size_t)3 * l * ENC_D * ENC_D; g.bias = e->eb_qkv + (size_t)3 * l * ENC_D;
            g.M = M; g.N = 3 * ENC_D; g.K = ENC_D; g.epi = CT_EPI_STORE;
            g.nseg = 3; g.seg_w = ENC_D;
            float *const qkv[3] = {e->eq, e->ek, e->ev};
            for (int i = 0; i < 3; i++) g.seg[i] = (CtSeg){.mode = CT_OUT_DENSE, .base = qkv[i], .ld = ENC_D};
            ctk_gemm(&g, s);
        }
        ctk_relpos_attn_packed(NULL, e->eo_h, e->eo_l, e->eq, e->ek, e->ev,
                               e->ep_all + (size_t)l * pos_rows * ENC_D, e->d.tmax, DW(L->sa_pbu),
                               DW(L->sa_pbv), e->e_seq_off, e->e_seq_T, e->e_blk_seq, e->e_blk_q0, nblk,
                               T_max, s);
        gemm_sp(e, e->eo_h, e->eo_l, M, ENC_D, L->sa_ow, L->sa_ob, e->ex, ENC_D, CT_EPI_FMADD, 1.0f);
        /* x += Conv(LN x) */
        ctk_layernorm_split(e->eln_h, e->eln_l, e->ex, DW(L->cv_lnw), DW(L->cv_lnb), M, ENC_D, s);
        {
            CtGemm g;
            memset(&g, 0, sizeof g);
            g.Ahi = e->eln_h; g.Alo = e->eln_l; g.lda = ENC_D; g.W = DW(L->cv_pw1w); g.bias = DW(L->cv_pw1b);
            g.Y = e->eg; g.ldy = ENC_D; g.M = M; g.N = 2 * ENC_D; g.K = ENC_D;
            g.epi = CT_EPI_GLU; g.glu_half = ENC_D;
            ctk_gemm(&g, s);
        }
        ctk_dwconv_bn_silu_packed(e->edw_h, e->edw_l, e->eg, M, e->e_row_start, e->e_row_len,
                                  DW(L->cv_dww), DW(L->cv_dwb), DW(L->cv_bnw), DW(L->cv_bnb),
                                  DW(L->cv_bnmean), DW(L->cv_bnvar), s);
        gemm_sp(e, e->edw_h, e->edw_l, M, ENC_D, L->cv_pw2w, L->cv_pw2b, e->ex, ENC_D, CT_EPI_FMADD, 1.0f);
        /* x += 0.5 FFN2(LN x); x = LN(x), with the next layer's first
         * LayerNorm in the same pass */
        ctk_layernorm_split(e->eln_h, ffl, e->ex, DW(L->ff2_lnw), DW(L->ff2_lnb), M, ENC_D, s);
        gemm_sp_silu_split(e, e->eln_h, ffl, M, L->ff2_w1, L->ff2_b1, e->emid_h, ffm);
        gemm_sp(e, e->emid_h, ffm, M, ENC_FF, L->ff2_w2, L->ff2_b2, e->ex, ENC_D, CT_EPI_FMADD, 0.5f);
        if (l + 1 < ENC_N)
            ctk_layernorm_pair_split(e->ex, e->eln_h, ffl, DW(L->out_lnw), DW(L->out_lnb),
                                     DW(W->enc[l + 1].ff1_lnw), DW(W->enc[l + 1].ff1_lnb), M, ENC_D, s);
        else
            ctk_layernorm(e->ex, e->ex, DW(L->out_lnw), DW(L->out_lnb), M, ENC_D, s);
    }
    /* the encoder output, packed (the Q workspace is free now), goes to
     * each request's entry of enc_pool; cross K/V go straight into the
     * head-major cross caches of the entries */
    float *eh = e->eq;
    gemm(e, e->ex, M, ENC_D, W->prw, W->prb, eh, DEC_D, CT_EPI_STORE, 0, NULL);
    ctk_copy_rows(e->enc_pool, eh, e->e_dstrow, M, DEC_D, s);
    const size_t cross_l = (size_t)e->d.max_req * DEC_H * e->d.tmax * DEC_DK;
    ctk_split(e->eln_h, e->eln_l, eh, (long)M * DEC_D, s);   /* LN planes are free now */
    for (int l = 0; l < DEC_N; l++) {
        CtGemm g;
        memset(&g, 0, sizeof g);
        g.Ahi = e->eln_h; g.Alo = e->eln_l; g.lda = DEC_D;
        g.W = e->wckv + (size_t)2 * l * DEC_D * DEC_D; g.bias = e->bckv + (size_t)2 * l * DEC_D;
        g.M = M; g.N = 2 * DEC_D; g.K = DEC_D; g.epi = CT_EPI_STORE;
        g.nseg = 2; g.seg_w = DEC_D;
        const int mode = e->esz == 2 ? CT_OUT_HEADS_BF16 : CT_OUT_HEADS_F32;
        g.seg[0] = (CtSeg){.mode = mode, .base = (char *)e->kcross + l * cross_l * e->esz,
                           .rowoff = e->e_rowoff, .hstride = (long)e->d.tmax * DEC_DK};
        g.seg[1] = (CtSeg){.mode = mode, .base = (char *)e->vcross + l * cross_l * e->esz,
                           .rowoff = e->e_rowoff, .hstride = (long)e->d.tmax * DEC_DK};
        ctk_gemm(&g, s);
    }
    ECHK(hipStreamSynchronize(s));
    free(row_start); free(row_len); free(dstrow); free(rowoff); free(seq_off); free(seq_T); free(blk_seq);
    free(blk_q0);
}

/* Copies n ints src[0..n) into the device ring dst at positions [lo, lo + n)
 * (wrapping), on stream s. */
static void ring_put_seq(HipbEngine *e, int *dst, const int *src, long lo, int n, hipStream_t s) {
    if (n <= 0) return;
    const int mask = e->ring - 1, a = (int)(lo & mask), n1 = n < e->ring - a ? n : e->ring - a;
    ECHK(hipMemcpyAsync(dst + a, src, (size_t)n1 * sizeof(int), hipMemcpyHostToDevice, s));
    if (n > n1) ECHK(hipMemcpyAsync(dst, src + n1, (size_t)(n - n1) * sizeof(int), hipMemcpyHostToDevice, s));
}

/* Publishes the encoded requests ids[0..n) (their cross K/V are written: the
 * encoder stream has been drained): their encoder entries into their
 * request-ring slots (an entry >= 0 marks a request encoded; a released
 * chained successor is admitted only then), the publication count q[7],
 * then the requests that wait for no predecessor appended to the fresh
 * queue in the order given (the ids first, then the new count).  All copies
 * go on the encoder stream, which is then drained; the step kernel reads the
 * words with acquire loads, possibly while running on the other stream. */
static void publish(HipbEngine *e, const int *ids, int n) {
    const int P = e->d.max_req;
    int *words = e->h_enc + 10 * P + 8;   /* [0] publications, [1] fresh count */
    int *fresh = e->h_enc + 10 * P + 16, *pairs = fresh + P, k = 0;
    /* at most P requests hold entries, so n <= P */
    if (n > P) CT_FATAL("publish: more requests than encoder entries");
    for (int i = 0; i < n; i++) {
        pairs[2 * i] = ids[i];
        pairs[2 * i + 1] = e->req[ids[i]].entry;
    }
    if (n) {
        ECHK(hipMemcpyAsync(e->d_pairs, pairs, (size_t)2 * n * sizeof(int), hipMemcpyHostToDevice, e->enc_s));
        ctk_ring_scatter(e->d.req_entry, e->d_pairs, n, e->ring - 1, e->enc_s);
    }
    words[0] = ++e->n_pub;
    ECHK(hipMemcpyAsync(e->d.q + 7, &words[0], sizeof(int), hipMemcpyHostToDevice, e->enc_s));
    for (int i = 0; i < n; i++)
        if (!e->req[ids[i]].chained) fresh[k++] = ids[i];
    if (k) {
        ring_put_seq(e, e->d.fq, fresh, e->fq_count, k, e->enc_s);
        e->fq_count += k;
        words[1] = e->fq_count;
        ECHK(hipMemcpyAsync(e->d.q + 5, &words[1], sizeof(int), hipMemcpyHostToDevice, e->enc_s));
    }
    ECHK(hipStreamSynchronize(e->enc_s));
    atomic_store(&e->published, e->n_pub);
}

static void release_inputs(HipbEngine *e, const int *ids, int n) {
    for (int i = 0; i < n; i++) {
        HostReq *q = &e->req[ids[i]];
        free(q->mel); q->mel = NULL;
        free(q->pcm); q->pcm = NULL;
    }
}

/* The next batch of not yet encoded requests in encode order: positions
 * [p, p1) of e->order with at most max_batch_frames encoder frames and at
 * most max_n requests (at least one request). */
static int next_batch(const HipbEngine *e, int p, int max_batch_frames, int max_n) {
    int frames = 0, p1 = p;
    while (p1 < e->n_req &&
           (p1 == p || (frames + e->req[e->order[p1]].T_enc <= max_batch_frames && p1 - p < max_n))) {
        frames += e->req[e->order[p1]].T_enc;
        p1++;
    }
    return p1;
}

typedef struct { int key, id; } OrderKey;

static int order_cmp(const void *a, const void *b) {
    const OrderKey *x = a, *y = b;
    return x->key != y->key ? (x->key < y->key ? -1 : 1) : (x->id < y->id ? -1 : x->id > y->id);
}

/* Encode (and so admission) order of the requests not yet encoded: as
 * submitted, or with admit_order 1 the largest token budget first (a
 * recording's chunks keep their order, together, under the first chunk's
 * budget).  Longest-first shortens the pass: fewer slots idle at its end. */
static void plan_order(HipbEngine *e) {
    const int p0 = e->n_enc, n = e->n_req - p0;
    if (e->cfg.admit_order != 1 || n < 2) return;
    OrderKey *k = malloc((size_t)n * sizeof *k);
    if (!k) CT_FATAL("out of host memory");
    for (int i = 0; i < n; i++) {
        const int r = e->order[p0 + i];
        int h = r;
        while (e->req[h].chained) h--;
        k[i] = (OrderKey){-e->req[h].limit, r};
    }
    qsort(k, (size_t)n, sizeof *k, order_cmp);
    for (int i = 0; i < n; i++) e->order[p0 + i] = k[i].id;
    free(k);
}

/* Encoder entries free right now (thread-safe). */
static int free_entries(HipbEngine *e) {
    pthread_mutex_lock(&e->mu);
    const int n = (int)(e->free_tail - e->free_head);
    pthread_mutex_unlock(&e->mu);
    return n;
}

/* Gives the requests at encode positions [p0, p1) encoder entries from the
 * free FIFO (the caller made sure there are enough). */
static void take_entries(HipbEngine *e, int p0, int p1) {
    const int P = e->d.max_req;
    pthread_mutex_lock(&e->mu);
    if (e->free_tail - e->free_head < p1 - p0) CT_FATAL("encode: fewer free encoder entries than requests");
    for (int p = p0; p < p1; p++) {
        const int r = e->order[p], ent = e->free_ent[e->free_head++ % P];
        e->req[r].entry = ent;
        e->ent_owner[ent] = r;
    }
    atomic_store(&e->n_assigned, p1);
    pthread_mutex_unlock(&e->mu);
}

/* Marks the requests that retired since the last call (the device's
 * retirement ring, up to `finished` of them) done and returns their
 * encoder entries to the free FIFO.  Synchronises the engine stream. */
static void recycle(HipbEngine *e, int finished) {
    const int n = finished - e->ret_seen;
    if (n <= 0) return;
    if (n > e->ring)
        CT_FATAL("recycle: more requests retired than the retirement ring holds since the host last "
                 "looked (stepping with hipb_step alone: call hipb_finished between steps)");
    const int mask = e->ring - 1, a = e->ret_seen & mask, n1 = n < e->ring - a ? n : e->ring - a;
    ECHK(hipMemcpyAsync(e->h_ret, e->d.ret + a, (size_t)n1 * sizeof(int), hipMemcpyDeviceToHost, e->s));
    if (n > n1)
        ECHK(hipMemcpyAsync(e->h_ret + n1, e->d.ret, (size_t)(n - n1) * sizeof(int), hipMemcpyDeviceToHost, e->s));
    ECHK(hipStreamSynchronize(e->s));
    const int P = e->d.max_req;
    pthread_mutex_lock(&e->mu);
    for (int i = 0; i < n; i++) {
        const int r = e->h_ret[i];
        if (r < 0 || r >= e->n_req) CT_FATAL("recycle: bad retired request id");
        HostReq *q = &e->req[r];
        q->done = 1;
        if (q->entry >= 0 && e->ent_owner[q->entry] == r) e->free_ent[e->free_tail++ % P] = q->entry;
    }
    pthread_cond_broadcast(&e->cv);
    pthread_mutex_unlock(&e->mu);
    e->ret_seen = finished;
}

/* True when requests without an entry outnumber the free entries, so that
 * retired requests' entries should be recycled. */
static int entries_short(HipbEngine *e) {
    return e->n_req - atomic_load(&e->n_assigned) > free_entries(e);
}

/* Encodes (on the engine's encoder stream, synchronously) the submitted
 * requests not yet encoded, as far as free encoder entries go, and
 * publishes them. */
static void encode_available(HipbEngine *e, int max_batch_frames) {
    plan_order(e);
    int p = e->n_enc;
    while (p < e->n_req) {
        const int avail = free_entries(e);
        if (!avail) break;
        const int p1 = next_batch(e, p, max_batch_frames, avail);
        take_entries(e, p, p1);
        encode_batch(e, e->order + p, p1 - p);
        release_inputs(e, e->order + p, p1 - p);
        p = p1;
    }
    const int p0 = e->n_enc;
    e->n_enc = p;
    publish(e, e->order + p0, p - p0);
}

void hipb_encode(HipbEngine *e, int max_batch_frames) {
    flush_meta(e);
    if (max_batch_frames < e->d.tmax) max_batch_frames = e->d.tmax;
    e->batch_frames = max_batch_frames;
    if (e->n_enc < e->n_req && entries_short(e)) {
        int q[CT_Q_WORDS];
        read_queue(e, q);
        recycle(e, q[2]);
    }
    encode_available(e, max_batch_frames);
}

/* ------------------------------------------------------------------ */
/* The decode step                                                     */
/* ------------------------------------------------------------------ */
/* Decode attention of every slot; the output goes split into attf (frag
 * layout) for the out-projection.  The query is q (self) or the Q
 * projection's K-slice partials plus bias (cross). */
/* Decode GEMMs read the tiled weight copies (one contiguous 1 KB per
 * wavefront load).  Launches that read the next decode GEMMs' weight tiles
 * ahead into the L2 their workgroups read from (CT_WARM_ROWS read-ahead
 * workgroups per XCD): the LayerNorm before each layer's QKV projection
 * reads that projection's; the self attention the out- and cross-query
 * projections'; the cross attention the FFN's; the final residual update
 * half of the LM head's.  HIPB_READ_AHEAD=0 at engine creation turns it off. */
#define CT_WARM_ROWS 32
/* LM-head columns the final residual update reads ahead */
#define CT_WARM_LM_COLS 8192
/* Queues the weight tiles of the launch gv() makes for (Wd, N, K, out) for
 * the next attention or LayerNorm launch to read ahead. */
static void warm_add(HipbEngine *e, const uint16_t *Wd, int N, int K, int out) {
    if (e->warm.n >= 4) return;
    CtGemv g;
    memset(&g, 0, sizeof g);
    g.W = Wd; g.wtile = 1; g.M = e->M; g.N = N; g.K = K; g.out = out;
    g.ksplit = out == CT_GV_PARTIAL ? ctk_gemv_ksplit(N, K) : 1;
    ctk_gemv_warm(&g, &e->warm.t[e->warm.n++]);
}

/* Hands the queued read-ahead to a launch and clears the queue. */
static void warm_take(HipbEngine *e, CtWarmSet *ws) {
    memset(ws, 0, sizeof *ws);
    if (!e->warm.n) return;
    *ws = e->warm;
    ws->rows = CT_WARM_ROWS;
    ws->magic = 0x5bd1e995u;
    ws->sink = e->warm_sink;
    e->warm.n = 0;
}

static void attn(HipbEngine *e, const void *K, const void *V, long item_stride, long head_stride,
                 int rows, const int *lens, const int *kv_index, int kv_direct, const int *rank) {
    CtAttn a;
    memset(&a, 0, sizeof a);
    a.Q = e->q; a.q_sb = DEC_D; a.q_st = DEC_D;
    a.K = K; a.V = V; a.kv_bf16 = e->esz == 2;
    a.kv_sb = item_stride; a.kv_st = DEC_DK; a.kv_sh = head_stride;
    a.lens = lens; a.lens_step = 1; a.kv_index = kv_index; a.kv_direct = kv_direct; a.kv_rows = rows;
    a.rank = e->M >= e->d.rank_min ? rank : NULL;
    a.T_q = 1; a.B = e->M; a.H = DEC_H;
    a.scale = 0.08838834764831845f;   /* 1/sqrt(128) */
    a.out_frag = e->attf;
    warm_take(e, &a.warm);
    ctk_attn(&a, e->s);
}

static void self_kv(HipbEngine *e, int l, void **k, void **v) {
    const size_t per = (size_t)e->d.slots * DEC_H * e->d.kv_rows * DEC_DK * e->esz;
    *k = (char *)e->kself + l * per;
    *v = (char *)e->vself + l * per;
}

static void cross_kv(HipbEngine *e, int l, void **k, void **v) {
    const size_t per = (size_t)e->d.max_req * DEC_H * e->d.tmax * DEC_DK * e->esz;
    *k = (char *)e->kcross + l * per;
    *v = (char *)e->vcross + l * per;
}

static void step_attention(HipbEngine *e, int l, int cross) {
    void *k, *v;
    if (!cross) {
        self_kv(e, l, &k, &v);
        /* row s is slot s's own row: only the spare rows of a wide step
         * need the row -> slot table, and only they wait for it */
        attn(e, k, v, (long)DEC_H * e->d.kv_rows * DEC_DK, (long)e->d.kv_rows * DEC_DK, e->d.kv_rows,
             e->d.pos_len, e->M > e->d.slots ? e->d.row_slot : NULL, e->d.slots, e->d.rank_self);
    } else {
        cross_kv(e, l, &k, &v);
        attn(e, k, v, (long)DEC_H * e->d.tmax * DEC_DK, (long)e->d.tmax * DEC_DK, e->d.tmax,
             e->d.cross_len, e->d.cross_idx, 0, e->d.rank_cross);
    }
}

/* A decode GEMM launch, or (bench_floor) its weight reads alone. */
static void launch_gemv(HipbEngine *e, const CtGemv *g) {
    if (!e->bench_floor) {
        ctk_gemv(g, e->s);
        return;
    }
    if (ctk_gemv_read_floor_blocks(g) > e->floor_cap) CT_FATAL("hipb_bench_read_floor: sink too small");
    ctk_gemv_read_floor(g, e->floor_sink, e->s);
}

/* A decode GEMM over all rows on LayerNorm(h), the LayerNorm folded in: A
 * is lnf = frag(h * w), written with the row statistics by the residual
 * projection (or the embedding) before it; c = the GEMM's (c1, c2). */
static void gv_fold(HipbEngine *e, const uint16_t *Wd, const float *const c[2], int N, int out, int relu,
                    float *Y, long ldy, uint16_t *F) {
    CtGemv g;
    memset(&g, 0, sizeof g);
    g.A = e->lnf; g.W = Wd; g.wtile = 1;
    g.M = e->M; g.N = N; g.K = DEC_D; g.ksplit = 1;
    g.m_active = e->M > e->d.slots ? e->d.q + 6 : NULL;
    g.out = out; g.relu = relu;
    g.lnstat = e->lnstat; g.fold_c1 = c[0]; g.fold_c2 = c[1];
    g.Y = Y; g.ldy = ldy; g.F = F;
    launch_gemv(e, &g);
}

/* A plain decode GEMM over all rows into a dense output (the LM head). */
static void gv_dense(HipbEngine *e, const uint16_t *A, const uint16_t *Wd, const uint16_t *bd, int N, int K,
                     float *Y, long ldy) {
    CtGemv g;
    memset(&g, 0, sizeof g);
    g.A = A; g.W = Wd; g.bias = bd; g.wtile = 1;
    g.M = e->M; g.N = N; g.K = K; g.ksplit = 1;
    g.m_active = e->M > e->d.slots ? e->d.q + 6 : NULL;
    g.out = CT_GV_DENSE;
    g.Y = Y; g.ldy = ldy;
    launch_gemv(e, &g);
}

/* A K-split decode GEMM: its slices' partial sums go to parts. */
static void gv_partial(HipbEngine *e, const uint16_t *A, const uint16_t *Wd, int N, int K) {
    CtGemv g;
    memset(&g, 0, sizeof g);
    g.A = A; g.W = Wd; g.wtile = 1;
    g.M = e->M; g.N = N; g.K = K; g.ksplit = ctk_gemv_ksplit(N, K);
    g.m_active = e->M > e->d.slots ? e->d.q + 6 : NULL;
    g.out = CT_GV_PARTIAL;
    g.Y = e->parts;
    launch_gemv(e, &g);
}

/* Output projection onto the residual rows (h += A W^T + b) that leaves the
 * input of the next GEMM with its LayerNorm (gain lnw) folded in: the rows'
 * statistics per 32-column block in lnstat and lnf = frag(h * lnw). */
static void gv_resid(HipbEngine *e, const uint16_t *A, const uint16_t *Wd, const uint16_t *bd, int K,
                     const uint16_t *lnw) {
    CtGemv g;
    memset(&g, 0, sizeof g);
    g.A = A; g.W = Wd; g.bias = bd; g.wtile = 1;
    g.M = e->M; g.N = DEC_D; g.K = K; g.ksplit = 1;
    g.m_active = e->M > e->d.slots ? e->d.q + 6 : NULL;
    g.out = CT_GV_RESID;
    g.Y = e->h; g.ldy = DEC_D; g.lnstat = e->lnstat;
    g.F = e->lnf; g.fold_w = lnw;
    launch_gemv(e, &g);
}

/* One decode step over slots rows, or (wide) over slots + prefill_rows rows
 * whose spare rows feed prompts several tokens a step.  full == 0 launches
 * only its GEMMs (timing support).
 *
 * Every LayerNorm of the decoder but the last runs inside the GEMM that
 * consumes it: the residual projections of the attention outputs, the
 * residual update after the FFN and the embedding leave h, its block
 * statistics and frag(h * w) of the next LayerNorm's gain, and the next GEMM
 * corrects each row in its epilogue (gemv_kernel FOLD).  A layer is 9
 * launches: QKV, self attention, out projection, cross query, cross
 * attention, cross out projection, FFN up, FFN down (8 K-slices), residual
 * update (the next layer's, or with the final LayerNorm before the LM
 * head). */
static void step_kernels(HipbEngine *e, int full, int wide) {
    const Weights *W = &e->W;
    const int B = wide ? e->d.rows : e->d.slots;
    hipStream_t s = e->s;
    e->M = B;
    if (full) ctk_eng_begin(&e->d, B - e->d.slots, s);
    for (int l = 0; l < DEC_N; l++) {
        const DLayer *L = &W->dec[l];
        void *ks, *vs;
        self_kv(e, l, &ks, &vs);
        const uint16_t *w_qkv = e->wt_qkv[l], *w_o = e->wt_o[l], *w_cq = e->wt_cq[l];
        const uint16_t *w_co = e->wt_co[l], *w_f1 = e->wt_f1[l], *w_f2 = e->wt_f2[l];
        if (full && e->read_ahead) warm_add(e, w_qkv, 3 * DEC_D, DEC_D, CT_GV_QKV);
        if (full && l == 0) {
            /* h = the embedding LayerNorm, with the first layer's folded input */
            CtWarmSet ws;
            warm_take(e, &ws);
            ctk_embed_fold(e->h, e->lnstat, e->lnf, e->d.tok, e->d.pos_len, e->d.act, DW(W->etw),
                           DW(W->epw), DW(W->elnw), DW(W->elnb), DW(L->sa_lnw), B, &ws, s);
        } else if (full) {
            /* h += the previous layer's FFN (its K-slices and bias), with this
             * layer's folded input */
            CtWarmSet ws;
            warm_take(e, &ws);
            ctk_resid_fold(e->h, e->lnstat, e->lnf, e->parts, ctk_gemv_ksplit(DEC_D, DEC_FF),
                           DW(W->dec[l - 1].ffn_b2), DW(L->sa_lnw), NULL, B, &ws, s);
        }
        CtGemv g;
        memset(&g, 0, sizeof g);
        g.A = e->lnf;
        g.W = w_qkv; g.wtile = 1;
        g.M = B; g.N = 3 * DEC_D; g.K = DEC_D; g.ksplit = 1; g.out = CT_GV_QKV;
        g.m_active = B > e->d.slots ? e->d.q + 6 : NULL;
        g.lnstat = e->lnstat; g.fold_c1 = e->fc_qkv[l][0]; g.fold_c2 = e->fc_qkv[l][1];
        g.Y = e->q; g.ldy = DEC_D;
        g.kc = ks; g.vc = vs; g.rowoff = e->d.kv_rowoff; g.hstride = (long)e->d.kv_rows * DEC_DK;
        g.kv_bf16 = e->esz == 2;
        launch_gemv(e, &g);
        if (full && e->read_ahead) warm_add(e, w_o, DEC_D, DEC_D, CT_GV_RESID);
        if (full && e->read_ahead) warm_add(e, w_cq, DEC_D, DEC_D, CT_GV_DENSE);
        if (full) step_attention(e, l, 0);
        /* h += self-attention out-projection; the cross-attention query from
         * LayerNorm(h) */
        gv_resid(e, e->attf, w_o, DW(L->sa_ob), DEC_D, DW(L->ca_lnw));
        gv_fold(e, w_cq, e->fc_cq[l], DEC_D, CT_GV_DENSE, 0, e->q, DEC_D, NULL);
        if (full && e->read_ahead) warm_add(e, w_f1, DEC_FF, DEC_D, CT_GV_FRAG);
        if (full && e->read_ahead) warm_add(e, w_f2, DEC_D, DEC_FF, CT_GV_PARTIAL);
        if (full) step_attention(e, l, 1);
        /* h += cross-attention out-projection; the FFN on LayerNorm(h), its
         * down projection in K-slices summed into h by the next launch */
        gv_resid(e, e->attf, w_co, DW(L->ca_ob), DEC_D, DW(L->ffn_lnw));
        gv_fold(e, w_f1, e->fc_f1[l], DEC_FF, CT_GV_FRAG, 1, NULL, 0, e->midf);
        gv_partial(e, e->midf, w_f2, DEC_D, DEC_FF);
    }
    /* h += the last FFN, then the final LayerNorm */
    if (full) {
        /* that launch reads the LM head's first CT_WARM_LM_COLS columns of
         * weights ahead (16.8 MB: the whole head, 33.6 MB, does not stay in
         * the L2s); workgroup i of the LM head keeps its XCD whatever the
         * column count, so a prefix GEMM's tiles are the head's own */
        CtWarmSet lws;
        memset(&lws, 0, sizeof lws);
        if (e->read_ahead) {
            const int rows = e->M;
            e->M = e->d.slots;
            warm_add(e, e->wt_lm, CT_WARM_LM_COLS, DEC_D, CT_GV_DENSE);
            e->M = rows;
            warm_take(e, &lws);
        }
        ctk_resid_fold(e->h, e->lnstat, e->lnf, e->parts, ctk_gemv_ksplit(DEC_D, DEC_FF),
                       DW(W->dec[DEC_N - 1].ffn_b2), DW(W->dlnw), DW(W->dlnb), B, &lws, s);
    }
    /* logits only for the slots' own rows */
    e->M = e->d.slots;
    gv_dense(e, e->lnf, e->wt_lm, DW(W->hdb), VOCAB, DEC_D, e->logits, VOCAB);
    if (full) ctk_eng_end(&e->d, e->logits, s);
    e->M = e->d.slots;
}

static void step_launch(HipbEngine *e, int wide) { step_kernels(e, 1, wide); }

/* With spare prompt rows every step is the wide one: a request admitted by
 * any step has its prompt fed at once, and while no spare row is in use the
 * GEMM workgroups past the slots' rows exit at once (q[6]). */
static int want_wide(const HipbEngine *e) { return e->d.rows > e->d.slots; }

static void read_queue(HipbEngine *e, int *q);

void hipb_step(HipbEngine *e) {
    flush_meta(e);
    step_launch(e, want_wide(e));
}

void hipb_attention_only(HipbEngine *e) {
    for (int l = 0; l < DEC_N; l++) {
        step_attention(e, l, 0);
        step_attention(e, l, 1);
    }
}

/* Reads the queue words (synchronises). */
static void read_queue(HipbEngine *e, int *q) {
    ECHK(hipMemcpyAsync(e->h_tmp, e->d.q, CT_Q_WORDS * sizeof(int), hipMemcpyDeviceToHost, e->s));
    ECHK(hipStreamSynchronize(e->s));
    memcpy(q, e->h_tmp, CT_Q_WORDS * sizeof(int));
}

static void recycle(HipbEngine *e, int finished);

int hipb_finished(HipbEngine *e) {
    int q[CT_Q_WORDS];
    read_queue(e, q);
    recycle(e, q[2]);
    return q[2];
}

/* Steps a run or process loop may launch between two looks at the queue:
 * fewer than a quarter of the retirement ring can fill meanwhile. */
static int clamp_chunk(const HipbEngine *e, int chunk) {
    const int most = e->ring / (4 * e->d.slots);
    return chunk < 1 ? 1 : chunk > most ? most : chunk;
}

static void ensure_graph(HipbEngine *e, int wide) {
    if (e->have_graph[wide] || e->eager) return;
    ECHK(hipStreamBeginCapture(e->s, hipStreamCaptureModeThreadLocal));
    step_launch(e, wide);
    ECHK(hipStreamEndCapture(e->s, &e->graph[wide]));
    ECHK(hipGraphInstantiate(&e->exec[wide], e->graph[wide], NULL, NULL, 0));
    e->have_graph[wide] = 1;
}

static void launch_step(HipbEngine *e, int wide) {
    if (e->eager) step_launch(e, wide);
    else ECHK(hipGraphLaunch(e->exec[wide], e->s));
}

void hipb_bench_steps(HipbEngine *e, int n) {
    const int wide = want_wide(e);
    ensure_graph(e, wide);
    for (int i = 0; i < n; i++) launch_step(e, wide);
}

long hipb_run(HipbEngine *e, int chunk) {
    flush_meta(e);
    chunk = clamp_chunk(e, chunk);
    const int spare = e->d.rows - e->d.slots;
    ensure_graph(e, 0);
    if (spare) ensure_graph(e, 1);
    if (e->batch_frames < e->d.tmax) e->batch_frames = 8192 > e->d.tmax ? 8192 : e->d.tmax;
    long steps = 0;
    /* every admitted request finishes within prompt + limit <= prompt +
     * MAX_SEQ steps of its admission, and some request is admitted whenever
     * a slot frees up */
    const long bound = (long)(e->n_req + 2) * (MAX_SEQ + CT_PROMPT_MAX + 1);
    for (;;) {
        int q[CT_Q_WORDS];
        read_queue(e, q);
        if (q[2] - e->ret_seen >= e->ring / 4) recycle(e, q[2]);
        if (e->n_enc < e->n_req) {
            /* requests still waiting for an encoder entry: take those that
             * retired requests returned */
            recycle(e, q[2]);
            const int before = e->n_enc;
            encode_available(e, e->batch_frames);
            if (e->n_enc > before) continue;
        }
        if (q[2] >= e->n_req) {
            recycle(e, q[2]);
            break;
        }
        if (steps > bound) CT_FATAL("hipb_run: requests did not finish within the step bound");
        const int wide = want_wide(e);
        for (int i = 0; i < chunk; i++) launch_step(e, wide);
        steps += chunk;
    }
    return steps;
}

/* hipb_process: the encoder runs on a worker thread and the second stream,
 * publishing each batch to the fresh queue as soon as its cross K/V are
 * written, while the calling thread keeps launching decode steps and
 * returns retired requests' encoder entries to the free FIFO when the
 * encoder is short of them. */
static void *enc_worker(void *arg) {
    HipbEngine *e = arg;
    ECHK(hipSetDevice(e->dev));
    ct_t.dev = e->dev;                 /* weight pointers translate per device */
    int batches = 0;
    for (int p = e->n_enc; p < e->n_req;) {
        pthread_mutex_lock(&e->mu);
        while (e->free_tail == e->free_head) pthread_cond_wait(&e->cv, &e->mu);
        const int avail = (int)(e->free_tail - e->free_head);
        pthread_mutex_unlock(&e->mu);
        const int p1 = next_batch(e, p, e->proc_batch, avail);
        take_entries(e, p, p1);
        encode_batch(e, e->order + p, p1 - p);
        release_inputs(e, e->order + p, p1 - p);
        publish(e, e->order + p, p1 - p);
        p = p1;
        if (++batches == e->hold_batches) {
            /* test support: a bounded host-side wait (60 s) */
            int waited = 0;
            while (atomic_load(&e->seen_finished) < e->hold_finished && waited < 600000) {
                usleep(100);
                waited++;
            }
            e->hold_expired = atomic_load(&e->seen_finished) < e->hold_finished;
        }
    }
    atomic_store(&e->enc_done, 1);
    return NULL;
}

long hipb_process(HipbEngine *e, int max_batch_frames, int chunk) {
    flush_meta(e);
    chunk = clamp_chunk(e, chunk);
    if (max_batch_frames < e->d.tmax) max_batch_frames = e->d.tmax;
    const int spare = e->d.rows - e->d.slots;
    /* graphs captured and every encoder buffer sized before the worker
     * starts: no capture, allocation or free runs beside the other stream.
     * The worker's batches are cut by frames and by the free entries, so
     * each lies inside the frames-only batch that starts where it starts:
     * sizing for those from every start covers them all. */
    ensure_graph(e, 0);
    if (spare) ensure_graph(e, 1);
    plan_order(e);
    {
        int frames_max = 0, tmel_max = 0;
        for (int p = e->n_enc; p < e->n_req; p++) {
            const int p1 = next_batch(e, p, max_batch_frames, e->n_req);
            int f = 0;
            for (int i = p; i < p1; i++) {
                f += e->req[e->order[i]].T_enc;
                if (e->req[e->order[i]].T_mel > tmel_max) tmel_max = e->req[e->order[i]].T_mel;
            }
            if (f > frames_max) frames_max = f;
            batch_buffers(e, e->order + p, p1 - p);
        }
        if (frames_max) {
            enc_reserve(e, frames_max, tmel_max);
            pos_tables(e);
        }
    }
    ECHK(hipStreamSynchronize(e->s));
    e->enc_s = e->s2;
    e->proc_batch = max_batch_frames;
    atomic_store(&e->enc_done, 0);
    atomic_store(&e->seen_finished, 0);
    e->hold_expired = 0;
    pthread_t th;
    if (pthread_create(&th, NULL, enc_worker, e)) CT_FATAL("hipb_process: cannot start the encoder thread");
    long steps = 0;
    const long bound = (long)(e->n_req + 2) * (MAX_SEQ + CT_PROMPT_MAX + 1);
    for (;;) {
        int q[CT_Q_WORDS];
        read_queue(e, q);
        atomic_store(&e->seen_finished, q[2]);
        if (entries_short(e) || q[2] - e->ret_seen >= e->ring / 4) recycle(e, q[2]);
        const int done = atomic_load(&e->enc_done);
        if (done && q[2] >= e->n_req) {
            recycle(e, q[2]);
            break;
        }
        /* every admitted request finished and none can be admitted: wait
         * for the encoder instead of stepping empty slots.  No successor
         * waits (released q[10] = admitted q[0]), or the one at the ring's
         * head waits for its encoding (q[8]) and nothing was published since
         * that admission saw the watermark (q[9]). */
        const int ring_idle = q[10] <= q[0] || (q[8] && q[9] >= atomic_load(&e->published));
        if (!done && q[2] >= q[0] + q[4] && ring_idle && q[4] >= q[5]) {
            usleep(50);
            continue;
        }
        if (steps > bound) CT_FATAL("hipb_process: requests did not finish within the step bound");
        const int wide = want_wide(e);
        for (int i = 0; i < chunk; i++) launch_step(e, wide);
        steps += chunk;
    }
    pthread_join(th, NULL);
    e->enc_s = e->s;
    e->n_enc = e->n_req;
    return steps;
}

void hipb_test_hold_encoder(HipbEngine *e, int after_batches, int until_finished) {
    e->hold_batches = after_batches;
    e->hold_finished = until_finished;
}

int hipb_test_hold_expired(HipbEngine *e) { return e->hold_expired; }

/* ------------------------------------------------------------------ */
/* Results                                                             */
/* ------------------------------------------------------------------ */
/* Tokens (what = 0) or scores (what = 1) of request req: from the host copy
 * once its ring slot was handed to a later request, else from the slot. */
static int req_results(HipbEngine *e, int req, void *out, int cap, int what) {
    if (req < 0 || req >= e->n_req) return 0;
    const HostReq *q = &e->req[req];
    int n = 0;
    if (q->collected) {
        n = q->n_out < cap ? q->n_out : cap;
        if (n > 0) memcpy(out, what ? (const void *)q->score : (const void *)q->out, (size_t)n * 4);
        return n;
    }
    /* fields not uploaded yet: the ring slot may still hold the results of
     * request req - ring */
    if (req >= e->meta_lo) return 0;
    const size_t slot = (size_t)(req & (e->ring - 1));
    ECHK(hipStreamSynchronize(e->s));
    ECHK(hipMemcpy(&n, e->d.req_ngen + slot, sizeof(int), hipMemcpyDeviceToHost));
    if (n > cap) n = cap;
    if (n > 0) {
        const void *src = what ? (const void *)(e->d.req_score + slot * e->d.smax)
                               : (const void *)(e->d.req_out + slot * e->d.smax);
        ECHK(hipMemcpy(out, src, (size_t)n * 4, hipMemcpyDeviceToHost));
    }
    return n;
}

int hipb_tokens(HipbEngine *e, int req, int *out, int cap) { return req_results(e, req, out, cap, 0); }

int hipb_token_scores(HipbEngine *e, int req, float *out, int cap) { return req_results(e, req, out, cap, 1); }

int hipb_slot_of(HipbEngine *e, int req) {
    ECHK(hipStreamSynchronize(e->s));
    ECHK(hipMemcpy(e->h_tmp, e->d.slot_req, e->d.slots * sizeof(int), hipMemcpyDeviceToHost));
    for (int s = 0; s < e->d.slots; s++)
        if (e->h_tmp[s] == req) return s;
    return -1;
}

void hipb_logits(HipbEngine *e, int slot, float *out) {
    ECHK(hipStreamSynchronize(e->s));
    ECHK(hipMemcpy(out, e->logits + (size_t)slot * VOCAB, VOCAB * sizeof(float), hipMemcpyDeviceToHost));
}

void hipb_enc_out(HipbEngine *e, int req, float *out) {
    if (req < 0 || req >= e->n_req) CT_FATAL("hipb_enc_out: no such request");
    pthread_mutex_lock(&e->mu);
    const int ent = e->req[req].entry, owner = ent >= 0 ? e->ent_owner[ent] : -1;
    pthread_mutex_unlock(&e->mu);
    if (ent < 0) CT_FATAL("hipb_enc_out: request not encoded");
    if (owner != req)
        CT_FATAL("hipb_enc_out: the request's encoder entry was recycled for a later request");
    ECHK(hipStreamSynchronize(e->s));
    ECHK(hipMemcpy(out, e->enc_pool + (size_t)ent * e->d.tmax * DEC_D,
                   (size_t)e->req[req].T_enc * DEC_D * sizeof(float), hipMemcpyDeviceToHost));
}

/* ------------------------------------------------------------------ */
/* Microbenchmark state                                                */
/* ------------------------------------------------------------------ */
void hipb_bench_fill(HipbEngine *e, const int *S, const int *T_enc, uint64_t seed) {
    const int B = e->d.slots;
    if (e->n_req) CT_FATAL("hipb_bench_fill: engine already has requests");
    if (B > e->d.max_req) CT_FATAL("hipb_bench_fill: needs max_requests >= slots");
    int *buf = e->h_tmp;
    for (int s = 0; s < B; s++) {
        if (S[s] < 1 || S[s] > e->d.smax - 64) CT_FATAL("hipb_bench_fill: S outside [1, max_tokens-64]");
        if (T_enc[s] < 1 || T_enc[s] > e->d.tmax) CT_FATAL("hipb_bench_fill: T_enc outside [1, max_frames]");
    }
    /* one synthetic request per slot: no prompt, one generated token, never
     * finishes within the benchmark (limit max_tokens, EOS suppressed) */
    for (int s = 0; s < B; s++) buf[s] = s;
    ECHK(hipMemcpy(e->d.slot_req, buf, B * sizeof(int), hipMemcpyHostToDevice));
    for (int s = 0; s < B; s++) buf[s] = S[s] - 1;
    ECHK(hipMemcpy(e->d.slot_S, buf, B * sizeof(int), hipMemcpyHostToDevice));
    ECHK(hipMemcpy(e->d.req_T, T_enc, B * sizeof(int), hipMemcpyHostToDevice));
    for (int s = 0; s < B; s++) buf[s] = e->d.smax;
    ECHK(hipMemcpy(e->d.req_limit, buf, B * sizeof(int), hipMemcpyHostToDevice));
    for (int s = 0; s < B; s++) buf[s] = HIPB_SUPPRESS_EOS;
    ECHK(hipMemcpy(e->d.req_flags, buf, B * sizeof(int), hipMemcpyHostToDevice));
    for (int s = 0; s < B; s++) buf[s] = 0;
    ECHK(hipMemcpy(e->d.req_np, buf, B * sizeof(int), hipMemcpyHostToDevice));
    for (int s = 0; s < B; s++) buf[s] = 1;
    ECHK(hipMemcpy(e->d.req_ngen, buf, B * sizeof(int), hipMemcpyHostToDevice));
    for (int s = 0; s < B; s++)
        ECHK(hipMemcpy(e->d.req_out + (size_t)s * e->d.smax, &(int){100 + s}, sizeof(int), hipMemcpyHostToDevice));
    /* request s holds encoder entry s */
    for (int s = 0; s < B; s++) buf[s] = s;
    ECHK(hipMemcpy(e->d.req_entry, buf, B * sizeof(int), hipMemcpyHostToDevice));
    /* the slots' copies of those fields, as admission would have made them */
    int *const sf[7] = {e->d.slot_np, e->d.slot_T, e->d.slot_flags, e->d.slot_lim, e->d.slot_ng, e->d.slot_tok,
                        e->d.slot_ent};
    for (int f = 0; f < 7; f++) {
        for (int s = 0; s < B; s++)
            buf[s] = f == 0 ? 0 : f == 1 ? T_enc[s] : f == 2 ? HIPB_SUPPRESS_EOS : f == 3 ? e->d.smax
                   : f == 4 ? 1 : f == 5 ? 100 + s : s;
        ECHK(hipMemcpy(sf[f], buf, B * sizeof(int), hipMemcpyHostToDevice));
    }
    int q[CT_Q_WORDS] = {B, B, 0, 0, 0, 0, 0, B};
    q[9] = B;
    q[10] = B;
    ECHK(hipMemcpy(e->d.q, q, sizeof q, hipMemcpyHostToDevice));
    const long self_el = (long)DEC_N * B * DEC_H * e->d.kv_rows * DEC_DK;
    const long cross_el = (long)DEC_N * e->d.max_req * DEC_H * e->d.tmax * DEC_DK;
    ctk_fill_random(e->kself, self_el, e->esz == 2, 0.1f, seed, e->s);
    ctk_fill_random(e->vself, self_el, e->esz == 2, 0.1f, seed + 1, e->s);
    ctk_fill_random(e->kcross, cross_el, e->esz == 2, 0.1f, seed + 2, e->s);
    ctk_fill_random(e->vcross, cross_el, e->esz == 2, 0.1f, seed + 3, e->s);
    ECHK(hipStreamSynchronize(e->s));
    e->n_enc = B;
    e->bench_mode = 1;
}

void hipb_bench_decode_gemms(HipbEngine *e) { step_kernels(e, 0, 0); }

void hipb_bench_read_floor(HipbEngine *e) {
    const long cap = 256L * ((e->d.rows + 15) / 16);     /* <= 256 workgroups per 16 rows */
    if (e->floor_cap < cap) {
        if (e->floor_sink) ECHK(hipFree(e->floor_sink));
        e->floor_sink = dmalloc((size_t)cap * sizeof(float));
        e->floor_cap = cap;
    }
    e->bench_floor = 1;
    step_kernels(e, 0, 0);
    e->bench_floor = 0;
}

void hipb_bench_encoder_gemm(HipbEngine *e, int M) {
    if (M < 1) CT_FATAL("hipb_bench_encoder_gemm: M < 1");
    const int sp = e->cfg.enc_ffn_bf16;
    if (M > e->enc_cap || e->bench_gemm_M != M) {
        enc_reserve(e, M, 8);
        /* seeded operand, split as the producers write it: hi ~ N(0,1),
         * lo ~ N(0,1) * 2^-9 */
        ctk_fill_random(e->eln_h, (long)M * ENC_D, 1, 1.0f, 71, e->s);
        if (!sp) ctk_fill_random(e->eln_l, (long)M * ENC_D, 1, 1.0f / 512.0f, 72, e->s);
        e->bench_gemm_M = M;
    }
    const ELayer *L = &e->W.enc[0];
    gemm_sp_silu_split(e, e->eln_h, sp ? NULL : e->eln_l, M, L->ff1_w1, L->ff1_b1, e->emid_h,
                       sp ? NULL : e->emid_l);
}

void hipb_mel(HipbEngine *e, const float *pcm, int n_samples, float *mel_out) {
    if (n_samples < HOP_LEN) CT_FATAL("hipb_mel: clip shorter than one hop (160 samples)");
    const int T = 1 + n_samples / HOP_LEN;
    float *dp = dmalloc((size_t)n_samples * 4), *dm = dmalloc((size_t)N_MELS * T * 4);
    CtMelClip *dc = dmalloc(sizeof(CtMelClip));
    int *fc = dmalloc((size_t)T * sizeof(int));
    const CtMelClip c = {dp, n_samples, 0, T, 0};
    ECHK(hipMemcpyAsync(dp, pcm, (size_t)n_samples * 4, hipMemcpyHostToDevice, e->s));
    ECHK(hipMemcpyAsync(dc, &c, sizeof c, hipMemcpyHostToDevice, e->s));
    ECHK(hipMemsetAsync(fc, 0, (size_t)T * sizeof(int), e->s));
    ctk_mel(dm, dc, 1, fc, T, &e->mel_tab, e->s);
    ECHK(hipMemcpyAsync(mel_out, dm, (size_t)N_MELS * T * 4, hipMemcpyDeviceToHost, e->s));
    ECHK(hipStreamSynchronize(e->s));
    ECHK(hipFree(dp)); ECHK(hipFree(dm)); ECHK(hipFree(dc)); ECHK(hipFree(fc));
}
