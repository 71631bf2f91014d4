/* ct_launch.h — C-callable launchers for the gfx950 kernels.
 *
 * Plain pointers, sizes and a hipStream_t: the C glue (abi.c) and the decode
 * engine call these; no C++ or device types cross this header.
 */
#ifndef CT_LAUNCH_H
#define CT_LAUNCH_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

/* Longest clip (encoder frames) backend_rel_pos_mhsa_noalloc serves: 30 s,
 * the longest file the reference batches unchunked (transcribe.c:894). */
#define CT_STATIC_MHSA_MAX_T 376
/* Scratch floats of backend_rel_pos_mhsa at T frames: Q, K, V (T rows each),
 * P (2T - 1 rows) and O (T rows) of ENC_D (1280) floats. */
#define CT_MHSA_SCRATCH_FLOATS(T) ((size_t)(6 * (T) - 1) * 1280)

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- GEMM: Y = epi(A W^T + b) ---------------- */
enum {
    CT_EPI_STORE = 0,   /* Y = s                                   */
    CT_EPI_SILU  = 1,   /* Y = s * sigmoid(s)                      */
    CT_EPI_RELU  = 2,   /* Y = max(s, 0)                           */
    CT_EPI_FMADD = 3,   /* Y += scale * s                          */
    CT_EPI_GLU   = 4    /* Y[:, j] = s_j * sigmoid(s_{j+glu_half}) */
};

/* Output segment of a GEMM: columns [i*seg_w, (i+1)*seg_w) go to seg[i]. */
enum { CT_OUT_DENSE = 0, CT_OUT_HEADS_F32 = 1, CT_OUT_HEADS_BF16 = 2, CT_OUT_SPLIT = 3 };
typedef struct {
    int         mode;
    void       *base;
    long        ld;           /* DENSE / SPLIT: row stride in elements           */
    void       *base_lo;      /* SPLIT: lo plane (base is the hi plane)          */
    const long *rowoff;       /* HEADS: per-row element offset (< 0: skip row);  */
    long        hstride;      /* column c -> base + rowoff[m] + (c/128)*hstride + c%128 */
} CtSeg;

typedef struct {
    const float    *A;        /* [M][lda] fp32 activations                 */
    long            lda;
    /* Pre-split activations: when Ahi != NULL, A = Ahi + Alo (bf16 [M][lda]
     * each, written by the producing kernel) and A is not read. */
    const uint16_t *Ahi, *Alo;
    const uint16_t *W;        /* [N][K] bf16 weights, row-major            */
    const uint16_t *bias;     /* [N] bf16 or NULL                          */
    float          *Y;        /* output rows of ldy floats                 */
    long            ldy;
    int M, N, K;
    int epi;
    float scale;              /* CT_EPI_FMADD                              */
    /* Row scatter (KV-cache append): when row_len != NULL, result row m is
     * written to Y row m*row_stride + row_len[m*row_len_step] - 1.          */
    const int      *row_len;
    int             row_len_step;
    long            row_stride;
    int             glu_half; /* CT_EPI_GLU: N == 2*glu_half               */
    const int      *row_mask; /* rows m with row_mask[m] == 0 are not written */
    int             nseg;     /* > 0: segmented output (epi must be STORE)  */
    int             seg_w;
    CtSeg           seg[3];
} CtGemm;

void ctk_gemm(const CtGemm *g, hipStream_t s);
/* Tests: 128 or 256 forces the pre-split kernels' tile (0: the tile-count
 * model); sizeof(CtGemm) for the tests' struct mirror. */
void ctk_gemm_force_tile(int rows);
int  ctk_gemm_sizeof(void);

/* ---------------- decode GEMM on fragment-ordered activations ----------------
 * "Frag" layout of an activation matrix X[M][K] (K % 32 == 0), as the decode
 * GEMM's MFMA lanes consume it: rows in blocks of 64, each block in K-steps of
 * 32, each K-step in four 16-row groups; one group is 1024 uint16 = the hi
 * plane (64 lanes x 8 bf16) then the lo plane.  Lane l of a group holds row
 * 16*g + (l & 15), columns 8*(l >> 4) .. +7 of the K-step.  X = hi + lo.
 * Element (m, k) of plane p sits at ct_frag_off(m, k, K) + 512*p. */
#ifdef __HIPCC__
#define CT_HD __host__ __device__
#else
#define CT_HD
#endif
static inline CT_HD long ct_frag_off(int m, int k, int K) {
    return ((((long)(m >> 6) * (K >> 5) + (k >> 5)) * 4 + ((m >> 4) & 3)) << 10) +
           ((long)((((k >> 3) & 3) << 4) + (m & 15)) << 3) + (k & 7);
}
/* uint16 elements of a frag buffer for M rows (rows padded to 64). */
static inline long ct_frag_elems(int M, int K) { return (long)((M + 63) / 64) * 64 * K * 2; }

enum {
    CT_GV_PARTIAL = 0,  /* Y[(ks*M + m)*N + n] = partial sum over K-slice ks (no bias)  */
    CT_GV_DENSE   = 1,  /* Y[m*ldy + n] = act(s + b)                                    */
    CT_GV_FRAG    = 2,  /* F (frag layout, K' = N) = act(s + b), split hi/lo           */
    CT_GV_QKV     = 3,  /* n < 1024: Y[m*ldy + n] (query); n in [1024, 3072): key/value */
                        /* rows of the head-major caches kc/vc at rowoff[m] (< 0: skip) */
    CT_GV_RESID   = 4   /* residual update Y[m*ldy + n] += s + b (N = DEC_D, no K split), */
                        /* and each row's LayerNorm statistics per 32-column block b:     */
                        /* lnstat[m*32 + b] = (mean, sum of squared deviations)          */
};
#define CT_LN_BLOCKS 32 /* 32-column blocks of a DEC_D row in lnstat                    */
typedef struct {
    const uint16_t *A;        /* frag-ordered activations [M][K]                      */
    const uint16_t *W;        /* [N][K] bf16, or tiled (wtile)                         */
    const uint16_t *bias;     /* [N] bf16 or NULL (ignored for CT_GV_PARTIAL)          */
    int M, N, K;
    int ksplit;               /* K-slices (workgroups along K); 1 unless PARTIAL       */
    int out, relu;
    float *Y;  long ldy;
    uint16_t *F;
    void *kc, *vc;            /* CT_GV_QKV caches, element offset rowoff[m] + (c/128)*hstride + c%128 */
    const long *rowoff;
    long hstride;
    int kv_bf16;
    int wtile;                /* 1: W in the tile layout of ctk_tile_w                 */
    const int *m_active;      /* device int or NULL: rows at or past *m_active are
                                 unused this launch (workgroups of only such rows
                                 exit, their row blocks are not computed)           */
    float *lnstat;            /* CT_GV_RESID output; with fold_c1 the row statistics */
    const uint16_t *fold_w;   /* CT_GV_RESID with F: F = frag(h_new * fold_w), the A
                                 of a GEMM on LayerNorm(h_new) with gain fold_w     */
    const float *fold_c1, *fold_c2;
                              /* NULL, or the GEMM's A is frag(h * w) of rows h whose
                                 statistics a CT_GV_RESID launch left in lnstat, and
                                 each output is rstd (s - mu c1[n]) + c2[n]: the GEMM
                                 of LayerNorm(h) (gain w, bias b) plus bias, with
                                 c1 = W w and c2 = W b + bias (ctk_fold_cols); bias
                                 is then ignored                                    */
} CtGemv;
/* Requires N % 16 == 0 (N % 64 == 0 when N >= 8192), K % (256 * steps) == 0. */
void ctk_gemv(const CtGemv *g, hipStream_t s);
/* Column constants of a GEMM on a folded LayerNorm (CtGemv.fold_c1/c2) for a
 * row-major W[N][K], LayerNorm gain w and bias b (bf16, K entries) and the
 * GEMM's bias (bf16, N entries, or NULL): c1[n] = sum_k w_k W_nk and c2[n] =
 * sum_k b_k W_nk + bias_n, each summed in double over k in order and rounded
 * to fp32 once. */
void ctk_fold_cols(const uint16_t *W, const uint16_t *w, const uint16_t *b, const uint16_t *bias,
                   int N, int K, float *c1, float *c2, hipStream_t s);
/* The GEMM's weight reads alone (tiled weights, same grid as ctk_gemv for
 * g): one value per workgroup to sink (ctk_gemv_read_floor_blocks(g)
 * floats).  A floor for the GEMM's duration, for benchmarking. */
void ctk_gemv_read_floor(const CtGemv *g, float *sink, hipStream_t s);
long ctk_gemv_read_floor_blocks(const CtGemv *g);
/* The weight tiles one decode-GEMM launch reads, by workgroup: workgroup i
 * of its first row group (of gx * gy, i = K-slice + gy * column position,
 * column block x = i / gy, or ct_qkv_col(i / gy, cb) for a QKV launch) reads,
 * for each of its cb column blocks c, the per consecutive 1-KB tiles from
 * tile (x * cb + c) * nsteps + (i % gy) * per of W (tile layout).  Workgroup
 * i runs on XCD i % 8, like every launch's workgroup i; the other row groups'
 * workgroups i + gx * gy * z read the same tiles on the same XCD (gx * gy is
 * a multiple of 8 for every decoder shape). */
typedef struct {
    const uint16_t *W;
    int gx, gy, cb, per, nsteps;
    int heads;                /* 1: a QKV launch, column positions dealt by head */
} CtWarm;
/* Column block of a QKV launch's workgroup at position p (blocks of 16*cb
 * columns, cb in {1, 2, 4}): positions p % 8 == h take head h's 8/cb query,
 * 8/cb key and 8/cb value blocks, so they run on XCD h, where the attention's
 * workgroups of head h read them. */
static inline CT_HD int ct_qkv_col(int p, int cb) {
    const int j = p >> 3, bph = 8 / cb;
    return (j / bph) * (64 / cb) + (p & 7) * bph + j % bph;
}
/* Fills w for the launch ctk_gemv(g) makes; w->gx = 0 when g's weights are
 * not in the tile layout. */
void ctk_gemv_warm(const CtGemv *g, CtWarm *w);
/* sizeof(CtWarmSet), for callers that mirror the struct (ctypes). */
int ctk_warmset_sizeof(void);
/* Read-ahead a launch carries for the next n decode GEMMs: 8 * rows more
 * workgroups, rows of them on each XCD, read the weight tiles each GEMM
 * workgroup will read into the L2 of that workgroup's XCD.  sink (>= 1 KB) is
 * written only if the tiles' XOR equals magic (so the reads stay). */
typedef struct {
    CtWarm t[4];
    int n, rows;
    unsigned magic;
    unsigned *sink;
} CtWarmSet;
/* sizeof(CtGemv), for callers that mirror the struct (ctypes). */
int ctk_gemv_sizeof(void);
/* Tile layout of a decode-GEMM weight W[N][K] (N % 16 == 0, K % 32 == 0):
 * one 1024-entry tile per (16 output rows, K-step of 32), tiles ordered
 * row block major; lane l of a tile holds W[16*rb + (l & 15)][32*st +
 * 8*(l >> 4) .. +7], so a wavefront's weight load is one contiguous 1 KB. */
static inline CT_HD long ct_wtile_off(int n, int k, int K) {
    return ((((long)(n >> 4) * (K >> 5) + (k >> 5)) * 64 + (((k >> 3) & 3) << 4) + (n & 15)) << 3) + (k & 7);
}
void ctk_tile_w(const uint16_t *W, uint16_t *Wt, int N, int K, hipStream_t s);
/* K-slices the decode GEMM uses for an N x K weight (a function of the shape
 * only, so every row's result is independent of M). */
int  ctk_gemv_ksplit(int N, int K);

/* Residual update after a K-split projection (rows r < M): h[r] += ((parts[0][r]
 * + parts[1][r]) + ...) + pbias, the nparts = 8 slices M * DEC_D floats
 * apart; then, with b NULL, the folded input of the next GEMM's LayerNorm
 * with gain w (CtGemv.fold_c1): each 32-column block's (mean, squared
 * deviations) of h[r] into lnstat[r*32 + b] and frag(h[r] * w); with b,
 * frag(LayerNorm(h[r])) with gain w and bias b.  Carries the read-ahead warm
 * (NULL: none). */
void ctk_resid_fold(float *h, float *lnstat, uint16_t *frag, const float *parts, int nparts,
                    const uint16_t *pbias, const uint16_t *w, const uint16_t *b, int M,
                    const CtWarmSet *warm, hipStream_t s);
/* The decode step's embedding: for active rows r < M, h[r] = LN_e(etw[tokens[r]]
 * + epw[pos_len[r] - 1]) (as ctk_embed_ln); then for every row the folded
 * input of the first layer's LayerNorm with gain w (CtGemv.fold_c1): each
 * 32-column block's (mean, squared deviations) of h[r] into lnstat[r*32 + b]
 * and frag(h[r] * w), carrying the read-ahead warm (NULL: none). */
void ctk_embed_fold(float *h, float *lnstat, uint16_t *frag, const int *tokens, const int *pos_len,
                    const int *active, const uint16_t *etw, const uint16_t *epw,
                    const uint16_t *elnw, const uint16_t *elnb, const uint16_t *w, int M,
                    const CtWarmSet *warm, hipStream_t s);

/* fp32 -> (hi, lo) bf16 pair, the split every GEMM applies to activations. */
void ctk_split(uint16_t *hi, uint16_t *lo, const float *x, long n, hipStream_t s);

/* ---------------- row-wise ops ---------------- */
/* LayerNorm writing the normalised rows pre-split (hi, lo bf16). */
void ctk_layernorm_split(uint16_t *hi, uint16_t *lo, const float *src, const uint16_t *w,
                         const uint16_t *b, int T, int D, hipStream_t s);
void ctk_layernorm(float *dst, const float *src, const uint16_t *w, const uint16_t *b,
                   int T, int D, hipStream_t s);
/* x = LayerNorm(x; w1, b1) in place, then LayerNorm(x; w2, b2) pre-split
 * (hi, lo bf16; lo may be NULL): the bits of ctk_layernorm followed by
 * ctk_layernorm_split, in one pass over x. */
void ctk_layernorm_pair_split(float *x, uint16_t *hi, uint16_t *lo, const uint16_t *w1,
                              const uint16_t *b1, const uint16_t *w2, const uint16_t *b2, int T,
                              int D, hipStream_t s);
void ctk_add(float *dst, const float *src, long n, hipStream_t s);
/* dst row dst_row[m] = src row m, M rows of D floats. */
void ctk_copy_rows(float *dst, const float *src, const int *dst_row, int M, int D, hipStream_t s);
void ctk_causal_mask(float *mask, int S, hipStream_t s);
/* pe rows p = 0..2T-2 hold relative position T-1-p; inv_freq[k] (ENC_D/2
 * entries) is exp(-2k ln(1e4)/ENC_D), computed on the host. */
void ctk_rel_pos_emb(float *pe, int T, const float *inv_freq, hipStream_t s);
/* h[r] = LN(etw[tok] + epw[pos]) for r in [0, R): tok = tokens[r]; pos =
 * pos_len ? pos_len[r] - 1 : pos_start + r; rows with active[r] == 0 are
 * skipped when active != NULL. */
void ctk_embed_ln(float *h, const int *tokens, int R, int pos_start, const int *pos_len,
                  const int *active, const uint16_t *etw, const uint16_t *epw,
                  const uint16_t *lnw, const uint16_t *lnb, hipStream_t s);
/* out[r] = first index of the maximum of logits[r][0..n) (rows with
 * active[r] == 0 untouched). */
void ctk_argmax(int *out, const float *logits, int R, int n, const int *active, hipStream_t s);
void ctk_inc(int *p, hipStream_t s);

/* ---------------- attention ---------------- */
typedef struct {
    float       *out;         /* out[b][qi][h*dk + d]                                  */
    const float *Q;
    long q_sb, q_st;          /* Q/out strides (floats) per item and per query row     */
    const void  *K, *V;       /* fp32 or bf16 (kv_bf16)                                */
    int   kv_bf16;
    long  kv_sb, kv_st, kv_sh;/* K/V element strides per item, per key row, per head   */
    const int *lens;          /* keys per item: lens[b*lens_step] (device) ...         */
    int   lens_step;
    int   len_const;          /* ... or this when lens == NULL                          */
    const int   *kv_index;    /* optional: item b reads K/V block kv_index[b]          */
    int   kv_direct;          /* with kv_index: items b < kv_direct read block b itself
                                 (no index load before their first keys)             */
    const int   *rank;        /* optional (T_q == 1): items by descending length; launch
                                 position p takes item rank[snake(p)], so the items that
                                 share a CU pair long with short                      */
    int   kv_rows;            /* key rows allocated per item (0: unknown); with at least
                                 one key trip's rows (32) of bf16 the first keys are
                                 read before the length                                */
    const float *mask;        /* optional additive [T_q][T_k] mask (B == 1)            */
    int   T_q, B, H;
    float scale;
    /* optional: write the output split hi/lo in frag layout (K = H*128),
     * row b*T_q + qi, instead of out */
    uint16_t       *out_frag;
    /* optional read-ahead of the next decode GEMMs' weights (warm.n > 0,
     * H % 8 == 0): warm.rows more rows of H workgroups */
    CtWarmSet       warm;
} CtAttn;
/* Head dim fixed at DEC_DK (128). */
void ctk_attn(const CtAttn *a, hipStream_t s);

/* ---------------- encoder ---------------- */
/* Relative-position MHSA core for one clip: O = softmax(((Q+u)K^T +
 * rel_shift((Q+v)P^T)) * scale) V, per head; P has 2T-1 rows. */
void ctk_relpos_attn(float *O, const float *Q, const float *K, const float *V,
                     const float *P, const uint16_t *pbu, const uint16_t *pbv,
                     int T, hipStream_t s);
/* Packed clips: sequence i has T = seq_T[i] rows starting at row seq_off[i]
 * of Q/K/V/O; its P rows are the window of a table built for T_max, shifted
 * by T_max - T (model.h:586-592).  Work items (clip, 16-query block) are
 * listed in blk_seq/blk_q0 (n_blk entries, built by ctk_relpos_plan).  The
 * output goes to O (fp32) or, with O NULL, split hi/lo into the planes Oh, Ol. */
int  ctk_relpos_plan(int *blk_seq, int *blk_q0, const int *seq_T, int n_seq);
void ctk_relpos_attn_packed(float *O, uint16_t *Oh, uint16_t *Ol, const float *Q,
                            const float *K, const float *V, const float *P, int T_max,
                            const uint16_t *pbu, const uint16_t *pbv, const int *seq_off,
                            const int *seq_T, const int *blk_seq, const int *blk_q0, int n_blk,
                            int max_T, hipStream_t s);
/* Depthwise conv k=9 (zero pad 4 inside the sequence) + BN + SiLU.  With
 * row_start/row_len (per row: first row and length of its sequence) the rows
 * are packed sequences; otherwise one sequence of T rows. */
void ctk_dwconv_bn_silu(float *out, const float *in, int T,
                        const uint16_t *dww, const uint16_t *dwb,
                        const uint16_t *bnw, const uint16_t *bnb,
                        const uint16_t *bnm, const uint16_t *bnv, hipStream_t s);
/* Packed form; writes its output pre-split (hi, lo bf16) for the next GEMM. */
void ctk_dwconv_bn_silu_packed(uint16_t *out_hi, uint16_t *out_lo, const float *in, int M,
                               const int *row_start, const int *row_len,
                               const uint16_t *dww, const uint16_t *dwb,
                               const uint16_t *bnw, const uint16_t *bnb,
                               const uint16_t *bnm, const uint16_t *bnv, hipStream_t s);
/* Subsampling stages (position-major [t][f][ch] activations). */
void ctk_sub_conv0(float *out, const float *mel, int T_mel, int stride,
                   const uint16_t *w, const uint16_t *b, hipStream_t s);
void ctk_sub_dwconv(float *out, const float *in, int H, int Wd,
                    const uint16_t *w, const uint16_t *b, hipStream_t s);
/* [T][16][256] -> [T][256*16] (channel-major flatten per frame). */
void ctk_sub_flatten(float *out, const float *in, int T, hipStream_t s);
/* The subsampling convolutions over n requests packed along time: request r
 * owns rows off[r] .. off[r + 1] (off: n + 1 ascending device ints from 0) of
 * each stage; rows2 / rows_out = off[n] of the output stage.  Outputs are
 * written split hi/lo (bf16 planes) for the pointwise GEMM after each.
 * conv0_dw runs the 3x3 stride-2 conv (1 -> 256, ReLU) and the first
 * depthwise stage in one pass ([.][32][256] rows); it reads request r's mel
 * (N_MELS x tmel[r], row stride tmel[r]) at mel + moff[r].  dw_split is a
 * depthwise stage over [.][Wd][256] input rows. */
void ctk_sub_conv0_dw_packed(uint16_t *out_hi, uint16_t *out_lo, const float *mel, const int *o1,
                             const int *o2, const int *tmel, const int *moff, int n, int rows2,
                             const uint16_t *w0, const uint16_t *b0, const uint16_t *wd,
                             const uint16_t *bd, hipStream_t s);
void ctk_sub_dw_split_packed(uint16_t *out_hi, uint16_t *out_lo, const float *in, const int *oin,
                             const int *oout, int n, int rows_out, int Wd, const uint16_t *w,
                             const uint16_t *b, hipStream_t s);
/* The same, written as hi/lo bf16 planes (row stride 4096). */
void ctk_sub_flatten_split(uint16_t *hi, uint16_t *lo, const float *in, int T, hipStream_t s);

/* ---------------- log-mel front-end ---------------- */
typedef struct {
    const float *pcm; /* the clip's samples (device memory)               */
    int  n;        /* samples                                             */
    long mel0;     /* first float of the clip's [N_MELS][T] mel block     */
    int  T;        /* frames = 1 + n / HOP_LEN                            */
    int  frame0;   /* global index of the clip's frame 0                  */
} CtMelClip;

typedef struct {
    const float *hann;          /* [WIN_LEN]                          */
    const float *twr, *twi;     /* [N_FFT/2] exp(-2 pi i k / N_FFT)   */
    const float *fb;            /* [N_MELS][N_BINS] Slaney filterbank */
    const int *fb_lo, *fb_hi;   /* non-zero bin range per filter      */
} CtMelTables;

/* mel for n_clips packed clips; frame_clip[f] names the clip of global
 * frame f (n_frames = sum of T). */
void ctk_mel(float *mel, const CtMelClip *clips, int n_clips,
             const int *frame_clip, int n_frames, const CtMelTables *tab, hipStream_t s);

/* Device scratch of backend_rel_pos_mhsa_noalloc: looked up once per device
 * (with that device current), then its address for that device. */
void ct_static_init(int dev);
float *ct_static_scratch(int dev);
size_t ct_static_scratch_floats(void);

#ifdef __cplusplus
}
#endif
#endif
