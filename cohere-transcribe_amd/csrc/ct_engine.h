/* ct_engine.h — device-resident decode state of the engine (C and HIP). */
#ifndef CT_ENGINE_H
#define CT_ENGINE_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Prompt ids a request may hold: a submitted prompt (at most
 * CT_PROMPT_SUBMIT_MAX) plus the tokens a chained chunk carries over from
 * its predecessor (at most CT_CARRY_MAX, transcribe.c:476). */
#define CT_PROMPT_SUBMIT_MAX 16
#define CT_CARRY_MAX 64
#define CT_PROMPT_MAX (CT_PROMPT_SUBMIT_MAX + CT_CARRY_MAX)
#define CT_ENG_MAX_SLOTS 256  /* slots an engine may have (the ABI's MAX_BATCH) */
/* Default of HIPB_RANK_MIN_ROWS: steps of at least this many rows deal their
 * attention items to CUs by length rank (long with short): with >= 3 items per CU position the balance
 * outweighs the extra dependent load per workgroup; at 64 slots + 16 prompt
 * rows it measured even (the 128-slot step: 27.8 -> 24.0 us per launch). */
#ifndef CT_RANK_MIN_ROWS
#define CT_RANK_MIN_ROWS 96
#endif
/* Spare rows per (slot, head) of the self caches: without them every
 * (slot, head) block starts on the same 256-KB boundary and the workgroups
 * of a step stream from the same memory channels at the same time (16 rows:
 * stream RTFx +0.1% over none, 8 rows +0.05%). */
#ifndef CT_KV_PAD
#define CT_KV_PAD 16
#endif

/* All pointers are device memory.  Slot-major arrays have `slots` entries.
 * Request-major arrays are rings of ring_mask + 1 entries: request id r
 * lives at r & ring_mask while it is outstanding (submitted, results not
 * yet collected).  Encoder state (cross K/V, encoder output) is held in
 * max_req entries, taken when a request is encoded and recycled after it
 * retires. */
typedef struct {
    int slots, max_req, smax, tmax;
    int ring_mask;     /* request ring size - 1 (a power of two minus one)    */
    int rank_min;      /* steps of at least this many rows rank their rows    */
    int rows;          /* step rows: slots + spare prompt rows                  */
    int kv_rows;       /* rows per (slot, head) of the self caches (>= smax)    */
    /* slot table */
    int  *slot_req;    /* request in the slot, -1 when free                    */
    int  *slot_S;      /* tokens already in the slot's self cache              */
    /* the slot's request fields, copied at admission so the step kernels
     * read them beside the slot table: prompt ids, encoder frames, flags,
     * token limit, tokens generated, and the last token generated */
    int  *slot_np, *slot_T, *slot_flags, *slot_lim, *slot_ng, *slot_tok;
    int  *slot_ent;    /* encoder entry of the slot's request                 */
    /* step rows [rows]: row s < slots is slot s's row, rows past `slots`
     * carry extra prompt tokens of a slot (row_slot) */
    int  *act;         /* 1 if the row decodes this step                       */
    int  *tok;         /* token embedded in the row                            */
    int  *pos_len;     /* self length the row attends to (position + 1)        */
    int  *cross_len;   /* encoder frames of the row's request (0 when idle)    */
    int  *cross_idx;   /* encoder entry whose cross K/V the row reads          */
    int  *row_slot;    /* slot whose self cache the row writes and reads       */
    /* rows of this step by descending self / cross length (ties by row):
     * the attention launches deal them to CUs so long and short rows pair */
    int  *rank_self, *rank_cross;
    long *kv_rowoff;   /* element offset of the row's self K/V entry, -1 idle  */
    /* requests (rings) */
    int  *req_T, *req_limit, *req_flags, *req_np, *req_ngen;
    int  *req_entry;   /* encoder entry, written when the request is published */
    int  *req_prompt;  /* [ring][CT_PROMPT_MAX]                                */
    int  *req_out;     /* [ring][smax] generated tokens                        */
    float *req_score;  /* [ring][smax] the largest logit the argmax weighed
                          for each token (EOS left out when suppressed): the
                          step's logits bits, for batch-vs-single checks      */
    /* chained chunks of one long recording: the request admitted after
     * this one finishes (its prompt then gets the carried tokens), or -1 */
    int  *req_next;
    /* successor ring: chained chunks released by their predecessors;
     * rq[q[0]..q[1]) wait for a slot and for their encoding (q[7]), in ring
     * order.  pend[slot] is a successor that eng_end released in that slot
     * this step (-1 if none); eng_begin appends them in slot order.  Only the
     * step kernels write rq and pend. */
    int  *rq, *pend;
    /* retired request ids in retirement order: ret[k & ring_mask] is the
     * k-th request to finish (q[2] counts them) */
    int  *ret;
    /* fresh queue: requests that wait for no predecessor, in submission
     * order, published by the host once encoded (the ids, then the count
     * q[5]); fq[q[4]..q[5]) wait for a slot.  Read with device-coherent
     * loads: the host may publish while steps run on another stream. */
    int  *fq;
    /* q[0] next successor to admit, q[1] successors written, q[2] requests
     * finished, q[3] prompt tokens not yet fed after the last step, q[4] next
     * fresh request to admit, q[5] fresh requests published, q[6] rows the
     * current step uses (the slots' rows plus the spare rows dealt out),
     * q[7] publications of encoded batches so far (each writes its
     * requests' encoder entries first: a released successor is admitted
     * only once its entry is there), q[8] 1 when the successor at the head
     * of rq waits for its encoding after the last admission, q[9] the
     * publication count that admission saw, q[10] successors
     * released so far (by eng_end; q[10] - q[0] wait in pend or rq) */
    int  *q;
} CtEngDev;

#define CT_Q_WORDS 16      /* ints in q */

/* Admission + the step's rows (one workgroup; admission and spare-row
 * dealing go in slot order, so scheduling is deterministic).  extra: spare
 * prompt rows this step may use (0 .. rows - slots). */
void ctk_eng_begin(const CtEngDev *d, int extra, hipStream_t s);
/* Argmax with the request's policy, token append, retirement. */
void ctk_eng_end(const CtEngDev *d, const float *logits, hipStream_t s);
/* dst[pairs[2i] & mask] = pairs[2i + 1], i < n (request-ring writes). */
void ctk_ring_scatter(int *dst, const int *pairs, int n, int mask, hipStream_t s);
/* Seeded fill of n elements (N(0,1)*scale approx.), bf16 or fp32. */
void ctk_fill_random(void *p, long n, int bf16, float scale, uint64_t seed, hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif
