/* hipb.h — the MI355X decode engine behind the drop-in backend.
 *
 * The reference has no counterpart for these entry points: they extend the
 * 40-function ABI (backend.h) with what the batched ragged decode needs and
 * the ABI cannot express (backends/backend.h:181-228 covers one step with
 * host-side active[]/S[] arrays, transcribe.c:733-795 drives it):
 *
 *  - a device-resident slot table: each of `slots` KV slots holds one request;
 *    a finished request's slot is refilled from the request queue by a device
 *    kernel at the start of the next step (continuous batching, no host
 *    round trip);
 *  - KV caches in HBM as [layer][slot][head][position][128] (self) and
 *    [layer][request][head][frame][128] (cross), bf16 or fp32;
 *  - the prompt is fed through the same step kernels (one token per step,
 *    or several per step in spare prompt rows), so a request's numbers
 *    never depend on its slot, its step rows or the other requests;
 *  - the forced-length policy of the benchmark configurations on device:
 *    EOS excluded from the argmax and/or EOS forced at token `limit`;
 *  - the encoder on packed ragged batches (M = sum of frames).
 *
 * Threading: an engine belongs to the thread that created it, which must have
 * called backend_init(dev) after backend_weights_upload_blob().  Errors print
 * and exit(1) like the ABI.
 */
#ifndef CT_HIPB_H
#define CT_HIPB_H

#include "model_types.h"
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct HipbEngine HipbEngine;

typedef struct {
    int slots;          /* concurrent KV slots (decode batch), 1..256          */
    int max_requests;   /* encoder-state entries: requests holding cross K/V and
                           an encoder output at once (each ~14 MB at 376 frames,
                           bf16 KV); an entry is taken when a request is
                           encoded and recycled after it finishes, so any
                           number of requests flows through.  Up to
                           max(4 x max_requests, 32 x slots, 1024) may be
                           outstanding (submitted, not finished).  The host
                           keeps each request's record and results (8 bytes
                           a token) until hipb_reset, which a long-running
                           serving loop calls between batches of requests */
    int max_frames;     /* largest encoder length a request may have (<= 2048) */
    int kv_bf16;        /* 1: bf16 KV caches, 0: fp32                           */
    int max_tokens;     /* longest prompt + limit of any request (sizes the self
                           caches), <= MAX_SEQ; 0 means MAX_SEQ                 */
    int prefill_rows;   /* spare step rows for prompts (0..256): while prompt
                           tokens wait, hipb_run launches a step of slots +
                           prefill_rows rows that feeds several prompt tokens
                           of a slot at once (same bits as one per step)       */
    int admit_order;    /* 0: requests are encoded and admitted in submission
                           order; 1: largest token budget (limit) first, a
                           recording's chunks together in order under the
                           first chunk's budget (shortens a pass: fewer slots
                           idle at its end); results are the same bits      */
    int enc_ffn_bf16;   /* 1: the encoder's FFN projections (70% of its flops)
                           take their activations as bf16 (one MFMA pass)
                           instead of the hi + lo pair (two passes): encoder
                           output within ~4e-3 of the fp32 path instead of
                           ~1e-5; logits within ~6e-4 on the specified weights
                           (bf16 KV alone: ~4e-4); 0: both passes          */
} HipbConfig;

/* Request policy flags. */
#define HIPB_SUPPRESS_EOS 1   /* EOS never chosen by the argmax              */
#define HIPB_FORCE_EOS    2   /* token number `limit` is EOS                  */

/* Creates an engine on the calling thread's device for the weights W (host
 * pointers into the uploaded blob, as every ABI call takes them). */
HipbEngine *hipb_create(const HipbConfig *cfg, const Weights *W);
void hipb_destroy(HipbEngine *e);

/* Queues a request: mel (N_MELS x T_mel, row stride T_mel, host memory),
 * prompt ids, at most `limit` generated tokens.  Returns the request id
 * (0, 1, 2, ... in submission order, until hipb_reset).  Fatal if more
 * requests are outstanding than the request ring holds (see
 * max_requests). */
int  hipb_submit(HipbEngine *e, const float *mel, int T_mel, const int *prompt, int n_prompt,
                 int limit, int flags);
/* Queues a request given 16 kHz mono PCM (host memory); its log-mel
 * spectrogram is computed on the GPU at encode time (transcribe.c:177-214). */
int  hipb_submit_pcm(HipbEngine *e, const float *pcm, int n_samples, const int *prompt,
                     int n_prompt, int limit, int flags);
/* Long recordings (transcribe.c:397-535): splits 16 kHz PCM (host memory)
 * at silences and queues one request per chunk, ids consecutive from
 * *first_req.  Chunk c + 1 is admitted only after chunk c has finished; its
 * prompt is then this prompt with chunk c's last <= 64 generated ids (the
 * final one excluded) inserted after the first two ids.  silence_db NAN picks
 * the threshold from the recording's noise floor; the reference's defaults
 * are silence_dur 0.2 s and target_sec 20 s.  Requires n_prompt >= 2 and
 * n_prompt + 64 + limit <= max_tokens; every chunk must fit max_frames.
 * Returns the number of chunks. */
int  hipb_submit_pcm_chunked(HipbEngine *e, const float *pcm, int n_samples, const int *prompt,
                             int n_prompt, int limit, int flags, float silence_db,
                             float silence_dur, float target_sec, int *first_req);
/* The chunk boundaries alone: chunk i is samples [bounds[2i], bounds[2i+1]).
 * Returns the number of chunks (at most cap), -1 if out of memory. */
int  hipb_chunk_bounds(const float *pcm, int n_samples, float silence_db, float silence_dur,
                       float target_sec, int *bounds, int cap);
/* The same with the samples already in device memory (not copied; they must
 * stay valid until the hipb_encode or hipb_process call that encodes them
 * returns). */
int  hipb_submit_pcm_device(HipbEngine *e, const float *dev_pcm, int n_samples, const int *prompt,
                            int n_prompt, int limit, int flags);
/* Log-mel of one clip on the GPU, synchronously (N_MELS x (1 + n/160)). */
void hipb_mel(HipbEngine *e, const float *pcm, int n_samples, float *mel_out);
/* Drops every request and frees all slots (caches and weights stay). */
void hipb_reset(HipbEngine *e);
/* Runs the encoder and cross-attention K/V for the submitted requests not yet
 * encoded, in packed batches of at most max_batch_frames encoder frames, as
 * far as free encoder entries go (hipb_run encodes the rest as entries are
 * recycled). */
void hipb_encode(HipbEngine *e, int max_batch_frames);
/* One decode step over all slots (admission, embed, 8 layers, LM head,
 * argmax/policy).  Returns nothing; state stays on the device. */
void hipb_step(HipbEngine *e);
/* Runs decode steps until every submitted request has finished, encoding
 * the requests still waiting for an encoder entry as finished requests
 * return theirs; steps are replayed from one captured graph (launched one by
 * one instead when the environment sets HIPB_EAGER=1, e.g. under a tracing
 * profiler), chunk steps per host check (at most ring / (4 x slots)).  Two scheduling knobs, read at hipb_create, change where
 * work runs but not the results (same bits): HIPB_RANK_MIN_ROWS (steps of at
 * least this many rows deal attention items to compute units by length rank;
 * default 96) and HIPB_READ_AHEAD=0 (no weight read-ahead workgroups).
 * Returns the number of steps run. */
long hipb_run(HipbEngine *e, int chunk);
/* hipb_encode and hipb_run overlapped: a worker thread encodes the requests
 * not yet encoded on a second stream, in packed batches of at most
 * max_batch_frames encoder frames, each published to the slot table as soon
 * as its cross-attention K/V are written, while the calling thread runs
 * decode steps (chunk per host check) until every submitted request has
 * finished.  A chained chunk released by its predecessor is admitted only
 * once its own batch has been published (requests are encoded in submission
 * order; the published watermark gates it), so the tokens are those of
 * hipb_encode then hipb_run.  Device PCM passed to hipb_submit_pcm_device
 * must stay valid until hipb_process returns.  Returns the number of
 * steps. */
long hipb_process(HipbEngine *e, int max_batch_frames, int chunk);
/* Test support for hipb_process: after publishing `after_batches` encoder
 * batches the encoder thread waits (host-side, at most 60 s) until the decode
 * loop has seen `until_finished` requests finish, so a test can make a
 * chained chunk's predecessor retire before the chunk is encoded.  0
 * batches: no hold.  hipb_test_hold_expired reports whether the last hold
 * ran out of time. */
void hipb_test_hold_encoder(HipbEngine *e, int after_batches, int until_finished);
int  hipb_test_hold_expired(HipbEngine *e);
/* Number of requests finished so far (device counter, synchronises; also
 * returns the finished requests' encoder entries for reuse). */
int  hipb_finished(HipbEngine *e);

/* Results and inspection (synchronise the engine's stream). */
int  hipb_tokens(HipbEngine *e, int req, int *out, int cap);        /* returns count */
/* Per generated token, the largest logit the argmax weighed at that step (EOS
 * left out when suppressed; also for a forced EOS): a request's logits bits
 * in compact form, for batch-vs-single checks.  Returns the count. */
int  hipb_token_scores(HipbEngine *e, int req, float *out, int cap);
int  hipb_slot_of(HipbEngine *e, int req);                          /* -1 if none    */
void hipb_logits(HipbEngine *e, int slot, float *out);              /* VOCAB floats  */
/* Encoder output of a request while it still holds its encoder entry
 * (fatal once the entry went to a later request). */
void hipb_enc_out(HipbEngine *e, int req, float *out);              /* T_enc x DEC_D */
int  hipb_req_frames(HipbEngine *e, int req);

/* Microbenchmark support: fills the self and cross caches of every slot with
 * seeded values (N(0,1)*0.1, bf16/fp32 as configured) at lengths S[slot] and
 * T_enc[slot] and marks the slots active without a request queue, so
 * hipb_step runs decode steps at exactly those lengths. */
void hipb_bench_fill(HipbEngine *e, const int *S, const int *T_enc, uint64_t seed);
/* Launches only the 16 decode-attention kernels of one step (8 layers x self
 * and cross) on the engine stream, for per-kernel timing. */
void hipb_attention_only(HipbEngine *e);
/* Launches only the decode GEMMs of one step (8 layers x QKV, out, cross Q,
 * cross out, FFN up, FFN down, then the LM head) over the current step
 * buffers on the engine stream, for per-kernel timing. */
void hipb_bench_decode_gemms(HipbEngine *e);
/* The same launches with each GEMM replaced by its weight reads alone (same
 * grid, same 1 KB tiles per workgroup, no activations, no MFMAs): the floor
 * the decode GEMMs are measured against. */
void hipb_bench_read_floor(HipbEngine *e);
/* Launches the packed encoder's FFN up-projection (layer 0 weights: M frames
 * x 1280 -> 5120, SiLU, pre-split input and output; the encoder runs this
 * GEMM twice per layer) once on the engine stream, in the engine's FFN
 * precision mode (enc_ffn_bf16: bf16 input and output, no lo halves).  The
 * input is seeded when M changes. */
void hipb_bench_encoder_gemm(HipbEngine *e, int M);

/* Launches n decode steps (graph replays, or eager steps under HIPB_EAGER=1)
 * on the engine's stream without waiting and without checking for finished
 * requests: the step-time benchmark over slots filled by hipb_bench_fill.
 * With spare prompt rows configured these are the wide steps hipb_run
 * launches (spare rows idle: no slot is feeding a prompt). */
void hipb_bench_steps(HipbEngine *e, int n);
/* The engine's HIP stream (hipStream_t), for events and profiling. */
void *hipb_stream(HipbEngine *e);

#ifdef __cplusplus
}
#endif
#endif
