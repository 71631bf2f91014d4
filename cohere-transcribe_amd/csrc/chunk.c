/* chunk.c — silence-based chunking of long recordings (host side).
 *
 * Behaviour follows transcribe.c:397-535 of the reference: 10 ms frame RMS,
 * an automatic threshold from the recording's own noise floor (the 5th
 * percentile of frame RMS on a 1024-bucket histogram, +20 dB) unless a level
 * in dB is given, candidate cuts at the middle of every silence run of at
 * least `silence_dur` seconds that ends before the recording does, and a
 * cut kept only once `target_sec` seconds have passed since the last kept
 * cut.  The float arithmetic (a sequential fused multiply-add sum of squares
 * per frame, the same float expressions for the thresholds) is kept as the
 * reference evaluates it, so the cut points are the same sample indices.
 *
 * The engine admits chunk c + 1 of a recording only after chunk c has
 * finished and builds its prompt from chunk c's tokens on the device
 * (k_engine.hip, eng_end).
 */
#include "../../include/hipb.h"
#include "../../include/model_types.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define RMS_BUCKETS 1024   /* transcribe.c:408 */
#define MAX_CUTS 4096      /* transcribe.c:500 */

static float frame_rms(const float *x) {
    float acc = 0.0f;
    for (int i = 0; i < HOP_LEN; i++) acc = fmaf(x[i], x[i], acc);
    return sqrtf(acc / HOP_LEN);
}

int hipb_chunk_bounds(const float *pcm, int n_samples, float silence_db, float silence_dur,
                      float target_sec, int *bounds, int cap) {
    if (n_samples <= 0 || cap < 1) return 0;
    const int nf = n_samples / HOP_LEN;
    float *rms = malloc((size_t)(nf > 0 ? nf : 1) * sizeof(float));
    int *cut = malloc(MAX_CUTS * sizeof(int));
    if (!rms || !cut) { free(rms); free(cut); return -1; }
    for (int f = 0; f < nf; f++) rms[f] = frame_rms(pcm + (size_t)f * HOP_LEN);

    float thresh;
    if (isnan(silence_db)) {
        /* first bucket at which the running count reaches nf / 20 */
        int hist[RMS_BUCKETS];
        memset(hist, 0, sizeof hist);
        for (int f = 0; f < nf; f++) {
            const int b = (int)(rms[f] * RMS_BUCKETS);
            hist[b < RMS_BUCKETS ? b : RMS_BUCKETS - 1]++;
        }
        const int need = nf / 20;
        int b = 0, seen = hist[0];
        while (seen < need && b + 1 < RMS_BUCKETS) seen += hist[++b];
        thresh = seen >= need ? ((float)b / RMS_BUCKETS) * 10.0f : 1.0f;
    } else {
        thresh = powf(10.0f, silence_db / 20.0f);
    }

    /* candidate cuts: midpoints of quiet runs of >= min_run frames */
    const int min_run = (int)(silence_dur * SR / HOP_LEN);
    int ncut = 0, run0 = -1;
    for (int f = 0; f < nf; f++) {
        if (rms[f] < thresh) {
            if (run0 < 0) run0 = f;
            continue;
        }
        if (run0 >= 0 && f - run0 >= min_run && ncut < MAX_CUTS) cut[ncut++] = ((run0 + f) / 2) * HOP_LEN;
        run0 = -1;
    }
    free(rms);

    /* keep a cut once target_samp samples have passed since the last kept one */
    const int target_samp = (int)(target_sec * SR);
    int kept = 0, last = 0;
    for (int i = 0; i < ncut; i++)
        if (cut[i] - last >= target_samp) last = cut[kept++] = cut[i];

    /* chunks [start, end); empty ones are dropped */
    int n = 0, start = 0;
    for (int c = 0; c <= kept; c++) {
        const int end = c < kept ? cut[c] : n_samples;
        if (end > start) {
            if (n >= cap) break;
            bounds[2 * n] = start;
            bounds[2 * n + 1] = end;
            n++;
        }
        start = end;
    }
    free(cut);
    return n;
}
