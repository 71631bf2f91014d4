/* engine_demo.c — the decode engine driven from plain C, as a serving host
 * would use it: seeded synthetic weights at the model's dimensions, uploaded
 * the way transcribe.c uploads its blob (transcribe.c:1376-1379), then
 * clips of seeded synthetic audio submitted as 16 kHz PCM, encoded and
 * decoded with continuous batching, and each request's tokens printed as
 * one line "req <id>: <n> <tok> <tok> ...".
 *
 *   engine_demo <weight seed> <weight variant> <clips> <slots>
 *
 * Clip i has 8000 + 3000 i samples (audio seed 500 + i) and a forced length
 * of 4 + 3 (i mod 5) tokens with EOS suppressed before it.
 */
#include <stdio.h>
#include <stdlib.h>
#include "../../include/backend.h"
#include "../../include/hipb.h"
#include "../host/synth.h"

static const int PROMPT[] = {13764, 7, 4, 16, 62, 62, 6, 9, 11, 13};

int main(int argc, char **argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s <weight seed> <weight variant> <clips> <slots>\n", argv[0]);
        return 2;
    }
    const unsigned long long seed = strtoull(argv[1], NULL, 10);
    const int variant = atoi(argv[2]), n = atoi(argv[3]), slots = atoi(argv[4]);
    if (n < 1 || n > 64 || slots < 1 || slots > 64) {
        fprintf(stderr, "clips and slots must be in [1, 64]\n");
        return 2;
    }
    const size_t bytes = ct_synth_file_bytes();
    uint8_t *image = malloc(bytes);
    if (!image || ct_synth_weights(image, bytes, seed, variant, 0) != 0) {
        fprintf(stderr, "cannot build the synthetic weights\n");
        return 1;
    }
    Weights W;
    const uint8_t *data;
    size_t data_bytes;
    if (ct_weights_bind(image, bytes, &W, &data, &data_bytes) != 0) {
        fprintf(stderr, "weights image is missing a tensor\n");
        return 1;
    }
    backend_weights_upload_blob(data, data_bytes);
    backend_init(0);

    HipbConfig cfg = {.slots = slots, .max_requests = n, .max_frames = 376, .kv_bf16 = 1,
                      .max_tokens = 32, .prefill_rows = 0, .admit_order = 1, .enc_ffn_bf16 = 1};
    HipbEngine *e = hipb_create(&cfg, &W);
    const int np = (int)(sizeof PROMPT / sizeof PROMPT[0]);
    for (int i = 0; i < n; i++) {
        const int ns = 8000 + 3000 * i;
        float *pcm = malloc((size_t)ns * sizeof(float));
        if (!pcm) return 1;
        ct_synth_audio(pcm, ns, 500 + (unsigned)i);
        hipb_submit_pcm(e, pcm, ns, PROMPT, np, 4 + 3 * (i % 5), HIPB_SUPPRESS_EOS | HIPB_FORCE_EOS);
        free(pcm);
    }
    hipb_encode(e, 4096);
    hipb_run(e, 4);
    int toks[32];
    for (int i = 0; i < n; i++) {
        const int k = hipb_tokens(e, i, toks, 32);
        printf("req %d: %d", i, k);
        for (int j = 0; j < k; j++) printf(" %d", toks[j]);
        printf("\n");
    }
    hipb_destroy(e);
    backend_thread_cleanup();
    free(image);
    return 0;
}
