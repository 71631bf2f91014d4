/* synth.h — seeded synthetic workload: BF16 safetensors weights at the
 * model's dimensions, laid out as the reference converter writes them, and
 * seeded test audio.  No network, no checkpoint: every byte is a function of
 * (seed, variant).
 */
#ifndef CT_SYNTH_H
#define CT_SYNTH_H

#include "../../include/model_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* variant 0: the specified random init — linear/conv/embedding/pos tensors
 *            N(0, 0.02), norm and BN gains 1, biases 0, BN mean 0, var 1.
 * variant 1: the same plus perturbed affine terms (biases and BN shift
 *            N(0,0.02), gains 1+N(0,0.02), BN var 1+|N(0,0.1)|), which makes
 *            every bias/gain path observable in parity tests.
 * variant 2: the spec init with decoder-layer linear weights N(0, 0.12).  With
 *            the tied LM head and sigma 0.02 the final hidden state stays
 *            aligned with the input token's embedding, so greedy decoding
 *            repeats the last prompt token; the larger decoder weights make
 *            the residual dominate and greedy decoding input-dependent, which
 *            gives token-id parity tests near-ties to survive.
 * variant 3: the spec init with decoder-layer linear weights N(0, 0.08): the
 *            smallest of these scales whose greedy decoding is input-dependent
 *            while the bf16 rounding of K/V moves the fp32 logits by less than
 *            1e-2 (about 6e-3; 1-1.7% with 0.12). */
#define CT_SYNTH_SPEC      0
#define CT_SYNTH_PERTURBED 1
#define CT_SYNTH_DEC_HOT   2
#define CT_SYNTH_DEC_WARM  3

/* Number of tensors and total file size (8-byte length + JSON header + data). */
int    ct_synth_tensor_count(void);
size_t ct_synth_file_bytes(void);
/* Writes the complete safetensors file image into buf (cap >= file bytes).
 * nthreads <= 0 uses all cores.  Returns 0 on success. */
int    ct_synth_weights(uint8_t *buf, size_t cap, uint64_t seed, int variant, int nthreads);

/* Parses a safetensors image (synthetic or converted) and fills W with
 * pointers into it.  *data / *data_bytes receive the data section (the blob
 * handed to backend_weights_upload_blob).  Returns 0, or -1 if a tensor the
 * model needs is missing. */
int    ct_weights_bind(const uint8_t *image, size_t size, Weights *W,
                       const uint8_t **data, size_t *data_bytes);

/* Seeded clip: five sinusoids f~U(100,4000) Hz, random phase, amplitudes
 * U(0,0.1), plus N(0, 0.01^2) noise; 16 kHz fp32. */
void   ct_synth_audio(float *out, int n_samples, uint64_t seed);

/* Counter-based generator shared by the workload generators:
 * the 64-bit hash of (key, i), and N(0,1) by inverse CDF on 16 bits. */
uint64_t ct_hash64(uint64_t key, uint64_t i);
float    ct_normal16(uint64_t h);

#ifdef __cplusplus
}
#endif
#endif
