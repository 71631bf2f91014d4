/* model_types.h — model dimensions and the weight-pointer structs that cross
 * the backend boundary.
 *
 * This is part of the drop-in ABI: transcribe.c / model.h pass pointers to
 * ELayer / DLayer / Weights into backend functions, so the field ORDER of the
 * three structs below must stay exactly as in the reference
 * (backends/model_types.h:52-77) and the constants must keep their values
 * (backends/model_types.h:14-37).  Everything else here is this backend's own.
 */
#ifndef CT_MODEL_TYPES_H
#define CT_MODEL_TYPES_H

#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>

/* Conformer encoder (backends/model_types.h:14-20). */
#define ENC_D    1280
#define ENC_FF   5120
#define ENC_H    8
#define ENC_DK   160
#define ENC_N    48
#define ENC_CK   9
#define SUB_CH   256

/* Transformer decoder (backends/model_types.h:22-26). */
#define DEC_D    1024
#define DEC_FF   4096
#define DEC_H    8
#define DEC_DK   128
#define DEC_N    8

#define VOCAB    16384
#define MAX_SEQ  1024
#define MAX_VOCAB 16384

/* Audio front-end (backends/model_types.h:32-37). */
#define SR       16000
#define N_FFT    512
#define HOP_LEN  160
#define WIN_LEN  400
#define N_MELS   128
#define N_BINS   257

/* A bf16 value is the high half of an fp32 bit pattern; widening is exact.
 * Same contract as backends/model_types.h:42-47. */
static inline float bf16(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* Weight-pointer structs.  All pointers are bf16 tensors inside the host
 * safetensors blob; backends translate them to device addresses by offset.
 * Field order is ABI (backends/model_types.h:52-77). */
typedef struct {
    const uint16_t *ff1_lnw, *ff1_lnb, *ff1_w1, *ff1_b1, *ff1_w2, *ff1_b2;
    const uint16_t *sa_lnw, *sa_lnb, *sa_qw, *sa_qb, *sa_kw, *sa_kb,
                   *sa_vw, *sa_vb, *sa_pw, *sa_ow, *sa_ob, *sa_pbu, *sa_pbv;
    const uint16_t *cv_lnw, *cv_lnb, *cv_pw1w, *cv_pw1b, *cv_dww, *cv_dwb,
                   *cv_bnw, *cv_bnb, *cv_bnmean, *cv_bnvar, *cv_pw2w, *cv_pw2b;
    const uint16_t *ff2_lnw, *ff2_lnb, *ff2_w1, *ff2_b1, *ff2_w2, *ff2_b2;
    const uint16_t *out_lnw, *out_lnb;
} ELayer;

typedef struct {
    const uint16_t *sa_lnw, *sa_lnb, *sa_qw, *sa_qb, *sa_kw, *sa_kb,
                   *sa_vw, *sa_vb, *sa_ow, *sa_ob;
    const uint16_t *ca_lnw, *ca_lnb, *ca_qw, *ca_qb, *ca_kw, *ca_kb,
                   *ca_vw, *ca_vb, *ca_ow, *ca_ob;
    const uint16_t *ffn_lnw, *ffn_lnb, *ffn_w1, *ffn_b1, *ffn_w2, *ffn_b2;
} DLayer;

typedef struct {
    const uint16_t *s0w, *s0b, *s2w, *s2b, *s3w, *s3b, *s5w, *s5b, *s6w, *s6b, *sow, *sob;
    ELayer enc[ENC_N];
    const uint16_t *prw, *prb;
    const uint16_t *etw, *epw, *elnw, *elnb;
    DLayer dec[DEC_N];
    const uint16_t *dlnw, *dlnb, *hdb;
} Weights;

#endif /* CT_MODEL_TYPES_H */
