/* ct_abi_state.h — per-thread backend state (C). */
#ifndef CT_ABI_STATE_H
#define CT_ABI_STATE_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#define CT_MAX_DEVICES 8
#define CT_MAX_BATCH 256      /* backends/cpu/backend.c:31, backends/cuda/backend.cu:57 */
#define CT_GRAPH_CAP 1026     /* encoder + precompute + up to MAX_SEQ decoder graphs */

typedef struct {
    int tag, T, S, B;
    void *arena;
    hipGraph_t graph;
    hipGraphExec_t exec;
} CtGraph;

typedef struct {
    int dev;
    hipStream_t stream;
    float *arena;
    size_t arena_bytes;
    int *d_tokens;     /* [MAX_SEQ] staged token ids                    */
    int *d_S;          /* [1] device-side sequence counter (batch = 1)  */
    int *d_S_batch;    /* [256] latched self lengths                    */
    int *d_T_enc;      /* [256] latched cross lengths                   */
    int *d_active;     /* [256] active flags                            */
    int *d_out;        /* [256] current tokens / argmax results         */
    int *h_stage;      /* pinned host staging, 4*256 + MAX_SEQ ints      */
    CtGraph *graphs;
    int n_graphs, graph_cap;
} CtThread;

extern _Thread_local CtThread ct_t;

void ct_fatal(const char *what, const char *file, int line);
void ct_hip_check(hipError_t e, const char *expr, const char *file, int line);
const void *ct_dev_w(const void *host_ptr);
const float *ct_inv_freq(void);

#define CT_FATAL(msg) ct_fatal((msg), __FILE__, __LINE__)
#define CHK(x) ct_hip_check((x), #x, __FILE__, __LINE__)
#define CT_W(p) ((const uint16_t *)ct_dev_w(p))

#endif
