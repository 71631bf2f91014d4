// k_engine.hip — slot-table kernels of the decode engine.
//
// eng_begin admits queued requests into free slots and prepares each slot's
// step inputs (token, position, cache lengths, KV row offset); eng_end turns
// each active slot's logits into its next token under the request's policy
// and retires finished requests, freeing the slot for the next eng_begin.
// Together they replace the host loop of transcribe.c:733-795 (gather
// tokens, advance S, argmax, append, retire on EOS or MAX_SEQ) with no host
// round trip.
#include "ct_dev.h"
#include "ct_engine.h"
#include "../../include/model_types.h"
#include <limits.h>
#include <stdio.h>
#include <stdlib.h>

#define EOS_ID 3   // model.h:24

namespace {

// Writes row `row` of the step: token `tok` of slot s's request, whose
// encoder state (T_enc frames of cross K/V) is in entry `ent`, at position
// pos (0-based) of the slot's self cache.
__device__ __forceinline__ void set_row(const CtEngDev &d, int row, int s, int ent, int T, int tok, int pos) {
    d.act[row] = 1;
    d.tok[row] = tok;
    d.pos_len[row] = pos + 1;
    d.cross_len[row] = T;
    d.cross_idx[row] = ent;
    d.row_slot[row] = s;
    d.kv_rowoff[row] = ((long)s * DEC_H * d.kv_rows + pos) * DEC_DK;
}

__device__ __forceinline__ void clear_row(const CtEngDev &d, int row) {
    d.act[row] = 0;
    d.tok[row] = 0;
    d.pos_len[row] = 0;
    d.cross_len[row] = 0;
    d.cross_idx[row] = 0;
    d.row_slot[row] = 0;
    d.kv_rowoff[row] = -1;
}

// Admission, then the rows of this step.  Slot s always owns row s, which
// carries the slot's last token of the step (so the LM head and eng_end stay
// per slot).  With `extra` spare rows (rows slots .. slots+extra-1), a slot
// still feeding its prompt takes up to `extra` more prompt tokens this step,
// spare rows dealt in slot order; each row is an ordinary decode row at its
// own position, so a prompt fed k tokens per step gives the same bits as one
// per step.  q[3] receives the prompt tokens still unfed after this step.
// Thread s serves slot s (slots <= 256).  A slot that keeps its request finds
// everything it needs in the slot table (the request's fields are copied there
// at admission, the last generated token by eng_end), so a step with no
// admission and no prompt ids to feed makes one round of loads; newly
// admitted slots load their request's fields, prompt-feeding slots their ids.
// Exclusive prefix of v over the workgroup's 256 threads in thread order
// (one barrier); total receives the sum.  sums: 4 ints of LDS for this call.
__device__ __forceinline__ int block_prefix(int v, int *sums, int &total) {
    const int tid = threadIdx.x;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if ((tid & 63) >= o) x += y;
    }
    if ((tid & 63) == 63) sums[tid >> 6] = x;
    __syncthreads();
    int base = x - v;
    for (int w = 0; w < (tid >> 6); w++) base += sums[w];
    total = (sums[0] + sums[1]) + (sums[2] + sums[3]);
    return base;
}

__global__ __launch_bounds__(256) void eng_begin_kernel(CtEngDev d, int extra) {
    const int tid = threadIdx.x, s = tid;
    __shared__ int s_app[CT_ENG_MAX_SLOTS], s_cand[CT_ENG_MAX_SLOTS], s_q[6], s_asum[4];
    __shared__ int s_wsum[4], s_left[4];
    __shared__ int s_pl[2 * CT_ENG_MAX_SLOTS], s_cl[2 * CT_ENG_MAX_SLOTS];   // row lengths this step
    int r = -1, S = 0, np = 0, T = 0, tok = 0, ent = 0, pend = -1, q0 = 0, q1 = 0, f0 = 0, f1 = 0, wm = 0;
    const int mk = d.ring_mask;
    if (s < d.slots) {
        r = d.slot_req[s];
        pend = d.pend[s];
        S = d.slot_S[s];
        np = d.slot_np[s];
        T = d.slot_T[s];
        tok = d.slot_tok[s];
        ent = d.slot_ent[s];
    }
    if (tid == 0) {
        q0 = d.q[0]; q1 = d.q[1]; f0 = d.q[4];
        // host-published words (possibly written while this step runs on
        // another stream): acquire, so the queue entries read after them are
        // at least as new
        f1 = __hip_atomic_load(&d.q[5], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
        wm = __hip_atomic_load(&d.q[7], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
        s_q[0] = q0; s_q[1] = q1; s_q[2] = f0; s_q[3] = f1; s_q[4] = wm;
    }
    // Released successors join the ring rq in slot order, then the free
    // slots, in slot order, take the waiting successors (rq[q0..), the ones
    // joining now last) up to the first one not yet encoded, i.e. without an
    // encoder entry published (ring order is kept: it and those behind it
    // wait), then fresh requests (fq[q4..q5), all encoded when published):
    // the c-th free slot takes the c-th of them.
    // One prefix counts both (pending in the low 16 bits, free in the high).
    const bool is_p = s < d.slots && pend >= 0, is_f = s < d.slots && r < 0;
    int tot;
    const int pre = block_prefix((int)is_p | ((int)is_f << 16), s_asum, tot);
    const int pidx = pre & 0xffff, fidx = pre >> 16, npend = tot & 0xffff, nfree = tot >> 16;
    q0 = s_q[0]; q1 = s_q[1]; f0 = s_q[2]; f1 = s_q[3]; wm = s_q[4];
    if (is_p) {
        d.rq[(q1 + pidx) & mk] = pend;
        s_app[pidx] = pend;
    }
    if (tid == 0) s_q[5] = INT_MAX;
    __syncthreads();
    const int waiting = q1 - q0, avail = waiting + npend;
    // the first lim ring entries (one past what the free slots can take, so
    // the head left behind is checked too): the admissible prefix ends at
    // the first entry whose encoder batch is not published
    const int lim = min(min(avail, nfree + 1), (int)CT_ENG_MAX_SLOTS);
    if (tid < lim) {
        const int c = tid < waiting ? d.rq[(q0 + tid) & mk] : s_app[tid - waiting];
        s_cand[tid] = c;
        if (d.req_entry[c & mk] < 0) atomicMin(&s_q[5], tid);   // not published yet
    }
    __syncthreads();
    const int blocked = s_q[5];                  // INT_MAX: none of the lim
    const int ready = min(blocked, avail);       // admissible successors
    const int from_rq = min(nfree, ready);
    bool fresh = false;
    if (is_f) {
        if (fidx < from_rq) { r = s_cand[fidx]; fresh = true; }
        else if (fidx - from_rq < f1 - f0) {
            r = __hip_atomic_load(&d.fq[(f0 + fidx - from_rq) & mk], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
            fresh = true;
        }
    }
    if (tid == 0) {
        d.q[0] = q0 + from_rq;
        d.q[1] = q1 + npend;
        d.q[4] = f0 + min(nfree - from_rq, f1 - f0);
        d.q[8] = blocked < lim ? 1 : 0;
        d.q[9] = wm;
    }
    int want = 0;
    if (s < d.slots) {
        if (pend >= 0) d.pend[s] = -1;
        d.slot_req[s] = r;
        if (fresh) {
            const int rs = r & mk;
            S = 0;
            np = d.req_np[rs]; T = d.req_T[rs]; ent = d.req_entry[rs];
            const int fl = d.req_flags[rs], lim = d.req_limit[rs], ng = d.req_ngen[rs];
            d.slot_np[s] = np; d.slot_T[s] = T; d.slot_ent[s] = ent;
            d.slot_flags[s] = fl; d.slot_lim[s] = lim; d.slot_ng[s] = ng;
        }
        if (r >= 0 && S < np) want = min(np - S, 1 + extra) - 1;
    }
    // exclusive prefix of the spare rows wanted, in slot order
    int x = want;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if ((tid & 63) >= o) x += y;
    }
    if ((tid & 63) == 63) s_wsum[tid >> 6] = x;
    __syncthreads();
    int base = x - want;
    for (int w = 0; w < (tid >> 6); w++) base += s_wsum[w];
    const int wanted = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
    const int granted = max(0, min(want, extra - base));
    int left = 0;
    if (s < d.slots && r >= 0) {
        const int k = 1 + granted;
        const int *prompt = d.req_prompt + (long)(r & mk) * CT_PROMPT_MAX;
        for (int j = 0; j < granted; j++) {
            set_row(d, d.slots + base + j, s, ent, T, prompt[S + j], S + j);
            s_pl[d.slots + base + j] = S + j + 1;
            s_cl[d.slots + base + j] = T;
        }
        const int p = S + k - 1;
        const int t = p < np ? prompt[p] : tok;
        set_row(d, s, s, ent, T, t, p);
        s_pl[s] = p + 1;
        s_cl[s] = T;
        d.slot_S[s] = S + k;
        left = max(0, np - (S + k));
    } else if (s < d.slots) {
        clear_row(d, s);
        s_pl[s] = s_cl[s] = 0;
    }
    // spare rows nobody took this step
    for (int i = min(wanted, extra) + tid; i < extra; i += 256) {
        clear_row(d, d.slots + i);
        s_pl[d.slots + i] = s_cl[d.slots + i] = 0;
    }
    // prompt tokens still to feed, summed over slots
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) left += __shfl_xor(left, o, 64);
    if ((tid & 63) == 0) s_left[tid >> 6] = left;
    __syncthreads();
    if (tid == 0) {
        d.q[3] = s_left[0] + s_left[1] + s_left[2] + s_left[3];
        d.q[6] = d.slots + min(wanted, extra);
    }
    // the step's rows by descending self and cross length (ties by row),
    // for steps large enough that the attention deals its items by them
    const int B = d.slots + extra;
    for (int row = tid; B >= d.rank_min && row < B; row += 256) {
        const int lp = s_pl[row], lc = s_cl[row];
        int rp = 0, rc = 0;
        for (int j = 0; j < B; j++) {
            const int pj = s_pl[j], cj = s_cl[j];
            rp += (pj > lp) || (pj == lp && j < row);
            rc += (cj > lc) || (cj == lc && j < row);
        }
        d.rank_self[rp] = row;
        d.rank_cross[rc] = row;
    }
}

__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

// First maximum (ties -> lowest id, NaN never chosen unless at id 0, as the
// sequential scan of backends/cpu/backend.c:446-456), optionally skipping EOS.
__global__ __launch_bounds__(256) void eng_end_kernel(CtEngDev d, const float *logits) {
    const int s = blockIdx.x;
    // one round of loads: the slot's state and its logits row
    const float *x = logits + (long)s * VOCAB;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    float4 v[VOCAB / 1024];
#pragma unroll
    for (int k = 0; k < VOCAB / 1024; k++) v[k] = x4[threadIdx.x + 256 * k];
    const int act = d.act[s], r = d.slot_req[s], S = d.slot_S[s], np = d.slot_np[s];
    const int flags = d.slot_flags[s], lim = d.slot_lim[s], ng = d.slot_ng[s];
    if (!act || S < np) return;                  // idle, or still feeding the prompt
    const int skip = (flags & 1) ? EOS_ID : -1;
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int k = 0; k < VOCAB / 1024; k++) {
        const int i = 4 * (threadIdx.x + 256 * k);
        if (i != skip) better(bv, bi, v[k].x, i);
        if (i + 1 != skip) better(bv, bi, v[k].y, i + 1);
        if (i + 2 != skip) better(bv, bi, v[k].z, i + 2);
        if (i + 3 != skip) better(bv, bi, v[k].w, i + 3);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        better(bv, bi, ov, oi);
    }
    __shared__ float sv[4];
    __shared__ int si[4];
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wv] = bv; si[wv] = bi; }
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int k = 1; k < 4; k++) better(bv, bi, sv[k], si[k]);
    const int first = skip == 0 ? 1 : 0;
    const float xf = first ? v[0].y : v[0].x;   // thread 0 holds logits 0..3
    int best = (xf != xf || bi == INT_MAX) ? first : bi;
    if ((flags & 2) && ng == lim - 1) best = EOS_ID;
    const int rs = r & d.ring_mask;
    d.req_out[(long)rs * d.smax + ng] = best;
    d.req_score[(long)rs * d.smax + ng] = bv;
    d.req_ngen[rs] = ng + 1;
    d.slot_ng[s] = ng + 1;
    d.slot_tok[s] = best;
    const bool fin = (best == EOS_ID && !(flags & 1)) || ng + 1 >= lim || S >= d.smax;
    if (fin) {
        d.slot_req[s] = -1;
        const int nx = d.req_next[rs];
        if (nx >= 0) {
            // The successor's prompt becomes pre + carry + post: its first two
            // ids, then the last <= CT_CARRY_MAX generated ids of this
            // request without its final one, then the rest of its own prompt
            // (transcribe.c:382-387, 510-529).
            const int gen = ng + 1;
            const int nc = min(gen > 0 ? gen - 1 : 0, CT_CARRY_MAX);
            const int ns = nx & d.ring_mask;
            int *pp = d.req_prompt + (long)ns * CT_PROMPT_MAX;
            const int np = d.req_np[ns];
            for (int i = np - 1; i >= 2; i--) pp[i + nc] = pp[i];
            const int *og = d.req_out + (long)rs * d.smax;
            for (int i = 0; i < nc; i++) pp[2 + i] = og[gen - 1 - nc + i];
            d.req_np[ns] = np + nc;
            d.pend[s] = nx;
            atomicAdd(&d.q[10], 1);
        }
        // retirement order, for the host to recycle the encoder entry
        const int k = atomicAdd(&d.q[2], 1);
        d.ret[k & d.ring_mask] = r;
    }
}

// dst[pairs[2i] & mask] = pairs[2i + 1] for i < n.
__global__ void ring_scatter_kernel(int *dst, const int *pairs, int n, int mask) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[pairs[2 * i] & mask] = pairs[2 * i + 1];
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

// Approximately normal: sum of four 16-bit uniforms, centred and scaled to
// unit variance (Irwin-Hall).  Synthetic cache contents for the microbench.
__global__ void fill_random_kernel(void *p, long n, int bf16, float scale, uint64_t seed) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t h = mix64(seed + 0x9E3779B97F4A7C15ULL * (uint64_t)(i + 1));
        const float u = (float)(h & 0xffff) + (float)((h >> 16) & 0xffff) +
                        (float)((h >> 32) & 0xffff) + (float)(h >> 48);
        const float z = (u / 65536.0f - 2.0f) * 1.7320508f;
        if (bf16) reinterpret_cast<uint16_t *>(p)[i] = f2bf(z * scale);
        else reinterpret_cast<float *>(p)[i] = z * scale;
    }
}

}  // namespace

extern "C" void ctk_eng_begin(const CtEngDev *d, int extra, hipStream_t s) {
    if (d->slots > CT_ENG_MAX_SLOTS || extra < 0 || d->slots + extra > d->rows) {
        fprintf(stderr, "ctk_eng_begin: %d slots + %d spare rows exceed the engine's %d rows\n",
                d->slots, extra, d->rows);
        exit(1);
    }
    hipLaunchKernelGGL(eng_begin_kernel, dim3(1), dim3(256), 0, s, *d, extra);
}

extern "C" void ctk_eng_end(const CtEngDev *d, const float *logits, hipStream_t s) {
    hipLaunchKernelGGL(eng_end_kernel, dim3(d->slots), dim3(256), 0, s, *d, logits);
}

extern "C" void ctk_ring_scatter(int *dst, const int *pairs, int n, int mask, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(ring_scatter_kernel, dim3((n + 255) / 256), dim3(256), 0, s, dst, pairs, n, mask);
}

extern "C" void ctk_fill_random(void *p, long n, int bf16, float scale, uint64_t seed, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(fill_random_kernel, dim3(4096), dim3(256), 0, s, p, n, bf16, scale, seed);
}
