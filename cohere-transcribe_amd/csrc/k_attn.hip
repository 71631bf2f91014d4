// k_attn.hip — ragged scaled-dot-product attention for the decoder.
//
// One workgroup per (item, query row, head).  Sixteen 16-lane groups stream
// the item's keys (group g takes keys g, g+16, ...); each lane owns 8 of the
// 128 head dimensions, so a key row is read as one contiguous 256 B (bf16) or
// 512 B (fp32) segment.  Each group keeps an online softmax (running max,
// running sum, weighted V); the 16 partial states are merged in LDS in a fixed
// order.  The key split depends only on the item's own length, so an item's
// result is the same whatever else is in the batch.
//
// Semantics: backends/cpu/backend.c:339-360 (scores * 1/sqrt(128) + mask,
// softmax, weighted sum of V), 410-413 (T_k from the device counter),
// 478-500 (ragged batch: T_k per item from the latched S or T_enc).
#include "ct_dev.h"
#include "ct_launch.h"
#include "../../include/model_types.h"

namespace {

template <bool BF16, bool VEC>
__device__ __forceinline__ void load8(const void *base, long off, float (&v)[8]) {
    if (!VEC) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = BF16 ? bf2f(reinterpret_cast<const uint16_t *>(base)[off + i])
                        : reinterpret_cast<const float *>(base)[off + i];
    } else if (BF16) {
        const u16x8 w = *reinterpret_cast<const u16x8 *>(reinterpret_cast<const uint16_t *>(base) + off);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = bf2f(w[i]);
    } else {
        const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(base) + off);
        const float4 x0 = p[0], x1 = p[1];
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    }
}

// Output element col of row bq (= b*T_q + qi): plain fp32 at out[off], or
// split hi/lo into the frag layout the next decode GEMM reads.
__device__ __forceinline__ void store_out(const CtAttn &a, int bq, int col, long off, float v) {
    if (a.out_frag) {
        uint16_t hh, ll;
        split_bf16(v, hh, ll);
        const long o = ct_frag_off(bq, col, a.H * DEC_DK);
        a.out_frag[o] = hh;
        a.out_frag[o + 512] = ll;
    } else {
        a.out[off] = v;
    }
}

template <bool BF16, bool VEC>
__global__ __launch_bounds__(256) void attn_kernel(CtAttn a) {
    const int bq = blockIdx.x, h = blockIdx.y;
    const int b = bq / a.T_q, qi = bq % a.T_q;
    const int T = a.lens ? a.lens[(long)b * a.lens_step] : a.len_const;
    const int tid = threadIdx.x, g = tid >> 4, l16 = tid & 15;
    const long qoff = (long)b * a.q_sb + (long)qi * a.q_st + h * DEC_DK;
    if (T <= 0) {
        if (tid < DEC_DK) store_out(a, bq, h * DEC_DK + tid, qoff + tid, 0.0f);
        return;
    }
    float q[8];
    if (a.q_parts) {
        // query = ((part 0 + part 1) + ...) + bias, the decode GEMM's K-slices
        const float *qp = a.q_parts + qoff + l16 * 8;
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = qp[i];
        for (int p = 1; p < a.q_nparts; p++)
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] += qp[p * a.q_pstride + i];
        if (a.q_bias)
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] += bf2f(a.q_bias[h * DEC_DK + l16 * 8 + i]);
    } else {
        const float *qp = a.Q + qoff + l16 * 8;
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = qp[i];
    }
    const float *mrow = a.mask ? a.mask + (long)qi * T : nullptr;
    const long item = a.kv_index ? (long)a.kv_index[b] : (long)b;
    const long base = item * a.kv_sb + (long)h * a.kv_sh + l16 * 8;

    float m = -INFINITY, l = 0.0f, o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = 0.0f;

    for (int k = g; k < T; k += 32) {
        // two keys in flight per group: k and k + 16
        const int k2 = k + 16;
        const bool has2 = k2 < T;
        float kv0[8], kv1[8], vv0[8], vv1[8];
        load8<BF16, VEC>(a.K, base + (long)k * a.kv_st, kv0);
        load8<BF16, VEC>(a.V, base + (long)k * a.kv_st, vv0);
        if (has2) {
            load8<BF16, VEC>(a.K, base + (long)k2 * a.kv_st, kv1);
            load8<BF16, VEC>(a.V, base + (long)k2 * a.kv_st, vv1);
        }
        float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) d0 += q[i] * kv0[i];
        if (has2) {
#pragma unroll
            for (int i = 0; i < 8; i++) d1 += q[i] * kv1[i];
        }
        float s0 = group16_sum(d0) * a.scale + (mrow ? mrow[k] : 0.0f);
        float s1 = group16_sum(d1) * a.scale + ((mrow && has2) ? mrow[k2] : 0.0f);
        {
            const float mn = fmaxf(m, s0);
            const float c = expf(m - mn), p = expf(s0 - mn);
            l = l * c + p;
#pragma unroll
            for (int i = 0; i < 8; i++) o[i] = o[i] * c + p * vv0[i];
            m = mn;
        }
        if (has2) {
            const float mn = fmaxf(m, s1);
            const float c = expf(m - mn), p = expf(s1 - mn);
            l = l * c + p;
#pragma unroll
            for (int i = 0; i < 8; i++) o[i] = o[i] * c + p * vv1[i];
            m = mn;
        }
    }

    __shared__ float sm[16], sl[16], so[16][DEC_DK];
    if (l16 == 0) { sm[g] = m; sl[g] = l; }
#pragma unroll
    for (int i = 0; i < 8; i++) so[g][l16 * 8 + i] = o[i];
    __syncthreads();
    if (tid < DEC_DK) {
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < 16; j++) M = fmaxf(M, sm[j]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (sm[j] == -INFINITY) continue;
            const float w = expf(sm[j] - M);
            num += w * so[j][tid];
            den += w * sl[j];
        }
        store_out(a, bq, h * DEC_DK + tid, qoff + tid, num / den);
    }
}

}  // namespace

extern "C" void ctk_attn(const CtAttn *a, hipStream_t s) {
    if (a->B <= 0 || a->T_q <= 0) return;
    const dim3 grid(a->B * a->T_q, a->H);
    // 16-byte vector loads need every 8-element K/V segment aligned.
    const long esz = a->kv_bf16 ? 2 : 4, need = 16 / esz;
    const bool vec = ((uintptr_t)a->K % 16 == 0) && ((uintptr_t)a->V % 16 == 0) &&
                     a->kv_sb % need == 0 && a->kv_st % need == 0 && a->kv_sh % need == 0;
    if (a->kv_bf16) {
        if (vec) hipLaunchKernelGGL((attn_kernel<true, true>), grid, dim3(256), 0, s, *a);
        else hipLaunchKernelGGL((attn_kernel<true, false>), grid, dim3(256), 0, s, *a);
    } else {
        if (vec) hipLaunchKernelGGL((attn_kernel<false, true>), grid, dim3(256), 0, s, *a);
        else hipLaunchKernelGGL((attn_kernel<false, false>), grid, dim3(256), 0, s, *a);
    }
}
