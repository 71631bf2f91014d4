// k_attn.hip — ragged scaled-dot-product attention for the decoder.
//
// One workgroup per (item, query row, head).  Sixteen 16-lane groups stream
// the item's keys (group g takes keys g, g+16, ..., KPI of them per loop
// trip, one softmax update per trip, the next trip's loads in flight while
// the current one is used); each lane owns 8 of the 128 head dimensions, so
// a key row is read as one contiguous 256 B (bf16) or 512 B (fp32) segment.
// Each group keeps an online softmax (running max, running sum, weighted V)
// in base 2 on the hardware exp2; the 16 partial states are merged in LDS in
// a fixed order.  The key split depends only on the item's own length, so an item's
// result is the same whatever else is in the batch.
//
// Semantics: backends/cpu/backend.c:339-360 (scores * 1/sqrt(128) + mask,
// softmax, weighted sum of V), 410-413 (T_k from the device counter),
// 478-500 (ragged batch: T_k per item from the latched S or T_enc).
#include <type_traits>
#include "ct_dev.h"
#include <stdio.h>
#include <stdlib.h>
#include "ct_launch.h"
#include "ct_warm.h"
#include "../../include/model_types.h"

namespace {

// lanes per key: 16, each owning 8 of the 128 head dimensions (one 16-byte
// bf16 piece); 8 lanes per key (16 dimensions a lane) measured slower
constexpr int CT_ATTN_LPK = 16;
// threads per workgroup (NT / LPK lane groups)
constexpr int CT_ATTN_NT = 256;
// keys per lane group per trip (bf16; fp32 caches use 4)
constexpr int CT_ATTN_KPI = 2;
// rows per item (CtAttn.kv_rows) from which the first key trip (of bf16
// caches) is issued ahead of the item's length: one trip's keys
constexpr int CT_ATTN_EARLY_ROWS = CT_ATTN_NT / CT_ATTN_LPK * CT_ATTN_KPI;

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

// Softmax weights as 2^x on the hardware exp2 (e^y = 2^(y log2 e), the
// log2 e folded into the score scale); 2^-inf = 0.
constexpr float LOG2E = 1.4426950408889634f;
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Sum over aligned groups of 16 lanes (one DPP row), every lane gets the
// result.
__device__ __forceinline__ float group_sum16(float v) {
    v += dpp_row<0xB1>(v);
    v += dpp_row<0x4E>(v);
    v += dpp_row<0x141>(v);
    return v + dpp_row<0x140>(v);
}

// LPK lanes per key: lane s of a group owns head dims [s*DPL, s*DPL + DPL),
// DPL = 128 / LPK, read as NV 16-byte (bf16) pieces; NG = NT / LPK groups
// stream keys g, g + NG, ... (KPI of them per trip, loads first).
template <bool BF16, bool VEC, int LPK, bool MASK, int NT, bool EARLY>
__global__ __launch_bounds__(NT) void attn_kernel(CtAttn a) {
    static_assert(LPK == 16, "one 16-lane DPP row per key");
    constexpr int DPL = DEC_DK / LPK, NV = DPL / 8, NG = NT / LPK;
    if ((int)blockIdx.y >= a.B * a.T_q) {
        // read-ahead rows: launch position h + H * row runs on XCD h (H % 8 == 0)
        ct_warm_tiles<NT>(a.warm, blockIdx.x, blockIdx.y - a.B * a.T_q);
        return;
    }
    // heads vary fastest in launch order: workgroup i runs on XCD i % 8, so
    // an item's 8 heads spread over all XCDs and every CU gets several items
    // (with items fastest, a CU held 2 heads of one item and the longest
    // item's CUs set the launch's duration)
    const int h = blockIdx.x;
    int bq = blockIdx.y;
    if (a.rank) {
        // positions p, p + 32, ... share a CU (32 per XCD); in alternate
        // blocks of 32 positions the ranks run backwards, so a CU's items
        // pair long with short
        const int p = blockIdx.y, blk = p >> 5, o = p & 31, w = min(32, a.B - (blk << 5));
        bq = a.rank[(blk << 5) + ((blk & 1) ? w - 1 - o : o)];
    }
    const int b = bq / a.T_q, qi = bq % a.T_q;
    const int tid = threadIdx.x, g = tid / LPK, ls = tid % LPK;
    const long qoff = (long)b * a.q_sb + (long)qi * a.q_st + h * DEC_DK;
    // Every load the prologue needs is issued before any of them is used:
    // the length, the cache index, (EARLY) the first key trip and the query
    // (or its K-slice partials).
    const int T = a.lens ? a.lens[(long)b * a.lens_step] : a.len_const;
    const long item = a.kv_index && b >= a.kv_direct ? (long)a.kv_index[b] : (long)b;
    const long base = item * a.kv_sb + (long)h * a.kv_sh + ls * DPL;
    constexpr int KPI = BF16 ? CT_ATTN_KPI : 4;
    constexpr int STEP = NG * KPI;
    static_assert(!EARLY || STEP <= CT_ATTN_EARLY_ROWS, "the first trip must stay inside the allocation");
    // raw 16-byte pieces stay in registers until use (bf16: 4 VGPRs a piece)
    using Raw = typename std::conditional<BF16 && VEC, u16x8, float[8]>::type;
    auto load_key = [&](int k, int v, Raw &kr, Raw &vr) {
        const long off = base + (long)k * a.kv_st + 8 * v;
        if constexpr (BF16 && VEC) {
            // non-temporal: a step reads each cache row once, so the rows do not
            // displace the weight tiles the launch's read-ahead rows bring into L2
            kr = __builtin_nontemporal_load(reinterpret_cast<const u16x8 *>(reinterpret_cast<const uint16_t *>(a.K) + off));
            vr = __builtin_nontemporal_load(reinterpret_cast<const u16x8 *>(reinterpret_cast<const uint16_t *>(a.V) + off));
        } else {
            load8<BF16, VEC>(a.K, off, kr);
            load8<BF16, VEC>(a.V, off, vr);
        }
    };
    Raw kA[KPI][NV], vA[KPI][NV];
    if constexpr (EARLY) {
        // keys g + NG*j < STEP <= rows allocated per item: in bounds whatever
        // the length; keys past it are never used
#pragma unroll
        for (int j = 0; j < KPI; j++)
#pragma unroll
            for (int v = 0; v < NV; v++) load_key(g + NG * j, v, kA[j][v], vA[j][v]);
    }
    float q[DPL];
    {
        const float *qp = a.Q + qoff + ls * DPL;
#pragma unroll
        for (int i = 0; i < DPL; i++) q[i] = qp[i];
    }
    if (T <= 0) {
        if (tid < DEC_DK) store_out(a, bq, h * DEC_DK + tid, qoff + tid, 0.0f);
        return;
    }
    const int kb = 0, ke = T;
    const float *mrow = MASK ? a.mask + (long)qi * T : nullptr;
    // scores and running maxima are kept in base 2: s * scale * log2(e)
    const float scale2 = a.scale * LOG2E;

    float m = -INFINITY, l = 0.0f, o[DPL];
#pragma unroll
    for (int i = 0; i < DPL; i++) o[i] = 0.0f;

    // trip at k0: keys k0 + NG*j (j < KPI) of this lane group.  Keys past
    // the end re-read the last key (in bounds, never used): the loads carry
    // no branch, so the wait before each use counts exactly the loads
    // issued after it and the next trip's loads stay in flight.
    auto load_trip = [&](int k0, Raw (&kr)[KPI][NV], Raw (&vr)[KPI][NV]) {
#pragma unroll
        for (int j = 0; j < KPI; j++) {
            const int k = min(k0 + NG * j, ke - 1);
#pragma unroll
            for (int v = 0; v < NV; v++) load_key(k, v, kr[j][v], vr[j][v]);
        }
    };
    // chunked online softmax: the trip's scores together, one rescale
    auto use_trip = [&](int k0, const Raw (&kr)[KPI][NV], const Raw (&vr)[KPI][NV]) {
        float sc[KPI];
#pragma unroll
        for (int j = 0; j < KPI; j++) {
            float d = 0.0f;
#pragma unroll
            for (int v = 0; v < NV; v++)
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float kf;
                    if constexpr (BF16 && VEC) kf = bf2f(kr[j][v][i]);
                    else kf = kr[j][v][i];
                    d += q[8 * v + i] * kf;
                }
            sc[j] = d;
        }
#pragma unroll
        for (int j = 0; j < KPI; j++) {
            const int k = k0 + NG * j;
            sc[j] = k < ke ? group_sum16(sc[j]) * scale2 + (MASK ? mrow[k] * LOG2E : 0.0f) : -INFINITY;
        }
        float mx = sc[0];
#pragma unroll
        for (int j = 1; j < KPI; j++) mx = fmaxf(mx, sc[j]);
        const float mn = fmaxf(m, mx);
        const float c = exp2_hw(m - mn);
        float p[KPI], ps = 0.0f;
#pragma unroll
        for (int j = 0; j < KPI; j++) {
            p[j] = k0 + NG * j < ke ? exp2_hw(sc[j] - mn) : 0.0f;
            ps += p[j];
        }
        l = l * c + ps;
#pragma unroll
        for (int v = 0; v < NV; v++)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float acc = o[8 * v + i] * c;
#pragma unroll
                for (int j = 0; j < KPI; j++) {
                    if (k0 + NG * j >= ke) break;
                    float vf;
                    if constexpr (BF16 && VEC) vf = bf2f(vr[j][v][i]);
                    else vf = vr[j][v][i];
                    acc += p[j] * vf;
                }
                o[8 * v + i] = acc;
            }
        m = mn;
    };
    // two trips in flight: the next trip's loads are issued before the
    // current trip is used (register sets A and B alternate)
    Raw kB[KPI][NV], vB[KPI][NV];
    int k0 = kb + g;
    if (!EARLY && k0 < ke) load_trip(k0, kA, vA);
    for (; k0 < ke; k0 += 2 * STEP) {
        const int k1 = k0 + STEP;
        load_trip(k1, kB, vB);
        use_trip(k0, kA, vA);
        if (k1 >= ke) break;
        load_trip(k1 + STEP, kA, vA);
        use_trip(k1, kB, vB);
    }

    __shared__ float sm[NG], sl[NG], so[NG][DEC_DK];
    if (ls == 0) { sm[g] = m; sl[g] = l; }
#pragma unroll
    for (int i = 0; i < DPL; i++) so[g][ls * DPL + i] = o[i];
    __syncthreads();
    if (tid < DEC_DK) {
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < NG; j++) M = fmaxf(M, sm[j]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int j = 0; j < NG; j++) {
            if (sm[j] == -INFINITY) continue;
            const float w = exp2_hw(sm[j] - M);
            num += w * so[j][tid];
            den += w * sl[j];
        }
        store_out(a, bq, h * DEC_DK + tid, qoff + tid, num / den);
    }
}

}  // namespace

extern "C" void ctk_attn(const CtAttn *a, hipStream_t s) {
    if (a->B <= 0 || a->T_q <= 0) return;
    if (a->rank && a->T_q != 1) {
        fprintf(stderr, "ctk_attn: a rank permutation needs one query per item\n");
        exit(1);
    }
    const int wrows = ct_warm_rows(&a->warm, "ctk_attn");
    if (wrows && (a->H != 8)) {
        fprintf(stderr, "ctk_attn: read-ahead rows need H == 8 (one workgroup per XCD)\n");
        exit(1);
    }
    const dim3 grid(a->H, a->B * a->T_q + wrows);
    // 16-byte vector loads need every 8-element K/V segment aligned.
    const long esz = a->kv_bf16 ? 2 : 4, need = 16 / esz;
    const bool vec = ((uintptr_t)a->K % 16 == 0) && ((uintptr_t)a->V % 16 == 0) &&
                     a->kv_sb % need == 0 && a->kv_st % need == 0 && a->kv_sh % need == 0;
    constexpr int LPK = CT_ATTN_LPK;
    constexpr int NT = CT_ATTN_NT;
    // the first key trip ahead of the length: decode caches (bf16, vector
    // loads) with enough rows per item
    const bool early = !a->mask && a->kv_bf16 && vec && a->kv_rows >= CT_ATTN_EARLY_ROWS;
#define AK(B, V, M, E) hipLaunchKernelGGL((attn_kernel<B, V, LPK, M, NT, E>), grid, dim3(NT), 0, s, *a)
    if (a->mask) {
        if (a->kv_bf16) { if (vec) AK(true, true, true, false); else AK(true, false, true, false); }
        else { if (vec) AK(false, true, true, false); else AK(false, false, true, false); }
    } else if (early) {
        AK(true, true, false, true);
    } else {
        if (a->kv_bf16) { if (vec) AK(true, true, false, false); else AK(true, false, false, false); }
        else { if (vec) AK(false, true, false, false); else AK(false, false, false, false); }
    }
#undef AK
}
