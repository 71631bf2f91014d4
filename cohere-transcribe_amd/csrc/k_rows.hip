// k_rows.hip — row-wise kernels: layernorm, embedding+LN, argmax, small
// elementwise helpers.  One wavefront per row; rows are independent, so
// results never depend on how many rows a launch covers.
#include "ct_dev.h"
#include "ct_launch.h"
#include "../../include/model_types.h"
#include <limits.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "ct_warm.h"

namespace {

constexpr int LN_MAXV = 32;   // register-cached elements per lane (D <= 2048)

// LayerNorm of one row held in registers: mean, then the mean of squared
// deviations, 1/sqrt(var + 1e-5), scale and shift
// (backends/cpu/backend.c:109-122).
__device__ __forceinline__ void ln_row(float (&v)[LN_MAXV], int D, int lane,
                                       const uint16_t *w, const uint16_t *b, float *dst) {
    // gain and bias loaded before the reductions, so their latency overlaps
    float wv[LN_MAXV], bv[LN_MAXV];
#pragma unroll
    for (int i = 0; i < LN_MAXV; i++) {
        const int d = lane + i * 64;
        wv[i] = d < D ? bf2f(w[d]) : 0.0f;
        bv[i] = d < D ? bf2f(b[d]) : 0.0f;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < LN_MAXV; i++) {
        const int d = lane + i * 64;
        if (d < D) s += v[i];
    }
    const float mu = wave_sum(s) / (float)D;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < LN_MAXV; i++) {
        const int d = lane + i * 64;
        if (d < D) { const float c = v[i] - mu; q += c * c; }
    }
    const float rs = 1.0f / sqrtf(wave_sum(q) / (float)D + 1e-5f);
#pragma unroll
    for (int i = 0; i < LN_MAXV; i++) {
        const int d = lane + i * 64;
        if (d < D) dst[d] = (v[i] - mu) * rs * wv[i] + bv[i];
    }
}

__global__ __launch_bounds__(256) void layernorm_kernel(float *dst, const float *src,
                                                        const uint16_t *w, const uint16_t *b,
                                                        int T, int D) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= T) return;
    const float *x = src + (long)row * D;
    float v[LN_MAXV];
#pragma unroll
    for (int i = 0; i < LN_MAXV; i++) {
        const int d = lane + i * 64;
        v[i] = d < D ? x[d] : 0.0f;
    }
    ln_row(v, D, lane, w, b, dst + (long)row * D);
}

// D = 256*V (the model's 1024 and 1280): each lane holds V float4 of the row
// (elements 4(lane + 64i) .. + 3), all loaded before any arithmetic.

// Mean, then 1/sqrt(mean squared deviation + 1e-5), of such a row.
template <int V>
__device__ __forceinline__ void ln_stats(const float4 (&v)[V], float &mu, float &rs) {
    constexpr int D = 256 * V;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; i++) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    mu = wave_sum(s) / (float)D;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        const float a = v[i].x - mu, bb = v[i].y - mu, c = v[i].z - mu, d = v[i].w - mu;
        q += (a * a + bb * bb) + (c * c + d * d);
    }
    rs = 1.0f / sqrtf(wave_sum(q) / (float)D + 1e-5f);
}

// (v - mu) * rs * gain + bias, elementwise (backends/cpu/backend.c:109-122).
__device__ __forceinline__ float4 ln_apply(const float4 &v, float mu, float rs, ushort4 w, ushort4 b) {
    float4 o;
    o.x = (v.x - mu) * rs * bf2f(w.x) + bf2f(b.x);
    o.y = (v.y - mu) * rs * bf2f(w.y) + bf2f(b.y);
    o.z = (v.z - mu) * rs * bf2f(w.z) + bf2f(b.z);
    o.w = (v.w - mu) * rs * bf2f(w.w) + bf2f(b.w);
    return o;
}

template <int V>
__device__ __forceinline__ void ln_params(const uint16_t *w, const uint16_t *b, int lane, ushort4 (&w4)[V],
                                          ushort4 (&b4)[V]) {
#pragma unroll
    for (int i = 0; i < V; i++) {
        w4[i] = reinterpret_cast<const ushort4 *>(w)[lane + 64 * i];
        b4[i] = reinterpret_cast<const ushort4 *>(b)[lane + 64 * i];
    }
}

// Element group lane + 64i of a row written as its hi/lo bf16 split (lo
// plane optional).
__device__ __forceinline__ void ln_store_split(uint16_t *hi, uint16_t *lo, long off, int idx, float4 o) {
    ushort4 h4, l4;
    split_bf16(o.x, h4.x, l4.x);
    split_bf16(o.y, h4.y, l4.y);
    split_bf16(o.z, h4.z, l4.z);
    split_bf16(o.w, h4.w, l4.w);
    reinterpret_cast<ushort4 *>(hi + off)[idx] = h4;
    if (lo) reinterpret_cast<ushort4 *>(lo + off)[idx] = l4;
}

template <int V>
__global__ __launch_bounds__(256) void layernorm_vec_kernel(float *dst, const float *src,
                                                            const uint16_t *w, const uint16_t *b, int T) {
    constexpr int D = 256 * V;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= T) return;
    const float4 *x = reinterpret_cast<const float4 *>(src + (long)row * D);
    float4 v[V];
    ushort4 w4[V], b4[V];
#pragma unroll
    for (int i = 0; i < V; i++) v[i] = x[lane + 64 * i];
    ln_params<V>(w, b, lane, w4, b4);
    float mu, rs;
    ln_stats<V>(v, mu, rs);
    float4 *y = reinterpret_cast<float4 *>(dst + (long)row * D);
#pragma unroll
    for (int i = 0; i < V; i++) y[lane + 64 * i] = ln_apply(v[i], mu, rs, w4[i], b4[i]);
}

// Same as layernorm_vec_kernel, writing each output as its hi/lo bf16 split.
template <int V>
__global__ __launch_bounds__(256) void layernorm_split_kernel(uint16_t *hi, uint16_t *lo,
                                                              const float *src, const uint16_t *w,
                                                              const uint16_t *b, int T) {
    constexpr int D = 256 * V;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= T) return;
    const float4 *x = reinterpret_cast<const float4 *>(src + (long)row * D);
    float4 v[V];
    ushort4 w4[V], b4[V];
#pragma unroll
    for (int i = 0; i < V; i++) v[i] = x[lane + 64 * i];
    ln_params<V>(w, b, lane, w4, b4);
    float mu, rs;
    ln_stats<V>(v, mu, rs);
#pragma unroll
    for (int i = 0; i < V; i++) ln_store_split(hi, lo, (long)row * D, lane + 64 * i, ln_apply(v[i], mu, rs, w4[i], b4[i]));
}

// Two LayerNorms in a row, as the encoder runs them from one layer's output
// norm into the next layer's first FFN norm: x = LN1(x) in place, then
// LN2(x) as its hi/lo split.  The second norm works on the first one's fp32
// results in registers, the values a separate launch would read back, so the
// bits are those of layernorm_vec_kernel followed by layernorm_split_kernel.
template <int V>
__global__ __launch_bounds__(256) void layernorm_pair_split_kernel(float *xio, uint16_t *hi, uint16_t *lo,
                                                                   const uint16_t *w1, const uint16_t *b1,
                                                                   const uint16_t *w2, const uint16_t *b2,
                                                                   int T) {
    constexpr int D = 256 * V;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= T) return;
    float4 *x = reinterpret_cast<float4 *>(xio + (long)row * D);
    float4 v[V];
    ushort4 w4[V], b4[V], w4b[V], b4b[V];
#pragma unroll
    for (int i = 0; i < V; i++) v[i] = x[lane + 64 * i];
    ln_params<V>(w1, b1, lane, w4, b4);
    ln_params<V>(w2, b2, lane, w4b, b4b);
    float mu, rs;
    ln_stats<V>(v, mu, rs);
#pragma unroll
    for (int i = 0; i < V; i++) {
        v[i] = ln_apply(v[i], mu, rs, w4[i], b4[i]);
        x[lane + 64 * i] = v[i];
    }
    ln_stats<V>(v, mu, rs);
#pragma unroll
    for (int i = 0; i < V; i++) ln_store_split(hi, lo, (long)row * D, lane + 64 * i, ln_apply(v[i], mu, rs, w4b[i], b4b[i]));
}

// Rows longer than 2048: three passes over the (cache-resident) row.
__global__ __launch_bounds__(64) void layernorm_long_kernel(float *dst, const float *src,
                                                            const uint16_t *w, const uint16_t *b,
                                                            int T, int D) {
    const int row = blockIdx.x, lane = threadIdx.x;
    if (row >= T) return;
    const float *x = src + (long)row * D;
    float *y = dst + (long)row * D;
    float s = 0.0f;
    for (int d = lane; d < D; d += 64) s += x[d];
    const float mu = wave_sum(s) / (float)D;
    float q = 0.0f;
    for (int d = lane; d < D; d += 64) { const float c = x[d] - mu; q += c * c; }
    const float rs = 1.0f / sqrtf(wave_sum(q) / (float)D + 1e-5f);
    for (int d = lane; d < D; d += 64) y[d] = (x[d] - mu) * rs * bf2f(w[d]) + bf2f(b[d]);
}

// h[r] = LN(etw[tok] + epw[pos]) (backends/cpu/backend.c:362-371, 425-435).
__global__ __launch_bounds__(256) void embed_ln_kernel(float *h, const int *tokens, int R,
                                                       int pos_start, const int *pos_len,
                                                       const int *active,
                                                       const uint16_t *etw, const uint16_t *epw,
                                                       const uint16_t *lnw, const uint16_t *lnb) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= R) return;
    if (active && !active[r]) return;
    const long tok = tokens[r];
    const long pos = pos_len ? (long)pos_len[r] - 1 : (long)pos_start + r;
    float v[LN_MAXV];
#pragma unroll
    for (int i = 0; i < LN_MAXV; i++) {
        const int d = lane + i * 64;
        v[i] = d < DEC_D ? bf2f(etw[tok * DEC_D + d]) + bf2f(epw[pos * DEC_D + d]) : 0.0f;
    }
    ln_row(v, DEC_D, lane, lnw, lnb, h + (long)r * DEC_D);
}

// First index of the maximum with the sequential scan's rules
// (backends/cpu/backend.c:446-456): strict '>', so ties keep the lowest index
// and NaN never wins; a NaN at index 0 stays the answer.
__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__global__ __launch_bounds__(256) void argmax_kernel(int *out, const float *logits, int n,
                                                     const int *active) {
    const int r = blockIdx.x;
    if (active && !active[r]) return;
    const float *x = logits + (long)r * n;
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int i = threadIdx.x; i < n; i += 256) better(bv, bi, x[i], i);
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
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; k++) better(bv, bi, sv[k], si[k]);
        out[r] = (x[0] != x[0] || bi == INT_MAX) ? 0 : bi;
    }
}

__global__ void add_kernel(float *dst, const float *src, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] += src[i];
}

// Row m of src (D floats, D % 4 == 0) to row dst_row[m] of dst.
__global__ void copy_rows_kernel(float *dst, const float *src, const int *dst_row, int M, int D) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x, per = D / 4;
    if (i >= (long)M * per) return;
    const int m = (int)(i / per), c = (int)(i % per);
    reinterpret_cast<float4 *>(dst + (long)dst_row[m] * D)[c] = reinterpret_cast<const float4 *>(src + (long)m * D)[c];
}

__global__ void causal_mask_kernel(float *mask, int S) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)S * S) return;
    const int q = (int)(i / S), k = (int)(i % S);
    mask[i] = k > q ? -1e9f : 0.0f;
}

// pe[p][2k] = sin(pos w_k), pe[p][2k+1] = cos(pos w_k), pos = T-1-p
// (backends/cpu/backend.c:231-242); w_k comes from the host (glibc expf).
__global__ void rel_pos_emb_kernel(float *pe, int T, const float *inv_freq) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long L = 2L * T - 1;
    if (i >= L * (ENC_D / 2)) return;
    const int p = (int)(i / (ENC_D / 2)), k = (int)(i % (ENC_D / 2));
    const float arg = (float)(T - 1 - p) * inv_freq[k];
    pe[(long)p * ENC_D + 2 * k] = sinf(arg);
    pe[(long)p * ENC_D + 2 * k + 1] = cosf(arg);
}

__global__ void inc_kernel(int *p) {
    if (threadIdx.x == 0) *p += 1;
}

// The folded input of a GEMM on LayerNorm(h) (gemv_kernel FOLD) from one row
// of h held as a float4 per thread (256 threads, thread t: columns 4t..4t+3):
// each 32-column block's (mean, squared deviations) into lnstat (a block is 8
// consecutive lanes), and frag(h * w), each product rounded on its own.
__device__ __forceinline__ void fold_tail(float4 v, ushort4 w4, float *lnstat, uint16_t *frag, int row) {
    const int t = threadIdx.x;
    float sum = (v.x + v.y) + (v.z + v.w);
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    const float mean = sum / 32.0f;
    const float c0 = v.x - mean, c1 = v.y - mean, c2 = v.z - mean, c3 = v.w - mean;
    float m2 = (c0 * c0 + c1 * c1) + (c2 * c2 + c3 * c3);
    m2 += __shfl_xor(m2, 1);
    m2 += __shfl_xor(m2, 2);
    m2 += __shfl_xor(m2, 4);
    if ((t & 7) == 0)
        reinterpret_cast<float2 *>(lnstat)[(long)row * CT_LN_BLOCKS + (t >> 3)] = make_float2(mean, m2);
    const float o[4] = {mul_rn(v.x, bf2f(w4.x)), mul_rn(v.y, bf2f(w4.y)), mul_rn(v.z, bf2f(w4.z)),
                        mul_rn(v.w, bf2f(w4.w))};
    uint16_t hh[4], ll[4];
#pragma unroll
    for (int j = 0; j < 4; j++) split_bf16(o[j], hh[j], ll[j]);
    const long off = ct_frag_off(row, 4 * t, DEC_D);
    *reinterpret_cast<ushort4 *>(frag + off) = make_ushort4(hh[0], hh[1], hh[2], hh[3]);
    *reinterpret_cast<ushort4 *>(frag + off + 512) = make_ushort4(ll[0], ll[1], ll[2], ll[3]);
}

// The two-pass LayerNorm of one row held as a float4 per thread (mean, then
// the variance of the centred values, eps 1e-5; backends/cpu/backend.c:
// 109-122), each output split hi/lo into frag.
__device__ __forceinline__ void ln_tail(float4 v, ushort4 w4, ushort4 b4, uint16_t *frag, int row) {
    const int t = threadIdx.x, wv = t >> 6, lane = t & 63;
    __shared__ float red[2][4];
    const float s = wave_sum((v.x + v.y) + (v.z + v.w));
    if (lane == 0) red[0][wv] = s;
    __syncthreads();
    const float mu = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) / (float)DEC_D;
    const float c0 = v.x - mu, c1 = v.y - mu, c2 = v.z - mu, c3 = v.w - mu;
    const float q = wave_sum((c0 * c0 + c1 * c1) + (c2 * c2 + c3 * c3));
    if (lane == 0) red[1][wv] = q;
    __syncthreads();
    const float var = ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) / (float)DEC_D;
    const float rs = 1.0f / sqrtf(var + 1e-5f);
    const float o[4] = {c0 * rs * bf2f(w4.x) + bf2f(b4.x), c1 * rs * bf2f(w4.y) + bf2f(b4.y),
                        c2 * rs * bf2f(w4.z) + bf2f(b4.z), c3 * rs * bf2f(w4.w) + bf2f(b4.w)};
    uint16_t hh[4], ll[4];
#pragma unroll
    for (int j = 0; j < 4; j++) split_bf16(o[j], hh[j], ll[j]);
    const long off = ct_frag_off(row, 4 * t, DEC_D);
    *reinterpret_cast<ushort4 *>(frag + off) = make_ushort4(hh[0], hh[1], hh[2], hh[3]);
    *reinterpret_cast<ushort4 *>(frag + off + 512) = make_ushort4(ll[0], ll[1], ll[2], ll[3]);
}

// The decode step's first launch: row r's embedding LayerNorm (wave 0, the
// arithmetic of embed_ln_kernel), written to h for active rows (inactive rows
// keep their stale h), then the folded input of the first layer's QKV
// projection (fold_tail).
__global__ __launch_bounds__(256) void embed_fold_kernel(float *h, float *lnstat, uint16_t *frag,
                                                         const int *tokens, const int *pos_len,
                                                         const int *active, const uint16_t *etw,
                                                         const uint16_t *epw, const uint16_t *elnw,
                                                         const uint16_t *elnb, const uint16_t *w, int M,
                                                         CtWarmSet warm) {
    if ((int)blockIdx.x >= M) {
        ct_warm_tiles<256>(warm, blockIdx.x & 7, (blockIdx.x - M) >> 3);
        return;
    }
    const int row = blockIdx.x, t = threadIdx.x;
    __shared__ float4 s_h[DEC_D / 4];
    const ushort4 w4 = reinterpret_cast<const ushort4 *>(w)[t];
    const bool act = active[row] != 0;
    float4 *x = reinterpret_cast<float4 *>(h + (long)row * DEC_D);
    if (!act) {
        s_h[t] = x[t];
    } else if (t < 64) {
        const long tok = tokens[row], pos = (long)pos_len[row] - 1;
        float v[LN_MAXV];
#pragma unroll
        for (int i = 0; i < LN_MAXV; i++) {
            const int d = t + i * 64;
            v[i] = d < DEC_D ? bf2f(etw[tok * DEC_D + d]) + bf2f(epw[pos * DEC_D + d]) : 0.0f;
        }
        ln_row(v, DEC_D, t, elnw, elnb, reinterpret_cast<float *>(s_h));
    }
    __syncthreads();
    const float4 v = s_h[t];
    if (act) x[t] = v;
    fold_tail(v, w4, lnstat, frag, row);
}

// Residual update after a K-split projection, one 256-thread workgroup per
// row, a float4 per thread: h += ((parts[0] + parts[1]) + ...) + pbias (the
// slices in order, then the bias), every load issued before the first add;
// then (NORM false) the folded input of the next GEMM's LayerNorm with gain w
// (fold_tail), or (NORM) the LayerNorm itself with gain w and bias b (ln_tail).
template <int NP, bool NORM>
__global__ __launch_bounds__(256) void resid_fold_kernel(float *h, float *lnstat, uint16_t *frag,
                                                         const float *parts, long pstride,
                                                         const uint16_t *pbias, const uint16_t *w,
                                                         const uint16_t *b, int M, CtWarmSet warm) {
    if ((int)blockIdx.x >= M) {
        // read-ahead workgroups: launch position q runs on XCD q % 8
        ct_warm_tiles<256>(warm, blockIdx.x & 7, (blockIdx.x - M) >> 3);
        return;
    }
    const int row = blockIdx.x, t = threadIdx.x;
    float4 *x = reinterpret_cast<float4 *>(h + (long)row * DEC_D);
    float4 v = x[t];
    float4 pr[NP];
#pragma unroll
    for (int p = 0; p < NP; p++)
        pr[p] = reinterpret_cast<const float4 *>(parts + p * pstride + (long)row * DEC_D)[t];
    const ushort4 pb4 = pbias ? reinterpret_cast<const ushort4 *>(pbias)[t] : make_ushort4(0, 0, 0, 0);
    const ushort4 w4 = reinterpret_cast<const ushort4 *>(w)[t];
    const ushort4 b4 = NORM ? reinterpret_cast<const ushort4 *>(b)[t] : make_ushort4(0, 0, 0, 0);
    float4 a = pr[0];
#pragma unroll
    for (int p = 1; p < NP; p++) {
        a.x += pr[p].x; a.y += pr[p].y; a.z += pr[p].z; a.w += pr[p].w;
    }
    if (pbias) {
        a.x += bf2f(pb4.x); a.y += bf2f(pb4.y);
        a.z += bf2f(pb4.z); a.w += bf2f(pb4.w);
    }
    v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w;
    x[t] = v;
    if (NORM) ln_tail(v, w4, b4, frag, row);
    else fold_tail(v, w4, lnstat, frag, row);
}

}  // namespace

extern "C" void ctk_layernorm(float *dst, const float *src, const uint16_t *w, const uint16_t *b,
                              int T, int D, hipStream_t s) {
    if (T <= 0) return;
    const bool al = ((uintptr_t)dst % 16 == 0) && ((uintptr_t)src % 16 == 0) &&
                    ((uintptr_t)w % 8 == 0) && ((uintptr_t)b % 8 == 0);
    if (al && D == 1024)
        hipLaunchKernelGGL(layernorm_vec_kernel<4>, dim3((T + 3) / 4), dim3(256), 0, s, dst, src, w, b, T);
    else if (al && D == 1280)
        hipLaunchKernelGGL(layernorm_vec_kernel<5>, dim3((T + 3) / 4), dim3(256), 0, s, dst, src, w, b, T);
    else if (D <= 64 * LN_MAXV)
        hipLaunchKernelGGL(layernorm_kernel, dim3((T + 3) / 4), dim3(256), 0, s, dst, src, w, b, T, D);
    else
        hipLaunchKernelGGL(layernorm_long_kernel, dim3(T), dim3(64), 0, s, dst, src, w, b, T, D);
}

extern "C" void ctk_layernorm_split(uint16_t *hi, uint16_t *lo, const float *src, const uint16_t *w,
                                    const uint16_t *b, int T, int D, hipStream_t s) {
    if (T <= 0) return;
    if ((uintptr_t)src % 16 || (uintptr_t)hi % 8 || (uintptr_t)lo % 8 || (uintptr_t)w % 8 ||
        (uintptr_t)b % 8 || (D != 1024 && D != 1280)) {
        fprintf(stderr, "ctk_layernorm_split: needs D in {1024, 1280}, aligned rows and 8-byte aligned gain/bias\n");
        exit(1);
    }
    if (D == 1024)
        hipLaunchKernelGGL(layernorm_split_kernel<4>, dim3((T + 3) / 4), dim3(256), 0, s, hi, lo, src, w, b, T);
    else
        hipLaunchKernelGGL(layernorm_split_kernel<5>, dim3((T + 3) / 4), dim3(256), 0, s, hi, lo, src, w, b, T);
}

extern "C" void ctk_layernorm_pair_split(float *x, uint16_t *hi, uint16_t *lo, const uint16_t *w1,
                                         const uint16_t *b1, const uint16_t *w2, const uint16_t *b2, int T,
                                         int D, hipStream_t s) {
    if (T <= 0) return;
    if ((uintptr_t)x % 16 || (uintptr_t)hi % 8 || (uintptr_t)lo % 8 || (uintptr_t)w1 % 8 ||
        (uintptr_t)b1 % 8 || (uintptr_t)w2 % 8 || (uintptr_t)b2 % 8 || (D != 1024 && D != 1280)) {
        fprintf(stderr, "ctk_layernorm_pair_split: needs D in {1024, 1280}, aligned rows and 8-byte aligned "
                        "gains and biases\n");
        exit(1);
    }
    if (D == 1024)
        hipLaunchKernelGGL(layernorm_pair_split_kernel<4>, dim3((T + 3) / 4), dim3(256), 0, s, x, hi, lo, w1, b1,
                           w2, b2, T);
    else
        hipLaunchKernelGGL(layernorm_pair_split_kernel<5>, dim3((T + 3) / 4), dim3(256), 0, s, x, hi, lo, w1, b1,
                           w2, b2, T);
}

extern "C" void ctk_embed_ln(float *h, const int *tokens, int R, int pos_start, const int *pos_len,
                             const int *active, const uint16_t *etw, const uint16_t *epw,
                             const uint16_t *lnw, const uint16_t *lnb, hipStream_t s) {
    if (R <= 0) return;
    hipLaunchKernelGGL(embed_ln_kernel, dim3((R + 3) / 4), dim3(256), 0, s, h, tokens, R, pos_start,
                       pos_len, active, etw, epw, lnw, lnb);
}

extern "C" void ctk_resid_fold(float *h, float *lnstat, uint16_t *frag, const float *parts, int nparts,
                               const uint16_t *pbias, const uint16_t *w, const uint16_t *b, int M,
                               const CtWarmSet *warm, hipStream_t s) {
    if (M <= 0) return;
    if ((uintptr_t)h % 16 || (uintptr_t)frag % 16 || (uintptr_t)parts % 16 || (!b && (uintptr_t)lnstat % 8) ||
        (uintptr_t)w % 8 || (b && (uintptr_t)b % 8) || (pbias && (uintptr_t)pbias % 8)) {
        fprintf(stderr, "ctk_resid_fold: needs 16-byte aligned rows and partials, 8-byte aligned lnstat, "
                        "gain and biases\n");
        exit(1);
    }
    if (nparts != 8) {
        fprintf(stderr, "ctk_resid_fold: %d partial slices not supported (8)\n", nparts);
        exit(1);
    }
    CtWarmSet ws;
    memset(&ws, 0, sizeof ws);
    if (warm) ws = *warm;
    const int G = M + 8 * ct_warm_rows(&ws, "ctk_resid_fold");
    const long ps = (long)M * DEC_D;
    if (b)
        hipLaunchKernelGGL((resid_fold_kernel<8, true>), dim3(G), dim3(256), 0, s, h, lnstat, frag, parts, ps,
                           pbias, w, b, M, ws);
    else
        hipLaunchKernelGGL((resid_fold_kernel<8, false>), dim3(G), dim3(256), 0, s, h, lnstat, frag, parts, ps,
                           pbias, w, b, M, ws);
}

extern "C" void ctk_embed_fold(float *h, float *lnstat, uint16_t *frag, const int *tokens,
                               const int *pos_len, const int *active, const uint16_t *etw,
                               const uint16_t *epw, const uint16_t *elnw, const uint16_t *elnb,
                               const uint16_t *w, int M, const CtWarmSet *warm, hipStream_t s) {
    if (M <= 0) return;
    if ((uintptr_t)h % 16 || (uintptr_t)frag % 16 || (uintptr_t)lnstat % 8 || (uintptr_t)w % 8) {
        fprintf(stderr, "ctk_embed_fold: needs 16-byte aligned rows, 8-byte aligned lnstat and gain\n");
        exit(1);
    }
    CtWarmSet ws;
    memset(&ws, 0, sizeof ws);
    if (warm) ws = *warm;
    const int G = M + 8 * ct_warm_rows(&ws, "ctk_embed_fold");
    hipLaunchKernelGGL(embed_fold_kernel, dim3(G), dim3(256), 0, s, h, lnstat, frag, tokens, pos_len, active,
                       etw, epw, elnw, elnb, w, M, ws);
}

extern "C" void ctk_argmax(int *out, const float *logits, int R, int n, const int *active,
                           hipStream_t s) {
    if (R <= 0) return;
    hipLaunchKernelGGL(argmax_kernel, dim3(R), dim3(256), 0, s, out, logits, n, active);
}

extern "C" void ctk_add(float *dst, const float *src, long n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst, src, n);
}

extern "C" void ctk_copy_rows(float *dst, const float *src, const int *dst_row, int M, int D, hipStream_t s) {
    if (M <= 0) return;
    if (D % 4 || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15)) {
        fprintf(stderr, "ctk_copy_rows: needs D %% 4 == 0 and 16-byte aligned rows\n");
        exit(1);
    }
    const long n = (long)M * (D / 4);
    hipLaunchKernelGGL(copy_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst, src, dst_row,
                       M, D);
}

extern "C" void ctk_causal_mask(float *mask, int S, hipStream_t s) {
    const long n = (long)S * S;
    if (n <= 0) return;
    hipLaunchKernelGGL(causal_mask_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, mask, S);
}

extern "C" void ctk_rel_pos_emb(float *pe, int T, const float *inv_freq, hipStream_t s) {
    const long n = (2L * T - 1) * (ENC_D / 2);
    if (n <= 0) return;
    hipLaunchKernelGGL(rel_pos_emb_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, pe, T,
                       inv_freq);
}

extern "C" void ctk_inc(int *p, hipStream_t s) {
    hipLaunchKernelGGL(inc_kernel, dim3(1), dim3(64), 0, s, p);
}
