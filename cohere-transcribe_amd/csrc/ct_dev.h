// ct_dev.h — device-side helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

#define CT_WAVE 64

__device__ __forceinline__ float bf2f(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

// fp32 -> bf16, round to nearest even, on gfx950's conversion instruction
// (v_cvt_pk_bf16_f32).  For every non-NaN input it gives the bits of the
// integer form (u + 0x7fff + ((u >> 16) & 1)) >> 16, checked over all 2^32
// patterns on the device; a NaN stays a NaN.
__device__ __forceinline__ uint16_t f2bf(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
}

// 1 / (1 + e^-x) on the hardware exp2 (e^-x = 2^(-x log2 e)) and
// reciprocal, each about 1 ulp: within a few units in the last place of the
// expf-and-divide forms of SiLU and the GLU gate (backends/cpu/backend.c:62,
// 149, 309), at a handful of instructions instead of a libm call and a
// division.  x -> -inf gives 0, x -> +inf gives 1.
__device__ __forceinline__ float sigmoid_hw(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// a * b rounded to fp32 on its own: never contracted into a later add or
// subtract (hipcc contracts across statements, __fmul_rn included)
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}

// x = hi + lo + r with hi, lo bf16 and |r| <= 2^-17 |x|: the two-term split
// that lets bf16 MFMA multiply an fp32 activation by an exact bf16 weight.
__device__ __forceinline__ void split_bf16(float x, uint16_t &hi, uint16_t &lo) {
    hi = f2bf(x);
    lo = f2bf(x - bf2f(hi));
}

__device__ __forceinline__ bf16x8 as_bf16x8(u16x8 v) {
    return __builtin_bit_cast(bf16x8, v);
}

// v from the lane DPP control CTRL names (row_ror, row_bcast); lanes of rows
// outside ROWS get 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}

// Sum / max over the 64 lanes of a wavefront (every lane gets the result).
// The sum stays in the VALU: rotations by 8, 4, 2 and 1 within each 16-lane
// row (every lane then holds its row's sum), row 15's lane added into rows 1
// and 3, lane 31 into rows 2 and 3, and lane 63's total read back for all.
// Call with the whole wavefront active.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0x128, 0xF>(v);
    v += dpp_f<0x124, 0xF>(v);
    v += dpp_f<0x122, 0xF>(v);
    v += dpp_f<0x121, 0xF>(v);
    v += dpp_f<0x142, 0xA>(v);
    v += dpp_f<0x143, 0xC>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, CT_WAVE));
    return v;
}
__device__ __forceinline__ unsigned wave_xor(unsigned v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v ^= (unsigned)__shfl_xor((int)v, o, CT_WAVE);
    return v;
}
// Lane exchange within a row of 16 lanes (DPP): CTRL 0xB1 = quad_perm
// [1,0,3,2], 0x4E = quad_perm [2,3,0,1], 0x141 = row_half_mirror (lane i of
// each 8 reads 7-i), 0x140 = row_mirror (lane i reads 15-i).
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of 16 lanes.  Each stage adds the same pair of
// partial sums as an xor-1/2/4/8 butterfly, so every lane holds the same
// value, computed in the same order.
__device__ __forceinline__ float group16_sum(float v) {
    v += dpp_row<0xB1>(v);
    v += dpp_row<0x4E>(v);
    v += dpp_row<0x141>(v);
    v += dpp_row<0x140>(v);
    return v;
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
