// kq_quant.hpp -- bit-exact activation quantizers shared by the standalone
// quantize kernels and the fused matvec prologue.
//
// Both follow lloom-tensor's from_float exactly (k_quants.rs:738-767 for
// Q8_0, :2400-2438 for Q8_K): same operations, same order, no contraction,
// IEEE division, half-away rounding and saturating casts.
#pragma once

#include "kq_common.hpp"

namespace lloom {

#pragma clang fp contract(off)

// Q8_K of one 256-element block held by a full wave, lane l owning
// elements 4l..4l+3 (x).  Returns the 4 quantized bytes packed little
// endian; *d is the block scale, *bsum the sum of this lane's 16-element
// group (identical on the 4 lanes of the group).
//   max = the signed value of the largest |x|, first index on ties
//   iscale = -127 / max; q = clamp(round(iscale * x), -128, 127); d = 1 / iscale
//   an all-zero block: d = 0, q = 0, bsums = 0
__device__ __forceinline__ uint32_t q8k_block_wave(float4 x, int lane, float* d, int* bsum) {
    float xs[4] = {x.x, x.y, x.z, x.w};
    float amax = 0.0f, mx = 0.0f;
    int idx = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float a = __builtin_fabsf(xs[j]);
        if (amax < a) {
            amax = a;
            mx = xs[j];
            idx = 4 * lane + j;
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        float oa = __shfl_xor(amax, o, 64);
        float om = __shfl_xor(mx, o, 64);
        int oi = __shfl_xor(idx, o, 64);
        if (oa > amax || (oa == amax && oi < idx)) {
            amax = oa;
            mx = om;
            idx = oi;
        }
    }
    uint32_t packed = 0;
    int s = 0;
    if (amax == 0.0f) {
        *d = 0.0f;
    } else {
        float iscale = -127.0f / mx;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float v = round_away(iscale * xs[j]);
            v = v < -128.0f ? -128.0f : (v > 127.0f ? 127.0f : v);
            int q = sat_i8(v);
            s += q;
            packed |= ((uint32_t)q & 0xffu) << (8 * j);
        }
        *d = 1.0f / iscale;
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    *bsum = s;
    return packed;
}

// Q8_0 of one 32-element block held by 8 consecutive lanes, sub-lane j
// owning elements 4j..4j+3.  d = amax / 127 (kept f32 for the rounding),
// id = 1/d or 0, q = round(x * id) as i8; *d16 is f16(d).
__device__ __forceinline__ uint32_t q8_0_block_8lanes(float4 x, uint16_t* d16) {
    float xs[4] = {x.x, x.y, x.z, x.w};
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) amax = __builtin_fmaxf(__builtin_fabsf(xs[j]), amax);
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 4, 64));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    *d16 = f32_to_f16(d);
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int q = sat_i8(round_away(xs[j] * id));
        packed |= ((uint32_t)q & 0xffu) << (8 * j);
    }
    return packed;
}

}  // namespace lloom
