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
__device__ __forceinline__ uint32_t q8k_block_wave(float4 x, float* d, int* bsum) {
    const float xs[4] = {x.x, x.y, x.z, x.w};
    // amax over the block (NaN never wins, as `amax < x.abs()` never holds)
    float la = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) la = __builtin_fmaxf(la, __builtin_fabsf(xs[j]));
    const float amax = wave_max(la);
    // The first element (lowest lane, then lowest j) with |x| == amax.  No
    // branch anywhere: the two blocks a wave may quantize back to back then
    // interleave, and the x loads stay ahead of the weight loads.
    float mine = 0.0f;
    bool hit = false;
#pragma unroll
    for (int j = 3; j >= 0; j--) {
        const bool h = __builtin_fabsf(xs[j]) == amax;
        mine = h ? xs[j] : mine;
        hit = hit || h;
    }
    const unsigned long long ballot = __ballot(hit);
    const int first = ballot ? __builtin_ctzll(ballot) : 0;
    const float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), first));
    // amax == 0 (all zeros, or all NaN): iscale is +-inf or NaN, every
    // product is NaN and converts to 0, and d is forced to +0 as the CPU's
    // early return leaves it.
    const float iscale = -127.0f / mx;
    uint32_t packed = 0;
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int q = clampi(nearest_int(iscale * xs[j]), -128, 127);
        s += q;
        packed |= ((uint32_t)q & 0xffu) << (8 * j);
    }
    const float dd = 1.0f / iscale;
    *d = amax == 0.0f ? 0.0f : dd;
    s += dppi<DPP_XOR1>(s);
    s += dppi<DPP_XOR2>(s);
    *bsum = s;
    return packed;
}

// Q8_K of one 256-element block held by 16 lanes (a DPP row), lane j owning
// elements 16j .. 16j+15 (piece j of the GEMM's operand layout): the same
// operations as q8k_block_wave (max of |x|, first index on ties, iscale =
// -127 / max, round-half-away, saturate, d = 1 / iscale, d = 0 for an
// all-zero block), with the reductions over 16 lanes, so a wave quantizes
// four blocks at once.  Returns the lane's 16 bytes; *bsum is the sum of its
// 16 quants.
__device__ __forceinline__ uint4 q8k_block_row16(const float (&xs)[16], float* d, int* bsum) {
#pragma clang fp contract(off)
    float la = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) la = __builtin_fmaxf(la, __builtin_fabsf(xs[i]));
    la = __builtin_fmaxf(la, dpp<DPP_XOR1>(la));
    la = __builtin_fmaxf(la, dpp<DPP_XOR2>(la));
    la = __builtin_fmaxf(la, dpp<DPP_HALF_MIRROR>(la));
    const float amax = __builtin_fmaxf(la, dpp<DPP_ROW_MIRROR>(la));
    float mine = 0.0f;
    bool hit = false;
#pragma unroll
    for (int i = 15; i >= 0; i--) {
        const bool h = __builtin_fabsf(xs[i]) == amax;
        mine = h ? xs[i] : mine;
        hit = hit || h;
    }
    const int lane = __lane_id(), row = lane & 48;
    const uint32_t hits = (uint32_t)(__ballot(hit) >> row) & 0xffffu;
    const int first = hits ? __builtin_ctz(hits) : 0;
    const float mx = __shfl(mine, row + first, 64);
    const float iscale = -127.0f / mx;
    uint32_t w[4];
    int sum = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        uint32_t packed = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int q = clampi(nearest_int(iscale * xs[4 * c + b]), -128, 127);
            sum += q;
            packed |= ((uint32_t)q & 0xffu) << (8 * b);
        }
        w[c] = packed;
    }
    const float dd = 1.0f / iscale;
    *d = amax == 0.0f ? 0.0f : dd;
    *bsum = sum;
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Q8_0 of one 32-element block held by 8 consecutive lanes (aligned to 8),
// sub-lane j owning elements 4j..4j+3.  d = amax / 127 (kept f32 for the
// rounding), id = 1/d or 0, q = round(x * id) as i8; *d16 is f16(d).
__device__ __forceinline__ uint32_t q8_0_block_8lanes(float4 x, uint16_t* d16) {
    const float xs[4] = {x.x, x.y, x.z, x.w};
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) amax = __builtin_fmaxf(__builtin_fabsf(xs[j]), amax);
    amax = __builtin_fmaxf(amax, dpp<DPP_XOR1>(amax));
    amax = __builtin_fmaxf(amax, dpp<DPP_XOR2>(amax));
    amax = __builtin_fmaxf(amax, dpp<DPP_HALF_MIRROR>(amax));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    *d16 = f32_to_f16(d);
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int q = clampi(nearest_int(xs[j] * id), -128, 127);
        packed |= ((uint32_t)q & 0xffu) << (8 * j);
    }
    return packed;
}

// One wave quantizes block (mi, sb) of x [m][k] (Q8_K, bit-exact) into the
// split layout: qs permuted so one MFMA lane group's 8 bytes of every
// 32-element chunk are contiguous (or, tiled, into [mp/16][k/256][4][64][16]
// so a 16-row tile's operand pieces are 1 KB each), d into dt[sb][mp], and,
// with bsp, the eight 32-element sums as int8 (sum & 63, sum >> 6) into
// bsp[sb][mp][16].
__device__ __forceinline__ void q8k_split_block(const float* __restrict__ x, int8_t* __restrict__ qs,
                                                float* __restrict__ dt, int8_t* __restrict__ bsp, int k, int mp,
                                                int tiled, int mi, int sb, int lane) {
    const int nsb = k >> 8;
    const float4 v = *(const float4*)(x + (int64_t)mi * k + sb * 256 + 4 * lane);
    float d;
    int bs;
    const uint32_t q = q8k_block_wave(v, &d, &bs);
    // lane owns elements 4*lane..: sub-block lane/8, group (lane%8)/2, byte 4*(lane%2)
    const int off = 64 * ((lane & 7) >> 1) + 8 * (lane >> 3) + 4 * (lane & 1);
    if (tiled) {  // uniform
        const int64_t piece = (((int64_t)(mi >> 4) * nsb + sb) * 4 + ((off >> 4) & 3)) * 64 + 16 * (off >> 6) + (mi & 15);
        *(uint32_t*)(qs + piece * 16 + (off & 15)) = q;
    } else {
        *(uint32_t*)(qs + (int64_t)mi * k + sb * 256 + off) = q;
    }
    if (lane == 0) dt[(int64_t)sb * mp + mi] = d;
    if (bsp) {
        // bs is the 16-element sum of the lane's quad; the 8 lanes of
        // sub-block lane / 8 are two quads
        const int s32 = bs + dppi<DPP_HALF_MIRROR>(bs);
        if ((lane & 7) == 0) {
            int8_t* o = bsp + ((int64_t)sb * mp + mi) * 16 + (lane >> 3);
            o[0] = (int8_t)(s32 & 63);
            o[8] = (int8_t)(s32 >> 6);
        }
    }
}

}  // namespace lloom
