// kq_tasks.hpp -- a lane's "task" of a quantized weight row: the packed
// bytes of one 32-element piece (a 16-byte qs vector of a Q4_K superblock
// with its header, a 64-element quarter of a Q6_K superblock, or one Q8_0
// block), loaded as whole vectors and unpacked to int8 lanes and integer
// scales.  Shared by the decode matvec and the routed-expert kernels.
//
// Block layouts: k_quants.rs:154-159 (Q8_0), 216-223 (Q4_K), 254-261 (Q6_K);
// the Q4_K scale/min unpacking is get_scale_min_k4 (utils.rs:50-60).
#pragma once

#include "kq_common.hpp"

namespace lloom {

template <int TYPE>
struct MvTraits;
template <>
struct MvTraits<T_Q4K> {
    static constexpr int BE = 256, BB = Q4K_BYTES, P = 8, VT = T_Q8K;
};
template <>
struct MvTraits<T_Q6K> {
    static constexpr int BE = 256, BB = Q6K_BYTES, P = 4, VT = T_Q8K;
};
template <>
struct MvTraits<T_Q8_0> {
    static constexpr int BE = 32, BB = Q8_0_BYTES, P = 1, VT = T_Q8_0;
};

// Weight bytes a lane holds for one task.
struct TaskData {
    uint4 a, b, c, s;
    uint32_t e;
};

template <int TYPE>
__device__ __forceinline__ void load_task(const uint8_t* __restrict__ row, int blk, int p, TaskData& t) {
    if constexpr (TYPE == T_Q4K) {
        const uint8_t* b = row + (size_t)blk * Q4K_BYTES;
        t.s = *(const uint4*)b;                 // d, dmin, scales[12]
        t.a = *(const uint4*)(b + 16 + 16 * p);  // qs[16p .. 16p+16)
    } else if constexpr (TYPE == T_Q6K) {
        const uint8_t* b = row + (size_t)blk * Q6K_BYTES;
        int h = p >> 1, lq = (p & 1) * 16;
        t.a = load16_a2(b + 64 * h + lq);
        t.b = load16_a2(b + 64 * h + 32 + lq);
        t.c = load16_a2(b + Q6K_QH + 32 * h + lq);
        t.s = load16_a2(b + Q6K_SC);
        t.e = *(const uint16_t*)(b + Q6K_D);
    } else {
        const uint8_t* b = row + (size_t)blk * Q8_0_BYTES;
        uintptr_t a = (uintptr_t)b;
        const uint32_t* q = (const uint32_t*)(a & ~(uintptr_t)3);
        t.a = *(const uint4*)q;
        t.b = *(const uint4*)(q + 4);
        t.e = q[8];
        t.c.x = (uint32_t)(a & 3u);  // 0 or 2
    }
}

// Byte i (0..3) of the 4-dword group as a variable index.
__device__ __forceinline__ uint32_t dw_sel(const uint4& v, uint32_t i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// A task's weights unpacked to int8 lanes and integer scales, once per row,
// shared by every activation row.
template <int TYPE>
struct WPrep;
template <>
struct WPrep<T_Q4K> {
    uint32_t lo[4], hi[4];
    int sc0, sc1, m0, m1;
    float d, dmin;
};
template <>
struct WPrep<T_Q6K> {
    uint32_t q[4][4];
    int sc[4];
    float d;
};
template <>
struct WPrep<T_Q8_0> {
    uint32_t w[8];
    float d;
};

template <int TYPE>
__device__ __forceinline__ void prep_task(const TaskData& t, int p, WPrep<TYPE>& w) {
    if constexpr (TYPE == T_Q4K) {
        w.d = f16_to_f32(t.s.x & 0xffffu);
        w.dmin = f16_to_f32(t.s.x >> 16);
        const int j = p >> 1;
        // get_scale_min_k4 (utils.rs:50-60) for sub-blocks 2j and 2j+1: the
        // eight 6-bit scales (and mins) assembled one byte each into a
        // 64-bit word, then one shift by 16j picks the pair.  j varies
        // across the wave, and a select on it is compiled into a branch.
        const uint64_t sc8 = (uint64_t)(t.s.y & 0x3F3F3F3Fu) |
                             ((uint64_t)((t.s.w & 0x0F0F0F0Fu) | ((t.s.y >> 2) & 0x30303030u)) << 32);
        const uint64_t m8 = (uint64_t)(t.s.z & 0x3F3F3F3Fu) |
                            ((uint64_t)(((t.s.w >> 4) & 0x0F0F0F0Fu) | ((t.s.z >> 2) & 0x30303030u)) << 32);
        const uint32_t scp = (uint32_t)(sc8 >> (16 * j)), mp = (uint32_t)(m8 >> (16 * j));
        w.sc0 = (int)(scp & 0xffu);
        w.sc1 = (int)((scp >> 8) & 0xffu);
        w.m0 = (int)(mp & 0xffu);
        w.m1 = (int)((mp >> 8) & 0xffu);
        const uint32_t A[4] = {t.a.x, t.a.y, t.a.z, t.a.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w.lo[i] = A[i] & 0x0F0F0F0Fu;
            w.hi[i] = (A[i] >> 4) & 0x0F0F0F0Fu;
        }
    } else if constexpr (TYPE == T_Q6K) {
        w.d = f16_to_f32(t.e);
        const int h = p >> 1, odd = p & 1;
        // q6 bytes of the 4 groups g (elements 128h + 32g + 16*odd + 0..15)
        const uint32_t A[4] = {t.a.x, t.a.y, t.a.z, t.a.w};
        const uint32_t B[4] = {t.b.x, t.b.y, t.b.z, t.b.w};
        const uint32_t C[4] = {t.c.x, t.c.y, t.c.z, t.c.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w.q[0][i] = (A[i] & 0x0F0F0F0Fu) | ((C[i] & 0x03030303u) << 4);
            w.q[1][i] = (B[i] & 0x0F0F0F0Fu) | (((C[i] >> 2) & 0x03030303u) << 4);
            w.q[2][i] = ((A[i] >> 4) & 0x0F0F0F0Fu) | (((C[i] >> 4) & 0x03030303u) << 4);
            w.q[3][i] = ((B[i] >> 4) & 0x0F0F0F0Fu) | (((C[i] >> 6) & 0x03030303u) << 4);
        }
        // scales[8h + 2g + odd]: dword 2h (g < 2) or 2h + 1, byte (2g + odd) & 3
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t wd = dw_sel(t.s, 2 * h + (g >> 1));
            w.sc[g] = (int)(int8_t)byte_of(wd, (2 * g + odd) & 3);
        }
    } else {
        const uint32_t s = t.c.x;
        w.d = f16_to_f32(s == 0 ? (t.a.x & 0xffffu) : (t.a.x >> 16));
        const uint32_t W[9] = {t.a.x, t.a.y, t.a.z, t.a.w, t.b.x, t.b.y, t.b.z, t.b.w, t.e};
#pragma unroll
        for (int i = 0; i < 8; i++) w.w[i] = s == 0 ? __builtin_amdgcn_alignbyte(W[i + 1], W[i], 2) : W[i + 1];
    }
}

}  // namespace lloom
