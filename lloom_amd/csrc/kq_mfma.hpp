// kq_mfma.hpp -- weight-operand loads shared by the MFMA kernels: a Q4_K /
// Q6_K superblock row read contiguously (32 qs bytes a lane) and handed to
// the 16x16 MFMA operand layout (lane (g, row) owns the 8-byte piece g of
// every 32-byte chunk) through a wave-private LDS transpose.
#pragma once

#include "kq_common.hpp"
#include "kq_tasks.hpp"

namespace lloom {

typedef int v4i __attribute__((ext_vector_type(4)));

// 8 bytes at a 2-byte-aligned address (Q6_K blocks are 210 bytes).
__device__ __forceinline__ uint2 load8_a2(const uint8_t* p) {
    uintptr_t a = (uintptr_t)p;
    const uint32_t* q = (const uint32_t*)(a & ~(uintptr_t)3);
    const uint32_t s = (uint32_t)(a & 3u);
    const uint32_t v0 = q[0], v1 = q[1], v2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(v1, v0, s), __builtin_amdgcn_alignbyte(v2, v1, s));
}

template <int TYPE>
struct MfW;
template <>
struct MfW<T_Q4K> {
    uint4 hdr;
    uint2 q[4];
};
template <>
struct MfW<T_Q6K> {
    uint2 ql[4], qh[2];
    uint4 sc;
    uint32_t d;
};

template <int TYPE>
__device__ __forceinline__ void mf_load(const uint8_t* __restrict__ b, int g, MfW<TYPE>& w) {
    if constexpr (TYPE == T_Q4K) {
        w.hdr = *(const uint4*)b;
#pragma unroll
        for (int c = 0; c < 4; c++) w.q[c] = *(const uint2*)(b + 16 + 32 * c + 8 * g);
    } else {
        // ql byte 64h + 32(gq & 1) + 8g + t holds chunk j = 4h + gq (low
        // nibble for gq < 2), qh byte 32h + 8g + t its two high bits
#pragma unroll
        for (int c = 0; c < 4; c++) w.ql[c] = load8_a2(b + 32 * c + 8 * g);
#pragma unroll
        for (int h = 0; h < 2; h++) w.qh[h] = load8_a2(b + Q6K_QH + 32 * h + 8 * g);
        w.sc = load16_a2(b + Q6K_SC);
        w.d = *(const uint16_t*)(b + Q6K_D);
    }
}

// Load format of a superblock.  Q4_K: each lane reads 32 contiguous qs bytes
// of its row (chunk g: bytes 32g .. 32g+31) and the header, so the wave's
// loads cover each row's 128 qs bytes contiguously; mf_unpack then hands
// lane (g, row) the 8-byte piece g of every chunk c through a wave-private
// LDS tile (a 4 x 4 transpose among the four lanes of a row).  Loading the
// operand layout directly (four 8-byte pieces 32 bytes apart per lane)
// made each load instruction touch 16 rows x 32 bytes and cost ~1.5 us of
// a 6 us call.  Q6_K the same way: 32 contiguous ql bytes and 16 qh bytes a
// lane (2-byte-aligned blocks: dword loads and a byte realignment).
template <int TYPE>
struct MfL;
template <>
struct MfL<T_Q4K> {
    uint4 hdr, a, b;
};
template <>
struct MfL<T_Q6K> {
    uint4 a, b, h, sc;
    uint32_t d;
};
// LDS bytes per row of the transpose tile: the qs (Q4_K 128, Q6_K 128 ql +
// 64 qh) plus a 16-byte pad
template <int TYPE>
struct MfRs {
    static constexpr int V = TYPE == T_Q4K ? 144 : 208;
};

// 32 bytes at a 2-byte-aligned address: nine dword loads from the 4-byte
// floor and a byte realignment.
__device__ __forceinline__ void load32_a2(const uint8_t* p, uint4& r0, uint4& r1) {
    uintptr_t a = (uintptr_t)p;
    const uint32_t* q = (const uint32_t*)(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3u);
    const uint4 v0 = *(const uint4*)q, v1 = *(const uint4*)(q + 4);
    const uint32_t v8 = q[8];
    r0.x = __builtin_amdgcn_alignbyte(v0.y, v0.x, sh);
    r0.y = __builtin_amdgcn_alignbyte(v0.z, v0.y, sh);
    r0.z = __builtin_amdgcn_alignbyte(v0.w, v0.z, sh);
    r0.w = __builtin_amdgcn_alignbyte(v1.x, v0.w, sh);
    r1.x = __builtin_amdgcn_alignbyte(v1.y, v1.x, sh);
    r1.y = __builtin_amdgcn_alignbyte(v1.z, v1.y, sh);
    r1.z = __builtin_amdgcn_alignbyte(v1.w, v1.z, sh);
    r1.w = __builtin_amdgcn_alignbyte(v8, v1.w, sh);
}

template <int TYPE>
__device__ __forceinline__ void mf_load_l(const uint8_t* __restrict__ b, int g, MfL<TYPE>& l) {
    if constexpr (TYPE == T_Q4K) {
        l.hdr = *(const uint4*)b;
        l.a = *(const uint4*)(b + 16 + 32 * g);
        l.b = *(const uint4*)(b + 32 + 32 * g);
    } else {
        load32_a2(b + 32 * g, l.a, l.b);
        l.h = load16_a2(b + Q6K_QH + 16 * g);
        l.sc = load16_a2(b + Q6K_SC);
        l.d = *(const uint16_t*)(b + Q6K_D);
    }
}

// tile: this wave's [16][MfRs] bytes of LDS for this row tile.
template <int TYPE>
__device__ __forceinline__ void mf_unpack(const MfL<TYPE>& l, uint8_t* tile, int g, int c16, MfW<TYPE>& w) {
    uint8_t* row = tile + c16 * MfRs<TYPE>::V;
    if constexpr (TYPE == T_Q4K) {
        *(uint4*)(row + 32 * g) = l.a;
        *(uint4*)(row + 32 * g + 16) = l.b;
        // the wave's LDS operations complete in order; this also keeps the
        // compiler from moving the reads above the writes
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int c = 0; c < 4; c++) w.q[c] = *(const uint2*)(row + 32 * c + 8 * g);
        w.hdr = l.hdr;
    } else {
        *(uint4*)(row + 32 * g) = l.a;
        *(uint4*)(row + 32 * g + 16) = l.b;
        *(uint4*)(row + 128 + 16 * g) = l.h;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int c = 0; c < 4; c++) w.ql[c] = *(const uint2*)(row + 32 * c + 8 * g);
#pragma unroll
        for (int hh = 0; hh < 2; hh++) w.qh[hh] = *(const uint2*)(row + 128 + 32 * hh + 8 * g);
        w.sc = l.sc;
        w.d = l.d;
    }
}


}  // namespace lloom
