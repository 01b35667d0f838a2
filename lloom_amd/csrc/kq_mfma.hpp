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

// q6 (0..63) per byte -> q6 - 32 as int8: t = q6 ^ 32 is q6 - 32 in 6-bit
// two's complement; copying bit 5 into bits 6 and 7 (0x20 * 6 = 0xC0, no
// carry between bytes) sign-extends it to 8 bits.
__device__ __forceinline__ uint32_t q6_to_i8(uint32_t q6) {
    const uint32_t t = q6 ^ 0x20202020u;
    return t | ((t & 0x20202020u) * 6u);
}

// One superblock of one 16-row tile: returns the f32 contributions of the
// lane's four outputs.
template <int TYPE>
__device__ __forceinline__ void mf_compute(const MfW<TYPE>& w, const long (&a)[8], const float4& dy, int g,
                                           float (&out)[4]) {
    const v4i zero = {0, 0, 0, 0};
    if constexpr (TYPE == T_Q4K) {
        const float d = f16_to_f32(w.hdr.x & 0xffffu), dmin = f16_to_f32(w.hdr.x >> 16);
        v4i accs = {0, 0, 0, 0}, accm = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            if (j < 4) {
                sc = byte_of(w.hdr.y, j) & 63;
                mn = byte_of(w.hdr.z, j) & 63;
            } else {
                sc = (byte_of(w.hdr.w, j - 4) & 0xF) | ((byte_of(w.hdr.y, j - 4) >> 6) << 4);
                mn = (byte_of(w.hdr.w, j - 4) >> 4) | ((byte_of(w.hdr.z, j - 4) >> 6) << 4);
            }
            const int c = j >> 1, sh = (j & 1) * 4;
            const uint32_t lo = (w.q[c].x >> sh) & 0x0F0F0F0Fu, hi = (w.q[c].y >> sh) & 0x0F0F0F0Fu;
            const long bw = (long)(((uint64_t)hi << 32) | lo);
            const v4i dj = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], bw, zero, 0, 0, 0);
            const uint32_t mrep = (uint32_t)mn * 0x01010101u;
            const long bm = (long)(((uint64_t)mrep << 32) | mrep);
            accm = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], bm, accm, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; t++) accs[t] += __mul24(sc, dj[t]);
        }
        out[0] += dy.x * ((float)accs[0] * d - (float)accm[0] * dmin);
        out[1] += dy.y * ((float)accs[1] * d - (float)accm[1] * dmin);
        out[2] += dy.z * ((float)accs[2] * d - (float)accm[2] * dmin);
        out[3] += dy.w * ((float)accs[3] * d - (float)accm[3] * dmin);
    } else {
        const float d = f16_to_f32(w.d);
        const bool lo_half = g < 2;  // this lane's k range is sub-block 2j, else 2j + 1
        v4i accs = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int h = j >> 2, gq = j & 3, c = 2 * h + (gq & 1);
            const uint32_t nx = gq < 2 ? (w.ql[c].x & 0x0F0F0F0Fu) : ((w.ql[c].x >> 4) & 0x0F0F0F0Fu);
            const uint32_t ny = gq < 2 ? (w.ql[c].y & 0x0F0F0F0Fu) : ((w.ql[c].y >> 4) & 0x0F0F0F0Fu);
            const uint32_t hx = (w.qh[h].x >> (2 * gq)) & 0x03030303u, hy = (w.qh[h].y >> (2 * gq)) & 0x03030303u;
            const uint32_t vx = q6_to_i8(nx | (hx << 4)), vy = q6_to_i8(ny | (hy << 4));
            const long bw = (long)(((uint64_t)vy << 32) | vx);
            const v4i da = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], lo_half ? bw : 0l, zero, 0, 0, 0);
            const v4i db = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], lo_half ? 0l : bw, zero, 0, 0, 0);
            // scales[2j], scales[2j + 1]: dword j / 2, bytes 2(j & 1) and 2(j & 1) + 1
            const uint32_t sw = j < 2 ? w.sc.x : j < 4 ? w.sc.y : j < 6 ? w.sc.z : w.sc.w;
            const int sa = (int)(int8_t)byte_of(sw, 2 * (j & 1)), sb = (int)(int8_t)byte_of(sw, 2 * (j & 1) + 1);
#pragma unroll
            for (int t = 0; t < 4; t++) accs[t] += __mul24(sa, da[t]) + __mul24(sb, db[t]);
        }
        out[0] += (d * dy.x) * (float)accs[0];
        out[1] += (d * dy.y) * (float)accs[1];
        out[2] += (d * dy.z) * (float)accs[2];
        out[3] += (d * dy.w) * (float)accs[3];
    }
}

// mf_compute's Q4_K arithmetic with the min term on two MFMAs instead of
// eight: bsum_j = sum of the 32 quantized x of sub-block j = 64 hi_j + lo_j
// (both int8, from k_quantize_split_q8k's bsp); the activation operand `ab`
// holds lo_0..7 in lane group 0 and hi_0..7 in group 1 (zero in 2, 3), the
// weight operand the eight 6-bit mins in group 0 (for the lo sums) or group
// 1 (for the hi sums), so sum_j m_j bsum_j = D(lo) + 64 D(hi), exact.  The
// scales and mins are unpacked as whole dwords (scales 0-3 are bytes of
// hdr.y & 0x3f..., 4-7 are the low nibbles of hdr.w with hdr.y's top bits).
// Every integer sum equals mf_compute's, so do the outputs.
__device__ __forceinline__ void mf_compute_q4k_b(const MfW<T_Q4K>& w, const long (&a)[8], long ab, const float4& dy,
                                                 int g, float (&out)[4]) {
    const v4i zero = {0, 0, 0, 0};
    const float d = f16_to_f32(w.hdr.x & 0xffffu), dmin = f16_to_f32(w.hdr.x >> 16);
    const uint32_t sc_lo = w.hdr.y & 0x3F3F3F3Fu, sc_hi = (w.hdr.w & 0x0F0F0F0Fu) | ((w.hdr.y >> 2) & 0x30303030u);
    const uint32_t mn_lo = w.hdr.z & 0x3F3F3F3Fu,
                   mn_hi = ((w.hdr.w >> 4) & 0x0F0F0F0Fu) | ((w.hdr.z >> 2) & 0x30303030u);
    const long mins = (long)(((uint64_t)mn_hi << 32) | mn_lo);
    v4i accs = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int sc = (int)byte_of(j < 4 ? sc_lo : sc_hi, j & 3);
        const int c = j >> 1, sh = (j & 1) * 4;
        const uint32_t lo = (w.q[c].x >> sh) & 0x0F0F0F0Fu, hi = (w.q[c].y >> sh) & 0x0F0F0F0Fu;
        const long bw = (long)(((uint64_t)hi << 32) | lo);
        const v4i dj = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], bw, zero, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 4; t++) accs[t] += __mul24(sc, dj[t]);
    }
    v4i mh = __builtin_amdgcn_mfma_i32_16x16x32_i8(ab, g == 1 ? mins : 0l, zero, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < 4; t++) mh[t] <<= 6;
    const v4i accm = __builtin_amdgcn_mfma_i32_16x16x32_i8(ab, g == 0 ? mins : 0l, mh, 0, 0, 0);
    out[0] += dy.x * ((float)accs[0] * d - (float)accm[0] * dmin);
    out[1] += dy.y * ((float)accs[1] * d - (float)accm[1] * dmin);
    out[2] += dy.z * ((float)accs[2] * d - (float)accm[2] * dmin);
    out[3] += dy.w * ((float)accs[3] * d - (float)accm[3] * dmin);
}

}  // namespace lloom
