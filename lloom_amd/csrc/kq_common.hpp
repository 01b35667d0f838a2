// kq_common.hpp -- block layouts and device helpers shared by the gfx950
// kernels of the quantized-matmul path.
//
// Block layouts are GGUF's, as lloom-tensor declares them
// (lloom-tensor/src/quantized/k_quants.rs:154-159, 216-223, 254-261,
// 264-270): the kernels read the packed bytes exactly as a GGUF file stores
// them, so QStorage::from_data is a plain upload.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lloom {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;

constexpr int T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4K = 12, T_Q6K = 14, T_Q8K = 15;

constexpr int Q8_0_BYTES = 34;   // f16 d, i8 qs[32]
constexpr int Q4K_BYTES = 144;   // f16 d, f16 dmin, u8 scales[12], u8 qs[128]
constexpr int Q6K_BYTES = 210;   // u8 ql[128], u8 qh[64], i8 scales[16], f16 d
constexpr int Q8K_BYTES = 292;   // f32 d, i8 qs[256], i16 bsums[16]

// Offsets inside a Q6K block.
constexpr int Q6K_QH = 128, Q6K_SC = 192, Q6K_D = 208;
// Offsets inside a Q8K block.
constexpr int Q8K_QS = 4, Q8K_BS = 260;

// Tail pad after a weight buffer: realigning loads read at most 3 bytes
// past a block, the fused kernels never more than one 16-byte vector.
constexpr size_t WEIGHT_TAIL_PAD = 512;

__host__ __device__ inline int block_elems(int t) {
    return t == T_Q8_0 ? QK8_0 : (t == T_Q4K || t == T_Q6K || t == T_Q8K) ? QK_K : 0;
}
__host__ __device__ inline int block_bytes(int t) {
    return t == T_Q8_0 ? Q8_0_BYTES
         : t == T_Q4K  ? Q4K_BYTES
         : t == T_Q6K  ? Q6K_BYTES
         : t == T_Q8K  ? Q8K_BYTES
                       : 0;
}

#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC__)

// ------------------------------------------------------------ f16 bits --
// f16 -> f32 is exact; f32 -> f16 is IEEE round-to-nearest-even, which is
// what half::f16::from_f32 (F16C on x86) does.
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    // The barrier keeps the f32 value: without it the compiler folds a
    // preceding multiply into v_fma_mix (one rounding, -0 turned into +0).
    asm volatile("" : "+v"(f));
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

// ------------------------------------------------- Rust cast semantics --
// f32::round is half away from zero (llvm.round, not rint).
__device__ __forceinline__ float round_away(float v) { return __builtin_roundf(v); }
// `f32 as i32`: saturating, NaN -> 0 -- exactly what v_cvt_i32_f32 does
// (out-of-range inputs clamp to the int32 limits, NaN converts to 0).  The
// conversion is written as the instruction itself: a C cast of such a value
// is undefined, and the guards the compiler adds for it become branches.
__device__ __forceinline__ int32_t sat_i32(float v) {
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}
// `f32 as i8`: saturating, NaN -> 0.  Truncating to int32 first and then
// clamping gives the same value as clamping the real number first.
__device__ __forceinline__ int32_t sat_i8(float v) {
    return min(max(sat_i32(v), -128), 127);
}
// `v.round() as i32` in three instructions: add the largest float below
// one half, with v's sign, and convert (v_cvt_i32_f32 truncates).  Checked
// against roundf over every non-NaN f32: the one case the plain +0.5 trick
// gets wrong (0.49999997 -> 1) cannot occur, because the addend is itself
// below one half and a sum that lands halfway rounds to the even neighbour.
// The sum must stay a separate rounding (no fma with a preceding product):
// contraction is off here and in every caller.
__device__ __forceinline__ int32_t nearest_int(float v) {
#pragma clang fp contract(off)
    const float h = __builtin_copysignf(0x1.fffffep-2f, v);
    return sat_i32(v + h);
}
__device__ __forceinline__ int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

// ------------------------------------------------------------- loads --
__device__ __forceinline__ uint32_t byte_of(uint32_t w, uint32_t i) { return (w >> (8u * i)) & 0xffu; }

// 16 bytes starting at a 2-byte-aligned address: five dword loads from the
// 4-byte floor and a byte realignment (v_alignbyte_b32).  GGUF's 34- and
// 210-byte blocks put every other block at an address = 2 (mod 4).
__device__ __forceinline__ uint4 load16_a2(const uint8_t* p) {
    uintptr_t a = (uintptr_t)p;
    const uint32_t* q = (const uint32_t*)(a & ~(uintptr_t)3);
    uint32_t s = (uint32_t)(a & 3u);
    uint4 v0 = *(const uint4*)q;  // 4-byte aligned dwordx4
    uint32_t v4 = q[4];
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(v0.y, v0.x, s);
    r.y = __builtin_amdgcn_alignbyte(v0.z, v0.y, s);
    r.z = __builtin_amdgcn_alignbyte(v0.w, v0.z, s);
    r.w = __builtin_amdgcn_alignbyte(v4, v0.w, s);
    return r;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---------------------------------------------- cross-lane exchanges --
// DPP and permlane moves (pure VALU, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
constexpr int DPP_XOR1 = 0xb1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4e;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <-> 7-i within 8
constexpr int DPP_ROW_MIRROR = 0x140;   // lane i <-> 15-i within 16

// The value held by the partner 16-lane row (rows 0<->1, 2<->3) and by
// the partner 32-lane half, via v_permlane16_swap / v_permlane32_swap of a
// register with itself.  Selecting by lane parity gives the partner both
// when the compiler keeps the two operands in separate registers (the pair
// then holds even rows in .x and odd rows in .y) and when it gives both one
// register (then both results hold the rows swapped).
__device__ __forceinline__ float partner16(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                              false, false);
    return __builtin_bit_cast(float, ((__lane_id() >> 4) & 1) ? r[0] : r[1]);
}
__device__ __forceinline__ float partner32(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                              false, false);
    return __builtin_bit_cast(float, (__lane_id() >> 5) ? r[0] : r[1]);
}

// Sum over the 16 lanes of each row, the result in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<DPP_XOR1>(v);
    v += dpp<DPP_XOR2>(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    v += dpp<DPP_ROW_MIRROR>(v);
    return v;
}
// V <= 8 independent full-wave sums in one butterfly: the xor-32, xor-16
// and xor-8 exchanges each merge two values into one (a lane sends the
// value its partner keeps and adds what it receives), then one value per
// lane goes through the 8-lane sum.  Item i ends up in the 8 lanes l with
// 4 * ((l >> 3) & 1) + 2 * ((l >> 4) & 1) + (l >> 5) == i; items past V
// read as 0.  (The exchanges a value takes do not depend on V, so an item's
// sum is the same whatever V is.)
constexpr int DPP_ROW_ROR8 = 0x128;  // lane i <- lane i ^ 8 within 16
template <int V>
__device__ __forceinline__ float wave_sum_items(const float (&v)[V]) {
    static_assert(V >= 1 && V <= 8, "wave_sum_items merges at most eight sums");
    const bool up32 = __lane_id() >= 32, up16 = (__lane_id() >> 4) & 1, up8 = (__lane_id() >> 3) & 1;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int p = 0; p < 4; p++) {
        if (2 * p < V) {
            const float x = v[2 * p], y = 2 * p + 1 < V ? v[2 * p + 1] : 0.0f;
            a[p] = (up32 ? y : x) + partner32(up32 ? x : y);
        }
    }
    float b[2] = {0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < 2; q++) {
        if (4 * q < V) b[q] = (up16 ? a[2 * q + 1] : a[2 * q]) + partner16(up16 ? a[2 * q] : a[2 * q + 1]);
    }
    float c = b[0];
    if constexpr (V > 4) c = (up8 ? b[1] : b[0]) + dpp<DPP_ROW_ROR8>(up8 ? b[0] : b[1]);
    else c += dpp<DPP_ROW_ROR8>(c);
    c += dpp<DPP_XOR1>(c);
    c += dpp<DPP_XOR2>(c);
    return c + dpp<DPP_HALF_MIRROR>(c);
}
__device__ __forceinline__ int wave_sum_item_of_lane() {
    const int l = __lane_id();
    return 4 * ((l >> 3) & 1) + 2 * ((l >> 4) & 1) + (l >> 5);
}
// Full-wave (wave64) sum, the result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    v += partner16(v);
    return v + partner32(v);
}
// Full-wave max (NaN-ignoring, as fmaxf), the result in every lane.
// The quantized matmul's store epilogues (QMatMul::forward_silu /
// forward_mul_into, mod.rs:2102-2156; the Metal store types of
// kernels/metal_src/quantized_store.metal): the plain store, silu(v) =
// v / (1 + exp(-v)), and y = y * v into the buffer's own value (the SwiGLU's
// up projection multiplied into silu(gate)).
constexpr int EPI_STORE = 0, EPI_SILU = 1, EPI_MUL_INTO = 2;
__device__ __forceinline__ void store_epi(float* p, float v, int epi) {
    if (epi == EPI_SILU) v = v / (1.0f + expf(-v));
    else if (epi == EPI_MUL_INTO) v = *p * v;
    *p = v;
}
// The same, out of line: for kernels that store many values per lane, so
// the SiLU's code is not unrolled into every store.
__device__ __noinline__ void store_epi_slow(float* p, float v, int epi);
__device__ __noinline__ inline void store_epi_slow(float* p, float v, int epi) { store_epi(p, v, epi); }

__device__ __forceinline__ float wave_max(float v) {
    v = __builtin_fmaxf(v, dpp<DPP_XOR1>(v));
    v = __builtin_fmaxf(v, dpp<DPP_XOR2>(v));
    v = __builtin_fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    v = __builtin_fmaxf(v, dpp<DPP_ROW_MIRROR>(v));
    v = __builtin_fmaxf(v, partner16(v));
    return __builtin_fmaxf(v, partner32(v));
}

#endif

}  // namespace lloom
