// gemm_i8.hip -- Q4_K prefill GEMM on int8 MFMA (v_mfma_i32_32x32x32_i8).
//
// y[m, n] = sum_sb dy[m,sb] * ( d[n,sb] * I1 - dmin[n,sb] * I2 ),
//   I1 = sum_j sc[n,j] * sum_{k in j} x8[m,k] q[n,k],   I2 = sum_j mn[n,j] * S_j[m]
// is k_quants' Q4_K x Q8_K dot (k_quants.rs:1540-1620) with I1 and I2 exact
// and the f32 combination once per superblock.
//
// Arithmetic.  sc * q reaches 945, past an int8 operand, so the weights enter
// as two int8 planes, sc = 8 * s1 + s0 with s0, s1 <= 7: each plane byte is
// at most 105, and one v_pk_mul_lo_u16 scales four packed nibble bytes with
// no carry between them.  Two MFMA chains (lo, hi) sum a superblock, I1 =
// 8 * hi + lo.  The min term is two v_mfma_f32_32x32x16_f16 a tile and
// superblock: the eight 32-element sums S_j reach |S_j| <= 4064, past the
// integers fp16 holds exactly (2048), so the activation side holds them as
// S_j = 64 S_hi + S_lo (S_hi = S >> 6 in [-64, 63], S_lo = S & 63), one
// MFMA on the eight 64 S_hi twice and one on the eight S_lo twice (both
// exact in fp16), the weight side -dmin * mn_j split
// into an fp16 pair hi + lo (dmin * mn_j has at most 17 significant bits, so
// the pair is exact while it stays below 65504; a wave whose columns hold a
// dmin >= 1024 scales every dmin of the superblock by the same power of two
// 2^-s first, and gives 2^s to dy and 2^-s to d).  The epilogue per output
// and superblock is four VALU instructions:
//     v = fma(float(8 hi + lo), d, Dmin);  out = fma(v, dy, out)
//
// Operand roles.  The weights are the MFMA's A (rows = weight columns n),
// the activations its B (columns = activation rows m), so a lane's sixteen
// results share one activation row (dy is one value a lane) and sixteen
// weight columns whose d the wave shares through LDS once a superblock:
//   A  lane l: plane bytes of weight column l % 32, k = 32j + 16 (l/32) + 0..15
//   B  lane l: x8 of activation row l % 32, the same k
//   D  lane l, reg v: [n = 8 (v/4) + 4 (l/32) + v % 4][m = l % 32]
// (an MFMA sums over k whatever order the hardware gives it, as long as A
// and B agree, which they do lane by lane).
//
// Tiling.  512 threads = 8 waves, two a SIMD; the workgroup computes 128
// activation rows x 256 weight columns, each wave 128 x 32: four 32 x 32
// tiles share every unpacked weight operand, so a wave unpacks each weight
// byte of its columns once.  A superblock of K is one LDS stage, two
// stages: the loads of superblock sb + 1 are in flight while sb computes.
// Every byte arrives by global_load_lds of 1 KB of contiguous memory (the
// load issue cost grows with the cache lines an instruction touches) from a
// scalar base plus a per-lane offset fixed for the whole K loop.  Each
// activation operand of a tile is refilled with the next tile's as soon as
// its MFMAs are issued, so only the first tile of a superblock waits on LDS.
#include "kq_common.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"
#include "kq_gemm.hpp"


namespace lloom {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128, BN = 256, WAVES = 8, THREADS = 64 * WAVES, MT = BM / 32, STAGES = 2;
// LDS stage:
//   A  [16 pieces][128 rows][16 B] x8, piece-major: eight lanes reading one
//      piece of eight rows touch 32 consecutive dwords (no bank conflict)
//   W  [256 rows][144 B] the raw Q4_K superblocks (a 36-dword stride: eight
//      rows reading one piece hit eight bank groups)
//   S  [128 rows][16] fp16 (64 S_hi[8], S_lo[8]), D [128] f32
// Every global_load_lds moves 1 KB of contiguous memory (few cache lines:
// the load issue is the DMA's cost): the activation prep writes x8 in the
// order the stage holds it, 64 rows at a time, and S and dy superblock-major.
constexpr int A_BYTES = BM * 256, W_BYTES = BN * 144, S_BYTES = BM * 32, D_BYTES = BM * 4;
constexpr int A_OFF = 0, W_OFF = A_BYTES, S_OFF = W_OFF + W_BYTES, D_OFF = S_OFF + S_BYTES;
constexpr int STAGE = D_OFF + D_BYTES;
constexpr int SCR_OFF = STAGES * STAGE;  // per wave: d of its 32 columns
constexpr int LDS = SCR_OFF + WAVES * 128;
constexpr int A_PER_WAVE = A_BYTES / 1024 / WAVES;          // 4
constexpr int W_CHUNKS = W_BYTES / 1024;                    // 36
constexpr int W_PER_WAVE = (37 + WAVES - 1) / WAVES;  // 5: 37 weight instructions (7 rows each)
static_assert(A_PER_WAVE == 4 && W_CHUNKS == 36 && LDS <= 160 * 1024, "staging layout");
static_assert(4096 * 7 + 512 * 3 < 65536, "immediate LDS offsets past the per-region lane bases");

// Each 16-bit half of q times f (both halves' products below 2^16).
__device__ __forceinline__ int pk_mul(uint32_t q, uint32_t f2) {
    return __builtin_bit_cast(int, __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, f2));
}
// Byte b of w (compile-time b) in both 16-bit halves.
__device__ __forceinline__ uint32_t byte_pair(uint32_t w, int b) {
    const uint32_t sel = 0x0c000c00u | (uint32_t)b | ((uint32_t)b << 16);
    return __builtin_amdgcn_perm(0u, w, sel);
}

}  // namespace

// Activation prep: Q8_K of every (row, superblock), bit-exact (the CPU arm's
// from_float, k_quants.rs:2400-2438), into
//   xq  int8 [mp/64][k/256][16 pieces][64 rows][16 B]  x8, piece p of a
//       superblock = its elements 16p .. 16p+15
//   s16 fp16 [k/256][mp][16]  64 S_hi_j then S_lo_j for S_j = bsums[2j] +
//       bsums[2j + 1] = 64 S_hi_j + S_lo_j, S_lo_j in [0, 63]
//   dyt f32  [k/256][mp]
// with rows m .. mp-1 zero (the GEMM reads whole 128-row tiles).
struct I8Ptrs {
    int8_t* xq;
    _Float16* s16;
    float* dyt;
    int64_t mp;
};
static int64_t i8_rows(int64_t m) { return (m + BM - 1) / BM * BM; }
static I8Ptrs i8_ptrs(void* base, int64_t m, int64_t k) {
    const int64_t mp = i8_rows(m);
    const size_t a = ((size_t)mp * k + 255) & ~(size_t)255;
    const size_t b = ((size_t)mp * (k / 32) * 4 + 255) & ~(size_t)255;
    I8Ptrs p;
    p.xq = (int8_t*)base;
    p.s16 = (_Float16*)((uint8_t*)base + a);
    p.dyt = (float*)((uint8_t*)base + a + b);
    p.mp = mp;
    return p;
}
size_t gemm_i8_workspace_bytes(int64_t m, int64_t k) {
    const int64_t mp = i8_rows(m);
    const size_t a = ((size_t)mp * k + 255) & ~(size_t)255;
    const size_t b = ((size_t)mp * (k / 32) * 4 + 255) & ~(size_t)255;
    return a + b + (size_t)(k / 256) * mp * sizeof(float) + 256;
}
bool gemm_i8_fits(int64_t n, int64_t k, int64_t m) {
    // 32-bit DMA offsets (the scalar bases carry the superblock and row group)
    return k % 256 == 0 && i8_rows(m) * k < ((int64_t)1 << 31) && n * (k / 256) * Q4K_BYTES < ((int64_t)1 << 31);
}

// Each wave quantizes NB superblocks of 4 rows (a 16-lane row of the wave
// per activation row; lane j of it holds piece j: 16 elements, 64 contiguous
// bytes of x, 16 bytes of x8 written where the GEMM's stage wants them).
template <int NB>
__global__ __launch_bounds__(256) void k_gemm_prep_i8(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                      _Float16* __restrict__ s16, float* __restrict__ dyt, int m,
                                                      int mp, int k) {
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int nsb = k >> 8, ngr = nsb / NB;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (4-row group, superblock group)
    if (wid >= (int64_t)(mp / 4) * ngr) return;
    const int mi = (int)(wid / ngr) * 4 + (lane >> 4), sb0 = NB * (int)(wid % ngr);
    const bool real = mi < m;
    const float* xr = x + (int64_t)min(mi, m - 1) * k + 16 * j;
    float xs[NB][16];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 v = *(const float4*)(xr + (sb0 + b) * 256 + 4 * c);
            xs[b][4 * c] = v.x;
            xs[b][4 * c + 1] = v.y;
            xs[b][4 * c + 2] = v.z;
            xs[b][4 * c + 3] = v.w;
        }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int sb = sb0 + b;
        float d;
        int bs;
        uint4 q = q8k_block_row16(xs[b], &d, &bs);
        if (!real) {  // rows past m: zeros
            q = make_uint4(0, 0, 0, 0);
            d = 0.0f;
            bs = 0;
        }
        *(uint4*)(xq + ((((int64_t)(mi >> 6) * nsb + sb) * 16 + j) * 64 + (mi & 63)) * 16) = q;
        const int S = bs + __shfl_xor(bs, 1, 64);  // pieces 2i and 2i + 1: S_i
        if ((j & 1) == 0) {
            _Float16* sr = s16 + ((int64_t)sb * mp + mi) * 16 + (j >> 1);
            sr[0] = (_Float16)(float)(64 * (S >> 6));  // a multiple of 64 below 2^12 in size: exact
            sr[8] = (_Float16)(float)(S & 63);
        }
        if (j == 0) dyt[(int64_t)sb * mp + mi] = d;
    }
}

__global__ __launch_bounds__(THREADS) void k_gemm_q4k_i8(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                         const _Float16* __restrict__ s16,
                                                         const float* __restrict__ dyt, float* __restrict__ Y, int m,
                                                         int mp, int n, int k, int epi) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c32 = lane & 31;
    int bm, bn;
    tile_of(mp / BM, (n + BN - 1) / BN, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;
    const int nsb = k >> 8;
    const uint32_t rowbytes = (uint32_t)nsb * Q4K_BYTES;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds0 = lds_addr(smem);

    // ---- per-lane DMA offsets, fixed for the K loop ----
    // Activations: instruction q = wave + 8 i moves piece q >> 1 of row
    // group q & 1 (64 rows, 1 KB contiguous in the prep's layout; q & 1 =
    // wave & 1).  Weights: instruction q moves rows 7q .. 7q+6 of the tile
    // (lane l: row 7q + l / 9, piece l % 9; lane 63 loads piece 0 of row
    // 7q + 7, the bytes instruction q + 1 writes there too), so one per-lane
    // offset serves every instruction; the last moves rows 252..255 (36
    // lanes).  In the last column tile rows past n reload row n - 1
    // (computed, never stored).  S (waves 4..7, 1 KB each) and dy (wave 6,
    // lanes 0..31, 512 B), contiguous.
    const uint32_t lane16 = 16u * (uint32_t)lane;
    const bool ragged_n = n0 + BN > n;  // uniform
    const uint32_t wlane = (uint32_t)(lane / 9) * rowbytes + 16u * (uint32_t)(lane % 9);
    const int8_t* xq_tile = xq + ((size_t)(m0 >> 6) + (size_t)(wv & 1)) * nsb * 16384;
    auto issue = [&](int sb, int stg) {
        const uint32_t st = lds0 + (uint32_t)stg * STAGE;
        const int8_t* ab = xq_tile + (size_t)sb * 16384;
#pragma unroll
        for (int i = 0; i < A_PER_WAVE; i++) {
            const int q = wv + WAVES * i;
            dma16s(ab + 1024u * (uint32_t)(q >> 1), lane16,
                   st + A_OFF + 2048u * (uint32_t)(q >> 1) + 1024u * (uint32_t)(q & 1));
        }
        const uint8_t* wb = W + (size_t)n0 * rowbytes + (uint32_t)sb * Q4K_BYTES;
#pragma unroll
        for (int i = 0; i < W_PER_WAVE; i++) {
            const int q = wv + WAVES * i;  // 0 .. 36
            if (q > 36) continue;
            if (q < 36 || lane < 36) {
                if (!ragged_n) {
                    dma16s(wb + (size_t)7 * q * rowbytes, wlane, st + W_OFF + 1008u * (uint32_t)q);
                } else {
                    // rows clamped to n - 1: the offset from the tile's first
                    // row (never negative, below 256 rows)
                    const uint32_t off = (uint32_t)(min(n0 + 7 * q + lane / 9, n - 1) - n0) * rowbytes +
                                         16u * (uint32_t)(lane % 9);
                    dma16s(wb, off, st + W_OFF + 1008u * (uint32_t)q);
                }
            }
        }
        if (wv >= 4)
            dma16s((const uint8_t*)s16 + ((size_t)sb * mp + m0 + 32 * (wv - 4)) * 32u, lane16,
                   st + S_OFF + 1024u * (uint32_t)(wv - 4));
        if (wv == 6 && lane < 32) dma16s((const uint8_t*)(dyt + (int64_t)sb * mp + m0), lane16, st + D_OFF);
    };
    auto wait_all = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
    };

    v16f out[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) out[t][v] = 0.0f;

    // per-lane LDS bases (plus a stage offset); the rest of an address is a constant
    const int wrow = 32 * wave + c32;  // the lane's weight column in the tile
    const int la = A_OFF + 2048 * h + 16 * c32;
    const int lw = W_OFF + 144 * wrow + 16 + 16 * h, lh = W_OFF + 144 * wrow;
    const int ls = S_OFF + 32 * c32, ld = D_OFF + 4 * c32;
    float* const scr = (float*)(smem + SCR_OFF) + 32 * wave;

    issue(0, 0);
    wait_all();

    for (int sb = 0; sb < nsb; sb++) {
        const int so = (sb % STAGES) * STAGE;
        const int sa = la + so, sw = lw + so, sh = lh + so, ss = ls + so, sd = ld + so;
        // 1. this superblock's weight bytes, into registers; the columns' d
        //    to the lanes whose outputs use them (through LDS, within the wave)
        const uint4 hdr = *(const uint4*)(smem + sh);
        uint4 raw[4];
#pragma unroll
        for (int c = 0; c < 4; c++) raw[c] = *(const uint4*)(smem + sw + 32 * c);
        const float dmin = f16_to_f32(hdr.x >> 16);
        scr[c32] = f16_to_f32(hdr.x & 0xffffu);
        __builtin_amdgcn_wave_barrier();
        v16f dv;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 q = *(const float4*)(scr + 8 * g + 4 * h);
            dv[4 * g] = q.x;
            dv[4 * g + 1] = q.y;
            dv[4 * g + 2] = q.z;
            dv[4 * g + 3] = q.w;
        }
        // 2. queue superblock sb + 1 into the other stage
        __builtin_amdgcn_sched_barrier(0);
        if (sb + 1 < nsb) issue(sb + 1, (sb + 1) % STAGES);
        __builtin_amdgcn_sched_barrier(0);

        // 3. the weight operands: planes of the eight sub-blocks and the min
        //    term's.  s = 0 unless a column of the wave has dmin >= 1024: then
        //    dmin 2^-s < 1024 enters the fp16 pair, 2^-s goes to d and 2^s to
        //    dy (exact powers of two)
        float dys = 1.0f;
        float dmw = dmin;
        if (__ballot(dmin >= 1024.0f) != 0) {  // wave-uniform, rare
            const int e = (int)((__builtin_bit_cast(uint32_t, wave_max(dmin)) >> 23) & 0xffu) - 127 - 9;
            const float sdn = __builtin_bit_cast(float, (uint32_t)(127 - e) << 23);
            dys = __builtin_bit_cast(float, (uint32_t)(127 + e) << 23);
            dmw = dmin * sdn;
#pragma unroll
            for (int v = 0; v < 16; v++) dv[v] *= sdn;
        }
        // scales (get_scale_min_k4, k_quants utils.rs:50-60, four at a time)
        const uint32_t sc0 = hdr.y & 0x3F3F3F3Fu;
        const uint32_t sc1 = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
        const uint32_t mn0 = hdr.z & 0x3F3F3F3Fu;
        const uint32_t mn1 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
        const uint32_t s0a = sc0 & 0x07070707u, s0b = sc1 & 0x07070707u;
        const uint32_t s1a = (sc0 >> 3) & 0x07070707u, s1b = (sc1 >> 3) & 0x07070707u;
        v4i plo[8], phi[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint4 r = raw[j >> 1];
            const int shf = (j & 1) * 4;
            const uint32_t q0 = (r.x >> shf) & 0x0F0F0F0Fu, q1 = (r.y >> shf) & 0x0F0F0F0Fu,
                           q2 = (r.z >> shf) & 0x0F0F0F0Fu, q3 = (r.w >> shf) & 0x0F0F0F0Fu;
            const uint32_t f0 = byte_pair(j < 4 ? s0a : s0b, j & 3), f1 = byte_pair(j < 4 ? s1a : s1b, j & 3);
            plo[j] = v4i{pk_mul(q0, f0), pk_mul(q1, f0), pk_mul(q2, f0), pk_mul(q3, f0)};
            phi[j] = v4i{pk_mul(q0, f1), pk_mul(q1, f1), pk_mul(q2, f1), pk_mul(q3, f1)};
        }
        // min-term weight operand, k = 8h .. 8h+7: half 0 the fp16 hi of
        // -dmin' mn_j, half 1 the lo
        v8h amin;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v = dmw * (float)byte_of(j < 4 ? mn0 : mn1, j & 3);  // exact in f32
            const _Float16 vh = (_Float16)v;
            const _Float16 vl = (_Float16)(v - (float)vh);
            amin[j] = h ? -vl : -vh;
        }

        // 4. the four 32 x 32 tiles: sixteen int8 MFMAs (eight sub-blocks,
        //    two planes), each activation operand refilled with the next
        //    tile's as soon as its MFMAs are issued; then the min MFMA and the
        //    epilogue (the other wave of the SIMD runs its MFMAs meanwhile)
        v4i bx[8];
#pragma unroll
        for (int j = 0; j < 8; j++) bx[j] = *(const v4i*)(smem + sa + 4096 * j);
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const v8h svh = *(const v8h*)(smem + ss + 1024 * t);
            const v8h svl = *(const v8h*)(smem + ss + 1024 * t + 16);
            const float dy = *(const float*)(smem + sd + 128 * t) * dys;
            v16i lo, hi;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const v16i z = {};
                lo = __builtin_amdgcn_mfma_i32_32x32x32_i8(plo[j], bx[j], j ? lo : z, 0, 0, 0);
                hi = __builtin_amdgcn_mfma_i32_32x32x32_i8(phi[j], bx[j], j ? hi : z, 0, 0, 0);
                if (t + 1 < MT) bx[j] = *(const v4i*)(smem + sa + (4096 * j + 512 * (t + 1)));
            }
            const v16f zf = {};
            const v16f dm = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                amin, svl, __builtin_amdgcn_mfma_f32_32x32x16_f16(amin, svh, zf, 0, 0, 0), 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float f = (float)(hi[v] * 8 + lo[v]);
                out[t][v] = __builtin_fmaf(__builtin_fmaf(f, dv[v], dm[v]), dy, out[t][v]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        // 5. superblock sb + 1 has landed (this wave's share) and is visible to all
        wait_all();
    }

    // store: lane row m0 + 32 t + c32, columns n0 + 32 wave + 8 g + 4 h + 0..3
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int row = m0 + 32 * t + c32;
        if (row >= m) continue;
        float* yr = Y + (int64_t)row * n;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int col = n0 + 32 * wave + 8 * g + 4 * h;
            if (epi == EPI_STORE && col + 3 < n) {
                *(float4*)(yr + col) = make_float4(out[t][4 * g], out[t][4 * g + 1], out[t][4 * g + 2], out[t][4 * g + 3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (col + r < n) store_epi_slow(yr + col + r, out[t][4 * g + r], epi);
            }
        }
    }
}

hipError_t launch_gemm_i8(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* ws,
                          int epi, hipStream_t s) {
    if (hipError_t e = set_lds_limit((const void*)k_gemm_q4k_i8, LDS)) return e;
    const I8Ptrs p = i8_ptrs(ws, m, k);
    const int64_t nsb = k / 256;
    const int64_t waves2 = p.mp / 4 * (nsb / 2), waves1 = p.mp / 4 * nsb;
    if (nsb % 2 == 0)
        hipLaunchKernelGGL(k_gemm_prep_i8<2>, dim3((unsigned)((waves2 + 3) / 4)), dim3(256), 0, s, x, p.xq, p.s16,
                           p.dyt, (int)m, (int)p.mp, (int)k);
    else
        hipLaunchKernelGGL(k_gemm_prep_i8<1>, dim3((unsigned)((waves1 + 3) / 4)), dim3(256), 0, s, x, p.xq, p.s16,
                           p.dyt, (int)m, (int)p.mp, (int)k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const unsigned grid = (unsigned)((p.mp / BM) * ((n + BN - 1) / BN));
hipLaunchKernelGGL(k_gemm_q4k_i8, dim3(grid), dim3(THREADS), LDS, s, (const uint8_t*)w, p.xq, p.s16, p.dyt, y, (int)m,
                       (int)p.mp, (int)n, (int)k, epi);
    return hipGetLastError();
}

}  // namespace lloom
