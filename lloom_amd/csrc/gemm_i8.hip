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
// 8 * hi + lo.  The min term is one v_mfma_f32_32x32x16_f16 a tile and
// superblock: the activation side holds the eight 32-element sums S_j
// (|S_j| <= 4064, exact in fp16) twice, the weight side -dmin * mn_j split
// into an fp16 pair hi + lo (dmin * mn_j has at most 17 significant bits, so
// the pair is exact while it stays below 65504; a wave whose columns hold a
// dmin >= 1024 takes the operand -mn_j and scales by dmin in f32 instead).
// The epilogue per output and superblock is four VALU instructions:
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
// activation rows x 256 weight columns, each wave 128 x 32: four m tiles
// share every unpacked weight operand, so a wave unpacks each weight byte of
// its columns once.  A superblock of K is one LDS stage (activations 128 x
// 256 B, swizzled so eight rows reading one 16-byte piece hit eight bank
// groups; raw Q4_K rows 256 x 144 B; S [128][8] fp16; dy [128] f32), two
// stages: the loads of superblock sb + 1 are in flight while sb computes.
// Every byte arrives by global_load_lds from a scalar base plus per-lane
// offsets fixed for the whole K loop.
#include "kq_common.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"
#include "kq_gemm.hpp"

#include <cstdlib>
#include <type_traits>

namespace lloom {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128, BN = 256, WAVES = 8, THREADS = 64 * WAVES, MT16 = BM / 16;
// LDS, piece-major: a 16-byte piece of every row of a tile side by side, so
// one global_load_lds (64 lanes x 16 B contiguous) moves one piece of 64
// rows, eight lanes reading one piece of eight rows touch 32 consecutive
// dwords (no bank conflict), and every read address is a per-lane base
// plus a compile-time offset and a stage base.
//   A  [16 pieces][128 rows][16 B] x8
//   W  [9 pieces][256 rows][16 B]  pieces 0..7 = the qs bytes 16p .. 16p+15,
//                                  piece 8 = the 16-byte header (d, dmin, scales)
//   S  [128 rows][8] fp16, D [128] f32
constexpr int A_BYTES = BM * 256, W_BYTES = BN * 144, S_BYTES = BM * 16, D_BYTES = BM * 4;
constexpr int A_OFF = 0, W_OFF = 2 * A_BYTES, S_OFF = W_OFF + 2 * W_BYTES, D_OFF = S_OFF + 2 * S_BYTES;
constexpr int SCR_OFF = D_OFF + 2 * D_BYTES;  // per wave: d of its 32 columns
constexpr int LDS = SCR_OFF + WAVES * 128;
constexpr int A_PER_WAVE = A_BYTES / 1024 / WAVES;          // 4
constexpr int W_CHUNKS = W_BYTES / 1024;                    // 36
constexpr int W_PER_WAVE = (W_CHUNKS + WAVES - 1) / WAVES;  // 5 (waves 4..7: 4)
static_assert(A_PER_WAVE == 4 && W_CHUNKS == 36 && LDS <= 160 * 1024, "staging layout");
static_assert(A_BYTES + 7 * 4096 + 3 * 512 < 65536 && W_BYTES + 6 * 4096 < 65536, "immediate LDS offsets");

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
//   xq  int8 [mp][k]       natural order
//   s16 fp16 [mp][k/32]    S_j = bsums[2j] + bsums[2j + 1]
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
    const size_t b = ((size_t)mp * (k / 32) * 2 + 255) & ~(size_t)255;
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
    const size_t b = ((size_t)mp * (k / 32) * 2 + 255) & ~(size_t)255;
    return a + b + (size_t)(k / 256) * mp * sizeof(float) + 256;
}
bool gemm_i8_fits(int64_t n, int64_t k, int64_t m) {
    // 32-bit DMA offsets (the scalar bases carry the superblock and row group)
    return k % 256 == 0 && i8_rows(m) * k < ((int64_t)1 << 31) && n * (k / 256) * Q4K_BYTES < ((int64_t)1 << 31);
}

// NB consecutive superblocks of one row a wave: their loads go out together.
template <int NB>
__global__ __launch_bounds__(256) void k_gemm_prep_i8(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                      _Float16* __restrict__ s16, float* __restrict__ dyt, int m,
                                                      int mp, int k) {
    const int lane = threadIdx.x & 63;
    const int nsb = k >> 8, ngr = nsb / NB;
    const int64_t grp = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (grp >= (int64_t)mp * ngr) return;
    const int mi = (int)(grp / ngr), sb0 = NB * (int)(grp - (int64_t)mi * ngr);
    float4 v[NB];
    if (mi < m) {  // wave-uniform
#pragma unroll
        for (int b = 0; b < NB; b++) v[b] = *(const float4*)(x + (int64_t)mi * k + (sb0 + b) * 256 + 4 * lane);
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        uint32_t q = 0;
        float d = 0.0f;
        int bs = 0;
        if (mi < m) q = q8k_block_wave(v[b], &d, &bs);
        const int sb = sb0 + b;
        *(uint32_t*)(xq + (int64_t)mi * k + sb * 256 + 4 * lane) = q;
        const int S = bs + __shfl_xor(bs, 4, 64);  // lanes 8j .. 8j+7: S_j
        if ((lane & 7) == 0) s16[((int64_t)mi * nsb + sb) * 8 + (lane >> 3)] = (_Float16)(float)S;
        if (lane == 0) dyt[(int64_t)sb * mp + mi] = d;
    }
}

template <int EXP>
__global__ __launch_bounds__(THREADS) void k_gemm_q4k_i8(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                         const _Float16* __restrict__ s16,
                                                         const float* __restrict__ dyt, float* __restrict__ Y, int m,
                                                         int mp, int n, int k, int epi) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int bm, bn;
    tile_of(mp / BM, (n + BN - 1) / BN, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;
    const int nsb = k >> 8;
    const uint32_t rowbytes = (uint32_t)nsb * Q4K_BYTES;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds0 = lds_addr(smem);

    // ---- per-lane DMA offsets, fixed for the K loop ----
    // activations: instruction q = wave + 8 i moves piece q >> 1 of rows
    // 64 (q & 1) .. +63; q & 1 = wave & 1 for every i
    const uint32_t aoff = (uint32_t)(m0 + 64 * (wave & 1) + lane) * (uint32_t)k;
    // weights: instruction q = wave + 8 i moves LDS piece q >> 2 of rows
    // 64 (q & 3) .. +63 (q & 3 = wave & 3); rows past n reload row n - 1
    // (computed, never stored)
    const uint32_t woff = (uint32_t)min(n0 + 64 * (wave & 3) + lane, n - 1) * rowbytes;
    // S (waves 4, 5: 64 rows each) and dy (wave 6, lanes 0..31: 4 rows each)
    const uint32_t sdoff = wave == 6 ? (uint32_t)(m0 + 4 * (lane & 31)) * 4u
                                     : (uint32_t)(m0 + 64 * (wave & 1) + lane) * (uint32_t)(k / 16);

    auto issue = [&](int sb, int stg) {
        const uint32_t al = lds0 + A_OFF + (uint32_t)stg * A_BYTES;
#pragma unroll
        for (int i = 0; i < A_PER_WAVE; i++) {
            const int q = wv + WAVES * i;
            dma16s(xq + (uint32_t)sb * 256u + 16u * (uint32_t)(q >> 1), aoff, al + 2048u * (uint32_t)(q >> 1) +
                                                                                  1024u * (uint32_t)(q & 1));
        }
        const uint32_t wl = lds0 + W_OFF + (uint32_t)stg * W_BYTES;
#pragma unroll
        for (int i = 0; i < W_PER_WAVE; i++) {
            const int q = wv + WAVES * i, p = q >> 2;
            if (q < W_CHUNKS)
                dma16s(W + (uint32_t)sb * Q4K_BYTES + (p < 8 ? 16u + 16u * (uint32_t)p : 0u), woff,
                       wl + 4096u * (uint32_t)p + 1024u * (uint32_t)(q & 3));
        }
        if (wv == 4 || wv == 5)
            dma16s((const uint8_t*)s16 + (uint32_t)sb * 16u, sdoff,
                   lds0 + S_OFF + (uint32_t)stg * S_BYTES + 1024u * (uint32_t)(wv - 4));
        if (wv == 6 && lane < 32)
            dma16s((const uint8_t*)(dyt + (int64_t)sb * mp), sdoff, lds0 + D_OFF + (uint32_t)stg * D_BYTES);
    };

    // Per lane: g = lane / 16 picks 16 of an MFMA's 64 k (and 4 of its 16
    // output rows), r16 = lane % 16 its row (A) or column (B).
    const int g = lane >> 4, r16 = lane & 15;
    v4f out[MT16][2];
#pragma unroll
    for (int t = 0; t < MT16; t++)
#pragma unroll
        for (int u = 0; u < 2; u++) out[t][u] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    // per-lane LDS bases; everything else in a read address is a constant
    const int wrow = 32 * wave + r16;  // the lane's weight column in n tile 0 (+16 in tile 1)
    const int abase = A_OFF + 2048 * g + 16 * r16;
    const int wbase = W_OFF + 4096 * (g & 1) + 16 * wrow, hbase = W_OFF + 8 * 4096 + 16 * wrow;
    const int sbase = S_OFF + 16 * r16 + 8 * (g & 1), dbase = D_OFF + 4 * r16;
    float* const scr = (float*)(smem + SCR_OFF) + 32 * wave;
    // the lane's nibble half (k 32..63 of a 64-k step are the high nibbles)
    // and its scale byte, ((2c + g/2) & 3) for step c, as a v_perm selector
    const int nsh = 4 * (g >> 1);
    const uint32_t sel0 = 0x0c000c00u | (uint32_t)(g >> 1) * 0x00010001u, sel2 = sel0 + 0x00020002u;

    issue(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();

    // One superblock from stage sb & 1, the loads of sb + 1 queued into the other.
    for (int sb = 0; sb < nsb; sb++) {
        const int stg = sb & 1;
        const int sa = abase + stg * A_BYTES, sw = wbase + stg * W_BYTES, sh8 = hbase + stg * W_BYTES;
        const int ss = sbase + stg * S_BYTES, sd = dbase + stg * D_BYTES;
        // 1. this superblock's weight bytes, into registers; the columns' d
        //    to the lanes whose outputs use them (through LDS, within the wave)
        uint4 hdr[2], raw[2][4];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            hdr[u] = *(const uint4*)(smem + sh8 + 256 * u);
#pragma unroll
            for (int c = 0; c < 4; c++) raw[u][c] = *(const uint4*)(smem + sw + (2 * c * 4096 + 256 * u));
        }
        float dmin[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            scr[16 * u + r16] = f16_to_f32(hdr[u].x & 0xffffu);
            dmin[u] = f16_to_f32(hdr[u].x >> 16);
        }
        __builtin_amdgcn_wave_barrier();
        v4f dv[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float4 q = *(const float4*)(scr + 16 * u + 4 * g);
            dv[u] = v4f{q.x, q.y, q.z, q.w};
        }
        // 2. queue the next superblock into the other stage
        __builtin_amdgcn_sched_barrier(0);
        if (sb + 1 < nsb && !(EXP & 4)) issue(sb + 1, 1 - stg);
        __builtin_amdgcn_sched_barrier(0);

        // 3. the weight operands: planes of the four 64-k steps of both n
        //    tiles, and the min term's; s = 0 unless a column of the wave
        //    has dmin >= 1024: then dmin 2^-s < 1024 enters the fp16 pair,
        //    2^-s goes to d and 2^s to dy (exact powers of two)
        float dys = 1.0f, sdn = 1.0f;
        if (__ballot(dmin[0] >= 1024.0f || dmin[1] >= 1024.0f) != 0) {  // wave-uniform, rare
            const float mx = wave_max(__builtin_fmaxf(dmin[0], dmin[1]));
            const int e = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xffu) - 127 - 9;
            sdn = __builtin_bit_cast(float, (uint32_t)(127 - e) << 23);
            dys = __builtin_bit_cast(float, (uint32_t)(127 + e) << 23);
#pragma unroll
            for (int u = 0; u < 2; u++) dv[u] *= sdn;
        }
        v4i plo[2][4], phi[2][4];
        v4h amin[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint4 hd = hdr[u];
            // scales (get_scale_min_k4, k_quants utils.rs:50-60, four at a time)
            const uint32_t sc0 = hd.y & 0x3F3F3F3Fu;
            const uint32_t sc1 = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
            const uint32_t mn = (g & 1) ? (((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u))
                                        : (hd.z & 0x3F3F3F3Fu);
            const uint32_t s0a = sc0 & 0x07070707u, s0b = sc1 & 0x07070707u;
            const uint32_t s1a = (sc0 >> 3) & 0x07070707u, s1b = (sc1 >> 3) & 0x07070707u;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint4 r = raw[u][c];
                const uint32_t q0 = (r.x >> nsh) & 0x0F0F0F0Fu, q1 = (r.y >> nsh) & 0x0F0F0F0Fu,
                               q2 = (r.z >> nsh) & 0x0F0F0F0Fu, q3 = (r.w >> nsh) & 0x0F0F0F0Fu;
                const uint32_t sel = (c & 1) ? sel2 : sel0;
                const uint32_t f0 = __builtin_amdgcn_perm(0u, c < 2 ? s0a : s0b, sel);
                const uint32_t f1 = __builtin_amdgcn_perm(0u, c < 2 ? s1a : s1b, sel);
                if (EXP & 8) {
                    plo[u][c] = v4i{(int)r.x, (int)r.y, (int)r.z, (int)r.w};
                    phi[u][c] = v4i{(int)r.y, (int)r.z, (int)r.w, (int)r.x};
                } else {
                plo[u][c] = v4i{pk_mul(q0, f0), pk_mul(q1, f0), pk_mul(q2, f0), pk_mul(q3, f0)};
                phi[u][c] = v4i{pk_mul(q0, f1), pk_mul(q1, f1), pk_mul(q2, f1), pk_mul(q3, f1)};
                }
            }
            // min-term weight operand, k = 4g .. 4g+3: lanes g = 0, 1 the fp16
            // hi of -dmin' mn_j for j = 4g .. 4g+3, lanes g = 2, 3 the lo
            const float dm = dmin[u] * sdn;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = dm * (float)byte_of(mn, i);  // exact in f32
                const _Float16 vh = (_Float16)v;
                const _Float16 vl = (_Float16)(v - (float)vh);
                amin[u][i] = (g >> 1) ? -vl : -vh;
            }
        }
        // 4. the tiles: 16 activation rows x 16 weight columns, eight int8
        //    MFMAs (four steps, two planes), the min MFMA, the epilogue.
        //    Software-pipelined: tile i's MFMAs are issued with tile i - 1's
        //    epilogue between them, and the next m tile's activations are
        //    read while the current one's MFMAs run.
        v4i bx[2][4];
        v4h sv[2];
        float dy[2];
        v4i lo[2], hi[2];
        v4f dmv[2];
        float dyv[2];
        auto load_b = [&](int t, int buf) {
#pragma unroll
            for (int c = 0; c < 4; c++) bx[buf][c] = *(const v4i*)(smem + sa + (8192 * c + 256 * t));
            sv[buf] = *(const v4h*)(smem + ss + 256 * t);
            dy[buf] = *(const float*)(smem + sd + 64 * t) * dys;
        };
        auto mfmas = [&](int buf, int u, int slot) {
            const v4i z = {0, 0, 0, 0};
            lo[slot] = __builtin_amdgcn_mfma_i32_16x16x64_i8(plo[u][0], bx[buf][0], z, 0, 0, 0);
            hi[slot] = __builtin_amdgcn_mfma_i32_16x16x64_i8(phi[u][0], bx[buf][0], z, 0, 0, 0);
#pragma unroll
            for (int c = 1; c < 4; c++) {
                lo[slot] = __builtin_amdgcn_mfma_i32_16x16x64_i8(plo[u][c], bx[buf][c], lo[slot], 0, 0, 0);
                hi[slot] = __builtin_amdgcn_mfma_i32_16x16x64_i8(phi[u][c], bx[buf][c], hi[slot], 0, 0, 0);
            }
            const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
            dmv[slot] = __builtin_amdgcn_mfma_f32_16x16x16f16(amin[u], sv[buf], zf, 0, 0, 0);
            dyv[slot] = dy[buf];
        };
        auto epi = [&](int t, int u, int buf, int slot) {
            if (EXP & 64) return;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float f = (float)(hi[slot][v] * 8 + lo[slot][v]);
                out[t][u][v] = __builtin_fmaf(__builtin_fmaf(f, dv[u][v], dmv[slot][v]), dyv[slot], out[t][u][v]);
            }
        };
        load_b(0, 0);
#pragma unroll
        for (int i = 0; i < 2 * MT16; i++) {
            const int t = i >> 1, u = i & 1, buf = t & 1, slot = i & 1;
            if (u == 0 && t + 1 < MT16) load_b(t + 1, buf ^ 1);
            mfmas(buf, u, slot);
            if (i > 0) epi((i - 1) >> 1, (i - 1) & 1, ((i - 1) >> 1) & 1, slot ^ 1);
            // interleave: the reads first, then the MFMAs with the previous
            // tile's epilogue between them, starting a few MFMAs in (its
            // inputs have landed by then)
            if (u == 0 && t + 1 < MT16) __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
            if (EXP & 128) {
                __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
#pragma unroll
                for (int k = 0; k < 6; k++) {
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
            } else {
#pragma unroll
                for (int k = 0; k < 9; k++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                }
            }
        }
        epi(MT16 - 1, 1, (MT16 - 1) & 1, 1);
        if (EXP & 64)
            for (int v = 0; v < 4; v++) out[0][0][v] += (float)(lo[0][v] + hi[1][v]) + dmv[0][v] + dmv[1][v];
        // 5. the next stage has landed (this wave's share) and is visible to all
        __builtin_amdgcn_sched_barrier(0);
        if (!(EXP & 2)) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
    }

    // store: lane row m0 + 16 t + r16, columns n0 + 32 wave + 16 u + 4 g + 0..3
#pragma unroll
    for (int t = 0; t < MT16; t++) {
        const int row = m0 + 16 * t + r16;
        if (row >= m) continue;
        float* yr = Y + (int64_t)row * n;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int col = n0 + 32 * wave + 16 * u + 4 * g;
            if (epi == EPI_STORE && col + 3 < n) {
                *(float4*)(yr + col) = make_float4(out[t][u][0], out[t][u][1], out[t][u][2], out[t][u][3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (col + r < n) store_epi_slow(yr + col + r, out[t][u][r], epi);
            }
        }
    }
}


hipError_t launch_gemm_i8(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* ws,
                          int epi, hipStream_t s) {
    static int exp_mode = [] { const char* e = getenv("LLOOM_HIP_I8_EXP"); return e ? atoi(e) : 0; }();
    static bool attr_set = false;
    if (!attr_set) {
        for (const void* f : {(const void*)k_gemm_q4k_i8<0>, (const void*)k_gemm_q4k_i8<2>, (const void*)k_gemm_q4k_i8<4>,
                              (const void*)k_gemm_q4k_i8<12>, (const void*)k_gemm_q4k_i8<20>,
                              (const void*)k_gemm_q4k_i8<28>, (const void*)k_gemm_q4k_i8<36>,
                              (const void*)k_gemm_q4k_i8<44>, (const void*)k_gemm_q4k_i8<68>,
                              (const void*)k_gemm_q4k_i8<76>, (const void*)k_gemm_q4k_i8<128>,
                              (const void*)k_gemm_q4k_i8<132>}) {
            hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
            if (e != hipSuccess) return e;
        }
        attr_set = true;
    }
    const I8Ptrs p = i8_ptrs(ws, m, k);
    const int64_t nsb = k / 256;
    if (nsb % 4 == 0)
        hipLaunchKernelGGL(k_gemm_prep_i8<4>, dim3((unsigned)((p.mp * (nsb / 4) + 3) / 4)), dim3(256), 0, s, x, p.xq,
                           p.s16, p.dyt, (int)m, (int)p.mp, (int)k);
    else
        hipLaunchKernelGGL(k_gemm_prep_i8<1>, dim3((unsigned)((p.mp * nsb + 3) / 4)), dim3(256), 0, s, x, p.xq, p.s16,
                           p.dyt, (int)m, (int)p.mp, (int)k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const unsigned grid = (unsigned)((p.mp / BM) * ((n + BN - 1) / BN));
#define LAUNCH_I8(X) hipLaunchKernelGGL(k_gemm_q4k_i8<X>, dim3(grid), dim3(THREADS), LDS, s, (const uint8_t*)w, p.xq, \
                                        p.s16, p.dyt, y, (int)m, (int)p.mp, (int)n, (int)k, epi)
    switch (exp_mode) {
        case 2: LAUNCH_I8(2); break;
        case 4: LAUNCH_I8(4); break;
        case 12: LAUNCH_I8(12); break;
        case 20: LAUNCH_I8(20); break;
        case 28: LAUNCH_I8(28); break;
        case 36: LAUNCH_I8(36); break;
        case 44: LAUNCH_I8(44); break;
        case 68: LAUNCH_I8(68); break;
        case 76: LAUNCH_I8(76); break;
        case 128: LAUNCH_I8(128); break;
        case 132: LAUNCH_I8(132); break;
        default: LAUNCH_I8(0);
    }
#undef LAUNCH_I8
    return hipGetLastError();
}

}  // namespace lloom
