// gemm_i8.hip -- Q4_K prefill GEMM on int8 MFMA (v_mfma_i32_16x16x64_i8).
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
// 8 * hi + lo.  The min term is one v_mfma_f32_16x16x32_f16 per 16 x 16
// block and superblock.  Its activation side is the eight 32-element sums
// S_j, |S_j| <= 4064: past the integers fp16 holds exactly (2048), so each
// enters as 64 S_hi + S_lo (S_hi = S >> 6, S_lo = S & 63, both exact).  Its
// weight side is -dmin * mn_j as an exact fp16 pair hi + lo (dmin * mn_j has
// at most 17 significant bits); the 32 K slots are the four products
// {hi, lo} x {64 S_hi, S_lo} of the eight sub-blocks.  A 32-column group
// whose dmin * 63 reaches 2^15 gets its pairs, and its d, scaled by 2^-e
// and its dy by 2^e (powers of two: exact).  The epilogue per output and
// superblock is four VALU instructions:
//     v = fma(float(8 hi + lo), d, Dmin);  out = fma(v, dy, out)
//
// Weight-side prep.  The launch that quantizes the activations also writes,
// per (weight column, superblock), a 40-byte record (the min operand's hi
// and lo halves, the eight 6-bit sub-block scales) and d as f32, so the
// GEMM spends no VALU on them.
//
// Operand roles.  The weights are the MFMA's A (rows = weight columns n),
// the activations its B (columns = activation rows m).  A K step of 64 is
// one nibble half of 64 consecutive qs bytes, so all lanes of a step mask
// or shift alike and every raw qs byte serves two steps:
//   step ks = 2p + h (p = 0, 1; h = low / high nibble): lane group g = l/16
//   takes qs bytes 64p + 16g .. +15 of weight column l % 16, i.e. elements
//   16 (8p + 4(g>>1) + 2h + (g&1)) .. +15, all in sub-block 4p + 2(g>>1) + h;
//   B lane l takes the same 16 elements of activation row l % 16.
//   D lane l, reg v: [n = 4 (l/16) + v][m = l % 16]
// (an MFMA sums over k whatever order the hardware gives it, as long as A
// and B agree, which they do lane by lane).
//
// Tiling and schedule.  512 threads = 8 waves, two a SIMD; the workgroup
// computes 128 activation rows x 256 weight columns, each wave 32 columns x
// 128 rows (2 x 8 blocks of 16 x 16): the planes it builds from its columns
// serve eight row blocks.  Waves 0-3 (group A) and 4-7 (group B, one on
// each SIMD beside an A wave) run half a superblock apart, so that one wave
// of a SIMD builds planes (VALU) while the other issues MFMAs.  Each
// superblock is two halves, each ending in a workgroup barrier:
//   half 1: A builds planes(sb), row blocks 0-3 of sb; B row blocks 4-7 of sb-1
//   half 2: A row blocks 4-7 of sb;  B builds planes(sb), row blocks 0-3 of sb
// Staging (LDS, two slots each): the weights and records of a superblock
// (read in both halves), activation rows 0-63 (both halves of the same
// superblock) and rows 64-127 (half 2 of sb and half 1 of sb + 1).  Each is
// refilled as soon as its last reader has passed a barrier, one superblock
// ahead: the weights and rows 0-63 of sb + 1 during half 1 of sb, rows
// 64-127 of sb + 1 during its half 2, one or two instructions after each
// row block (issued all at once, the eight waves of a CU queued on the
// memory pipeline for ~1500 cycles a superblock).  Every byte arrives by
// global_load_lds of 1 KB of contiguous memory (or 256 B / 32 B for dy and
// the scale exponents) from a scalar base plus a per-lane offset fixed for
// the whole K loop.
//
// What bounds it (per-wave timestamps, C3 m = 2048): a wave issues at most
// one VALU instruction every ~8 cycles (two waves of a SIMD: one every 4),
// and MFMAs share that issue port.  A superblock costs a wave ~480 VALU
// (256 epilogue, ~140 plane building, the rest addressing) beside its 144
// MFMAs, so two waves a SIMD keep the MFMA pipe about half busy: ~9600
// cycles a superblock against the 4608 of MFMA work.
#include "kq_common.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"
#include "kq_gemm.hpp"


namespace lloom {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128, WAVES = 8, THREADS = 64 * WAVES;
constexpr int REC = 40;  // bytes per (column, superblock) record: min hi[8], min lo[8] (fp16), sc[8]
// LDS, for a tile of BN = 128 NCW weight columns (NCW = 2: each wave 32
// columns; NCW = 1: 16).  Weight slot: qs [BN columns][128 B] with piece p
// of column c at slot p ^ (c & 7) (16 lanes reading one piece of 16 columns
// spread over the banks), the records [BN][40 B], d [BN] f32, the 32-column
// groups' dy scales [BN / 32] f32.  Activation half slot: x8 [16 pieces][64
// rows][16 B], S [64 rows][64 S_hi[8], S_lo[8]] fp16, dy [64] f32.
constexpr int WQ_OFF = 0;
constexpr int AX_OFF = 0, AS_OFF = 16384, AD_OFF = AS_OFF + 2048, A_HALF = AD_OFF + 256;
// DMA instructions a wave issues per weight slot: qs BN / 64, then the
// records, d and exponents: NCW = 2 one or two, NCW = 1 none or one; per
// activation half: x8 2 + S or dy 0 or 1.  The waits use the smallest
// counts, which is stricter for the waves that issue more.
constexpr int WAIT_HALF = 2;
template <int NCW>
struct I8C {
    static constexpr int BN = 128 * NCW;
    static constexpr int REC_OFF = BN * 128, DT_OFF = REC_OFF + BN * REC, ES_OFF = DT_OFF + BN * 4;
    static constexpr int W_SLOT = ES_OFF + 64;
    static constexpr int ALO_OFF = 2 * W_SLOT, AHI_OFF = ALO_OFF + 2 * A_HALF, LDS = AHI_OFF + 2 * A_HALF;
    static constexpr int WAIT_START = NCW == 2 ? 4 + 1 + 2 : 2 + 0 + 2;
    static_assert(LDS <= 160 * 1024, "staging layout");
};
// the workspace layout is sized by the wider tile
constexpr int BN = I8C<2>::BN;

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

// Workspace of a call: the activation prep's outputs, then the weight prep's.
//   xq   int8 [mp/64][k/256][16 pieces][64 rows][16 B]  x8, piece p = elements 16p .. 16p+15
//   s16  fp16 [k/256][mp][16]  64 S_hi_j then S_lo_j, S_j = bsums[2j] + bsums[2j+1]
//   dyt  f32  [k/256][mp]
//   rec  [np/BN][k/256][BN][40 B]  -dmin mn_j as fp16 hi[8], lo[8]; sc_j [8]
//   dt   f32  [np/BN][k/256][BN]   d (times the group's 2^-e)
//   es   f32  [np/BN][k/256][BN/32]  2^e of each 32-column group
// for the column tile width BN of the call (np a multiple of 256 either way)
// with rows m .. mp-1 zero and columns n .. np-1 zero.
struct I8Ptrs {
    int8_t* xq;
    _Float16* s16;
    float* dyt;
    uint8_t* rec;
    float* dt;
    float* es;
    int64_t mp, np;
};
static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }
static int64_t i8_rows(int64_t m) { return (m + BM - 1) / BM * BM; }
static int64_t i8_cols(int64_t n) { return (n + BN - 1) / BN * BN; }
static I8Ptrs i8_ptrs(void* base, int64_t n, int64_t m, int64_t k, size_t* total = nullptr) {
    I8Ptrs p;
    p.mp = i8_rows(m);
    p.np = i8_cols(n);
    const int64_t nsb = k / 256;
    uint8_t* b = (uint8_t*)base;
    size_t o = 0;
    p.xq = (int8_t*)(b + o);
    o += al256((size_t)p.mp * k);
    p.s16 = (_Float16*)(b + o);
    o += al256((size_t)p.mp * nsb * 32);
    p.dyt = (float*)(b + o);
    o += al256((size_t)p.mp * nsb * 4);
    p.rec = b + o;
    o += al256((size_t)p.np * nsb * REC);
    p.dt = (float*)(b + o);
    o += al256((size_t)p.np * nsb * 4);
    p.es = (float*)(b + o);
    o += al256((size_t)(p.np / 32) * nsb * 4);
    if (total) *total = o;
    return p;
}
size_t gemm_i8_workspace_bytes(int64_t n, int64_t m, int64_t k) {
    size_t t = 0;
    i8_ptrs(nullptr, n, m, k, &t);
    return t + 256;
}
bool gemm_i8_fits(int64_t n, int64_t k, int64_t m) {
    // 32-bit DMA offsets (the scalar bases carry the superblock and row group)
    return k % 256 == 0 && i8_rows(m) * k < ((int64_t)1 << 31) && n * (k / 256) * Q4K_BYTES < ((int64_t)1 << 31) &&
           i8_cols(n) * (k / 256) * REC < ((int64_t)1 << 31);
}

// Activation prep (blocks below `act_blocks`): each wave quantizes NB
// superblocks of 4 rows (a 16-lane row of the wave per activation row; lane
// j of it holds piece j: 16 elements, 64 contiguous bytes of x, 16 bytes of
// x8 written where the GEMM's stage wants them), bit-exact to the CPU arm's
// from_float (k_quants.rs:2400-2438).
// Weight prep (the blocks after): one thread per (column, superblock), a
// wave's lanes 64 consecutive columns of one superblock.
template <int NB, int BNR>
__global__ __launch_bounds__(256) void k_gemm_prep_i8(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                                      I8Ptrs p, int m, int n, int k, int act_blocks) {
    const int lane = threadIdx.x & 63;
    const int nsb = k >> 8;
    if ((int)blockIdx.x >= act_blocks) {
        const int64_t t = (int64_t)(blockIdx.x - act_blocks) * 256 + threadIdx.x;
        if (t >= p.np * nsb) return;  // whole waves: np is a multiple of 256
        const int sb = (int)(t / p.np), col = (int)(t % p.np);
        const bool real = col < n;
        uint4 hdr = make_uint4(0, 0, 0, 0);
        if (real) hdr = *(const uint4*)(W + ((int64_t)col * nsb + sb) * Q4K_BYTES);
        const float d = f16_to_f32(hdr.x & 0xffffu), dmin = f16_to_f32(hdr.x >> 16);
        // get_scale_min_k4 (k_quants utils.rs:50-60), four at a time
        const uint32_t sc0 = hdr.y & 0x3F3F3F3Fu;
        const uint32_t sc1 = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
        const uint32_t mn0 = hdr.z & 0x3F3F3F3Fu;
        const uint32_t mn1 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
        // the 32-column group's scale: dmin * 63 * 2^-e below 2^15
        float gm = real ? __builtin_fabsf(dmin) : 0.0f;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) gm = __builtin_fmaxf(gm, __shfl_xor(gm, o, 64));
        int e = 0;
        if (gm * 63.0f >= 32768.0f) e = (int)((__builtin_bit_cast(uint32_t, gm * 63.0f) >> 23) & 0xffu) - 127 - 14;
        const float down = __builtin_bit_cast(float, (uint32_t)(127 - e) << 23);
        const float dm = dmin * down;  // exact: a power of two
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            uint32_t h2 = 0, l2 = 0;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int jj = j + u;
                const float v = -dm * (float)(((jj < 4 ? mn0 : mn1) >> (8 * (jj & 3))) & 0xffu);  // exact in f32
                const _Float16 vh = (_Float16)v;
                const _Float16 vl = (_Float16)(v - (float)vh);
                h2 |= (uint32_t)__builtin_bit_cast(uint16_t, vh) << (16 * u);
                l2 |= (uint32_t)__builtin_bit_cast(uint16_t, vl) << (16 * u);
            }
            hi[j >> 1] = h2;
            lo[j >> 1] = l2;
        }
        const int tile = col / BNR, c = col % BNR;
        uint8_t* r = p.rec + (((int64_t)tile * nsb + sb) * BNR + c) * REC;
        *(uint4*)(r) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4*)(r + 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint2*)(r + 32) = make_uint2(sc0, sc1);
        p.dt[((int64_t)tile * nsb + sb) * BNR + c] = d * down;
        if ((lane & 31) == 0)
            p.es[((int64_t)tile * nsb + sb) * (BNR / 32) + c / 32] = __builtin_bit_cast(float, (uint32_t)(127 + e) << 23);
        return;
    }
    const int j = lane & 15;
    const int ngr = nsb / NB;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (4-row group, superblock group)
    if (wid >= (int64_t)(p.mp / 4) * ngr) return;
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
    const int mp = (int)p.mp;
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
        *(uint4*)(p.xq + ((((int64_t)(mi >> 6) * nsb + sb) * 16 + j) * 64 + (mi & 63)) * 16) = q;
        const int S = bs + __shfl_xor(bs, 1, 64);  // pieces 2i and 2i + 1: S_i
        if ((j & 1) == 0) {
            _Float16* sr = p.s16 + ((int64_t)sb * mp + mi) * 16 + (j >> 1);
            sr[0] = (_Float16)(float)(64 * (S >> 6));  // a multiple of 64 below 2^12 in size: exact
            sr[8] = (_Float16)(float)(S & 63);
        }
        if (j == 0) p.dyt[(int64_t)sb * mp + mi] = d;
    }
}

template <int NCW>
__global__ __launch_bounds__(THREADS) void k_gemm_q4k_i8(const uint8_t* __restrict__ W, I8Ptrs p,
                                                         float* __restrict__ Y, int m, int n, int k, int epi) {
    // NCW 16-column halves a wave: a tile of 8 x 16 NCW weight columns
    using C = I8C<NCW>;
    constexpr int BN = C::BN, WC = 16 * NCW;
    constexpr int REC_OFF = C::REC_OFF, DT_OFF = C::DT_OFF, ES_OFF = C::ES_OFF, W_SLOT = C::W_SLOT;
    constexpr int ALO_OFF = C::ALO_OFF, AHI_OFF = C::AHI_OFF, WAIT_START = C::WAIT_START;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4, G = g >> 1;
    const int mp = (int)p.mp;
    int bm, bn;
    tile_of(mp / BM, (n + BN - 1) / BN, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;
    const int nsb = k >> 8;
    const uint32_t rowbytes = (uint32_t)nsb * Q4K_BYTES;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const bool grpB = wv >= 4;
    const uint32_t lds0 = lds_addr(smem);

    // ---- DMA issue (offsets fixed for the K loop) ----
    // qs: instruction q moves columns 8q .. 8q+7 (lane l: column 8q + l/8,
    // LDS slot l % 8 holding piece (l % 8) ^ (l / 8)); in the last column
    // tile columns past n reload column n - 1 (computed, never stored).
    const uint32_t lane16 = 16u * (uint32_t)lane;
    const bool ragged_n = n0 + BN > n;  // uniform
    const uint32_t qlane = (uint32_t)(lane >> 3) * rowbytes + 16u * (uint32_t)((lane & 7) ^ (lane >> 3));
    const uint8_t* recb = p.rec + (size_t)bn * nsb * (BN * REC);
    const uint8_t* dtb = (const uint8_t*)(p.dt + (size_t)bn * nsb * BN);
    const uint8_t* esb = (const uint8_t*)(p.es + (size_t)bn * nsb * (BN / 32));
    // part 0 / 1: qs instructions 0-1 / 2-3 of the wave; part 2: the rest
    auto issue_w = [&](int sb, int slot, int part) {
        const uint32_t st = lds0 + (uint32_t)slot * W_SLOT;
        const uint8_t* wb = W + (size_t)n0 * rowbytes + (uint32_t)sb * Q4K_BYTES + 16;
#pragma unroll
        for (int i = 0; i < BN / 64; i++) {
            if (part != (NCW == 2 ? i / 2 : i)) continue;
            const int q = wv + WAVES * i;  // 0 .. 31
            if (!ragged_n) {
                dma16s(wb + (size_t)8 * q * rowbytes, qlane, st + WQ_OFF + 1024u * (uint32_t)q);
            } else {
                const int cl = min(n0 + 8 * q + (lane >> 3), n - 1) - n0;
                const uint32_t off = (uint32_t)cl * rowbytes + 16u * (uint32_t)((lane & 7) ^ (lane >> 3));
                dma16s(wb, off, st + WQ_OFF + 1024u * (uint32_t)q);
            }
        }
        if (part != 2) return;
        const uint8_t* rb = recb + (size_t)sb * (BN * REC);
        if constexpr (NCW == 2) {
            // records (10 KB), d (1 KB), group exponents (32 B): 12 more
            // instructions, waves 0-3 two each, 4-7 one each
            dma16s(rb + 1024u * (uint32_t)wv, lane16, st + REC_OFF + 1024u * (uint32_t)wv);
            if (wv < 2) dma16s(rb + 1024u * (uint32_t)(8 + wv), lane16, st + REC_OFF + 1024u * (uint32_t)(8 + wv));
            if (wv == 2) dma16s(dtb + (size_t)sb * (BN * 4), lane16, st + DT_OFF);
            if (wv == 3 && lane < 8) dma4s(esb + (size_t)sb * 32, 4u * (uint32_t)lane, st + ES_OFF);
        } else {
            // records 5 KB (waves 0-4), d 512 B (wave 5, lanes 0-31),
            // exponents 16 B (wave 6)
            if (wv < 5) dma16s(rb + 1024u * (uint32_t)wv, lane16, st + REC_OFF + 1024u * (uint32_t)wv);
            if (wv == 5 && lane < 32) dma16s(dtb + (size_t)sb * (BN * 4), lane16, st + DT_OFF);
            if (wv == 6 && lane < 4) dma4s(esb + (size_t)sb * 16, 4u * (uint32_t)lane, st + ES_OFF);
        }
    };
    // activation rows 64 hf .. 64 hf + 63: x8 16 KB (two instructions a
    // wave), S 2 KB (waves 4, 5), dy 256 B (wave 6)
    auto issue_a = [&](int sb, int hf, int slot) {
        const uint32_t st = lds0 + (hf ? AHI_OFF : ALO_OFF) + (uint32_t)slot * A_HALF;
        const int8_t* xb = p.xq + ((size_t)((m0 >> 6) + hf) * nsb + sb) * 16384;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int q = wv + WAVES * i;  // piece
            dma16s(xb + 1024u * (uint32_t)q, lane16, st + AX_OFF + 1024u * (uint32_t)q);
        }
        const size_t row0 = (size_t)sb * mp + m0 + 64 * hf;
        if (wv == 4 || wv == 5)
            dma16s((const uint8_t*)p.s16 + row0 * 32 + 1024u * (uint32_t)(wv - 4), lane16,
                   st + AS_OFF + 1024u * (uint32_t)(wv - 4));
        if (wv == 6) dma4s((const uint8_t*)(p.dyt + row0), 4u * (uint32_t)lane, st + AD_OFF);
    };

    v4f out[8][NCW];
#pragma unroll
    for (int r = 0; r < 8; r++)
#pragma unroll
        for (int c = 0; c < NCW; c++) out[r][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    // per-wave state of the superblock whose planes are built
    v4i plo[NCW][4], phi[NCW][4];
    v8h amin[NCW];
    v4f dv[NCW];
    float esc = 1.0f;
#pragma unroll
    for (int c = 0; c < NCW; c++) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) plo[c][ks] = phi[c][ks] = v4i{0, 0, 0, 0};
        amin[c] = v8h{0, 0, 0, 0, 0, 0, 0, 0};
        dv[c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // planes of a superblock from weight slot `slot` (the wave's 32 columns)
    auto build = [&](int slot) {
        const int sw = slot * W_SLOT;
        esc = *(const float*)(smem + sw + ES_OFF + 4 * ((WC * wv) >> 5));
#pragma unroll
        for (int c = 0; c < NCW; c++) {
            const int col = WC * wv + 16 * c + l16;
            const uint8_t* cq = smem + sw + WQ_OFF + 128 * col;
            const uint4 r0 = *(const uint4*)(cq + 16 * (g ^ (col & 7)));
            const uint4 r1 = *(const uint4*)(cq + 16 * ((4 + g) ^ (col & 7)));
            const uint8_t* rc = smem + sw + REC_OFF + REC * col;
            amin[c] = *(const v8h*)(rc + 16 * G);
            const uint2 scb = *(const uint2*)(rc + 32);
            dv[c] = *(const v4f*)(smem + sw + DT_OFF + 4 * (WC * wv + 16 * c + 4 * g));
            // the lane's four scales: sub-blocks 2G, 2G + 1, 4 + 2G, 5 + 2G (steps 0..3)
            const uint32_t s4 = __builtin_amdgcn_perm(scb.y, scb.x, G ? 0x07060302u : 0x05040100u);
            const uint32_t s0w = s4 & 0x07070707u, s1w = (s4 >> 3) & 0x07070707u;
            const uint32_t rw[2][4] = {{r0.x, r0.y, r0.z, r0.w}, {r1.x, r1.y, r1.z, r1.w}};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const int pp = ks >> 1, h = ks & 1;
                const uint32_t f0 = byte_pair(s0w, ks), f1 = byte_pair(s1w, ks);
                int a0[4], a1[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint32_t q = (rw[pp][t] >> (4 * h)) & 0x0F0F0F0Fu;
                    a0[t] = pk_mul(q, f0);
                    a1[t] = pk_mul(q, f1);
                }
                plo[c][ks] = v4i{a0[0], a0[1], a0[2], a0[3]};
                phi[c][ks] = v4i{a1[0], a1[1], a1[2], a1[3]};
            }
        }
    };
    // the lane's x8 piece for step ks: 8p + 4G + 2h + (g & 1)
    const int pbase = 1024 * (4 * G + (g & 1)) + 16 * l16;
    // row blocks R0 .. R0+3 (R0 = 0 or 4) from the activation half slot at
    // `ah`, dy times `ys` (0 for a half-step with no superblock: finite data
    // and zero planes or the last planes, so out is unchanged)
    // hook(rr) runs after row block rr's MFMAs: the DMA issue of the half,
    // spread over the row blocks so the waves of a CU do not all queue on
    // the memory pipeline at once
    auto rows = [&](int ah, const int R0, float ys, auto&& hook) {
        auto load_b = [&](int rr, v4i(&b)[4]) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
                b[ks] = *(const v4i*)(smem + ah + AX_OFF + pbase + 1024 * (8 * (ks >> 1) + 2 * (ks & 1)) + 256 * rr);
        };
        auto mfmas = [&](int c, const v4i(&b)[4], const v8h& sv, v4i& lo, v4i& hi, v4f& dm) {
            lo = v4i{0, 0, 0, 0};
            hi = v4i{0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(plo[c][ks], b[ks], lo, 0, 0, 0);
                hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(phi[c][ks], b[ks], hi, 0, 0, 0);
            }
            dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(amin[c], sv, v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        };
        auto epi = [&](int R, int c, const v4i& lo, const v4i& hi, const v4f& dm, float dy) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float f = (float)(hi[v] * 8 + lo[v]);
                out[R][c][v] = __builtin_fmaf(__builtin_fmaf(f, dv[c][v], dm[v]), dy, out[R][c][v]);
            }
        };
        // software pipeline: row block rr's c = 0 MFMAs run beside the
        // epilogue of rr - 1's c = 1, its c = 1 MFMAs beside its own c = 0
        // epilogue; an empty asm after each step pins the epilogues there
        // (left to the compiler they sink to the end of the half-step, and
        // every block's MFMA results stay live)
        v4i bx[4], lo1, hi1;
        v4f dm1;
        float dy1 = 0.0f;
        load_b(0, bx);
        if constexpr (NCW == 2) {
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
                const int ml = 16 * rr + l16;
                v4i bn[4];
                if (rr < 3) load_b(rr + 1, bn);
                const v8h sv = *(const v8h*)(smem + ah + AS_OFF + 32 * ml + 16 * (g & 1));
                const float dy = *(const float*)(smem + ah + AD_OFF + 4 * ml) * ys;
                v4i lo0, hi0;
                v4f dm0;
                mfmas(0, bx, sv, lo0, hi0, dm0);
                if (rr > 0) epi(R0 + rr - 1, 1, lo1, hi1, dm1, dy1);
                mfmas(1, bx, sv, lo1, hi1, dm1);
                epi(R0 + rr, 0, lo0, hi0, dm0, dy);
                dy1 = dy;
                if (rr > 0)
                    asm volatile("" : "+v"(out[R0 + rr - 1][1]), "+v"(out[R0 + rr][0]));
                else
                    asm volatile("" : "+v"(out[R0 + rr][0]));
                hook(rr);
                if (rr < 3)
#pragma unroll
                    for (int ks = 0; ks < 4; ks++) bx[ks] = bn[ks];
            }
            epi(R0 + 3, 1, lo1, hi1, dm1, dy1);
            asm volatile("" : "+v"(out[R0 + 3][1]));
        } else {
            // one 16-column half, two row blocks a step: their four MFMA
            // chains interleave, and the previous step's two epilogues run
            // beside them
            v4i bx2[4], lo1b, hi1b;
            v4f dm1b;
            float dy1b = 0.0f;
            load_b(1, bx2);
#pragma unroll
            for (int rp = 0; rp < 2; rp++) {
                const int r0 = 2 * rp;
                v4i bn[4], bn2[4];
                if (rp == 0) {
                    load_b(2, bn);
                    load_b(3, bn2);
                }
                const int ml = 16 * r0 + l16;
                const v8h sv = *(const v8h*)(smem + ah + AS_OFF + 32 * ml + 16 * (g & 1));
                const v8h sv2 = *(const v8h*)(smem + ah + AS_OFF + 32 * (ml + 16) + 16 * (g & 1));
                const float dy = *(const float*)(smem + ah + AD_OFF + 4 * ml) * ys;
                const float dy2 = *(const float*)(smem + ah + AD_OFF + 4 * (ml + 16)) * ys;
                v4i lo0 = v4i{0, 0, 0, 0}, hi0 = lo0, lo0b = lo0, hi0b = lo0;
#pragma unroll
                for (int ks = 0; ks < 4; ks++) {
                    lo0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(plo[0][ks], bx[ks], lo0, 0, 0, 0);
                    lo0b = __builtin_amdgcn_mfma_i32_16x16x64_i8(plo[0][ks], bx2[ks], lo0b, 0, 0, 0);
                    hi0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(phi[0][ks], bx[ks], hi0, 0, 0, 0);
                    hi0b = __builtin_amdgcn_mfma_i32_16x16x64_i8(phi[0][ks], bx2[ks], hi0b, 0, 0, 0);
                }
                const v4f z = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                const v4f dm0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(amin[0], sv, z, 0, 0, 0);
                const v4f dm0b = __builtin_amdgcn_mfma_f32_16x16x32_f16(amin[0], sv2, z, 0, 0, 0);
                if (rp > 0) {
                    epi(R0 + r0 - 2, 0, lo1, hi1, dm1, dy1);
                    epi(R0 + r0 - 1, 0, lo1b, hi1b, dm1b, dy1b);
                    asm volatile("" : "+v"(out[R0 + r0 - 2][0]), "+v"(out[R0 + r0 - 1][0]));
                }
                lo1 = lo0;
                hi1 = hi0;
                dm1 = dm0;
                dy1 = dy;
                lo1b = lo0b;
                hi1b = hi0b;
                dm1b = dm0b;
                dy1b = dy2;
                hook(r0);
                hook(r0 + 1);
                if (rp == 0)
#pragma unroll
                    for (int ks = 0; ks < 4; ks++) {
                        bx[ks] = bn[ks];
                        bx2[ks] = bn2[ks];
                    }
            }
            epi(R0 + 2, 0, lo1, hi1, dm1, dy1);
            epi(R0 + 3, 0, lo1b, hi1b, dm1b, dy1b);
            asm volatile("" : "+v"(out[R0 + 2][0]), "+v"(out[R0 + 3][0]));
        }
    };

    // workgroup barrier after this wave's own waits; the empty asm keeps the
    // compiler from moving LDS reads across it
    auto bar = [&]() {
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };

    issue_w(0, 0, 0);
    issue_w(0, 0, 1);
    issue_w(0, 0, 2);
    issue_a(0, 0, 0);
    issue_a(0, 1, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    bar();

    // Half-steps: group A's superblock of half-step s is s / 2 (half 1 when s
    // is even), group B's (s - 1) / 2.  out[0..3] holds the row blocks a
    // wave works on in its half 1 (A: 0-3, B: 4-7), out[4..7] those of its
    // half 2, so both groups update the same registers in every half-step.
    for (int it = 0; it <= nsb; it++) {
        const bool more = it + 1 < nsb;
        // ---- half 1 (half-step 2 it)
        __builtin_amdgcn_sched_barrier(0);
        {
            auto hook1 = [&](int rr) {
                if (!more) return;
                if (rr < 3) issue_w(it + 1, (it + 1) & 1, rr);
                else issue_a(it + 1, 0, (it + 1) & 1);
            };
            const int sbw = grpB ? it - 1 : it;  // A: half 1 of it; B: half 2 of it - 1
            const bool live = sbw >= 0 && sbw < nsb;
            if (!grpB && it < nsb) build(it & 1);
            // no superblock: any slot that holds data (that of sb 0)
            rows((grpB ? AHI_OFF : ALO_OFF) + (live ? (sbw & 1) * A_HALF : 0), 0, live ? esc : 0.0f, hook1);
        }
        if (it == nsb) break;
        __builtin_amdgcn_sched_barrier(0);
        if (more)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAIT_START) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        bar();
        // ---- half 2 (half-step 2 it + 1): A half 2 of it, B half 1 of it
        __builtin_amdgcn_sched_barrier(0);
        if (grpB) build(it & 1);
        rows((grpB ? ALO_OFF : AHI_OFF) + (it & 1) * A_HALF, 4, esc, [&](int rr) {
            if (more && rr == 0) issue_a(it + 1, 1, (it + 1) & 1);
        });
        __builtin_amdgcn_sched_barrier(0);
        if (more)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAIT_HALF) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        bar();
    }

    // store: out[i] is row block i (group A) or i ^ 4 (group B); lane row
    // m0 + 16 R + l16, columns n0 + 32 wave + 16 c + 4 g + 0..3
#pragma unroll
    for (int R = 0; R < 8; R++) {
        const int row = m0 + 16 * (grpB ? R ^ 4 : R) + l16;
        if (row >= m) continue;
        float* yr = Y + (int64_t)row * n;
#pragma unroll
        for (int c = 0; c < NCW; c++) {
            const int col = n0 + WC * wave + 16 * c + 4 * g;
            if (epi == EPI_STORE && col + 3 < n) {
                *(float4*)(yr + col) = make_float4(out[R][c][0], out[R][c][1], out[R][c][2], out[R][c][3]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    if (col + v < n) store_epi_slow(yr + col + v, out[R][c][v], epi);
            }
        }
    }
}

// The 128-column tiling is used while its grid fits one workgroup a CU (at
// most 256, so the 256-column one leaves at least half the CUs idle): one
// workgroup holds a CU either way (LDS), and a 128-column one takes ~0.7 of
// the time of a 256-column one (C3 shape, m 256 / 512: 26 / 29 us against
// 40 / 42), so past one round the 256-column tiling's fewer rounds win.
constexpr int64_t I8_NARROW_MAX = 128;

template <int NCW>
static hipError_t launch_i8(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* ws,
                            int epi, hipStream_t s) {
    constexpr int BNT = I8C<NCW>::BN, LDST = I8C<NCW>::LDS;
    if (hipError_t e = set_lds_limit((const void*)k_gemm_q4k_i8<NCW>, LDST)) return e;
    const I8Ptrs p = i8_ptrs(ws, n, m, k);
    const int64_t nsb = k / 256;
    const int64_t wblocks = p.np * nsb / 256;
    if (nsb % 2 == 0) {
        const int64_t ablocks = (p.mp / 4 * (nsb / 2) + 3) / 4;
        hipLaunchKernelGGL((k_gemm_prep_i8<2, BNT>), dim3((unsigned)(ablocks + wblocks)), dim3(256), 0, s, x,
                           (const uint8_t*)w, p, (int)m, (int)n, (int)k, (int)ablocks);
    } else {
        const int64_t ablocks = (p.mp / 4 * nsb + 3) / 4;
        hipLaunchKernelGGL((k_gemm_prep_i8<1, BNT>), dim3((unsigned)(ablocks + wblocks)), dim3(256), 0, s, x,
                           (const uint8_t*)w, p, (int)m, (int)n, (int)k, (int)ablocks);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const unsigned grid = (unsigned)((p.mp / BM) * ((n + BNT - 1) / BNT));
    hipLaunchKernelGGL(k_gemm_q4k_i8<NCW>, dim3(grid), dim3(THREADS), LDST, s, (const uint8_t*)w, p, y, (int)m,
                       (int)n, (int)k, epi);
    return hipGetLastError();
}

hipError_t launch_gemm_i8(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* ws,
                          int epi, hipStream_t s) {
    const int64_t mp = i8_ptrs(ws, n, m, k).mp;
    if ((mp / BM) * ((n + BN - 1) / BN) <= I8_NARROW_MAX) return launch_i8<1>(w, x, y, n, k, m, ws, epi, s);
    return launch_i8<2>(w, x, y, n, k, m, ws, epi, s);
}

}  // namespace lloom
