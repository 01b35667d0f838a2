// gemm.hip -- prefill-shaped Q4_K matmul (m > 16 activation rows): the fp16
// routes (k_gemm_q4k_skinny for up to 128 rows, k_gemm_q4k_x16 past that, the
// default) further down, the routing (launch_gemm), and first the int8-plane
// kernel k_gemm_q4k that LLOOM_HIP_MMA_INT8 falls back to when
// k_gemm_q4k_i8 (gemm_i8.hip) cannot address the shape with 32-bit offsets.
//
// k_gemm_q4k, on int8 MFMA (v_mfma_i32_32x32x32_i8):
//
// y[m, n] = sum_sb dy[m,sb] * ( d[n,sb] * sum_j sc[n,j] * sum_{k in j} x8[m,k] q[n,k]
//                              - dmin[n,sb] * sum_j mn[n,j] * sum_{k in j} x8[m,k] )
// is k_quants' Q4_K x Q8_K dot (k_quants.rs:1540-1620) with every integer sum
// exact and the f32 combination per superblock.
//
// The 6-bit sub-block scale times the 4-bit quant reaches 945 and does not fit
// an int8 operand, so the weights enter the MFMA as two int8 planes,
// sc = 8 * sc_hi + sc_lo with both parts <= 7: q * sc_part <= 105, and one
// v_mul_u32_u24 scales the four packed nibble bytes of a dword at once with
// no carry between bytes.  The MFMA then accumulates a whole 256-element
// superblock in its C operand (two chains, hi and lo), and the f32 epilogue
// runs once per superblock.  The min term is two v_mfma_i32_32x32x16_i8 per
// superblock against the activations' 32-element sums S_j, split into int8
// planes S = 64 * S_hi + S_lo by the activation-prep kernel.
//
// Tiling: a 256-thread workgroup = 2 x 2 waves computes a 128 x 128 block of
// y; each wave 2 x 2 MFMA tiles of 32 x 32.  Each superblock of K is staged
// in LDS (activations, raw Q4_K rows, S planes, dy), double buffered: the
// global loads of superblock sb+1 are in flight while sb is computed.
// MFMA operand layout (same k-set for A and B in a lane, so the hardware's
// own k order never matters):
//   A (activations): lane l holds x8[m = l%32][32j + 16(l/32) + 0..15]
//   B (weights):     lane l holds q[n = l%32][32j + 16(l/32) + 0..15]
//   D:               lane l, reg r holds D[m = 8(r/4) + 4(l/32) + r%4][n = l%32]
#include <cstdlib>
#include <type_traits>

#include "kq_common.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"
#include "kq_gemm.hpp"

namespace lloom {

typedef int v4i __attribute__((ext_vector_type(4)));

// --------------------------------------------------- activation prep --
// Q8_K of every (row, superblock) block, bit-exact, into:
//   xq  int8 [m][k]           natural order
//   sp  int8 [m][k/256][16]   S_hi[0..8) then S_lo[0..8), S_j = bsums[2j] + bsums[2j+1]
//   dyt f32  [k/256][m]
struct PrepPtrs {
    int8_t* xq;
    int8_t* sp;
    float* dyt;
};

static PrepPtrs prep_ptrs(void* base, int64_t m, int64_t k) {
    const size_t q = ((size_t)m * k + 255) & ~(size_t)255;
    const size_t s = ((size_t)m * (k / 256) * 16 + 255) & ~(size_t)255;
    PrepPtrs p;
    p.xq = (int8_t*)base;
    p.sp = (int8_t*)base + q;
    p.dyt = (float*)((uint8_t*)base + q + s);
    return p;
}

static size_t prep_bytes(int64_t m, int64_t k) {
    const size_t q = ((size_t)m * k + 255) & ~(size_t)255;
    const size_t s = ((size_t)m * (k / 256) * 16 + 255) & ~(size_t)255;
    return q + s + (size_t)(k / 256) * m * sizeof(float) + 256;
}

__global__ __launch_bounds__(256) void k_gemm_prep_q8k(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                       int8_t* __restrict__ sp, float* __restrict__ dyt, int m,
                                                       int k) {
    const int lane = threadIdx.x & 63;
    const int nsb = k >> 8;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= (int64_t)m * nsb) return;
    const int mi = (int)(blk / nsb), sb = (int)(blk - (int64_t)mi * nsb);
    const float4 v = *(const float4*)(x + (int64_t)mi * k + sb * 256 + 4 * lane);
    float d;
    int bs;
    const uint32_t q = q8k_block_wave(v, &d, &bs);
    *(uint32_t*)(xq + (int64_t)mi * k + sb * 256 + 4 * lane) = q;
    // lanes 4g..4g+3 hold bsum g; S_j = bsum[2j] + bsum[2j+1] lives on lanes 8j..8j+7
    const int other = __shfl_xor(bs, 4, 64);
    const int S = bs + other;  // on lanes 8j.. (and 8j+4..) S_j
    if ((lane & 7) == 0) {
        const int j = lane >> 3;
        int8_t* o = sp + ((int64_t)mi * nsb + sb) * 16;
        o[j] = (int8_t)(S >> 6);       // S_hi in [-64, 63]
        o[8 + j] = (int8_t)(S & 63);   // S_lo in [0, 63]
    }
    if (lane == 0) dyt[(int64_t)sb * m + mi] = d;
}

// -------------------------------------------------------- Q4_K GEMM ----
constexpr int G_WM = 2, G_WN = 2, G_MT = 2, G_NT = 2;
constexpr int G_BM = G_WM * G_MT * 32, G_BN = G_WN * G_NT * 32;  // 128 x 128
constexpr int G_WAVES = G_WM * G_WN;
constexpr int G_THREADS = 64 * G_WAVES;
// One LDS stage per superblock, filled by global_load_lds_dwordx4 (64 lanes x
// 16 B = 1 KB contiguous per instruction, no staging registers):
//   A  [BM][16 pieces of 16 B], piece p of row r at position p ^ (r & 7):
//      eight consecutive rows reading one piece hit eight bank groups
//   B  [BN][9 pieces] the raw 144-byte Q4_K superblocks (9 is odd: eight
//      consecutive rows reading one piece already hit eight bank groups)
//   S  [BM][16] int8 min-term planes, D [BM] f32 dy
constexpr int G_A_BYTES = G_BM * 256;
constexpr int G_B_BYTES = G_BN * 144;
constexpr int G_S_BYTES = G_BM * 16;
constexpr int G_D_BYTES = G_BM * 4;
constexpr int G_STAGE = G_A_BYTES + G_B_BYTES + G_S_BYTES + G_D_BYTES;
constexpr int G_LDS = 2 * G_STAGE;
constexpr int G_A_CHUNKS = G_A_BYTES / 1024;             // 32
constexpr int G_B_CHUNKS = (G_B_BYTES + 1023) / 1024;    // 18 (the last one partial)
static_assert(G_BM == 128 && G_BN == 128, "staging assumes 128 x 128 tiles");

typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Each 16-bit half of q times f (f < 2^16), modulo 2^16 per half.
__device__ __forceinline__ int pk_mul_u16(uint32_t q, uint32_t f) {
    const u16x2 a = __builtin_bit_cast(u16x2, q);
    const u16x2 b = {(unsigned short)f, (unsigned short)f};
    return __builtin_bit_cast(int, a * b);
}

__device__ __forceinline__ void lds_load16(const void* g, uint8_t* lds_chunk) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_chunk, 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void* g, uint8_t* lds_chunk) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_chunk, 4, 0, 0);
}

// Per-lane byte offsets of this wave's share of a stage, fixed for the
// whole K loop: the superblock only moves the (uniform) base pointers, so
// the loads take the scalar-base + 32-bit-offset form and a stage costs no
// per-lane address arithmetic.
constexpr int G_A_PER_WAVE = G_A_CHUNKS / G_WAVES;                 // 8
constexpr int G_B_PER_WAVE = (G_B_CHUNKS + G_WAVES - 1) / G_WAVES;  // 5
struct StageOffs {
    uint32_t a[G_A_PER_WAVE];
    uint32_t b[G_B_PER_WAVE];
    uint32_t sd;
};

__device__ __forceinline__ StageOffs stage_offsets(int m0, int n0, int m, int n, int k) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nsb = k >> 8;
    const uint32_t rowbytes = (uint32_t)nsb * Q4K_BYTES;
    StageOffs o;
#pragma unroll
    for (int i = 0; i < G_A_PER_WAVE; i++) {
        const int q = wave * G_A_PER_WAVE + i;
        const int row = 4 * q + (lane >> 4);
        const int piece = (lane & 15) ^ (row & 7);
        const int grow = min(m0 + row, m - 1);
        o.a[i] = (uint32_t)grow * (uint32_t)k + 16u * piece;
    }
#pragma unroll
    for (int i = 0; i < G_B_PER_WAVE; i++) {
        const int q = wave + G_WAVES * i;
        const int pc = min(64 * q + lane, G_BN * 9 - 1);
        const int row = pc / 9, piece = pc - row * 9;
        const int grow = min(n0 + row, n - 1);
        o.b[i] = (uint32_t)grow * rowbytes + 16u * piece;
    }
    if (wave < 2) {
        const int grow = min(m0 + 64 * wave + lane, m - 1);
        o.sd = (uint32_t)grow * (uint32_t)nsb * 16u;
    } else {
        const int grow = min(m0 + 64 * (wave - 2) + lane, m - 1);
        o.sd = 4u * (uint32_t)grow;
    }
    return o;
}

// Queue the loads of superblock sb into one LDS stage (each wave its share).
__device__ __forceinline__ void stage_issue(uint8_t* stage, const int8_t* __restrict__ xq,
                                            const int8_t* __restrict__ sp, const float* __restrict__ dyt,
                                            const uint8_t* __restrict__ W, const StageOffs& o, int m, int sb) {
    const int wave = threadIdx.x >> 6;
    uint8_t* A = stage;
    uint8_t* B = stage + G_A_BYTES;
    uint8_t* S = B + G_B_BYTES;
    uint8_t* D = S + G_S_BYTES;
    const int8_t* xb = xq + sb * 256;
    const uint8_t* wb = W + sb * Q4K_BYTES;
#pragma unroll
    for (int i = 0; i < G_A_PER_WAVE; i++) lds_load16(xb + o.a[i], A + 1024 * (wave * G_A_PER_WAVE + i));
#pragma unroll
    for (int i = 0; i < G_B_PER_WAVE; i++) {
        const int q = wave + G_WAVES * i;
        if (q < G_B_CHUNKS) lds_load16(wb + o.b[i], B + 1024 * q);  // wave-uniform
    }
    if (wave < 2) lds_load16(sp + sb * 16 + o.sd, S + 1024 * wave);
    else lds_load4((const uint8_t*)(dyt + (int64_t)sb * m) + o.sd, D + 256 * (wave - 2));
}

// All of this wave's queued LDS loads have landed; then the barrier makes
// every wave's share visible.  The scheduling barrier keeps the compute of
// the current stage ahead of the wait: the asm orders memory operations
// only, and without it the MFMAs drift below the wait and the next stage's
// load latency is no longer hidden.
__device__ __forceinline__ void stage_wait() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

__global__ __launch_bounds__(G_THREADS) void k_gemm_q4k(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                        const int8_t* __restrict__ sp, const float* __restrict__ dyt,
                                                        float* __restrict__ Y, int m, int n, int k, int epi) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / G_WN, wn = wave % G_WN;
    const int h = lane >> 5, c32 = lane & 31;
    int bm, bn;
    tile_of((m + G_BM - 1) / G_BM, (n + G_BN - 1) / G_BN, bm, bn);
    const int m0 = bm * G_BM, n0 = bn * G_BN;
    const int nsb = k >> 8;

    float out[G_MT][G_NT][16];
#pragma unroll
    for (int a = 0; a < G_MT; a++)
#pragma unroll
        for (int b = 0; b < G_NT; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) out[a][b][r] = 0.0f;

    const StageOffs so = stage_offsets(m0, n0, m, n, k);
    stage_issue(smem, xq, sp, dyt, W, so, m, 0);
    stage_wait();

    for (int sb = 0; sb < nsb; sb++) {
        const uint8_t* cur = smem + (sb & 1) * G_STAGE;
        const uint8_t* A = cur;
        const uint8_t* B = cur + G_A_BYTES;
        const int8_t* S = (const int8_t*)(B + G_B_BYTES);
        const float* D = (const float*)((const uint8_t*)S + G_S_BYTES);
        // 1. everything this superblock needs, from LDS into registers, before
        //    the next stage's loads are queued: the compiler cannot tell the
        //    async LDS writes from these reads and would otherwise wait for
        //    the next stage before the first read of this one.
        uint4 hdr[G_NT], raw[G_NT][4];
#pragma unroll
        for (int b = 0; b < G_NT; b++) {
            const uint8_t* rb = B + (wn * G_NT * 32 + b * 32 + c32) * 144;
            hdr[b] = *(const uint4*)rb;
#pragma unroll
            for (int c = 0; c < 4; c++) raw[b][c] = *(const uint4*)(rb + 16 + 32 * c + 16 * h);
        }
        v4i av[G_MT][8];
        long smin[G_MT];
        float4 dy[G_MT][4];
#pragma unroll
        for (int a = 0; a < G_MT; a++) {
            const int row = wm * G_MT * 32 + a * 32 + c32;
#pragma unroll
            for (int j = 0; j < 8; j++) av[a][j] = *(const v4i*)(A + row * 256 + 16 * ((2 * j + h) ^ (row & 7)));
            smin[a] = *(const long*)(S + row * 16 + 8 * h);
            const float* dyp = D + wm * G_MT * 32 + a * 32 + 4 * h;
#pragma unroll
            for (int g = 0; g < 4; g++) dy[a][g] = *(const float4*)(dyp + 8 * g);
        }
        // 2. queue the next superblock into the other stage
        if (sb + 1 < nsb) stage_issue(smem + ((sb + 1) & 1) * G_STAGE, xq, sp, dyt, W, so, m, sb + 1);

        // 3. the MFMA work, from registers
        v16i dh[G_MT][G_NT], dl[G_MT][G_NT];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int c = j >> 1, sh = (j & 1) * 4;
#pragma unroll
            for (int b = 0; b < G_NT; b++) {
                int sc;
                if (j < 4)
                    sc = byte_of(hdr[b].y, j) & 63;
                else
                    sc = (byte_of(hdr[b].w, j - 4) & 0xF) | ((byte_of(hdr[b].y, j - 4) >> 6) << 4);
                const uint32_t q0 = (raw[b][c].x >> sh) & 0x0F0F0F0Fu, q1 = (raw[b][c].y >> sh) & 0x0F0F0F0Fu,
                               q2 = (raw[b][c].z >> sh) & 0x0F0F0F0Fu, q3 = (raw[b][c].w >> sh) & 0x0F0F0F0Fu;
                const uint32_t shi = (uint32_t)sc >> 3, slo = (uint32_t)sc & 7u;
                // four nibble bytes times a 3-bit factor: at most 105 per byte,
                // so one packed 16-bit multiply (v_pk_mul_lo_u16, full rate)
                // scales two bytes per half with no carry between them
                const v4i bhi = {pk_mul_u16(q0, shi), pk_mul_u16(q1, shi), pk_mul_u16(q2, shi), pk_mul_u16(q3, shi)};
                const v4i blo = {pk_mul_u16(q0, slo), pk_mul_u16(q1, slo), pk_mul_u16(q2, slo), pk_mul_u16(q3, slo)};
#pragma unroll
                for (int a = 0; a < G_MT; a++) {
                    if (j == 0) {
                        const v16i zero = {};
                        dh[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a][j], bhi, zero, 0, 0, 0);
                        dl[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a][j], blo, zero, 0, 0, 0);
                    } else {
                        dh[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a][j], bhi, dh[a][b], 0, 0, 0);
                        dl[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a][j], blo, dl[a][b], 0, 0, 0);
                    }
                }
            }
        }
        // superblock epilogue: min term on MFMA, then the f32 combination
#pragma unroll
        for (int b = 0; b < G_NT; b++) {
            const float d = f16_to_f32(hdr[b].x & 0xffffu), dmin = f16_to_f32(hdr[b].x >> 16);
            uint32_t mlo = 0, mhi = 0;  // the 8 six-bit mins, one byte each
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint32_t mn = j < 4 ? (byte_of(hdr[b].z, j) & 63)
                                          : ((byte_of(hdr[b].w, j - 4) >> 4) | ((byte_of(hdr[b].z, j - 4) >> 6) << 4));
                if (j < 4) mlo |= mn << (8 * j);
                else mhi |= mn << (8 * (j - 4));
            }
            const long mins = (long)(((uint64_t)mhi << 32) | mlo);
            const long b1 = h == 0 ? mins : 0l;  // pairs with S_hi (k 0..7)
            const long b2 = h == 0 ? 0l : mins;  // pairs with S_lo (k 8..15)
#pragma unroll
            for (int a = 0; a < G_MT; a++) {
                const v16i zero = {};
                const v16i mh = __builtin_amdgcn_mfma_i32_32x32x16_i8(smin[a], b1, zero, 0, 0, 0);
                const v16i ml = __builtin_amdgcn_mfma_i32_32x32x16_i8(smin[a], b2, zero, 0, 0, 0);
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float dys[4] = {dy[a][g].x, dy[a][g].y, dy[a][g].z, dy[a][g].w};
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int r = 4 * g + u;
                        const int tot = dh[a][b][r] * 8 + dl[a][b][r];
                        const int mn = mh[r] * 64 + ml[r];
                        out[a][b][r] = __builtin_fmaf(dys[u], __builtin_fmaf((float)tot, d, -((float)mn * dmin)),
                                                      out[a][b][r]);
                    }
                }
            }
        }
        // 4. the next stage has landed (this wave's share) and is visible to all
        stage_wait();
    }

#pragma unroll
    for (int a = 0; a < G_MT; a++)
#pragma unroll
        for (int b = 0; b < G_NT; b++) {
            const int col = n0 + wn * G_NT * 32 + b * 32 + c32;
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * G_MT * 32 + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < m) {
                    if (epi == EPI_STORE) Y[(int64_t)row * n + col] = out[a][b][r];
                    else store_epi_slow(&Y[(int64_t)row * n + col], out[a][b][r], epi);
                }
            }
        }
}

// ------------------------------------- Q4_K GEMM on exact fp16 MFMA --
// The same integer sums with the operands in fp16: the quantized
// activations x8 (|x8| <= 127) and the scaled weights sc * q (<= 945) are
// integers fp16 holds exactly, every product is exact, and
// v_mfma_f32_32x32x16_f16 accumulates a superblock's 256 products per output
// in f32 (partial sums stay below 2^25, so at worst the last bit of a sum
// past 2^24 is rounded).  One MFMA chain instead of the int8 kernel's two
// (hi and lo scale planes), at half the int8 rate: the same MFMA time, but
// the superblock result is f32 already.  The min term is one more MFMA per
// tile and superblock with operands [S_hi | S_lo] (activation side, S_j =
// 64 S_hi + S_lo) and [64 m | m] (weight side; 64 m is exact in fp16 too),
// so the f32 epilogue per output and superblock is three instructions:
//     out += dy * (d * D - dmin * Dmin)
//
// Tiling: 256 threads = 2 x 2 waves, a 256 x 128 block of y, each wave
// 4 x 2 tiles of 32 x 32 (128 x 64; one wave per SIMD).  K moves in steps
// of 64 (a quarter superblock).  Everything the loop reads from memory
// arrives by global_load_lds: the fp16 activation tile (from
// k_gemm_prep_x16; a ring of three stages), the step's 32 packed nibble
// bytes of each weight row (a ring of four slots), and per superblock the
// weight headers, the min-term operands and dy.  No load in the loop has a
// register result, so the only memory waits are the counted ones before
// each barrier.  A lane builds its weight operands in registers from 16 of
// its column's bytes (two values per v_pk_fma_f16), one step ahead, while
// the MFMAs of the current step run.  Inside each 64-element step the k
// order is the one the nibble layout gives (element e at slot e with bits
// 0 and 1 swapped); the activation prep writes the same order, and an MFMA
// never depends on the order of k.
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Tile geometry: MT = 32 x 32 tiles per wave along M (2 or 4), WNW waves
// along N (2: 2 x 2 waves, a 64 MT x 128 block; 4: 1 x 4 waves, a 32 MT x 256
// block).  A wave always owns 32 MT rows x 64 columns.  The 1 x 4 layout
// moves 2/3 of the 2 x 2 layout's bytes per MFMA (the fp16 activation tile
// is half as tall for the same work) and unpacks every weight column once
// instead of in two waves.
template <int MT, int WNW, int WV = 4>
struct XCfg {
    static constexpr int WAVES = WV, WMW = WAVES / WNW;
    static constexpr int BM = 32 * MT * WMW, BN = 64 * WNW, BK = 64;
    static constexpr int THREADS = 64 * WAVES, NT = 2;
    static constexpr int A_STAGES = 3, R_SLOTS = 4;
    static constexpr int A_BYTES = BM * BK * 2;  // 1 KB DMA chunks
    static constexpr int R_BYTES = BN * 32;      // the step's qs bytes of BN rows
    static constexpr int A_PER_WAVE = A_BYTES / 1024 / WAVES;
    // weight DMA: 1 KB chunks of 32 columns (the step's bytes, or a
    // superblock's headers), R_PER_WAVE chunks per wave
    static constexpr int R_PER_WAVE = BN / 32 / WAVES;
    // per superblock: min operands [BM][32 B], dy [BM] f32 (256 B per
    // wave), weight headers [BN][16 B] (1 KB per chunk: lanes 32..63 reload
    // lanes 0..31's columns into a copy nobody reads, so every wave issues
    // the same loads)
    // (with more waves than min-operand chunks, the extra waves' loads go
    // to a trash chunk, so every wave issues the same number of loads)
    static constexpr int S_CHUNKS = BM * 32 / 1024;
    static constexpr int S_PER_WAVE = S_CHUNKS >= WAVES ? S_CHUNKS / WAVES : 1;
    static constexpr int SB_AMIN = 0, SB_DY = (S_CHUNKS + 1) * 1024, SB_HDR = SB_DY + 256 * WAVES;
    static constexpr int SB_BYTES = SB_HDR + 1024 * WAVES * R_PER_WAVE;
    static constexpr int R_OFF = A_STAGES * A_BYTES, SB_OFF = R_OFF + R_SLOTS * R_BYTES;
    static constexpr int LDS = SB_OFF + 2 * SB_BYTES;
    // loads per wave and step: SB (first step of a superblock), A(s + 2), raw(s + 3)
    static constexpr int DMA_AFTER_RAW = A_PER_WAVE + R_PER_WAVE;
    static_assert(R_PER_WAVE >= 1 && BN % (32 * WAVES) == 0, "weight DMA shares");
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(BM <= 256 && (S_CHUNKS % WAVES == 0 || S_CHUNKS < WAVES), "row DMA shares");
    static_assert(64 * WAVES >= BM, "dy DMA covers the tile's rows");
    static_assert(A_PER_WAVE == 1 || A_PER_WAVE == 2 || A_PER_WAVE % 4 == 0,
                  "activation DMA spread over the four slices of a step");
};

// Row r of a [rows][64 halves] tile: 8 pieces of 16 bytes, piece p at
// position p ^ (r & 7) (rows that read one piece hit eight bank groups).
__device__ __forceinline__ int x_pos(int row, int piece) { return row * 128 + 16 * (piece ^ (row & 7)); }

// Activation prep: Q8_K of every (row, superblock), bit-exact, into
//   x16  fp16 [m][k]          x8, each 64-element step in slot order
//   amin fp16 [m][k/256][16]  S_hi[0..8) then S_lo[0..8)
//   dyt  f32  [k/256][m]
struct X16Ptrs {
    _Float16* x16;
    _Float16* amin;
    float* dyt;
};
static X16Ptrs x16_ptrs(void* base, int64_t m, int64_t k) {
    const size_t a = ((size_t)m * k * 2 + 255) & ~(size_t)255;
    const size_t b = ((size_t)m * (k / 256) * 32 + 255) & ~(size_t)255;
    X16Ptrs p;
    p.x16 = (_Float16*)base;
    p.amin = (_Float16*)((uint8_t*)base + a);
    p.dyt = (float*)((uint8_t*)base + a + b);
    return p;
}
static size_t x16_bytes(int64_t m, int64_t k) {
    const size_t a = ((size_t)m * k * 2 + 255) & ~(size_t)255;
    const size_t b = ((size_t)m * (k / 256) * 32 + 255) & ~(size_t)255;
    return a + b + (size_t)(k / 256) * m * sizeof(float) + 256;
}

__global__ __launch_bounds__(256) void k_gemm_prep_x16(const float* __restrict__ x, _Float16* __restrict__ x16,
                                                       _Float16* __restrict__ amin, float* __restrict__ dyt, int m,
                                                       int k) {
    // four blocks a wave, one a 16-lane row; lane j of a row holds elements
    // 16j .. 16j+15 of its block (q8k_block_row16)
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int nsb = k >> 8;
    const int64_t nblk = (int64_t)m * nsb;
    const int64_t blk0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
    const bool real = blk0 < nblk;  // per 16-lane row
    const int64_t blk = real ? blk0 : 0;
    const int mi = (int)(blk / nsb), sb = (int)(blk - (int64_t)mi * nsb);
    const float* xr = x + (int64_t)mi * k + sb * 256 + 16 * j;
    float xs[16];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float4 v = *(const float4*)(xr + 4 * c);
        xs[4 * c] = v.x;
        xs[4 * c + 1] = v.y;
        xs[4 * c + 2] = v.z;
        xs[4 * c + 3] = v.w;
    }
    float d;
    int bs;
    const uint4 q = q8k_block_row16(xs, &d, &bs);
    const int S = bs + __shfl_xor(bs, 1, 64);  // pieces 2i and 2i + 1: S_i
    if (!real) return;
    // elements 4l .. 4l+3 go to slots 4l, 4l+2, 4l+1, 4l+3 (bits 0, 1 swapped)
    typedef _Float16 v8hh __attribute__((ext_vector_type(8)));
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    v8hh o[2];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t v = w[c];
        o[c >> 1][4 * (c & 1)] = (_Float16)(float)(int8_t)(v & 0xff);
        o[c >> 1][4 * (c & 1) + 1] = (_Float16)(float)(int8_t)((v >> 16) & 0xff);
        o[c >> 1][4 * (c & 1) + 2] = (_Float16)(float)(int8_t)((v >> 8) & 0xff);
        o[c >> 1][4 * (c & 1) + 3] = (_Float16)(float)(int8_t)(v >> 24);
    }
    _Float16* xo = x16 + (int64_t)mi * k + sb * 256 + 16 * j;
    *(v8hh*)xo = o[0];
    *(v8hh*)(xo + 8) = o[1];
    if ((j & 1) == 0) {
        _Float16* a = amin + ((int64_t)mi * nsb + sb) * 16;
        a[j >> 1] = (_Float16)(float)(S >> 6);      // S_hi in [-64, 63]
        a[8 + (j >> 1)] = (_Float16)(float)(S & 63);  // S_lo in [0, 63]
    }
    if (j == 0) dyt[(int64_t)sb * m + mi] = d;
}

// Four nibbles (one per byte of w, each 0..15) times sc, as fp16 in slot
// order [q0 q2 q1 q3]: v_perm_b32 puts each nibble under the exponent byte
// 0x64, making the fp16 1024 + q exactly, and one packed fma gives
// (1024 + q) * sc - 1024 * sc = q * sc, exact (q * sc <= 945, rounded once).
__device__ __forceinline__ uint2 nib4_to_h(uint32_t w, h2 sc, h2 off) {
    const uint32_t e = __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u);  // [q0, q2]
    const uint32_t o = __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);  // [q1, q3]
    const h2 ve = __builtin_elementwise_fma(__builtin_bit_cast(h2, e), sc, off);
    const h2 vo = __builtin_elementwise_fma(__builtin_bit_cast(h2, o), sc, off);
    return make_uint2(__builtin_bit_cast(uint32_t, ve), __builtin_bit_cast(uint32_t, vo));
}

// MFMA slice kk of a step, lane half h: piece (kk & 1) + 4 (kk >> 1) + 2h,
// i.e. low nibbles of parts 2h, 2h + 1 (kk 0, 1), then their high nibbles:
// a lane's weight operands of a step are the 16 contiguous bytes 16h ..
// 16h+15 of its column's 32.
__device__ __forceinline__ int x_piece(int kk, int h) { return (kk & 1) + 4 * (kk >> 1) + 2 * h; }

// The weight operands of one step from the lane's 16 bytes: scales of
// sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles) from the header
// (bscale), then MFMA slice kk (build_kk).
struct BScale {
    h2 scl, sch, offl, offh;
};
// (c is a compile-time step index at every call.)  The pair's two 6-bit
// scales go under the fp16 exponent byte 0x64 by one v_perm_b32 (1024 + sc,
// exact) and one packed subtract leaves [sc0, sc1]; the halves are then
// broadcast into the packed fma's operands.
__device__ __forceinline__ BScale bscale(const uint4& hdr, int c) {
    const uint32_t w = c < 2 ? (hdr.y & 0x3F3F3F3Fu) : ((hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u));
    const uint32_t sel = (c & 1) ? 0x04030402u : 0x04010400u;  // bytes 2(c&1), 2(c&1)+1
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const h2 p = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, sel)) - k1024;
    const h2 o = p * (_Float16)(-1024.0f);
    BScale b;
    b.scl = __builtin_shufflevector(p, p, 0, 0);
    b.sch = __builtin_shufflevector(p, p, 1, 1);
    b.offl = __builtin_shufflevector(o, o, 0, 0);
    b.offh = __builtin_shufflevector(o, o, 1, 1);
    return b;
}
// The min-term weight operand of a column (lane half h): its eight 6-bit
// mins m_j as fp16, times 64 for h = 0 (the operand pairs them with the
// activation sums' S_hi, then S_lo), by the same v_perm_b32 exponent trick.
__device__ __forceinline__ v8h bmins(const uint4& hdr, int h) {
    const uint32_t ml = hdr.z & 0x3F3F3F3Fu, mh = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const _Float16 f = h == 0 ? (_Float16)64.0f : (_Float16)1.0f;
    const h2 fs = {f, f};
    const h2 p0 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, ml, 0x04010400u)) - k1024) * fs;
    const h2 p1 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, ml, 0x04030402u)) - k1024) * fs;
    const h2 p2 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, mh, 0x04010400u)) - k1024) * fs;
    const h2 p3 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, mh, 0x04030402u)) - k1024) * fs;
    return __builtin_bit_cast(v8h, make_uint4(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                                              __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)));
}
__device__ __forceinline__ v8h build_kk(const uint4& raw, const BScale& bs, int kk) {
    const uint32_t w0 = kk & 1 ? raw.z : raw.x, w1 = kk & 1 ? raw.w : raw.y;
    const uint32_t m0w = kk < 2 ? (w0 & 0x0F0F0F0Fu) : ((w0 >> 4) & 0x0F0F0F0Fu);
    const uint32_t m1w = kk < 2 ? (w1 & 0x0F0F0F0Fu) : ((w1 >> 4) & 0x0F0F0F0Fu);
    const uint2 p0 = nib4_to_h(m0w, kk < 2 ? bs.scl : bs.sch, kk < 2 ? bs.offl : bs.offh);
    const uint2 p1 = nib4_to_h(m1w, kk < 2 ? bs.scl : bs.sch, kk < 2 ? bs.offl : bs.offh);
    return __builtin_bit_cast(v8h, make_uint4(p0.x, p0.y, p1.x, p1.y));
}

template <int MT, int WNW, int WV>
__global__ __launch_bounds__(64 * WV) void k_gemm_q4k_x16(const uint8_t* __restrict__ W,
                                                            const _Float16* __restrict__ x16,
                                                            const _Float16* __restrict__ amin,
                                                            const float* __restrict__ dyt, float* __restrict__ Y,
                                                            int m, int n, int k, int epi) {
    using C = XCfg<MT, WNW, WV>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WNW, wn = wave % WNW;  // WMW x WNW waves, 32 MT x 64 each
    const int h = lane >> 5, c32 = lane & 31;
    int bm, bn;
    tile_of((m + C::BM - 1) / C::BM, (n + C::BN - 1) / C::BN, bm, bn);
    const int m0 = bm * C::BM, n0 = bn * C::BN;
    const int nsb = k >> 8, nsteps = nsb * 4;
    const uint32_t rowbytes = (uint32_t)nsb * Q4K_BYTES;

    // Per-lane byte offsets, fixed for the whole K loop.
    // activation DMA: chunk q = 8 rows x 128 B, piece p of row r at position p ^ (r & 7)
    uint32_t aoff[C::A_PER_WAVE];
#pragma unroll
    for (int i = 0; i < C::A_PER_WAVE; i++) {
        const int q = wave * C::A_PER_WAVE + i;
        const int row = 8 * q + (lane >> 3);
        const int piece = (lane & 7) ^ (row & 7);
        aoff[i] = (uint32_t)min(m0 + row, m - 1) * (uint32_t)k * 2u + 16u * piece;
    }
    // weight-byte DMA: wave w moves columns 32w .. 32w+31; slot (16 B) l
    // holds half l >> 5 of column 32w + (l & 31), so the 32 lanes reading one
    // half read 32 consecutive slots
    uint32_t colw[C::R_PER_WAVE];
#pragma unroll
    for (int i = 0; i < C::R_PER_WAVE; i++)
        colw[i] = (uint32_t)min(n0 + 32 * (C::R_PER_WAVE * wave + i) + c32, n - 1) * rowbytes;
    // min operands: wave w moves rows 32 (C::S_PER_WAVE w + i) + lane / 2, halves lane & 1
    uint32_t soff[C::S_PER_WAVE];
#pragma unroll
    for (int i = 0; i < C::S_PER_WAVE; i++)
        soff[i] = (uint32_t)min(m0 + 32 * min(C::S_PER_WAVE * wave + i, C::S_CHUNKS - 1) + (lane >> 1), m - 1) *
                      (uint32_t)nsb * 32u +
                  16u * (lane & 1);
    const uint32_t dyoff = (uint32_t)min(m0 + 64 * wave + lane, m - 1) * 4u;
    // the wave index as a scalar: the DMA destinations are then SGPR math
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds0 = lds_addr(smem);
    uint32_t colwh[C::R_PER_WAVE];  // the lane's half (16 h) of the step's 32 bytes
#pragma unroll
    for (int i = 0; i < C::R_PER_WAVE; i++) colwh[i] = colw[i] + 16u * (uint32_t)h;

    auto issue_a = [&](int src, int dst) {
        const uint32_t A = lds0 + (dst % C::A_STAGES) * C::A_BYTES;
        const uint8_t* ab = (const uint8_t*)x16 + (uint32_t)src * (C::BK * 2);
#pragma unroll
        for (int i = 0; i < C::A_PER_WAVE; i++) dma16s(ab, aoff[i], A + 1024 * (wv * C::A_PER_WAVE + i));
    };
    auto issue_raw = [&](int src, int dst) {
        const uint32_t R = lds0 + C::R_OFF + (dst % C::R_SLOTS) * C::R_BYTES;
        const uint8_t* rb = W + (uint32_t)(src >> 2) * Q4K_BYTES + 32u * (src & 3) + 16u;
#pragma unroll
        for (int i = 0; i < C::R_PER_WAVE; i++) dma16s(rb, colwh[i], R + 1024 * (C::R_PER_WAVE * wv + i));
    };
    auto issue_sb = [&](int sb) {
        const uint32_t SB = lds0 + C::SB_OFF + (sb & 1) * C::SB_BYTES;
#pragma unroll
        for (int i = 0; i < C::S_PER_WAVE; i++)
            dma16s((const uint8_t*)amin + (uint32_t)sb * 32u, soff[i],
                   SB + C::SB_AMIN + 1024 * min(C::S_PER_WAVE * wv + i, C::S_CHUNKS));
        dma4s(dyt + (int64_t)sb * m, dyoff, SB + C::SB_DY + 256 * wv);
        const uint8_t* hb = W + (uint32_t)sb * Q4K_BYTES;
#pragma unroll
        for (int i = 0; i < C::R_PER_WAVE; i++)
            dma16s(hb, colw[i], SB + C::SB_HDR + 1024 * (C::R_PER_WAVE * wv + i));
    };
    auto read_raw = [&](int step, uint4 (&r)[C::NT]) {
        const uint8_t* R = smem + C::R_OFF + (step % C::R_SLOTS) * C::R_BYTES;
#pragma unroll
        for (int b = 0; b < C::NT; b++) r[b] = *(const uint4*)(R + 1024 * (C::NT * wn + b) + 16 * (32 * h + c32));
    };
    auto read_hdr = [&](int sb, uint4 (&hd)[C::NT]) {
        const uint8_t* SB = smem + C::SB_OFF + (sb & 1) * C::SB_BYTES + C::SB_HDR;
#pragma unroll
        for (int b = 0; b < C::NT; b++) hd[b] = *(const uint4*)(SB + 1024 * (C::NT * wn + b) + 16 * c32);
    };

    v16f acc[MT][C::NT], out[MT][C::NT];
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int b = 0; b < C::NT; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) out[a][b][r] = 0.0f;

    // Order of this wave's DMA loads (vmcnt retires in order; the scheduling
    // barriers keep the groups in order):
    //   prologue: SB(0), A(0), raw(0), raw(1), A(1), raw(2)
    //   step s:   SB(sb + 1) at a superblock's first step, A(s + 2), raw(s + 3)
    // At the end of step s, vmcnt(C::DMA_AFTER_RAW) leaves only A(s + 2) and
    // raw(s + 3) in flight: A(s + 1) (read in step s + 1), raw(s + 2) (unpacked
    // in step s + 1) and SB(sb + 1) have landed.  Steps and superblocks past
    // the end reload the last one into buffers nobody reads again, so the
    // counts never change.  The barriers are bare s_barrier:
    // __syncthreads() would wait for every load in flight.
    issue_sb(0);
    issue_a(0, 0);
    issue_raw(0, 0);
    issue_raw(min(1, nsteps - 1), 1);
    issue_a(min(1, nsteps - 1), 1);
    issue_raw(min(2, nsteps - 1), 2);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C::DMA_AFTER_RAW) : "memory");
    __builtin_amdgcn_s_barrier();

    // Registers across the loop: the current step's weight bytes (raw) and
    // scales (bs), the operands of the MFMA slice in flight (bcur) and the
    // activation fragments of two slices (abuf: slice kk + 1 is read from
    // LDS while slice kk's MFMAs run).  The next step's bytes are read in
    // slice 1 and its first operands built in slice 3, so only a step's
    // first activation read waits on LDS.
    uint4 hdr[C::NT], raw[C::NT];
    BScale bs[C::NT];
    v8h bcur[C::NT];
    v8h abuf[2][MT];
    read_hdr(0, hdr);
    read_raw(0, raw);
#pragma unroll
    for (int b = 0; b < C::NT; b++) {
        bs[b] = bscale(hdr[b], 0);
        bcur[b] = build_kk(raw[b], bs[b], 0);
    }

    for (int sb = 0; sb < nsb; sb++) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int s = 4 * sb + c;
            const uint8_t* A = smem + (s % C::A_STAGES) * C::A_BYTES;
#pragma unroll
            for (int a = 0; a < MT; a++)
                abuf[0][a] = *(const v8h*)(A + x_pos(wm * (32 * MT) + a * 32 + c32, x_piece(0, h)));
            uint4 rawn[C::NT], hn[C::NT];
            BScale bsn[C::NT];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                // 2. the next slice's activations; the next step's bytes
                if (kk < 3) {
#pragma unroll
                    for (int a = 0; a < MT; a++)
                        abuf[(kk + 1) & 1][a] =
                            *(const v8h*)(A + x_pos(wm * (32 * MT) + a * 32 + c32, x_piece(kk + 1, h)));
                }
                if (kk == 1) {
                    read_raw(s + 1, rawn);
                    if (c == 3) read_hdr(sb + 1, hn);
                }
                // 1. queue, spread over the slices (a burst of DMA issues
                //    stalls the wave): the next superblock's operands (first
                //    step), A(s + 2) into the stage step s - 1 used, raw(s + 3)
                //    into step s - 1's slot, in that order
                if (kk == 0 && c == 0) issue_sb(min(sb + 1, nsb - 1));
                {
                    const uint32_t Ad = lds0 + ((s + 2) % C::A_STAGES) * C::A_BYTES;
                    const uint8_t* ab = (const uint8_t*)x16 + (uint32_t)min(s + 2, nsteps - 1) * (C::BK * 2);
#pragma unroll
                    for (int i = 0; i < C::A_PER_WAVE; i++)
                        if (i * 4 / C::A_PER_WAVE == kk)  // compile-time
                            dma16s(ab, aoff[i], Ad + 1024 * (wv * C::A_PER_WAVE + i));
                }
                if (kk == 3) issue_raw(min(s + 3, nsteps - 1), s + 3);
                // the reads above stay ahead of this slice's MFMAs (the
                // scheduler would otherwise sink them to their use)
                __builtin_amdgcn_sched_barrier(0);
                // 3. the next slice's weight operands (the next step's first
                //    in slice 3)
                v8h bnext[C::NT];
#pragma unroll
                for (int b = 0; b < C::NT; b++) {
                    if (kk < 3) {
                        bnext[b] = build_kk(raw[b], bs[b], kk + 1);
                    } else {
                        bsn[b] = bscale(c == 3 ? hn[b] : hdr[b], (c + 1) & 3);
                        bnext[b] = build_kk(rawn[b], bsn[b], 0);
                    }
                }
                // 4. this slice's MFMAs
#pragma unroll
                for (int a = 0; a < MT; a++)
#pragma unroll
                    for (int b = 0; b < C::NT; b++) {
                        if (kk == 0 && c == 0) {
                            const v16f z = {};
                            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(abuf[kk & 1][a], bcur[b], z, 0, 0, 0);
                        } else {
                            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(abuf[kk & 1][a], bcur[b],
                                                                              acc[a][b], 0, 0, 0);
                        }
                    }
#pragma unroll
                for (int b = 0; b < C::NT; b++) bcur[b] = bnext[b];
                // one MFMA, then three VALU (the next slice's unpack), in turn
#pragma unroll
                for (int i = 0; i < MT * C::NT; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int b = 0; b < C::NT; b++) {
                raw[b] = rawn[b];
                bs[b] = bsn[b];
            }
            // 5. superblock epilogue: min term on MFMA, then
            //    out += dy * (d * D - dmin * Dmin)
            if (c == 3) {
                const uint8_t* SB = smem + C::SB_OFF + (sb & 1) * C::SB_BYTES;
#pragma unroll
                for (int b = 0; b < C::NT; b++) {
                    // this lane's column: d, dmin and the mins as [64 m | m]
                    const float d = f16_to_f32(hdr[b].x & 0xffffu), dmin = f16_to_f32(hdr[b].x >> 16);
                    const v8h bmv = bmins(hdr[b], h);
#pragma unroll
                    for (int a = 0; a < MT; a++) {
                        const int row = wm * (32 * MT) + a * 32 + c32;
                        const v8h am = *(const v8h*)(SB + C::SB_AMIN + row * 32 + 16 * h);
                        const v16f z = {};
                        const v16f dm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bmv, z, 0, 0, 0);
                        const float* dyp = (const float*)(SB + C::SB_DY) + wm * (32 * MT) + a * 32 + 4 * h;
#pragma unroll
                        for (int g = 0; g < 4; g++) {
                            const float4 dy4 = *(const float4*)(dyp + 8 * g);
                            const float dys[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
#pragma unroll
                            for (int u = 0; u < 4; u++) {
                                const int r = 4 * g + u;
                                // fused: the integer sums are exact, the
                                // f32 combination is within the tolerance
                                out[a][b][r] = __builtin_fmaf(
                                    dys[u], __builtin_fmaf(d, acc[a][b][r], -(dmin * dm[r])), out[a][b][r]);
                            }
                        }
                    }
                }
#pragma unroll
                for (int b = 0; b < C::NT; b++) hdr[b] = hn[b];
            }
            // 6. A(s + 1), raw(s + 2), SB(sb + 1) have landed; every wave is
            //    past its reads of the stage and slot the next step's DMA
            //    overwrites (step s's)
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C::DMA_AFTER_RAW) : "memory");
            __builtin_amdgcn_s_barrier();
        }
    }
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int b = 0; b < C::NT; b++) {
            const int col = n0 + wn * 64 + b * 32 + c32;
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * (32 * MT) + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < m) {
                    if (epi == EPI_STORE) Y[(int64_t)row * n + col] = out[a][b][r];
                    else store_epi_slow(&Y[(int64_t)row * n + col], out[a][b][r], epi);
                }
            }
        }
}

// ---------------------------------------- few activation rows (17..) --
// The x16 GEMM's arithmetic (exact integer operands on
// v_mfma_f32_32x32x16_f16, the same per-superblock epilogue, the same
// prepared activations) for a few dozen activation rows, where its 128-row
// LDS tiles leave most CUs idle.  A workgroup owns 32 activation rows (grid
// y) and NT tiles of 32 weight columns (grid x); its KS waves split K (wave
// w takes superblocks w, w + KS, ...) and load their operands straight from
// memory into registers, the next step's activations in flight during this
// step's MFMAs; each activation operand serves the NT weight tiles (the
// activations re-read per column block are this kernel's main traffic).
// The waves' partial sums meet in LDS in a fixed order.
template <int KS, int NT>
__global__ __launch_bounds__(64 * KS) void k_gemm_q4k_skinny(const uint8_t* __restrict__ W,
                                                               const _Float16* __restrict__ x16,
                                                               const _Float16* __restrict__ amin,
                                                               const float* __restrict__ dyt, float* __restrict__ Y,
                                                               int m, int n, int k, int epi) {
    __shared__ float part[KS - 1][NT][16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c32 = lane & 31;
    const int n0 = blockIdx.x * 32 * NT, m0 = blockIdx.y * 32;
    const int nsb = k >> 8;
    const uint8_t* wcol[NT];
#pragma unroll
    for (int b = 0; b < NT; b++) wcol[b] = W + (int64_t)min(n0 + 32 * b + c32, n - 1) * nsb * Q4K_BYTES;
    const int arow = min(m0 + c32, m - 1);

    v16f out[NT];
#pragma unroll
    for (int b = 0; b < NT; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) out[b][r] = 0.0f;

    for (int sb = wave; sb < nsb; sb += KS) {
        uint4 hdr[NT], raw[NT][4];
#pragma unroll
        for (int b = 0; b < NT; b++) {
            const uint8_t* wb = wcol[b] + (size_t)sb * Q4K_BYTES;
            hdr[b] = *(const uint4*)wb;
#pragma unroll
            for (int c = 0; c < 4; c++) raw[b][c] = *(const uint4*)(wb + 16 + 32 * c + 16 * h);
        }
        // activations one step ahead of the MFMAs that use them (all four
        // steps at once measured slower: the registers cost waves)
        auto load_a = [&](int c, v8h (&av)[4]) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                av[kk] = *(const v8h*)(x16 + (size_t)arow * k + 256 * sb + 64 * c + 8 * x_piece(kk, h));
        };
        v8h av[4];
        load_a(0, av);
        v16f acc[NT];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            v8h avn[4];
            if (c < 3) load_a(c + 1, avn);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int b = 0; b < NT; b++) {
                const BScale bs = bscale(hdr[b], c);
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const v8h bw = build_kk(raw[b][c], bs, kk);
                    if (c == 0 && kk == 0) {
                        const v16f z = {};
                        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[kk], bw, z, 0, 0, 0);
                    } else {
                        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[kk], bw, acc[b], 0, 0, 0);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (c < 3) {
#pragma unroll
                for (int kk = 0; kk < 4; kk++) av[kk] = avn[kk];
            }
        }
        // superblock epilogue: min term on MFMA, then out += dy (d D - dmin Dmin)
        const v8h am = *(const v8h*)(amin + ((size_t)arow * nsb + sb) * 16 + 8 * h);
        float dys[16];
#pragma unroll
        for (int r = 0; r < 16; r++) dys[r] = dyt[(size_t)sb * m + min(m0 + 8 * (r >> 2) + 4 * h + (r & 3), m - 1)];
#pragma unroll
        for (int b = 0; b < NT; b++) {
            const float d = f16_to_f32(hdr[b].x & 0xffffu), dmin = f16_to_f32(hdr[b].x >> 16);
            const v8h bmv = bmins(hdr[b], h);
            const v16f z = {};
            const v16f dm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bmv, z, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++)
                out[b][r] = __builtin_fmaf(dys[r], __builtin_fmaf(d, acc[b][r], -(dmin * dm[r])), out[b][r]);
        }
    }
    if constexpr (KS > 1) {
        if (wave) {
#pragma unroll
            for (int b = 0; b < NT; b++)
#pragma unroll
                for (int r = 0; r < 16; r++) part[wave - 1][b][r][lane] = out[b][r];
        }
        __syncthreads();
        if (wave) return;
#pragma unroll
        for (int w = 0; w < KS - 1; w++)
#pragma unroll
            for (int b = 0; b < NT; b++)
#pragma unroll
                for (int r = 0; r < 16; r++) out[b][r] += part[w][b][r][lane];
    }
#pragma unroll
    for (int b = 0; b < NT; b++) {
        const int col = n0 + 32 * b + c32;
        if (col < n) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < m) store_epi(&Y[(int64_t)row * n + col], out[b][r], epi);
            }
        }
    }
}

// ------------------------------------------------------------ dispatch --

// The kernels index activations and weights with 32-bit byte offsets.
static bool fits_32bit(int64_t n, int64_t k, int64_t m) {
    const int64_t rowbytes = (k / 256) * Q4K_BYTES;
    return n * rowbytes < ((int64_t)1 << 31) && m * k * 2 < ((int64_t)1 << 31) &&
           m * (k / 256) * 32 < ((int64_t)1 << 31);
}

// Q6_K below k_gemm_q6k's row count takes the MFMA decode kernel with 64
// activation rows per workgroup layer (launch_mq); Q4_K does only past the skinny kernel's
// limit and up to LLOOM_HIP_MQ_MAX_ROWS (default 64, read once), or with
// the int8-plane GEMM selected.
static int64_t mq_max_rows() {
    static const int64_t v = [] {
        const char* e = getenv("LLOOM_HIP_MQ_MAX_ROWS");
        return e ? (int64_t)atoll(e) : (int64_t)64;
    }();
    return v;
}

static bool use_mq(int type, int64_t m) { return type == T_Q6K || (type == T_Q4K && m <= mq_max_rows()); }

// Q6_K from this many rows takes k_gemm_q6k (LLOOM_HIP_Q6_MIN_ROWS, read
// once, overrides the default)
static int64_t q6_min_rows() {
    static const int64_t v = [] {
        const char* e = getenv("LLOOM_HIP_Q6_MIN_ROWS");
        return e ? (int64_t)atoll(e) : (int64_t)Q6_GEMM_MIN_ROWS;
    }();
    return v;
}

// Q4_K with 17..128 rows and k <= 2048 takes the multi-tile DMA decode
// kernel (either prefill mode: its dots are int8 MFMAs on the Q8_K
// activations, as the decode path's); LLOOM_HIP_MV_DMA_MA=0 (read once)
// turns it off.
static bool use_dma_ma(int type, int64_t k, int64_t m) {
    static const bool on = [] {
        const char* e = getenv("LLOOM_HIP_MV_DMA_MA");
        return !(e && atoi(e) == 0);
    }();
    return on && mv_dma_ma_fits(type, k, m);
}

static int64_t skinny_max_rows();
size_t gemm_workspace_bytes(int type, int64_t n, int64_t k, int64_t m, int mode) {
    mode = gemm_mode(mode, m);
    if (use_dma_ma(type, k, m)) return split_q8k_bytes(k, m);
    if (type == T_Q4K && m <= skinny_max_rows() && fits_32bit(0, k, m) && mode != GEMM_INT8) return x16_bytes(m, k);
    if (type == T_Q6K && m >= q6_min_rows() && q6_gemm_fits(n, k, m)) return q6_gemm_workspace_bytes(n, k, m);
    if (use_mq(type, m)) return split_q8k_bytes(k, m);
    if (type == T_Q8_0 && q8_gemm_fits(n, k, m)) return q8_gemm_workspace_bytes(m, k);
    if (type == T_Q4K && mode == GEMM_INT8 && gemm_i8_fits(n, k, m)) return gemm_i8_workspace_bytes(n, m, k);
    if (type == T_Q4K && fits_32bit(0, k, m)) return mode == GEMM_INT8 ? prep_bytes(m, k) : x16_bytes(m, k);
    return matvec_workspace_bytes(type, n, k, 16);
}

template <int MT, int WNW, int WV>
static hipError_t launch_x16(const void* w, const X16Ptrs& p, float* y, int64_t n, int64_t k, int64_t m,
                             int epi, hipStream_t s) {
    using C = XCfg<MT, WNW, WV>;
    if (hipError_t e = set_lds_limit((const void*)k_gemm_q4k_x16<MT, WNW, WV>, C::LDS)) return e;
    const unsigned grid = (unsigned)(((m + C::BM - 1) / C::BM) * ((n + C::BN - 1) / C::BN));
    hipLaunchKernelGGL((k_gemm_q4k_x16<MT, WNW, WV>), dim3(grid), dim3(C::THREADS), C::LDS, s, (const uint8_t*)w,
                       p.x16, p.amin, p.dyt, y, (int)m, (int)n, (int)k, epi);
    return hipGetLastError();
}

// LLOOM_HIP_X16_TILE (read once) picks the tile for tuning: 0 = 256 x 128,
// 1 = 128 x 256, 2 = 128 x 128 (4 waves, 128 x 64 or 64 x 64 each), 3 =
// 128 x 256 with 8 waves of 64 x 64 (two per SIMD), 4 = 64 x 128 (4 waves
// of 32 x 64); -1 (default) chooses by m.
static int x16_tile_env() {
    static const int v = [] {
        const char* e = getenv("LLOOM_HIP_X16_TILE");
        return e ? atoi(e) : -1;
    }();
    return v;
}

// Q4_K from 17 to 128 activation rows takes k_gemm_q4k_skinny (measured
// on [8192, 2048]: m = 24 11.3 us against 14.8 for the MFMA decode kernel,
// m = 96 24.6 against 34.8 for the x16 GEMM; from m = 256 its per-column-
// block re-reads of the activations lose to the GEMM's LDS tiles).
// LLOOM_HIP_SKINNY_MAX_ROWS overrides the limit (read once).
static int64_t skinny_max_rows() {
    static const int64_t v = [] {
        const char* e = getenv("LLOOM_HIP_SKINNY_MAX_ROWS");
        return e ? (int64_t)atoll(e) : (int64_t)128;
    }();
    return v;
}

hipError_t launch_gemm(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                       void* qbuf, size_t ws_cap, int mode, int epi, hipStream_t s) {
    mode = gemm_mode(mode, m);
    if (gemm_workspace_bytes(type, n, k, m, mode) > ws_cap) return hipErrorInvalidValue;
    if (use_dma_ma(type, k, m)) return launch_mv_dma_ma(type, w, x, y, n, k, m, qbuf, epi, s);
    if (type == T_Q4K && m <= skinny_max_rows() && fits_32bit(n, k, m) && mode != GEMM_INT8) {
        X16Ptrs p = x16_ptrs(qbuf, m, k);
        const int64_t nb = m * (k / 256);
        hipLaunchKernelGGL(k_gemm_prep_x16, dim3((unsigned)((nb + 15) / 16)), dim3(256), 0, s, x, p.x16, p.amin,
                           p.dyt, (int)m, (int)k);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        // NT column tiles a workgroup: as many as keep ~256 workgroups
        // (each activation operand then serves NT tiles); K split over 8
        // waves with one tile, 4 with more (their registers)
        const int64_t layers = (m + 31) / 32, ctiles = (n + 31) / 32;
        const int nt = ctiles * layers >= 4 * 256 ? 4 : ctiles * layers >= 2 * 256 ? 2 : 1;
        const dim3 grid((unsigned)((ctiles + nt - 1) / nt), (unsigned)layers);
        const uint8_t* wb = (const uint8_t*)w;
        if (nt == 4)
            hipLaunchKernelGGL((k_gemm_q4k_skinny<4, 4>), grid, dim3(256), 0, s, wb, p.x16, p.amin, p.dyt, y, (int)m,
                               (int)n, (int)k, epi);
        else if (nt == 2)
            hipLaunchKernelGGL((k_gemm_q4k_skinny<4, 2>), grid, dim3(256), 0, s, wb, p.x16, p.amin, p.dyt, y, (int)m,
                               (int)n, (int)k, epi);
        else if (k >= 8 * 256)
            hipLaunchKernelGGL((k_gemm_q4k_skinny<8, 1>), grid, dim3(512), 0, s, wb, p.x16, p.amin, p.dyt, y, (int)m,
                               (int)n, (int)k, epi);
        else
            hipLaunchKernelGGL((k_gemm_q4k_skinny<4, 1>), grid, dim3(256), 0, s, wb, p.x16, p.amin, p.dyt, y, (int)m,
                               (int)n, (int)k, epi);
        return hipGetLastError();
    }
    if (type == T_Q6K && m >= q6_min_rows() && q6_gemm_fits(n, k, m))
        return launch_q6_gemm(w, x, y, n, k, m, qbuf, ws_cap, epi, s);
    if (use_mq(type, m)) return launch_mq(type, w, x, y, n, k, m, qbuf, epi, s);
    if (type == T_Q4K && mode == GEMM_INT8 && gemm_i8_fits(n, k, m))
        return launch_gemm_i8(w, x, y, n, k, m, qbuf, epi, s);
    if (type == T_Q4K && fits_32bit(n, k, m) && mode != GEMM_INT8) {
        X16Ptrs p = x16_ptrs(qbuf, m, k);
        const int64_t nb = m * (k / 256);
        hipLaunchKernelGGL(k_gemm_prep_x16, dim3((unsigned)((nb + 15) / 16)), dim3(256), 0, s, x, p.x16, p.amin,
                           p.dyt, (int)m, (int)k);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        // 128 x 256 tiles (8 waves) past 512 rows: there the 128 x 128
        // tiles start a second, mostly empty round of workgroups (measured
        // on [8192, 2048]: m = 640 53.7 against 70.1 us, m = 512 52.2
        // against 42.0); 64 x 128 tiles to 256 rows, twice the workgroups
        // of 128 x 128 (m = 160 26.6 against 32.5 us, m = 256 27.6 / 32.7;
        // m = 320 35.4 / 33.9)
        int tile = x16_tile_env();
        if (tile < 0) tile = m > 512 ? 3 : m > 256 ? 2 : 4;
        switch (tile) {
            case 0: return launch_x16<4, 2, 4>(w, p, y, n, k, m, epi, s);
            case 1: return launch_x16<4, 4, 4>(w, p, y, n, k, m, epi, s);
            case 3: return launch_x16<2, 4, 8>(w, p, y, n, k, m, epi, s);
            case 4: return launch_x16<1, 2, 4>(w, p, y, n, k, m, epi, s);
            default: return launch_x16<2, 2, 4>(w, p, y, n, k, m, epi, s);
        }
    }
    if (type == T_Q4K && fits_32bit(n, k, m)) {
        if (hipError_t e = set_lds_limit((const void*)k_gemm_q4k, G_LDS)) return e;
        PrepPtrs p = prep_ptrs(qbuf, m, k);
        const int64_t nb = m * (k / 256);
        hipLaunchKernelGGL(k_gemm_prep_q8k, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x, p.xq, p.sp, p.dyt,
                           (int)m, (int)k);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const unsigned grid = (unsigned)(((m + G_BM - 1) / G_BM) * ((n + G_BN - 1) / G_BN));
        hipLaunchKernelGGL(k_gemm_q4k, dim3(grid), dim3(G_THREADS), G_LDS, s, (const uint8_t*)w, p.xq, p.sp, p.dyt,
                           y, (int)m, (int)n, (int)k, epi);
        return hipGetLastError();
    }
    if (type == T_Q8_0 && q8_gemm_fits(n, k, m)) return launch_q8_gemm(w, x, y, n, k, m, qbuf, ws_cap, epi, s);
    // Q8_0 (and Q4_K past 32-bit offsets): tiles of 16 activation rows
    // through the decode kernels
    for (int64_t r = 0; r < m; r += 16) {
        const int64_t mm = m - r < 16 ? m - r : 16;
        hipError_t e = launch_matvec(type, w, x + r * k, y + r * n, n, k, mm, qbuf, epi, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lloom
