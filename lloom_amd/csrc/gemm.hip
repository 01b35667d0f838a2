// gemm.hip -- prefill-shaped quantized matmul (m > 16 activation rows) on
// int8 MFMA (v_mfma_i32_32x32x32_i8).
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
#include "kq_common.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"

namespace lloom {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Tile order.  Workgroups are dealt round-robin to the 8 XCDs; renumber them
// XCD-major so each XCD gets a contiguous range, then walk that range in
// groups of GM m-blocks (column-major inside a group): the ~32 workgroups an
// XCD runs at once cover a 4 x 8 block of tiles whose activation and weight
// tiles fit its 4 MB L2, instead of re-reading them for every tile.
__device__ __forceinline__ void tile_of(int nbm, int nbn, int& bm, int& bn) {
    constexpr int GM = 4;
    int pid = blockIdx.x;
    if ((gridDim.x & 7) == 0) pid = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
    const int per_group = GM * nbn;
    const int group = pid / per_group;
    const int first = group * GM;
    const int gsz = min(nbm - first, GM);
    const int in = pid - group * per_group;
    bm = first + in % gsz;
    bn = in / gsz;
}

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

__device__ __forceinline__ void lds_load16(const void* g, uint8_t* lds_chunk) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_chunk, 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void* g, uint8_t* lds_chunk) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_chunk, 4, 0, 0);
}

// Queue the loads of superblock sb into one LDS stage (each wave its share).
__device__ __forceinline__ void stage_issue(uint8_t* stage, const int8_t* __restrict__ xq,
                                            const int8_t* __restrict__ sp, const float* __restrict__ dyt,
                                            const uint8_t* __restrict__ W, int m0, int n0, int m, int n, int k,
                                            int sb) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nsb = k >> 8;
    const int64_t rowbytes = (int64_t)nsb * Q4K_BYTES;
    uint8_t* A = stage;
    uint8_t* B = stage + G_A_BYTES;
    uint8_t* S = B + G_B_BYTES;
    uint8_t* D = S + G_S_BYTES;
#pragma unroll
    for (int i = 0; i < G_A_CHUNKS / G_WAVES; i++) {
        const int q = wave * (G_A_CHUNKS / G_WAVES) + i;
        const int row = 4 * q + (lane >> 4);
        const int piece = (lane & 15) ^ (row & 7);
        const int grow = min(m0 + row, m - 1);
        lds_load16(xq + (int64_t)grow * k + sb * 256 + 16 * piece, A + 1024 * q);
    }
#pragma unroll
    for (int i = 0; i < (G_B_CHUNKS + G_WAVES - 1) / G_WAVES; i++) {
        const int q = wave + G_WAVES * i;
        if (q < G_B_CHUNKS) {  // wave-uniform
            const int pc = min(64 * q + lane, G_BN * 9 - 1);
            const int row = pc / 9, piece = pc - row * 9;
            const int grow = min(n0 + row, n - 1);
            lds_load16(W + grow * rowbytes + sb * Q4K_BYTES + 16 * piece, B + 1024 * q);
        }
    }
    if (wave < 2) {
        const int row = 64 * wave + lane;
        const int grow = min(m0 + row, m - 1);
        lds_load16(sp + ((int64_t)grow * nsb + sb) * 16, S + 1024 * wave);
    } else {
        const int row = 64 * (wave - 2) + lane;
        const int grow = min(m0 + row, m - 1);
        lds_load4(dyt + (int64_t)sb * m + grow, D + 256 * (wave - 2));
    }
}

// All of this wave's queued LDS loads have landed; then the barrier makes
// every wave's share visible.
__device__ __forceinline__ void stage_wait() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

__global__ __launch_bounds__(G_THREADS) void k_gemm_q4k(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                        const int8_t* __restrict__ sp, const float* __restrict__ dyt,
                                                        float* __restrict__ Y, int m, int n, int k) {
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

    stage_issue(smem, xq, sp, dyt, W, m0, n0, m, n, k, 0);
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
        if (sb + 1 < nsb) stage_issue(smem + ((sb + 1) & 1) * G_STAGE, xq, sp, dyt, W, m0, n0, m, n, k, sb + 1);

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
                const v4i bhi = {(int)(q0 * shi), (int)(q1 * shi), (int)(q2 * shi), (int)(q3 * shi)};
                const v4i blo = {(int)(q0 * slo), (int)(q1 * slo), (int)(q2 * slo), (int)(q3 * slo)};
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
                        out[a][b][r] += dys[u] * ((float)tot * d - (float)mn * dmin);
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
                if (row < m) Y[(int64_t)row * n + col] = out[a][b][r];
            }
        }
}

// ------------------------------------------------ Q4_K GEMM on fp16 MFMA --
// The same product with both operands dequantized to fp16 (activations as
// f16(dy * q8) of the bit-exact Q8_K quantization, weights as f16 of
// d*sc*q - dmin*m) and v_mfma_f32_32x32x16_f16 accumulating all of K in f32:
// no per-superblock epilogue at all, at half the int8 MFMA rate.  The
// operand rounding (11 significant bits) costs about 1e-4 of a typical
// output, which keeps a wide row inside the 1e-3 * max|y row| tolerance but
// not a row of a handful of outputs near zero: opt-in, not the default.
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// x f32 [m][k] -> Q8_K (bit-exact) -> f16(d * q) [m][k]
__global__ __launch_bounds__(256) void k_gemm_prep_f16(const float* __restrict__ x, _Float16* __restrict__ xh, int m,
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
    uint2 out;
    out.x = (uint32_t)f32_to_f16(d * (float)(int8_t)(q & 0xff)) |
            ((uint32_t)f32_to_f16(d * (float)(int8_t)((q >> 8) & 0xff)) << 16);
    out.y = (uint32_t)f32_to_f16(d * (float)(int8_t)((q >> 16) & 0xff)) |
            ((uint32_t)f32_to_f16(d * (float)(int8_t)(q >> 24)) << 16);
    *(uint2*)(xh + (int64_t)mi * k + sb * 256 + 4 * lane) = out;
}

constexpr int H_BM = 128, H_BN = 128, H_BK = 64;
constexpr int H_THREADS = 256;
constexpr int H_TILE = H_BM * H_BK * 2;  // bytes of one A (or B) stage: 16 KB
// LDS stage = A tile then B tile, each [128 rows][8 pieces of 8 halves],
// piece p of row r at position p ^ (r & 7).
__device__ __forceinline__ int h_pos(int row, int piece) { return row * 128 + 16 * (piece ^ (row & 7)); }

__global__ __launch_bounds__(H_THREADS) void k_gemm_q4k_f16(const uint8_t* __restrict__ W,
                                                            const _Float16* __restrict__ xh, float* __restrict__ Y,
                                                            int m, int n, int k) {
    __shared__ __align__(16) uint8_t smem[2][2 * H_TILE];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5, c32 = lane & 31;
    int bm, bn;
    tile_of((m + H_BM - 1) / H_BM, (n + H_BN - 1) / H_BN, bm, bn);
    const int m0 = bm * H_BM, n0 = bn * H_BN;
    const int nsteps = k / H_BK;
    const int64_t rowbytes = (int64_t)(k >> 8) * Q4K_BYTES;

    // weight dequant role: thread -> (row, half of the 32 qs bytes of a chunk)
    const int brow = t >> 1, bhalf = t & 1;
    const uint8_t* wrow = W + (int64_t)min(n0 + brow, n - 1) * rowbytes;
    // activation DMA role: wave w moves chunks 4w..4w+3 (8 rows x 8 pieces each)
    auto issue_a = [&](uint8_t* stage, int step) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = wave * 4 + i;
            const int row = 8 * q + (lane >> 3);
            const int piece = (lane & 7) ^ (row & 7);
            const int grow = min(m0 + row, m - 1);
            __builtin_amdgcn_global_load_lds(xh + (int64_t)grow * k + step * H_BK + 8 * piece,
                                             (__attribute__((address_space(3))) void*)(stage + 1024 * q), 16, 0, 0);
        }
    };
    auto dequant_b = [&](uint8_t* stage, const uint4& hdr, const uint4& raw, int step) {
        const int c = step & 3;
        const float d = f16_to_f32(hdr.x & 0xffffu), dmin = f16_to_f32(hdr.x >> 16);
        int sc0, m0s, sc1, m1s;
        if (c < 2) {
            sc0 = byte_of(hdr.y, 2 * c) & 63;
            m0s = byte_of(hdr.z, 2 * c) & 63;
            sc1 = byte_of(hdr.y, 2 * c + 1) & 63;
            m1s = byte_of(hdr.z, 2 * c + 1) & 63;
        } else {
            const uint32_t i0 = 2 * c - 4, i1 = 2 * c - 3;
            sc0 = (byte_of(hdr.w, i0) & 0xF) | ((byte_of(hdr.y, i0) >> 6) << 4);
            m0s = (byte_of(hdr.w, i0) >> 4) | ((byte_of(hdr.z, i0) >> 6) << 4);
            sc1 = (byte_of(hdr.w, i1) & 0xF) | ((byte_of(hdr.y, i1) >> 6) << 4);
            m1s = (byte_of(hdr.w, i1) >> 4) | ((byte_of(hdr.z, i1) >> 6) << 4);
        }
        const float d1 = d * (float)sc0, mm1 = dmin * (float)m0s;
        const float d2 = d * (float)sc1, mm2 = dmin * (float)m1s;
        const uint32_t R[4] = {raw.x, raw.y, raw.z, raw.w};
        uint32_t lo[8], hi[8];  // 16 halves each, packed in pairs
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t wl = R[i] & 0x0F0F0F0Fu, wh = (R[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const _Float16 l0 = (_Float16)(d1 * (float)byte_of(wl, e) - mm1);
                const _Float16 l1 = (_Float16)(d1 * (float)byte_of(wl, e + 1) - mm1);
                const _Float16 h0 = (_Float16)(d2 * (float)byte_of(wh, e) - mm2);
                const _Float16 h1 = (_Float16)(d2 * (float)byte_of(wh, e + 1) - mm2);
                lo[2 * i + e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
                hi[2 * i + e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            }
        }
        uint8_t* B = stage + H_TILE;
        // sub-block 2c -> k 0..31 (pieces 0..3), sub-block 2c+1 -> k 32..63 (pieces 4..7)
        *(uint4*)(B + h_pos(brow, 2 * bhalf)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint4*)(B + h_pos(brow, 2 * bhalf + 1)) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        *(uint4*)(B + h_pos(brow, 4 + 2 * bhalf)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4*)(B + h_pos(brow, 4 + 2 * bhalf + 1)) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    };

    v16f acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][b][r] = 0.0f;

    uint4 hdr = *(const uint4*)wrow;
    uint4 raw = *(const uint4*)(wrow + 16 + 16 * bhalf);
    issue_a(smem[0], 0);
    dequant_b(smem[0], hdr, raw, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    for (int s = 0; s < nsteps; s++) {
        const uint8_t* A = smem[s & 1];
        const uint8_t* B = smem[s & 1] + H_TILE;
        // operands of this step, LDS -> registers, before the next stage is queued
        v8h av[2][4], bv[2][4];
#pragma unroll
        for (int a = 0; a < 2; a++) {
            const int row = wm * 64 + a * 32 + c32;
#pragma unroll
            for (int kk = 0; kk < 4; kk++) av[a][kk] = *(const v8h*)(A + h_pos(row, 2 * kk + h));
        }
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int row = wn * 64 + b * 32 + c32;
#pragma unroll
            for (int kk = 0; kk < 4; kk++) bv[b][kk] = *(const v8h*)(B + h_pos(row, 2 * kk + h));
        }
        const bool more = s + 1 < nsteps;
        if (more) {
            issue_a(smem[(s + 1) & 1], s + 1);
            const int sb = (s + 1) >> 2, c = (s + 1) & 3;
            if (c == 0) hdr = *(const uint4*)(wrow + sb * Q4K_BYTES);
            raw = *(const uint4*)(wrow + sb * Q4K_BYTES + 16 + 32 * c + 16 * bhalf);
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[a][kk], bv[b][kk], acc[a][b], 0, 0, 0);
        if (more) dequant_b(smem[(s + 1) & 1], hdr, raw, s + 1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int col = n0 + wn * 64 + b * 32 + c32;
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * 64 + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < m) Y[(int64_t)row * n + col] = acc[a][b][r];
            }
        }
}

// ------------------------------------------------------------ dispatch --

size_t gemm_workspace_bytes(int type, int64_t k, int64_t m, int mode) {
    if (type == T_Q4K) {
        const size_t f16 = ((size_t)m * k * 2 + 255) & ~(size_t)255;
        return mode == GEMM_INT8 ? prep_bytes(m, k) : f16;
    }
    return matvec_workspace_bytes(type, k, 16);
}

hipError_t launch_gemm(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                       void* qbuf, int mode, hipStream_t s) {
    if (type == T_Q4K && mode != GEMM_INT8) {
        _Float16* xh = (_Float16*)qbuf;
        const int64_t nb = m * (k / 256);
        hipLaunchKernelGGL(k_gemm_prep_f16, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x, xh, (int)m, (int)k);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const unsigned grid = (unsigned)(((m + H_BM - 1) / H_BM) * ((n + H_BN - 1) / H_BN));
        hipLaunchKernelGGL(k_gemm_q4k_f16, dim3(grid), dim3(H_THREADS), 0, s, (const uint8_t*)w, xh, y, (int)m,
                           (int)n, (int)k);
        return hipGetLastError();
    }
    if (type == T_Q4K) {
        static bool attr_set = false;
        if (!attr_set) {
            hipError_t e = hipFuncSetAttribute((const void*)k_gemm_q4k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               G_LDS);
            if (e != hipSuccess) return e;
            attr_set = true;
        }
        PrepPtrs p = prep_ptrs(qbuf, m, k);
        const int64_t nb = m * (k / 256);
        hipLaunchKernelGGL(k_gemm_prep_q8k, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x, p.xq, p.sp, p.dyt,
                           (int)m, (int)k);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const unsigned grid = (unsigned)(((m + G_BM - 1) / G_BM) * ((n + G_BN - 1) / G_BN));
        hipLaunchKernelGGL(k_gemm_q4k, dim3(grid), dim3(G_THREADS), G_LDS, s, (const uint8_t*)w, p.xq, p.sp, p.dyt,
                           y, (int)m, (int)n, (int)k);
        return hipGetLastError();
    }
    // Q8_0 / Q6_K: tiles of 16 activation rows through the decode kernels
    for (int64_t r = 0; r < m; r += 16) {
        const int64_t mm = m - r < 16 ? m - r : 16;
        hipError_t e = launch_matvec(type, w, x + r * k, y + r * n, n, k, mm, qbuf, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lloom
