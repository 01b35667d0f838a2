// gemm_q8.hip -- Q8_0 matmul from five activation rows up (prefill and
// batched decode) on int8 MFMA.  Built with the MFMA results in VGPRs (-amdgpu-mfma-vgpr-form):
// every result is read by the VALU epilogue right away, and from AGPRs each
// read would cost one more instruction.
#include <cstdlib>
#include <type_traits>

#include "kq_common.hpp"
#include "kq_gemm.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"

namespace lloom {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ------------------------------------------------------ Q8_0 GEMM ----
// y[m, n] = sum_b (sum_{k in b} x8[m,k] w8[n,k]) * dx[m,b] * dw[n,b] over
// 32-element blocks b: k_quants' Q8_0 x Q8_0 dot (vec_dot_unopt,
// k_quants.rs:800-818) with the activations quantized by
// BlockQ8_0::from_float (k_quants.rs:738-767) and both scales taken as
// f32(f16 d), as the reference does.  One v_mfma_i32_32x32x32_i8 is one block
// of one 32 x 32 tile (its K is the block's 32), so every block's integer sum
// is exact and the scales apply per block in f32: out += f32(S) * (dx * dw).
// The tile's dx * dw products come from the matrix core too (a K = 2 f32
// MFMA, below), which leaves two VALU instructions per output and block,
// convert and fma.  Measured at m = 2048 on [8192, 2048], VALU and MFMA
// work do not overlap much here: 41.7 M VALU and 100.7 M MFMA-busy cycles a
// call (3 VALU: 57.4 M and 33.6 M) take the same ~155 us.
//
// Activation prep (bit-exact Q8_0, the weights' own block layout stays):
//   xq  int8 [m][k]
//   dxt f32  [k/32][mp]   mp = m rounded up to 4, then 128 floats of pad
struct Q8Ptrs {
    int8_t* xq;
    float* dxt;
    int64_t mp;
};

static Q8Ptrs q8_ptrs(void* base, int64_t m, int64_t k) {
    Q8Ptrs p;
    p.xq = (int8_t*)base;
    p.dxt = (float*)((uint8_t*)base + (((size_t)m * k + 255) & ~(size_t)255));
    p.mp = (m + 3) & ~(int64_t)3;
    return p;
}

static size_t q8_prep_bytes(int64_t m, int64_t k) {
    const int64_t mp = (m + 3) & ~(int64_t)3;
    return (((size_t)m * k + 255) & ~(size_t)255) +
           ((((size_t)(k / 32) * mp + 128) * sizeof(float) + 255) & ~(size_t)255);
}

// One wave a (row, 256 elements): eight blocks of eight lanes.
__global__ __launch_bounds__(256) void k_gemm_prep_q8_0(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                        float* __restrict__ dxt, int m, int k, int mp) {
    const int lane = threadIdx.x & 63;
    const int nc = k >> 8;
    const int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (c >= (int64_t)m * nc) return;
    const int mi = (int)(c / nc), cc = (int)(c - (int64_t)mi * nc);
    const int64_t off = (int64_t)mi * k + 256 * cc + 4 * lane;
    const float4 v = *(const float4*)(x + off);
    uint16_t d16;
    const uint32_t q = q8_0_block_8lanes(v, &d16);
    *(uint32_t*)(xq + off) = q;
    if ((lane & 7) == 0) dxt[(int64_t)(8 * cc + (lane >> 3)) * mp + mi] = f16_to_f32(d16);
}

// Tiling: WM x WN waves, each MT x NT tiles of 32 x 32: a BM x BN block of
// y (BM = 32 WM MT, BN = 32 WN NT).  K moves in steps of 256 (eight blocks,
// 272 weight bytes a row: 16-byte aligned, as a row of blocks is 2176
// bytes), one LDS stage a step, a ring of S stages, every byte by
// global_load_lds:
//   A  [BM][256] int8, piece p (16 B) of row r at p ^ (r & 7)
//   B  [BN][272] the raw Q8_0 bytes of the step (17 pieces a row; odd, so
//      eight consecutive rows reading one piece hit eight bank groups)
//   DX [8][BM] f32, the step's activation scales
// Every wave issues the same number of loads a stage (a wave past the
// last chunk of a part repeats one: the same bytes to the same place), so
// a counted vmcnt wait before each barrier leaves exactly the later stages
// in flight.
// MFMA operands (the same k-set for A and B in a lane): lane l holds row
// (or column) l % 32, elements 16 (l / 32) .. +15 of the block.  A block's
// 32 quants start 2 bytes into its 34, so a lane reads the aligned 32-byte
// window around its 16 bytes and shifts them out with v_alignbyte.
template <int WM_, int WN_, int MT_, int NT_, int S_>
struct Q8Cfg {
    static constexpr int WM = WM_, WN = WN_, MT = MT_, NT = NT_, S = S_;
    static constexpr int WAVES = WM * WN, THREADS = 64 * WAVES;
    static constexpr int BM = 32 * WM * MT, BN = 32 * WN * NT;
    static constexpr int A = BM * 256, B = BN * 272, DX = 8 * BM * 4;
    static constexpr int STAGE = A + B + DX, LDS = S * STAGE;
    static constexpr int A_CHUNKS = A / 1024, B_CHUNKS = (B + 1023) / 1024, DX_CHUNKS = DX / 1024;
    static constexpr int A_PER_WAVE = A_CHUNKS / WAVES;
    static constexpr int B_PER_WAVE = (B_CHUNKS + WAVES - 1) / WAVES;
    static constexpr int DX_PER_WAVE = (DX_CHUNKS + WAVES - 1) / WAVES;
    static constexpr int DMA = A_PER_WAVE + B_PER_WAVE + DX_PER_WAVE;  // loads a wave issues a stage
    static_assert(A_CHUNKS % WAVES == 0 && B % 1024 == 0 && DX % 1024 == 0, "stage parts in whole 1 KB chunks");
    static_assert((S - 2) * DMA <= 63, "vmcnt counts to 63");
    static_assert(LDS <= 160 * 1024, "LDS");
};

// The lane's 16 quants of block j (h: which half) from row base rb (LDS),
// a 16-byte-aligned window: the block's quants start at 34 j + 2.
template <int J>
__device__ __forceinline__ v4i q8_operand(const uint8_t* rb, int h) {
    constexpr int START = 34 * J + 2, BASE = START & ~15, SH = START - BASE, Q = SH >> 2, R = SH & 3;
    const uint8_t* p = rb + BASE + 16 * h;
    const uint4 lo = *(const uint4*)p;
    if constexpr (SH == 0) {
        return __builtin_bit_cast(v4i, lo);
    } else {
        const uint4 hi = *(const uint4*)(p + 16);
        const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        v4i r;
#pragma unroll
        for (int i = 0; i < 4; i++)
            r[i] = R == 0 ? (int)w[Q + i] : (int)__builtin_amdgcn_alignbyte(w[Q + i + 1], w[Q + i], R);
        return r;
    }
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <class C>
__global__ __launch_bounds__(C::THREADS) void k_gemm_q8_0(const uint8_t* __restrict__ W,
                                                            const int8_t* __restrict__ xq,
                                                            const float* __restrict__ dxt, float* __restrict__ Y,
                                                            int m, int n, int k, int mp, int epi) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / C::WN, wn = wave % C::WN;
    const int h = lane >> 5, c32 = lane & 31;
    int bm, bn;
    tile_of((m + C::BM - 1) / C::BM, (n + C::BN - 1) / C::BN, bm, bn);
    const int m0 = bm * C::BM, n0 = bn * C::BN;
    const int nsteps = k >> 8;
    const uint32_t rowbytes = (uint32_t)(k / 32) * Q8_0_BYTES;

    // per-lane byte offsets of this wave's DMA share, fixed for the K loop
    uint32_t aoff[C::A_PER_WAVE];
#pragma unroll
    for (int i = 0; i < C::A_PER_WAVE; i++) {
        const int q = wave * C::A_PER_WAVE + i;
        const int row = 4 * q + (lane >> 4);
        const int piece = (lane & 15) ^ (row & 7);
        aoff[i] = (uint32_t)min(m0 + row, m - 1) * (uint32_t)k + 16u * piece;
    }
    uint32_t boff[C::B_PER_WAVE];
#pragma unroll
    for (int i = 0; i < C::B_PER_WAVE; i++) {
        const int q = min(wave + C::WAVES * i, C::B_CHUNKS - 1);
        const int pc = 64 * q + lane;
        const int row = pc / 17, piece = pc - row * 17;
        boff[i] = (uint32_t)min(n0 + row, n - 1) * rowbytes + 16u * piece;
    }
    // DX chunk c: BM / 4 lanes a block (four rows each), 256 / BM blocks
    uint32_t dxoff[C::DX_PER_WAVE];
#pragma unroll
    for (int i = 0; i < C::DX_PER_WAVE; i++) {
        constexpr int LPB = C::BM / 4;
        const int c = min(wave + C::WAVES * i, C::DX_CHUNKS - 1);
        const int blk = c * (64 / LPB) + lane / LPB;
        dxoff[i] = ((uint32_t)blk * (uint32_t)mp + (uint32_t)(m0 + 4 * (lane % LPB))) * 4u;
    }
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds0 = lds_addr(smem);

    auto issue = [&](int s, int slot) {
        const uint32_t st = lds0 + slot * C::STAGE;
        const uint8_t* ab = (const uint8_t*)xq + (uint32_t)s * 256u;
#pragma unroll
        for (int i = 0; i < C::A_PER_WAVE; i++) dma16s(ab, aoff[i], st + 1024 * (wv * C::A_PER_WAVE + i));
        const uint8_t* bb = W + (uint32_t)s * 272u;
#pragma unroll
        for (int i = 0; i < C::B_PER_WAVE; i++)
            dma16s(bb, boff[i], st + C::A + 1024 * min(wv + C::WAVES * i, C::B_CHUNKS - 1));
        const uint8_t* db = (const uint8_t*)(dxt + (int64_t)s * 8 * mp);
#pragma unroll
        for (int i = 0; i < C::DX_PER_WAVE; i++)
            dma16s(db, dxoff[i], st + C::A + C::B + 1024 * min(wv + C::WAVES * i, C::DX_CHUNKS - 1));
    };

    float out[C::MT][C::NT][16];
#pragma unroll
    for (int a = 0; a < C::MT; a++)
#pragma unroll
        for (int b = 0; b < C::NT; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) out[a][b][r] = 0.0f;

    // prologue: stages 0 .. S-2 (steps past the end reload the last one
    // into a slot nobody reads, so the counts never change)
#pragma unroll
    for (int i = 0; i < C::S - 1; i++) issue(min(i, nsteps - 1), i);
    __builtin_amdgcn_sched_barrier(0);
    vm_wait<(C::S - 2) * C::DMA>();
    __builtin_amdgcn_s_barrier();

    for (int s = 0; s < nsteps; s++) {
        // step s + S - 1 into the slot step s - 1 used (its readers passed
        // the last barrier)
        issue(min(s + C::S - 1, nsteps - 1), (s + C::S - 1) % C::S);
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* A = smem + (s % C::S) * C::STAGE;
        const uint8_t* B = A + C::A;
        const float* DX = (const float*)(B + C::B);
        const uint8_t* brow[C::NT];
#pragma unroll
        for (int b = 0; b < C::NT; b++) brow[b] = B + (wn * 32 * C::NT + b * 32 + c32) * 272;
        auto block = [&](auto jc) {
            constexpr int j = decltype(jc)::value;
            v4i av[C::MT], bv[C::NT];
            float dw[C::NT];
#pragma unroll
            for (int a = 0; a < C::MT; a++) {
                const int row = wm * 32 * C::MT + a * 32 + c32;
                av[a] = *(const v4i*)(A + row * 256 + 16 * ((2 * j + h) ^ (row & 7)));
            }
#pragma unroll
            for (int b = 0; b < C::NT; b++) {
                bv[b] = q8_operand<j>(brow[b], h);
                dw[b] = f16_to_f32(*(const uint16_t*)(brow[b] + 34 * j));
            }
            v16i d[C::MT][C::NT];
#pragma unroll
            for (int a = 0; a < C::MT; a++)
#pragma unroll
                for (int b = 0; b < C::NT; b++) {
                    const v16i z = {};
                    d[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a], bv[b], z, 0, 0, 0);
                }
            // the scale products dx * dw of the tile, on the matrix core: a
            // K = 2 f32 MFMA whose two k-slots (lanes 0-31, 32-63) both hold
            // the lane's row scale and column scale gives 2 dx dw, exactly
            // (two products of 11-bit significands, summed), in the layout
            // of the integer sums; the factor 2 leaves with one exact
            // halving at the store
            v16f p2[C::MT][C::NT];
#pragma unroll
            for (int a = 0; a < C::MT; a++) {
                const float dxl = DX[j * C::BM + wm * 32 * C::MT + a * 32 + c32];
#pragma unroll
                for (int b = 0; b < C::NT; b++) {
                    const v16f zf = {};
                    p2[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(dxl, dw[b], zf, 0, 0, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int a = 0; a < C::MT; a++)
#pragma unroll
                for (int b = 0; b < C::NT; b++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        out[a][b][r] = __builtin_fmaf((float)d[a][b][r], p2[a][b][r], out[a][b][r]);
        };
        block(std::integral_constant<int, 0>{});
        block(std::integral_constant<int, 1>{});
        block(std::integral_constant<int, 2>{});
        block(std::integral_constant<int, 3>{});
        block(std::integral_constant<int, 4>{});
        block(std::integral_constant<int, 5>{});
        block(std::integral_constant<int, 6>{});
        block(std::integral_constant<int, 7>{});
        // step s + 1 has landed (this wave's share; S - 2 later stages stay
        // in flight) and every wave is done reading step s
        __builtin_amdgcn_sched_barrier(0);
        vm_wait<(C::S - 2) * C::DMA>();
        __builtin_amdgcn_s_barrier();
    }
#pragma unroll
    for (int a = 0; a < C::MT; a++)
#pragma unroll
        for (int b = 0; b < C::NT; b++) {
            const int col = n0 + wn * 32 * C::NT + b * 32 + c32;
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * 32 * C::MT + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                const float v = 0.5f * out[a][b][r];
                if (row < m) {
                    if (epi == EPI_STORE) Y[(int64_t)row * n + col] = v;
                    else store_epi_slow(&Y[(int64_t)row * n + col], v, epi);
                }
            }
        }
}

// ------------------------------------------------- few rows: split K --
// For a few dozen activation rows the tiles above leave most CUs idle and
// each wave's block chain (LDS reads, MFMA, epilogue) runs unhidden.  Here a
// workgroup owns a BM x BN block of y (MT x NT tiles of 32 x 32) and its KS
// waves split K: wave w takes steps w, w + KS, ..., each through its own
// ring of S stages (no barrier inside the loop), and the KS partial sums
// meet in LDS in wave order at the end.  Per step and block the arithmetic
// is k_gemm_q8_0's.
template <int KS_, int MT_, int NT_, int S_>
struct Q8KCfg {
    static constexpr int KS = KS_, MT = MT_, NT = NT_, S = S_;
    static constexpr int THREADS = 64 * KS;
    static constexpr int BM = 32 * MT, BN = 32 * NT;
    static constexpr int A = BM * 256, B = ((BN * 272 + 1023) / 1024) * 1024, DX = 8 * BM * 4;
    static constexpr int STAGE = A + B + DX;
    static constexpr int A_CHUNKS = A / 1024, B_CHUNKS = B / 1024, DX_CHUNKS = DX / 1024;
    static constexpr int DMA = A_CHUNKS + B_CHUNKS + DX_CHUNKS;  // loads a wave issues a stage
    static constexpr int RED = KS * MT * NT * 16 * 64 * 4;       // the partial sums
    static constexpr int LDS = KS * S * STAGE > RED ? KS * S * STAGE : RED;
    static_assert(DX % 1024 == 0, "DX in whole chunks");
    static_assert((S - 1) * DMA <= 63, "vmcnt counts to 63");
    static_assert(LDS <= 160 * 1024, "LDS");
};

template <class C>
__global__ __launch_bounds__(C::THREADS) void k_gemm_q8_0_splitk(const uint8_t* __restrict__ W,
                                                                   const int8_t* __restrict__ xq,
                                                                   const float* __restrict__ dxt,
                                                                   float* __restrict__ Y, int m, int n, int k, int mp,
                                                                   int epi) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int h = lane >> 5, c32 = lane & 31;
    const int m0 = blockIdx.y * C::BM, n0 = blockIdx.x * C::BN;
    const int nsteps = k >> 8;
    const uint32_t rowbytes = (uint32_t)(k / 32) * Q8_0_BYTES;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int mine = nsteps > wv ? (nsteps - wv + C::KS - 1) / C::KS : 0;  // this wave's steps (uniform)

    // per-lane byte offsets of a stage (the wave loads the whole stage)
    uint32_t aoff[C::A_CHUNKS];
#pragma unroll
    for (int q = 0; q < C::A_CHUNKS; q++) {
        const int row = 4 * q + (lane >> 4);
        const int piece = (lane & 15) ^ (row & 7);
        aoff[q] = (uint32_t)min(m0 + row, m - 1) * (uint32_t)k + 16u * piece;
    }
    uint32_t boff[C::B_CHUNKS];
#pragma unroll
    for (int q = 0; q < C::B_CHUNKS; q++) {
        const int pc = min(64 * q + lane, C::BN * 17 - 1);  // lanes past the last piece repeat it
        const int row = pc / 17, piece = pc - row * 17;
        boff[q] = (uint32_t)min(n0 + row, n - 1) * rowbytes + 16u * piece;
    }
    uint32_t dxoff[C::DX_CHUNKS];
#pragma unroll
    for (int c = 0; c < C::DX_CHUNKS; c++) {
        constexpr int LPB = C::BM / 4;
        const int blk = c * (64 / LPB) + lane / LPB;
        dxoff[c] = ((uint32_t)blk * (uint32_t)mp + (uint32_t)(m0 + 4 * (lane % LPB))) * 4u;
    }
    const uint32_t ring = lds_addr(smem) + (uint32_t)wv * (C::S * C::STAGE);
    const uint8_t* ringp = smem + wave * (C::S * C::STAGE);

    // the wave's i-th step into slot i % S (past its last step: the last one again)
    auto issue = [&](int i) {
        const int s = wv + C::KS * min(i, mine - 1);
        const uint32_t st = ring + (i % C::S) * C::STAGE;
        const uint8_t* ab = (const uint8_t*)xq + (uint32_t)s * 256u;
#pragma unroll
        for (int q = 0; q < C::A_CHUNKS; q++) dma16s(ab, aoff[q], st + 1024 * q);
        const uint8_t* bb = W + (uint32_t)s * 272u;
#pragma unroll
        for (int q = 0; q < C::B_CHUNKS; q++) dma16s(bb, boff[q], st + C::A + 1024 * q);
        const uint8_t* db = (const uint8_t*)(dxt + (int64_t)s * 8 * mp);
#pragma unroll
        for (int c = 0; c < C::DX_CHUNKS; c++) dma16s(db, dxoff[c], st + C::A + C::B + 1024 * c);
    };

    float out[C::MT][C::NT][16];
#pragma unroll
    for (int a = 0; a < C::MT; a++)
#pragma unroll
        for (int b = 0; b < C::NT; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) out[a][b][r] = 0.0f;

    if (mine > 0) {
#pragma unroll
        for (int i = 0; i < C::S - 1; i++) issue(i);
        for (int i = 0; i < mine; i++) {
            issue(i + C::S - 1);
            __builtin_amdgcn_sched_barrier(0);
            vm_wait<(C::S - 1) * C::DMA>();
            const uint8_t* A = ringp + (i % C::S) * C::STAGE;
            const uint8_t* B = A + C::A;
            const float* DX = (const float*)(B + C::B);
            const uint8_t* brow[C::NT];
#pragma unroll
            for (int b = 0; b < C::NT; b++) brow[b] = B + (b * 32 + c32) * 272;
            auto block = [&](auto jc) {
                constexpr int j = decltype(jc)::value;
                v4i av[C::MT], bv[C::NT];
                float dw[C::NT];
#pragma unroll
                for (int a = 0; a < C::MT; a++) {
                    const int row = a * 32 + c32;
                    av[a] = *(const v4i*)(A + row * 256 + 16 * ((2 * j + h) ^ (row & 7)));
                }
#pragma unroll
                for (int b = 0; b < C::NT; b++) {
                    bv[b] = q8_operand<j>(brow[b], h);
                    dw[b] = f16_to_f32(*(const uint16_t*)(brow[b] + 34 * j));
                }
                v16i d[C::MT][C::NT];
#pragma unroll
                for (int a = 0; a < C::MT; a++)
#pragma unroll
                    for (int b = 0; b < C::NT; b++) {
                        const v16i z = {};
                        d[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a], bv[b], z, 0, 0, 0);
                    }
#pragma unroll
                for (int a = 0; a < C::MT; a++) {
                    const float* dxp = DX + j * C::BM + a * 32 + 4 * h;
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const float4 d4 = *(const float4*)(dxp + 8 * g);
                        const float dxs[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const int r = 4 * g + u;
#pragma unroll
                            for (int b = 0; b < C::NT; b++)
                                out[a][b][r] = __builtin_fmaf((float)d[a][b][r], dxs[u] * dw[b], out[a][b][r]);
                        }
                    }
                }
            };
            block(std::integral_constant<int, 0>{});
            block(std::integral_constant<int, 1>{});
            block(std::integral_constant<int, 2>{});
            block(std::integral_constant<int, 3>{});
            block(std::integral_constant<int, 4>{});
            block(std::integral_constant<int, 5>{});
            block(std::integral_constant<int, 6>{});
            block(std::integral_constant<int, 7>{});
            __builtin_amdgcn_sched_barrier(0);
        }
        vm_wait<0>();  // the repeated loads past the last step
    }
    // partial sums meet in LDS (over the stages: every wave is past them)
    __syncthreads();
    float* red = (float*)smem;
#pragma unroll
    for (int a = 0; a < C::MT; a++)
#pragma unroll
        for (int b = 0; b < C::NT; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) red[(((wave * C::MT + a) * C::NT + b) * 16 + r) * 64 + lane] = out[a][b][r];
    __syncthreads();
    // wave w stores tiles w, w + KS, ... of the MT x NT, adding the waves in order
    for (int tt = wave; tt < C::MT * C::NT; tt += C::KS) {
        const int a = tt / C::NT, b = tt % C::NT;
        const int col = n0 + b * 32 + c32;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < C::KS; w++) v += red[(((w * C::MT + a) * C::NT + b) * 16 + r) * 64 + lane];
            const int row = m0 + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (row < m && col < n) store_epi(&Y[(int64_t)row * n + col], v, epi);
        }
    }
}

template <class C>
static hipError_t launch_q8k_cfg(const void* w, const Q8Ptrs& p, float* y, int64_t n, int64_t k, int64_t m, int epi,
                                 hipStream_t s) {
    if (hipError_t e = set_lds_limit((const void*)k_gemm_q8_0_splitk<C>, C::LDS)) return e;
    const dim3 grid((unsigned)((n + C::BN - 1) / C::BN), (unsigned)((m + C::BM - 1) / C::BM));
    hipLaunchKernelGGL(k_gemm_q8_0_splitk<C>, grid, dim3(C::THREADS), C::LDS, s, (const uint8_t*)w, p.xq, p.dxt, y,
                       (int)m, (int)n, (int)k, (int)p.mp, epi);
    return hipGetLastError();
}

// K in whole 256-element steps and 32-bit DMA offsets.
bool q8_gemm_fits(int64_t n, int64_t k, int64_t m) {
    return k % 256 == 0 && n * (k / 32) * Q8_0_BYTES < ((int64_t)1 << 32) && m * k < ((int64_t)1 << 32);
}

template <class C>
static hipError_t launch_q8_cfg(const void* w, const Q8Ptrs& p, float* y, int64_t n, int64_t k, int64_t m, int epi,
                                hipStream_t s) {
    if (hipError_t e = set_lds_limit((const void*)k_gemm_q8_0<C>, C::LDS)) return e;
    const unsigned grid = (unsigned)(((m + C::BM - 1) / C::BM) * ((n + C::BN - 1) / C::BN));
    hipLaunchKernelGGL(k_gemm_q8_0<C>, dim3(grid), dim3(C::THREADS), C::LDS, s, (const uint8_t*)w, p.xq, p.dxt, y,
                       (int)m, (int)n, (int)k, (int)p.mp, epi);
    return hipGetLastError();
}

// LLOOM_HIP_Q8_TILE (read once) picks the tile for tuning; -1 (default)
// chooses by m.
static int q8_tile_env() {
    static const int v = [] {
        const char* e = getenv("LLOOM_HIP_Q8_TILE");
        return e ? atoi(e) : -1;
    }();
    return v;
}

size_t q8_gemm_workspace_bytes(int64_t m, int64_t k) { return q8_prep_bytes(m, k); }

hipError_t launch_q8_gemm(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* qbuf,
                          size_t ws_cap, int epi, hipStream_t s) {
    if (q8_prep_bytes(m, k) > ws_cap) return hipErrorInvalidValue;
    const Q8Ptrs p = q8_ptrs(qbuf, m, k);
    const int64_t nc = m * (k / 256);
    hipLaunchKernelGGL(k_gemm_prep_q8_0, dim3((unsigned)((nc + 3) / 4)), dim3(256), 0, s, x, p.xq, p.dxt, (int)m,
                       (int)k, (int)p.mp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // by m (measured on [8192, 2048], graph replay with the prep launch):
    // to 32 rows 32 x 32 blocks with K split over 8 waves (m = 9..32
    // 11.5-12.7 us, against 25-26 for the best output tiling); to 144 the
    // same over 4 waves (m = 64 15.3, m = 128 24.0 against 26.6 and 28.3;
    // m = 160 30.5 against ~33);
    // to 384 64 x 128 tiles with 8 waves (m = 256 34.2 against 41.4); past
    // that 128 x 128 with 8 waves (m = 512 46.2, 1024 87.0, 2048 166.6 us)
    int tile = q8_tile_env();
    if (tile < 0) tile = m <= 32 ? 10 : m <= 144 ? 15 : m <= 384 ? 6 : 0;
    switch (tile) {
        case 10: return launch_q8k_cfg<Q8KCfg<8, 1, 1, 1>>(w, p, y, n, k, m, epi, s);
        case 11: return launch_q8k_cfg<Q8KCfg<4, 1, 1, 2>>(w, p, y, n, k, m, epi, s);
        case 12: return launch_q8k_cfg<Q8KCfg<4, 1, 2, 1>>(w, p, y, n, k, m, epi, s);
        case 13: return launch_q8k_cfg<Q8KCfg<4, 2, 1, 1>>(w, p, y, n, k, m, epi, s);
        case 14: return launch_q8k_cfg<Q8KCfg<2, 1, 1, 3>>(w, p, y, n, k, m, epi, s);
        case 15: return launch_q8k_cfg<Q8KCfg<4, 1, 1, 1>>(w, p, y, n, k, m, epi, s);
        case 1: return launch_q8_cfg<Q8Cfg<2, 2, 2, 2, 2>>(w, p, y, n, k, m, epi, s);   // 128 x 128, 4 waves
        case 2: return launch_q8_cfg<Q8Cfg<2, 2, 1, 1, 4>>(w, p, y, n, k, m, epi, s);   // 64 x 64, 4 stages
        case 3: return launch_q8_cfg<Q8Cfg<1, 2, 1, 1, 4>>(w, p, y, n, k, m, epi, s);   // 32 x 64, 4 stages
        case 4: return launch_q8_cfg<Q8Cfg<1, 4, 2, 1, 2>>(w, p, y, n, k, m, epi, s);   // 64 x 128
        case 5: return launch_q8_cfg<Q8Cfg<1, 4, 2, 1, 3>>(w, p, y, n, k, m, epi, s);   // 64 x 128, 3 stages
        case 6: return launch_q8_cfg<Q8Cfg<2, 4, 1, 1, 3>>(w, p, y, n, k, m, epi, s);   // 64 x 128, 8 waves, 3 stages
        default: return launch_q8_cfg<Q8Cfg<2, 4, 2, 1, 2>>(w, p, y, n, k, m, epi, s);  // 128 x 128, 8 waves
    }
}

}  // namespace lloom
