// gemm_q6.hip -- Q6_K prefill-shaped matmul (from 48 activation rows) on int8
// MFMA.
//
// y[m, n] = sum_sb d[n,sb] * dy[m,sb] * sum_j sc[n,j] * sum_{k in j} x8[m,k] (q6[n,k] - 32)
// over superblocks sb and their 16 sub-blocks j: k_quants' Q6_K x Q8_K dot
// (vec_dot_unopt, k_quants.rs:2115-2172) with the activations quantized by
// BlockQ8K::from_float (k_quants.rs:2400-2438).  One v_mfma_i32_32x32x16_i8
// is one sub-block of one 32 x 32 tile (its K is the sub-block's 16), q6 - 32
// enters as int8 directly, the signed 8-bit scale multiplies the exact
// integer sum on the VALU (one v_mad_i32_i24 per output), and the f32
// d * dy applies once per superblock.  Every integer sum is exact.
//
// Built with the MFMA results in VGPRs (-amdgpu-mfma-vgpr-form): each is
// read by the VALU right away.
#include <cstdlib>
#include <type_traits>

#include "kq_common.hpp"
#include "kq_gemm.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"

namespace lloom {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

// Activation prep (Q8_K of every (row, superblock), bit-exact):
//   xq  int8 [m][k]
//   dyt f32  [k/256][mp]   mp = m rounded up to 4, then 128 floats of pad
struct Q6Ptrs {
    int8_t* xq;
    float* dyt;
    int64_t mp;
};

// (xq_rows >= m: rows of xq allocated, the two-plane route's tiles read
// whole 256-row blocks)
static Q6Ptrs q6_ptrs(void* base, int64_t m, int64_t k, int64_t xq_rows = 0) {
    Q6Ptrs p;
    p.xq = (int8_t*)base;
    p.dyt = (float*)((uint8_t*)base + (((size_t)(xq_rows > m ? xq_rows : m) * k + 255) & ~(size_t)255));
    p.mp = (m + 3) & ~(int64_t)3;
    return p;
}

static size_t q6_prep_bytes(int64_t m, int64_t k, int64_t xq_rows = 0) {
    const int64_t mp = (m + 3) & ~(int64_t)3;
    return (((size_t)(xq_rows > m ? xq_rows : m) * k + 255) & ~(size_t)255) + (((size_t)(k / 256) * mp + 128) * sizeof(float) + 255 & ~(size_t)255);
}


// Each 16-lane row of a wave quantizes one (row, superblock) block
// (q8k_block_row16: lane j holds elements 16j .. 16j+15, which are 16
// contiguous bytes of xq), RB blocks a row: a workgroup of W waves takes
// 4 W RB consecutive blocks of x ([m][k], so 4 W RB KB of contiguous input),
// every load issued first, two a row; calls with fewer blocks than fill the
// GPU with such workgroups take one block a wave (k_gemm_prep_q6_wave).
// (Block indices are 32-bit: m * k / 256 < 2^31.)
constexpr int64_t Q6_XPREP_RB2 = 256 * 32;  // blocks from which a row takes two
template <int RB, int W>
__device__ __forceinline__ void q6_prep_x(const float* __restrict__ x, int8_t* __restrict__ xq,
                                          float* __restrict__ dyt, int m, int k, int mp, uint32_t bid) {
    const int lane = threadIdx.x & 63, j = lane & 15;
    const uint32_t nsb = (uint32_t)k >> 8, nblk = (uint32_t)m * nsb;
    const uint32_t b0 = bid * (4 * W * RB) + 4 * (threadIdx.x >> 6) + (lane >> 4);
    float xs[RB][16];
#pragma unroll
    for (int r = 0; r < RB; r++) {
        const uint32_t blk = min(b0 + 4 * W * r, nblk - 1);  // past the end: a duplicate, not stored
        const float4* src = (const float4*)(x + (size_t)blk * 256 + 16 * j);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float4 v = src[u];
            xs[r][4 * u] = v.x;
            xs[r][4 * u + 1] = v.y;
            xs[r][4 * u + 2] = v.z;
            xs[r][4 * u + 3] = v.w;
        }
    }
#pragma unroll
    for (int r = 0; r < RB; r++) {
        const uint32_t blk = b0 + 4 * W * r;
        float d;
        int bs;
        const uint4 q = q8k_block_row16(xs[r], &d, &bs);  // every lane of the row: DPP inside
        if (blk < nblk) {
            *(uint4*)(xq + (size_t)blk * 256 + 16 * j) = q;
            const uint32_t mi = blk / nsb, sb = blk - mi * nsb;
            if (j == 0) dyt[(size_t)sb * mp + mi] = d;
        }
    }
}

template <int RB, int W>
__global__ __launch_bounds__(64 * W) void k_gemm_prep_q6(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                         float* __restrict__ dyt, int m, int k, int mp) {
    q6_prep_x<RB, W>(x, xq, dyt, m, k, mp, blockIdx.x);
}
// The same blocks, one a wave (its 64 lanes four elements each), for calls
// with few blocks: more waves, each with less to do.
__global__ __launch_bounds__(256) void k_gemm_prep_q6_wave(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                           float* __restrict__ dyt, int m, int k, int mp) {
    const int lane = threadIdx.x & 63;
    const uint32_t nsb = (uint32_t)k >> 8, nblk = (uint32_t)m * nsb;
    const uint32_t blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblk) return;
    const float4 v = *(const float4*)(x + (size_t)blk * 256 + 4 * lane);
    float d;
    int bs;
    const uint32_t q = q8k_block_wave(v, &d, &bs);
    *(uint32_t*)(xq + (size_t)blk * 256 + 4 * lane) = q;
    const uint32_t mi = blk / nsb, sb = blk - mi * nsb;
    if (lane == 0) dyt[(size_t)sb * mp + mi] = d;
}
// The launch for nb blocks.
static hipError_t launch_prep_q6(const float* x, int8_t* xq, float* dyt, int64_t m, int64_t k, int64_t mp, hipStream_t s) {
    const int64_t nb = m * (k / 256);
    if (nb >= Q6_XPREP_RB2)
        hipLaunchKernelGGL((k_gemm_prep_q6<2, 4>), dim3((unsigned)((nb + 31) / 32)), dim3(256), 0, s, x, xq, dyt,
                           (int)m, (int)k, (int)mp);
    else  // few blocks: one a wave (more waves in flight)
        hipLaunchKernelGGL(k_gemm_prep_q6_wave, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x, xq, dyt, (int)m,
                           (int)k, (int)mp);
    return hipGetLastError();
}

// Tiling: WM x WN waves, each MT x NT tiles of 32 x 32 (BM = 32 WM MT, BN =
// 32 WN NT).  K moves one superblock a step through a ring of S LDS stages,
// every byte by global_load_lds:
//   A  [BM][256] int8, sub-block j (16 B) of row r at position j ^ (r & 15)
//   B  [BN][240] the 16-byte-aligned window around each weight row's
//      superblock: Q6_K rows are 210 bytes a superblock, so the block sits
//      (row start + 210 sb) mod 16 bytes into its window (an even number);
//      224 bytes would hold it, 240 (15 pieces) puts the rows 60 dwords
//      apart, so 32 lanes reading one offset of their columns hit 16 banks
//      rather than 8 (LDS bank conflicts at m = 2048: 35 % of the cycles)
//   DY [BM] f32, the step's activation scales (one 1 KB chunk)
// Every wave issues the same number of loads a stage (a wave past the last
// chunk of a part repeats one), so a counted vmcnt wait before each
// barrier leaves exactly the later stages in flight.
// MFMA operands (the same k-set for A and B in a lane): lane l holds row
// (or column) l % 32, elements 8 (l / 32) .. +7 of the sub-block.
constexpr int Q6_PIECES = 15, Q6_WIN = 16 * Q6_PIECES;  // a row's window in LDS

template <int WM_, int WN_, int MT_, int NT_, int S_>
struct Q6Cfg {
    static constexpr int WM = WM_, WN = WN_, MT = MT_, NT = NT_, S = S_;
    static constexpr int WAVES = WM * WN, THREADS = 64 * WAVES;
    static constexpr int BM = 32 * WM * MT, BN = 32 * WN * NT;
    static constexpr int A = BM * 256, B = ((BN * Q6_WIN + 1023) / 1024) * 1024, DY = 1024;
    static constexpr int STAGE = A + B + DY, LDS = S * STAGE;
    static constexpr int A_CHUNKS = A / 1024, B_CHUNKS = B / 1024;
    static constexpr int A_PER_WAVE = A_CHUNKS / WAVES;
    static constexpr int B_PER_WAVE = (B_CHUNKS + WAVES - 1) / WAVES;
    static constexpr int DMA = A_PER_WAVE + B_PER_WAVE + 1;  // loads a wave issues a stage
    static_assert(A_CHUNKS % WAVES == 0, "A in whole chunks a wave");
    static_assert(BM <= 256, "DY in one chunk");
    static_assert((S - 2) * DMA <= 63, "vmcnt counts to 63");
    static_assert(LDS <= 160 * 1024, "LDS");
};

template <int N>
__device__ __forceinline__ void q6_vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Eight bytes at p + r2 (r2 = 0 or 2; p 4-byte aligned, LDS) as two dwords.
__device__ __forceinline__ uint2 lds8_shift(const uint8_t* p, uint32_t r2) {
    const uint32_t* q = (const uint32_t*)p;  // 4-byte aligned only
    const uint32_t a0 = q[0], a1 = q[1], a2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(a1, a0, r2), __builtin_amdgcn_alignbyte(a2, a1, r2));
}

// q6 - 32 as int8, four per dword: t = q6 ^ 32 is q6 - 32 in 6-bit two's
// complement; copying bit 5 into bits 6 and 7 sign-extends it.
__device__ __forceinline__ uint32_t q6_i8(uint32_t q6) {
    const uint32_t t = q6 ^ 0x20202020u;
    return t | ((t & 0x20202020u) * 6u);
}

template <class C>
__global__ __launch_bounds__(C::THREADS) void k_gemm_q6k(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                         const float* __restrict__ dyt, float* __restrict__ Y, int m,
                                                         int n, int k, int mp, int epi, int sps,
                                                         float* __restrict__ psum) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / C::WN, wn = wave % C::WN;
    const int h = lane >> 5, c32 = lane & 31;
    int bm, bn;
    tile_of((m + C::BM - 1) / C::BM, (n + C::BN - 1) / C::BN, bm, bn);
    const int m0 = bm * C::BM, n0 = bn * C::BN;
    const int nsb = k >> 8;
    const uint32_t rowbytes = (uint32_t)nsb * Q6K_BYTES;
    // split K (grid y): this workgroup's superblocks [s0, s0 + nsteps), its
    // sums to psum[split] for k_q6_sum_splits
    const int s0 = blockIdx.y * sps, nsteps = min(sps, nsb - s0);

    // per-lane DMA offsets (B: the row start; the window moves per step)
    uint32_t aoff[C::A_PER_WAVE];
#pragma unroll
    for (int i = 0; i < C::A_PER_WAVE; i++) {
        const int q = wave * C::A_PER_WAVE + i;
        const int row = 4 * q + (lane >> 4);
        const int piece = (lane & 15) ^ (row & 15);
        aoff[i] = (uint32_t)min(m0 + row, m - 1) * (uint32_t)k + 16u * piece;
    }
    uint32_t brs[C::B_PER_WAVE], bpc[C::B_PER_WAVE];
#pragma unroll
    for (int i = 0; i < C::B_PER_WAVE; i++) {
        const int q = min(wave + C::WAVES * i, C::B_CHUNKS - 1);
        const int pc = min(64 * q + lane, C::BN * Q6_PIECES - 1);
        const int row = pc / Q6_PIECES;
        brs[i] = (uint32_t)min(n0 + row, n - 1) * rowbytes;
        bpc[i] = 16u * (uint32_t)(pc - row * Q6_PIECES);
    }
    const uint32_t dyoff = (uint32_t)(m0 + 4 * min(lane, C::BM / 4 - 1)) * 4u;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds0 = lds_addr(smem);

    auto issue = [&](int i, int slot) {
        const int s = s0 + i;
        const uint32_t st = lds0 + slot * C::STAGE;
        const uint8_t* ab = (const uint8_t*)xq + (uint32_t)s * 256u;
#pragma unroll
        for (int i = 0; i < C::A_PER_WAVE; i++) dma16s(ab, aoff[i], st + 1024 * (wv * C::A_PER_WAVE + i));
        const uint32_t sb = (uint32_t)s * Q6K_BYTES;
#pragma unroll
        for (int i = 0; i < C::B_PER_WAVE; i++)
            dma16s(W, ((brs[i] + sb) & ~15u) + bpc[i], st + C::A + 1024 * min(wv + C::WAVES * i, C::B_CHUNKS - 1));
        dma16s((const uint8_t*)(dyt + (int64_t)s * mp), dyoff, st + C::A + C::B);
    };

    float out[C::MT][C::NT][16];
#pragma unroll
    for (int a = 0; a < C::MT; a++)
#pragma unroll
        for (int b = 0; b < C::NT; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) out[a][b][r] = 0.0f;
    // this lane's columns: row start (for the per-step shift) and LDS window
    uint32_t crs[C::NT];
#pragma unroll
    for (int b = 0; b < C::NT; b++) crs[b] = (uint32_t)min(n0 + wn * 32 * C::NT + b * 32 + c32, n - 1) * rowbytes;

#pragma unroll
    for (int i = 0; i < C::S - 1; i++) issue(min(i, nsteps - 1), i);
    __builtin_amdgcn_sched_barrier(0);
    q6_vm_wait<(C::S - 2) * C::DMA>();
    __builtin_amdgcn_s_barrier();

    for (int s = 0; s < nsteps; s++) {
        issue(min(s + C::S - 1, nsteps - 1), (s + C::S - 1) % C::S);
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* A = smem + (s % C::S) * C::STAGE;
        const uint8_t* B = A + C::A;
        const float* DY = (const float*)(B + C::B);
        // this lane's weight bytes of the superblock, per column tile b:
        //   ql[64 H + 32 G + 16 L + 8 h .. +8]  (H, G, L in 0..1) -> qlw[b][4H + 2G + L]
        //   qh[32 H + 16 L + 8 h .. +8]                          -> qhw[b][2H + L]
        //   scales[0 .. 16], d
        uint2 qlw[C::NT][8], qhw[C::NT][4];
        int scw[C::NT][4];
        float dw[C::NT];
#pragma unroll
        for (int b = 0; b < C::NT; b++) {
            const uint32_t sh = (crs[b] + (uint32_t)(s0 + s) * Q6K_BYTES) & 15u;
            const uint8_t* win = B + (wn * 32 * C::NT + b * 32 + c32) * Q6_WIN + (sh & ~3u);
            const uint32_t r2 = sh & 3u;
#pragma unroll
            for (int i = 0; i < 8; i++) qlw[b][i] = lds8_shift(win + 64 * (i >> 2) + 32 * ((i >> 1) & 1) + 16 * (i & 1) + 8 * h, r2);
#pragma unroll
            for (int i = 0; i < 4; i++) qhw[b][i] = lds8_shift(win + Q6K_QH + 32 * (i >> 1) + 16 * (i & 1) + 8 * h, r2);
            const uint2 s0 = lds8_shift(win + Q6K_SC, r2), s1 = lds8_shift(win + Q6K_SC + 8, r2);
            scw[b][0] = (int)s0.x;
            scw[b][1] = (int)s0.y;
            scw[b][2] = (int)s1.x;
            scw[b][3] = (int)s1.y;
            const uint32_t dd = *(const uint32_t*)(win + Q6K_D);
            dw[b] = f16_to_f32((dd >> (8 * r2)) & 0xffffu);
        }
        int acc[C::MT][C::NT][16];
        // sub-block j = 8 H + 2 g + L: elements 128 H + 32 g + 16 L + (0..16)
        auto sub = [&](auto jc) {
            constexpr int j = decltype(jc)::value;
            constexpr int H = j >> 3, g = (j >> 1) & 3, L = j & 1;
            long bv[C::NT];
            int sc[C::NT];
#pragma unroll
            for (int b = 0; b < C::NT; b++) {
                const uint2 ql = qlw[b][4 * H + 2 * (g & 1) + L], qh = qhw[b][2 * H + L];
                uint32_t w[2];
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const uint32_t lo = ((u ? ql.y : ql.x) >> (4 * (g >> 1))) & 0x0F0F0F0Fu;
                    const uint32_t hi = (((u ? qh.y : qh.x) >> (2 * g)) & 0x03030303u) << 4;
                    w[u] = q6_i8(lo | hi);
                }
                bv[b] = (long)(((uint64_t)w[1] << 32) | w[0]);
                sc[b] = (int)(int8_t)byte_of(scw[b][j >> 2], j & 3);
            }
#pragma unroll
            for (int a = 0; a < C::MT; a++) {
                const int row = wm * 32 * C::MT + a * 32 + c32;
                const long av = *(const long*)(A + row * 256 + 16 * (j ^ (row & 15)) + 8 * h);
#pragma unroll
                for (int b = 0; b < C::NT; b++) {
                    const v16i z = {};
                    const v16i d = __builtin_amdgcn_mfma_i32_32x32x16_i8(av, bv[b], z, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        if constexpr (j == 0) acc[a][b][r] = __mul24(sc[b], d[r]);
                        else acc[a][b][r] += __mul24(sc[b], d[r]);
                    }
                }
            }
        };
        sub(std::integral_constant<int, 0>{});
        sub(std::integral_constant<int, 1>{});
        sub(std::integral_constant<int, 2>{});
        sub(std::integral_constant<int, 3>{});
        sub(std::integral_constant<int, 4>{});
        sub(std::integral_constant<int, 5>{});
        sub(std::integral_constant<int, 6>{});
        sub(std::integral_constant<int, 7>{});
        sub(std::integral_constant<int, 8>{});
        sub(std::integral_constant<int, 9>{});
        sub(std::integral_constant<int, 10>{});
        sub(std::integral_constant<int, 11>{});
        sub(std::integral_constant<int, 12>{});
        sub(std::integral_constant<int, 13>{});
        sub(std::integral_constant<int, 14>{});
        sub(std::integral_constant<int, 15>{});
        // superblock epilogue: out += f32(acc) * (d * dy)
#pragma unroll
        for (int a = 0; a < C::MT; a++) {
            const float* dyp = DY + wm * 32 * C::MT + a * 32 + 4 * h;
#pragma unroll
            for (int gq = 0; gq < 4; gq++) {
                const float4 d4 = *(const float4*)(dyp + 8 * gq);
                const float dys[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int r = 4 * gq + u;
#pragma unroll
                    for (int b = 0; b < C::NT; b++)
                        out[a][b][r] = __builtin_fmaf((float)acc[a][b][r], dw[b] * dys[u], out[a][b][r]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        q6_vm_wait<(C::S - 2) * C::DMA>();
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
                if (row < m) {
                    if (psum) psum[((int64_t)blockIdx.y * m + row) * n + col] = out[a][b][r];
                    else if (epi == EPI_STORE) Y[(int64_t)row * n + col] = out[a][b][r];
                    else store_epi_slow(&Y[(int64_t)row * n + col], out[a][b][r], epi);
                }
            }
        }
}

// The split-K partial sums, added in split order, then the call's store
// epilogue; four consecutive outputs a thread (16-byte loads and stores
// where the four are in range and aligned, one at a time otherwise).
__global__ __launch_bounds__(256) void k_q6_sum_splits(const float* __restrict__ psum, int splits, int64_t mn,
                                                       float* __restrict__ Y, int epi) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (i >= mn) return;
    if (i + 4 <= mn && (mn & 3) == 0 && ((uintptr_t)Y & 15) == 0) {
        float4 v = *(const float4*)(psum + i);
        for (int z = 1; z < splits; z++) {
            const float4 u = *(const float4*)(psum + z * mn + i);
            v.x += u.x;
            v.y += u.y;
            v.z += u.z;
            v.w += u.w;
        }
        if (epi == EPI_STORE) {
            *(float4*)(Y + i) = v;
        } else {
            store_epi(&Y[i], v.x, epi);
            store_epi(&Y[i + 1], v.y, epi);
            store_epi(&Y[i + 2], v.z, epi);
            store_epi(&Y[i + 3], v.w, epi);
        }
        return;
    }
    for (int64_t t = i; t < min(i + 4, mn); t++) {
        float v = psum[t];
        for (int z = 1; z < splits; z++) v += psum[z * mn + t];
        store_epi(&Y[t], v, epi);
    }
}

// ------------------------------------------------ two-plane route ----
// From a few hundred rows the per-sub-block VALU work above (the scale
// multiply-add on every output, the per-lane weight realignment) bounds
// k_gemm_q6k.  Here a prep launch folds each weight's scale into it once a
// call: v = sc[e / 16] * (q6[e] - 32) lies in [-4096, 4096] and splits
// exactly as v = 64 hi + lo with lo in [-32, 31] and hi in [-64, 64], two
// int8 planes.  Then every superblock of every 32 x 32 tile is sixteen
// chained v_mfma_i32_32x32x32_i8 (eight 32-element chunks, two planes)
// whose sums are exact (|64 Dhi + Dlo| <= 256 * 128 * 4096 = 2^27), and the
// VALU work is four instructions an output and superblock: 64 hi + lo,
// convert, d * dy, fma.  The integer sum is the reference's per-superblock
// isum (sum_j sc_j sum_{k in j} x8 (q6 - 32)), the float part its
// d_x * d_w scaling (k_quants.rs:2115-2172).
//
// Weight prep (per call, into the workspace):
//   planes int8 [n][k/256][4][2][64]: superblock sb of column c is 512
//          bytes, quarter q (elements 64 q ..) at 128 q: hi plane then lo
//   dwt    f32 [k/256][np]  f32(d), np = n rounded up to 4, 128 floats of pad
struct Q6PPtrs {
    int8_t* planes;
    float* dwt;
    int64_t np;
};

// (columns rounded up to whole 128-column blocks, read by the last block)
static size_t q6p_plane_bytes(int64_t n, int64_t k) { return (size_t)((n + 127) & ~(int64_t)127) * 2 * k; }
static size_t q6p_dw_bytes(int64_t n, int64_t k) {
    const int64_t np = (n + 3) & ~(int64_t)3;
    return (((size_t)(k / 256) * np + 128) * sizeof(float) + 255) & ~(size_t)255;
}
static Q6PPtrs q6p_ptrs(void* base, int64_t n, int64_t k) {
    Q6PPtrs p;
    p.planes = (int8_t*)base;
    p.dwt = (float*)((uint8_t*)base + q6p_plane_bytes(n, k));
    p.np = (n + 3) & ~(int64_t)3;
    return p;
}

// One wave four consecutive (column, superblock) blocks: W is [n][k/256]
// blocks, so they are 840 contiguous bytes (2-byte aligned), which come in
// as the 212 dwords around them (four loads a lane, all issued first)
// through LDS; then each lane makes four elements of each block (4 l ..
// 4 l + 3 share their scale and bit positions; two elements a 16-bit lane).
// This half of the prep is bound by its VALU work, so it runs in
// the same launch as the activations' (bound by memory), on the grid's last
// workgroups.  (Block indices are 32-bit.)
constexpr int Q6P_PLANE_WG = 16;  // blocks a workgroup
__device__ __forceinline__ void q6_planes(const uint8_t* __restrict__ W, int8_t* __restrict__ planes,
                                          float* __restrict__ dwt, int n, int k, int np, uint32_t bid,
                                          uint32_t (&raw)[4][256]) {
    const int lane = threadIdx.x & 63, wq = threadIdx.x >> 6;
    const uint32_t nsb = (uint32_t)k >> 8, nblk = (uint32_t)n * nsb;
    const uint32_t blk0 = bid * Q6P_PLANE_WG + 4 * wq;
    const int64_t first = blk0 < nblk ? (int64_t)blk0 * Q6K_BYTES : 0;
    const uint32_t* src = (const uint32_t*)(W + (first & ~(int64_t)3));
    const int sh = (int)(first & 3);  // 0 or 2
    // (W's last block may end 2 bytes into its last dword)
    const int64_t left = (((int64_t)nblk * Q6K_BYTES + 3) >> 2) - (first >> 2);
    const int lim = (int)min(left, (int64_t)212);
    uint32_t wd[4];
#pragma unroll
    for (int i = 0; i < 4; i++) wd[i] = 64 * i + lane < lim ? src[64 * i + lane] : 0u;
#pragma unroll
    for (int i = 0; i < 4; i++) raw[wq][64 * i + lane] = wd[i];
    __syncthreads();
    const int e0 = 4 * lane, hh = e0 >> 7, r = e0 & 127, g = r >> 5, l = r & 31;
    const uint8_t* rb = (const uint8_t*)raw[wq];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t blk = blk0 + j;
        if (blk >= nblk) return;
        // the block starts sh + 210 j bytes into the wave's LDS copy (an even
        // offset); its four ql bytes and four qh bytes of this lane's
        // elements are 4-byte aligned within the block
        const int bo = sh + j * Q6K_BYTES, al = bo & 3;
        const uint32_t* q1 = (const uint32_t*)(rb + ((bo + 64 * hh + 32 * (g & 1) + l) & ~3));
        const uint32_t* q2 = (const uint32_t*)(rb + ((bo + Q6K_QH + 32 * hh + l) & ~3));
        const uint32_t qlw = __builtin_amdgcn_alignbyte(q1[1], q1[0], al);
        const uint32_t qhw = __builtin_amdgcn_alignbyte(q2[1], q2[0], al);
        const uint8_t* b = rb + bo;
        const uint32_t c = blk / nsb, sb = blk - c * nsb;
        const int sc = (int)(int8_t)b[Q6K_SC + (e0 >> 4)];
        // q6 of the four elements, one a byte (0..63)
        const uint32_t q = ((qlw >> (4 * (g >> 1))) & 0x0f0f0f0fu) | (((qhw >> (2 * g)) & 0x03030303u) << 4);
        // v = sc q - 32 sc in 16-bit lanes (|sc q| <= 8064: the low 16 bits
        // of the product are the signed result), elements 0, 2 and 1, 3
        const u16x2 sc2 = {(uint16_t)sc, (uint16_t)sc};
        const u16x2 sc32 = {(uint16_t)(32 * sc), (uint16_t)(32 * sc)};
        const u16x2 ve = __builtin_bit_cast(u16x2, q & 0x00ff00ffu) * sc2 - sc32;
        const u16x2 vo = __builtin_bit_cast(u16x2, (q >> 8) & 0x00ff00ffu) * sc2 - sc32;
        // lo = ((v + 32) & 63) - 32, hi = (v - lo) >> 6 (arithmetic)
        const u16x2 c32 = {32, 32}, m63 = {63, 63};
        const u16x2 le = ((ve + c32) & m63) - c32, lo_ = ((vo + c32) & m63) - c32;
        const s16x2 he = __builtin_bit_cast(s16x2, (u16x2)(ve - le)) >> (s16x2){6, 6};
        const s16x2 ho = __builtin_bit_cast(s16x2, (u16x2)(vo - lo_)) >> (s16x2){6, 6};
        // bytes 0-3 = elements 0-3: the low bytes of (even, odd, even, odd)
        const uint32_t lo4 = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, lo_), __builtin_bit_cast(uint32_t, le),
                                                   0x06020400u);
        const uint32_t hi4 = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, ho), __builtin_bit_cast(uint32_t, he),
                                                   0x06020400u);
        int8_t* o = planes + (size_t)c * 2 * k + 512 * sb + 128 * (e0 >> 6) + (e0 & 63);
        *(uint32_t*)o = hi4;
        *(uint32_t*)(o + 64) = lo4;
        if (lane == 0) dwt[(size_t)sb * np + c] = f16_to_f32(*(const uint16_t*)(b + Q6K_D));
    }
}

// The two-plane route's prep, one launch: xwg workgroups quantize the
// activations (as k_gemm_prep_q6) and the others build the weight planes,
// spread evenly through the grid (workgroup b is activation workgroup
// floor(b xwg / grid) when that count steps up at b, else a plane one), so
// the memory-bound and the VALU-bound halves share the CUs.
__global__ __launch_bounds__(256) void k_q6p_prep(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                  float* __restrict__ dyt, int m, int k, int mp, uint32_t xwg,
                                                  const uint8_t* __restrict__ W, int8_t* __restrict__ planes,
                                                  float* __restrict__ dwt, int n, int np) {
    __shared__ uint32_t raw[4][256];
    const uint64_t b = blockIdx.x, T = gridDim.x;
    const uint32_t xi = (uint32_t)(b * xwg / T);
    if ((uint32_t)((b + 1) * xwg / T) > xi) q6_prep_x<2, 4>(x, xq, dyt, m, k, mp, xi);  // uniform
    else q6_planes(W, planes, dwt, n, k, np, (uint32_t)b - xi, raw);
}

// Tiling: 4 x 2 waves of 64 x 64 (2 x 2 tiles of 32 x 32): a 256 x 128
// block of y.  K moves a quarter superblock (64) a stage through a ring of
// four, three in flight, every byte by global_load_lds:
//   A   [256][64] int8: row r's 16-byte piece p at p ^ (((r >> 1) ^ (r >> 3)) & 3)
//   B   [128][128] the column's hi then lo plane: piece p at p ^ (c & 7) ^ ((c >> 3) & 1)
//   DY  [256] f32, DW [128] f32 (a superblock's scales, in every stage; the
//       four stages' scales sit together at the start of LDS)
// The swizzles put the lanes of one ds_read_b128 on distinct 16-byte bank
// groups (both for 8 and for 16 lanes a pass), and neither key changes
// 32 rows or columns on, so a lane's second tile is an immediate offset.  Every wave issues 5 loads a
// stage (A 2, B 2, one scale chunk: wave 0 DY, the others DW, the same
// bytes to the same place), so a counted vmcnt wait leaves exactly the two
// later stages in flight.
// MFMA operands: lane l holds row (column) l % 32, elements 16 (l / 32) ..
// +15 of the 32-element chunk; the result's lane l holds column l % 32 and
// rows 8 (i / 4) + 4 (l / 32) + i % 4.
struct Q6P {
    static constexpr int WM = 4, WN = 2, WAVES = 8, THREADS = 512, BM = 256, BN = 128, S = 4;
    // LDS: the four scale slots first (so a slot's scales are an immediate
    // offset from one address), then the four A + B slots
    static constexpr int A = BM * 64, B = BN * 128, SC = 2048, STAGE = A + B, AB0 = S * SC, LDS = AB0 + S * STAGE;
    static constexpr int A_PER_WAVE = A / 1024 / WAVES, B_PER_WAVE = B / 1024 / WAVES;
    static constexpr int DMA = A_PER_WAVE + B_PER_WAVE + 1;
    static_assert(LDS <= 160 * 1024, "LDS");
    static_assert((S - 2) * DMA <= 63, "vmcnt counts to 63");
};

__device__ __forceinline__ int q6p_akey(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }
__device__ __forceinline__ int q6p_bkey(int col) { return (col & 7) ^ ((col >> 3) & 1); }

__global__ __launch_bounds__(Q6P::THREADS) void k_gemm_q6p(const int8_t* __restrict__ P, const float* __restrict__ dwt,
                                                          const int8_t* __restrict__ xq,
                                                          const float* __restrict__ dyt, float* __restrict__ Y, int m,
                                                          int n, int k, int mp, int np, int epi, int sps,
                                                          float* __restrict__ psum) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / Q6P::WN, wn = wave % Q6P::WN;
    const int h = lane >> 5, c32 = lane & 31;
    int bm, bn;
    tile_of((m + Q6P::BM - 1) / Q6P::BM, (n + Q6P::BN - 1) / Q6P::BN, bm, bn);
    const int m0 = bm * Q6P::BM, n0 = bn * Q6P::BN;
    const int nsb = k >> 8;
    const int s0 = blockIdx.y * sps, nst = 4 * min(sps, nsb - s0);  // quarter superblocks

    // chunk q (1 KB) of A is rows 16 q .., of B columns 8 q ..; wave w loads
    // chunks w and w + 8, so a lane's swizzled piece is the same in both and
    // they differ by a uniform offset (128 rows, 64 columns).  Rows and
    // columns of the last block past m and n read the padding of xq and the
    // planes: their sums land in rows and columns that are not stored.
    const int arow0 = 16 * wave + (lane >> 2), bcol0 = 8 * wave + (lane >> 3);
    const uint32_t aoff = (uint32_t)(m0 + arow0) * (uint32_t)k + 16u * ((lane & 3) ^ q6p_akey(arow0));
    const uint32_t boff = (uint32_t)(n0 + bcol0) * (uint32_t)(2 * k) + 16u * ((lane & 7) ^ q6p_bkey(bcol0));
    // wave 0: 64 lanes x 4 activation scales; the others: 32 lanes x 4
    // weight scales (lanes 32.. repeat lane 31's into the chunk's upper
    // half), clamped into the padded rows
    const uint32_t scoff = wave == 0 ? (uint32_t)min(m0 + 4 * lane, mp - 4) * 4u
                                     : (uint32_t)min(n0 + 4 * min(lane, 31), np - 4) * 4u;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds0 = lds_addr(smem);

    auto issue = [&](int i, int slot) {
        const int s = s0 + (i >> 2), qq = i & 3;
        const uint32_t st = lds0 + Q6P::AB0 + slot * Q6P::STAGE, sc = lds0 + slot * Q6P::SC;
        const int8_t* ab = xq + (uint32_t)s * 256u + 64u * qq;
#pragma unroll
        for (int j = 0; j < Q6P::A_PER_WAVE; j++)
            dma16s(ab + (uint32_t)(128 * j) * (uint32_t)k, aoff, st + 1024 * (wv + Q6P::WAVES * j));
        const int8_t* bb = P + (uint32_t)s * 512u + 128u * qq;
#pragma unroll
        for (int j = 0; j < Q6P::B_PER_WAVE; j++)
            dma16s(bb + (uint32_t)(64 * j) * (uint32_t)(2 * k), boff, st + Q6P::A + 1024 * (wv + Q6P::WAVES * j));
        // the scales of the superblock stage i - 1 belongs to (see below)
        const int ss = s0 + (max(i - 1, 0) >> 2);
        if (wv == 0) dma16s(dyt + (int64_t)ss * mp, scoff, sc);
        else dma16s(dwt + (int64_t)ss * np, scoff, sc + 1024);
    };

    float out[2][2][16];
    v16i hi[2][2], lo[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) out[a][b][r] = 0.0f;
    // this lane's operand addresses in a stage, per chunk c of the quarter:
    // A rows r0 and r0 + 32, B columns c0 and c0 + 32 (hi and lo planes)
    const int r0 = wm * 64 + c32, c0 = wn * 64 + c32;
    int aad[2], bhad[2], blad[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        aad[c] = r0 * 64 + 16 * ((2 * c + h) ^ q6p_akey(r0));
        bhad[c] = Q6P::A + c0 * 128 + 16 * ((2 * c + h) ^ q6p_bkey(c0));
        blad[c] = Q6P::A + c0 * 128 + 16 * ((4 + 2 * c + h) ^ q6p_bkey(c0));
    }

    // quarter Q of a superblock, from slot Q of the ring
    auto quarter = [&](auto qc) {
        constexpr int Q = decltype(qc)::value;
        const uint8_t* st = smem + Q6P::AB0 + Q * Q6P::STAGE;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            v4i av[2], bh[2], bl[2];
#pragma unroll
            for (int a = 0; a < 2; a++) av[a] = *(const v4i*)(st + aad[c] + 32 * 64 * a);
#pragma unroll
            for (int b = 0; b < 2; b++) {
                bh[b] = *(const v4i*)(st + bhad[c] + 32 * 128 * b);
                bl[b] = *(const v4i*)(st + blad[c] + 32 * 128 * b);
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    const v16i z = {};
                    hi[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a], bh[b], (Q == 0 && c == 0) ? z : hi[a][b], 0, 0, 0);
                    lo[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a], bl[b], (Q == 0 && c == 0) ? z : lo[a][b], 0, 0, 0);
                }
        }
    };
    // a finished superblock: out += f32(64 hi + lo) * (d * dy), its scales
    // from the stage in `slot`
    auto epilogue = [&](int slot) {
        {
            const float* DY = (const float*)(smem + slot * Q6P::SC);
            const float* DW = DY + 256;
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const float dw = DW[wn * 64 + b * 32 + c32];
#pragma unroll
                for (int a = 0; a < 2; a++) {
                    const float* dyp = DY + wm * 64 + a * 32 + 4 * h;
#pragma unroll
                    for (int gq = 0; gq < 4; gq++) {
                        const float4 d4 = *(const float4*)(dyp + 8 * gq);
                        const float dys[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const int r = 4 * gq + u;
                            const int v = hi[a][b][r] * 64 + lo[a][b][r];
                            out[a][b][r] = __builtin_fmaf((float)v, dw * dys[u], out[a][b][r]);
                        }
                    }
                }
            }
        }
    };
    // stage i + 3 goes into the slot stage i - 1 used (its readers passed
    // the last barrier); past the end it reloads the last stage into a slot
    // nobody reads, so the counts never change.  The two waves of a SIMD
    // (w and w + 4) take their superblock epilogues a quarter apart, so one
    // runs its VALU work under the other's MFMAs: waves 0-3 after quarter 3,
    // waves 4-7 before quarter 0 of the next superblock (and after the
    // loop).  A stage carries the scales of the superblock of the stage
    // before it, which is the finished one at both points.
    const bool grpB = wave >= 4;
    auto step = [&](int i, auto qc) {
        constexpr int Q = decltype(qc)::value;
        issue(min(i + 3, nst - 1), (Q + 3) & 3);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (Q == 0) {
            if (grpB && i > 0) epilogue(0);
            __builtin_amdgcn_sched_barrier(0);
        }
        quarter(qc);
        if constexpr (Q == 3) {
            if (!grpB) epilogue(3);
        }
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((Q6P::S - 2) * Q6P::DMA) : "memory");
        __builtin_amdgcn_s_barrier();
    };

#pragma unroll
    for (int i = 0; i < 3; i++) issue(min(i, nst - 1), i);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((Q6P::S - 2) * Q6P::DMA) : "memory");
    __builtin_amdgcn_s_barrier();
    for (int i = 0; i < nst; i += 4) {
        step(i, std::integral_constant<int, 0>{});
        step(i + 1, std::integral_constant<int, 1>{});
        step(i + 2, std::integral_constant<int, 2>{});
        step(i + 3, std::integral_constant<int, 3>{});
    }
    if (grpB) epilogue(3);
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int col = n0 + wn * 64 + b * 32 + c32;
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * 64 + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < m) {
                    if (psum) psum[((int64_t)blockIdx.y * m + row) * n + col] = out[a][b][r];
                    else if (epi == EPI_STORE) Y[(int64_t)row * n + col] = out[a][b][r];
                    else store_epi_slow(&Y[(int64_t)row * n + col], out[a][b][r], epi);
                }
            }
        }
}

// Splits of K for a grid of `tiles` workgroups: up to ~256 workgroups, at
// least 4 superblocks each, at most 8.
static int q6_splits(int64_t tiles, int64_t nsb) {
    int sp = 1;
    while (sp < 8 && tiles * sp * 2 <= 256 && nsb / (sp * 2) >= 4) sp *= 2;
    return sp;
}

template <class C>
static int64_t q6_tiles(int64_t n, int64_t m) {
    return ((m + C::BM - 1) / C::BM) * ((n + C::BN - 1) / C::BN);
}

template <class C>
static hipError_t launch_q6_cfg(const void* w, const Q6Ptrs& p, float* y, int64_t n, int64_t k, int64_t m, int epi,
                                hipStream_t s, float* psum, int sp) {
    if (hipError_t e = set_lds_limit((const void*)k_gemm_q6k<C>, C::LDS)) return e;
    const int64_t tiles = q6_tiles<C>(n, m), nsb = k / 256;
    const int sps = (int)((nsb + sp - 1) / sp);
    hipLaunchKernelGGL(k_gemm_q6k<C>, dim3((unsigned)tiles, sp), dim3(C::THREADS), C::LDS, s, (const uint8_t*)w, p.xq,
                       p.dyt, y, (int)m, (int)n, (int)k, (int)p.mp, epi, sps, sp > 1 ? psum : nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || sp == 1) return e;
    const int64_t mn = m * n;
    hipLaunchKernelGGL(k_q6_sum_splits, dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0, s, psum, sp, mn, y, epi);
    return hipGetLastError();
}

// Weight rows 2-byte aligned (always: 210 bytes a superblock) and 32-bit
// DMA offsets.
bool q6_gemm_fits(int64_t n, int64_t k, int64_t m) {
    return k % 256 == 0 && n * (k / 256) * Q6K_BYTES + 256 < ((int64_t)1 << 32) && m * k < ((int64_t)1 << 32);
}

// LLOOM_HIP_Q6_PLANES (read once): "0" never the two-plane route, "1" from
// the GEMM's first row count; unset: from Q6P_MIN_ROWS rows.  Measured on
// [2048, 8192] (n 2048, k 8192), whole calls, graph replay, rotating weight
// copies: m = 512 60.7 us, the same as k_gemm_q6k; 1024 77.5 against
// 105.1, 2048 122.0 against 182.0 (of which k_gemm_q6p ~82, the prep
// launch ~25, the split-K sum ~9); at 256 the first form of this route
// measured 52.9 against 38.7.
constexpr int64_t Q6P_MIN_ROWS = 640;
static int q6p_env() {
    static const int v = [] {
        const char* e = getenv("LLOOM_HIP_Q6_PLANES");
        return e ? atoi(e) : -1;
    }();
    return v;
}
static int64_t q6p_rows(int64_t m) { return (m + Q6P::BM - 1) / Q6P::BM * Q6P::BM; }
// (32-bit DMA offsets into the padded xq and planes)
static bool q6p_route(int64_t n, int64_t k, int64_t m) {
    const int e = q6p_env();
    return e != 0 && (e == 1 || m >= Q6P_MIN_ROWS) && ((n + 127) & ~(int64_t)127) * 2 * k < ((int64_t)1 << 32) &&
           q6p_rows(m) * k < ((int64_t)1 << 32);
}
static int q6p_launch_splits(int64_t n, int64_t k, int64_t m) {
    const int64_t tiles = ((m + Q6P::BM - 1) / Q6P::BM) * ((n + Q6P::BN - 1) / Q6P::BN), nsb = k / 256;
    const int sp = q6_splits(tiles, nsb);
    const int64_t sps = (nsb + sp - 1) / sp;
    return (int)((nsb + sps - 1) / sps);
}
static size_t q6p_workspace_bytes(int64_t n, int64_t k, int64_t m) {
    const int sp = q6p_launch_splits(n, k, m);
    return q6_prep_bytes(m, k, q6p_rows(m)) + q6p_plane_bytes(n, k) + q6p_dw_bytes(n, k) +
           (sp > 1 ? (size_t)sp * m * n * sizeof(float) : 0);
}

static hipError_t launch_q6p(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* qbuf,
                             size_t ws_cap, int epi, hipStream_t s) {
    if (q6p_workspace_bytes(n, k, m) > ws_cap) return hipErrorInvalidValue;
    const int sp = q6p_launch_splits(n, k, m);
    const Q6Ptrs p = q6_ptrs(qbuf, m, k, q6p_rows(m));
    uint8_t* wbase = (uint8_t*)qbuf + q6_prep_bytes(m, k, q6p_rows(m));
    const Q6PPtrs pp = q6p_ptrs(wbase, n, k);
    float* psum = (float*)(wbase + q6p_plane_bytes(n, k) + q6p_dw_bytes(n, k));
    const int64_t nsb = k / 256, nb = m * nsb, wb = n * nsb;
    const uint32_t xwg = (uint32_t)((nb + 31) / 32);
    const uint32_t pwg = (uint32_t)((wb + Q6P_PLANE_WG - 1) / Q6P_PLANE_WG);
    hipLaunchKernelGGL(k_q6p_prep, dim3(xwg + pwg), dim3(256), 0, s, x, p.xq, p.dyt, (int)m, (int)k, (int)p.mp, xwg,
                       (const uint8_t*)w, pp.planes, pp.dwt, (int)n, (int)pp.np);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if ((e = set_lds_limit((const void*)k_gemm_q6p, Q6P::LDS))) return e;
    const int64_t tiles = ((m + Q6P::BM - 1) / Q6P::BM) * ((n + Q6P::BN - 1) / Q6P::BN);
    const int sps = (int)((nsb + sp - 1) / sp);
    hipLaunchKernelGGL(k_gemm_q6p, dim3((unsigned)tiles, sp), dim3(Q6P::THREADS), Q6P::LDS, s, pp.planes, pp.dwt, p.xq,
                       p.dyt, y, (int)m, (int)n, (int)k, (int)p.mp, (int)pp.np, epi, sps, sp > 1 ? psum : nullptr);
    if ((e = hipGetLastError()) != hipSuccess || sp == 1) return e;
    const int64_t mn = m * n;
    hipLaunchKernelGGL(k_q6_sum_splits, dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0, s, psum, sp, mn, y, epi);
    return hipGetLastError();
}

// LLOOM_HIP_Q6_TILE (read once) picks the tile for tuning; -1 (default)
// chooses by m.
static int q6_tile_env() {
    static const int v = [] {
        const char* e = getenv("LLOOM_HIP_Q6_TILE");
        return e ? atoi(e) : -1;
    }();
    return v;
}

// The tile for m rows (LLOOM_HIP_Q6_TILE overrides): to 128 rows 64 x 64,
// past that 128 x 128 (measurements below, at the launch).
static int q6_tile_of(int64_t m) {
    const int t = q6_tile_env();
    return t >= 0 ? t : m <= 128 ? 2 : 0;
}

// The K splits a launch of m rows will take (1: no partial sums).
static int q6_launch_splits(int64_t n, int64_t k, int64_t m) {
    int64_t tiles;
    switch (q6_tile_of(m)) {
        case 1: tiles = q6_tiles<Q6Cfg<2, 2, 2, 2, 2>>(n, m); break;
        case 2: tiles = q6_tiles<Q6Cfg<2, 2, 1, 1, 3>>(n, m); break;
        case 3: tiles = q6_tiles<Q6Cfg<2, 4, 1, 1, 3>>(n, m); break;
        default: tiles = q6_tiles<Q6Cfg<2, 4, 2, 1, 2>>(n, m); break;
    }
    const int64_t nsb = k / 256;
    const int sp = q6_splits(tiles, nsb);
    const int64_t sps = (nsb + sp - 1) / sp;
    return (int)((nsb + sps - 1) / sps);
}

// The prepared activations, then the split-K partial sums when the launch
// splits K.
size_t q6_gemm_workspace_bytes(int64_t n, int64_t k, int64_t m) {
    if (q6p_route(n, k, m)) return q6p_workspace_bytes(n, k, m);
    const int sp = q6_launch_splits(n, k, m);
    return q6_prep_bytes(m, k) + (sp > 1 ? (size_t)sp * m * n * sizeof(float) : 0);
}

hipError_t launch_q6_gemm(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* qbuf,
                          size_t ws_cap, int epi, hipStream_t s) {
    if (q6p_route(n, k, m)) return launch_q6p(w, x, y, n, k, m, qbuf, ws_cap, epi, s);
    // the split count sizes the partial-sum region: one computation serves
    // the workspace size and the launch, and the caller's capacity is checked
    const int sp = q6_launch_splits(n, k, m);
    if (q6_prep_bytes(m, k) + (sp > 1 ? (size_t)sp * m * n * sizeof(float) : 0) > ws_cap) return hipErrorInvalidValue;
    const Q6Ptrs p = q6_ptrs(qbuf, m, k);
    hipError_t e = launch_prep_q6(x, p.xq, p.dyt, m, k, p.mp, s);
    if (e != hipSuccess) return e;
    float* psum = (float*)((uint8_t*)qbuf + q6_prep_bytes(m, k));
    const int tile = q6_tile_of(m);
    // by m (measured with the prep launch, graph replay, [2048, 8192] /
    // [8192, 2048]): to 128 rows 64 x 64 tiles, 3 stages (m = 64 22.3 / 23.2
    // us against 34.8 / 35.5 for 128 x 128, m = 128 34.4 / 30.7); past that
    // 128 x 128 with 8 waves (m = 256 42.4 / 44.8, m = 2048 219.5 / 222.8
    // us against 59.2 / 54.9 and 383 / 405 for 64 x 64).  Few tiles split K.
    switch (tile) {
        case 1: return launch_q6_cfg<Q6Cfg<2, 2, 2, 2, 2>>(w, p, y, n, k, m, epi, s, psum, sp);  // 128 x 128, 4 waves
        case 2: return launch_q6_cfg<Q6Cfg<2, 2, 1, 1, 3>>(w, p, y, n, k, m, epi, s, psum, sp);  // 64 x 64, 3 stages
        case 3: return launch_q6_cfg<Q6Cfg<2, 4, 1, 1, 3>>(w, p, y, n, k, m, epi, s, psum, sp);  // 64 x 128, 8 waves
        default: return launch_q6_cfg<Q6Cfg<2, 4, 2, 1, 2>>(w, p, y, n, k, m, epi, s, psum, sp);  // 128 x 128, 8 waves
    }
}

}  // namespace lloom
