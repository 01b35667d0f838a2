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

// Activation prep (Q8_K of every (row, superblock), bit-exact):
//   xq  int8 [m][k]
//   dyt f32  [k/256][mp]   mp = m rounded up to 4, then 128 floats of pad
struct Q6Ptrs {
    int8_t* xq;
    float* dyt;
    int64_t mp;
};

static Q6Ptrs q6_ptrs(void* base, int64_t m, int64_t k) {
    Q6Ptrs p;
    p.xq = (int8_t*)base;
    p.dyt = (float*)((uint8_t*)base + (((size_t)m * k + 255) & ~(size_t)255));
    p.mp = (m + 3) & ~(int64_t)3;
    return p;
}

static size_t q6_prep_bytes(int64_t m, int64_t k) {
    const int64_t mp = (m + 3) & ~(int64_t)3;
    return (((size_t)m * k + 255) & ~(size_t)255) + (((size_t)(k / 256) * mp + 128) * sizeof(float) + 255 & ~(size_t)255);
}


// One wave a (row, superblock).
__global__ __launch_bounds__(256) void k_gemm_prep_q6(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                      float* __restrict__ dyt, int m, int k, int mp) {
    const int lane = threadIdx.x & 63;
    const int nsb = k >> 8;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= (int64_t)m * nsb) return;
    const int mi = (int)(blk / nsb), sb = (int)(blk - (int64_t)mi * nsb);
    const int64_t off = (int64_t)mi * k + 256 * sb + 4 * lane;
    const float4 v = *(const float4*)(x + off);
    float d;
    int bs;
    const uint32_t q = q8k_block_wave(v, &d, &bs);
    *(uint32_t*)(xq + off) = q;
    if (lane == 0) dyt[(int64_t)sb * mp + mi] = d;
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
// epilogue.
__global__ __launch_bounds__(256) void k_q6_sum_splits(const float* __restrict__ psum, int splits, int64_t mn,
                                                       float* __restrict__ Y, int epi) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= mn) return;
    float v = psum[i];
    for (int z = 1; z < splits; z++) v += psum[z * mn + i];
    store_epi(&Y[i], v, epi);
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
    hipLaunchKernelGGL(k_q6_sum_splits, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, psum, sp, mn, y, epi);
    return hipGetLastError();
}

// Weight rows 2-byte aligned (always: 210 bytes a superblock) and 32-bit
// DMA offsets.
bool q6_gemm_fits(int64_t n, int64_t k, int64_t m) {
    return k % 256 == 0 && n * (k / 256) * Q6K_BYTES + 256 < ((int64_t)1 << 32) && m * k < ((int64_t)1 << 32);
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
    const int sp = q6_launch_splits(n, k, m);
    return q6_prep_bytes(m, k) + (sp > 1 ? (size_t)sp * m * n * sizeof(float) : 0);
}

hipError_t launch_q6_gemm(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* qbuf,
                          size_t ws_cap, int epi, hipStream_t s) {
    // the split count sizes the partial-sum region: one computation serves
    // the workspace size and the launch, and the caller's capacity is checked
    const int sp = q6_launch_splits(n, k, m);
    if (q6_prep_bytes(m, k) + (sp > 1 ? (size_t)sp * m * n * sizeof(float) : 0) > ws_cap) return hipErrorInvalidValue;
    const Q6Ptrs p = q6_ptrs(qbuf, m, k);
    const int64_t nb = m * (k / 256);
    hipLaunchKernelGGL(k_gemm_prep_q6, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x, p.xq, p.dyt, (int)m, (int)k,
                       (int)p.mp);
    hipError_t e = hipGetLastError();
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
