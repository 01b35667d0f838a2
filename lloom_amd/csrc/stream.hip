// stream.hip -- Q4_K decode (2..16 activation rows) on large weights: a
// persistent, pipelined form of the 16-row MFMA decode.
//
// The arithmetic is k_quants' Q4_K x Q8_K dot (k_quants.rs:1540-1620), as
// in every other MFMA decode kernel here (mf_compute_q4k_b: integer sums
// exact, the f32 combination per superblock), on activations quantized once
// per call by k_quantize_split_q8k (tiled layout, bit-exact Q8_K).
//
// Why another kernel: k_mv_dma_ma and k_mv_mfma give each workgroup one or
// two 16-row weight tiles, which it loads, waits for, computes and stores.
// On weights of tens of MB that leaves a CU's memory pipe idle between its
// workgroups and re-reads the activations once per tile.  Here:
//  * one workgroup per CU (the grid is the CU count), each owning every
//    CU-count-th 16-row weight tile;
//  * its 8 waves split K, wave w taking superblocks [w S, w S + S) of every
//    row (S = k / 2048), so the wave's activation operands (S superblocks,
//    16 activation rows) are loaded into registers once and kept for the
//    whole run;
//  * each wave moves its own part of each tile (16 rows x S superblocks,
//    S * 2304 bytes) into a private LDS ring of D stages by 1 KB
//    global_load_lds DMAs, D - 1 tiles ahead of the tile it computes, and
//    waits for a tile by a counted vmcnt (loads retire in order), so the
//    weight stream never waits on compute or on the other waves;
//  * the eight partial sums of a tile (one per wave, 4 floats a lane) meet
//    in one of R LDS slots; each wave, after writing its partial, counts
//    itself in with an LDS atomic, and the eighth to arrive adds the eight
//    in wave order (a fixed order: bit-reproducible) and stores the tile.
//    No barrier couples the waves: a wave only waits (on an LDS counter)
//    when it would overwrite a slot whose previous tile is not yet added,
//    so waves whose DMAs landed first run ahead and keep the CU's memory
//    pipe full while the others catch up.
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "kq_common.hpp"
#include "kq_gemm.hpp"
#include "kq_mfma.hpp"
#include "kernels.hpp"

namespace lloom {

constexpr int ST_WAVES = 8;
constexpr int ST_SBB = 16 * Q4K_BYTES;  // one superblock of a 16-row tile: 2304 bytes

template <int S>
struct StCfg {
    static constexpr int WSTAGE = S * ST_SBB;                  // a wave's bytes of a tile
    static constexpr int NI = (WSTAGE + 1023) / 1024;          // its DMA instructions
    static constexpr int WPITCH = NI * 1024;                   // its LDS bytes a stage
    // stages: as many as fit beside the partial-sum slots; R slots of
    // partial sums (8 KB each) and their counters
    static constexpr int D = S == 1 ? 4 : S == 2 ? 3 : 2;
    static constexpr int R = S == 4 ? 1 : 4;
    static constexpr int RING = D * ST_WAVES * WPITCH;
    static constexpr int PART = R * ST_WAVES * 64 * 16;
    static constexpr int LDS = RING + PART + 2 * R * 4;
    static_assert(LDS <= 160 * 1024, "LDS budget");
};

// Compile-time index loop: f(std::integral_constant<int, i>) for i < N.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int S>
__global__ __launch_bounds__(64 * ST_WAVES) void k_mv_stream(const uint8_t* __restrict__ W,
                                                             const int8_t* __restrict__ xt,
                                                             const float* __restrict__ xd,
                                                             const int8_t* __restrict__ bsp, float* __restrict__ Y,
                                                             int n, int m, int mp, int epi) {
    using C = StCfg<S>;
    constexpr int NSB = 8 * S;  // superblocks a row
    constexpr uint32_t ROWB = (uint32_t)NSB * Q4K_BYTES;
    constexpr int D = C::D, NI = C::NI;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int tiles = (n + 15) >> 4;
    // this workgroup's tiles: blockIdx.x + it * gridDim.x, it < T (dealt
    // round-robin: contiguous runs left some workgroups tens of percent
    // slower than others, and the launch waits for the slowest)
    const int G = gridDim.x;
    const int T = (tiles - (int)blockIdx.x + G - 1) / G;
    if (T <= 0) return;  // uniform
    auto tile_of = [&](int it) { return (int)blockIdx.x + it * G; };
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    if (threadIdx.x < 2 * C::R) ((uint32_t*)(smem + C::RING + C::PART))[threadIdx.x] = 0;
    __syncthreads();  // nothing is in flight yet

    // this wave's activation operands (tile 0 of the tiled layout; rows past
    // m are the quantizer's padding and never stored), kept for the run
    long av[S][8], ab[S];
    float4 dy[S];
#pragma unroll
    for (int i = 0; i < S; i++) {
        const int sb = wave * S + i;
        const int8_t* src = xt + (int64_t)sb * 4 * 1024 + 16 * lane;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 v = *(const uint4*)(src + 1024 * q);
            av[i][2 * q] = (long)(((uint64_t)v.y << 32) | v.x);
            av[i][2 * q + 1] = (long)(((uint64_t)v.w << 32) | v.z);
        }
        dy[i] = *(const float4*)(xd + (int64_t)sb * mp + 4 * g);
        const long v = *(const long*)(bsp + ((int64_t)sb * mp + c16) * 16 + 8 * min(g, 1));
        ab[i] = v & -(long)(g < 2 && c16 < m);
    }

    // DMA instruction j of a tile for this lane: byte L = 1024 j + 16 lane
    // of the wave's stage = superblock L / 2304, row (L % 2304) / 144, piece
    // L % 144 (pad lanes past the stage reload its last piece)
    uint32_t voff[NI];
#pragma unroll
    for (int j = 0; j < NI; j++) {
        const int L = min(1024 * j + 16 * lane, C::WSTAGE - 16);
        const int sbi = L / ST_SBB, rem = L - sbi * ST_SBB, row = rem / Q4K_BYTES, piece = rem - row * Q4K_BYTES;
        voff[j] = (uint32_t)row * ROWB + (uint32_t)(wave * S + sbi) * Q4K_BYTES + (uint32_t)piece;
    }
    const uint32_t lds0 = lds_addr(smem) + (uint32_t)wv * C::WPITCH;
    // the last tile of the matrix is shifted to end at row n - 1 (n >= 16):
    // its rows before 16 t are the previous tile's and are not stored
    auto tile_row0 = [&](int t) { return min(16 * t, n - 16); };
    // instructions [j0, j1) of tile t into ring slot `slot`
    auto issue = [&](int t, int slot, int j0, int j1) {
        const uint8_t* base = W + (int64_t)tile_row0(t) * ROWB;
        const uint32_t dst = lds0 + (uint32_t)slot * (ST_WAVES * C::WPITCH);
#pragma unroll
        for (int j = 0; j < NI; j++)
            if (j >= j0 && j < j1) dma16s(base, voff[j], dst + 1024 * j);
    };

    constexpr int R = C::R;
    float4* part = (float4*)(smem + C::RING);
    // per slot: arrivals (8 a tile, never reset) and tiles added so far
    uint32_t* arrived = (uint32_t*)(smem + C::RING + C::PART);
    uint32_t* added = arrived + R;
    // prologue: the run's first tile, then a use of every operand register,
    // where the compiler puts its waits for the loads above (they come
    // after the first tile's DMAs, so it waits for that tile too, which the
    // first dots need anyway; at the registers' first use inside the loop
    // its counts would ignore the DMAs in flight), then tiles 1 .. D - 1.
    // Issuing all D tiles first made every wave wait for all of them before
    // its first dots (k = 8192: the first tile ready at 7.1 us, 10.6 for the
    // second wave of each SIMD)
    if (T > 0) issue(tile_of(0), 0, 0, NI);
#pragma unroll
    for (int i = 0; i < S; i++) {
#pragma unroll
        for (int q = 0; q < 8; q++) asm volatile("" : "+v"(av[i][q]));
        asm volatile("" : "+v"(ab[i]), "+v"(dy[i].x), "+v"(dy[i].y), "+v"(dy[i].z), "+v"(dy[i].w));
    }
#pragma unroll
    for (int d = 1; d < D; d++)
        if (d < T) issue(tile_of(d), d, 0, NI);

    // Ring discipline, per superblock i of tile t (slot t mod D): wait until
    // the DMA instruction holding its last byte, need(i), has landed; compute
    // it; then refill the instructions of the slot that lie wholly in
    // superblocks <= i with tile t + D.  Loads retire in order, so the wait
    // is a count of the instructions issued after need(i): steady(i) while
    // the run refills, tail(i, r) once it does not (r = tiles issued after
    // t).
    constexpr auto need = [](int i) { return (ST_SBB * (i + 1) - 1) / 1024; };
    constexpr auto last_free = [](int i) { return i == S - 1 ? NI - 1 : (ST_SBB * (i + 1)) / 1024 - 1; };
    constexpr auto first_free = [](int i) { return i == 0 ? 0 : (ST_SBB * i) / 1024; };
    for (int it = 0; it < T; it++) {
        const int t = tile_of(it), slot = it % D;
        const bool refill = it + D < T;  // uniform
        const int r = min(D - 1, T - 1 - it);
        const uint8_t* st = smem + slot * (ST_WAVES * C::WPITCH) + wave * C::WPITCH;
        float out[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        static_for<S>([&](auto I) {
            constexpr int i = decltype(I)::value;
            constexpr int tail0 = NI - 1 - need(i);
            __builtin_amdgcn_sched_barrier(0);
            if (refill) {
                vm_wait<D * NI - 1 - need(i) + first_free(i)>();
            } else if (r == 0) {
                vm_wait<tail0>();
            } else {
                vm_wait<0>();
            }
            MfW<T_Q4K> wu;
            mf_load<T_Q4K>(st + (i * 16 + c16) * Q4K_BYTES, g, wu);
            mf_compute_q4k_b(wu, av[i], ab[i], dy[i], g, out);
            // the superblock's sums are complete here, before the next wait:
            // otherwise they are sunk past it and every superblock's loads
            // and products stay live across the tile
            asm volatile("" : "+v"(out[0]), "+v"(out[1]), "+v"(out[2]), "+v"(out[3]));
            __builtin_amdgcn_sched_barrier(0);
            if (refill) issue(tile_of(it + D), slot, first_free(i), last_free(i) + 1);
        });
        // this tile's slot: free once its previous tile (it - R) is added
        const int ps = it % R;
        const uint32_t use = (uint32_t)(it / R);
        for (int spin = 0; spin < (1 << 24); spin++) {  // bounded: always exits
            if (__hip_atomic_load(&added[ps], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == use) break;
            __builtin_amdgcn_s_sleep(1);
        }
        // (relaxed atomics, ordered by these compiler barriers and by the
        // wave's LDS operations completing in issue order)
        asm volatile("" ::: "memory");
        float4* pb = part + ps * (ST_WAVES * 64);
        pb[wave * 64 + lane] = make_float4(out[0], out[1], out[2], out[3]);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the partial is in LDS
        uint32_t prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(&arrived[ps], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        prev = __builtin_amdgcn_readfirstlane(prev);
        asm volatile("" ::: "memory");
        if ((prev & (ST_WAVES - 1)) == ST_WAVES - 1) {  // uniform: the eighth arrival adds
            float4 acc = pb[lane];
#pragma unroll
            for (int w = 1; w < ST_WAVES; w++) {
                const float4 p = pb[w * 64 + lane];
                acc.x += p.x;
                acc.y += p.y;
                acc.z += p.z;
                acc.w += p.w;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot is read
            if (lane == 0) __hip_atomic_fetch_add(&added[ps], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            const int row = tile_row0(t) + c16;
            const float o[4] = {acc.x, acc.y, acc.z, acc.w};
            if (row >= 16 * t) {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    if (4 * g + v < m) store_epi(&Y[(int64_t)(4 * g + v) * n + row], o[v], epi);
            }
        }
    }
    // no DMA may still be writing this workgroup's LDS when it exits
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// CUs of the current device, asked once per device.
int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
    if (dev < 64) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    if (dev < 64) cache[dev].store(c, std::memory_order_relaxed);
    return c;
}

// LLOOM_HIP_STREAM_MIN_MB (read once): weights of at least this many MB
// (default 24) take the streaming kernel; 0 turns it off.
static int64_t stream_min_bytes() {
    static const int64_t v = [] {
        const char* e = getenv("LLOOM_HIP_STREAM_MIN_MB");
        return (e ? (int64_t)atoll(e) : (int64_t)24) << 20;
    }();
    return v;
}

// Where it wins (measured on rotating copies, against the kernels that take
// the call otherwise): from 4 rows at k = 4096 .. 8192 and 24 MB up ([14336,
// 4096] B = 4 / 16: 17.9 / 18.1 against 19.1 / 20.6 us; [57344, 4096]
// 38.6 / 40.1 against 55.7 / 60.3), 2-3 rows only from ~96 MB ([28672, 8192]
// B = 2 36.0 against 44.1 us; at 54-63 MB it ties or loses), and at k = 2048
// 2-4 rows from ~48 MB ([57344, 2048] B = 4 25.4 against 32.9 us; from 5
// rows k_mv_dma_ma is faster).  One row stays on the dot4 kernel.
bool mv_stream_fits(int type, int64_t n, int64_t k, int64_t m) {
    const int64_t minb = stream_min_bytes();
    if (type != T_Q4K || minb <= 0 || m < 2 || m > 16 || n < 16) return false;
    if (k % 2048 || k > 4 * 2048 || (k == 2048 && m > 4)) return false;
    const int64_t bytes = n * (k / 256) * Q4K_BYTES;
    if (k == 2048) return bytes >= 2 * minb && n < ((int64_t)1 << 30);
    if (m < 4) return bytes >= 4 * minb && n < ((int64_t)1 << 30);
    return bytes >= minb && n < ((int64_t)1 << 30);
}

template <int S>
static hipError_t launch_stream_s(const void* w, float* y, int64_t n, int64_t m, const int8_t* xt, const float* xd,
                                  const int8_t* bsp, int epi, hipStream_t s) {
    using C = StCfg<S>;
    if (hipError_t e = set_lds_limit((const void*)k_mv_stream<S>, C::LDS)) return e;
    const int64_t tiles = (n + 15) / 16;
    const int64_t cus = cu_count();
    const int64_t grid = tiles < cus ? tiles : cus;
    const int mp = (int)((m + 15) & ~(int64_t)15);
    hipLaunchKernelGGL((k_mv_stream<S>), dim3((unsigned)grid), dim3(64 * ST_WAVES), C::LDS, s, (const uint8_t*)w, xt,
                       xd, bsp, y, (int)n, (int)m, mp, epi);
    return hipGetLastError();
}

hipError_t launch_mv_stream(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                            void* ws, int epi, hipStream_t s) {
    if (!mv_stream_fits(type, n, k, m)) return hipErrorInvalidValue;
    int8_t* xt;
    float* xd;
    int8_t* bsp;
    split_q8k_ptrs(ws, k, m, &xt, &xd, &bsp);
    hipError_t e = launch_quantize_split_q8k(x, m, k, xt, xd, s, bsp, true);
    if (e != hipSuccess) return e;
    switch (k / 2048) {
        case 1: return launch_stream_s<1>(w, y, n, m, xt, xd, bsp, epi, s);
        case 2: return launch_stream_s<2>(w, y, n, m, xt, xd, bsp, epi, s);
        case 3: return launch_stream_s<3>(w, y, n, m, xt, xd, bsp, epi, s);
        default: return launch_stream_s<4>(w, y, n, m, xt, xd, bsp, epi, s);
    }
}

}  // namespace lloom
