// matvec.hip -- decode-shaped quantized matmul (m <= 16 activation rows).
//
// y[m, n] = x[m, k] . W[n, k]^T with W packed Q8_0 / Q4_K / Q6_K, the CPU
// arm's arithmetic (k_quants::matmul, k_quants.rs:2455-2641): x is quantized
// to the VecDotType (Q8_0 or Q8_K, bit-exact), each dot is an exact integer
// sum per block combined with f32 scales.
//
// MI355X layout of the work:
//  * a 256-thread workgroup = 4 wave64s; each wave owns R consecutive weight
//    rows, each lane one "task" (a 16-byte qs vector of a Q4_K superblock,
//    a 64-element quarter of a Q6_K superblock, or a 34-byte Q8_0 block) per
//    row, so a wave streams a row as one contiguous, coalesced sweep;
//  * the weight loads of a K-chunk are issued first, then the workgroup
//    quantizes the chunk of x into LDS (every block exactly as from_float),
//    so the HBM latency of the weights hides under the quantization;
//  * the dots are v_dot4_i32_i8 on 4 int8 lanes at a time; the Q4_K min term
//    uses the Q8_K bsums, the Q6_K "-32" uses them too;
//  * each lane accumulates f32 partials for its rows and activation rows,
//    reduced across the wave at the end.
// The float summation order differs from the CPU's (lane partials), which
// is why parity is to a tolerance; every integer sum is exact.
#include "kq_common.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"

namespace lloom {

constexpr int MV_WAVES = 4;
constexpr int MV_THREADS = 64 * MV_WAVES;

template <int TYPE>
struct MvTraits;
template <>
struct MvTraits<T_Q4K> {
    static constexpr int BE = 256, BB = Q4K_BYTES, P = 8, VT = T_Q8K;
};
template <>
struct MvTraits<T_Q6K> {
    static constexpr int BE = 256, BB = Q6K_BYTES, P = 4, VT = T_Q8K;
};
template <>
struct MvTraits<T_Q8_0> {
    static constexpr int BE = 32, BB = Q8_0_BYTES, P = 1, VT = T_Q8_0;
};

// Weight bytes a lane holds for one task.
struct TaskData {
    uint4 a, b, c, s;
    uint32_t e;
};

template <int TYPE>
__device__ __forceinline__ void load_task(const uint8_t* __restrict__ row, int blk, int p, TaskData& t) {
    if constexpr (TYPE == T_Q4K) {
        const uint8_t* b = row + (size_t)blk * Q4K_BYTES;
        t.s = *(const uint4*)b;                 // d, dmin, scales[12]
        t.a = *(const uint4*)(b + 16 + 16 * p);  // qs[16p .. 16p+16)
    } else if constexpr (TYPE == T_Q6K) {
        const uint8_t* b = row + (size_t)blk * Q6K_BYTES;
        int h = p >> 1, lq = (p & 1) * 16;
        t.a = load16_a2(b + 64 * h + lq);
        t.b = load16_a2(b + 64 * h + 32 + lq);
        t.c = load16_a2(b + Q6K_QH + 32 * h + lq);
        t.s = load16_a2(b + Q6K_SC);
        t.e = *(const uint16_t*)(b + Q6K_D);
    } else {
        const uint8_t* b = row + (size_t)blk * Q8_0_BYTES;
        uintptr_t a = (uintptr_t)b;
        const uint32_t* q = (const uint32_t*)(a & ~(uintptr_t)3);
        t.a = *(const uint4*)q;
        t.b = *(const uint4*)(q + 4);
        t.e = q[8];
        t.c.x = (uint32_t)(a & 3u);  // 0 or 2
    }
}

// Byte i (0..3) of the 4-dword group as a variable index.
__device__ __forceinline__ uint32_t dw_sel(const uint4& v, uint32_t i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <int TYPE, int MB>
__device__ __forceinline__ void compute_task(const TaskData& t, int p, int blk_local, int m, int KC,
                                             const int8_t* __restrict__ lqs, const float* __restrict__ ld,
                                             const int* __restrict__ lbs, int nbc, float* acc) {
    if constexpr (TYPE == T_Q4K) {
        const float d = f16_to_f32(t.s.x & 0xffffu);
        const float dmin = f16_to_f32(t.s.x >> 16);
        const int j = p >> 1, half = p & 1;
        // get_scale_min_k4 (utils.rs:50-60) for sub-blocks 2j and 2j+1
        int sc0, m0, sc1, m1;
        if (j < 2) {
            sc0 = byte_of(t.s.y, 2 * j) & 63;
            m0 = byte_of(t.s.z, 2 * j) & 63;
            sc1 = byte_of(t.s.y, 2 * j + 1) & 63;
            m1 = byte_of(t.s.z, 2 * j + 1) & 63;
        } else {
            uint32_t i0 = 2 * j - 4, i1 = 2 * j - 3;
            sc0 = (byte_of(t.s.w, i0) & 0xF) | ((byte_of(t.s.y, i0) >> 6) << 4);
            m0 = (byte_of(t.s.w, i0) >> 4) | ((byte_of(t.s.z, i0) >> 6) << 4);
            sc1 = (byte_of(t.s.w, i1) & 0xF) | ((byte_of(t.s.y, i1) >> 6) << 4);
            m1 = (byte_of(t.s.w, i1) >> 4) | ((byte_of(t.s.z, i1) >> 6) << 4);
        }
        const uint32_t lo0 = t.a.x & 0x0F0F0F0Fu, lo1 = t.a.y & 0x0F0F0F0Fu, lo2 = t.a.z & 0x0F0F0F0Fu,
                       lo3 = t.a.w & 0x0F0F0F0Fu;
        const uint32_t hi0 = (t.a.x >> 4) & 0x0F0F0F0Fu, hi1 = (t.a.y >> 4) & 0x0F0F0F0Fu,
                       hi2 = (t.a.z >> 4) & 0x0F0F0F0Fu, hi3 = (t.a.w >> 4) & 0x0F0F0F0Fu;
        const int eoff = blk_local * 256 + 64 * j + 16 * half;
#pragma unroll
        for (int mi = 0; mi < MB; mi++) {
            if (mi < m) {
                const int8_t* xq = lqs + mi * KC + eoff;
                uint4 xl = *(const uint4*)xq;
                uint4 xh = *(const uint4*)(xq + 32);
                int sl = dot4(lo0, xl.x, 0);
                sl = dot4(lo1, xl.y, sl);
                sl = dot4(lo2, xl.z, sl);
                sl = dot4(lo3, xl.w, sl);
                int sh = dot4(hi0, xh.x, 0);
                sh = dot4(hi1, xh.y, sh);
                sh = dot4(hi2, xh.z, sh);
                sh = dot4(hi3, xh.w, sh);
                const int* bs = lbs + (mi * nbc + blk_local) * 16 + 4 * j + half;
                int S = sc0 * sl + sc1 * sh;
                int Mn = m0 * bs[0] + m1 * bs[2];
                float dy = ld[mi * nbc + blk_local];
                acc[mi] += dy * ((float)S * d - (float)Mn * dmin);
            }
        }
    } else if constexpr (TYPE == T_Q6K) {
        const float d = f16_to_f32(t.e);
        const int h = p >> 1, odd = p & 1;
        // q6 bytes of the 4 groups g (elements 128h + 32g + 16*odd + 0..15)
        uint32_t q[4][4];
        const uint32_t A[4] = {t.a.x, t.a.y, t.a.z, t.a.w};
        const uint32_t B[4] = {t.b.x, t.b.y, t.b.z, t.b.w};
        const uint32_t C[4] = {t.c.x, t.c.y, t.c.z, t.c.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            q[0][i] = (A[i] & 0x0F0F0F0Fu) | ((C[i] & 0x03030303u) << 4);
            q[1][i] = (B[i] & 0x0F0F0F0Fu) | (((C[i] >> 2) & 0x03030303u) << 4);
            q[2][i] = ((A[i] >> 4) & 0x0F0F0F0Fu) | (((C[i] >> 4) & 0x03030303u) << 4);
            q[3][i] = ((B[i] >> 4) & 0x0F0F0F0Fu) | (((C[i] >> 6) & 0x03030303u) << 4);
        }
        // scales[8h + 2g + odd]: dword 2h (g < 2) or 2h + 1, byte (2g + odd) & 3
        int sc[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t w = dw_sel(t.s, 2 * h + (g >> 1));
            sc[g] = (int)(int8_t)byte_of(w, (2 * g + odd) & 3);
        }
#pragma unroll
        for (int mi = 0; mi < MB; mi++) {
            if (mi < m) {
                int tot = 0;
                const int8_t* xb = lqs + mi * KC + blk_local * 256 + 128 * h + 16 * odd;
                const int* bs = lbs + (mi * nbc + blk_local) * 16 + 8 * h + odd;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    uint4 xv = *(const uint4*)(xb + 32 * g);
                    int s = dot4(q[g][0], xv.x, 0);
                    s = dot4(q[g][1], xv.y, s);
                    s = dot4(q[g][2], xv.z, s);
                    s = dot4(q[g][3], xv.w, s);
                    tot += sc[g] * (s - 32 * bs[2 * g]);
                }
                float dy = ld[mi * nbc + blk_local];
                acc[mi] += (d * dy) * (float)tot;
            }
        }
    } else {
        const uint32_t s = t.c.x;
        const float dx = f16_to_f32(s == 0 ? (t.a.x & 0xffffu) : (t.a.x >> 16));
        const uint32_t W[9] = {t.a.x, t.a.y, t.a.z, t.a.w, t.b.x, t.b.y, t.b.z, t.b.w, t.e};
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = s == 0 ? __builtin_amdgcn_alignbyte(W[i + 1], W[i], 2) : W[i + 1];
#pragma unroll
        for (int mi = 0; mi < MB; mi++) {
            if (mi < m) {
                const int8_t* xb = lqs + mi * KC + blk_local * 32;
                uint4 x0 = *(const uint4*)xb;
                uint4 x1 = *(const uint4*)(xb + 16);
                int sum = dot4(w[0], x0.x, 0);
                sum = dot4(w[1], x0.y, sum);
                sum = dot4(w[2], x0.z, sum);
                sum = dot4(w[3], x0.w, sum);
                sum = dot4(w[4], x1.x, sum);
                sum = dot4(w[5], x1.y, sum);
                sum = dot4(w[6], x1.z, sum);
                sum = dot4(w[7], x1.w, sum);
                acc[mi] += (float)sum * (dx * ld[mi * nbc + blk_local]);
            }
        }
    }
}

// Activation prologue, split in two so the x loads are issued before the
// weight loads (vmcnt retires loads in order: waiting for x must not mean
// waiting for the weights).  A wave quantizes up to XN blocks per chunk
// (XN <= XQ); the loads are unconditional (a block past the end reloads
// block 0) so no load sits under a branch.
constexpr int XQ = 8;

template <int VT, int XN>
__device__ __forceinline__ void prefetch_x(const float* __restrict__ x, int64_t K, int kc0, int KC, int m,
                                           float4 (&xv)[XN]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (VT == T_Q8K) {
        const int nbc = KC / 256, total = m * nbc;
#pragma unroll
        for (int i = 0; i < XN; i++) {
            const int b = wave + MV_WAVES * i;
            const int bb = b < total ? b : 0;
            const int mi = bb / nbc, sb = bb - mi * nbc;
            xv[i] = *(const float4*)(x + mi * K + kc0 + sb * 256 + 4 * lane);
        }
    } else {
        const int nbc = KC / 32, total = m * nbc;
#pragma unroll
        for (int i = 0; i < XN; i++) {
            const int b = wave * 8 + 8 * MV_WAVES * i + (lane >> 3);
            const int bb = b < total ? b : 0;
            const int mi = bb / nbc, bl = bb - mi * nbc;
            xv[i] = *(const float4*)(x + mi * K + kc0 + bl * 32 + 4 * (lane & 7));
        }
    }
}

// Quantize the prefetched blocks (every block exactly as from_float) into
// LDS: qs [m][KC], d [m][KC / block], Q8_K bsums [m][KC / 16].
template <int VT, int XN>
__device__ __forceinline__ void quantize_lds(const float4 (&xv)[XN], int KC, int m, int8_t* lqs, float* ld,
                                             int* lbs) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (VT == T_Q8K) {
        const int nbc = KC / 256, total = m * nbc;
#pragma unroll
        for (int i = 0; i < XN; i++) {
            const int b = wave + MV_WAVES * i;
            if (b < total) {  // wave-uniform
                const int mi = b / nbc, sb = b - mi * nbc;
                float d;
                int bs;
                const uint32_t q = q8k_block_wave(xv[i], &d, &bs);
                *(uint32_t*)(lqs + mi * KC + sb * 256 + 4 * lane) = q;
                if ((lane & 3) == 0) lbs[b * 16 + (lane >> 2)] = bs;
                if (lane == 0) ld[b] = d;
            }
        }
    } else {
        const int nbc = KC / 32, total = m * nbc;
#pragma unroll
        for (int i = 0; i < XN; i++) {
            const int b0 = wave * 8 + 8 * MV_WAVES * i;
            if (b0 < total) {  // wave-uniform; the 8-lane groups stay whole
                const int b = b0 + (lane >> 3), sub = lane & 7;
                uint16_t d16;
                const uint32_t q = q8_0_block_8lanes(xv[i], &d16);
                if (b < total) {
                    const int mi = b / nbc, bl = b - mi * nbc;
                    *(uint32_t*)(lqs + mi * KC + bl * 32 + 4 * sub) = q;
                    if (sub == 0) ld[b] = f16_to_f32(d16);
                }
            }
        }
    }
}

template <int TYPE, int MB, int R, int XN>
__global__ __launch_bounds__(MV_THREADS) void k_matvec(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                        float* __restrict__ Y, int n, int K, int m, int KC) {
    using Tr = MvTraits<TYPE>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * MV_WAVES + wave) * R;
    const int64_t rowbytes = (int64_t)(K / Tr::BE) * Tr::BB;
    const int nbc = KC / Tr::BE;
    int8_t* lqs = (int8_t*)smem;
    float* ld = (float*)(smem + m * KC);
    int* lbs = (int*)(ld + m * nbc);

    float acc[R][MB];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int mi = 0; mi < MB; mi++) acc[r][mi] = 0.0f;

    const int T = nbc * Tr::P;  // tasks per row per chunk
    for (int kc0 = 0; kc0 < K; kc0 += KC) {
        const int blk0 = kc0 / Tr::BE;
        if (kc0) __syncthreads();  // the previous chunk's readers are done with LDS
        float4 xv[XN];
        prefetch_x<Tr::VT, XN>(X, K, kc0, KC, m, xv);
        // first round of weight loads; rows past n and tasks past T load a
        // valid block (row n-1, task 0) and are never accumulated
        TaskData td[R];
        int ti = lane;
        const int t0 = ti < T ? ti : 0;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, n - 1);
            load_task<TYPE>(W + row * rowbytes, blk0 + t0 / Tr::P, t0 % Tr::P, td[r]);
        }
        quantize_lds<Tr::VT, XN>(xv, KC, m, lqs, ld, lbs);
        __syncthreads();
        for (; ti < T; ti += 64) {
            if (ti != lane) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int row = min(row0 + r, n - 1);
                    load_task<TYPE>(W + row * rowbytes, blk0 + ti / Tr::P, ti % Tr::P, td[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < R; r++)
                if (row0 + r < n)
                    compute_task<TYPE, MB>(td[r], ti % Tr::P, ti / Tr::P, m, KC, lqs, ld, lbs, nbc, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
#pragma unroll
        for (int mi = 0; mi < MB; mi++) {
            if (mi < m) {
                const float v = wave_sum(acc[r][mi]);
                if (lane == 0 && row < n) Y[(int64_t)mi * n + row] = v;
            }
        }
    }
}

// --------------------------------------------- Q4_K decode on int8 MFMA --
// For more activation rows the dot4 kernel turns ALU-bound; this one puts
// the per-sub-block dot on v_mfma_i32_16x16x32_i8.  A workgroup owns 16*NT
// weight rows (NT tiles of 16); its KS waves split the superblocks of K and
// add their partials through LDS.  Operands (k within one 32-element
// sub-block j, g = lane / 16):
//   A (activations): lane l holds x_q8[m = l%16][32j + 8g + 0..7]
//   B (weights):     lane l holds q4[n = l%16][32j + 8g + 0..7]
//   D:               lane l holds D[m = 4g + t][n = l%16], t = 0..3
// so the lane's four outputs all belong to its own weight row and the row's
// sub-block scale is a lane-local integer: acc += sc[j] * D_j.  The Q4_K min
// term sum_j m[j] * sum_{k in j} x_k is a second MFMA chain against the 6-bit
// mins broadcast to all 8 bytes, accumulated over the superblock in the
// MFMA's own C operand.  Activations come pre-quantized (Q8_K, bit-exact)
// from k_quantize_split_q8k, laid out so a lane's 64 bytes of a superblock
// (its 8 bytes of each sub-block) are contiguous: one A tile serves NT weight
// tiles.
typedef int v4i __attribute__((ext_vector_type(4)));

template <int KS, int NT>
__global__ __launch_bounds__(64 * KS) void k_mv_mfma_q4k(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                         const float* __restrict__ xd, float* __restrict__ Y, int n,
                                                         int K, int m) {
    __shared__ float4 part[KS > 1 ? KS - 1 : 1][NT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int nsb = K >> 8;
    const int64_t rowbytes = (int64_t)nsb * Q4K_BYTES;
    const uint8_t* wrow[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) wrow[t] = W + (int64_t)min(blockIdx.x * 16 * NT + 16 * t + c16, n - 1) * rowbytes;
    const bool arow_ok = c16 < m;
    const int8_t* xrow = xq + (int64_t)(arow_ok ? c16 : 0) * K + 64 * g;
    float out[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++) out[t][0] = out[t][1] = out[t][2] = out[t][3] = 0.0f;
    for (int sb = wave; sb < nsb; sb += KS) {
        uint4 hdr[NT];
        uint2 q[NT][4];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const uint8_t* b = wrow[t] + sb * Q4K_BYTES;
            hdr[t] = *(const uint4*)b;
#pragma unroll
            for (int c = 0; c < 4; c++) q[t][c] = *(const uint2*)(b + 16 + 32 * c + 8 * g);
        }
        // unconditional loads (row clamped above), zeroed by select: a load
        // under a divergent branch makes the compiler serialize them
        uint4 av[4];
#pragma unroll
        for (int i = 0; i < 4; i++) av[i] = *(const uint4*)(xrow + sb * 256 + 16 * i);
        const float4 dy = *(const float4*)(xd + sb * 16 + 4 * g);
        long a[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a[2 * i] = arow_ok ? (long)(((uint64_t)av[i].y << 32) | av[i].x) : 0l;
            a[2 * i + 1] = arow_ok ? (long)(((uint64_t)av[i].w << 32) | av[i].z) : 0l;
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float d = f16_to_f32(hdr[t].x & 0xffffu), dmin = f16_to_f32(hdr[t].x >> 16);
            v4i accs = {0, 0, 0, 0}, accm = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                int sc, mn;
                if (j < 4) {
                    sc = byte_of(hdr[t].y, j) & 63;
                    mn = byte_of(hdr[t].z, j) & 63;
                } else {
                    sc = (byte_of(hdr[t].w, j - 4) & 0xF) | ((byte_of(hdr[t].y, j - 4) >> 6) << 4);
                    mn = (byte_of(hdr[t].w, j - 4) >> 4) | ((byte_of(hdr[t].z, j - 4) >> 6) << 4);
                }
                const int c = j >> 1, sh = (j & 1) * 4;
                const uint32_t lo = (q[t][c].x >> sh) & 0x0F0F0F0Fu, hi = (q[t][c].y >> sh) & 0x0F0F0F0Fu;
                const long bw = (long)(((uint64_t)hi << 32) | lo);
                const v4i zero = {0, 0, 0, 0};
                const v4i dj = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], bw, zero, 0, 0, 0);
                const uint32_t mrep = (uint32_t)mn * 0x01010101u;
                const long bm = (long)(((uint64_t)mrep << 32) | mrep);
                accm = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], bm, accm, 0, 0, 0);
                accs[0] += sc * dj[0];
                accs[1] += sc * dj[1];
                accs[2] += sc * dj[2];
                accs[3] += sc * dj[3];
            }
            out[t][0] += dy.x * ((float)accs[0] * d - (float)accm[0] * dmin);
            out[t][1] += dy.y * ((float)accs[1] * d - (float)accm[1] * dmin);
            out[t][2] += dy.z * ((float)accs[2] * d - (float)accm[2] * dmin);
            out[t][3] += dy.w * ((float)accs[3] * d - (float)accm[3] * dmin);
        }
    }
    if (KS > 1) {
        if (wave != 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) part[wave - 1][t][lane] = make_float4(out[t][0], out[t][1], out[t][2], out[t][3]);
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int w = 0; w < KS - 1; w++)
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float4 p = part[w][t][lane];
                out[t][0] += p.x;
                out[t][1] += p.y;
                out[t][2] += p.z;
                out[t][3] += p.w;
            }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int nrow = blockIdx.x * 16 * NT + 16 * t + c16;
        if (nrow < n) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int mi = 4 * g + u;
                if (mi < m) Y[(int64_t)mi * n + nrow] = out[t][u];
            }
        }
    }
}

// Chunk of K staged in LDS at a time: the prologue quantizes at most
// XQ blocks per wave, m * KC <= XQ * MV_WAVES * 256 elements.
static int pick_kc(int type, int64_t K, int m) {
    const int be = type == T_Q8_0 ? 32 : 256;
    int64_t kc = (int64_t)XQ * MV_WAVES * 256 / m;
    kc -= kc % be;
    if (kc < be) kc = be;
    if (kc >= K) return (int)K;
    while (K % kc) kc -= be;  // chunks tile K exactly
    return (int)kc;
}

static size_t lds_bytes(int type, int KC, int m) {
    const int be = type == T_Q8_0 ? 32 : 256;
    size_t b = (size_t)m * KC + (size_t)m * (KC / be) * 4;
    if (type != T_Q8_0) b += (size_t)m * (KC / 16) * 4;
    return b;
}

template <int TYPE, int MB, int XN>
static void launch_xn(const void* w, const float* x, float* y, int n, int K, int m, int KC, hipStream_t s) {
    constexpr int R = 2;
    const size_t shm = lds_bytes(TYPE, KC, m);
    const dim3 grid((n + MV_WAVES * R - 1) / (MV_WAVES * R));
    hipLaunchKernelGGL((k_matvec<TYPE, MB, R, XN>), grid, dim3(MV_THREADS), shm, s, (const uint8_t*)w, x, y, n, K,
                       m, KC);
}

template <int TYPE, int MB>
static hipError_t launch_mb(const void* w, const float* x, float* y, int n, int K, int m, hipStream_t s) {
    const int KC = pick_kc(TYPE, K, m);
    // blocks a wave quantizes per chunk: 256 elements (Q8_K) or 8 lanes x 32 (Q8_0) per step
    const int per_step = TYPE == T_Q8_0 ? 32 * 8 * MV_WAVES : 256 * MV_WAVES;
    const int steps = (m * KC + per_step - 1) / per_step;
    if (steps <= 1) launch_xn<TYPE, MB, 1>(w, x, y, n, K, m, KC, s);
    else if (steps <= 2) launch_xn<TYPE, MB, 2>(w, x, y, n, K, m, KC, s);
    else if (steps <= 4) launch_xn<TYPE, MB, 4>(w, x, y, n, K, m, KC, s);
    else launch_xn<TYPE, MB, 8>(w, x, y, n, K, m, KC, s);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_type(const void* w, const float* x, float* y, int n, int K, int m, hipStream_t s) {
    if (m <= 1) return launch_mb<TYPE, 1>(w, x, y, n, K, m, s);
    if (m <= 2) return launch_mb<TYPE, 2>(w, x, y, n, K, m, s);
    if (m <= 4) return launch_mb<TYPE, 4>(w, x, y, n, K, m, s);
    if (m <= 8) return launch_mb<TYPE, 8>(w, x, y, n, K, m, s);
    return launch_mb<TYPE, 16>(w, x, y, n, K, m, s);
}

size_t matvec_workspace_bytes(int type, int64_t k, int64_t m) {
    if (type != T_Q4K || m <= MV_DOT_MAX_ROWS) return 0;
    return split_q8k_bytes(k, m);
}

hipError_t launch_matvec(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                         void* ws, hipStream_t s) {
    if (type == T_Q4K && m > MV_DOT_MAX_ROWS) {
        int8_t* xq;
        float* xd;
        split_q8k_ptrs(ws, k, m, &xq, &xd);
        hipError_t e = launch_quantize_split_q8k(x, m, k, xq, xd, s);
        if (e != hipSuccess) return e;
        constexpr int KS = 8, NT = 2;
        hipLaunchKernelGGL((k_mv_mfma_q4k<KS, NT>), dim3((unsigned)((n + 16 * NT - 1) / (16 * NT))), dim3(64 * KS),
                           0, s, (const uint8_t*)w, xq, xd, y, (int)n, (int)k, (int)m);
        return hipGetLastError();
    }
    switch (type) {
        case T_Q4K: return launch_type<T_Q4K>(w, x, y, (int)n, (int)k, (int)m, s);
        case T_Q6K: return launch_type<T_Q6K>(w, x, y, (int)n, (int)k, (int)m, s);
        case T_Q8_0: return launch_type<T_Q8_0>(w, x, y, (int)n, (int)k, (int)m, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace lloom
