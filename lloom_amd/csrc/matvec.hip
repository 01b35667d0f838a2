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
#include "kq_tasks.hpp"
#include "kq_mfma.hpp"
#include <cstdlib>

#include "kernels.hpp"

namespace lloom {

// The quantized activations of one task for one activation row.
template <int TYPE>
struct XTask;
template <>
struct XTask<T_Q4K> {
    uint4 xl, xh;
    int bs0, bs2;
    float dy;
};
template <>
struct XTask<T_Q6K> {
    uint4 xv[4];
    int bs[4];
    float dy;
};
template <>
struct XTask<T_Q8_0> {
    uint4 x0, x1;
    float dy;
};

template <int TYPE>
__device__ __forceinline__ void load_x(int p, int blk_local, int mi, int KC, int nbc, const int8_t* __restrict__ lqs,
                                       const float* __restrict__ ld, const int* __restrict__ lbs, XTask<TYPE>& x) {
    if constexpr (TYPE == T_Q4K) {
        const int j = p >> 1, half = p & 1;
        const int8_t* xq = lqs + mi * KC + blk_local * 256 + 64 * j + 16 * half;
        x.xl = *(const uint4*)xq;
        x.xh = *(const uint4*)(xq + 32);
        const int* bs = lbs + (mi * nbc + blk_local) * 16 + 4 * j + half;
        x.bs0 = bs[0];
        x.bs2 = bs[2];
        x.dy = ld[mi * nbc + blk_local];
    } else if constexpr (TYPE == T_Q6K) {
        const int h = p >> 1, odd = p & 1;
        const int8_t* xb = lqs + mi * KC + blk_local * 256 + 128 * h + 16 * odd;
        const int* bs = lbs + (mi * nbc + blk_local) * 16 + 8 * h + odd;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            x.xv[g] = *(const uint4*)(xb + 32 * g);
            x.bs[g] = bs[2 * g];
        }
        x.dy = ld[mi * nbc + blk_local];
    } else {
        const int8_t* xb = lqs + mi * KC + blk_local * 32;
        x.x0 = *(const uint4*)xb;
        x.x1 = *(const uint4*)(xb + 16);
        x.dy = ld[mi * nbc + blk_local];
    }
}

// One task's contribution: the exact integer block sums, then the f32
// scales in the CPU's order (k_quants.rs vec_dot).
template <int TYPE>
__device__ __forceinline__ float task_dot(const WPrep<TYPE>& w, const XTask<TYPE>& x) {
    if constexpr (TYPE == T_Q4K) {
        int sl = dot4(w.lo[0], x.xl.x, 0);
        sl = dot4(w.lo[1], x.xl.y, sl);
        sl = dot4(w.lo[2], x.xl.z, sl);
        sl = dot4(w.lo[3], x.xl.w, sl);
        int sh = dot4(w.hi[0], x.xh.x, 0);
        sh = dot4(w.hi[1], x.xh.y, sh);
        sh = dot4(w.hi[2], x.xh.z, sh);
        sh = dot4(w.hi[3], x.xh.w, sh);
        // |sl|, |sh| <= 16*15*128 and |bsum| <= 16*128: 24-bit multiplies
        const int S = __mul24(w.sc0, sl) + __mul24(w.sc1, sh);
        const int Mn = __mul24(w.m0, x.bs0) + __mul24(w.m1, x.bs2);
        return x.dy * ((float)S * w.d - (float)Mn * w.dmin);
    } else if constexpr (TYPE == T_Q6K) {
        int tot = 0;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int s = dot4(w.q[g][0], x.xv[g].x, 0);
            s = dot4(w.q[g][1], x.xv[g].y, s);
            s = dot4(w.q[g][2], x.xv[g].z, s);
            s = dot4(w.q[g][3], x.xv[g].w, s);
            tot += __mul24(w.sc[g], s - 32 * x.bs[g]);  // |s - 32 bs| < 2^18
        }
        return (w.d * x.dy) * (float)tot;
    } else {
        int sum = dot4(w.w[0], x.x0.x, 0);
        sum = dot4(w.w[1], x.x0.y, sum);
        sum = dot4(w.w[2], x.x0.z, sum);
        sum = dot4(w.w[3], x.x0.w, sum);
        sum = dot4(w.w[4], x.x1.x, sum);
        sum = dot4(w.w[5], x.x1.y, sum);
        sum = dot4(w.w[6], x.x1.z, sum);
        sum = dot4(w.w[7], x.x1.w, sum);
        return (float)sum * (w.d * x.dy);
    }
}

// Activation prologue, split in two so the x loads are issued before the
// weight loads (vmcnt retires loads in order: waiting for x must not mean
// waiting for the weights).  Each of the WV waves quantizes up to XN blocks
// per chunk; the loads are unconditional (a block past the end reloads
// block 0) so no load sits under a branch.
constexpr int XQ = 8;

// v / nbc for the block index v < 2^16 by a multiply-high: mg = ceil(2^32 /
// nbc) (exact while v * nbc < 2^32), or 0 for nbc = 1.  A runtime integer
// divide would sit in front of the first x load.
static uint32_t nbc_magic(int nbc) { return nbc <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + nbc - 1) / nbc); }
__device__ __forceinline__ int div_nbc(int v, uint32_t mg) { return mg ? (int)__umulhi((uint32_t)v, mg) : v; }

template <int VT, int WV, int XN>
__device__ __forceinline__ void prefetch_x(const float* __restrict__ x, int64_t K, int kc0, int KC, int m,
                                           uint32_t mg, float4 (&xv)[XN]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (VT == T_Q8K && XN % 4 == 0) {
        // four blocks a step, one per 16-lane row (q8k_block_row16): lane j
        // of row r holds elements 16j .. 16j+15 of block wave + WV*(4s + r)
        // in xv[4s .. 4s+3]
        const int nbc = KC / 256, total = m * nbc, j = lane & 15, r = lane >> 4;
#pragma unroll
        for (int st = 0; st < XN / 4; st++) {
            const int b = wave + WV * (4 * st + r);
            const int bb = b < total ? b : 0;
            const int mi = div_nbc(bb, mg), sb = bb - mi * nbc;
            const float4* src = (const float4*)(x + mi * K + kc0 + sb * 256 + 16 * j);
#pragma unroll
            for (int c = 0; c < 4; c++) xv[4 * st + c] = src[c];
        }
    } else if constexpr (VT == T_Q8K) {
        const int nbc = KC / 256, total = m * nbc;
#pragma unroll
        for (int i = 0; i < XN; i++) {
            const int b = wave + WV * i;
            const int bb = b < total ? b : 0;
            const int mi = div_nbc(bb, mg), sb = bb - mi * nbc;
            xv[i] = *(const float4*)(x + mi * K + kc0 + sb * 256 + 4 * lane);
        }
    } else {
        const int nbc = KC / 32, total = m * nbc;
#pragma unroll
        for (int i = 0; i < XN; i++) {
            const int b = wave * 8 + 8 * WV * i + (lane >> 3);
            const int bb = b < total ? b : 0;
            const int mi = div_nbc(bb, mg), bl = bb - mi * nbc;
            xv[i] = *(const float4*)(x + mi * K + kc0 + bl * 32 + 4 * (lane & 7));
        }
    }
}

// Quantize the prefetched blocks (every block exactly as from_float) into
// LDS: qs [m][KC], d [m][KC / block], Q8_K bsums [m][KC / 16].
template <int VT, int WV, int XN>
__device__ __forceinline__ void quantize_lds(const float4 (&xv)[XN], int KC, int m, uint32_t mg, int8_t* lqs,
                                             float* ld, int* lbs) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (VT == T_Q8K && XN % 4 == 0) {
        // the layout prefetch_x loads for four or more blocks a wave: the
        // 16-lane quantizer shares its two divisions and its reductions
        // among four blocks (Q6_K [2048, 8192]: one row 7.8 -> 7.2 us, two
        // rows 10.2 -> 8.8)
        const int nbc = KC / 256, total = m * nbc, j = lane & 15, r = lane >> 4;
#pragma unroll
        for (int st = 0; st < XN / 4; st++) {
            const int b = wave + WV * (4 * st + r);
            float xs[16];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 v = xv[4 * st + c];
                xs[4 * c] = v.x;
                xs[4 * c + 1] = v.y;
                xs[4 * c + 2] = v.z;
                xs[4 * c + 3] = v.w;
            }
            float d;
            int bs;
            const uint4 q = q8k_block_row16(xs, &d, &bs);  // unconditional, as below
            if (b < total) {
                const int mi = div_nbc(b, mg), sb = b - mi * nbc;
                *(uint4*)(lqs + mi * KC + sb * 256 + 16 * j) = q;
                lbs[b * 16 + j] = bs;
                if (j == 0) ld[b] = d;
            }
        }
    } else if constexpr (VT == T_Q8K) {
        const int nbc = KC / 256, total = m * nbc;
#pragma unroll
        for (int i = 0; i < XN; i++) {
            const int b = wave + WV * i;
            // computed unconditionally (a block past the end is a copy of
            // block 0), stored only if real: the x loads are then used on
            // every path and cannot sink below the weight loads
            float d;
            int bs;
            const uint32_t q = q8k_block_wave(xv[i], &d, &bs);
            if (b < total) {  // wave-uniform
                const int mi = div_nbc(b, mg), sb = b - mi * nbc;
                *(uint32_t*)(lqs + mi * KC + sb * 256 + 4 * lane) = q;
                if ((lane & 3) == 0) lbs[b * 16 + (lane >> 2)] = bs;
                if (lane == 0) ld[b] = d;
            }
        }
    } else {
        const int nbc = KC / 32, total = m * nbc;
#pragma unroll
        for (int i = 0; i < XN; i++) {
            const int b = wave * 8 + 8 * WV * i + (lane >> 3), sub = lane & 7;
            uint16_t d16;
            const uint32_t q = q8_0_block_8lanes(xv[i], &d16);  // unconditional, as above
            if (b < total) {
                const int mi = div_nbc(b, mg), bl = b - mi * nbc;
                *(uint32_t*)(lqs + mi * KC + bl * 32 + 4 * sub) = q;
                if (sub == 0) ld[b] = f16_to_f32(d16);
            }
        }
    }
}

// WV waves of R weight rows each; MB >= m activation rows; XN x blocks
// quantized per wave per chunk of KC elements of K.
template <int TYPE, int MB, int R, int WV, int XN, int PF>
__global__ __launch_bounds__(64 * WV) void k_matvec(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                     float* __restrict__ Y, int n, int K, int m, int KC,
                                                     uint32_t mg, int epi) {
    using Tr = MvTraits<TYPE>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * WV + wave) * R;
    const int64_t rowbytes = (int64_t)(K / Tr::BE) * Tr::BB;
    const int nbc = KC / Tr::BE;
    int8_t* lqs = (int8_t*)smem;
    float* ld = (float*)(smem + m * KC);
    int* lbs = (int*)(ld + m * nbc);
    // rows past n load row n-1 and are never stored
    const uint8_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; r++) wrow[r] = W + min(row0 + r, n - 1) * rowbytes;

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
        prefetch_x<Tr::VT, WV, XN>(X, K, kc0, KC, m, mg, xv);
        // With one or two Q8_K x blocks a wave (Q4_K: up to four, K <= 2048),
        // every wave's x load goes out ahead of any
        // wave's weight loads: a barrier between them.  Otherwise the waves'
        // issue interleaves, and a wave's x load (a cache hit) queues behind
        // other waves' weight loads (HBM misses) in the CU's memory pipeline,
        // holding up the quantization every dot waits for (C2 at B = 1:
        // 4.36 -> 4.07 us, B = 2 5.07 -> 4.52; with four blocks a wave, Q6_K
        // [2048, 8192], the barrier cost more than it saved: 7.81 -> 8.15,
        // and for Q8_0's short blocks too: C1 5.62 -> 5.72)
        if (TYPE != T_Q8_0 && (XN <= 2 || (TYPE == T_Q4K && KC <= 2048))) {  // uniform
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
        // weight loads of the first PF rounds of 64 tasks (tasks past T
        // load task 0, unused; every load is unconditional, so none sits
        // under a branch and the waits stay counted): rows of several rounds
        // (long K) keep PF rounds of loads in flight instead of one
        TaskData td[PF][R];
        auto issue = [&](int base) {
#pragma unroll
            for (int j = 0; j < PF; j++) {
                const int t = base + lane + 64 * j;
                const int tc = t < T ? t : 0;
#pragma unroll
                for (int r = 0; r < R; r++) load_task<TYPE>(wrow[r], blk0 + tc / Tr::P, tc % Tr::P, td[j][r]);
            }
        };
        issue(0);
        // every load above is issued before the quantization starts: the
        // scheduler would otherwise interleave them with the x math and
        // issue the last weight loads only after x has arrived
        __builtin_amdgcn_sched_barrier(0);
        quantize_lds<Tr::VT, WV, XN>(xv, KC, m, mg, lqs, ld, lbs);
        // The quantized x is in LDS once every wave's LDS writes are done:
        // a bare s_barrier after lgkmcnt(0).  __syncthreads() would also
        // wait for this wave's weight loads (vmcnt(0)), so every wave would
        // start its dots only when the slowest wave's weights had landed.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        for (int base = 0; base < T; base += 64 * PF) {
            if (base) issue(base);
#pragma unroll
            for (int j = 0; j < PF; j++) {
                const int t = base + lane + 64 * j;
                if (t < T) {
                    const int p = t % Tr::P, bl = t / Tr::P;
                    WPrep<TYPE> wp[R];
#pragma unroll
                    for (int r = 0; r < R; r++) prep_task<TYPE>(td[j][r], p, wp[r]);
#pragma unroll
                    for (int mi = 0; mi < MB; mi++) {
                        if (mi < m) {
                            XTask<TYPE> xt;
                            load_x<TYPE>(p, bl, mi, KC, nbc, lqs, ld, lbs, xt);
#pragma unroll
                            for (int r = 0; r < R; r++) acc[r][mi] += task_dot<TYPE>(wp[r], xt);
                        }
                    }
                }
            }
        }
    }
    if constexpr (R * MB <= 8) {
        // all R * MB sums in one butterfly (item = r * MB + mi)
        float v[R * MB];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int mi = 0; mi < MB; mi++) v[r * MB + mi] = acc[r][mi];
        const float tot = wave_sum_items<R * MB>(v);
        const int item = wave_sum_item_of_lane();
        const int r = item / MB, mi = item % MB;
        if ((lane & 7) == 0 && item < R * MB && mi < m && row0 + r < n) store_epi(&Y[(int64_t)mi * n + row0 + r], tot, epi);
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
#pragma unroll
            for (int mi = 0; mi < MB; mi++) {
                if (mi < m) {
                    const float v = wave_sum(acc[r][mi]);
                    if (lane == 0 && row < n) store_epi(&Y[(int64_t)mi * n + row], v, epi);
                }
            }
        }
    }
}

// ------------------------------------- Q4_K / Q6_K decode on int8 MFMA --
// For more activation rows the dot4 kernel turns ALU-bound; this one puts
// the sub-block dots on v_mfma_i32_16x16x32_i8.  A workgroup owns 16*NT
// weight rows (NT tiles of 16); its KS waves split the superblocks of K and
// add their partials through LDS.  Operands (k within one 32-element chunk
// j of a superblock, g = lane / 16):
//   A (activations): lane l holds x_q8[m = l%16][32j + 8g + 0..7]
//   B (weights):     lane l holds q[n = l%16][32j + 8g + 0..7]
//   D:               lane l holds D[m = 4g + t][n = l%16], t = 0..3
// so the lane's four outputs all belong to its own weight row and the row's
// sub-block scales are lane-local integers.
//  * Q4_K: a chunk is one sub-block: acc += sc[j] * D_j; the min term
//    sum_j m[j] * sum_{k in j} x_k is a second MFMA chain against the 6-bit
//    mins broadcast to all 8 bytes, accumulated in the MFMA's C operand.
//  * Q6_K: a chunk holds sub-blocks 2j (g < 2) and 2j+1 (g >= 2); the q - 32
//    values are int8 already, and two MFMAs with the other half of B zeroed
//    give each sub-block its own sum for its signed 8-bit scale.
// Activations come pre-quantized (Q8_K, bit-exact) from
// k_quantize_split_q8k, laid out so a lane's 64 bytes of a superblock (its
// 8 bytes of each chunk) are contiguous: one A tile serves NT weight tiles.
// The loads of a wave's next superblock are issued before the current one
// is computed.  The per-superblock arithmetic (mf_compute,
// mf_compute_q4k_b) is in kq_mfma.hpp.

// MA > 1 (prefill): a workgroup layer (grid y) covers MA 16-row activation
// tiles against the same weight tiles, so each weight superblock is unpacked
// once for 16 MA activation rows; the activation operands then load at the
// top of each superblock instead of one superblock ahead.
template <int TYPE, int KS, int NT, int MA>
__global__ __launch_bounds__(64 * KS) void k_mv_mfma(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                     const float* __restrict__ xd, float* __restrict__ Y, int n,
                                                     int K, int m, int mp, int epi, int sbs,
                                                     float* __restrict__ psum) {
    constexpr int BB = TYPE == T_Q4K ? Q4K_BYTES : Q6K_BYTES;
    __shared__ float4 part[KS > 1 ? KS - 1 : 1][NT][MA][64];
    __shared__ __align__(16) uint8_t mft[KS][NT][16 * MfRs<TYPE>::V];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    // split K (grid z): this workgroup's superblocks [sb0, nsb), its sums to
    // psum[z] for k_sum_splits
    const int nsb_all = K >> 8;
    const int sb0 = blockIdx.z * sbs, nsb = min(sb0 + sbs, nsb_all);
    const int64_t rowbytes = (int64_t)nsb_all * BB;
    const uint8_t* wrow[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) wrow[t] = W + (int64_t)min(blockIdx.x * 16 * NT + 16 * t + c16, n - 1) * rowbytes;
    const int mt0 = blockIdx.y * MA;  // first activation tile of this layer
    bool arow_ok[MA];
    const int8_t* xrow[MA];
#pragma unroll
    for (int u = 0; u < MA; u++) {
        const int ar = 16 * (mt0 + u) + c16;
        arow_ok[u] = ar < m;
        xrow[u] = xq + (int64_t)(arow_ok[u] ? ar : 0) * K + 64 * g;
    }
    float out[NT][MA][4];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int u = 0; u < MA; u++) out[t][u][0] = out[t][u][1] = out[t][u][2] = out[t][u][3] = 0.0f;

    // registers of the superblock in flight (the row and superblock
    // indices are clamped, so no load sits under a divergent branch)
    MfL<TYPE> wc[NT];
    uint4 avc[MA == 1 ? 4 : 1];
    float4 dyc;
    auto issue = [&](int sb, MfL<TYPE>(&w)[NT], uint4(&av)[MA == 1 ? 4 : 1], float4& dy) {
        const int sbc = min(sb, nsb - 1);
#pragma unroll
        for (int t = 0; t < NT; t++) mf_load_l<TYPE>(wrow[t] + (int64_t)sbc * BB, g, w[t]);
        if constexpr (MA == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = *(const uint4*)(xrow[0] + sbc * 256 + 16 * i);
            dy = *(const float4*)(xd + (int64_t)sbc * mp + 16 * mt0 + 4 * g);
        }
    };
    issue(sb0 + wave, wc, avc, dyc);
    for (int sb = sb0 + wave; sb < nsb; sb += KS) {
        // the next superblock's loads, when this wave has one (wave-uniform)
        const bool more = sb + KS < nsb;
        MfL<TYPE> wn[NT];
        uint4 avn[MA == 1 ? 4 : 1];
        float4 dyn;
        if (more) issue(sb + KS, wn, avn, dyn);
        MfW<TYPE> wu[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) mf_unpack<TYPE>(wc[t], &mft[wave][t][0], g, c16, wu[t]);
        if constexpr (MA == 1) {
            // activation rows past m are zeroed by select (a load under a
            // divergent branch would serialize the waits)
            long a[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a[2 * i] = arow_ok[0] ? (long)(((uint64_t)avc[i].y << 32) | avc[i].x) : 0l;
                a[2 * i + 1] = arow_ok[0] ? (long)(((uint64_t)avc[i].w << 32) | avc[i].z) : 0l;
            }
#pragma unroll
            for (int t = 0; t < NT; t++) mf_compute<TYPE>(wu[t], a, dyc, g, out[t][0]);
        } else {
            uint4 av[MA][4];
            float4 dy[MA];
#pragma unroll
            for (int u = 0; u < MA; u++) {
#pragma unroll
                for (int i = 0; i < 4; i++) av[u][i] = *(const uint4*)(xrow[u] + sb * 256 + 16 * i);
                dy[u] = *(const float4*)(xd + (int64_t)sb * mp + 16 * (mt0 + u) + 4 * g);
            }
#pragma unroll
            for (int u = 0; u < MA; u++) {
                if (16 * (mt0 + u) < m) {  // uniform: a tile wholly past m is skipped
                    long a[8];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        a[2 * i] = arow_ok[u] ? (long)(((uint64_t)av[u][i].y << 32) | av[u][i].x) : 0l;
                        a[2 * i + 1] = arow_ok[u] ? (long)(((uint64_t)av[u][i].w << 32) | av[u][i].z) : 0l;
                    }
#pragma unroll
                    for (int t = 0; t < NT; t++) mf_compute<TYPE>(wu[t], a, dy[u], g, out[t][u]);
                }
            }
        }
        if (!more) break;
#pragma unroll
        for (int t = 0; t < NT; t++) wc[t] = wn[t];
        if constexpr (MA == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) avc[i] = avn[i];
            dyc = dyn;
        }
    }
    if (KS > 1) {
        if (wave != 0) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int u = 0; u < MA; u++)
                    part[wave - 1][t][u][lane] = make_float4(out[t][u][0], out[t][u][1], out[t][u][2], out[t][u][3]);
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int w = 0; w < KS - 1; w++)
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int u = 0; u < MA; u++) {
                    const float4 p = part[w][t][u][lane];
                    out[t][u][0] += p.x;
                    out[t][u][1] += p.y;
                    out[t][u][2] += p.z;
                    out[t][u][3] += p.w;
                }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int nrow = blockIdx.x * 16 * NT + 16 * t + c16;
        if (nrow < n) {
#pragma unroll
            for (int u = 0; u < MA; u++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int mi = 16 * (mt0 + u) + 4 * g + v;
                    if (mi < m) {
                        if (psum) psum[((int64_t)blockIdx.z * m + mi) * n + nrow] = out[t][u][v];
                        else store_epi(&Y[(int64_t)mi * n + nrow], out[t][u][v], epi);
                    }
                }
        }
    }
}

// ----------------------------- 3..4 rows in one launch (short K) --
// The MFMA decode with the activation quantization inside: a workgroup of
// 16 waves owns 32 weight rows (two 16-row tiles) and K of KS = k / 256
// superblocks (4 or 8); wave (tile, sb) first issues its superblock's weight
// loads, then the workgroup quantizes all m x KS blocks of x into LDS in the
// MFMA operand layout (Q8_K, bit-exact, at most two blocks per wave), and
// after one barrier each wave runs its superblock's MFMAs; the KS partials
// of a row meet in LDS.  For m <= 4 this saves the quantizer's launch; with
// more rows every workgroup re-reading B x k f32 of x costs more than that
// launch (measured: 6.2 us against 7.3 us at m = 3, 10.3 against 8.4 at
// m = 16, n = 6144, k = 2048).  Per output the arithmetic is k_mv_mfma's,
// so the results are bit-identical to it.
constexpr int FUSED_MAX_ROWS = 4;

template <int TYPE, int KS>
__global__ __launch_bounds__(128 * KS) void k_mv_fused(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                       float* __restrict__ Y, int n, int m, int epi) {
    constexpr int BB = TYPE == T_Q4K ? Q4K_BYTES : Q6K_BYTES;
    constexpr int WV = 2 * KS, K = 256 * KS;
    constexpr int XN = (FUSED_MAX_ROWS * KS + WV - 1) / WV;  // blocks quantized per wave
    __shared__ __align__(16) int8_t xs[KS][16][256];
    __shared__ __align__(16) float dl[KS][16];
    __shared__ __align__(16) uint8_t mft[WV][16 * MfRs<TYPE>::V];
    __shared__ float4 red[KS - 1][2][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int kw = wave % KS, rt = wave / KS;
    const int row = (blockIdx.x * 2 + rt) * 16 + c16;
    const uint8_t* wrow = W + (int64_t)min(row, n - 1) * ((int64_t)KS * BB);
    // x blocks q = mi * KS + sb, q = wave + WV * t (a block past the end
    // reloads block 0 and is not stored); every wave's x loads go out ahead
    // of every weight load (a barrier between them), so the quantization
    // does not wait behind other waves' weight loads in the CU's memory
    // pipeline
    const int nblk = m * KS;
    float4 xv[XN];
#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int q = wave + WV * t;
        const int qq = q < nblk ? q : 0;
        xv[t] = *(const float4*)(X + (int64_t)(qq / KS) * K + (qq % KS) * 256 + 4 * lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    MfL<TYPE> wl;
    mf_load_l<TYPE>(wrow + (int64_t)kw * BB, g, wl);
    __builtin_amdgcn_sched_barrier(0);
    // element 4*lane.. of a block: sub-block lane / 8, lane group (lane % 8) / 2,
    // byte 4 * (lane % 2) of the group's 8 (k_quantize_split_q8k's layout)
    const int off = 64 * ((lane & 7) >> 1) + 8 * (lane >> 3) + 4 * (lane & 1);
#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int q = wave + WV * t;
        float d;
        int bs;
        const uint32_t qv = q8k_block_wave(xv[t], &d, &bs);
        if (q < nblk) {  // wave-uniform
            *(uint32_t*)(&xs[q % KS][q / KS][off]) = qv;
            if (lane == 0) dl[q % KS][q / KS] = d;
        }
    }
    MfW<TYPE> wu;
    mf_unpack<TYPE>(wl, &mft[wave][0], g, c16, wu);
    __syncthreads();
    const bool arow_ok = c16 < m;
    long a[8];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint4 v = *(const uint4*)(&xs[kw][c16][64 * g + 16 * c]);
        a[2 * c] = arow_ok ? (long)(((uint64_t)v.y << 32) | v.x) : 0l;
        a[2 * c + 1] = arow_ok ? (long)(((uint64_t)v.w << 32) | v.z) : 0l;
    }
    const float4 dy = *(const float4*)(&dl[kw][4 * g]);
    float out[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    mf_compute<TYPE>(wu, a, dy, g, out);
    if (kw) red[kw - 1][rt][lane] = make_float4(out[0], out[1], out[2], out[3]);
    __syncthreads();
    if (kw) return;
#pragma unroll
    for (int w = 0; w < KS - 1; w++) {
        const float4 p = red[w][rt][lane];
        out[0] += p.x;
        out[1] += p.y;
        out[2] += p.z;
        out[3] += p.w;
    }
    if (row < n) {
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (4 * g + u < m) store_epi(&Y[(int64_t)(4 * g + u) * n + row], out[u], epi);
    }
}

template <int TYPE>
static hipError_t launch_fused(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, int epi,
                               hipStream_t s) {
    const dim3 grid((unsigned)((n + 31) / 32));
    if (k == 2048)
        hipLaunchKernelGGL((k_mv_fused<TYPE, 8>), grid, dim3(1024), 0, s, (const uint8_t*)w, x, y, (int)n, (int)m, epi);
    else
        hipLaunchKernelGGL((k_mv_fused<TYPE, 4>), grid, dim3(512), 0, s, (const uint8_t*)w, x, y, (int)n, (int)m, epi);
    return hipGetLastError();
}

// Chunk of K staged in LDS at a time: the prologue quantizes at most
// XQ blocks per wave, m * KC <= XQ * WV * 256 elements.
static int pick_kc(int type, int64_t K, int m, int wv) {
    const int be = type == T_Q8_0 ? 32 : 256;
    int64_t kc = (int64_t)XQ * wv * 256 / m;
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

template <int TYPE, int MB, int WV, int R, int PF>
static void launch_xn(int steps, dim3 grid, dim3 block, size_t shm, hipStream_t s, const uint8_t* wb, const float* x,
                      float* y, int n, int K, int m, int KC, uint32_t mg, int epi) {
    if (steps <= 1) hipLaunchKernelGGL((k_matvec<TYPE, MB, R, WV, 1, PF>), grid, block, shm, s, wb, x, y, n, K, m, KC, mg, epi);
    else if (steps <= 2) hipLaunchKernelGGL((k_matvec<TYPE, MB, R, WV, 2, PF>), grid, block, shm, s, wb, x, y, n, K, m, KC, mg, epi);
    else if (steps <= 4) hipLaunchKernelGGL((k_matvec<TYPE, MB, R, WV, 4, PF>), grid, block, shm, s, wb, x, y, n, K, m, KC, mg, epi);
    else hipLaunchKernelGGL((k_matvec<TYPE, MB, R, WV, 8, PF>), grid, block, shm, s, wb, x, y, n, K, m, KC, mg, epi);
}

template <int TYPE, int MB, int WV, int R>
static hipError_t launch_cfg(const void* w, const float* x, float* y, int n, int K, int m, int epi, hipStream_t s) {
    const int KC = pick_kc(TYPE, K, m, WV);
    // blocks a wave quantizes per chunk: 256 elements (Q8_K) or 8 lanes x 32 (Q8_0) per step
    const int per_step = TYPE == T_Q8_0 ? 32 * 8 * WV : 256 * WV;
    const int steps = (m * KC + per_step - 1) / per_step;
    const size_t shm = lds_bytes(TYPE, KC, m);
    const dim3 grid((n + WV * R - 1) / (WV * R)), block(64 * WV);
    const uint8_t* wb = (const uint8_t*)w;
    const uint32_t mg = nbc_magic(KC / (TYPE == T_Q8_0 ? 32 : 256));
    // rows of more than one round of 64 tasks keep several rounds of loads
    // in flight with one or two rows a wave; Q6_K's four-group tasks hold
    // more registers: two rounds with one row a wave (8.11 -> 7.93 us on
    // [2048, 8192]), one otherwise
    const int tasks = (KC / MvTraits<TYPE>::BE) * MvTraits<TYPE>::P;
    constexpr int PFL = TYPE == T_Q6K ? (R == 1 ? 2 : 1) : R == 1 ? 4 : R == 2 ? 2 : 1;
    if (PFL > 1 && tasks > 64)
        launch_xn<TYPE, MB, WV, R, PFL>(steps, grid, block, shm, s, wb, x, y, n, K, m, KC, mg, epi);
    else
        launch_xn<TYPE, MB, WV, R, 1>(steps, grid, block, shm, s, wb, x, y, n, K, m, KC, mg, epi);
    return hipGetLastError();
}

// One or two activation rows: 8 waves per workgroup, each wave R rows, R
// chosen so the grid is about one workgroup per CU (each workgroup
// quantizes x once; fewer, fuller workgroups quantize it fewer times).
template <int TYPE, int MB>
static hipError_t launch_small(const void* w, const float* x, float* y, int n, int K, int m, int epi, hipStream_t s) {
    // Q8_0 rows are short tasks (a 34-byte block each): its loads fill the
    // memory pipe with fewer rows a wave and more workgroups, about 1024 for
    // one activation row and 512 for two (C1, [8192, 2048]: 5.9 us against
    // 6.4 with four rows a wave)
    const int per_wg = TYPE == T_Q8_0 ? 8 * 1024 / MB : 8 * 256;
    const int r = (n + per_wg - 1) / per_wg;
    if (r <= 1) return launch_cfg<TYPE, MB, 8, 1>(w, x, y, n, K, m, epi, s);
    if (r <= 2) return launch_cfg<TYPE, MB, 8, 2>(w, x, y, n, K, m, epi, s);
    if (r <= 3) return launch_cfg<TYPE, MB, 8, 3>(w, x, y, n, K, m, epi, s);
    return launch_cfg<TYPE, MB, 8, 4>(w, x, y, n, K, m, epi, s);
}

template <int TYPE>
static hipError_t launch_type(const void* w, const float* x, float* y, int n, int K, int m, int epi, hipStream_t s) {
    if (m <= 1) return launch_small<TYPE, 1>(w, x, y, n, K, m, epi, s);
    if (m <= 2) return launch_small<TYPE, 2>(w, x, y, n, K, m, epi, s);
    if constexpr (TYPE == T_Q4K) {
        if (m <= 3) return launch_small<TYPE, 3>(w, x, y, n, K, m, epi, s);
        return launch_small<TYPE, 4>(w, x, y, n, K, m, epi, s);
    }
    if (m <= 4) return launch_cfg<TYPE, 4, 4, 2>(w, x, y, n, K, m, epi, s);
    if (m <= 8) return launch_cfg<TYPE, 8, 4, 2>(w, x, y, n, K, m, epi, s);
    return launch_cfg<TYPE, 16, 4, 2>(w, x, y, n, K, m, epi, s);
}

// Splits of K across workgroups for the 16-wave shape (fewer 16-row tiles
// than CUs and a long K): enough to reach ~256 workgroups, at least 16
// superblocks (one a wave) each.
static int mv_splits(int64_t n, int64_t k) {
    const int64_t tiles = (n + 15) / 16, nsb = k / 256;
    if (n >= 16 * 256 || k < 16 * 256) return 1;
    int sp = 1;
    while (sp < 4 && tiles * sp * 2 <= 256 && nsb / (sp * 2) >= 16) sp *= 2;
    return sp;
}

size_t matvec_workspace_bytes(int type, int64_t n, int64_t k, int64_t m) {
    if (mv_stream_fits(type, n, k, m)) return (split_q8k_bytes(k, m) + 255) & ~(size_t)255;
    if (type == T_Q8_0 || m <= MV_DOT_MAX_ROWS) return 0;
    const size_t q = (split_q8k_bytes(k, m) + 255) & ~(size_t)255;
    const int sp = mv_splits(n, k);
    return q + (sp > 1 ? (size_t)sp * m * n * sizeof(float) : 0);
}

// The split-K partial sums after the quantized activations in the workspace.
static float* mv_psum(void* ws, int64_t k, int64_t m) {
    return (float*)((uint8_t*)ws + ((split_q8k_bytes(k, m) + 255) & ~(size_t)255));
}

// The split-K partial sums of k_mv_mfma, added in split order, then the
// call's store epilogue.
__global__ __launch_bounds__(256) void k_sum_splits(const float* __restrict__ psum, int splits, int64_t mn,
                                                    float* __restrict__ Y, int epi) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= mn) return;
    float v = psum[i];
    for (int z = 1; z < splits; z++) v += psum[z * mn + i];
    store_epi(&Y[i], v, epi);
}

// ------------------- 3..128 rows, K <= 2048: weight DMAs, tiled activations --
// Every weight byte goes to LDS as global_load_lds DMAs of 1 KB a wave
// instruction, so every load instruction covers eight whole cache lines;
// loading the MFMA operand layout straight from global memory (16 rows x 48
// bytes an instruction) multiplies the memory requests and cost ~2 us of a
// ~6 us call in the kernel before this one.
constexpr int MV_DMA_KMAX = 2048;

__device__ __forceinline__ void dma16(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// LDS pitch of a row of `bytes` (a multiple of 16): padded so that its
// dword count is 4 mod 8 (mod 32 banks: rows r and r + 8 share banks, so a
// 16-row b128 read takes two passes instead of sixteen).
constexpr int lds_pitch(int bytes) {
    int p = (bytes + 15) & ~15;
    while ((p / 4) % 8 != 4) p += 16;
    return p;
}

// DMA of `rows` rows of `bytes` bytes (global row stride `gstride`) into
// LDS rows of pitch P: the LDS image is cut in 1 KB wave instructions; a
// lane's 16 bytes are data of one row or pad (pad lanes reload the last
// data piece).  `lim` clamps every source offset to the valid bytes.
template <int P, int WV>
__device__ __forceinline__ void dma_rows(const uint8_t* __restrict__ src, int bytes, int rows, int64_t gstride, int lim,
                                         uint8_t* lds, int wave, int lane) {
    const int total = rows * P;
    for (int i = wave; i * 1024 < total; i += WV) {
        const int L = i * 1024 + 16 * lane;
        const int r = L / P, c = L - r * P;
        const int64_t off = (int64_t)r * gstride + min(c, bytes - 16);
        dma16(src + min(off, (int64_t)lim), lds + i * 1024);
    }
}

// LLOOM_HIP_MV_DMA: 0 = off (k_mv_mfma), 1 / 2 = weight tiles a workgroup,
// unset = two from 384 weight tiles up (n >= 6144), one below (fewer
// workgroups than CUs: n = 2048, m = 16 6.97 against 6.17 us with one)
static int mv_dma_env() {
    static const int v = [] {
        const char* e = getenv("LLOOM_HIP_MV_DMA");
        return e ? atoi(e) : -1;
    }();
    return v;
}
static bool mv_dma_on() { return mv_dma_env() != 0; }
static int mv_dma_nt(int64_t tiles) { return mv_dma_env() > 0 ? mv_dma_env() : tiles >= 384 ? 2 : 1; }

// Q4_K / Q6_K with k <= 2048 on 16-row activation tiles, from 3 rows
// (decode) to 128 (short prefill; Q6_K to 16): MA 16-row activation tiles
// (16 MA >= m) against NT 16-row weight tiles, one superblock a wave (NSB
// waves), so every unpacked weight superblock serves the MA activation
// tiles and every activation operand the NT weight tiles.  The weights move
// as 1 KB DMAs of whole rows into padded LDS rows; the activations, MA times
// the bytes of a decode call, skip LDS: each wave loads its superblock's
// operands from the tiled layout of k_quantize_split_q8k straight into
// registers, 1 KB of contiguous bytes an instruction, issued with the DMAs.
// The NSB partial sums of each (weight tile, activation tile) meet in LDS
// and are added in superblock order, one pair a wave.  Rows past m in the
// last tile read the tile's padding and are never stored (an activation row
// of the MFMA reaches only its own outputs).
template <int TYPE, int NSB, int NT, int MA>
__global__ __launch_bounds__(64 * NSB) void k_mv_dma_ma(const uint8_t* __restrict__ W, const int8_t* __restrict__ xt,
                                                      const float* __restrict__ xd, const int8_t* __restrict__ bsp,
                                                      float* __restrict__ Y, int n, int m, int mp, int epi) {
    constexpr int BB = TYPE == T_Q4K ? Q4K_BYTES : Q6K_BYTES, RB = NSB * BB;
    static_assert(NSB <= 8, "one superblock a wave, at most 8 waves");
    static_assert(RB % 16 == 0, "rows must be whole 16-byte DMA pieces");
    constexpr int WP = lds_pitch(RB);
    __shared__ __align__(16) uint8_t wl[NT][16 * WP + 1024];
    __shared__ float4 part[NSB][NT * MA][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int sb = wave;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int r0 = (blockIdx.x * NT + t) * 16;
        const int valid = max(1, min(16, n - r0));
        dma_rows<WP, NSB>(W + (int64_t)min(r0, n - 1) * RB, RB, 16, RB, (valid * RB - 1) & ~15, &wl[t][0], wave,
                          lane);
    }
    const int tiles = mp >> 4;  // activation tiles present (the rest load the last)
    uint4 xv[MA][4];
    float4 dy[MA];
    long ab[MA];
#pragma unroll
    for (int a = 0; a < MA; a++) {
        const int at = min(a, tiles - 1);
        const int8_t* src = xt + ((int64_t)(at * NSB + sb) * 4) * 1024 + 16 * lane;
#pragma unroll
        for (int i = 0; i < 4; i++) xv[a][i] = *(const uint4*)(src + 1024 * i);
        dy[a] = *(const float4*)(xd + (int64_t)sb * mp + 16 * at + 4 * g);
        if constexpr (TYPE == T_Q4K) {
            // groups 0 and 1 read the lo and hi sums of row c16 (masked past
            // m; loaded by every lane: a load under the condition would wait
            // for the DMAs in flight)
            const long v = *(const long*)(bsp + ((int64_t)sb * mp + 16 * at + c16) * 16 + 8 * min(g, 1));
            ab[a] = v & -(long)(g < 2 && 16 * a + c16 < m);
        } else {
            ab[a] = 0;
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; t++) {
        MfW<TYPE> wu;
        mf_load<TYPE>(&wl[t][c16 * WP] + sb * BB, g, wu);
#pragma unroll
        for (int a = 0; a < MA; a++) {
            long av[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4 v = xv[a][i];
                av[2 * i] = (long)(((uint64_t)v.y << 32) | v.x);
                av[2 * i + 1] = (long)(((uint64_t)v.w << 32) | v.z);
            }
            float out[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (TYPE == T_Q4K) mf_compute_q4k_b(wu, av, ab[a], dy[a], g, out);
            else mf_compute<TYPE>(wu, av, dy[a], g, out);
            part[sb][t * MA + a][lane] = make_float4(out[0], out[1], out[2], out[3]);
        }
    }
    __syncthreads();
    for (int pr = wave; pr < NT * MA; pr += NSB) {  // uniform
        const int t = pr / MA, a = pr - t * MA;
        float4 acc = part[0][pr][lane];
#pragma unroll
        for (int w = 1; w < NSB; w++) {
            const float4 p = part[w][pr][lane];
            acc.x += p.x;
            acc.y += p.y;
            acc.z += p.z;
            acc.w += p.w;
        }
        const int row = (blockIdx.x * NT + t) * 16 + c16;
        const float o[4] = {acc.x, acc.y, acc.z, acc.w};
        if (row < n) {
#pragma unroll
            for (int v = 0; v < 4; v++)
                if (16 * a + 4 * g + v < m) store_epi(&Y[(int64_t)(16 * a + 4 * g + v) * n + row], o[v], epi);
        }
    }
}

template <int TYPE, int NSB, int MA>
static hipError_t launch_mv_dma_ma_k(const void* w, float* y, int64_t n, int64_t m, const int8_t* xt,
                                     const float* xd, const int8_t* bsp, int epi, hipStream_t s) {
    const int mp = (int)((m + 15) & ~(int64_t)15);
    const int64_t tiles = (n + 15) / 16;
    // two weight tiles a workgroup from 384 weight tiles up to four
    // activation tiles; past that one, so the partial sums fit LDS
    constexpr bool two = MA <= 4;
    if (two && mv_dma_nt(tiles) == 2)
        hipLaunchKernelGGL((k_mv_dma_ma<TYPE, NSB, two ? 2 : 1, MA>), dim3((unsigned)((tiles + 1) / 2)), dim3(64 * NSB),
                           0, s, (const uint8_t*)w, xt, xd, bsp, y, (int)n, (int)m, mp, epi);
    else
        hipLaunchKernelGGL((k_mv_dma_ma<TYPE, NSB, 1, MA>), dim3((unsigned)tiles), dim3(64 * NSB), 0, s,
                           (const uint8_t*)w, xt, xd, bsp, y, (int)n, (int)m, mp, epi);
    return hipGetLastError();
}

template <int MA>
static hipError_t launch_mv_dma_ma_m(int type, const void* w, float* y, int64_t n, int64_t k, int64_t m,
                                     const int8_t* xt, const float* xd, const int8_t* bsp, int epi, hipStream_t s) {
    if (type == T_Q6K) {
        if constexpr (MA == 1) return launch_mv_dma_ma_k<T_Q6K, 8, 1>(w, y, n, m, xt, xd, bsp, epi, s);
        return hipErrorInvalidValue;
    }
    switch (k / 256) {
        case 1: return launch_mv_dma_ma_k<T_Q4K, 1, MA>(w, y, n, m, xt, xd, bsp, epi, s);
        case 2: return launch_mv_dma_ma_k<T_Q4K, 2, MA>(w, y, n, m, xt, xd, bsp, epi, s);
        case 3: return launch_mv_dma_ma_k<T_Q4K, 3, MA>(w, y, n, m, xt, xd, bsp, epi, s);
        case 4: return launch_mv_dma_ma_k<T_Q4K, 4, MA>(w, y, n, m, xt, xd, bsp, epi, s);
        case 5: return launch_mv_dma_ma_k<T_Q4K, 5, MA>(w, y, n, m, xt, xd, bsp, epi, s);
        case 6: return launch_mv_dma_ma_k<T_Q4K, 6, MA>(w, y, n, m, xt, xd, bsp, epi, s);
        case 7: return launch_mv_dma_ma_k<T_Q4K, 7, MA>(w, y, n, m, xt, xd, bsp, epi, s);
        default: return launch_mv_dma_ma_k<T_Q4K, 8, MA>(w, y, n, m, xt, xd, bsp, epi, s);
    }
}

// Shapes k_mv_dma_ma takes: Q4_K with k <= 2048 in whole superblocks, to
// 128 rows; Q6_K at k = 2048 (its rows are whole 16-byte DMA pieces at 8
// superblocks), to 16 rows.  Longer k stays on the split-K MFMA kernel: a
// single-tile workgroup streaming a whole long row block measured slower
// (Q6_K [2048, 8192] at m = 16: 16.7 against 13.4 us).
bool mv_dma_ma_fits(int type, int64_t k, int64_t m) {
    if (k % 256 || !mv_dma_on() || m > MV_DMA_MA_MAX_ROWS) return false;
    if (type == T_Q4K) return k <= MV_DMA_KMAX;
    if (type == T_Q6K) return k == MV_DMA_KMAX && m <= 16;
    return false;
}

hipError_t launch_mv_dma_ma(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                            void* ws, int epi, hipStream_t s) {
    int8_t* xt;
    float* xd;
    int8_t* bsp;
    split_q8k_ptrs(ws, k, m, &xt, &xd, &bsp);
    hipError_t e = launch_quantize_split_q8k(x, m, k, xt, xd, s, type == T_Q4K ? bsp : nullptr, true);
    if (e != hipSuccess) return e;
    if (m <= 16) return launch_mv_dma_ma_m<1>(type, w, y, n, k, m, xt, xd, bsp, epi, s);
    if (m <= 32) return launch_mv_dma_ma_m<2>(type, w, y, n, k, m, xt, xd, bsp, epi, s);
    if (m <= 48) return launch_mv_dma_ma_m<3>(type, w, y, n, k, m, xt, xd, bsp, epi, s);
    if (m <= 64) return launch_mv_dma_ma_m<4>(type, w, y, n, k, m, xt, xd, bsp, epi, s);
    if (m <= 96) return launch_mv_dma_ma_m<6>(type, w, y, n, k, m, xt, xd, bsp, epi, s);
    return launch_mv_dma_ma_m<8>(type, w, y, n, k, m, xt, xd, bsp, epi, s);
}

template <int TYPE, int MA>
static hipError_t launch_mv_mfma(const void* w, float* y, int64_t n, int64_t k, int64_t m, const int8_t* xq,
                                 const float* xd, int epi, hipStream_t s, float* psum = nullptr) {
    // 8 waves split K; 2 row tiles per workgroup unless that leaves fewer
    // than ~256 workgroups
    constexpr int KS = 8;
    const unsigned layers = (unsigned)((m + 16 * MA - 1) / (16 * MA));
    const int mp = (int)((m + 15) & ~(int64_t)15);
    const int nsb = (int)(k / 256);
    if constexpr (MA == 1) {
        if (n >= 2 * 16 * 256) {
            hipLaunchKernelGGL((k_mv_mfma<TYPE, KS, 2, MA>), dim3((unsigned)((n + 31) / 32), layers), dim3(64 * KS), 0,
                               s, (const uint8_t*)w, xq, xd, y, (int)n, (int)k, (int)m, mp, epi, nsb, nullptr);
            return hipGetLastError();
        }
        if (n < 16 * 256 && k >= 16 * 256) {
            // fewer row tiles than CUs and a long K: 16 waves split K, and
            // with a partial-sum buffer the workgroups split it too
            const int sp = psum ? mv_splits(n, k) : 1;
            const int sbs = (nsb + sp - 1) / sp;
            hipLaunchKernelGGL((k_mv_mfma<TYPE, 16, 1, MA>), dim3((unsigned)((n + 15) / 16), layers, sp),
                               dim3(64 * 16), 0, s, (const uint8_t*)w, xq, xd, y, (int)n, (int)k, (int)m, mp, epi, sbs,
                               sp > 1 ? psum : nullptr);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess || sp == 1) return e;
            const int64_t mn = m * n;
            hipLaunchKernelGGL(k_sum_splits, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, psum, sp, mn, y,
                               epi);
            return hipGetLastError();
        }
    }
    {
        hipLaunchKernelGGL((k_mv_mfma<TYPE, KS, 1, MA>), dim3((unsigned)((n + 15) / 16), layers), dim3(64 * KS), 0, s,
                           (const uint8_t*)w, xq, xd, y, (int)n, (int)k, (int)m, mp, epi, nsb, nullptr);
    }
    return hipGetLastError();
}

hipError_t launch_mq(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* ws,
                     int epi, hipStream_t s) {
    int8_t* xq;
    float* xd;
    split_q8k_ptrs(ws, k, m, &xq, &xd);
    hipError_t e = launch_quantize_split_q8k(x, m, k, xq, xd, s);
    if (e != hipSuccess) return e;
    return type == T_Q4K ? launch_mv_mfma<T_Q4K, 4>(w, y, n, k, m, xq, xd, epi, s)
                         : launch_mv_mfma<T_Q6K, 4>(w, y, n, k, m, xq, xd, epi, s);
}

// Rows of Q4_K / Q6_K on the dot4 kernel: one or two, and Q4_K with 3-4
// rows on a small weight (n k <= 2048^2: [2048, 2048] at m = 4 5.04 us
// against 6.23 for the fused MFMA kernel; on [6144, 2048] 7.63 against
// 6.49, and Q6_K [2048, 8192] 15.8 against 12.0).
static bool mv_dot(int type, int64_t n, int64_t k, int64_t m) {
    return m <= MV_DOT_MAX_ROWS || (type == T_Q4K && m <= 4 && n * k <= 2048 * 2048);
}

hipError_t launch_matvec(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                         void* ws, int epi, hipStream_t s) {
    // large Q4_K weights: the persistent streaming kernel
    if (mv_stream_fits(type, n, k, m)) return launch_mv_stream(type, w, x, y, n, k, m, ws, epi, s);
    if (type != T_Q8_0 && !mv_dot(type, n, k, m) && m <= FUSED_MAX_ROWS && (k == 2048 || k == 1024))
        return type == T_Q4K ? launch_fused<T_Q4K>(w, x, y, n, k, m, epi, s)
                             : launch_fused<T_Q6K>(w, x, y, n, k, m, epi, s);
    // Past the dot4 and fused kernels, up to 2048 elements of k: the split
    // quantizer in its tiled layout, then k_mv_dma_ma with one activation
    // tile (C2, B = 8 / 16: 7.28 / 7.37 us against 7.41 / 7.62 for the
    // earlier kernel with x staged in LDS; Q6_K [8192, 2048] 11.35 / 11.34
    // against 11.87 / 12.19)
    if (type != T_Q8_0 && !mv_dot(type, n, k, m) && mv_dma_ma_fits(type, k, m))
        return launch_mv_dma_ma(type, w, x, y, n, k, m, ws, epi, s);
    if (type != T_Q8_0 && !mv_dot(type, n, k, m)) {
        int8_t* xq;
        float* xd;
        split_q8k_ptrs(ws, k, m, &xq, &xd);
        hipError_t e = launch_quantize_split_q8k(x, m, k, xq, xd, s);
        if (e != hipSuccess) return e;
        float* ps = mv_psum(ws, k, m);
        return type == T_Q4K ? launch_mv_mfma<T_Q4K, 1>(w, y, n, k, m, xq, xd, epi, s, ps)
                             : launch_mv_mfma<T_Q6K, 1>(w, y, n, k, m, xq, xd, epi, s, ps);
    }
    switch (type) {
        case T_Q4K: return launch_type<T_Q4K>(w, x, y, (int)n, (int)k, (int)m, epi, s);
        case T_Q6K: return launch_type<T_Q6K>(w, x, y, (int)n, (int)k, (int)m, epi, s);
        case T_Q8_0: return launch_type<T_Q8_0>(w, x, y, (int)n, (int)k, (int)m, epi, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace lloom
