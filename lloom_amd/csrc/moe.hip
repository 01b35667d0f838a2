// moe.hip -- routed-expert matmul, QTensor::indexed_moe_forward.
//
// The CPU arm (matmul_t_indexed, lloom-tensor/src/quantized/mod.rs:766-810)
// dequantizes each routed weight row to f32 and takes an f32 dot with the
// unquantized activation; this arm keeps that arithmetic contract (f32
// activations, exactly dequantized weights, f32 accumulation) but
// reorganizes the work for HBM:
//  1. k_moe_route groups the (b, t) planes by expert on the device (a
//     counting sort; ids never leave the GPU) and flags ids >= n_experts;
//  2. k_moe_lds runs one workgroup per (active expert, block of rows): the
//     activation planes routed to the expert are staged in LDS (up to eight
//     at a time), each lane dequantizes its piece of R weight rows once and
//     dots it with every staged plane, so each weight byte is read from HBM
//     once per call and each activation element from L2 once per workgroup.
//     k_moe_rows (activations read from L2 per row) is kept for rows too long
//     to stage.
#include <cstdlib>
#include <type_traits>

#include "kq_common.hpp"
#include "kq_mfma.hpp"
#include "kq_tasks.hpp"
#include "kernels.hpp"
#include "kq_gemm.hpp"

namespace lloom {

#pragma clang fp contract(off)

// Workspace (ints): [0] error flag, [1] active experts,
// [2 .. 2+E) count, [2+E .. 2+2E) start, [2+2E .. 2+3E) active list,
// [2+3E .. 2+3E+P) planes sorted by expert, [.. +E) fill cursor.
size_t moe_workspace_ints(int64_t n_experts, int64_t planes) { return 2 + 4 * (size_t)n_experts + (size_t)planes; }

// One workgroup: count planes per expert, scan, scatter -- in LDS, one
// global write per output.  The order of the planes inside an expert's list
// follows the LDS atomics, but every plane's dot is computed on its own, so
// no result depends on it.
__global__ __launch_bounds__(1024) void k_moe_route(const uint32_t* __restrict__ ids, int planes, int E, int* ws,
                                                    int* sticky, float* __restrict__ y, float* __restrict__ y2, int n) {
    extern __shared__ int s_mem[];  // [E] counts, then [E] cursors
    __shared__ int s_part[1024];
    __shared__ int s_bad, s_active;
    int* s_count = s_mem;
    int* s_cur = s_mem + E;
    int* count = ws + 2;
    int* start = count + E;
    int* active = start + E;
    int* sorted = active + E;
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int e = tid; e < E; e += nt) s_count[e] = 0;
    if (tid == 0) {
        s_bad = 0;
        s_active = 0;
    }
    __syncthreads();
    for (int p = tid; p < planes; p += nt) {
        const uint32_t e = ids[p];
        if (e < (uint32_t)E) {
            atomicAdd(&s_count[e], 1);
        } else {
            s_bad = 1;
            for (int r = 0; r < n; r++) y[(int64_t)p * n + r] = 0.0f;
            if (y2)
                for (int r = 0; r < n; r++) y2[(int64_t)p * n + r] = 0.0f;
        }
    }
    __syncthreads();
    // exclusive scan: thread t owns experts [t*per, (t+1)*per)
    const int per = (E + nt - 1) / nt;
    const int e0 = min(tid * per, E), e1 = min(e0 + per, E);
    int local = 0, nact = 0;
    for (int e = e0; e < e1; e++) {
        local += s_count[e];
        nact += s_count[e] > 0;
    }
    // scan of (local, nact) packed: nact < 2^15, local < 2^16 per thread is
    // not guaranteed, so two passes
    int incl = local;
    for (int o = 1; o < nt; o <<= 1) {
        s_part[tid] = incl;
        __syncthreads();
        if (tid >= o) incl += s_part[tid - o];
        __syncthreads();
    }
    int run = incl - local;
    int ainc = nact;
    for (int o = 1; o < nt; o <<= 1) {
        s_part[tid] = ainc;
        __syncthreads();
        if (tid >= o) ainc += s_part[tid - o];
        __syncthreads();
    }
    int arun = ainc - nact;
    for (int e = e0; e < e1; e++) {
        const int c = s_count[e];
        count[e] = c;
        start[e] = run;
        s_cur[e] = run;
        if (c) active[arun++] = e;
        run += c;
    }
    if (tid == nt - 1) s_active = ainc;
    __syncthreads();
    for (int p = tid; p < planes; p += nt) {
        const uint32_t e = ids[p];
        if (e < (uint32_t)E) sorted[atomicAdd(&s_cur[e], 1)] = p;
    }
    if (tid == 0) {
        ws[0] = s_bad;             // this call: read back by a strict call
        if (s_bad) sticky[0] = 1;  // until the next lloom_hip_ctx_sync
        ws[1] = s_active;
    }
}

template <int TYPE>
struct MoeTraits;
template <>
struct MoeTraits<T_Q4K> {
    static constexpr int BE = 256, BB = Q4K_BYTES, P = 8, RUNS = 2;
};
template <>
struct MoeTraits<T_Q6K> {
    static constexpr int BE = 256, BB = Q6K_BYTES, P = 4, RUNS = 4;
};
template <>
struct MoeTraits<T_Q8_0> {
    static constexpr int BE = 32, BB = Q8_0_BYTES, P = 1, RUNS = 2;
};

// Dequantize one task (RUNS runs of 16 consecutive elements) of a weight
// row exactly as to_float does; *off[r] is the element offset of run r
// inside the row.
template <int TYPE>
__device__ __forceinline__ void dequant_task(const uint8_t* __restrict__ row, int blk, int p,
                                             float (*w)[16], int* off) {
    if constexpr (TYPE == T_Q4K) {
        const uint8_t* b = row + (size_t)blk * Q4K_BYTES;
        uint4 s = *(const uint4*)b;
        uint4 a = *(const uint4*)(b + 16 + 16 * p);
        const float d = f16_to_f32(s.x & 0xffffu), dmin = f16_to_f32(s.x >> 16);
        const int j = p >> 1, half = p & 1;
        int sc0, m0, sc1, m1;
        if (j < 2) {
            sc0 = byte_of(s.y, 2 * j) & 63;
            m0 = byte_of(s.z, 2 * j) & 63;
            sc1 = byte_of(s.y, 2 * j + 1) & 63;
            m1 = byte_of(s.z, 2 * j + 1) & 63;
        } else {
            uint32_t i0 = 2 * j - 4, i1 = 2 * j - 3;
            sc0 = (byte_of(s.w, i0) & 0xF) | ((byte_of(s.y, i0) >> 6) << 4);
            m0 = (byte_of(s.w, i0) >> 4) | ((byte_of(s.z, i0) >> 6) << 4);
            sc1 = (byte_of(s.w, i1) & 0xF) | ((byte_of(s.y, i1) >> 6) << 4);
            m1 = (byte_of(s.w, i1) >> 4) | ((byte_of(s.z, i1) >> 6) << 4);
        }
        const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
        const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
        const uint32_t A[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            uint32_t q = byte_of(A[i >> 2], i & 3);
            w[0][i] = d1 * (float)(q & 0xF) - mm1;
            w[1][i] = d2 * (float)(q >> 4) - mm2;
        }
        off[0] = blk * 256 + 64 * j + 16 * half;
        off[1] = off[0] + 32;
    } else if constexpr (TYPE == T_Q6K) {
        const uint8_t* b = row + (size_t)blk * Q6K_BYTES;
        const int h = p >> 1, odd = p & 1;
        uint4 a = load16_a2(b + 64 * h + 16 * odd);
        uint4 bb = load16_a2(b + 64 * h + 32 + 16 * odd);
        uint4 c = load16_a2(b + Q6K_QH + 32 * h + 16 * odd);
        const int8_t* sc = (const int8_t*)(b + Q6K_SC);
        const float d = f16_to_f32(*(const uint16_t*)(b + Q6K_D));
        const uint32_t A[4] = {a.x, a.y, a.z, a.w}, B[4] = {bb.x, bb.y, bb.z, bb.w}, C[4] = {c.x, c.y, c.z, c.w};
        float ds[4];
#pragma unroll
        for (int g = 0; g < 4; g++) ds[g] = d * (float)sc[8 * h + 2 * g + odd];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            uint32_t lo = byte_of(A[i >> 2], i & 3), lo2 = byte_of(B[i >> 2], i & 3), hb = byte_of(C[i >> 2], i & 3);
            int q1 = (int)((lo & 0xF) | ((hb & 3) << 4)) - 32;
            int q2 = (int)((lo2 & 0xF) | (((hb >> 2) & 3) << 4)) - 32;
            int q3 = (int)((lo >> 4) | (((hb >> 4) & 3) << 4)) - 32;
            int q4 = (int)((lo2 >> 4) | (((hb >> 6) & 3) << 4)) - 32;
            w[0][i] = ds[0] * (float)q1;
            w[1][i] = ds[1] * (float)q2;
            w[2][i] = ds[2] * (float)q3;
            w[3][i] = ds[3] * (float)q4;
        }
#pragma unroll
        for (int g = 0; g < 4; g++) off[g] = blk * 256 + 128 * h + 32 * g + 16 * odd;
    } else {
        const uint8_t* b = row + (size_t)blk * Q8_0_BYTES;
        const float d = f16_to_f32(*(const uint16_t*)b);
        uint4 q0 = load16_a2(b + 2), q1 = load16_a2(b + 18);
        const uint32_t Q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int i = 0; i < 32; i++) w[i >> 4][i & 15] = (float)(int8_t)byte_of(Q[i >> 2], i & 3) * d;
        off[0] = blk * 32;
        off[1] = off[0] + 16;
    }
}

// One workgroup: (row block, active-expert slot).  LPR lanes share a row
// (LPR = tasks per row rounded up to a power of two, at most 64), so short
// rows (k = 768) still keep most lanes busy.
template <int TYPE, int LPR, int PG>
__global__ __launch_bounds__(256) void k_moe_rows(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                  float* __restrict__ Y, const int* __restrict__ ws, int E, int n,
                                                  int K, int in_dim1, int topk, const uint8_t* __restrict__ W2,
                                                  float* __restrict__ Y2) {
    // the second weight of a pair (gate, up) is grid layer z = 1
    if (blockIdx.z) {
        W = W2;
        Y = Y2;
    }
    using Tr = MoeTraits<TYPE>;
    constexpr int RPW = 64 / LPR;  // rows per wave
    const int* count = ws + 2;
    const int* start = count + E;
    const int* active = start + E;
    const int* sorted = active + E;
    const int slot = blockIdx.y;
    if (slot >= ws[1]) return;
    const int e = active[slot];
    const int np = count[e], p0 = start[e];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / LPR, tl = lane % LPR;
    const int row = (blockIdx.x * 4 + wave) * RPW + sub;
    const bool row_ok = row < n;
    const int64_t rowbytes = (int64_t)(K / Tr::BE) * Tr::BB;
    const uint8_t* wrow = W + ((int64_t)e * n + (row_ok ? row : 0)) * rowbytes;
    const int T = (K / Tr::BE) * Tr::P;

    for (int g0 = 0; g0 < np; g0 += PG) {
        float acc[PG];
        int xoff[PG];
#pragma unroll
        for (int q = 0; q < PG; q++) {
            acc[q] = 0.0f;
            int pl = g0 + q < np ? sorted[p0 + g0 + q] : -1;
            int b = pl >= 0 ? pl / topk : 0, t = pl >= 0 ? pl - b * topk : 0;
            xoff[q] = pl >= 0 ? (b * in_dim1 + (in_dim1 == 1 ? 0 : t)) * K : -1;
        }
        for (int ti = tl; ti < T; ti += LPR) {
            if (!row_ok) break;
            float w[Tr::RUNS][16];
            int off[Tr::RUNS];
            dequant_task<TYPE>(wrow, ti / Tr::P, ti % Tr::P, w, off);
#pragma unroll
            for (int q = 0; q < PG; q++) {
                if (xoff[q] < 0) continue;
                const float* xr = X + xoff[q];
                float s = acc[q];
#pragma unroll
                for (int r = 0; r < Tr::RUNS; r++) {
                    const float4* xv = (const float4*)(xr + off[r]);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        float4 v = xv[i];
                        s += w[r][4 * i] * v.x;
                        s += w[r][4 * i + 1] * v.y;
                        s += w[r][4 * i + 2] * v.z;
                        s += w[r][4 * i + 3] * v.w;
                    }
                }
                acc[q] = s;
            }
        }
#pragma unroll
        for (int q = 0; q < PG; q++) {
            float v = acc[q];
#pragma unroll
            for (int o = LPR / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            if (tl == 0 && row_ok && xoff[q] >= 0) Y[(int64_t)sorted[p0 + g0 + q] * n + row] = v;
        }
    }
}

// ---------------------------------------------------- LDS-staged planes --
// A task's weights as runs of 16 consecutive elements sharing one affine
// dequantization value = a * q - b (k_quants.rs to_float):
//   Q4_K  q = nibble,    a = d * sc,  b = dmin * m   (two runs)
//   Q6_K  q = q6,        a = d * sc,  b = 32 * a     (four runs)
//   Q8_0  q = int8,      a = d,       b = 0          (two runs)
// The dot with f32 activations is taken as a * sum(q * x) - b * sum(x): the
// q are small integers (exact in f32), and sum(x) over each 16-element run
// is computed once per staged plane.
template <int TYPE>
struct MoeRuns;
template <>
struct MoeRuns<T_Q4K> {
    static constexpr int N = 2;
};
template <>
struct MoeRuns<T_Q6K> {
    static constexpr int N = 4;
};
template <>
struct MoeRuns<T_Q8_0> {
    static constexpr int N = 2;
};

template <int TYPE>
__device__ __forceinline__ void task_runs(const WPrep<TYPE>& w, float (&q)[MoeRuns<TYPE>::N][16],
                                          float (&a)[MoeRuns<TYPE>::N], float (&b)[MoeRuns<TYPE>::N],
                                          float fp8_inv) {
    // Q4_K: a nibble byte q (0..15) read as an FP8 E4M3 value is exactly
    // q * u (the exponent field is 0 or 1, so the value is linear in q), and
    // v_cvt_pk_f32_fp8 converts two bytes an instruction; the unit u (a power
    // of two, measured once by the kernel as fp8_inv = 1 / u) moves into the
    // scale: (a / u) * sum((q u) x) is a * sum(q x) bit for bit.
    // Q6_K: the empty asm hides the words' known-zero bits (with them visible
    // the compiler converts each byte with a bit-field extract and
    // v_cvt_f32_ubyte0 instead of one v_cvt_f32_ubyteN).
    if constexpr (TYPE == T_Q4K) {
        a[0] = w.d * (float)w.sc0 * fp8_inv;
        b[0] = w.dmin * (float)w.m0;
        a[1] = w.d * (float)w.sc1 * fp8_inv;
        b[1] = w.dmin * (float)w.m1;
        typedef float f2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const f2 l0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w.lo[i], false);
            const f2 l1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w.lo[i], true);
            const f2 h0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w.hi[i], false);
            const f2 h1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w.hi[i], true);
            q[0][4 * i] = l0.x;
            q[0][4 * i + 1] = l0.y;
            q[0][4 * i + 2] = l1.x;
            q[0][4 * i + 3] = l1.y;
            q[1][4 * i] = h0.x;
            q[1][4 * i + 1] = h0.y;
            q[1][4 * i + 2] = h1.x;
            q[1][4 * i + 3] = h1.y;
        }
    } else if constexpr (TYPE == T_Q6K) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            a[g] = w.d * (float)w.sc[g];
            b[g] = 32.0f * a[g];
            uint32_t qw[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                qw[i] = w.q[g][i];
                asm("" : "+v"(qw[i]));
            }
#pragma unroll
            for (int i = 0; i < 16; i++) q[g][i] = (float)byte_of(qw[i >> 2], i & 3);
        }
    } else {
        a[0] = a[1] = w.d;
        b[0] = b[1] = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) q[i >> 4][i & 15] = (float)(int8_t)byte_of(w.w[i >> 2], i & 3);
    }
}

// Element offset (within the row) of run r of task ti.
template <int TYPE>
__device__ __forceinline__ int run_offset(int ti, int r) {
    using Tr = MvTraits<TYPE>;
    const int blk = ti / Tr::P, p = ti % Tr::P;
    if constexpr (TYPE == T_Q4K) return blk * 256 + 64 * (p >> 1) + 16 * (p & 1) + 32 * r;
    else if constexpr (TYPE == T_Q6K) return blk * 256 + 128 * (p >> 1) + 32 * r + 16 * (p & 1);
    else return blk * 32 + 16 * r;
}

// Sum over the LPR lanes of a group (LPR a power of two, at most 16).
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (LPR >= 2) v += dpp<DPP_XOR1>(v);
    if constexpr (LPR >= 4) v += dpp<DPP_XOR2>(v);
    if constexpr (LPR >= 8) v += dpp<DPP_HALF_MIRROR>(v);
    if constexpr (LPR >= 16) v += dpp<DPP_ROW_MIRROR>(v);
    return v;
}

constexpr int MOE_PG = 8;          // planes staged per pass
constexpr int MOE_FUSE_MAX = 1024;  // planes routed inside k_moe_lds (an LDS list per workgroup)
constexpr int MOE_LDS = 72 * 1024;  // bytes of staged planes and run sums
// Floats of a staged plane: element e at e + 4 (e / 64) + 16 (e / 256), then
// the K / 16 run sums come after all the planes.
__host__ __device__ constexpr int moe_plane_floats(int K) { return K + K / 8; }
__host__ __device__ inline int moe_plane_idx(int e) { return e + 4 * (e >> 6) + 16 * (e >> 8); }

// One workgroup (4 waves) per (block of rows, active-expert slot).  In a
// wave, 64 / LPR groups of LPR lanes each own R consecutive rows and walk
// the row's tasks LPR apart (TPL of them loaded at once); a lane's R rows
// share its activation reads.
// A gate/up pair (indexed_moe_forward_pair, mod.rs:1365-1455) is one launch
// of two grid layers, z = 1 reading W2 into Y2.  GLU (indexed_moe_forward
// _glu_as, mod.rs:1457-1531): a lane holds R rows of the gate W and the same
// R rows of the up weight W2, and stores silu(gate) * up, the SwiGLU's
// element (silu_mul order) over the two sums the pair would store.
template <int TYPE, int LPR, int R, int TPL, bool GLU>
__global__ __launch_bounds__(256) void k_moe_lds(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                 float* __restrict__ Y, int* ws, int E, int n, int K, int in_dim1,
                                                 int topk, int pgmax, const uint8_t* __restrict__ W2,
                                                 float* __restrict__ Y2, const uint32_t* __restrict__ ids,
                                                 int planes, int* sticky, int route) {
    using Tr = MvTraits<TYPE>;
    constexpr int NR = MoeRuns<TYPE>::N;
    constexpr int RR = GLU ? 2 * R : R;  // weight rows a lane holds
    constexpr int ROWS = 4 * (64 / LPR) * R;  // rows of a workgroup
    if (!GLU && blockIdx.z) {
        W = W2;
        Y = Y2;
    }
    // Routing.  With `route` 0 the workgroup of expert blockIdx.y collects
    // the planes routed to it from ids itself, and the grid layer y = E
    // zeroes the outputs of out-of-range ids and raises the flags (what
    // k_moe_route does, without its launch); otherwise k_moe_route has
    // sorted the planes and y is the active-expert slot.
    __shared__ int s_list[MOE_FUSE_MAX];
    __shared__ int s_np;
    int e, np;
    const int* list;
    if (!route) {
        if ((int)blockIdx.y == E) {
            const int r0 = blockIdx.x * ROWS, r1 = min(r0 + ROWS, n);
            int bad = 0;
            for (int p = threadIdx.x; p < planes; p += 256) {
                if (ids[p] >= (uint32_t)E) {
                    bad = 1;
                    for (int r = r0; r < r1; r++) Y[(int64_t)p * n + r] = 0.0f;
                }
            }
            bad = __syncthreads_or(bad);
            if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.z == 0) {
                ws[0] = bad;  // this call: read back by a strict call
                if (bad) sticky[0] = 1;
            }
            return;
        }
        e = blockIdx.y;
        if (threadIdx.x == 0) s_np = 0;
        __syncthreads();
        // the list's order follows the LDS atomics; every plane's dot is
        // computed on its own, so no result depends on it
        for (int p = threadIdx.x; p < planes; p += 256)
            if (ids[p] == (uint32_t)e) s_list[atomicAdd(&s_np, 1)] = p;
        __syncthreads();
        np = s_np;
        if (np == 0) return;  // uniform
        list = s_list;
    } else {
        const int* count = ws + 2;
        const int* start = count + E;
        const int* active = start + E;
        const int* sorted = active + E;
        if ((int)blockIdx.y >= ws[1]) return;  // uniform: fewer active experts than slots
        e = active[blockIdx.y];
        np = count[e];
        list = sorted + start[e];
    }
    // [pgmax][KP] planes, then [pgmax][K / 16] run sums.  A plane stores
    // element e at e + 4 (e / 64) + 16 (e / 256): the eight tasks of a
    // superblock (16 lanes: two superblocks) read 16-byte pieces that this
    // spreads over distinct banks, the second superblock's 32 banks from the
    // first's.
    extern __shared__ __align__(16) float xs[];
    const int KP = moe_plane_floats(K);
    float* sx = xs + pgmax * KP;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane / LPR, tl = lane % LPR;
    const int row0 = ((blockIdx.x * 4 + wave) * (64 / LPR) + grp) * R;
    const int64_t rowbytes = (int64_t)(K / Tr::BE) * Tr::BB;
    const uint8_t* wrow[RR];
#pragma unroll
    for (int r = 0; r < RR; r++)
        wrow[r] = (r < R ? W : W2) + ((int64_t)e * n + min(row0 + r % R, n - 1)) * rowbytes;
    const int T = (K / Tr::BE) * Tr::P;
    const float fp8_inv = 1.0f / __builtin_amdgcn_cvt_f32_fp8(1, 0);  // 1 / (FP8 byte 1), a power of two
    const int k16 = K >> 4;

    for (int g0 = 0; g0 < np; g0 += pgmax) {
        const int pg = min(pgmax, np - g0);
        float acc[RR][MOE_PG];
#pragma unroll
        for (int r = 0; r < RR; r++)
#pragma unroll
            for (int q = 0; q < MOE_PG; q++) acc[r][q] = 0.0f;
        // Tasks in chunks of TPL per lane.  Software-pipelined: the next
        // chunk's loads are issued before this chunk's dots (the last
        // chunk's "next" reloads chunk 0, from L2, so that no load sits
        // under a branch and the waits stay counted).
        auto load_chunk = [&](int c0, TaskData (&td)[TPL][RR]) {
#pragma unroll
            for (int c = 0; c < TPL; c++) {
                const int ti = c0 + c * LPR + tl;
                const int tc = ti < T ? ti : tl;
#pragma unroll
                for (int r = 0; r < RR; r++) load_task<TYPE>(wrow[r], tc / Tr::P, tc % Tr::P, td[c][r]);
            }
        };
        TaskData tda[TPL][RR];
        load_chunk(0, tda);
        // stage planes g0 .. g0 + pg of this expert (the first chunk's
        // weights are in flight meanwhile) and the sum of each 16-element run
        if (g0) __syncthreads();  // the previous group's readers are done
        for (int i = threadIdx.x; i < pg * k16; i += 256) {
            const int q = i / k16, c = i - q * k16;
            const int pl = list[g0 + q];
            const int b = pl / topk, t = pl - b * topk;
            const float4* xr = (const float4*)(X + (int64_t)(b * in_dim1 + (in_dim1 == 1 ? 0 : t)) * K + 16 * c);
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = xr[u];
            float4* dst = (float4*)(xs + q * KP + moe_plane_idx(16 * c));
            float sum = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                dst[u] = v[u];
                sum += v[u].x + v[u].y + v[u].z + v[u].w;
            }
            sx[q * k16 + c] = sum;
        }
        __syncthreads();
        for (int c0 = 0; c0 < T; c0 += TPL * LPR) {
            TaskData tdb[TPL][RR];
            load_chunk(c0 + TPL * LPR, tdb);
#pragma unroll
            for (int c = 0; c < TPL; c++) {
                const int ti = c0 + c * LPR + tl;
                if (ti < T) {
                    float qv[RR][NR][16], ra[RR][NR], rb[RR][NR];
#pragma unroll
                    for (int r = 0; r < RR; r++) {
                        WPrep<TYPE> wp;
                        prep_task<TYPE>(tda[c][r], ti % Tr::P, wp);
                        task_runs<TYPE>(wp, qv[r], ra[r], rb[r], fp8_inv);
                    }
                    int off[NR];
#pragma unroll
                    for (int u = 0; u < NR; u++) off[u] = run_offset<TYPE>(ti, u);
#pragma unroll
                    for (int q = 0; q < MOE_PG; q++) {
                        if (q < pg) {  // uniform
                            const float* xq = xs + q * KP;
#pragma unroll
                            for (int u = 0; u < NR; u++) {
                                float dq[RR];
#pragma unroll
                                for (int r = 0; r < RR; r++) dq[r] = 0.0f;
#pragma unroll
                                for (int i4 = 0; i4 < 4; i4++) {
                                    const float4 xv = *(const float4*)(xq + moe_plane_idx(off[u]) + 4 * i4);
#pragma unroll
                                    for (int r = 0; r < RR; r++) {
                                        dq[r] = __builtin_fmaf(qv[r][u][4 * i4], xv.x, dq[r]);
                                        dq[r] = __builtin_fmaf(qv[r][u][4 * i4 + 1], xv.y, dq[r]);
                                        dq[r] = __builtin_fmaf(qv[r][u][4 * i4 + 2], xv.z, dq[r]);
                                        dq[r] = __builtin_fmaf(qv[r][u][4 * i4 + 3], xv.w, dq[r]);
                                    }
                                }
                                const float s16 = sx[q * k16 + (off[u] >> 4)];
#pragma unroll
                                for (int r = 0; r < RR; r++)
                                    acc[r][q] =
                                        __builtin_fmaf(ra[r][u], dq[r], __builtin_fmaf(-rb[r][u], s16, acc[r][q]));
                            }
                        }
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < TPL; c++)
#pragma unroll
                for (int r = 0; r < RR; r++) tda[c][r] = tdb[c][r];
        }
        // sum over the LPR lanes of the group; lane tl == 0 stores
#pragma unroll
        for (int q = 0; q < MOE_PG; q++) {
            if (q < pg) {
                const int pl = list[g0 + q];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    float v = group_sum<LPR>(acc[r][q]);
                    if constexpr (GLU) {
                        const float u = group_sum<LPR>(acc[R + r][q]);
                        v = v / (1.0f + expf(-v)) * u;
                    }
                    if (tl == 0 && row0 + r < n) Y[(int64_t)pl * n + row0 + r] = v;
                }
            }
        }
    }
}

// ------------------------------------------- Q4_K experts on fp16 MFMA --
// The same contract (f32 activations, exactly dequantized weights, f32
// accumulation) on v_mfma_f32_16x16x32_f16.  A workgroup (4 waves) owns
// 64 NT weight rows of one expert; each wave NT 16-row tiles over all of K.
// Operands of the MFMA for sub-block j of superblock sb (g = lane / 16):
//   A (planes):  lane l holds x'[plane l%16][256 sb + 32 j + 8 g + 0..7]
//   B (weights): lane l holds sc_j * q[row l%16][the same 8 elements]
//   D:           lane l holds D[plane 4 g + v][row l%16], v = 0..3
// * The planes are staged in LDS once per workgroup, each scaled by a power
//   of two (x' = x * 2^s, max |x'| in [2^13, 2^14): exact) and split into
//   fp16 hi + lo (x' = hi + lo to about 2^-22 relative); the two halves take
//   one MFMA each into the same f32 accumulator.  sc_j * q <= 945 is an exact
//   fp16 integer, so every product is exact and only the f32 sums round, as
//   in the VALU kernel.  MFMA rows past the staged planes repeat the last one
//   and are not stored.
// * Per superblock: acc = sum_j sc_j * S_j (16 MFMAs); the min term
//   sum_j m_j * X_j (X_j: sub-block sums of x', / 32 so they stay in fp16
//   range, hi and lo side by side in K) is one more MFMA against the mins;
//   out += d * acc - 32 dmin * accm.  The output is out * 2^-s.
typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef _Float16 mh2 __attribute__((ext_vector_type(2)));
typedef float mf4 __attribute__((ext_vector_type(4)));

// Four nibbles (one per byte, 0..15) times sc as fp16, in element order:
// v_perm_b32 puts each nibble under the exponent byte 0x64 (fp16 1024 + q),
// one packed fma gives (1024 + q) * sc - 1024 * sc = q * sc, exact.
__device__ __forceinline__ uint2 moe_nib4(uint32_t w, mh2 sc, mh2 off) {
    const uint32_t e = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);  // [q0, q1]
    const uint32_t o = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);  // [q2, q3]
    const mh2 ve = __builtin_elementwise_fma(__builtin_bit_cast(mh2, e), sc, off);
    const mh2 vo = __builtin_elementwise_fma(__builtin_bit_cast(mh2, o), sc, off);
    return make_uint2(__builtin_bit_cast(uint32_t, ve), __builtin_bit_cast(uint32_t, vo));
}

// Byte i of each of four bytes (each 0..63) as fp16, packed two a dword.
__device__ __forceinline__ uint2 moe_b4_h(uint32_t w) {
    const mh2 k = {(_Float16)(-1024.0f), (_Float16)(-1024.0f)};
    const mh2 e = __builtin_bit_cast(mh2, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)) + k;
    const mh2 o = __builtin_bit_cast(mh2, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)) + k;
    return make_uint2(__builtin_bit_cast(uint32_t, e), __builtin_bit_cast(uint32_t, o));
}

// bytes of staged planes a pass: 16 planes of k = 2048 (512 tokens top-8 on
// [128, 768, 2048]: 236 us against 273 with 11 planes a pass)
constexpr int MOEM_LDS = 140 * 1024;
constexpr int MOE_MFMA_DENSITY = 8;  // planes per active expert (at least) for the MFMA kernel
constexpr int MOEM_FUSE_MAX = 1024;  // planes routed inside the kernel (an LDS list per workgroup)
#ifndef MOEM_WAVES_EU
#define MOEM_WAVES_EU 2
#endif

// LDS bytes of a pass of pg planes: hi and lo [K/8][pg][8] fp16, the sums
// [K/256][pg][16] fp16; then scales and the waves' transpose tiles.
__host__ __device__ inline int moem_plane_bytes(int K) { return 4 * K + 32 * (K / 256); }
__host__ __device__ inline int moem_fixed_bytes(int waves) { return 256 + waves * 16 * MfRs<T_Q4K>::V; }

// One workgroup (4 waves) per (64 GW RG weight rows, expert).  A wave owns
// GW row groups of 16 RG rows (RG = 2 row tiles, or for GLU one tile of the
// gate and the same tile of the up weight) and streams its items (row
// group, superblock) over all of K with DEPTH items of weight loads in
// flight; the planes are staged in LDS once per workgroup and pass.
// Routing: with `route` 0 the workgroup of expert blockIdx.y collects the
// planes routed to it from ids itself (planes <= MOEM_FUSE_MAX), and the
// extra grid layer y = E zeroes the outputs of out-of-range ids and raises
// the flags; otherwise k_moe_route has sorted the planes and y is the
// active-expert slot.
template <int DEPTH, bool GLU>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MOEM_WAVES_EU))) void k_moe_mfma(
    const uint8_t* __restrict__ W, const float* __restrict__ X, float* __restrict__ Y,
    const uint32_t* __restrict__ ids, int planes, int* ws, int* sticky, int E, int n, int K, int in_dim1, int topk,
    int pgmax, const uint8_t* __restrict__ W2, float* __restrict__ Y2, int route, int gw) {
    constexpr int RT = 2;                 // weight tiles an item holds
    constexpr int RG = GLU ? 16 : 32;     // rows of a row group
    if (!GLU && blockIdx.z) {
        W = W2;
        Y = Y2;
    }
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_list[MOEM_FUSE_MAX];
    __shared__ int s_np;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int wrow0 = (blockIdx.x * 4 + wave) * gw * RG;  // this wave's first row
    const int brow0 = blockIdx.x * 4 * gw * RG, brow1 = min(brow0 + 4 * gw * RG, n);

    int e, np;
    const int* list;
    if (!route) {
        if ((int)blockIdx.y == E) {
            // out-of-range ids: their planes are zero in every output
            int bad = 0;
            for (int p = tid; p < planes; p += 256) {
                if (ids[p] >= (uint32_t)E) {
                    bad = 1;
                    for (int r = brow0; r < brow1; r++) Y[(int64_t)p * n + r] = 0.0f;
                }
            }
            bad = __syncthreads_or(bad);
            if (tid == 0 && blockIdx.x == 0 && blockIdx.z == 0) {
                ws[0] = bad;  // this call: read back by a strict call
                if (bad) sticky[0] = 1;
            }
            return;
        }
        e = blockIdx.y;
        if (tid == 0) s_np = 0;
        __syncthreads();
        // the list's order follows the LDS atomics; every plane's dot is
        // computed on its own, so no result depends on it
        for (int p = tid; p < planes; p += 256)
            if (ids[p] == (uint32_t)e) s_list[atomicAdd(&s_np, 1)] = p;
        __syncthreads();
        np = s_np;
        if (np == 0) return;  // uniform
        list = s_list;
    } else {
        const int* count = ws + 2;
        const int* start = count + E;
        const int* active = start + E;
        const int* sorted = active + E;
        if ((int)blockIdx.y >= ws[1]) return;  // uniform
        e = active[blockIdx.y];
        np = count[e];
        list = sorted + start[e];
    }

    const int nsb = K >> 8, k8 = K >> 3;
    const int nitems = gw * nsb;
    const int64_t rowbytes = (int64_t)nsb * Q4K_BYTES;
    const uint8_t* wbase = W + (int64_t)e * n * rowbytes;
    const uint8_t* wbase2 = (GLU ? W2 : W) + (int64_t)e * n * rowbytes;
    // item i: row group i / nsb, superblock i % nsb (indices past the end
    // reload the last item: no load sits under a branch)
    auto load_item = [&](int i, MfL<T_Q4K>(&b)[RT]) {
        i = min(i, nitems - 1);
        const int rg = i / nsb, sb = i - rg * nsb;
#pragma unroll
        for (int t = 0; t < RT; t++) {
            const int row = min(wrow0 + rg * RG + (GLU ? 0 : 16 * t) + c16, n - 1);
            mf_load_l<T_Q4K>((GLU && t ? wbase2 : wbase) + row * rowbytes + (int64_t)sb * Q4K_BYTES, g, b[t]);
        }
    };

    _Float16* xh = (_Float16*)smem;
    uint32_t* pmax = (uint32_t*)(smem + (size_t)pgmax * moem_plane_bytes(K));
    float* pscale = (float*)(pmax + 16);
    float* pinv = pscale + 16;
    uint8_t* tile = smem + (size_t)pgmax * moem_plane_bytes(K) + 256 + wave * 16 * MfRs<T_Q4K>::V;

    auto xoff = [&](int q) {
        const int pl = list[q];
        const int b = pl / topk, t = pl - b * topk;
        return (int64_t)(b * in_dim1 + (in_dim1 == 1 ? 0 : t)) * K;
    };

    for (int g0 = 0; g0 < np; g0 += pgmax) {
        const int pg = min(pgmax, np - g0);
        _Float16* xl = xh + (size_t)pg * K;
        _Float16* xs = xl + (size_t)pg * K;
        // the first items' weights are in flight during the staging
        MfL<T_Q4K> buf[DEPTH][RT];
#pragma unroll
        for (int d = 0; d < DEPTH; d++) load_item(d, buf[d]);

        if (g0) __syncthreads();  // the previous pass's readers are done
        if (tid < 16) pmax[tid] = 0u;
        __syncthreads();
        // 1. max |x| of each plane (non-negative floats order as their bits)
        for (int i = tid; i < pg * k8; i += 256) {
            const int q = i / k8, G = i - q * k8;
            const float4* xr = (const float4*)(X + xoff(g0 + q) + 8 * G);
            const float4 a = xr[0], b = xr[1];
            const float mx = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                                   fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
            atomicMax(&pmax[q], __float_as_uint(mx));
        }
        __syncthreads();
        if (tid < pg) {
            const float mx = __uint_as_float(pmax[tid]);
            const bool fin = mx > 0.0f && mx <= 3.4028234e38f;
            int ex = 0;
            if (fin) (void)frexpf(mx, &ex);
            const int sh = fin ? 14 - ex : 0;  // max |x'| in [2^13, 2^14)
            pscale[tid] = ldexpf(1.0f, sh);
            pinv[tid] = ldexpf(1.0f, -sh);
        }
        __syncthreads();
        // 2. x' = x * 2^s as hi + lo, and the sub-block sums of x' / 32
        //    (a quad of lanes holds the four 8-element groups of a sub-block)
        for (int i = tid; i < pg * k8; i += 256) {
            const int q = i / k8, G = i - q * k8;
            const float4* xr = (const float4*)(X + xoff(g0 + q) + 8 * G);
            const float4 a = xr[0], b = xr[1];
            const float sc = pscale[q];
            const float v[8] = {a.x * sc, a.y * sc, a.z * sc, a.w * sc, b.x * sc, b.y * sc, b.z * sc, b.w * sc};
            mh8 hv, lv;
            float sum = 0.0f;
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const _Float16 hu = (_Float16)v[u];
                hv[u] = hu;
                lv[u] = (_Float16)(v[u] - (float)hu);
                sum += v[u];
            }
            *(mh8*)(xh + ((size_t)G * pg + q) * 8) = hv;
            *(mh8*)(xl + ((size_t)G * pg + q) * 8) = lv;
            sum += __shfl_xor(sum, 1, 64);
            sum += __shfl_xor(sum, 2, 64);
            if ((G & 3) == 0) {
                const float s32 = sum * 0.03125f;
                const _Float16 sh = (_Float16)s32;
                _Float16* d = xs + ((size_t)(G >> 5) * pg + q) * 16 + ((G >> 2) & 7);
                d[0] = sh;
                d[8] = (_Float16)(s32 - (float)sh);
            }
        }
        __syncthreads();

        const int pc = min(c16, pg - 1);  // this lane's A row
        mf4 out[RT];
#pragma unroll
        for (int t = 0; t < RT; t++) out[t] = mf4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int it = 0; it < nitems; it++) {
            MfL<T_Q4K> nxt[RT];
            load_item(it + DEPTH, nxt);
            const int rg = it / nsb, sb = it - rg * nsb;
            {
            // min-term operand: K 0..7 the sums' hi, 8..15 their lo (lanes
            // g >= 2 repeat them against zero weights)
            const mh8 am = *(const mh8*)(xs + ((size_t)sb * pg + pc) * 16 + 8 * (g & 1));
            // the tiles' weights and scales, then the sub-blocks (one pair of
            // activation operands serves both tiles)
            MfW<T_Q4K> wu[RT];
            mh2 scp[RT][4];
            mf4 acc[RT];
#pragma unroll
            for (int t = 0; t < RT; t++) {
                mf_unpack<T_Q4K>(buf[0][t], tile, g, c16, wu[t]);
                const uint4 hd = wu[t].hdr;
                const uint32_t scl = hd.y & 0x3F3F3F3Fu, sch = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
                const uint2 sl = moe_b4_h(scl), shh = moe_b4_h(sch);
                scp[t][0] = __builtin_bit_cast(mh2, sl.x);
                scp[t][1] = __builtin_bit_cast(mh2, sl.y);
                scp[t][2] = __builtin_bit_cast(mh2, shh.x);
                scp[t][3] = __builtin_bit_cast(mh2, shh.y);
                acc[t] = mf4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int G = 32 * sb + 4 * j + g;
                const mh8 ah = *(const mh8*)(xh + ((size_t)G * pg + pc) * 8);
                const mh8 al = *(const mh8*)(xl + ((size_t)G * pg + pc) * 8);
                const int c = j >> 1, sh = 4 * (j & 1);
#pragma unroll
                for (int t = 0; t < RT; t++) {
                    const uint32_t lo = (wu[t].q[c].x >> sh) & 0x0F0F0F0Fu, hi = (wu[t].q[c].y >> sh) & 0x0F0F0F0Fu;
                    const _Float16 s1 = scp[t][j >> 1][j & 1];
                    const mh2 sv = {s1, s1};
                    const mh2 of = sv * (_Float16)(-1024.0f);
                    const uint2 p0 = moe_nib4(lo, sv, of), p1 = moe_nib4(hi, sv, of);
                    const mh8 bw = __builtin_bit_cast(mh8, make_uint4(p0.x, p0.y, p1.x, p1.y));
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bw, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bw, acc[t], 0, 0, 0);
                }
            }
#pragma unroll
            for (int t = 0; t < RT; t++) {
                const uint4 hd = wu[t].hdr;
                const float d = f16_to_f32(hd.x & 0xffffu), dmin = f16_to_f32(hd.x >> 16);
                const uint32_t mnl = hd.z & 0x3F3F3F3Fu,
                               mnh = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
                const uint2 ml = moe_b4_h(mnl), mh = moe_b4_h(mnh);
                const mh8 bm = g < 2 ? __builtin_bit_cast(mh8, make_uint4(ml.x, ml.y, mh.x, mh.y)) : mh8{};
                const mf4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                const mf4 accm = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bm, z, 0, 0, 0);
                const float dm32 = 32.0f * dmin;
#pragma unroll
                for (int v = 0; v < 4; v++)
                    out[t][v] = __builtin_fmaf(d, acc[t][v], __builtin_fmaf(-dm32, accm[v], out[t][v]));
            }
            // the row group is complete after its last superblock: store it
            if (sb == nsb - 1) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int q = 4 * g + v;
                    if (q < pg) {
                        const int pl = list[g0 + q];
                        const float inv = pinv[q];
                        const int row = wrow0 + rg * RG + c16;
                        if constexpr (GLU) {
                            const float y = out[0][v] * inv, u = out[1][v] * inv;
                            if (row < n) Y[(int64_t)pl * n + row] = y / (1.0f + expf(-y)) * u;
                        } else {
                            if (row < n) Y[(int64_t)pl * n + row] = out[0][v] * inv;
                            if (row + 16 < n) Y[(int64_t)pl * n + row + 16] = out[1][v] * inv;
                        }
                    }
                }
#pragma unroll
                for (int t = 0; t < RT; t++) out[t] = mf4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            }
#pragma unroll
            for (int d = 0; d + 1 < DEPTH; d++)
#pragma unroll
                for (int t = 0; t < RT; t++) buf[d][t] = buf[d + 1][t];
#pragma unroll
            for (int t = 0; t < RT; t++) buf[DEPTH - 1][t] = nxt[t];
        }
    }
}

// --------------------- Q4_K experts, decode-like routing, K split by wave --
// A few planes an expert (decode: C5 routes 2.25 planes to each of 114
// experts) on the fp16 MFMA arithmetic of k_moe_mfma, shaped like the dense
// decode kernels instead: one workgroup per (expert, run of `tpw` pairs of
// 16-row weight tiles; GLU: 16 rows of the gate and the same 16 of the up
// weight), K/256 waves, wave w owning superblock w of every row.
//  * the workgroup routes its expert's planes once, then streams its tile
//    pairs through an LDS ring of S stages by 1 KB global_load_lds DMAs of
//    whole rows, S - 1 pairs ahead of the pair it computes (every wave
//    issues the same number of DMAs a stage, so a counted vmcnt wait and a
//    barrier say a stage has landed);
//  * each wave loads only its superblock of each routed plane (lane l: plane
//    l % 8, the 8 elements 8 (l / 16) .. of each sub-block), scales it by
//    its own power of two (max |x'| in [2^13, 2^14) over the superblock:
//    exact) and splits it into fp16 hi + lo, with the 32-element sums / 32
//    for the min term.  The hi parts of 8 planes fill MFMA rows 0-7 and
//    their lo parts rows 8-15, so one 16x16x32 MFMA a sub-block gives both
//    (decode routes fewer than 8 planes to most experts); with at most 16
//    planes (two passes) these operands stay in registers for the whole run;
//  * per tile: sum_j sc_j S_j as 8 MFMAs (sc_j q exact fp16 integers), hi
//    and lo rows added, and the min term as one more MFMA, then
//    (d acc - 32 dmin accm) 2^-s; the K/256 partial sums meet in LDS and are
//    added in superblock order.
// More than 8 planes an expert take further passes over each staged pair
// (past 16, each reloading its operands).  Served for rows of 2048 elements
// (8 waves); see moe_dma_fits.

// LDS pitch of a row of `bytes` (a multiple of 16): its dword count 4 mod 8,
// so a 16-row b128 read takes two passes over the 32 banks, not sixteen.
constexpr int lds_pitch16(int bytes) {
    int p = (bytes + 15) & ~15;
    while ((p / 4) % 8 != 4) p += 16;
    return p;
}

template <int N>
__device__ __forceinline__ void vm_wait_moe() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int NSB>
struct MoedCfg {
    static constexpr int RB = NSB * Q4K_BYTES;
    static constexpr int WP = lds_pitch16(RB);
    static constexpr int NI = (16 * WP + 1023) / 1024;  // 1 KB DMA instructions a tile
    static constexpr int TILE = NI * 1024, STAGE = 2 * TILE;
    static constexpr int DPW = (2 * NI + NSB - 1) / NSB;  // DMAs a wave issues a stage
    static constexpr int PART = NSB * 2 * 64 * 16;
    static constexpr int FIXED = PART + MOEM_FUSE_MAX * 4 + 16;
    static constexpr int S = (160 * 1024 - FIXED) / STAGE >= 4 ? 4 : 3;
    static constexpr int LDS = S * STAGE + FIXED;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert((S - 2) * DPW <= 63, "vmcnt counts to 63");
};

template <int NSB, bool GLU>
__global__ __launch_bounds__(64 * NSB) void k_moe_dma(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                      float* __restrict__ Y, const uint32_t* __restrict__ ids,
                                                      int planes, int* ws, int* sticky, int E, int n, int in_dim1,
                                                      int topk, const uint8_t* __restrict__ W2,
                                                      float* __restrict__ Y2, int tpw) {
    using C = MoedCfg<NSB>;
    constexpr int K = NSB * 256, RB = C::RB, WP = C::WP, NI = C::NI, S = C::S, DPW = C::DPW;
    constexpr int ROWS = GLU ? 16 : 32;  // weight rows of a tile pair (of each weight, GLU)
    extern __shared__ __align__(16) uint8_t smem[];
    float4* part = (float4*)(smem + S * C::STAGE);  // [NSB][2][64]
    int* s_list = (int*)(smem + S * C::STAGE + C::PART);
    int* s_np = s_list + MOEM_FUSE_MAX;
    if (!GLU && blockIdx.z) {
        W = W2;
        Y = Y2;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int ntp = (n + ROWS - 1) / ROWS;
    const int tp0 = blockIdx.x * tpw, T = min(tpw, ntp - tp0);
    if (T <= 0) return;  // uniform
    if ((int)blockIdx.y == E) {
        // out-of-range ids: their planes are zero in every output
        const int r0 = tp0 * ROWS, r1 = min(r0 + T * ROWS, n);
        int bad = 0;
        for (int p = tid; p < planes; p += 64 * NSB) {
            if (ids[p] >= (uint32_t)E) {
                bad = 1;
                for (int r = r0; r < r1; r++) Y[(int64_t)p * n + r] = 0.0f;
            }
        }
        bad = __syncthreads_or(bad);
        if (tid == 0 && blockIdx.x == 0 && blockIdx.z == 0) {
            ws[0] = bad;  // this call: read back by a strict call
            if (bad) sticky[0] = 1;
        }
        return;
    }
    const int e = blockIdx.y;
    if (tid == 0) *s_np = 0;
    __syncthreads();
    // the list's order follows the LDS atomics; every plane's dot is
    // computed on its own, so no result depends on it
    for (int p = tid; p < planes; p += 64 * NSB)
        if (ids[p] == (uint32_t)e) s_list[atomicAdd(s_np, 1)] = p;
    __syncthreads();
    const int np = *s_np;
    if (np == 0) return;  // uniform

    // this wave's DMA instructions of a stage: chunk q = wave + NSB i of the
    // stage's 2 NI (tile q / NI, instruction q % NI; waves past the end
    // repeat the last); a lane's 16 bytes are row r, byte cc of the tile
    // (pad lanes reload the row's last piece, rows past n repeat row n - 1)
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    int rr[DPW], tsel[DPW];
    uint32_t cc[DPW], ldo[DPW];
#pragma unroll
    for (int i = 0; i < DPW; i++) {
        const int q = min(wv + NSB * i, 2 * NI - 1);
        const int t = q / NI, ii = q - t * NI;
        const int L = ii * 1024 + 16 * lane;
        rr[i] = min(L / WP, 15);
        cc[i] = (uint32_t)min(L - (L / WP) * WP, RB - 16);
        tsel[i] = t;
        ldo[i] = (uint32_t)(t * C::TILE + ii * 1024);
    }
    const uint32_t lds0 = lds_addr(smem);
    const int64_t ebase = (int64_t)e * n * RB;
    auto issue = [&](int it, int slot) {
        const int tp = tp0 + min(it, T - 1);
#pragma unroll
        for (int i = 0; i < DPW; i++) {
            const uint8_t* base = (GLU && tsel[i] ? W2 : W) + ebase;
            const int trow0 = GLU ? tp * 16 : tp * 32 + 16 * tsel[i];
            const uint32_t off = (uint32_t)min(trow0 + rr[i], n - 1) * (uint32_t)RB + cc[i];
            dma16s(base, off, lds0 + (uint32_t)(slot * C::STAGE) + ldo[i]);
        }
    };
#pragma unroll
    for (int i = 0; i < S - 1; i++) issue(i, i);

    const int sb = wave;
    // the operands of up to two passes (16 planes) stay in registers for the
    // run; past 16 planes every pass reloads its own into slot 0
    mh8 ax[2][8], am[2];
    float inv[2][4];
    // With at most 16 planes a pair's outputs are stored at the start of the
    // next iteration, before its DMAs: stores count in vmcnt, and a store
    // issued after a stage's DMAs would make the counted wait for the stage
    // before it wait for that stage too.  (A wave adds at most one item: NSB
    // >= 2.)
    static_assert(NSB >= 2, "one reduction item a wave");
    float pend[2][4];
    int prow[2] = {-1, -1};
    auto flush = [&]() {
#pragma unroll
        for (int ps = 0; ps < 2; ps++) {
            if (prow[ps] >= 0 && prow[ps] < n) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int q = 8 * ps + 4 * g + v;
                    if (g < 2 && q < np) Y[(int64_t)s_list[q] * n + prow[ps]] = pend[ps][v];
                }
            }
            prow[ps] = -1;
        }
    };
    for (int it = 0; it < T; it++) {
        const int slot = it % S, tp = tp0 + it;
        // pair it has landed (this wave's share, S - 2 later stages in
        // flight; then everyone's), and every wave is done with slot it - 1
        vm_wait_moe<(S - 2) * DPW>();
        __syncthreads();
        flush();
        issue(it + S - 1, (it + S - 1) % S);
        const uint8_t* st = smem + slot * C::STAGE;
        // one pass of (up to) 8 planes from g0; PS: its operand slot
        auto pass = [&](auto PSC, int g0, bool prep) {
            constexpr int PS = decltype(PSC)::value;
            const int pg = min(8, np - g0);
            if (prep) {  // uniform
                // this lane's plane (c16 % 8: MFMA rows 0-7 take the planes'
                // fp16 hi parts, rows 8-15 the lo parts) and its 64 elements
                // of superblock sb; lanes past the pass's planes hold zeros
                // (their MFMA rows are not stored)
                const int pq = c16 & 7;
                const int pl = s_list[g0 + min(pq, pg - 1)];
                const int b = pl / topk, tk = pl - b * topk;
                const float* xr = X + (int64_t)(b * in_dim1 + (in_dim1 == 1 ? 0 : tk)) * K + 256 * sb + 8 * g;
                float4 xa[8][2];
                const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                for (int j = 0; j < 8; j++) xa[j][0] = xa[j][1] = z4;
                if (pq < pg) {
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        xa[j][0] = *(const float4*)(xr + 32 * j);
                        xa[j][1] = *(const float4*)(xr + 32 * j + 4);
                    }
                }
                float mx = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(xa[j][h].x), fabsf(xa[j][h].y)),
                                             fmaxf(fabsf(xa[j][h].z), fabsf(xa[j][h].w))));
                mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const bool fin = mx > 0.0f && mx <= 3.4028234e38f;
                int ex = 0;
                if (fin) (void)frexpf(mx, &ex);
                const int sh = fin ? 14 - ex : 0;  // max |x'| in [2^13, 2^14)
                const float scl = ldexpf(1.0f, sh);
                // inverse scales of the planes of this lane's outputs (4g ..)
                const float invs = ldexpf(1.0f, -sh);
#pragma unroll
                for (int v = 0; v < 4; v++) inv[PS][v] = __shfl(invs, (4 * g + v) & 7, 64);
                float ssum[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float vv[8] = {xa[j][0].x * scl, xa[j][0].y * scl, xa[j][0].z * scl, xa[j][0].w * scl,
                                         xa[j][1].x * scl, xa[j][1].y * scl, xa[j][1].z * scl, xa[j][1].w * scl};
                    float s = 0.0f;
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const _Float16 hu = (_Float16)vv[u];
                        ax[PS][j][u] = c16 < 8 ? hu : (_Float16)(vv[u] - (float)hu);
                        s += vv[u];
                    }
                    ssum[j] = s;
                }
                // sub-block sums / 32 as the min-term operand: K 0..7 hi (g
                // even), 8..15 lo (g odd); lanes g >= 2 meet zero weights
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    float s = ssum[j] + __shfl_xor(ssum[j], 16, 64);
                    s += __shfl_xor(s, 32, 64);
                    const float s32 = s * 0.03125f;
                    const _Float16 hs = (_Float16)s32;
                    am[PS][j] = (g & 1) ? (_Float16)(s32 - (float)hs) : hs;
                }
            }
#pragma unroll
            for (int t = 0; t < 2; t++) {
                MfW<T_Q4K> wu;
                mf_load<T_Q4K>(st + t * C::TILE + c16 * WP + sb * Q4K_BYTES, g, wu);
                const uint4 hd = wu.hdr;
                const uint32_t scw = hd.y & 0x3F3F3F3Fu, sch = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
                const uint2 sl = moe_b4_h(scw), shh = moe_b4_h(sch);
                const mh2 scp[4] = {__builtin_bit_cast(mh2, sl.x), __builtin_bit_cast(mh2, sl.y),
                                    __builtin_bit_cast(mh2, shh.x), __builtin_bit_cast(mh2, shh.y)};
                // D[r][row]: rows r < 8 the planes' hi products, r >= 8 their
                // lo products; two chains (even and odd sub-blocks)
                mf4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int c = j >> 1, s4 = 4 * (j & 1);
                    const uint32_t lo = (wu.q[c].x >> s4) & 0x0F0F0F0Fu, hi = (wu.q[c].y >> s4) & 0x0F0F0F0Fu;
                    const _Float16 s1 = scp[j >> 1][j & 1];
                    const mh2 sv = {s1, s1};
                    const mh2 of = sv * (_Float16)(-1024.0f);
                    const uint2 p0 = moe_nib4(lo, sv, of), p1 = moe_nib4(hi, sv, of);
                    const mh8 bw = __builtin_bit_cast(mh8, make_uint4(p0.x, p0.y, p1.x, p1.y));
                    if (j & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[PS][j], bw, acc1, 0, 0, 0);
                    else acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[PS][j], bw, acc0, 0, 0, 0);
                }
                // lane (g, c16), g < 2: plane 4g + v's hi sum here, its lo sum
                // in lane (g + 2, c16)
                const mf4 acc2 = acc0 + acc1;
                mf4 acc;
#pragma unroll
                for (int v = 0; v < 4; v++) acc[v] = acc2[v] + __shfl_xor(acc2[v], 32, 64);
                const float d = f16_to_f32(hd.x & 0xffffu), dmin = f16_to_f32(hd.x >> 16);
                const uint32_t mnl = hd.z & 0x3F3F3F3Fu,
                               mnh = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
                const uint2 ml = moe_b4_h(mnl), mh = moe_b4_h(mnh);
                const mh8 bm = g < 2 ? __builtin_bit_cast(mh8, make_uint4(ml.x, ml.y, mh.x, mh.y)) : mh8{};
                const mf4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                const mf4 accm = __builtin_amdgcn_mfma_f32_16x16x32_f16(am[PS], bm, z, 0, 0, 0);
                const float dm32 = 32.0f * dmin;
                float o[4];
#pragma unroll
                for (int v = 0; v < 4; v++) o[v] = __builtin_fmaf(d, acc[v], -dm32 * accm[v]) * inv[PS][v];
                part[(sb * 2 + t) * 64 + lane] = make_float4(o[0], o[1], o[2], o[3]);
            }
            __syncthreads();
            // add the NSB partials in superblock order; lane (g, c16) holds
            // planes 4g .. 4g+3 of row c16 of the tile
            constexpr int ITEMS = GLU ? 1 : 2;
            for (int item = wave; item < ITEMS; item += NSB) {  // uniform
                float4 sum[2];
#pragma unroll
                for (int u = 0; u < (GLU ? 2 : 1); u++) {
                    const int t = GLU ? u : item;
                    float4 a = part[t * 64 + lane];
#pragma unroll
                    for (int w = 1; w < NSB; w++) {
                        const float4 p = part[(w * 2 + t) * 64 + lane];
                        a.x += p.x;
                        a.y += p.y;
                        a.z += p.z;
                        a.w += p.w;
                    }
                    sum[u] = a;
                }
                const int row = tp * ROWS + (GLU ? 0 : 16 * item) + c16;
                const float s0[4] = {sum[0].x, sum[0].y, sum[0].z, sum[0].w};
                const float s1[4] = {sum[1].x, sum[1].y, sum[1].z, sum[1].w};
                float val[4];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    if constexpr (GLU) {
                        const float y = s0[v], u = s1[v];
                        val[v] = y / (1.0f + expf(-y)) * u;
                    } else {
                        val[v] = s0[v];
                    }
                }
                if (np <= 16) {  // uniform: stored at the next iteration
#pragma unroll
                    for (int v = 0; v < 4; v++) pend[PS][v] = val[v];
                    prow[PS] = row;
                } else {
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int q = 4 * g + v;
                        if (g < 2 && q < pg && row < n) Y[(int64_t)s_list[g0 + q] * n + row] = val[v];
                    }
                }
            }
            __syncthreads();  // part is rewritten by the next pass or pair
        };
        if (np <= 16) {  // uniform
            pass(std::integral_constant<int, 0>{}, 0, it == 0);
            if (np > 8) pass(std::integral_constant<int, 1>{}, 8, it == 0);
        } else {
            for (int g0 = 0; g0 < np; g0 += 8) pass(std::integral_constant<int, 0>{}, g0, true);
        }
    }
    flush();
    // no DMA (the repeated tail stages) may still be writing this
    // workgroup's LDS when it exits
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int NSB>
static hipError_t moe_dma_nsb(const void* w, const float* x, float* y, const uint32_t* ids, int planes, int* ws,
                              int* sticky, int E, int n, int in_dim1, int topk, const void* w2, float* y2, int mode,
                              hipStream_t s) {
    using C = MoedCfg<NSB>;
    const bool glu = mode == MOE_GLU;
    const int rows = glu ? 16 : 32;
    const int ntp = (n + rows - 1) / rows;
    // pairs a workgroup: one round of workgroups over the CUs (as many a CU
    // as the LDS holds) for every expert's runs (the routing density this
    // kernel takes leaves few experts without planes)
    const int64_t per_cu = (160 * 1024) / C::LDS, slots = (int64_t)cu_count() * (per_cu > 0 ? per_cu : 1);
    const int64_t layers = (int64_t)E * (mode == MOE_PAIR ? 2 : 1);
    int tpw = (int)(((int64_t)ntp * layers + slots - 1) / slots);
    tpw = tpw < 1 ? 1 : tpw > ntp ? ntp : tpw;
    dim3 grid((ntp + tpw - 1) / tpw, E + 1, mode == MOE_PAIR ? 2 : 1);
    const void* kern = glu ? (const void*)k_moe_dma<NSB, true> : (const void*)k_moe_dma<NSB, false>;
    if (hipError_t e = set_lds_limit(kern, C::LDS)) return e;
    if (glu)
        hipLaunchKernelGGL((k_moe_dma<NSB, true>), grid, dim3(64 * NSB), C::LDS, s, (const uint8_t*)w, x, y, ids,
                           planes, ws, sticky, E, n, in_dim1, topk, (const uint8_t*)w2, y2, tpw);
    else
        hipLaunchKernelGGL((k_moe_dma<NSB, false>), grid, dim3(64 * NSB), C::LDS, s, (const uint8_t*)w, x, y, ids,
                           planes, ws, sticky, E, n, in_dim1, topk, (const uint8_t*)w2, y2, tpw);
    return hipGetLastError();
}

// LLOOM_HIP_MOE_DMA (read once): 0 keeps decode-like Q4_K routing on
// k_moe_lds; unset or 1 takes k_moe_dma where it fits.
static bool moe_dma_on() {
    static const bool v = [] {
        const char* e = getenv("LLOOM_HIP_MOE_DMA");
        return !e || atoi(e) != 0;
    }();
    return v;
}

// Rows of 2048 elements (8 superblocks, 8 waves) at 1.75 to 2.5 planes an
// expert on average (7 E <= 4 planes < 10 E): where it measured faster.
// C5's gate weight ([128, 768, 2048] Q4_K), T tokens top-8 (random experts),
// graph replays on rotating copies, this kernel against k_moe_lds:
//   T = 1, 8, 16, 24:   17, 37, 34, 34 us against 9.2, 17.4, 26.5, 30.8
//                       (few planes leave most of this kernel's one-round
//                       grid idle, and k_moe_lds's cost grows with planes)
//   T = 28 .. 38:       33.4 - 36 us against 36.7 - 47
//   T = 40, 48, 64:     57, 58, 58 us against 50, 50, 61 (some expert gets
//                       more than 8 planes: two passes, and that expert's
//                       two workgroups set the time)
// At k = 768 (3 waves) it lost on C5's down projection (41.8 against 39.3).
static bool moe_dma_fits(int type, int64_t n, int64_t k, int64_t E, int planes) {
    const int64_t p4 = 4 * (int64_t)planes;
    return type == T_Q4K && k == 2048 && n >= 1 && planes <= MOEM_FUSE_MAX && p4 >= 7 * E && p4 < 10 * E &&
           moe_dma_on();
}

static hipError_t launch_moe_dma(const void* w, const float* x, float* y, const uint32_t* ids, int planes, int* ws,
                                 int* sticky, int E, int n, int k, int in_dim1, int topk, const void* w2, float* y2,
                                 int mode, hipStream_t s) {
    if (k != 2048) return hipErrorInvalidValue;
    return moe_dma_nsb<8>(w, x, y, ids, planes, ws, sticky, E, n, in_dim1, topk, w2, y2, mode, s);
}

template <int DEPTH, bool GLU>
static hipError_t moe_mfma_cfg(const void* w, const float* x, float* y, const uint32_t* ids, int planes, int* ws,
                               int* sticky, int E, int n, int K, int in_dim1, int topk, int max_slots, int pgmax,
                               const void* w2, float* y2, int mode, bool route, int gw, hipStream_t s) {
    const size_t shm = (size_t)pgmax * moem_plane_bytes(K) + moem_fixed_bytes(4);
    if (hipError_t e = set_lds_limit((const void*)k_moe_mfma<DEPTH, GLU>, MOEM_LDS + moem_fixed_bytes(4))) return e;
    const int rows_wg = 4 * gw * (GLU ? 16 : 32);
    dim3 grid((n + rows_wg - 1) / rows_wg, route ? max_slots : E + 1, mode == MOE_PAIR ? 2 : 1);
    hipLaunchKernelGGL((k_moe_mfma<DEPTH, GLU>), grid, dim3(256), shm, s, (const uint8_t*)w, x, y, ids, planes, ws,
                       sticky, E, n, K, in_dim1, topk, pgmax, (const uint8_t*)w2, y2, route ? 1 : 0, gw);
    return hipGetLastError();
}

static bool moe_mfma_fits(int64_t k) {
    return (k % 256) == 0 && moem_plane_bytes((int)k) + moem_fixed_bytes(4) <= MOEM_LDS + 4096;
}

// The weights of one call: w alone (MOE_ONE), w and w2 into y and y2
// (MOE_PAIR), or silu(w . x) * (w2 . x) into y (MOE_GLU).
struct MoeOut {
    int mode;
    const void* w2;
    float* y2;
    const uint32_t* ids;  // the routing inputs, for a call routed in-kernel
    int planes;
    int* sticky;
    bool route;  // k_moe_route sorted the planes
};

template <int TYPE, int LPR, int R, bool GLU>
static hipError_t moe_lds_cfg(const void* w, const float* x, float* y, int* ws, int E, int n, int K, int in_dim1,
                              int topk, int max_slots, int pgmax, const MoeOut& o, hipStream_t s) {
    // one task per lane and chunk, the next chunk's loads in flight during
    // this chunk's dots (measured on the C5 gate call: 38.8 us, against 40.1
    // for two tasks unpipelined and 46.5 for four)
    constexpr int TPL = 1;
    constexpr int ROWS = 4 * (64 / LPR) * R;
    const size_t shm = (size_t)pgmax * (moe_plane_floats(K) + K / 16) * sizeof(float);
    if (hipError_t e = set_lds_limit((const void*)k_moe_lds<TYPE, LPR, R, TPL, GLU>, MOE_LDS)) return e;
    dim3 grid((n + ROWS - 1) / ROWS, o.route ? max_slots : E + 1, o.mode == MOE_PAIR ? 2 : 1);
    hipLaunchKernelGGL((k_moe_lds<TYPE, LPR, R, TPL, GLU>), grid, dim3(256), shm, s, (const uint8_t*)w, x, y, ws, E,
                       n, K, in_dim1, topk, pgmax, (const uint8_t*)o.w2, o.y2, o.ids, o.planes, o.sticky,
                       o.route ? 1 : 0);
    return hipGetLastError();
}

// LPR: a row's tasks spread over LPR lanes, up to 4 per lane.
// GLU holds each row of both weights: half the rows per lane of the plain
// kernel, the same registers.
template <int TYPE, bool GLU>
static hipError_t moe_lds_type(const void* w, const float* x, float* y, int* ws, int E, int n, int K,
                               int in_dim1, int topk, int max_slots, int pgmax, const MoeOut& o, hipStream_t s) {
    using Tr = MvTraits<TYPE>;
    constexpr int R = (TYPE == T_Q6K || GLU) ? 1 : 2;
    const int T = (K / Tr::BE) * Tr::P;
    if (T > 32) return moe_lds_cfg<TYPE, 16, R, GLU>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, pgmax, o, s);
    if (T > 16) return moe_lds_cfg<TYPE, 8, R, GLU>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, pgmax, o, s);
    return moe_lds_cfg<TYPE, 4, R, GLU>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, pgmax, o, s);
}

template <int TYPE, int LPR>
static hipError_t moe_rows_lpr(const void* w, const float* x, float* y, const int* ws, int E, int n, int K,
                               int in_dim1, int topk, int max_slots, const void* w2, float* y2, hipStream_t s) {
    constexpr int RPW = 64 / LPR;
    dim3 grid((n + 4 * RPW - 1) / (4 * RPW), max_slots, w2 ? 2 : 1);
    hipLaunchKernelGGL((k_moe_rows<TYPE, LPR, 4>), grid, dim3(256), 0, s, (const uint8_t*)w, x, y, ws, E, n, K,
                       in_dim1, topk, (const uint8_t*)w2, y2);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t moe_rows_type(const void* w, const float* x, float* y, const int* ws, int E, int n, int K,
                                int in_dim1, int topk, int max_slots, const void* w2, float* y2, hipStream_t s) {
    using Tr = MoeTraits<TYPE>;
    int T = (K / Tr::BE) * Tr::P;
    if (T > 32) return moe_rows_lpr<TYPE, 64>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, w2, y2, s);
    if (T > 16) return moe_rows_lpr<TYPE, 32>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, w2, y2, s);
    if (T > 8) return moe_rows_lpr<TYPE, 16>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, w2, y2, s);
    return moe_rows_lpr<TYPE, 8>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, w2, y2, s);
}

// silu(g) * u elementwise, the fallback GLU for rows too long to stage
__global__ __launch_bounds__(256) void k_silu_mul(float* __restrict__ g, const float* __restrict__ u, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < count) {
        const float v = g[i];
        g[i] = v / (1.0f + expf(-v)) * u[i];
    }
}

size_t moe_workspace_bytes(int64_t n_experts, int64_t planes, int64_t n, int64_t k, int mode) {
    size_t b = (moe_workspace_ints(n_experts, planes) * sizeof(int) + 255) & ~(size_t)255;
    if (mode == MOE_GLU && !moe_stages(k)) b += (size_t)planes * n * sizeof(float);
    return b;
}

bool moe_stages(int64_t k) {
    const int64_t per_plane = (moe_plane_floats((int)k) + k / 16) * (int64_t)sizeof(float);
    return MOE_LDS / per_plane >= 1 && (k & 15) == 0;
}

hipError_t launch_moe(int type, const void* w, int64_t E, int64_t n, int64_t k, const float* x, int64_t batch,
                      int64_t in_dim1, const uint32_t* ids, int64_t topk, float* y, int* ws, int* sticky,
                      int mode, const void* w2, float* y2, hipStream_t s) {
    int planes = (int)(batch * topk);
    // the staged kernel routes up to MOE_FUSE_MAX planes itself (no routing
    // launch); otherwise k_moe_route sorts them first.  Planes of bad ids are
    // zeroed in every output either way.
    const bool route = !moe_stages(k) || planes > MOE_FUSE_MAX;
    hipError_t err = hipSuccess;
    if (route) {
        hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(1024), 2 * E * sizeof(int), s, ids, planes, (int)E, ws, sticky,
                           y, mode == MOE_PAIR ? y2 : nullptr, (int)n);
        if ((err = hipGetLastError()) != hipSuccess) return err;
    }
    int max_slots = (int)(E < planes ? E : planes);
    const int64_t per_plane = (moe_plane_floats((int)k) + k / 16) * (int64_t)sizeof(float);
    int pgmax = MOE_LDS / per_plane < MOE_PG ? (int)(MOE_LDS / per_plane) : MOE_PG;
    // a decode-like routing (at most four planes per active expert on
    // average) stages four planes at a time: half the LDS, so more
    // workgroups share a CU (C5: 40 us against 46 us per routed call)
    if (planes <= 4 * max_slots && pgmax > 4) pgmax = 4;
    // Dense routing (prefill: many planes per expert) takes the fp16-MFMA
    // kernel, 16 planes a pass; decode-like routing keeps the VALU kernel
    // (C5, two planes an expert: 44 against 52 us for the MFMA kernel)
    // Decode-like routing (fewer than MOE_MFMA_DENSITY planes an active
    // expert) of Q4_K rows of 2048 elements: k_moe_dma, routed in-kernel
    if (planes < MOE_MFMA_DENSITY * max_slots && moe_dma_fits(type, n, k, E, planes))
        return launch_moe_dma(w, x, y, ids, planes, ws, sticky, (int)E, (int)n, (int)k, (int)in_dim1, (int)topk, w2,
                              y2, mode, s);
    if (type == T_Q4K && moe_mfma_fits(k) && planes >= MOE_MFMA_DENSITY * max_slots) {
        int pgm = MOEM_LDS / moem_plane_bytes((int)k);
        pgm = pgm > 16 ? 16 : pgm < 1 ? 1 : pgm;
        const bool mroute = planes > MOEM_FUSE_MAX;
        // row groups a wave: 4 when the planes fit one pass (more rows share
        // a staging; 128 tokens: 73 against 81 us), else 2 (512 tokens: 236
        // against 256)
        const int gw = planes <= pgm * max_slots ? 4 : 2;
        if (mroute && !route) {
            hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(1024), 2 * E * sizeof(int), s, ids, planes, (int)E, ws,
                               sticky, y, mode == MOE_PAIR ? y2 : nullptr, (int)n);
            if ((err = hipGetLastError()) != hipSuccess) return err;
        }
        if (mode == MOE_GLU)
            return moe_mfma_cfg<2, true>(w, x, y, ids, planes, ws, sticky, (int)E, (int)n, (int)k, (int)in_dim1,
                                         (int)topk, max_slots, pgm, w2, y2, mode, mroute, gw, s);
        return moe_mfma_cfg<2, false>(w, x, y, ids, planes, ws, sticky, (int)E, (int)n, (int)k, (int)in_dim1,
                                      (int)topk, max_slots, pgm, w2, y2, mode, mroute, gw, s);
    }
    const MoeOut o{mode, w2, y2, ids, planes, sticky, route};
    const int Ei = (int)E, ni = (int)n, ki = (int)k, d1 = (int)in_dim1, tk = (int)topk;
    if (moe_stages(k)) {
        if (mode == MOE_GLU) {
            switch (type) {
                case T_Q4K: return moe_lds_type<T_Q4K, true>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pgmax, o, s);
                case T_Q6K: return moe_lds_type<T_Q6K, true>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pgmax, o, s);
                case T_Q8_0: return moe_lds_type<T_Q8_0, true>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pgmax, o, s);
            }
            return hipErrorInvalidValue;
        }
        switch (type) {
            case T_Q4K: return moe_lds_type<T_Q4K, false>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pgmax, o, s);
            case T_Q6K: return moe_lds_type<T_Q6K, false>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pgmax, o, s);
            case T_Q8_0: return moe_lds_type<T_Q8_0, false>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pgmax, o, s);
        }
        return hipErrorInvalidValue;
    }
    // rows too long to stage: a GLU is the pair (up into the workspace
    // after the routing ints) and one elementwise launch
    const void* pw2 = mode == MOE_ONE ? nullptr : w2;
    float* py2 = mode == MOE_PAIR ? y2 : mode == MOE_GLU
        ? (float*)((uint8_t*)ws + ((moe_workspace_ints(E, planes) * sizeof(int) + 255) & ~(size_t)255)) : nullptr;
    switch (type) {
        case T_Q4K: err = moe_rows_type<T_Q4K>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pw2, py2, s); break;
        case T_Q6K: err = moe_rows_type<T_Q6K>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pw2, py2, s); break;
        case T_Q8_0: err = moe_rows_type<T_Q8_0>(w, x, y, ws, Ei, ni, ki, d1, tk, max_slots, pw2, py2, s); break;
        default: return hipErrorInvalidValue;
    }
    if (err != hipSuccess || mode != MOE_GLU) return err;
    const int64_t count = (int64_t)planes * n;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, y, py2, count);
    return hipGetLastError();
}

}  // namespace lloom
