// moe.hip -- routed-expert matmul, QTensor::indexed_moe_forward.
//
// The CPU arm (matmul_t_indexed, lloom-tensor/src/quantized/mod.rs:766-810)
// dequantizes each routed weight row to f32 and takes an f32 dot with the
// unquantized activation; this arm keeps that arithmetic contract (f32
// activations, exactly dequantized weights, f32 accumulation) but
// reorganizes the work for HBM:
//  1. k_moe_route groups the (b, t) planes by expert on the device (a
//     counting sort; ids never leave the GPU) and flags ids >= n_experts;
//  2. k_moe_rows runs one workgroup per (active expert, row block): each
//     weight row of a touched expert is read from HBM once and dotted with
//     every plane routed to that expert (in groups of PG planes), instead of
//     once per plane.
#include "kq_common.hpp"
#include "kernels.hpp"

namespace lloom {

#pragma clang fp contract(off)

// Workspace (ints): [0] error flag, [1] active experts,
// [2 .. 2+E) count, [2+E .. 2+2E) start, [2+2E .. 2+3E) active list,
// [2+3E .. 2+3E+P) planes sorted by expert, [.. +E) fill cursor.
size_t moe_workspace_ints(int64_t n_experts, int64_t planes) { return 2 + 4 * (size_t)n_experts + (size_t)planes; }

__global__ __launch_bounds__(1024) void k_moe_route(const uint32_t* __restrict__ ids, int planes, int E, int* ws,
                                                    int* sticky, float* __restrict__ y, int n) {
    int* count = ws + 2;
    if (threadIdx.x == 0) ws[0] = 0;
    int* start = count + E;
    int* active = start + E;
    int* sorted = active + E;
    int* cursor = sorted + planes;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        count[e] = 0;
        cursor[e] = 0;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < planes; p += blockDim.x) {
        uint32_t e = ids[p];
        if (e < (uint32_t)E) {
            atomicAdd(&count[e], 1);
        } else {
            ws[0] = 1;      // this call: read back by a strict call
            sticky[0] = 1;  // until the next lloom_hip_ctx_sync
            for (int r = 0; r < n; r++) y[(int64_t)p * n + r] = 0.0f;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int s = 0, a = 0;
        for (int e = 0; e < E; e++) {
            start[e] = s;
            s += count[e];
            if (count[e]) active[a++] = e;
        }
        ws[1] = a;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < planes; p += blockDim.x) {
        uint32_t e = ids[p];
        if (e < (uint32_t)E) sorted[start[e] + atomicAdd(&cursor[e], 1)] = p;
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
                                                  int K, int in_dim1, int topk) {
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

template <int TYPE, int LPR>
static hipError_t moe_rows_lpr(const void* w, const float* x, float* y, const int* ws, int E, int n, int K,
                               int in_dim1, int topk, int max_slots, hipStream_t s) {
    constexpr int RPW = 64 / LPR;
    dim3 grid((n + 4 * RPW - 1) / (4 * RPW), max_slots);
    hipLaunchKernelGGL((k_moe_rows<TYPE, LPR, 4>), grid, dim3(256), 0, s, (const uint8_t*)w, x, y, ws, E, n, K,
                       in_dim1, topk);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t moe_rows_type(const void* w, const float* x, float* y, const int* ws, int E, int n, int K,
                                int in_dim1, int topk, int max_slots, hipStream_t s) {
    using Tr = MoeTraits<TYPE>;
    int T = (K / Tr::BE) * Tr::P;
    if (T > 32) return moe_rows_lpr<TYPE, 64>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, s);
    if (T > 16) return moe_rows_lpr<TYPE, 32>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, s);
    if (T > 8) return moe_rows_lpr<TYPE, 16>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, s);
    return moe_rows_lpr<TYPE, 8>(w, x, y, ws, E, n, K, in_dim1, topk, max_slots, s);
}

hipError_t launch_moe(int type, const void* w, int64_t E, int64_t n, int64_t k, const float* x, int64_t batch,
                      int64_t in_dim1, const uint32_t* ids, int64_t topk, float* y, int* ws, int* sticky,
                      hipStream_t s) {
    int planes = (int)(batch * topk);
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(1024), 0, s, ids, planes, (int)E, ws, sticky, y, (int)n);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    int max_slots = (int)(E < planes ? E : planes);
    switch (type) {
        case T_Q4K: return moe_rows_type<T_Q4K>(w, x, y, ws, (int)E, (int)n, (int)k, (int)in_dim1, (int)topk, max_slots, s);
        case T_Q6K: return moe_rows_type<T_Q6K>(w, x, y, ws, (int)E, (int)n, (int)k, (int)in_dim1, (int)topk, max_slots, s);
        case T_Q8_0: return moe_rows_type<T_Q8_0>(w, x, y, ws, (int)E, (int)n, (int)k, (int)in_dim1, (int)topk, max_slots, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace lloom
