// quant.hip -- quantize (activations and weights) and dequantize kernels.
//
// All of these are bit-exact restatements of lloom-tensor's from_float /
// to_float (lloom-tensor/src/quantized/k_quants.rs) on gfx950: the same f32
// operations in the same order, contraction off, IEEE division, Rust's
// half-away rounding and saturating casts.  Work is spread one block per
// wave (Q8_K), per 8 lanes (Q8_0), or one sub-block per lane for the
// iterative weight fitters, which run their sequential loops unchanged.
#include "kq_common.hpp"
#include "kq_quant.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace lloom {

// ------------------------------------------------- activation quantizers --

// Q8_K: one 256-element block per wave, written in the GGUF block layout
// (f32 d, i8 qs[256], i16 bsums[16]).  nblocks = elems / 256.
__global__ __launch_bounds__(256) void k_quantize_q8k(const float* __restrict__ x,
                                                      uint8_t* __restrict__ out, int64_t nblocks) {
    int lane = threadIdx.x & 63;
    int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    float4 v = *(const float4*)(x + blk * 256 + 4 * lane);
    float d;
    int bs;
    uint32_t q = q8k_block_wave(v, &d, &bs);
    uint8_t* b = out + blk * Q8K_BYTES;
    *(uint32_t*)(b + Q8K_QS + 4 * lane) = q;
    if ((lane & 3) == 0) *(int16_t*)(b + Q8K_BS + 2 * (lane >> 2)) = (int16_t)bs;
    if (lane == 0) *(float*)b = d;
}

// Q8_K into the split layout read by the MFMA kernels: d [k/256][mp] (m
// padded to mp = a multiple of 16) and qs [m][k] with each 256-byte
// superblock permuted so that element 32j + 8g + b (sub-block j, lane group
// g, byte b) sits at 64g + 8j + b: an MFMA lane group's 8 bytes of every
// sub-block are then one contiguous 64-byte run.  One block per wave; the
// values are those of k_quantize_q8k.  With bsp, also the 32-element sums
// of every sub-block j as an MFMA operand: bsp [k/256][mp][16] bytes, byte j
// = sum & 63 and byte 8 + j = sum >> 6 (sum = 64 hi + lo, both int8).
// With `tiled`, qs is instead [mp/16][k/256][4][64][16] bytes: 16-row
// groups, and in each superblock the 64-byte run of lane group g of row r
// (the permuted offsets 64g .. 64g+63) split into four 16-byte pieces i,
// piece i at [i][16g + r % 16]: the MFMA lane 16g + r % 16 then loads its
// operand piece i of a row group's superblock from 1 KB of contiguous bytes.
__global__ __launch_bounds__(256) void k_quantize_split_q8k(const float* __restrict__ x, int8_t* __restrict__ qs,
                                                            float* __restrict__ dt, int8_t* __restrict__ bsp, int m,
                                                            int k, int mp, int tiled) {
    const int nsb = k >> 8;
    const int sb = blockIdx.y * 4 + (threadIdx.x >> 6), mi = blockIdx.x;
    if (sb >= nsb) return;
    q8k_split_block(x, qs, dt, bsp, k, mp, tiled, mi, sb, threadIdx.x & 63);
}

static int64_t pad16(int64_t m) { return (m + 15) & ~(int64_t)15; }

size_t split_q8k_bytes(int64_t k, int64_t m) {
    size_t qb = ((size_t)pad16(m) * k + 255) & ~(size_t)255;  // the tiled layout's padded rows
    return qb + (size_t)(k / 256) * pad16(m) * (sizeof(float) + 16);
}

void split_q8k_ptrs(void* base, int64_t k, int64_t m, int8_t** qs, float** d, int8_t** bsp) {
    size_t qb = ((size_t)pad16(m) * k + 255) & ~(size_t)255;
    *qs = (int8_t*)base;
    *d = (float*)((uint8_t*)base + qb);
    if (bsp) *bsp = (int8_t*)((uint8_t*)base + qb + (size_t)(k / 256) * pad16(m) * sizeof(float));
}

hipError_t launch_quantize_split_q8k(const float* x, int64_t m, int64_t k, int8_t* qs, float* d, hipStream_t s,
                                     int8_t* bsp, bool tiled) {
    const int64_t nsb = k / 256;
    hipLaunchKernelGGL(k_quantize_split_q8k, dim3((unsigned)m, (unsigned)((nsb + 3) / 4)), dim3(256), 0, s, x, qs, d,
                       bsp, (int)m, (int)k, (int)pad16(m), tiled ? 1 : 0);
    return hipGetLastError();
}

// Q8_0: one 32-element block per 8 lanes (f16 d, i8 qs[32]); the 34-byte
// blocks are 2-byte aligned, so bytes are stored as halves.
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ x,
                                                       uint8_t* __restrict__ out, int64_t nblocks) {
    int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    int64_t blk = t >> 3;
    int sub = (int)(t & 7);
    bool ok = blk < nblocks;
    float4 v = ok ? *(const float4*)(x + blk * 32 + 4 * sub) : make_float4(0, 0, 0, 0);
    uint16_t d16;
    uint32_t q = q8_0_block_8lanes(v, &d16);
    if (!ok) return;
    uint8_t* b = out + blk * Q8_0_BYTES;
    uint16_t* h = (uint16_t*)(b + 2 + 4 * sub);
    h[0] = (uint16_t)(q & 0xffffu);
    h[1] = (uint16_t)(q >> 16);
    if (sub == 0) *(uint16_t*)b = d16;
}

// ------------------------------------------------------ Q4_K from_float --
// utils.rs:227-290 make_qkx1_quants(nmax, ntry, x) -> (scale, -min), run
// sequentially by one lane over its 32 values.
__device__ void make_qkx1_quants_dev(int nmax, int ntry, const float* x, float* out_scale,
                                     float* out_min) {
    const int n = 32;
    uint8_t l[32];
    for (int i = 0; i < n; i++) l[i] = 0;
    // min_by(total_cmp) keeps the first minimum, max_by the last maximum.
    auto key = [](float f) -> int {
        int b = __builtin_bit_cast(int, f);
        return b ^ (int)(((unsigned)(b >> 31)) >> 1);
    };
    float mn = x[0], mx = x[0];
    int kmn = key(x[0]), kmx = kmn;
    for (int i = 1; i < n; i++) {
        int kk = key(x[i]);
        if (kk < kmn) { kmn = kk; mn = x[i]; }
        if (kk >= kmx) { kmx = kk; mx = x[i]; }
    }
    if (mx == mn) {
        *out_scale = 0.0f;
        *out_min = 0.0f;
        return;
    }
    float min = __builtin_fminf(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int it = 0; it < ntry; it++) {
        float sumlx = 0.0f;
        int suml2 = 0;
        bool did_change = false;
        for (int i = 0; i < n; i++) {
            int li = clampi(nearest_int(iscale * (x[i] - min)), 0, nmax);
            uint8_t cl = (uint8_t)li;
            if (cl != l[i]) {
                l[i] = cl;
                did_change = true;
            }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = -0.0f;
        for (int i = 0; i < n; i++) sum += x[i] - scale * (float)l[i];
        min = sum / (float)n;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *out_scale = scale;
    *out_min = -min;
}

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int* d, int* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// BlockQ4K::from_float (k_quants.rs:1622-1680).  8 lanes per superblock,
// lane j fits sub-block j; a 64-thread group covers 8 superblocks.
__global__ __launch_bounds__(64) void k_quantize_q4k(const float* __restrict__ x,
                                                     uint8_t* __restrict__ out, int64_t nblocks) {
    __shared__ uint8_t lbuf[8][256];
    int t = threadIdx.x;
    int g = t >> 3, j = t & 7;
    int64_t blk = (int64_t)blockIdx.x * 8 + g;
    bool ok = blk < nblocks;
    const float* xb = x + (ok ? blk : 0) * 256;
    float xs[32];
    for (int i = 0; i < 32; i++) xs[i] = ok ? xb[32 * j + i] : 0.0f;
    float sc, mn;
    make_qkx1_quants_dev(15, 5, xs, &sc, &mn);
    // every lane of the group sees all 8 (scale, min)
    float scales[8], mins[8];
    for (int i = 0; i < 8; i++) {
        scales[i] = __shfl(sc, (t & ~7) + i, 64);
        mins[i] = __shfl(mn, (t & ~7) + i, 64);
    }
    float max_scale = 0.0f, max_min = 0.0f;
    for (int i = 0; i < 8; i++) {
        max_scale = __builtin_fmaxf(scales[i], max_scale);
        max_min = __builtin_fmaxf(mins[i], max_min);
    }
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint8_t packed[12];
    for (int i = 0; i < 12; i++) packed[i] = 0;
    for (int i = 0; i < 8; i++) {
        int a = nearest_int(inv_scale * scales[i]);
        int c = nearest_int(inv_min * mins[i]);
        uint8_t ls = (uint8_t)(a < 63 ? a : 63);
        uint8_t lm = (uint8_t)(c < 63 ? c : 63);
        if (i < 4) {
            packed[i] = ls;
            packed[i + 4] = lm;
        } else {
            packed[i + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            packed[i - 4] |= (uint8_t)((ls >> 4) << 6);
            packed[i] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    uint16_t dh = f32_to_f16(max_scale / 63.0f);
    uint16_t mh = f32_to_f16(max_min / 63.0f);
    int s6, m6;
    scale_min_k4(j, packed, &s6, &m6);
    float d = f16_to_f32(dh) * (float)s6;
    for (int i = 0; i < 32; i++) lbuf[g][32 * j + i] = 0;
    if (d != 0.0f) {
        float dm = f16_to_f32(mh) * (float)m6;
        for (int i = 0; i < 32; i++) {
            int lv = nearest_int((xs[i] + dm) / d);
            lbuf[g][32 * j + i] = (uint8_t)clampi(lv, 0, 15);
        }
    }
    __syncthreads();
    if (!ok) return;
    uint8_t* b = out + blk * Q4K_BYTES;
    // lanes 2c and 2c+1 share the 32 bytes of qs[32c..32c+32)
    int c = j >> 1, half = j & 1;
    for (int i = 0; i < 16; i += 4) {
        uint32_t w = 0;
        for (int e = 0; e < 4; e++) {
            int l = 16 * half + i + e;
            uint32_t v = lbuf[g][64 * c + l] | (lbuf[g][64 * c + 32 + l] << 4);
            w |= v << (8 * e);
        }
        *(uint32_t*)(b + 16 + 32 * c + 16 * half + i) = w;
    }
    if (j == 0) {
        *(uint32_t*)b = (uint32_t)dh | ((uint32_t)mh << 16);
        for (int i = 0; i < 12; i += 4)
            *(uint32_t*)(b + 4 + i) = packed[i] | (packed[i + 1] << 8) | (packed[i + 2] << 16) |
                                      ((uint32_t)packed[i + 3] << 24);
    }
}

// ------------------------------------------------------ Q6_K from_float --
// utils.rs:62-225 make_qx_quants(n = 16, nmax, x, ls, rmse_type, qw = null).
__device__ float make_qx_quants_dev(int nmax, const float* x, int8_t* ls, int rmse_type) {
    const int n = 16;
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float ax = __builtin_fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax == 0.0f) {
        for (int i = 0; i < n; i++) ls[i] = 0;
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; i++) {
            int l = nearest_int(iscale * x[i]);
            ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
        }
        return 1.0f / iscale;
    }
    const bool wt = (rmse_type % 2) == 1;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        float xv = x[i];
        int l = clampi(nearest_int(iscale * xv), -nmax, nmax - 1);
        ls[i] = (int8_t)(l + nmax);
        float w = wt ? xv * xv : 1.0f;
        float lf = (float)l;
        sumlx += w * xv * lf;
        suml2 += w * lf * lf;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int itry = 0; itry < 3; itry++) {
        float is2 = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        bool changed = false;
        for (int i = 0; i < n; i++) {
            float xv = x[i];
            int l = clampi(nearest_int(is2 * xv), -nmax, nmax - 1);
            if (l + nmax != (int)ls[i]) changed = true;
            float w = wt ? xv * xv : 1.0f;
            float lf = (float)l;
            slx += w * xv * lf;
            sl2 += w * lf * lf;
        }
        if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
        for (int i = 0; i < n; i++) {
            int l = nearest_int(is2 * x[i]);
            ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
        }
        sumlx = slx;
        suml2 = sl2;
        scale = sumlx / suml2;
        best = scale * sumlx;
    }
    for (int itry = 0; itry < 5; itry++) {
        int n_changed = 0;
        for (int i = 0; i < n; i++) {
            float xv = x[i];
            float w = wt ? xv * xv : 1.0f;
            int l = (int)ls[i] - nmax;
            float slx = sumlx - w * xv * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                int new_l = clampi(nearest_int(xv * sl2 / slx), -nmax, nmax - 1);
                if (new_l != l) {
                    slx += w * xv * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        ls[i] = (int8_t)(nmax + new_l);
                        sumlx = slx;
                        suml2 = sl2;
                        scale = sumlx / suml2;
                        best = scale * sumlx;
                        n_changed++;
                    }
                }
            }
        }
        if (n_changed == 0) break;
    }
    if (rmse_type < 3) return scale;
    for (int is = -4; is < 4; is++) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / max;
        float slx = 0.0f, sl2 = 0.0f;
        for (int i = 0; i < n; i++) {
            float xv = x[i];
            int l = clampi(nearest_int(iscale * xv), -nmax, nmax - 1);
            float w = wt ? xv * xv : 1.0f;
            float lf = (float)l;
            slx += w * xv * lf;
            sl2 += w * lf * lf;
        }
        if (sl2 > 0.0f && slx * slx > best * sl2) {
            for (int i = 0; i < n; i++) {
                int l = nearest_int(iscale * x[i]);
                ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
            }
            scale = slx / sl2;
            best = scale * slx;
        }
    }
    return scale;
}

// BlockQ6K::from_float (k_quants.rs:2174-2244).  16 lanes per superblock,
// lane ib fits 16-element group ib; a 64-thread group covers 4 superblocks.
__global__ __launch_bounds__(64) void k_quantize_q6k(const float* __restrict__ x,
                                                     uint8_t* __restrict__ out, int64_t nblocks) {
    __shared__ int8_t lbuf[4][256];
    int t = threadIdx.x;
    int g = t >> 4, ib = t & 15;
    int64_t blk = (int64_t)blockIdx.x * 4 + g;
    bool ok = blk < nblocks;
    const float* xb = x + (ok ? blk : 0) * 256 + 16 * ib;
    float xs[16];
    for (int i = 0; i < 16; i++) xs[i] = ok ? xb[i] : 0.0f;
    int8_t l[16];
    float scale = make_qx_quants_dev(32, xs, l, 1);
    // max_abs_scale over ib ascending, strict '>' : the first maximum wins
    float a = __builtin_fabsf(scale);
    if (a != a) a = -1.0f;
    float best_a = a, best_s = scale;
    int best_i = ib;
    for (int o = 1; o < 16; o <<= 1) {
        float oa = __shfl_xor(best_a, o, 64);
        float os = __shfl_xor(best_s, o, 64);
        int oi = __shfl_xor(best_i, o, 64);
        if (oa > best_a || (oa == best_a && oi < best_i)) {
            best_a = oa;
            best_s = os;
            best_i = oi;
        }
    }
    float max_scale = best_a > 0.0f ? best_s : 0.0f;
    float iscale = -128.0f / max_scale;
    uint16_t dh = f32_to_f16(1.0f / iscale);
    int sv = nearest_int(iscale * scale);
    int8_t ysc = (int8_t)(sv < 127 ? sv : 127);
    float d = f16_to_f32(dh) * (float)ysc;
    if (d != 0.0f) {
        for (int i = 0; i < 16; i++) {
            int ll = clampi(nearest_int(xs[i] / d), -32, 31);
            l[i] = (int8_t)(ll + 32);
        }
    }
    for (int i = 0; i < 16; i++) lbuf[g][16 * ib + i] = l[i];
    // scales: every lane of the group needs the 16 i8 scales for the store
    __syncthreads();
    if (!ok) return;
    uint8_t* b = out + blk * Q6K_BYTES;
    // lane ib packs ql/qh for li in [2*ib, 2*ib+2) of each 128-half
    for (int h = 0; h < 2; h++) {
        const int8_t* L = lbuf[g] + 128 * h;
        for (int li = 2 * ib; li < 2 * ib + 2; li++) {
            uint8_t q1 = L[li] & 0xF, q2 = L[li + 32] & 0xF, q3 = L[li + 64] & 0xF,
                    q4 = L[li + 96] & 0xF;
            b[64 * h + li] = (uint8_t)(q1 | (q3 << 4));
            b[64 * h + li + 32] = (uint8_t)(q2 | (q4 << 4));
            b[Q6K_QH + 32 * h + li] = (uint8_t)((L[li] >> 4) | ((L[li + 32] >> 4) << 2) |
                                                ((L[li + 64] >> 4) << 4) | ((L[li + 96] >> 4) << 6));
        }
    }
    b[Q6K_SC + ib] = (uint8_t)ysc;
    if (ib == 0) {
        b[Q6K_D] = (uint8_t)(dh & 0xff);
        b[Q6K_D + 1] = (uint8_t)(dh >> 8);
    }
}

// ---------------------------------------------------------- dequantize --

template <typename OutT>
__device__ __forceinline__ void store_out(OutT* y, int64_t i, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* y, int64_t i, float v) { y[i] = v; }
template <>
__device__ __forceinline__ void store_out<uint16_t>(uint16_t* y, int64_t i, float v) {
    y[i] = f32_to_f16(v);
}

// Row gather of the dequantizers (QTensor::embedding, mod.rs:1101-1137; the
// CPU arm's QuantizedType::embedding, :812-838): output block ob belongs to
// output row ob / rb and reads block ob % rb of weight row ids[row].  With
// ids null the map is the identity (dequantize).  An id >= rows stores a
// zero row and raises flag[0] (sticky) and flag[1] (this call).
struct RowMap {
    const uint32_t* ids;
    int64_t rb, rows;
    int* flag;
};

// The source block of output block ob, or -1 for a bad id.
__device__ __forceinline__ int64_t src_block(int64_t ob, const RowMap& rm) {
    if (!rm.ids) return ob;
    const int64_t r = ob / rm.rb;
    const uint32_t id = rm.ids[r];
    if ((int64_t)id >= rm.rows) {
        if (ob % rm.rb == 0) {
            atomicOr(&rm.flag[0], 1);
            atomicOr(&rm.flag[1], 1);
        }
        return -1;
    }
    return (int64_t)id * rm.rb + (ob - r * rm.rb);
}

// BlockQ8_0::to_float (k_quants.rs:720-736): y = q * f32(d).
template <typename OutT>
__global__ __launch_bounds__(256) void k_dequant_q8_0(const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                      int64_t elems, RowMap rm) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= elems) return;
    const int64_t sb = src_block(i >> 5, rm);
    if (sb < 0) {
        store_out(y, i, 0.0f);
        return;
    }
    const uint8_t* b = w + sb * Q8_0_BYTES;
    float d = f16_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    store_out(y, i, (float)(int8_t)b[2 + (i & 31)] * d);
}

// BlockQ8K::to_float (k_quants.rs:2440-2451): y = d * q.
template <typename OutT>
__global__ __launch_bounds__(256) void k_dequant_q8k(const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                     int64_t elems, RowMap rm) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= elems) return;
    const int64_t sb = src_block(i >> 8, rm);
    if (sb < 0) {
        store_out(y, i, 0.0f);
        return;
    }
    const uint8_t* b = w + sb * Q8K_BYTES;
    float d = *(const float*)b;
    store_out(y, i, d * (float)(int8_t)b[Q8K_QS + (i & 255)]);
}

// BlockQ4K::to_float (k_quants.rs:1747-1774): per 64-chunk c, low nibbles
// y = d*sc(2c)*q - dmin*m(2c), high nibbles with sub-block 2c+1.
// 64 threads per superblock, each 2 bytes -> 4 outputs.
template <typename OutT>
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                     int64_t nblocks, RowMap rm) {
    int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    int t = threadIdx.x & 63;
    const int64_t sb = src_block(blk, rm);
    if (sb < 0) {
        for (int e = 0; e < 4; e++) store_out(y, blk * 256 + 4 * t + e, 0.0f);
        return;
    }
    const uint8_t* b = w + sb * Q4K_BYTES;
    float d = f16_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    float mn = f16_to_f32((uint32_t)b[2] | ((uint32_t)b[3] << 8));
    const uint8_t* sc = b + 4;
    int c = t >> 4, l0 = (t & 15) * 2;
    int s1, m1, s2, m2;
    scale_min_k4(2 * c, sc, &s1, &m1);
    scale_min_k4(2 * c + 1, sc, &s2, &m2);
    float d1 = d * (float)s1, mm1 = mn * (float)m1;
    float d2 = d * (float)s2, mm2 = mn * (float)m2;
    int64_t base = blk * 256 + 64 * c;
    for (int e = 0; e < 2; e++) {
        uint32_t q = b[16 + 32 * c + l0 + e];
        store_out(y, base + l0 + e, d1 * (float)(q & 0xF) - mm1);
        store_out(y, base + 32 + l0 + e, d2 * (float)(q >> 4) - mm2);
    }
}

// BlockQ6K::to_float (k_quants.rs:2327-2358): y = d * sc[is] * q, with
// q = (4 low bits | 2 high bits) - 32.  64 threads per superblock.
template <typename OutT>
__global__ __launch_bounds__(256) void k_dequant_q6k(const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                     int64_t nblocks, RowMap rm) {
    int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    int t = threadIdx.x & 63;
    const int64_t sb = src_block(blk, rm);
    if (sb < 0) {
        for (int e = 0; e < 4; e++) store_out(y, blk * 256 + 4 * t + e, 0.0f);
        return;
    }
    const uint8_t* b = w + sb * Q6K_BYTES;
    float d = f16_to_f32((uint32_t)b[Q6K_D] | ((uint32_t)b[Q6K_D + 1] << 8));
    int h = t >> 5, l = t & 31;
    const uint8_t* ql = b + 64 * h;
    const uint8_t* qh = b + Q6K_QH + 32 * h;
    const int8_t* sc = (const int8_t*)(b + Q6K_SC + 8 * h);
    int is = l / 16;
    int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
    int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
    int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
    int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
    int64_t base = blk * 256 + 128 * h;
    store_out(y, base + l, d * (float)sc[is] * (float)q1);
    store_out(y, base + l + 32, d * (float)sc[is + 2] * (float)q2);
    store_out(y, base + l + 64, d * (float)sc[is + 4] * (float)q3);
    store_out(y, base + l + 96, d * (float)sc[is + 6] * (float)q4);
}

// ------------------------------------------------------------- launches --

static inline unsigned grid_of(int64_t work, int64_t per) { return (unsigned)((work + per - 1) / per); }

hipError_t launch_quantize_act(int vt, const float* x, void* out, int64_t elems, hipStream_t s) {
    if (vt == T_Q8K) {
        int64_t nb = elems / 256;
        hipLaunchKernelGGL(k_quantize_q8k, dim3(grid_of(nb, 4)), dim3(256), 0, s, x, (uint8_t*)out, nb);
    } else {
        int64_t nb = elems / 32;
        hipLaunchKernelGGL(k_quantize_q8_0, dim3(grid_of(nb * 8, 256)), dim3(256), 0, s, x, (uint8_t*)out,
                           nb);
    }
    return hipGetLastError();
}

hipError_t launch_quantize_weights(int type, const float* x, void* out, int64_t elems, hipStream_t s) {
    switch (type) {
        case T_Q8_0:
        case T_Q8K: return launch_quantize_act(type, x, out, elems, s);
        case T_Q4K: {
            int64_t nb = elems / 256;
            hipLaunchKernelGGL(k_quantize_q4k, dim3(grid_of(nb, 8)), dim3(64), 0, s, x, (uint8_t*)out, nb);
            return hipGetLastError();
        }
        case T_Q6K: {
            int64_t nb = elems / 256;
            hipLaunchKernelGGL(k_quantize_q6k, dim3(grid_of(nb, 4)), dim3(64), 0, s, x, (uint8_t*)out, nb);
            return hipGetLastError();
        }
    }
    return hipErrorInvalidValue;
}

template <typename OutT>
static hipError_t dequant_t(int type, const void* w, OutT* y, int64_t elems, const RowMap& rm, hipStream_t s) {
    const uint8_t* b = (const uint8_t*)w;
    switch (type) {
        case T_Q8_0:
            hipLaunchKernelGGL(k_dequant_q8_0<OutT>, dim3(grid_of(elems, 256)), dim3(256), 0, s, b, y, elems, rm);
            break;
        case T_Q8K:
            hipLaunchKernelGGL(k_dequant_q8k<OutT>, dim3(grid_of(elems, 256)), dim3(256), 0, s, b, y, elems, rm);
            break;
        case T_Q4K:
            hipLaunchKernelGGL(k_dequant_q4k<OutT>, dim3(grid_of(elems / 256, 4)), dim3(256), 0, s, b, y,
                               elems / 256, rm);
            break;
        case T_Q6K:
            hipLaunchKernelGGL(k_dequant_q6k<OutT>, dim3(grid_of(elems / 256, 4)), dim3(256), 0, s, b, y,
                               elems / 256, rm);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequantize(int type, const void* w, void* y, int out_dtype, int64_t elems, hipStream_t s) {
    const RowMap rm{nullptr, 1, 0, nullptr};
    if (out_dtype == T_F16) return dequant_t<uint16_t>(type, w, (uint16_t*)y, elems, rm, s);
    return dequant_t<float>(type, w, (float*)y, elems, rm, s);
}

hipError_t launch_embedding(int type, const void* w, int64_t rows, int64_t hidden, const uint32_t* ids, int64_t n_ids,
                            void* y, int out_dtype, int* flag, hipStream_t s) {
    const RowMap rm{ids, hidden / block_elems(type), rows, flag};
    const int64_t elems = n_ids * hidden;
    if (out_dtype == T_F16) return dequant_t<uint16_t>(type, w, (uint16_t*)y, elems, rm, s);
    return dequant_t<float>(type, w, (float*)y, elems, rm, s);
}

// ---------------------------------------------------------------- cast --
// Tensor::to_dtype between F32 and F16 (the cast the CPU arm's callers make
// around a quantized matmul: matmul_t_f16 converts its f16 lhs to f32 first
// and its f32 sums to f16 last, k_quants.rs:2802-2835; indexed_moe_forward_as
// casts x to act first, mod.rs:1567-1571).  f16 -> f32 is exact, f32 -> f16
// round-to-nearest-even (half::f16::from_f32).  Four elements a lane.
__global__ __launch_bounds__(256) void k_cast_f32_f16(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                      int64_t count) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (i + 4 <= count) {
        const float4 v = *(const float4*)(x + i);
        uint2 o;
        o.x = (uint32_t)f32_to_f16(v.x) | ((uint32_t)f32_to_f16(v.y) << 16);
        o.y = (uint32_t)f32_to_f16(v.z) | ((uint32_t)f32_to_f16(v.w) << 16);
        *(uint2*)(y + i) = o;
    } else {
        for (int64_t j = i; j < count; j++) y[j] = f32_to_f16(x[j]);
    }
}

__global__ __launch_bounds__(256) void k_cast_f16_f32(const uint16_t* __restrict__ x, float* __restrict__ y,
                                                      int64_t count) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (i + 4 <= count) {
        const uint2 v = *(const uint2*)(x + i);
        *(float4*)(y + i) = make_float4(f16_to_f32(v.x & 0xffffu), f16_to_f32(v.x >> 16), f16_to_f32(v.y & 0xffffu),
                                        f16_to_f32(v.y >> 16));
    } else {
        for (int64_t j = i; j < count; j++) y[j] = f16_to_f32(x[j]);
    }
}

hipError_t launch_cast(int src_t, const void* src, int dst_t, void* dst, int64_t count, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((count + 1023) / 1024);
    if (src_t == T_F32 && dst_t == T_F16)
        hipLaunchKernelGGL(k_cast_f32_f16, dim3(grid), dim3(256), 0, s, (const float*)src, (uint16_t*)dst, count);
    else if (src_t == T_F16 && dst_t == T_F32)
        hipLaunchKernelGGL(k_cast_f16_f32, dim3(grid), dim3(256), 0, s, (const uint16_t*)src, (float*)dst, count);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace lloom
