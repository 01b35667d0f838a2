/*
 * kq_oracle.c -- CPU oracle (TEST INFRASTRUCTURE, never the product path).
 *
 * Restates lloom-tensor's CPU arithmetic for the quantized-matmul path in
 * plain C.  Every function cites the Rust it follows.  Build with
 * -O2 -ffp-contract=off (no fast-math) so f32 rounding matches Rust, which
 * never fuses a*b+c.  Rust semantics reproduced here:
 *   f32::round      half away from zero      -> roundf
 *   f32 as i32/i8   saturating, NaN -> 0     -> sat_i32 / sat_i8
 *   i32 as u8/i8    truncating               -> plain C casts
 *   f32::max/min    ignore a NaN operand     -> fmaxf / fminf
 *   half::f16       IEEE round-to-nearest-even (F16C on x86)
 *   Iterator::sum   sequential left fold
 */
#include "kq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- f16 -- */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (exp == 0x1fu) {
        x = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else {
        x = sign | ((exp + 127u - 15u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------ helpers -- */

static int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int32_t)(-2147483647 - 1);
    return (int32_t)v;
}

static int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* utils.rs:1-3 */
static int32_t nearest_int(float v) { return sat_i32(roundf(v)); }

static int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* utils.rs:50-60 */
static void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* total_cmp order for min_by / max_by (utils.rs:230-236): map the bits to a
 * signed integer whose order is IEEE totalOrder. */
static int64_t total_key(float f) {
    int32_t b;
    memcpy(&b, &f, 4);
    return (int64_t)(b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1));
}

/* utils.rs:227-290, make_qkx1_quants(nmax, ntry, x) -> (scale, -min) */
static void make_qkx1_quants(int nmax, int ntry, const float* x, int n, float* out_scale,
                             float* out_min) {
    uint8_t l[256];
    memset(l, 0, sizeof(l));
    /* min_by returns the first minimum, max_by the last maximum */
    float mn = x[0], mx = x[0];
    int64_t kmn = total_key(x[0]), kmx = kmn;
    for (int i = 1; i < n; i++) {
        int64_t kk = total_key(x[i]);
        if (kk < kmn) { kmn = kk; mn = x[i]; }
        if (kk >= kmx) { kmx = kk; mx = x[i]; }
    }
    if (mx == mn) {
        *out_scale = 0.0f;
        *out_min = 0.0f;
        return;
    }
    float min = fminf(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int it = 0; it < ntry; it++) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        int did_change = 0;
        for (int i = 0; i < n; i++) {
            int32_t li = clampi(nearest_int(iscale * (x[i] - min)), 0, nmax);
            uint8_t cl = (uint8_t)li;
            if (cl != l[i]) {
                l[i] = cl;
                did_change = 1;
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

/* utils.rs:62-225, make_qx_quants(n, nmax, x, ls, rmse_type, qw=null) */
static float make_qx_quants(int n, int nmax, const float* x, int8_t* ls, int rmse_type) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float ax = fabsf(x[i]);
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
            int32_t l = nearest_int(iscale * x[i]);
            ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
        }
        return 1.0f / iscale;
    }
    int weight_type = rmse_type % 2;
#define QX_W(xv) (weight_type == 1 ? (xv) * (xv) : 1.0f)
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        float xv = x[i];
        int32_t l = clampi(nearest_int(iscale * xv), -nmax, nmax - 1);
        ls[i] = (int8_t)(l + nmax);
        float w = QX_W(xv);
        float lf = (float)l;
        sumlx += w * xv * lf;
        suml2 += w * lf * lf;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int itry = 0; itry < 3; itry++) {
        float is2 = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        int changed = 0;
        for (int i = 0; i < n; i++) {
            float xv = x[i];
            int32_t l = clampi(nearest_int(is2 * xv), -nmax, nmax - 1);
            if (l + nmax != (int32_t)ls[i]) changed = 1;
            float w = QX_W(xv);
            float lf = (float)l;
            slx += w * xv * lf;
            sl2 += w * lf * lf;
        }
        if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
        for (int i = 0; i < n; i++) {
            int32_t l = nearest_int(is2 * x[i]);
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
            float w = QX_W(xv);
            int32_t l = (int32_t)ls[i] - nmax;
            float slx = sumlx - w * xv * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                int32_t new_l = clampi(nearest_int(xv * sl2 / slx), -nmax, nmax - 1);
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
            int32_t l = clampi(nearest_int(iscale * xv), -nmax, nmax - 1);
            float w = QX_W(xv);
            float lf = (float)l;
            slx += w * xv * lf;
            sl2 += w * lf * lf;
        }
        if (sl2 > 0.0f && slx * slx > best * sl2) {
            for (int i = 0; i < n; i++) {
                int32_t l = nearest_int(iscale * x[i]);
                ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
            }
            scale = slx / sl2;
            best = scale * slx;
        }
    }
#undef QX_W
    return scale;
}

/* -------------------------------------------------------------- Q8_0 -- */

/* k_quants.rs:738-767 */
static void from_float_q8_0(const float* x, size_t nb, orc_block_q8_0* y) {
    for (size_t i = 0; i < nb; i++) {
        const float* xs = x + i * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(fabsf(xs[j]), amax);
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = orc_f32_to_f16(d);
        for (int j = 0; j < 32; j++) y[i].qs[j] = sat_i8(roundf(xs[j] * id));
    }
}

/* k_quants.rs:720-736 */
static void to_float_q8_0(const orc_block_q8_0* x, size_t nb, float* y) {
    for (size_t i = 0; i < nb; i++) {
        float d = orc_f16_to_f32(x[i].d);
        for (int j = 0; j < 32; j++) y[i * 32 + j] = (float)x[i].qs[j] * d;
    }
}

/* k_quants.rs:800-818 */
static float vec_dot_q8_0_unopt(size_t nb, const orc_block_q8_0* x, const orc_block_q8_0* y) {
    float sumf = 0.0f;
    for (size_t i = 0; i < nb; i++) {
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += (int32_t)x[i].qs[j] * (int32_t)y[i].qs[j];
        sumf += (float)s * orc_f16_to_f32(x[i].d) * orc_f16_to_f32(y[i].d);
    }
    return sumf;
}

/* -------------------------------------------------------------- Q8_K -- */

/* k_quants.rs:2400-2438.  An all-zero block gets d = 0, qs = 0 and, here,
 * bsums = 0 (the Rust leaves bsums as they were: zero from qzeros). */
static void from_float_q8k(const float* x, size_t nb, orc_block_q8k* y) {
    for (size_t i = 0; i < nb; i++) {
        const float* xs = x + i * 256;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; j++) {
            if (amax < fabsf(xs[j])) {
                amax = fabsf(xs[j]);
                max = xs[j];
            }
        }
        if (amax == 0.0f) {
            y[i].d = 0.0f;
            memset(y[i].qs, 0, 256);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
        } else {
            float iscale = -127.0f / max;
            for (int j = 0; j < 256; j++) {
                float v = roundf(iscale * xs[j]);
                float c = v < -128.0f ? -128.0f : (v > 127.0f ? 127.0f : v);
                y[i].qs[j] = sat_i8(c);
            }
            for (int j = 0; j < 16; j++) {
                int32_t s = 0;
                for (int t = 0; t < 16; t++) s += y[i].qs[j * 16 + t];
                y[i].bsums[j] = (int16_t)s;
            }
            y[i].d = 1.0f / iscale;
        }
    }
}

/* k_quants.rs:2440-2451 */
static void to_float_q8k(const orc_block_q8k* x, size_t nb, float* y) {
    for (size_t i = 0; i < nb; i++)
        for (int j = 0; j < 256; j++) y[i * 256 + j] = x[i].d * (float)x[i].qs[j];
}

/* k_quants.rs:2380-2398 */
static float vec_dot_q8k_unopt(size_t nb, const orc_block_q8k* x, const orc_block_q8k* y) {
    float sumf = 0.0f;
    for (size_t i = 0; i < nb; i++) {
        int32_t s = 0;
        for (int j = 0; j < 256; j++) s += (int32_t)x[i].qs[j] * (int32_t)y[i].qs[j];
        sumf += (float)s * x[i].d * y[i].d;
    }
    return sumf;
}

/* -------------------------------------------------------------- Q4_K -- */

/* k_quants.rs:1622-1680 */
static void from_float_q4k(const float* xall, size_t nb, orc_block_q4k* blocks) {
    for (size_t b = 0; b < nb; b++) {
        const float* x = xall + b * 256;
        orc_block_q4k* block = &blocks[b];
        memset(block, 0, sizeof(*block));
        float mins[8], scales[8];
        for (int j = 0; j < 8; j++) make_qkx1_quants(15, 5, x + 32 * j, 32, &scales[j], &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            max_scale = fmaxf(scales[j], max_scale);
            max_min = fmaxf(mins[j], max_min);
        }
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        for (int j = 0; j < 8; j++) {
            int32_t a = nearest_int(inv_scale * scales[j]);
            int32_t c = nearest_int(inv_min * mins[j]);
            uint8_t ls = (uint8_t)(a < 63 ? a : 63);
            uint8_t lm = (uint8_t)(c < 63 ? c : 63);
            if (j < 4) {
                block->scales[j] = ls;
                block->scales[j + 4] = lm;
            } else {
                block->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                block->scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                block->scales[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        block->d = orc_f32_to_f16(max_scale / 63.0f);
        block->dmin = orc_f32_to_f16(max_min / 63.0f);
        uint8_t l[256];
        memset(l, 0, sizeof(l));
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            get_scale_min_k4(j, block->scales, &sc, &m);
            float d = orc_f16_to_f32(block->d) * (float)sc;
            if (d != 0.0f) {
                float dm = orc_f16_to_f32(block->dmin) * (float)m;
                for (int ii = 0; ii < 32; ii++) {
                    int32_t lv = nearest_int((x[32 * j + ii] + dm) / d);
                    l[32 * j + ii] = (uint8_t)clampi(lv, 0, 15);
                }
            }
        }
        for (int j = 0; j < 256; j += 64)
            for (int lv = 0; lv < 32; lv++)
                block->qs[(j / 64) * 32 + lv] = (uint8_t)(l[j + lv] | (l[j + lv + 32] << 4));
    }
}

/* k_quants.rs:1747-1774 */
static void to_float_q4k(const orc_block_q4k* xs, size_t nb, float* y) {
    for (size_t b = 0; b < nb; b++) {
        const orc_block_q4k* block = &xs[b];
        float d = orc_f16_to_f32(block->d);
        float min = orc_f16_to_f32(block->dmin);
        float* out = y + b * 256;
        int is = 0, yi = 0;
        for (int j = 0; j < 256; j += 64) {
            const uint8_t* q = block->qs + j / 2;
            uint8_t sc, m;
            get_scale_min_k4(is, block->scales, &sc, &m);
            float d1 = d * (float)sc, m1 = min * (float)m;
            get_scale_min_k4(is + 1, block->scales, &sc, &m);
            float d2 = d * (float)sc, m2 = min * (float)m;
            for (int l = 0; l < 32; l++) out[yi++] = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) out[yi++] = d2 * (float)(q[l] >> 4) - m2;
            is += 2;
        }
    }
}

/* k_quants.rs:1540-1620 */
static float vec_dot_q4k_unopt(size_t nb, const orc_block_q4k* xs, const orc_block_q8k* ys) {
    const uint32_t kmask1 = 0x3f3f3f3fu, kmask2 = 0x0f0f0f0fu, kmask3 = 0x03030303u;
    float sums[8] = {0};
    float sumf = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const orc_block_q4k* x = &xs[b];
        const orc_block_q8k* y = &ys[b];
        int8_t aux8[256];
        int32_t aux32[8] = {0};
        for (int c = 0; c < 4; c++) {
            for (int l = 0; l < 32; l++) aux8[64 * c + l] = (int8_t)(x->qs[32 * c + l] & 0xF);
            for (int l = 0; l < 32; l++) aux8[64 * c + 32 + l] = (int8_t)(x->qs[32 * c + l] >> 4);
        }
        uint32_t utmp[4];
        memcpy(utmp, x->scales, 12); /* little-endian read_u32_into */
        utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
        uint32_t uaux = utmp[1] & kmask1;
        utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
        utmp[2] = uaux;
        utmp[0] &= kmask1;
        uint8_t scales[8], mins[8];
        memcpy(scales, &utmp[0], 8);
        memcpy(mins, &utmp[2], 8);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)y->bsums[j] * (int32_t)mins[j / 2];
        int p = 0;
        for (int s = 0; s < 8; s++) {
            int32_t scale = scales[s];
            for (int r = 0; r < 4; r++) {
                int16_t aux16[8];
                for (int l = 0; l < 8; l++) aux16[l] = (int16_t)((int16_t)y->qs[p + l] * (int16_t)aux8[p + l]);
                for (int l = 0; l < 8; l++) aux32[l] += scale * (int32_t)aux16[l];
                p += 8;
            }
        }
        float d = orc_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = orc_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    float t = -0.0f;
    for (int l = 0; l < 8; l++) t += sums[l];
    return sumf + t;
}

/* -------------------------------------------------------------- Q6_K -- */

/* k_quants.rs:2174-2244 */
static void from_float_q6k(const float* xall, size_t nb, orc_block_q6k* ys) {
    int8_t l[256];
    memset(l, 0, sizeof(l));
    float scales[16];
    for (size_t b = 0; b < nb; b++) {
        const float* x = xall + b * 256;
        orc_block_q6k* y = &ys[b];
        memset(y, 0, sizeof(*y));
        float max_scale = 0.0f, max_abs_scale = 0.0f;
        for (int ib = 0; ib < 16; ib++) {
            float scale = make_qx_quants(16, 32, x + 16 * ib, l + 16 * ib, 1);
            scales[ib] = scale;
            float as = fabsf(scale);
            if (as > max_abs_scale) {
                max_abs_scale = as;
                max_scale = scale;
            }
        }
        float iscale = -128.0f / max_scale;
        y->d = orc_f32_to_f16(1.0f / iscale);
        for (int j = 0; j < 16; j++) {
            int32_t v = nearest_int(iscale * scales[j]);
            y->scales[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; j++) {
            float d = orc_f16_to_f32(y->d) * (float)y->scales[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ii++) {
                int32_t ll = clampi(nearest_int(x[16 * j + ii] / d), -32, 31);
                l[16 * j + ii] = (int8_t)(ll + 32);
            }
        }
        uint8_t* ql = y->ql;
        uint8_t* qh = y->qh;
        for (int j = 0; j < 256; j += 128) {
            for (int li = 0; li < 32; li++) {
                uint8_t q1 = (uint8_t)(l[j + li] & 0xF);
                uint8_t q2 = (uint8_t)(l[j + li + 32] & 0xF);
                uint8_t q3 = (uint8_t)(l[j + li + 64] & 0xF);
                uint8_t q4 = (uint8_t)(l[j + li + 96] & 0xF);
                ql[li] = (uint8_t)(q1 | (q3 << 4));
                ql[li + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[li] = (uint8_t)((l[j + li] >> 4) | ((l[j + li + 32] >> 4) << 2) |
                                   ((l[j + li + 64] >> 4) << 4) | ((l[j + li + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
    }
}

/* k_quants.rs:2327-2358 */
static void to_float_q6k(const orc_block_q6k* xs, size_t nb, float* y) {
    for (size_t b = 0; b < nb; b++) {
        const orc_block_q6k* x = &xs[b];
        float d = orc_f16_to_f32(x->d);
        for (int n = 0; n < 256; n += 128) {
            int idx = n / 128;
            float* ys = y + b * 256 + n;
            const int8_t* sc = x->scales + 8 * idx;
            const uint8_t* ql = x->ql + 64 * idx;
            const uint8_t* qh = x->qh + 32 * idx;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int8_t q1 = (int8_t)(((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
                int8_t q2 = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                int8_t q3 = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                int8_t q4 = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                ys[l] = d * (float)sc[is] * (float)q1;
                ys[l + 32] = d * (float)sc[is + 2] * (float)q2;
                ys[l + 64] = d * (float)sc[is + 4] * (float)q3;
                ys[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

/* k_quants.rs:2115-2172 */
static float vec_dot_q6k_unopt(size_t nb, const orc_block_q6k* xs, const orc_block_q8k* ys) {
    int8_t aux8[256];
    float sums[8] = {0};
    for (size_t b = 0; b < nb; b++) {
        const orc_block_q6k* x = &xs[b];
        const orc_block_q8k* y = &ys[b];
        float aux32[8] = {0};
        for (int j = 0; j < 256; j += 128) {
            int8_t* a = aux8 + j;
            const uint8_t* q4 = x->ql + j / 2;
            const uint8_t* qh = x->qh + j / 4;
            for (int l = 0; l < 32; l++) {
                a[l] = (int8_t)((int32_t)((q4[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
                a[l + 32] = (int8_t)((int32_t)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                a[l + 64] = (int8_t)((int32_t)((q4[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                a[l + 96] = (int8_t)((int32_t)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
            }
        }
        for (int j = 0; j < 16; j++) {
            float scale = (float)x->scales[j];
            const int8_t* q8 = y->qs + 16 * j;
            const int8_t* a = aux8 + 16 * j;
            for (int h = 0; h < 2; h++) {
                int16_t aux16[8];
                for (int l = 0; l < 8; l++) aux16[l] = (int16_t)((int16_t)q8[8 * h + l] * (int16_t)a[8 * h + l]);
                for (int l = 0; l < 8; l++) aux32[l] += scale * (float)aux16[l];
            }
        }
        float d = orc_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += aux32[l] * d;
    }
    float t = -0.0f;
    for (int l = 0; l < 8; l++) t += sums[l];
    return t;
}

/* ------------------------------------------------------------ dispatch -- */

size_t orc_block_bytes(int type) {
    switch (type) {
        case ORC_Q8_0: return sizeof(orc_block_q8_0);
        case ORC_Q4K: return sizeof(orc_block_q4k);
        case ORC_Q6K: return sizeof(orc_block_q6k);
        case ORC_Q8K: return sizeof(orc_block_q8k);
        default: return 0;
    }
}

size_t orc_block_elems(int type) {
    switch (type) {
        case ORC_Q8_0: return 32;
        case ORC_Q4K:
        case ORC_Q6K:
        case ORC_Q8K: return 256;
        default: return 0;
    }
}

int orc_quantize(int type, const float* x, size_t n, void* out) {
    size_t be = orc_block_elems(type);
    if (!be || n % be) return -1;
    size_t nb = n / be;
    switch (type) {
        case ORC_Q8_0: from_float_q8_0(x, nb, (orc_block_q8_0*)out); return 0;
        case ORC_Q4K: from_float_q4k(x, nb, (orc_block_q4k*)out); return 0;
        case ORC_Q6K: from_float_q6k(x, nb, (orc_block_q6k*)out); return 0;
        case ORC_Q8K: from_float_q8k(x, nb, (orc_block_q8k*)out); return 0;
    }
    return -1;
}

int orc_dequantize(int type, const void* blocks, size_t n, float* y) {
    size_t be = orc_block_elems(type);
    if (!be || n % be) return -1;
    size_t nb = n / be;
    switch (type) {
        case ORC_Q8_0: to_float_q8_0((const orc_block_q8_0*)blocks, nb, y); return 0;
        case ORC_Q4K: to_float_q4k((const orc_block_q4k*)blocks, nb, y); return 0;
        case ORC_Q6K: to_float_q6k((const orc_block_q6k*)blocks, nb, y); return 0;
        case ORC_Q8K: to_float_q8k((const orc_block_q8k*)blocks, nb, y); return 0;
    }
    return -1;
}

int orc_dequantize_f16(int type, const void* blocks, size_t n, uint16_t* y) {
    float* tmp = (float*)malloc(n * sizeof(float) + 1);
    if (!tmp) return -1;
    int rc = orc_dequantize(type, blocks, n, tmp);
    if (rc == 0)
        for (size_t i = 0; i < n; i++) y[i] = orc_f32_to_f16(tmp[i]);
    free(tmp);
    return rc;
}

float orc_vec_dot_unopt(int type, size_t n, const void* w, const void* a) {
    switch (type) {
        case ORC_Q8_0: return vec_dot_q8_0_unopt(n / 32, (const orc_block_q8_0*)w, (const orc_block_q8_0*)a);
        case ORC_Q4K: return vec_dot_q4k_unopt(n / 256, (const orc_block_q4k*)w, (const orc_block_q8k*)a);
        case ORC_Q6K: return vec_dot_q6k_unopt(n / 256, (const orc_block_q6k*)w, (const orc_block_q8k*)a);
        case ORC_Q8K: return vec_dot_q8k_unopt(n / 256, (const orc_block_q8k*)w, (const orc_block_q8k*)a);
    }
    return NAN;
}

static int vec_dot_type(int type) { return type == ORC_Q8_0 ? ORC_Q8_0 : ORC_Q8K; }

/* k_quants.rs:2455-2641: quantize every lhs row to the VecDotType, then each
 * output is vec_dot(k, weight row, lhs row).  The GEMM tiling of the Rust
 * (m > 1) calls the same vec_dot per output, so rows are order-independent. */
int orc_matmul(int type, size_t m, size_t k, size_t n, const float* lhs, const void* w,
               float* dst) {
    size_t be = orc_block_elems(type);
    if (!be || k % be) return -1;
    int vt = vec_dot_type(type);
    size_t kb = k / be;
    size_t abytes = orc_block_bytes(vt) * kb;
    size_t wbytes = orc_block_bytes(type) * kb;
    unsigned char* act = (unsigned char*)malloc(abytes * (m ? m : 1));
    if (!act) return -1;
    for (size_t r = 0; r < m; r++) orc_quantize(vt, lhs + r * k, k, act + r * abytes);
    for (size_t r = 0; r < m; r++)
        for (size_t c = 0; c < n; c++)
            dst[r * n + c] = orc_vec_dot_unopt(type, k, (const unsigned char*)w + c * wbytes,
                                               act + r * abytes);
    free(act);
    return 0;
}

/* mod.rs:766-810 */
int orc_matmul_indexed(int type, const void* w, size_t n_experts, size_t n, size_t k, const float* x,
                       size_t in_dim1, const uint32_t* ids, size_t batch, size_t topk,
                       float* dst) {
    size_t be = orc_block_elems(type);
    if (!be || k % be) return -1;
    size_t rb = orc_block_bytes(type) * (k / be);
    (void)n_experts;
    float* row = (float*)malloc(k * sizeof(float) + 1);
    if (!row) return -1;
    for (size_t b = 0; b < batch; b++) {
        for (size_t t = 0; t < topk; t++) {
            size_t e = ids[b * topk + t];
            if (e >= n_experts) {
                free(row);
                return -1;
            }
            size_t xi = in_dim1 == 1 ? 0 : t;
            const float* xrow = x + (b * in_dim1 + xi) * k;
            float* out = dst + (b * topk + t) * n;
            for (size_t r = 0; r < n; r++) {
                orc_dequantize(type, (const void*)((const unsigned char*)w + (e * n + r) * rb), k, row);
                float s = -0.0f;
                for (size_t i = 0; i < k; i++) s += row[i] * xrow[i];
                out[r] = s;
            }
        }
    }
    free(row);
    return 0;
}
