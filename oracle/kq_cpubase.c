/*
 * kq_cpubase.c -- the timed CPU baseline (TEST INFRASTRUCTURE, not product).
 *
 * A restatement of lloom-tensor's CPU QMatMul as it runs on an x86 host
 * with target-cpu=native (AVX2):
 *   activation quantization  k_quants.rs:2477-2508 (from kq_oracle.c)
 *   vec_dot_q8_0_q8_0        avx.rs:70-87
 *   vec_dot_q6k_q8k          avx.rs:130-216
 *   vec_dot_q4k_q8k          avx.rs:442-525
 *   matmul driver            k_quants.rs:2455-2641 (column quads split over
 *                            a persistent barrier pool, workers + caller;
 *                            M > 1: tiles of 4 quads x 16 rows)
 *   pool size                lloom-tensor/src/utils.rs:305-325 (physical cores)
 * The Rust source could not be built here (no Rust toolchain), so this C
 * restatement is what bench.py times as "cpu_baseline" (kind "port").
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "kq_oracle.h"

/* ------------------------------------------------------- AVX2 helpers -- */

static inline float hsum_float_8(__m256 x) {
    __m128 res = _mm256_extractf128_ps(x, 1);
    res = _mm_add_ps(res, _mm256_castps256_ps128(x));
    res = _mm_add_ps(res, _mm_movehl_ps(res, res));
    res = _mm_add_ss(res, _mm_movehdup_ps(res));
    return _mm_cvtss_f32(res);
}

static inline __m256 sum_i16_pairs_float(__m256i x) {
    return _mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_set1_epi16(1), x));
}

static inline __m256 mul_sum_i8_pairs_float(__m256i x, __m256i y) {
    __m256i ax = _mm256_sign_epi8(x, x);
    __m256i sy = _mm256_sign_epi8(y, x);
    return sum_i16_pairs_float(_mm256_maddubs_epi16(ax, sy));
}

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }

/* avx.rs:70-87 */
static float vd_q8_0(size_t nb, const orc_block_q8_0* x, const orc_block_q8_0* y) {
    __m256 acc = _mm256_setzero_ps();
    for (size_t i = 0; i < nb; i++) {
        __m256 d = _mm256_set1_ps(h2f(x[i].d) * h2f(y[i].d));
        __m256i bx = _mm256_loadu_si256((const __m256i*)x[i].qs);
        __m256i by = _mm256_loadu_si256((const __m256i*)y[i].qs);
        acc = _mm256_fmadd_ps(d, mul_sum_i8_pairs_float(bx, by), acc);
    }
    return hsum_float_8(acc);
}

/* avx.rs:442-525 */
static float vd_q4k(size_t nb, const orc_block_q4k* xs, const orc_block_q8k* ys) {
    const uint32_t kmask1 = 0x3f3f3f3fu, kmask2 = 0x0f0f0f0fu, kmask3 = 0x03030303u;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256 acc = _mm256_setzero_ps();
    __m128 acc_m = _mm_setzero_ps();
    for (size_t b = 0; b < nb; b++) {
        const orc_block_q4k* x = &xs[b];
        const orc_block_q8k* y = &ys[b];
        float d = y->d * h2f(x->d);
        float dmin = -y->d * h2f(x->dmin);
        uint32_t utmp[4];
        memcpy(utmp, x->scales, 12);
        utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
        uint32_t uaux = utmp[1] & kmask1;
        utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
        utmp[2] = uaux;
        utmp[0] &= kmask1;
        __m256i mins_and_scales = _mm256_cvtepu8_epi16(
            _mm_set_epi32((int)utmp[3], (int)utmp[2], (int)utmp[1], (int)utmp[0]));
        __m256i q8sums = _mm256_loadu_si256((const __m256i*)y->bsums);
        __m128i q8s = _mm_hadd_epi16(_mm256_extracti128_si256(q8sums, 0),
                                     _mm256_extracti128_si256(q8sums, 1));
        __m128i prod = _mm_madd_epi16(_mm256_extracti128_si256(mins_and_scales, 1), q8s);
        acc_m = _mm_fmadd_ps(_mm_set1_ps(dmin), _mm_cvtepi32_ps(prod), acc_m);
        /* the 16-bit sub-block scales, broadcast one at a time below */
        int16_t sc16[16];
        _mm256_storeu_si256((__m256i*)sc16, mins_and_scales);
        const uint8_t* q4 = x->qs;
        const int8_t* q8 = y->qs;
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            __m256i scale_l = _mm256_set1_epi16(sc16[2 * j]);
            __m256i scale_h = _mm256_set1_epi16(sc16[2 * j + 1]);
            __m256i q4bits = _mm256_loadu_si256((const __m256i*)q4);
            q4 += 32;
            __m256i q4l = _mm256_and_si256(q4bits, m4);
            __m256i q4h = _mm256_and_si256(_mm256_srli_epi16(q4bits, 4), m4);
            __m256i q8l = _mm256_loadu_si256((const __m256i*)q8);
            q8 += 32;
            __m256i p16l = _mm256_madd_epi16(scale_l, _mm256_maddubs_epi16(q4l, q8l));
            sumi = _mm256_add_epi32(sumi, p16l);
            __m256i q8h = _mm256_loadu_si256((const __m256i*)q8);
            q8 += 32;
            __m256i p16h = _mm256_madd_epi16(scale_h, _mm256_maddubs_epi16(q4h, q8h));
            sumi = _mm256_add_epi32(sumi, p16h);
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    acc_m = _mm_add_ps(acc_m, _mm_movehl_ps(acc_m, acc_m));
    acc_m = _mm_add_ss(acc_m, _mm_movehdup_ps(acc_m));
    return hsum_float_8(acc) + _mm_cvtss_f32(acc_m);
}

/* avx.rs:130-216 */
static float vd_q6k(size_t nb, const orc_block_q6k* xs, const orc_block_q8k* ys) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    const __m256i m2 = _mm256_set1_epi8(3);
    const __m256i m32s = _mm256_set1_epi8(32);
    __m256 acc = _mm256_setzero_ps();
    for (size_t b = 0; b < nb; b++) {
        const orc_block_q6k* x = &xs[b];
        const orc_block_q8k* y = &ys[b];
        float d = y->d * h2f(x->d);
        const uint8_t* q4 = x->ql;
        const uint8_t* qh = x->qh;
        const int8_t* q8 = y->qs;
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 2; j++) {
            /* 16 int16 scale lanes: 8 of scales[2g] then 8 of scales[2g+1] */
            __m256i sc[4];
            for (int g = 0; g < 4; g++) {
                int s0 = x->scales[8 * j + 2 * g], s1 = x->scales[8 * j + 2 * g + 1];
                sc[g] = _mm256_setr_epi16(s0, s0, s0, s0, s0, s0, s0, s0, s1, s1, s1, s1, s1, s1,
                                          s1, s1);
            }
            __m256i q4bits1 = _mm256_loadu_si256((const __m256i*)q4);
            q4 += 32;
            __m256i q4bits2 = _mm256_loadu_si256((const __m256i*)q4);
            q4 += 32;
            __m256i q4bits_h = _mm256_loadu_si256((const __m256i*)qh);
            qh += 32;
            __m256i q4h_0 = _mm256_slli_epi16(_mm256_and_si256(q4bits_h, m2), 4);
            __m256i q4h_1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(q4bits_h, 2), m2), 4);
            __m256i q4h_2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(q4bits_h, 4), m2), 4);
            __m256i q4h_3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(q4bits_h, 6), m2), 4);
            __m256i q4_0 = _mm256_or_si256(_mm256_and_si256(q4bits1, m4), q4h_0);
            __m256i q4_1 = _mm256_or_si256(_mm256_and_si256(q4bits2, m4), q4h_1);
            __m256i q4_2 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q4bits1, 4), m4), q4h_2);
            __m256i q4_3 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q4bits2, 4), m4), q4h_3);
            __m256i q8_0 = _mm256_loadu_si256((const __m256i*)q8);
            __m256i q8_1 = _mm256_loadu_si256((const __m256i*)(q8 + 32));
            __m256i q8_2 = _mm256_loadu_si256((const __m256i*)(q8 + 64));
            __m256i q8_3 = _mm256_loadu_si256((const __m256i*)(q8 + 96));
            q8 += 128;
            __m256i p16_0 = _mm256_sub_epi16(_mm256_maddubs_epi16(q4_0, q8_0), _mm256_maddubs_epi16(m32s, q8_0));
            __m256i p16_1 = _mm256_sub_epi16(_mm256_maddubs_epi16(q4_1, q8_1), _mm256_maddubs_epi16(m32s, q8_1));
            __m256i p16_2 = _mm256_sub_epi16(_mm256_maddubs_epi16(q4_2, q8_2), _mm256_maddubs_epi16(m32s, q8_2));
            __m256i p16_3 = _mm256_sub_epi16(_mm256_maddubs_epi16(q4_3, q8_3), _mm256_maddubs_epi16(m32s, q8_3));
            p16_0 = _mm256_madd_epi16(sc[0], p16_0);
            p16_1 = _mm256_madd_epi16(sc[1], p16_1);
            p16_2 = _mm256_madd_epi16(sc[2], p16_2);
            p16_3 = _mm256_madd_epi16(sc[3], p16_3);
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p16_0, p16_1));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p16_2, p16_3));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum_float_8(acc);
}

float cpb_vec_dot(int type, size_t n, const void* w, const void* a) {
    switch (type) {
        case ORC_Q8_0: return vd_q8_0(n / 32, (const orc_block_q8_0*)w, (const orc_block_q8_0*)a);
        case ORC_Q4K: return vd_q4k(n / 256, (const orc_block_q4k*)w, (const orc_block_q8k*)a);
        case ORC_Q6K: return vd_q6k(n / 256, (const orc_block_q6k*)w, (const orc_block_q8k*)a);
    }
    return 0.0f;
}

/* ------------------------------------------------------ barrier pool -- */

typedef struct {
    int type;
    size_t m, k, n, kb, wbytes, abytes, quads_total, quads_per_thread;
    const unsigned char* w;
    const unsigned char* act;
    float* dst;
    size_t row; /* decode row, or (size_t)-1 for the GEMM dispatch */
} job_t;

static pthread_t g_threads[256];
static int g_workers = -1;
static pthread_barrier_t g_start, g_done;
static job_t g_job;
static volatile int g_quit;

static void run_part(const job_t* j, size_t tid) {
    size_t start = tid * j->quads_per_thread;
    if (start >= j->quads_total) return;
    size_t end = j->quads_total < start + j->quads_per_thread ? j->quads_total
                                                              : start + j->quads_per_thread;
    if (j->row != (size_t)-1) {
        const unsigned char* a = j->act + j->row * j->abytes;
        float* out = j->dst + j->row * j->n;
        for (size_t q = start; q < end; q++)
            for (size_t c = 4 * q; c < 4 * q + 4; c++)
                out[c] = cpb_vec_dot(j->type, j->k, j->w + c * j->wbytes, a);
        return;
    }
    for (size_t ct = start; ct < end; ct += 4) {
        size_t ce = end < ct + 4 ? end : ct + 4;
        for (size_t rt = 0; rt < j->m; rt += 16) {
            size_t re = j->m < rt + 16 ? j->m : rt + 16;
            for (size_t q = ct; q < ce; q++)
                for (size_t r = rt; r < re; r++)
                    for (size_t c = 4 * q; c < 4 * q + 4; c++)
                        j->dst[r * j->n + c] =
                            cpb_vec_dot(j->type, j->k, j->w + c * j->wbytes, j->act + r * j->abytes);
        }
    }
}

static void* worker(void* arg) {
    size_t tid = (size_t)arg;
    for (;;) {
        pthread_barrier_wait(&g_start);
        if (g_quit) return NULL;
        run_part(&g_job, tid);
        pthread_barrier_wait(&g_done);
    }
}

/* Physical cores: distinct (physical id, core id) pairs of /proc/cpuinfo. */
int cpb_physical_cores(void) {
    FILE* f = fopen("/proc/cpuinfo", "r");
    if (!f) return (int)sysconf(_SC_NPROCESSORS_ONLN);
    char line[256];
    int phys = 0, core = 0, count = 0;
    static int seen[4096];
    memset(seen, 0, sizeof(seen));
    while (fgets(line, sizeof line, f)) {
        if (!strncmp(line, "physical id", 11)) phys = atoi(strchr(line, ':') + 1);
        if (!strncmp(line, "core id", 7)) {
            core = atoi(strchr(line, ':') + 1);
            int key = (phys * 512 + core) % 4096;
            if (!seen[key]) {
                seen[key] = 1;
                count++;
            }
        }
    }
    fclose(f);
    if (count <= 0) count = (int)sysconf(_SC_NPROCESSORS_ONLN);
    return count;
}

/* Start the pool with nthreads total threads (nthreads-1 workers + caller). */
int cpb_pool_init(int nthreads) {
    if (g_workers >= 0) return g_workers + 1;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    g_workers = nthreads - 1;
    pthread_barrier_init(&g_start, NULL, (unsigned)nthreads);
    pthread_barrier_init(&g_done, NULL, (unsigned)nthreads);
    for (int i = 0; i < g_workers; i++) pthread_create(&g_threads[i], NULL, worker, (void*)(size_t)i);
    return nthreads;
}

static void pool_execute(void) {
    pthread_barrier_wait(&g_start);
    run_part(&g_job, (size_t)g_workers);
    pthread_barrier_wait(&g_done);
}

/* k_quants::matmul (k_quants.rs:2455-2641) on the pool. */
int cpb_matmul(int type, size_t m, size_t k, size_t n, const float* lhs, const void* w,
               float* dst) {
    if (g_workers < 0) cpb_pool_init(cpb_physical_cores());
    size_t be = orc_block_elems(type);
    if (!be || k % be) return -1;
    int vt = type == ORC_Q8_0 ? ORC_Q8_0 : ORC_Q8K;
    size_t kb = k / be;
    static unsigned char* scratch = NULL;
    static size_t scratch_len = 0;
    size_t abytes = orc_block_bytes(vt) * kb;
    if (scratch_len < abytes * m) {
        free(scratch);
        scratch = (unsigned char*)malloc(abytes * m);
        scratch_len = abytes * m;
    }
    for (size_t r = 0; r < m; r++) orc_quantize(vt, lhs + r * k, k, scratch + r * abytes);
    size_t n_quad = n & ~(size_t)3;
    size_t nt = (size_t)g_workers + 1;
    job_t j = {type, m, k, n, kb, orc_block_bytes(type) * kb, abytes, n_quad / 4,
               (n_quad / 4 + nt - 1) / nt, (const unsigned char*)w, scratch, dst, 0};
    if (m > 1) {
        j.row = (size_t)-1;
        g_job = j;
        pool_execute();
        for (size_t r = 0; r < m; r++)
            for (size_t c = n_quad; c < n; c++)
                dst[r * n + c] = cpb_vec_dot(type, k, j.w + c * j.wbytes, scratch + r * abytes);
        return 0;
    }
    for (size_t r = 0; r < m; r++) {
        j.row = r;
        g_job = j;
        pool_execute();
        for (size_t c = n_quad; c < n; c++)
            dst[r * n + c] = cpb_vec_dot(type, k, j.w + c * j.wbytes, scratch + r * abytes);
    }
    return 0;
}
