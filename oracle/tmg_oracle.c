/*
 * TEST INFRASTRUCTURE ONLY -- the oracle.
 *
 * A CPU restatement, in plain C, of the TinyMiniGo Rust CPU path
 * (reference files src/tensor.rs and src/model.rs).  It exists to check the
 * HIP product path and to be timed as the CPU baseline.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library never links or calls it.
 *
 * Numerical contract: every function follows the reference's operation order
 * so that results are bit-identical to the Rust build on an AVX2+FMA host:
 *   - 8-lane FMA dot products with the reference's horizontal-sum order
 *     (src/tensor.rs:78-110);
 *   - no FMA contraction anywhere else (built with -ffp-contract=off; Rust
 *     never contracts);
 *   - glibc expf/powf/sinf/cosf/sqrtf, which Rust's f32 methods call on
 *     x86_64-linux-gnu.
 * The AVX2 path is taken when the CPU has AVX2+FMA (the reference's own
 * runtime dispatch, src/tensor.rs:9-23); otherwise a scalar path computes the
 * same lanes with fmaf(), which is exact, so both give the same bits.
 *
 * Threading mirrors the reference so the CPU baseline is timed the way the
 * reference runs: GEMV uses max(1, ncores/4) threads and is single-threaded
 * below 64 rows (src/tensor.rs:387-388); batched GEMM uses all cores in
 * 8-row jobs (src/tensor.rs:754-791); attention is single-threaded
 * (src/model.rs:441-459, src/tensor.rs:1113-1137) unless the caller raises
 * om_set_attn_threads() (head-parallel, bit-identical: each (token, head)
 * is computed independently).
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <immintrin.h>

#define OM_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* helpers                                                                   */
/* ------------------------------------------------------------------------ */

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16; /* exact widening, src/tensor.rs:85-88 */
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static int g_has_avx2 = -1;
static int has_avx2_fma(void) {
    if (g_has_avx2 < 0) {
        __builtin_cpu_init();
        g_has_avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    }
    return g_has_avx2;
}

/* Thread count: 0 = all logical cores (src/tensor.rs:172-188). */
static int g_threads = 0;
static int g_attn_threads = 1;

OM_API void om_set_num_threads(int n) { g_threads = n; }
OM_API void om_set_attn_threads(int n) { g_attn_threads = n < 1 ? 1 : n; }

static int num_threads(void) {
    if (g_threads > 0) return g_threads;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

OM_API int om_num_threads(void) { return num_threads(); }
OM_API int om_uses_avx2(void) { return has_avx2_fma(); }

/* Horizontal sum of 8 lanes in the order of reduce_add (src/tensor.rs:100-110):
 * ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)). */
static inline float reduce8(const float l[8]) {
    float s0 = l[0] + l[4], s1 = l[1] + l[5], s2 = l[2] + l[6], s3 = l[3] + l[7];
    return (s0 + s2) + (s1 + s3);
}

__attribute__((target("avx2,fma"))) static inline float reduce_add_avx(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    __m128 s2 = _mm_add_ps(s, _mm_movehl_ps(s, s));
    __m128 s3 = _mm_add_ss(s2, _mm_shuffle_ps(s2, s2, 0x55));
    return _mm_cvtss_f32(s3);
}

/* ------------------------------------------------------------------------ */
/* A5: dot products (src/tensor.rs:27-110)                                   */
/* ------------------------------------------------------------------------ */

__attribute__((target("avx2,fma"))) static float dot_bf16_avx2(const float *a, const uint16_t *b, size_t n) {
    __m256 acc = _mm256_setzero_ps();
    size_t chunks = n / 8;
    for (size_t i = 0; i < chunks; i++) {
        __m256 va = _mm256_loadu_ps(a + i * 8);
        __m128i w128 = _mm_loadu_si128((const __m128i *)(b + i * 8));
        __m256i w256 = _mm256_cvtepu16_epi32(w128);
        __m256 wf = _mm256_castsi256_ps(_mm256_slli_epi32(w256, 16));
        acc = _mm256_fmadd_ps(va, wf, acc);
    }
    float sum = reduce_add_avx(acc);
    for (size_t i = chunks * 8; i < n; i++) sum += a[i] * bf16_to_f32(b[i]);
    return sum;
}

static float dot_bf16_scalar8(const float *a, const uint16_t *b, size_t n) {
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t chunks = n / 8;
    for (size_t i = 0; i < chunks; i++)
        for (int j = 0; j < 8; j++) lane[j] = fmaf(a[i * 8 + j], bf16_to_f32(b[i * 8 + j]), lane[j]);
    float sum = reduce8(lane);
    for (size_t i = chunks * 8; i < n; i++) sum += a[i] * bf16_to_f32(b[i]);
    return sum;
}

/* dot_bf16 (src/tensor.rs:42-54 -> 78-96). */
OM_API float om_dot_bf16(const float *a, const uint16_t *b, size_t n) {
    return has_avx2_fma() ? dot_bf16_avx2(a, b, n) : dot_bf16_scalar8(a, b, n);
}

__attribute__((target("avx2,fma"))) static float dot_f32_avx2(const float *a, const float *b, size_t n) {
    __m256 acc = _mm256_setzero_ps();
    size_t chunks = n / 8;
    for (size_t i = 0; i < chunks; i++)
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i * 8), _mm256_loadu_ps(b + i * 8), acc);
    float sum = reduce_add_avx(acc);
    for (size_t i = chunks * 8; i < n; i++) sum += a[i] * b[i];
    return sum;
}

static float dot_f32_scalar8(const float *a, const float *b, size_t n) {
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t chunks = n / 8;
    for (size_t i = 0; i < chunks; i++)
        for (int j = 0; j < 8; j++) lane[j] = fmaf(a[i * 8 + j], b[i * 8 + j], lane[j]);
    float sum = reduce8(lane);
    for (size_t i = chunks * 8; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* dot (src/tensor.rs:27-36 -> 58-74). */
OM_API float om_dot(const float *a, const float *b, size_t n) {
    return has_avx2_fma() ? dot_f32_avx2(a, b, n) : dot_f32_scalar8(a, b, n);
}

/* ------------------------------------------------------------------------ */
/* A6: decode GEMV y = W x, W BF16 [out,in] (src/tensor.rs:331-460)          */
/* ------------------------------------------------------------------------ */

typedef struct {
    const float *x;
    const uint16_t *w;
    float *y;
    size_t in, start, end;
} gemv_job;

static void *gemv_worker(void *p) {
    gemv_job *j = (gemv_job *)p;
    for (size_t o = j->start; o < j->end; o++) j->y[o] = om_dot_bf16(j->x, j->w + o * j->in, j->in);
    return NULL;
}

/* matmul_w_into for WMat::BF16: rows split into ceil(out/nthreads) chunks,
 * one scoped thread each, nthreads = max(1, ncores/4) capped at out; single
 * thread when out < 64 (MIN_ROWS_FOR_THREADS). */
OM_API void om_matmul_w(const float *x, const uint16_t *w, size_t out, size_t in, float *y) {
    size_t nthreads = (size_t)num_threads() / 4;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > out) nthreads = out;
    if (nthreads <= 1 || out < 64) {
        for (size_t o = 0; o < out; o++) y[o] = om_dot_bf16(x, w + o * in, in);
        return;
    }
    size_t chunk = (out + nthreads - 1) / nthreads;
    pthread_t th[256];
    gemv_job jobs[256];
    size_t nt = 0;
    for (size_t s = 0; s < out && nt < 256; s += chunk, nt++) {
        jobs[nt] = (gemv_job){x, w, y, in, s, s + chunk < out ? s + chunk : out};
        pthread_create(&th[nt], NULL, gemv_worker, &jobs[nt]);
    }
    for (size_t i = 0; i < nt; i++) pthread_join(th[i], NULL);
}

/* matmul_w_into for WMat::F32 (src/tensor.rs:387-420): `dot` (dot_f32_avx2,
 * src/tensor.rs:58-74) per row, threaded like the BF16 arm. */
typedef struct {
    const float *x, *w;
    float *y;
    size_t in, start, end;
} gemv_f32_job;

static void *gemv_f32_worker(void *p) {
    gemv_f32_job *j = (gemv_f32_job *)p;
    for (size_t o = j->start; o < j->end; o++) j->y[o] = om_dot(j->x, j->w + o * j->in, j->in);
    return NULL;
}

OM_API void om_matmul_w_f32(const float *x, const float *w, size_t out, size_t in, float *y) {
    size_t nthreads = (size_t)num_threads() / 4;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > out) nthreads = out;
    if (nthreads <= 1 || out < 64) {
        for (size_t o = 0; o < out; o++) y[o] = om_dot(x, w + o * in, in);
        return;
    }
    size_t chunk = (out + nthreads - 1) / nthreads;
    pthread_t th[256];
    gemv_f32_job jobs[256];
    size_t nt = 0;
    for (size_t s = 0; s < out && nt < 256; s += chunk, nt++) {
        jobs[nt] = (gemv_f32_job){x, w, y, in, s, s + chunk < out ? s + chunk : out};
        pthread_create(&th[nt], NULL, gemv_f32_worker, &jobs[nt]);
    }
    for (size_t i = 0; i < nt; i++) pthread_join(th[i], NULL);
}

/* matmul_batch_w_into for WMat::F32 (src/tensor.rs:573-760): on an AVX2
 * host gemm_tile_avx2 loads f32 weight lanes where the BF16 arm widens
 * (load_w_m256, src/tensor.rs:899-904) and keeps dot's order per element,
 * so every element equals dot(x_t, w_o) (src/tensor.rs:734-738); the
 * scalar fallback is that dot too.  Rows are split over the cores. */
typedef struct {
    const float *x, *w;
    float *y;
    size_t out, in, T, start, end;
} gemm_f32_job;

static void *gemm_f32_worker(void *p) {
    gemm_f32_job *j = (gemm_f32_job *)p;
    for (size_t o = j->start; o < j->end; o++)
        for (size_t t = 0; t < j->T; t++) j->y[t * j->out + o] = om_dot(j->x + t * j->in, j->w + o * j->in, j->in);
    return NULL;
}

OM_API void om_matmul_batch_w_f32(const float *x, const float *w, size_t out, size_t in, size_t T, float *y) {
    size_t nthreads = (size_t)num_threads();
    if (nthreads < 1) nthreads = 1;
    if (nthreads > out) nthreads = out;
    if (nthreads > 256) nthreads = 256;
    size_t chunk = (out + nthreads - 1) / nthreads;
    pthread_t th[256];
    gemm_f32_job jobs[256];
    size_t nt = 0;
    for (size_t s = 0; s < out && nt < 256; s += chunk, nt++) {
        jobs[nt] = (gemm_f32_job){x, w, y, out, in, T, s, s + chunk < out ? s + chunk : out};
        pthread_create(&th[nt], NULL, gemm_f32_worker, &jobs[nt]);
    }
    for (size_t i = 0; i < nt; i++) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* A7: prefill GEMM Y[T,out] = X[T,in] W^T (src/tensor.rs:573-858)           */
/* ------------------------------------------------------------------------ */

/* gemm_tile_avx2 (src/tensor.rs:799-858): 4-token x 2-row register tile of
 * k-major 8-lane FMA chains.  Per element the order equals dot_bf16, so the
 * result is bit-identical to dot_bf16(x_t, w_o) (src/tensor.rs:734-738). */
__attribute__((target("avx2,fma"))) static void gemm_tile_avx2(const float *x, const uint16_t *w, size_t out,
                                                                size_t in, size_t T, float *y, size_t r0,
                                                                size_t r1) {
    size_t kchunks = in / 8, ktail = in % 8;
    size_t o = r0;
    while (o + 1 < r1) {
        size_t tblock = T - (T % 4);
        for (size_t tb = 0; tb < tblock; tb += 4) {
            __m256 acc[4][2];
            for (int t = 0; t < 4; t++) acc[t][0] = acc[t][1] = _mm256_setzero_ps();
            for (size_t k = 0; k < kchunks; k++) {
                size_t ki = k * 8;
                __m256 w0 = _mm256_castsi256_ps(_mm256_slli_epi32(
                    _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(w + o * in + ki))), 16));
                __m256 w1 = _mm256_castsi256_ps(_mm256_slli_epi32(
                    _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(w + (o + 1) * in + ki))), 16));
                for (int t = 0; t < 4; t++) {
                    __m256 xv = _mm256_loadu_ps(x + (tb + t) * in + ki);
                    acc[t][0] = _mm256_fmadd_ps(xv, w0, acc[t][0]);
                    acc[t][1] = _mm256_fmadd_ps(xv, w1, acc[t][1]);
                }
            }
            for (int t = 0; t < 4; t++) {
                float s0 = reduce_add_avx(acc[t][0]);
                float s1 = reduce_add_avx(acc[t][1]);
                for (size_t k = kchunks * 8; k < kchunks * 8 + ktail; k++) {
                    float xk = x[(tb + t) * in + k];
                    s0 += xk * bf16_to_f32(w[o * in + k]);
                    s1 += xk * bf16_to_f32(w[(o + 1) * in + k]);
                }
                y[(tb + t) * out + o] = s0;
                y[(tb + t) * out + o + 1] = s1;
            }
        }
        for (size_t t = tblock; t < T; t++) {
            y[t * out + o] = dot_bf16_avx2(x + t * in, w + o * in, in);
            y[t * out + o + 1] = dot_bf16_avx2(x + t * in, w + (o + 1) * in, in);
        }
        o += 2;
    }
    if (o < r1)
        for (size_t t = 0; t < T; t++) y[t * out + o] = dot_bf16_avx2(x + t * in, w + o * in, in);
}

typedef struct {
    const float *x;
    const uint16_t *w;
    float *y;
    size_t out, in, T, r0, r1;
} gemm_job;

static void *gemm_worker(void *p) {
    gemm_job *j = (gemm_job *)p;
    if (has_avx2_fma()) {
        gemm_tile_avx2(j->x, j->w, j->out, j->in, j->T, j->y, j->r0, j->r1);
    } else {
        for (size_t o = j->r0; o < j->r1; o++)
            for (size_t t = 0; t < j->T; t++)
                j->y[t * j->out + o] = dot_bf16_scalar8(j->x + t * j->in, j->w + o * j->in, j->in);
    }
    return NULL;
}

/* matmul_batch_w_into: T >= 2 takes the tiled path with 8-row jobs statically
 * split over all cores (src/tensor.rs:741-792); T == 1 takes the per-row dot
 * path (src/tensor.rs:590-637).  Both give dot_bf16 per element. */
OM_API void om_matmul_batch_w(const float *x, const uint16_t *w, size_t out, size_t in, size_t T, float *y) {
    if (T < 2) {
        for (size_t o = 0; o < out; o++)
            for (size_t t = 0; t < T; t++) y[t * out + o] = om_dot_bf16(x + t * in, w + o * in, in);
        return;
    }
    size_t rowblock = 8, njobs = (out + rowblock - 1) / rowblock;
    size_t nthreads = (size_t)num_threads();
    if (nthreads > njobs) nthreads = njobs;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if (nthreads <= 1) {
        gemm_job j = {x, w, y, out, in, T, 0, out};
        gemm_worker(&j);
        return;
    }
    size_t base = njobs / nthreads, extra = njobs % nthreads, js = 0, nt = 0;
    pthread_t th[256];
    gemm_job jobs[256];
    for (size_t ti = 0; ti < nthreads; ti++) {
        size_t nj = base + (ti < extra ? 1 : 0);
        if (nj == 0) break;
        size_t r0 = js * rowblock, r1 = (js + nj) * rowblock;
        if (r1 > out) r1 = out;
        js += nj;
        jobs[nt] = (gemm_job){x, w, y, out, in, T, r0, r1};
        pthread_create(&th[nt], NULL, gemm_worker, &jobs[nt]);
        nt++;
    }
    for (size_t i = 0; i < nt; i++) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* int8 weight-only mode, TMG_I8=1 (src/model.rs:57-76; src/tensor.rs:125-170, */
/* 275-293, 341-386, 795-945)                                                */
/* ------------------------------------------------------------------------ */

/* `v as i8` of a value already clamped to [-127, 127]: Rust's float-to-int
 * cast maps NaN to 0. */
static inline int8_t i8_of(float r) {
    if (r != r) return 0;
    return (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
}

/* WMat::quantize_i8 (src/tensor.rs:275-293): per row, scale = max|w| / 127
 * (1.0 for an all-zero row) and q = round(w / scale) clamped to [-127, 127].
 * f32::round rounds half away from zero, as roundf does; the max folds from
 * 0 with f32::max, which skips NaN like fmaxf. */
OM_API void om_quantize_i8(const float *w, size_t out, size_t in, int8_t *q, float *s) {
    for (size_t o = 0; o < out; o++) {
        const float *row = w + o * in;
        float maxabs = 0.0f;
        for (size_t i = 0; i < in; i++) maxabs = fmaxf(fabsf(row[i]), maxabs);
        const float scale = maxabs > 0.0f ? maxabs / 127.0f : 1.0f;
        s[o] = scale;
        for (size_t i = 0; i < in; i++) q[o * in + i] = i8_of(roundf(row[i] / scale));
    }
}

/* quantize_row_i8 (src/tensor.rs:125-139): one symmetric scale for the
 * activation vector; an all-zero vector gives zeros and scale 0.  Returns the
 * scale. */
OM_API float om_quantize_row_i8(const float *x, size_t n, int8_t *q) {
    float maxabs = 0.0f;
    for (size_t i = 0; i < n; i++) maxabs = fmaxf(fabsf(x[i]), maxabs);
    if (maxabs == 0.0f) {
        memset(q, 0, n);
        return 0.0f;
    }
    const float s = maxabs / 127.0f;
    const float inv = 1.0f / s;
    for (size_t i = 0; i < n; i++) q[i] = i8_of(roundf(x[i] * inv));
    return s;
}

/* dot_i8 (src/tensor.rs:144-170): exact integer dot; the AVX2 kernel's i16
 * pairwise madd and i32 lane sums only reorder integer additions, which wrap
 * modulo 2^32 in a release build. */
OM_API int32_t om_dot_i8(const int8_t *a, const int8_t *b, size_t n) {
    uint32_t acc = 0;
    for (size_t i = 0; i < n; i++) acc += (uint32_t)((int32_t)a[i] * (int32_t)b[i]);
    return (int32_t)acc;
}

typedef struct {
    const int8_t *xq, *q;
    const float *s;
    float xs, *y;
    size_t in, start, end;
} gemv_i8_job;

static void *gemv_i8_worker(void *p) {
    gemv_i8_job *j = (gemv_i8_job *)p;
    for (size_t o = j->start; o < j->end; o++)
        j->y[o] = (float)om_dot_i8(j->xq, j->q + o * j->in, j->in) * j->xs * j->s[o];
    return NULL;
}

/* matmul_w_into for WMat::I8 on an AVX2 host (src/tensor.rs:341-374): the
 * activation is quantized once, then y[o] = (dot as f32) * xs * scale[o],
 * multiplied left to right, rows split over max(1, ncores/4) threads in
 * ceil(out/nthreads) chunks (one thread below 64 rows).  (A host without AVX2
 * takes a dequantizing scalar loop instead, src/tensor.rs:376-385; the
 * reference's benchmarks and this restatement use the AVX2 path.) */
OM_API void om_matmul_w_i8(const float *x, const int8_t *q, const float *s, size_t out, size_t in, float *y) {
    int8_t *xq = (int8_t *)malloc(in ? in : 1);
    const float xs = om_quantize_row_i8(x, in, xq);
    size_t nthreads = (size_t)num_threads() / 4;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > out) nthreads = out;
    if (nthreads <= 1 || out < 64) {
        gemv_i8_job j = {xq, q, s, xs, y, in, 0, out};
        gemv_i8_worker(&j);
    } else {
        size_t chunk = (out + nthreads - 1) / nthreads;
        pthread_t th[256];
        gemv_i8_job jobs[256];
        size_t nt = 0;
        for (size_t st = 0; st < out && nt < 256; st += chunk, nt++) {
            jobs[nt] = (gemv_i8_job){xq, q, s, xs, y, in, st, st + chunk < out ? st + chunk : out};
            pthread_create(&th[nt], NULL, gemv_i8_worker, &jobs[nt]);
        }
        for (size_t i = 0; i < nt; i++) pthread_join(th[i], NULL);
    }
    free(xq);
}

/* Dequantizing dot of the scalar paths (dot_w_row_avx2's I8 arm,
 * src/tensor.rs:876-883, and the T == 1 loop, src/tensor.rs:622-633):
 * acc += x * (q as f32) in sequence, no FMA; then acc * scale. */
static float dot_deq_i8(const float *x, const int8_t *q, float scale, size_t in) {
    float acc = 0.0f;
    for (size_t k = 0; k < in; k++) acc += x[k] * (float)q[k];
    return acc * scale;
}

/* gemm_tile_avx2 over WMat::I8 (src/tensor.rs:799-858): the BF16 tile with
 * the weight lanes widened from int8 (load_w_m256, src/tensor.rs:916-921),
 * written as eight explicit FMA lanes (identical to the AVX2 FMAs), the row
 * scale applied at write-back.  In the k tail (in % 8 != 0) the reference
 * adds x * wf_elem = x * (q * scale) and then multiplies by the scale again
 * (src/tensor.rs:833-840, 940); that is restated as is.  Token tails and an
 * odd last row use the dequantizing scalar dot. */
static void gemm_tile_i8(const float *x, const int8_t *q, const float *s, size_t out, size_t in, size_t T, float *y,
                         size_t r0, size_t r1) {
    const size_t kchunks = in / 8, ktail = in % 8;
    size_t o = r0;
    while (o + 1 < r1) {
        const size_t tblock = T - (T % 4);
        for (size_t tb = 0; tb < tblock; tb += 4) {
            float acc[4][2][8];
            memset(acc, 0, sizeof(acc));
            for (size_t kc = 0; kc < kchunks; kc++) {
                const size_t ki = kc * 8;
                for (int t = 0; t < 4; t++)
                    for (int l = 0; l < 8; l++) {
                        const float xv = x[(tb + t) * in + ki + l];
                        acc[t][0][l] = fmaf(xv, (float)q[o * in + ki + l], acc[t][0][l]);
                        acc[t][1][l] = fmaf(xv, (float)q[(o + 1) * in + ki + l], acc[t][1][l]);
                    }
            }
            for (int t = 0; t < 4; t++) {
                float s0 = reduce8(acc[t][0]), s1 = reduce8(acc[t][1]);
                for (size_t k = kchunks * 8; k < kchunks * 8 + ktail; k++) {
                    const float xk = x[(tb + t) * in + k];
                    s0 += xk * ((float)q[o * in + k] * s[o]);
                    s1 += xk * ((float)q[(o + 1) * in + k] * s[o + 1]);
                }
                y[(tb + t) * out + o] = s0 * s[o];
                y[(tb + t) * out + o + 1] = s1 * s[o + 1];
            }
        }
        for (size_t t = tblock; t < T; t++) {
            y[t * out + o] = dot_deq_i8(x + t * in, q + o * in, s[o], in);
            y[t * out + o + 1] = dot_deq_i8(x + t * in, q + (o + 1) * in, s[o + 1], in);
        }
        o += 2;
    }
    if (o < r1)
        for (size_t t = 0; t < T; t++) y[t * out + o] = dot_deq_i8(x + t * in, q + o * in, s[o], in);
}

typedef struct {
    const float *x;
    const int8_t *q;
    const float *s;
    float *y;
    size_t out, in, T, r0, r1;
} gemm_i8_job;

static void *gemm_i8_worker(void *p) {
    gemm_i8_job *j = (gemm_i8_job *)p;
    gemm_tile_i8(j->x, j->q, j->s, j->out, j->in, j->T, j->y, j->r0, j->r1);
    return NULL;
}

/* matmul_batch_w_into for WMat::I8: T >= 2 takes the tile above in 8-row
 * jobs over all cores (src/tensor.rs:741-792); T == 1 the dequantizing loop
 * (src/tensor.rs:622-633; with several threads and out >= 64 the reference
 * reaches unreachable!() at src/tensor.rs:641 instead -- a one-token prompt
 * in int8 mode -- and this restates the single-thread result). */
OM_API void om_matmul_batch_w_i8(const float *x, const int8_t *q, const float *s, size_t out, size_t in, size_t T,
                                 float *y) {
    if (T < 2) {
        for (size_t o = 0; o < out; o++)
            for (size_t t = 0; t < T; t++) y[t * out + o] = dot_deq_i8(x + t * in, q + o * in, s[o], in);
        return;
    }
    size_t rowblock = 8, njobs = (out + rowblock - 1) / rowblock;
    size_t nthreads = (size_t)num_threads();
    if (nthreads > njobs) nthreads = njobs;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    size_t base = njobs / nthreads, extra = njobs % nthreads, js = 0, nt = 0;
    pthread_t th[256];
    gemm_i8_job jobs[256];
    for (size_t ti = 0; ti < nthreads; ti++) {
        size_t nj = base + (ti < extra ? 1 : 0);
        if (nj == 0) break;
        size_t r0 = js * rowblock, r1 = (js + nj) * rowblock;
        if (r1 > out) r1 = out;
        js += nj;
        jobs[nt] = (gemm_i8_job){x, q, s, y, out, in, T, r0, r1};
        pthread_create(&th[nt], NULL, gemm_i8_worker, &jobs[nt]);
        nt++;
    }
    for (size_t i = 0; i < nt; i++) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* A8: RMSNorm (src/tensor.rs:946-977)                                       */
/* ------------------------------------------------------------------------ */

/* rms_norm_into: ss sequential (no FMA), inv = 1/sqrt(ss/n + eps),
 * out = (v*inv)*w. */
OM_API void om_rms_norm(const float *x, const float *w, float eps, size_t n, float *out) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float mean = ss / (float)n;
    float inv = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* rms_norm_batch: same sum, but the row is scaled as v*(inv*w). */
OM_API void om_rms_norm_batch(float *x, const float *w, float eps, size_t n, size_t rows) {
    for (size_t r = 0; r < rows; r++) {
        float *row = x + r * n;
        float ss = 0.0f;
        for (size_t i = 0; i < n; i++) ss += row[i] * row[i];
        float inv = 1.0f / sqrtf(ss / (float)n + eps);
        for (size_t i = 0; i < n; i++) row[i] *= inv * w[i];
    }
}

/* ------------------------------------------------------------------------ */
/* A9: RoPE, rotate_half layout (src/tensor.rs:983-1038)                     */
/* ------------------------------------------------------------------------ */

/* rope_rotate (src/tensor.rs:983-994): per-call powf; test helper. */
OM_API void om_rope_rotate(float *v, size_t d, size_t pos, float theta) {
    size_t half = d / 2;
    for (size_t i = 0; i < half; i++) {
        float freq = powf(theta, 2.0f * (float)i / (float)d);
        float angle = (float)pos * (1.0f / freq);
        float s = sinf(angle), c = cosf(angle);
        float a = v[i], b = v[i + half];
        v[i] = a * c - b * s;
        v[i + half] = a * s + b * c;
    }
}

typedef struct {
    float *inv_freq;
    float *cos, *sin;
    size_t half, npos, cap;
} om_rope;

static void rope_init(om_rope *r, size_t head_dim, float theta) {
    r->half = head_dim / 2;
    r->inv_freq = (float *)malloc(sizeof(float) * (r->half ? r->half : 1));
    /* Rope::new: inv_freq[i] = (theta^(2i/hd)).recip() (src/tensor.rs:1005-1011) */
    for (size_t i = 0; i < r->half; i++) r->inv_freq[i] = 1.0f / powf(theta, 2.0f * (float)i / (float)head_dim);
    r->cos = r->sin = NULL;
    r->npos = r->cap = 0;
}

/* Rope::ensure (src/tensor.rs:1014-1023): tables grow one position at a time;
 * angle = pos as f32 * inv_freq[i]; (sin, cos) = angle.sin_cos(). */
static void rope_ensure(om_rope *r, size_t pos) {
    while (r->npos <= pos) {
        if (r->npos == r->cap) {
            r->cap = r->cap ? r->cap * 2 : 64;
            r->cos = (float *)realloc(r->cos, sizeof(float) * r->cap * r->half);
            r->sin = (float *)realloc(r->sin, sizeof(float) * r->cap * r->half);
        }
        size_t p = r->npos;
        for (size_t i = 0; i < r->half; i++) {
            float ang = (float)p * r->inv_freq[i];
            r->sin[p * r->half + i] = sinf(ang);
            r->cos[p * r->half + i] = cosf(ang);
        }
        r->npos++;
    }
}

/* Rope::rotate (src/tensor.rs:1026-1037). */
static void rope_rotate_tab(om_rope *r, float *v, size_t pos) {
    rope_ensure(r, pos);
    const float *c = r->cos + pos * r->half, *s = r->sin + pos * r->half;
    for (size_t i = 0; i < r->half; i++) {
        float a = v[i], b = v[i + r->half];
        v[i] = a * c[i] - b * s[i];
        v[i + r->half] = a * s[i] + b * c[i];
    }
}

static void rope_free(om_rope *r) {
    free(r->inv_freq);
    free(r->cos);
    free(r->sin);
}

/* The cos/sin table for positions [0, npos): exported so tests can compare
 * the product's host-built table with this one. */
OM_API void om_rope_table(size_t head_dim, float theta, size_t npos, float *cos_out, float *sin_out) {
    om_rope r;
    rope_init(&r, head_dim, theta);
    if (npos) rope_ensure(&r, npos - 1);
    memcpy(cos_out, r.cos, sizeof(float) * npos * r.half);
    memcpy(sin_out, r.sin, sizeof(float) * npos * r.half);
    rope_free(&r);
}

/* ------------------------------------------------------------------------ */
/* softmax, silu, argmax (src/tensor.rs:1043-1073)                           */
/* ------------------------------------------------------------------------ */

/* softmax: max fold with f32::max, exps = (v-max).exp(), sequential sum,
 * e/sum (src/tensor.rs:1055-1060).  f32::max ignores NaN operands. */
OM_API void om_softmax(const float *x, size_t n, float *out) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) m = fmaxf(m, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        out[i] = expf(x[i] - m);
        sum += out[i];
    }
    for (size_t i = 0; i < n; i++) out[i] = out[i] / sum;
}

/* silu: x/(1+exp(-x)) (src/tensor.rs:1043-1045). */
OM_API void om_silu(const float *x, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = x[i] / (1.0f + expf(-x[i]));
}

/* argmax: first strict maximum; all -inf/NaN returns 0 (src/tensor.rs:1063-1073). */
OM_API size_t om_argmax(const float *x, size_t n) {
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    return best;
}

/* ------------------------------------------------------------------------ */
/* A11: attention                                                            */
/* ------------------------------------------------------------------------ */

/* attention_row (src/tensor.rs:1079-1093): plain sequential dot (no 8-lane
 * order: the iterator sum), softmax, out += p*v. */
OM_API void om_attention_row(const float *q, const float *keys, const float *values, size_t n_keys, size_t d,
                             size_t mask_len, float scale, float *out) {
    size_t n = mask_len < n_keys ? mask_len : n_keys;
    float *scores = (float *)malloc(sizeof(float) * (n ? n : 1));
    float *probs = (float *)malloc(sizeof(float) * (n ? n : 1));
    for (size_t t = 0; t < n; t++) {
        float s = 0.0f;
        for (size_t i = 0; i < d; i++) s += q[i] * keys[t * d + i];
        scores[t] = s * scale;
    }
    om_softmax(scores, n, probs);
    for (size_t i = 0; i < d; i++) out[i] = 0.0f;
    for (size_t t = 0; t < n; t++)
        for (size_t i = 0; i < d; i++) out[i] += probs[t] * values[t * d + i];
    free(scores);
    free(probs);
}

/* One (query row, head) of causal attention over cache rows [0, n_ctx):
 * scores via the 8-lane dot, then softmax, then o += p*v sequentially.  This
 * is the body shared by the decode path (src/model.rs:441-459) and
 * attention_batch (src/tensor.rs:1116-1136). */
static void attn_head(const float *q, const float *keys, const float *vals, size_t kv_dim, size_t s, size_t hd,
                      size_t n_ctx, float scale, float *o, float *scores) {
    for (size_t t = 0; t < n_ctx; t++) scores[t] = om_dot(q, keys + t * kv_dim + s, hd) * scale;
    om_softmax(scores, n_ctx, scores);
    for (size_t i = 0; i < hd; i++) o[i] = 0.0f;
    for (size_t t = 0; t < n_ctx; t++) {
        const float *v = vals + t * kv_dim + s;
        float p = scores[t];
        for (size_t i = 0; i < hd; i++) o[i] += p * v[i];
    }
}

typedef struct {
    const float *q;
    const float *keys, *vals;
    float *out;
    size_t T, nq, nkv, hd, start_pos;
    size_t job0, job1; /* jobs index (token, head) pairs */
} attn_job;

static void *attn_worker(void *p) {
    attn_job *j = (attn_job *)p;
    size_t group = j->nq / j->nkv, kv_dim = j->nkv * j->hd;
    float scale = 1.0f / sqrtf((float)j->hd);
    float *scores = (float *)malloc(sizeof(float) * (j->start_pos + j->T + 1));
    for (size_t job = j->job0; job < j->job1; job++) {
        size_t ti = job / j->nq, h = job % j->nq;
        size_t s = (h / group) * j->hd;
        const float *q = j->q + ti * j->nq * j->hd + h * j->hd;
        float *o = j->out + ti * j->nq * j->hd + h * j->hd;
        attn_head(q, j->keys, j->vals, kv_dim, s, j->hd, j->start_pos + ti + 1, scale, o, scores);
    }
    free(scores);
    return NULL;
}

/* attention_batch (src/tensor.rs:1099-1139): causal, token ti attends to
 * positions [0, start_pos+ti]. */
OM_API void om_attention_batch(const float *q, const float *keys, const float *vals, size_t T, size_t nq,
                               size_t nkv, size_t hd, size_t start_pos, float *out) {
    size_t njobs = T * nq;
    size_t nt = (size_t)g_attn_threads;
    if (nt > njobs) nt = njobs;
    if (nt <= 1) {
        attn_job j = {q, keys, vals, out, T, nq, nkv, hd, start_pos, 0, njobs};
        attn_worker(&j);
        return;
    }
    if (nt > 256) nt = 256;
    pthread_t th[256];
    attn_job jobs[256];
    size_t per = (njobs + nt - 1) / nt, n = 0;
    for (size_t s = 0; s < njobs; s += per, n++) {
        jobs[n] = (attn_job){q, keys, vals, out, T, nq, nkv, hd, start_pos, s, s + per < njobs ? s + per : njobs};
        pthread_create(&th[n], NULL, attn_worker, &jobs[n]);
    }
    for (size_t i = 0; i < n; i++) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* A16/A17: repetition penalty and sampling (src/tensor.rs:1142-1213)        */
/* ------------------------------------------------------------------------ */

/* apply_repetition_penalty over the SET of generated ids: l>0 -> l/p,
 * else l*p; penalty 1.0 is a no-op (src/tensor.rs:1142-1154). */
OM_API void om_apply_repetition_penalty(float *logits, size_t V, const uint32_t *gen, size_t n_gen,
                                        float penalty) {
    if (penalty == 1.0f) return;
    unsigned char *seen = (unsigned char *)calloc(V, 1);
    for (size_t i = 0; i < n_gen; i++) {
        uint32_t t = gen[i];
        if (t < V && !seen[t]) {
            seen[t] = 1;
            float l = logits[t];
            logits[t] = l > 0.0f ? l / penalty : l * penalty;
        }
    }
    free(seen);
}

static const float *g_sort_keys;
/* descending by key; ties by ascending index.  The reference uses
 * sort_unstable_by, which leaves the order of equal keys unspecified; ties
 * are broken here by index so the oracle is deterministic. */
static int cmp_desc(const void *a, const void *b) {
    size_t ia = *(const size_t *)a, ib = *(const size_t *)b;
    float ka = g_sort_keys[ia], kb = g_sort_keys[ib];
    if (ka > kb) return -1;
    if (ka < kb) return 1;
    return ia < ib ? -1 : (ia > ib ? 1 : 0);
}

/* ---- the reference's RNG: StdRng::seed_from_u64 + StandardUniform f32 ----
 * generate (src/model.rs:629) makes StdRng::seed_from_u64(params.seed) and
 * sample (src/tensor.rs:1204) draws one StandardUniform f32 per sampled
 * step.  Those live in the crates rand 0.10.2, rand_core 0.10.1 and
 * chacha20 0.10.2 (Cargo.lock:744-752, :774-777, :140-143), whose sources
 * are not in the reference tree; this restates their published algorithms:
 *   - seed_from_u64 (rand_core): the 32-byte seed is eight outputs of a
 *     PCG32 stream, each little-endian -- per output the 64-bit state first
 *     advances (state * 6364136223846793005 + 11634580027462260723), then the
 *     XSH-RR output function of the new state;
 *   - StdRng = ChaCha12Rng (chacha20): key = the seed, 64-bit block counter
 *     from 0 in words 12-13, stream 0 in words 14-15, 12 rounds; next_u32
 *     returns the blocks' 16 words in order;
 *   - StandardUniform f32 (rand): (next_u32 >> 8) * 2^-24.
 * The ChaCha block function is pinned by the RFC 7539 vectors at 20 rounds
 * and by the all-zero key and IV vectors of the ChaCha test-vector draft
 * (draft-strombergson-chacha-test-vectors-00, TC1) at 8 and 12 rounds, the
 * XSH-RR output function by the PCG reference demo sequence, and the three
 * crate-specific steps by the crates' own value-stability vectors: the seed
 * expansion by rand_core's test_seed_from_u64 (seed 0 -> 5029875928683246316),
 * StdRng's key layout, counter, stream and word order by rand's
 * test_stdrng_construction (rngs/std.rs), and the f32 conversion by rand's
 * StandardUniform f32 value_stability test (distr/float.rs). */

static uint32_t om_rotl32(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

#define OM_QR(a, b, c, d)                   \
    do {                                    \
        x[a] += x[b]; x[d] = om_rotl32(x[d] ^ x[a], 16); \
        x[c] += x[d]; x[b] = om_rotl32(x[b] ^ x[c], 12); \
        x[a] += x[b]; x[d] = om_rotl32(x[d] ^ x[a], 8);  \
        x[c] += x[d]; x[b] = om_rotl32(x[b] ^ x[c], 7);  \
    } while (0)

/* One ChaCha block: constants, key[8], counter (words 12-13), stream
 * (words 14-15); `rounds` even. */
OM_API void om_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds,
                            uint32_t out[16]) {
    uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
    for (int i = 0; i < 8; i++) s[4 + i] = key[i];
    s[12] = (uint32_t)counter;
    s[13] = (uint32_t)(counter >> 32);
    s[14] = (uint32_t)stream;
    s[15] = (uint32_t)(stream >> 32);
    uint32_t x[16];
    memcpy(x, s, sizeof(x));
    for (int r = 0; r < rounds; r += 2) {
        OM_QR(0, 4, 8, 12); OM_QR(1, 5, 9, 13); OM_QR(2, 6, 10, 14); OM_QR(3, 7, 11, 15);
        OM_QR(0, 5, 10, 15); OM_QR(1, 6, 11, 12); OM_QR(2, 7, 8, 13); OM_QR(3, 4, 9, 14);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

/* PCG XSH-RR output function of a 64-bit state. */
OM_API uint32_t om_pcg_xsh_rr(uint64_t state) {
    const uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    const unsigned rot = (unsigned)(state >> 59);
    return (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
}

/* seed_from_u64: the eight key words. */
OM_API void om_stdrng_key(uint64_t seed, uint32_t key[8]) {
    uint64_t state = seed;
    for (int i = 0; i < 8; i++) {
        state = state * 6364136223846793005ull + 11634580027462260723ull;
        key[i] = om_pcg_xsh_rr(state);
    }
}

/* StandardUniform f32 of one next_u32 word: its top 24 bits times 2^-24
 * (exact), so the draws lie in [0, 1). */
OM_API float om_uniform_f32(uint32_t word) { return (float)(word >> 8) * (1.0f / 16777216.0f); }

/* The first n StandardUniform f32 draws of StdRng::seed_from_u64(seed). */
OM_API void om_stdrng_uniform(uint64_t seed, size_t n, float *out) {
    uint32_t key[8], blk[16];
    om_stdrng_key(seed, key);
    for (size_t j = 0; j < n; j++) {
        if (j % 16 == 0) om_chacha_block(key, (uint64_t)(j / 16), 0, 12, blk);
        out[j] = om_uniform_f32(blk[j % 16]);
    }
}


/* sample (src/tensor.rs:1157-1213) with the uniform draw r supplied by the
 * caller (the reference draws it from rand's StdRng, which cannot run here).
 * Optional outputs: the candidate ids in walk order (cand_ids, n_cand) and
 * their final probabilities (cand_probs). Returns the chosen id. */
OM_API size_t om_sample(const float *logits, size_t V, float temperature, size_t top_k, float top_p, float r,
                        uint32_t *cand_ids, float *cand_probs, size_t *n_cand) {
    if (temperature <= 0.0f) {
        size_t a = om_argmax(logits, V);
        if (n_cand) *n_cand = 0;
        return a;
    }
    float *scaled = (float *)malloc(sizeof(float) * V);
    size_t *idx = (size_t *)malloc(sizeof(size_t) * V);
    for (size_t i = 0; i < V; i++) {
        scaled[i] = logits[i] / temperature;
        idx[i] = i;
    }
    size_t n = V;
    if (top_k > 0 && top_k < n) {
        g_sort_keys = scaled;
        qsort(idx, n, sizeof(size_t), cmp_desc);
        n = top_k;
    }
    float *cand = (float *)malloc(sizeof(float) * n);
    float *probs = (float *)malloc(sizeof(float) * n);
    for (size_t i = 0; i < n; i++) cand[i] = scaled[idx[i]];
    om_softmax(cand, n, probs);
    if (top_p < 1.0f) {
        size_t *order = (size_t *)malloc(sizeof(size_t) * n);
        for (size_t i = 0; i < n; i++) order[i] = i;
        g_sort_keys = probs;
        qsort(order, n, sizeof(size_t), cmp_desc);
        float cum = 0.0f;
        size_t cutoff = n;
        for (size_t rank = 0; rank < n; rank++) {
            cum += probs[order[rank]];
            if (cum > top_p) {
                cutoff = rank + 1;
                break;
            }
        }
        float sum = 0.0f;
        for (size_t k = 0; k < cutoff; k++) sum += probs[order[k]];
        float *np = (float *)calloc(n, sizeof(float));
        for (size_t k = 0; k < cutoff; k++) np[order[k]] = probs[order[k]] / sum;
        memcpy(probs, np, sizeof(float) * n);
        free(np);
        free(order);
    }
    size_t chosen = (size_t)-1;
    float cum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        cum += probs[i];
        if (r < cum) {
            chosen = idx[i];
            break;
        }
    }
    if (chosen == (size_t)-1) {
        size_t first = 0;
        for (size_t i = 0; i < n; i++)
            if (probs[i] > 0.0f) {
                first = i;
                break;
            }
        chosen = idx[first];
    }
    if (n_cand) *n_cand = n;
    if (cand_ids)
        for (size_t i = 0; i < n; i++) cand_ids[i] = (uint32_t)idx[i];
    if (cand_probs) memcpy(cand_probs, probs, sizeof(float) * n);
    free(scaled);
    free(idx);
    free(cand);
    free(probs);
    return chosen;
}

/* ------------------------------------------------------------------------ */
/* A2/A3/A10: the model, KV cache, forward_token, forward_seq                */
/* ------------------------------------------------------------------------ */

typedef struct {
    int hidden, layers, n_heads, n_kv, head_dim, inter, vocab;
    float eps, theta;
    /* weights: raw BF16 [out,in] pointers per layer (owned by the caller) */
    const uint16_t **wq, **wk, **wv, **wo, **wg, **wu, **wd;
    const float **in_norm, **post_norm;
    const float *final_norm;
    const float *embed;    /* [V,H] f32, the reference converts at load */
    const uint16_t *lm_bf16; /* [V,H] BF16, or NULL when tied */
    /* int8 mode (TMG_I8=1, src/model.rs:57-76, 212-218): per-layer int8 rows
     * and row scales of q, k, v, o, gate, up, down, in that order; all NULL in
     * BF16 mode.  lm_head, norms and the embedding stay as above. */
    const int8_t **q8[7];
    const float **s8[7];
    /* WMat::F32 matrices (src/model.rs:49-55: F32 or F16 tensors converted
     * at load): per-layer f32 [out,in] rows of q, k, v, o, gate, up, down;
     * a NULL table, or a NULL entry, means that layer's matrix is BF16 */
    const float **wf[7];
    const float *lm_f32; /* untied f32 lm_head [V,H], or NULL */
} om_weights;

enum { W_Q, W_K, W_V, W_O, W_G, W_U, W_D };

static const uint16_t *w_bf16(const om_weights *w, int which, int l) {
    const uint16_t **t[7] = {w->wq, w->wk, w->wv, w->wo, w->wg, w->wu, w->wd};
    return t[which][l];
}

static const float *w_f32(const om_weights *w, int which, int l) { return w->wf[which] ? w->wf[which][l] : NULL; }

/* matmul_w_into / matmul_batch_w_into dispatch on the WMat variant. */
static void lin(const om_weights *w, int which, int l, const float *x, size_t out, size_t in, float *y) {
    if (w->q8[which])
        om_matmul_w_i8(x, w->q8[which][l], w->s8[which][l], out, in, y);
    else if (w_f32(w, which, l))
        om_matmul_w_f32(x, w_f32(w, which, l), out, in, y);
    else
        om_matmul_w(x, w_bf16(w, which, l), out, in, y);
}

static void lin_batch(const om_weights *w, int which, int l, const float *x, size_t out, size_t in, size_t T,
                      float *y) {
    if (w->q8[which])
        om_matmul_batch_w_i8(x, w->q8[which][l], w->s8[which][l], out, in, T, y);
    else if (w_f32(w, which, l))
        om_matmul_batch_w_f32(x, w_f32(w, which, l), out, in, T, y);
    else
        om_matmul_batch_w(x, w_bf16(w, which, l), out, in, T, y);
}

typedef struct {
    om_weights w;
    om_rope rope;
    /* scratch (src/model.rs:349-381) */
    float *x, *attn_in, *q, *k, *v, *attn_out, *proj, *mlp_in, *gate, *up, *down, *scores;
    size_t scores_cap;
} om_model;

typedef struct {
    int layers;
    size_t kv_dim;
    float **keys, **vals;
    size_t *lens, *caps;
} om_cache;

OM_API om_model *om_model_new(const om_weights *w) {
    om_model *m = (om_model *)calloc(1, sizeof(om_model));
    m->w = *w;
    size_t L = (size_t)w->layers;
    const void ***fields[] = {(const void ***)&m->w.wq, (const void ***)&m->w.wk, (const void ***)&m->w.wv,
                              (const void ***)&m->w.wo, (const void ***)&m->w.wg, (const void ***)&m->w.wu,
                              (const void ***)&m->w.wd, (const void ***)&m->w.in_norm,
                              (const void ***)&m->w.post_norm};
    for (size_t f = 0; f < sizeof(fields) / sizeof(fields[0]); f++) {
        const void **copy = (const void **)malloc(sizeof(void *) * L);
        memcpy(copy, *fields[f], sizeof(void *) * L);
        *fields[f] = copy;
    }
    for (int f = 0; f < 7; f++) {
        if (!w->q8[f]) continue;
        const int8_t **qc = (const int8_t **)malloc(sizeof(void *) * L);
        const float **sc = (const float **)malloc(sizeof(void *) * L);
        memcpy(qc, w->q8[f], sizeof(void *) * L);
        memcpy(sc, w->s8[f], sizeof(void *) * L);
        m->w.q8[f] = qc;
        m->w.s8[f] = sc;
    }
    rope_init(&m->rope, (size_t)w->head_dim, w->theta);
    size_t H = w->hidden, qd = (size_t)w->n_heads * w->head_dim, kvd = (size_t)w->n_kv * w->head_dim;
    size_t I = w->inter;
    m->x = calloc(H, 4);
    m->attn_in = calloc(H, 4);
    m->q = calloc(qd, 4);
    m->k = calloc(kvd, 4);
    m->v = calloc(kvd, 4);
    m->attn_out = calloc(qd, 4);
    m->proj = calloc(H, 4);
    m->mlp_in = calloc(H, 4);
    m->gate = calloc(I, 4);
    m->up = calloc(I, 4);
    m->down = calloc(H, 4);
    return m;
}

OM_API void om_model_free(om_model *m) {
    if (!m) return;
    free((void *)m->w.wq);
    free((void *)m->w.wk);
    free((void *)m->w.wv);
    free((void *)m->w.wo);
    free((void *)m->w.wg);
    free((void *)m->w.wu);
    free((void *)m->w.wd);
    free((void *)m->w.in_norm);
    free((void *)m->w.post_norm);
    for (int f = 0; f < 7; f++) {
        free((void *)m->w.q8[f]);
        free((void *)m->w.s8[f]);
    }
    rope_free(&m->rope);
    free(m->x);
    free(m->attn_in);
    free(m->q);
    free(m->k);
    free(m->v);
    free(m->attn_out);
    free(m->proj);
    free(m->mlp_in);
    free(m->gate);
    free(m->up);
    free(m->down);
    free(m->scores);
    free(m);
}

/* KvCache::new + set_kv_dim (src/model.rs:262-276). */
OM_API om_cache *om_cache_new(int layers, size_t kv_dim) {
    om_cache *c = (om_cache *)calloc(1, sizeof(om_cache));
    c->layers = layers;
    c->kv_dim = kv_dim;
    c->keys = (float **)calloc(layers, sizeof(float *));
    c->vals = (float **)calloc(layers, sizeof(float *));
    c->lens = (size_t *)calloc(layers, sizeof(size_t));
    c->caps = (size_t *)calloc(layers, sizeof(size_t));
    return c;
}

OM_API void om_cache_free(om_cache *c) {
    if (!c) return;
    for (int l = 0; l < c->layers; l++) {
        free(c->keys[l]);
        free(c->vals[l]);
    }
    free(c->keys);
    free(c->vals);
    free(c->lens);
    free(c->caps);
    free(c);
}

OM_API size_t om_cache_len(const om_cache *c, int layer) { return c->lens[layer]; }
OM_API const float *om_cache_keys(const om_cache *c, int layer) { return c->keys[layer]; }
OM_API const float *om_cache_values(const om_cache *c, int layer) { return c->vals[layer]; }

/* KvCache::reset (src/model.rs:324-331). */
OM_API void om_cache_reset(om_cache *c) {
    for (int l = 0; l < c->layers; l++) c->lens[l] = 0;
}

/* KvCache::push (src/model.rs:288-293): append one [kv_dim] row. */
OM_API void om_cache_push(om_cache *c, int layer, const float *k, const float *v) {
    if (c->lens[layer] == c->caps[layer]) {
        size_t cap = c->caps[layer] ? c->caps[layer] * 2 : 64;
        c->keys[layer] = (float *)realloc(c->keys[layer], sizeof(float) * cap * c->kv_dim);
        c->vals[layer] = (float *)realloc(c->vals[layer], sizeof(float) * cap * c->kv_dim);
        c->caps[layer] = cap;
    }
    memcpy(c->keys[layer] + c->lens[layer] * c->kv_dim, k, sizeof(float) * c->kv_dim);
    memcpy(c->vals[layer] + c->lens[layer] * c->kv_dim, v, sizeof(float) * c->kv_dim);
    c->lens[layer]++;
}

static void lm_head(const om_model *m, const float *x, float *logits) {
    const om_weights *w = &m->w;
    if (w->lm_bf16) {
        om_matmul_w(x, w->lm_bf16, (size_t)w->vocab, (size_t)w->hidden, logits);
    } else if (w->lm_f32) {
        om_matmul_w_f32(x, w->lm_f32, (size_t)w->vocab, (size_t)w->hidden, logits);
    } else {
        /* tied: WMat::F32(embed) (src/model.rs:230-233) -> matmul_w_into's f32
         * dot path, threaded the same way as the BF16 path. */
        size_t V = w->vocab, H = w->hidden;
        for (size_t o = 0; o < V; o++) logits[o] = om_dot(x, w->embed + o * H, H);
    }
}

/* Model::forward_token (src/model.rs:392-491).  pos = cache.len(layer);
 * writes vocab logits. */
OM_API int om_forward_token(om_model *m, om_cache *c, uint32_t token, float *logits) {
    const om_weights *w = &m->w;
    size_t H = w->hidden, hd = w->head_dim, nq = w->n_heads, nkv = w->n_kv, I = w->inter;
    size_t group = nq / nkv, qd = nq * hd, kvd = nkv * hd;
    if (token >= (uint32_t)w->vocab) return -1;
    memcpy(m->x, w->embed + (size_t)token * H, H * 4);
    float *x = m->x;
    for (int l = 0; l < w->layers; l++) {
        om_rms_norm(x, w->in_norm[l], w->eps, H, m->attn_in);
        lin(w, W_Q, l, m->attn_in, qd, H, m->q);
        lin(w, W_K, l, m->attn_in, kvd, H, m->k);
        lin(w, W_V, l, m->attn_in, kvd, H, m->v);
        size_t pos = c->lens[l];
        for (size_t h = 0; h < nq; h++) rope_rotate_tab(&m->rope, m->q + h * hd, pos);
        for (size_t h = 0; h < nkv; h++) rope_rotate_tab(&m->rope, m->k + h * hd, pos);
        om_cache_push(c, l, m->k, m->v);
        float scale = 1.0f / sqrtf((float)hd);
        size_t n_ctx = c->lens[l];
        if (m->scores_cap < n_ctx) {
            m->scores_cap = n_ctx * 2;
            m->scores = (float *)realloc(m->scores, sizeof(float) * m->scores_cap);
        }
        for (size_t h = 0; h < nq; h++)
            attn_head(m->q + h * hd, c->keys[l], c->vals[l], kvd, (h / group) * hd, hd, n_ctx, scale,
                      m->attn_out + h * hd, m->scores);
        lin(w, W_O, l, m->attn_out, H, qd, m->proj);
        for (size_t i = 0; i < H; i++) x[i] += m->proj[i];
        om_rms_norm(x, w->post_norm[l], w->eps, H, m->mlp_in);
        lin(w, W_G, l, m->mlp_in, I, H, m->gate);
        lin(w, W_U, l, m->mlp_in, I, H, m->up);
        for (size_t i = 0; i < I; i++) {
            float g = m->gate[i];
            m->gate[i] = g / (1.0f + expf(-g)) * m->up[i];
        }
        lin(w, W_D, l, m->gate, H, I, m->down);
        for (size_t i = 0; i < H; i++) x[i] += m->down[i];
    }
    om_rms_norm(x, w->final_norm, w->eps, H, m->attn_in);
    if (logits) lm_head(m, m->attn_in, logits);
    return 0;
}

/* Model::forward_seq (src/model.rs:503-590): batched prefill from the
 * current cache length; writes the LAST token's logits.  Optional hidden_out
 * receives the final-normed last row (for diagnostics). */
OM_API int om_forward_seq(om_model *m, om_cache *c, const uint32_t *tokens, size_t T, float *logits) {
    const om_weights *w = &m->w;
    if (T == 0) return -2; /* bail!("empty prompt") in prefill */
    size_t H = w->hidden, hd = w->head_dim, nq = w->n_heads, nkv = w->n_kv, I = w->inter;
    size_t qd = nq * hd, kvd = nkv * hd;
    size_t start = c->lens[0];
    for (size_t t = 0; t < T; t++)
        if (tokens[t] >= (uint32_t)w->vocab) return -1;
    float *x = (float *)malloc(sizeof(float) * T * H);
    float *normed = (float *)malloc(sizeof(float) * T * H);
    float *q = (float *)malloc(sizeof(float) * T * qd);
    float *k = (float *)malloc(sizeof(float) * T * kvd);
    float *v = (float *)malloc(sizeof(float) * T * kvd);
    float *att = (float *)malloc(sizeof(float) * T * qd);
    float *proj = (float *)malloc(sizeof(float) * T * H);
    float *gate = (float *)malloc(sizeof(float) * T * I);
    float *up = (float *)malloc(sizeof(float) * T * I);
    for (size_t t = 0; t < T; t++) memcpy(x + t * H, w->embed + (size_t)tokens[t] * H, H * 4);
    for (int l = 0; l < w->layers; l++) {
        memcpy(normed, x, sizeof(float) * T * H);
        om_rms_norm_batch(normed, w->in_norm[l], w->eps, H, T);
        lin_batch(w, W_Q, l, normed, qd, H, T, q);
        lin_batch(w, W_K, l, normed, kvd, H, T, k);
        lin_batch(w, W_V, l, normed, kvd, H, T, v);
        for (size_t t = 0; t < T; t++) {
            size_t pos = start + t;
            for (size_t h = 0; h < nq; h++) rope_rotate_tab(&m->rope, q + t * qd + h * hd, pos);
            for (size_t h = 0; h < nkv; h++) rope_rotate_tab(&m->rope, k + t * kvd + h * hd, pos);
        }
        for (size_t t = 0; t < T; t++) om_cache_push(c, l, k + t * kvd, v + t * kvd);
        om_attention_batch(q, c->keys[l], c->vals[l], T, nq, nkv, hd, start, att);
        lin_batch(w, W_O, l, att, H, qd, T, proj);
        for (size_t i = 0; i < T * H; i++) x[i] += proj[i];
        memcpy(normed, x, sizeof(float) * T * H);
        om_rms_norm_batch(normed, w->post_norm[l], w->eps, H, T);
        lin_batch(w, W_G, l, normed, I, H, T, gate);
        lin_batch(w, W_U, l, normed, I, H, T, up);
        for (size_t i = 0; i < T * I; i++) {
            float g = gate[i];
            gate[i] = g / (1.0f + expf(-g)) * up[i];
        }
        lin_batch(w, W_D, l, gate, H, I, T, proj);
        for (size_t i = 0; i < T * H; i++) x[i] += proj[i];
    }
    float *last = x + (T - 1) * H;
    om_rms_norm_batch(last, w->final_norm, w->eps, H, 1);
    if (logits) lm_head(m, last, logits);
    free(x);
    free(normed);
    free(q);
    free(k);
    free(v);
    free(att);
    free(proj);
    free(gate);
    free(up);
    return 0;
}
