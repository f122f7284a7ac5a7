/* v7_oracle_avx2.c -- AVX2 restatement of v7's fused per-layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY: this is the CPU baseline the benchmark times next
 * to the GPU kernels (labelled "port": a restatement, not the reference
 * binary, which needs nasm to build).  It restates the same NASM kernels as
 * v7_oracle.c with AVX2/FMA intrinsics in the reference's own vector shapes,
 * and the test suite checks that it agrees with the scalar oracle bit for bit.
 *
 * Reference kernels: src/asm/add_rmsnorm_kernel.inc:15-129,
 * src/asm/v7_macros.inc:38-45,98-160,263-354, src/asm/quantize_kernel.inc:44-159,
 * src/asm/prefill_q8.inc:1159-1166, src/asm/forward.inc:13-42.
 */
#include "v7_oracle.h"
#include "v7_oracle_fpenv.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define AVX2 __attribute__((target("avx2,fma")))

int orc_avx2_available(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

/* HADD_YMM, v7_macros.inc:38-45 */
static AVX2 float hadd_ymm(__m256 v)
{
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    __m128 t = _mm_movehdup_ps(lo);
    lo = _mm_add_ps(lo, t);
    t = _mm_movehl_ps(t, lo);
    lo = _mm_add_ss(lo, t);
    return _mm_cvtss_f32(lo);
}

/* COMPUTE_RMS_SCALE, v7_macros.inc:348-354 */
static AVX2 float rms_scale(float ss, int n, float eps)
{
    __m128 v = _mm_set_ss(ss);
    v = _mm_div_ss(v, _mm_set_ss((float)n));
    v = _mm_add_ss(v, _mm_set_ss(eps));
    v = _mm_sqrt_ss(v);
    v = _mm_div_ss(_mm_set_ss(1.0f), v);
    return _mm_cvtss_f32(v);
}

/* add_rmsnorm_kernel.inc:15-129 */
AVX2 void orc_avx2_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int dim,
                                     float eps)
{
    ORC_REFERENCE_FP_ENV;
    int blocks = dim >> 3;
    __m256 a = _mm256_setzero_ps(), b = _mm256_setzero_ps(), c = _mm256_setzero_ps(), d = _mm256_setzero_ps();
    float *r = residual;
    const float *p = add;
    for (int i = 0; i < (blocks & 3); ++i) {
        __m256 x = _mm256_add_ps(_mm256_loadu_ps(r), _mm256_loadu_ps(p));
        _mm256_storeu_ps(r, x);
        a = _mm256_fmadd_ps(x, x, a);
        r += 8;
        p += 8;
    }
    for (int g = 0; g < (blocks >> 2); ++g) {
        __m256 x0 = _mm256_add_ps(_mm256_loadu_ps(r), _mm256_loadu_ps(p));
        __m256 x1 = _mm256_add_ps(_mm256_loadu_ps(r + 8), _mm256_loadu_ps(p + 8));
        __m256 x2 = _mm256_add_ps(_mm256_loadu_ps(r + 16), _mm256_loadu_ps(p + 16));
        __m256 x3 = _mm256_add_ps(_mm256_loadu_ps(r + 24), _mm256_loadu_ps(p + 24));
        a = _mm256_fmadd_ps(x0, x0, a);
        b = _mm256_fmadd_ps(x1, x1, b);
        c = _mm256_fmadd_ps(x2, x2, c);
        d = _mm256_fmadd_ps(x3, x3, d);
        _mm256_storeu_ps(r, x0);
        _mm256_storeu_ps(r + 8, x1);
        _mm256_storeu_ps(r + 16, x2);
        _mm256_storeu_ps(r + 24, x3);
        r += 32;
        p += 32;
    }
    a = _mm256_add_ps(a, b);
    c = _mm256_add_ps(c, d);
    a = _mm256_add_ps(a, c);
    __m256 s = _mm256_set1_ps(rms_scale(hadd_ymm(a), dim, eps));
    for (int i = 0; i < blocks; ++i) {
        __m256 x = _mm256_mul_ps(s, _mm256_loadu_ps(residual + 8 * i));
        x = _mm256_mul_ps(x, _mm256_loadu_ps(weight + 8 * i));
        _mm256_storeu_ps(o + 8 * i, x);
    }
}

/* RMSNORM_ROPE_BODY, v7_macros.inc:263-340, for each head */
AVX2 void orc_avx2_rmsnorm_rope_heads(float *buf, int n_heads, int head_dim, const float *w, const float *cos_table,
                                      const float *sin_table, int pos, int rope_max_dim, float eps)
{
    ORC_REFERENCE_FP_ENV;
    const float *ct = cos_table + (long long)pos * rope_max_dim;
    const float *st = sin_table + (long long)pos * rope_max_dim;
    int half = head_dim / 2;
    for (int h = 0; h < n_heads; ++h) {
        float *x = buf + (long long)h * head_dim;
        __m256 a = _mm256_setzero_ps(), b = _mm256_setzero_ps(), c = _mm256_setzero_ps(), d = _mm256_setzero_ps();
        for (int i = 0; i < head_dim; i += 32) {
            __m256 x0 = _mm256_loadu_ps(x + i), x1 = _mm256_loadu_ps(x + i + 8);
            a = _mm256_fmadd_ps(x0, x0, a);
            b = _mm256_fmadd_ps(x1, x1, b);
            __m256 x2 = _mm256_loadu_ps(x + i + 16), x3 = _mm256_loadu_ps(x + i + 24);
            c = _mm256_fmadd_ps(x2, x2, c);
            d = _mm256_fmadd_ps(x3, x3, d);
        }
        a = _mm256_add_ps(a, b);
        c = _mm256_add_ps(c, d);
        a = _mm256_add_ps(a, c);
        __m256 s = _mm256_set1_ps(rms_scale(hadd_ymm(a), head_dim, eps));
        if (pos == 0) {
            for (int i = 0; i < head_dim; i += 8) {
                __m256 v = _mm256_mul_ps(_mm256_loadu_ps(x + i), s);
                _mm256_storeu_ps(x + i, _mm256_mul_ps(v, _mm256_loadu_ps(w + i)));
            }
            continue;
        }
        for (int j = 0; j < half; j += 8) {
            __m256 cv = _mm256_loadu_ps(ct + j), sv = _mm256_loadu_ps(st + j);
            __m256 xe = _mm256_mul_ps(_mm256_loadu_ps(x + j), s);
            __m256 xo = _mm256_mul_ps(_mm256_loadu_ps(x + half + j), s);
            xe = _mm256_mul_ps(xe, _mm256_loadu_ps(w + j));
            xo = _mm256_mul_ps(xo, _mm256_loadu_ps(w + half + j));
            __m256 re = _mm256_mul_ps(xe, cv);
            __m256 ro = _mm256_mul_ps(xe, sv);
            re = _mm256_fnmadd_ps(xo, sv, re);
            ro = _mm256_fmadd_ps(xo, cv, ro);
            _mm256_storeu_ps(x + j, re);
            _mm256_storeu_ps(x + half + j, ro);
        }
    }
}

/* EVAL_SIGMOID ps, v7_macros.inc:98-160 */
/* v7s_rmsnorm (src/asm/rmsnorm_kernel.inc:12-75): the order of orc_avx2_fused_add_rmsnorm without the add
 * (leftover 8-float blocks into A first, then groups of four blocks into A..D; (A+B)+(C+D); HADD_YMM). */
AVX2 void orc_avx2_rmsnorm(float *o, const float *x, const float *weight, int dim, float eps)
{
    ORC_REFERENCE_FP_ENV;
    int blocks = dim >> 3;
    __m256 a = _mm256_setzero_ps(), b = _mm256_setzero_ps(), c = _mm256_setzero_ps(), d = _mm256_setzero_ps();
    const float *r = x;
    for (int i = 0; i < (blocks & 3); ++i) {
        __m256 v = _mm256_loadu_ps(r);
        a = _mm256_fmadd_ps(v, v, a);
        r += 8;
    }
    for (int g = 0; g < (blocks >> 2); ++g) {
        __m256 x0 = _mm256_loadu_ps(r), x1 = _mm256_loadu_ps(r + 8);
        __m256 x2 = _mm256_loadu_ps(r + 16), x3 = _mm256_loadu_ps(r + 24);
        a = _mm256_fmadd_ps(x0, x0, a);
        b = _mm256_fmadd_ps(x1, x1, b);
        c = _mm256_fmadd_ps(x2, x2, c);
        d = _mm256_fmadd_ps(x3, x3, d);
        r += 32;
    }
    a = _mm256_add_ps(a, b);
    c = _mm256_add_ps(c, d);
    a = _mm256_add_ps(a, c);
    __m256 s = _mm256_set1_ps(rms_scale(hadd_ymm(a), dim, eps));
    for (int i = 0; i < blocks; ++i) {
        __m256 v = _mm256_mul_ps(s, _mm256_loadu_ps(x + 8 * i));
        _mm256_storeu_ps(o + 8 * i, _mm256_mul_ps(v, _mm256_loadu_ps(weight + 8 * i)));
    }
}

/* v7s_add_inplace (src/asm/add_kernel.inc:26-49) and PQ_BIAS_ADD (src/asm/v7_macros.inc:366-383): x = x + y
 * with vaddps, 8 floats at a time; the last n % 8 one at a time. */
AVX2 void orc_avx2_add_inplace(float *x, const float *y, long long n)
{
    ORC_REFERENCE_FP_ENV;
    long long i = 0;
    for (; i + 8 <= n; i += 8)
        _mm256_storeu_ps(x + i, _mm256_add_ps(_mm256_loadu_ps(x + i), _mm256_loadu_ps(y + i)));
    for (; i < n; ++i)
        x[i] = x[i] + y[i];
}

/* RoPE without the norm, v7s_rope_only_head (src/asm/rope_only_kernel.inc:11-53): per 8 pairs
 * vmulps lo*cos, vmulps lo*sin, vfnmadd231ps (lo*cos - up*sin), vfmadd231ps (lo*sin + up*cos); pos == 0
 * leaves the heads as they are.  Bit for bit the scalar orc_rope_only_heads (tests/test_oracle.py). */
AVX2 void orc_avx2_rope_only_heads(float *buf, int n_heads, int head_dim, const float *cos_table,
                                   const float *sin_table, int pos, int rope_max_dim)
{
    ORC_REFERENCE_FP_ENV;
    if (pos == 0)
        return;
    const float *c = cos_table + (long long)pos * rope_max_dim;
    const float *s = sin_table + (long long)pos * rope_max_dim;
    const int half = head_dim / 2;
    for (int h = 0; h < n_heads; ++h) {
        float *lo = buf + (long long)h * head_dim, *up = lo + half;
        int j = 0;
        for (; j + 8 <= half; j += 8) {
            const __m256 cv = _mm256_loadu_ps(c + j), sv = _mm256_loadu_ps(s + j);
            const __m256 l = _mm256_loadu_ps(lo + j), u = _mm256_loadu_ps(up + j);
            const __m256 re = _mm256_fnmadd_ps(u, sv, _mm256_mul_ps(l, cv));
            const __m256 ro = _mm256_fmadd_ps(u, cv, _mm256_mul_ps(l, sv));
            _mm256_storeu_ps(lo + j, re);
            _mm256_storeu_ps(up + j, ro);
        }
        for (; j < half; ++j) {
            const float l = lo[j], u = up[j];
            lo[j] = fmaf(-u, s[j], l * c[j]);
            up[j] = fmaf(u, c[j], l * s[j]);
        }
    }
}

static AVX2 __m256 sigmoid_ps(__m256 g)
{
    const __m256 sign = _mm256_castsi256_ps(_mm256_set1_epi32((int)0x80000000u));
    __m256 x = _mm256_xor_ps(g, sign);
    x = _mm256_max_ps(x, _mm256_set1_ps(-80.0f));
    x = _mm256_min_ps(x, _mm256_set1_ps(80.0f));
    __m256 fx = _mm256_mul_ps(x, _mm256_set1_ps((float)1.4426950408889634));
    __m256 ip = _mm256_round_ps(fx, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 fp = _mm256_sub_ps(fx, ip);
    __m256i e2 = _mm256_cvttps_epi32(ip);
    e2 = _mm256_add_epi32(e2, _mm256_set1_epi32(127));
    e2 = _mm256_slli_epi32(e2, 23);
    __m256 p = _mm256_castsi256_ps(_mm256_set1_epi32(0x3AADD303));
    p = _mm256_fmadd_ps(fp, p, _mm256_castsi256_ps(_mm256_set1_epi32(0x3C1E7411)));
    p = _mm256_fmadd_ps(fp, p, _mm256_castsi256_ps(_mm256_set1_epi32(0x3D635B9B)));
    p = _mm256_fmadd_ps(fp, p, _mm256_castsi256_ps(_mm256_set1_epi32(0x3E75FCE0)));
    p = _mm256_fmadd_ps(fp, p, _mm256_castsi256_ps(_mm256_set1_epi32(0x3F317215)));
    p = _mm256_fmadd_ps(fp, p, _mm256_set1_ps(1.0f));
    __m256 e = _mm256_mul_ps(_mm256_castsi256_ps(e2), p);
    __m256 one = _mm256_set1_ps(1.0f);
    return _mm256_div_ps(one, _mm256_add_ps(e, one));
}

/* .pq_ffn_silu, prefill_q8.inc:1159-1166; n % 8 == 0 on the vector path */
AVX2 void orc_avx2_swiglu(float *out, const float *gate, const float *up, long long n)
{
    ORC_REFERENCE_FP_ENV;
    long long i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 g = _mm256_loadu_ps(gate + i);
        __m256 s = sigmoid_ps(g);
        s = _mm256_mul_ps(s, g);
        _mm256_storeu_ps(out + i, _mm256_mul_ps(s, _mm256_loadu_ps(up + i)));
    }
    if (i < n)
        orc_swiglu(out + i, gate + i, up + i, n - i);
}

/* QUANTIZE_32, quantize_kernel.inc:91-105 */
static AVX2 void quant32(int8_t *q, const float *x, __m256 recip)
{
    const __m256i perm = _mm256_setr_epi32(0, 4, 1, 5, 2, 6, 3, 7);
    __m256i a = _mm256_cvtps_epi32(_mm256_mul_ps(recip, _mm256_loadu_ps(x)));
    __m256i b = _mm256_cvtps_epi32(_mm256_mul_ps(recip, _mm256_loadu_ps(x + 8)));
    __m256i c = _mm256_cvtps_epi32(_mm256_mul_ps(recip, _mm256_loadu_ps(x + 16)));
    __m256i d = _mm256_cvtps_epi32(_mm256_mul_ps(recip, _mm256_loadu_ps(x + 24)));
    __m256i ab = _mm256_packs_epi32(a, b);
    __m256i cd = _mm256_packs_epi32(c, d);
    __m256i v = _mm256_packs_epi16(ab, cd);
    v = _mm256_max_epi8(v, _mm256_set1_epi8(-127));
    v = _mm256_permutevar8x32_epi32(v, perm);
    _mm256_storeu_si256((__m256i *)q, v);
}

/* v7s_quantize_chunk, quantize_kernel.inc:44-159, for gs in {32, 64} */
AVX2 void orc_avx2_quantize(int8_t *out_q, const float *in_x, float *out_s, long long n, int gs)
{
    ORC_REFERENCE_FP_ENV;
    const __m256 absmask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7FFFFFFF));
    long long full = n / gs;
    for (long long g = 0; g < full; ++g) {
        const float *x = in_x + g * gs;
        __m256 v[8];
        for (int j = 0; j < 8; ++j)
            v[j] = j < gs / 8 ? _mm256_and_ps(absmask, _mm256_loadu_ps(x + 8 * j)) : _mm256_setzero_ps();
        /* the reference's pairing (quantize_kernel.inc:62-83), which fixes where a NaN survives */
        __m256 m = _mm256_max_ps(_mm256_max_ps(v[0], v[1]), _mm256_max_ps(v[2], v[3]));
        if (gs == 64)
            m = _mm256_max_ps(m, _mm256_max_ps(_mm256_max_ps(v[4], v[5]), _mm256_max_ps(v[6], v[7])));
        __m128 l = _mm_max_ps(_mm256_castps256_ps128(m), _mm256_extractf128_ps(m, 1));
        l = _mm_max_ps(l, _mm_movehl_ps(l, l));
        l = _mm_max_ps(l, _mm_movehdup_ps(l));
        l = _mm_max_ss(l, _mm_set_ss(1.4928778e-36f));
        __m128 sc = _mm_div_ss(l, _mm_set_ss(127.0f));
        out_s[g] = _mm_cvtss_f32(sc);
        __m256 recip = _mm256_set1_ps(_mm_cvtss_f32(_mm_div_ss(_mm_set_ss(1.0f), sc)));
        for (int i = 0; i < gs; i += 32)
            quant32(out_q + g * gs + i, x + i, recip);
    }
    if (n > full * gs)
        orc_quantize(out_q + full * gs, in_x + full * gs, out_s + full, n - full * gs, gs);
}

/* forward.inc:13-42 */
AVX2 void orc_avx2_embedding_row(float *out, int token, int dim, const int8_t *table_q, const float *table_s)
{
    long long base = (long long)token * dim;
    const int8_t *q = table_q + base;
    const float *s = table_s + (base >> 6);
    for (int i = 0; i < dim; i += 64) {
        __m256 sc = _mm256_set1_ps(s[i >> 6]);
        for (int k = 0; k < 64; k += 8) {
            __m128i b = _mm_loadl_epi64((const __m128i *)(q + i + k));
            __m256 v = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b));
            _mm256_storeu_ps(out + i + k, _mm256_mul_ps(v, sc));
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Row-parallel per-layer chain, driven per token row as the reference engine
 * drives these kernels (prefill_q8.inc:317-350, 815-911, 1154-1183;
 * forward_f32.inc:324-332). */
typedef struct {
    const orc_chain_args *a;
    int t0, t1, reps;
} chain_job;

static void chain_rows(const orc_chain_args *a, int t0, int t1)
{
    int dim = a->dim, hd = a->head_dim, hidden = a->hidden;
    int spr = (hidden + a->gs - 1) / a->gs;
    for (int t = t0; t < t1; ++t) {
        long long td = (long long)t * dim;
        orc_avx2_embedding_row(a->emb_out + td, a->ids[t], dim, a->table_q, a->table_s);
        orc_avx2_fused_add_rmsnorm(a->normed + td, a->residual + td, a->add + td, a->w_norm, dim, a->eps);
        orc_avx2_rmsnorm_rope_heads(a->q + (long long)t * a->n_q_heads * hd, a->n_q_heads, hd, a->q_w, a->cos_table,
                                    a->sin_table, a->positions[t], a->rope_max_dim, a->eps);
        orc_avx2_rmsnorm_rope_heads(a->k + (long long)t * a->n_kv_heads * hd, a->n_kv_heads, hd, a->k_w,
                                    a->cos_table, a->sin_table, a->positions[t], a->rope_max_dim, a->eps);
        orc_avx2_swiglu(a->act + (long long)t * hidden, a->gate + (long long)t * hidden, a->up + (long long)t * hidden,
                        hidden);
        orc_avx2_quantize(a->codes + (long long)t * hidden, a->act + (long long)t * hidden,
                          a->scales + (long long)t * spr, hidden, a->gs);
    }
}

static void *chain_thread(void *p)
{
    ORC_REFERENCE_FP_ENV;
    chain_job *j = (chain_job *)p;
    for (int r = 0; r < j->reps; ++r)
        chain_rows(j->a, j->t0, j->t1);
    return 0;
}

double orc_avx2_chain_bench(const orc_chain_args *a, int n_threads, int reps)
{
    if (n_threads < 1)
        n_threads = 1;
    if (n_threads > 256)
        n_threads = 256;
    pthread_t th[256];
    chain_job jobs[256];
    struct timespec ts0, ts1;
    clock_gettime(CLOCK_MONOTONIC, &ts0);
    for (int i = 0; i < n_threads; ++i) {
        jobs[i].a = a;
        jobs[i].t0 = (int)((long long)a->n_tokens * i / n_threads);
        jobs[i].t1 = (int)((long long)a->n_tokens * (i + 1) / n_threads);
        jobs[i].reps = reps;
        if (i > 0)
            pthread_create(&th[i], 0, chain_thread, &jobs[i]);
    }
    chain_thread(&jobs[0]);
    for (int i = 1; i < n_threads; ++i)
        pthread_join(th[i], 0);
    clock_gettime(CLOCK_MONOTONIC, &ts1);
    return (double)(ts1.tv_sec - ts0.tv_sec) + 1e-9 * (double)(ts1.tv_nsec - ts0.tv_nsec);
}

/* kv_f16c.inc:12-52: vcvtps2ph with imm 0 (nearest-even), 8 floats at a time; n % 8 == 0. */
__attribute__((target("avx2,f16c"))) void orc_avx2_kv_pack_f16(uint16_t *dst, const float *src, long long n)
{
    for (long long i = 0; i + 8 <= n; i += 8) {
        __m128i h = _mm256_cvtps_ph(_mm256_loadu_ps(src + i), 0);
        _mm_storeu_si128((__m128i *)(dst + i), h);
    }
}

int orc_f16c_available(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("f16c");
}

/* Compares orc_f32_to_f16_bits with the F16C instruction (vcvtps2ph imm 0, the reference's instruction)
 * for every binary32 bit pattern in [lo, lo + count), split over n_threads threads.  Returns the number
 * of mismatches (NaN inputs included: both keep the top payload bits and set the quiet bit). */
typedef struct {
    uint64_t lo, hi;
    unsigned long long bad;
} f16_job;

static __attribute__((target("avx2,f16c"))) void *f16_check_thread(void *p)
{
    f16_job *j = (f16_job *)p;
    unsigned long long bad = 0;
    uint32_t in[8];
    uint16_t hw[8];
    for (uint64_t b = j->lo; b < j->hi; b += 8) {
        for (int k = 0; k < 8; ++k)
            in[k] = (uint32_t)(b + (uint64_t)k < j->hi ? b + (uint64_t)k : j->hi - 1);
        __m256 v = _mm256_loadu_ps((const float *)in);
        _mm_storeu_si128((__m128i *)hw, _mm256_cvtps_ph(v, 0));
        for (int k = 0; k < 8; ++k) {
            float f;
            memcpy(&f, &in[k], 4);
            bad += orc_f32_to_f16_bits(f) != hw[k];
        }
    }
    j->bad = bad;
    return 0;
}

unsigned long long orc_check_f16_vs_f16c(uint64_t lo, uint64_t count, int n_threads)
{
    if (n_threads < 1)
        n_threads = 1;
    if (n_threads > 64)
        n_threads = 64;
    pthread_t th[64];
    f16_job jobs[64];
    uint64_t per = (count + (uint64_t)n_threads - 1) / (uint64_t)n_threads;
    per = (per + 7) & ~(uint64_t)7;
    for (int i = 0; i < n_threads; ++i) {
        jobs[i].lo = lo + (uint64_t)i * per;
        jobs[i].hi = jobs[i].lo + per;
        if (jobs[i].hi > lo + count)
            jobs[i].hi = lo + count;
        if (jobs[i].lo > jobs[i].hi)
            jobs[i].lo = jobs[i].hi;
        jobs[i].bad = 0;
        pthread_create(&th[i], 0, f16_check_thread, &jobs[i]);
    }
    unsigned long long total = 0;
    for (int i = 0; i < n_threads; ++i) {
        pthread_join(th[i], 0);
        total += jobs[i].bad;
    }
    return total;
}
