/* v7_oracle.c -- scalar CPU oracle for v7's fused per-layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  The test suite, the smoke check and the
 * benchmark's CPU-baseline leg are the only users; the product (the HIP
 * library) never links or calls it.
 *
 * Each function restates one NASM kernel of the reference engine,
 * cpki-gmbh/v7multiplikator, in plain C.  The restatement follows the
 * reference instruction by instruction wherever the order of floating-point
 * operations is observable:
 *   - every vaddps/vmulps/vdivps/vsqrtps is one correctly rounded C operator,
 *   - every vfmadd/vfnmadd is one fmaf() call (the hardware FMA, -mfma),
 *   - the path functions run under the reference's MXCSR FTZ+DAZ
 *     (v7_oracle_fpenv.h), as the reference's kernels do,
 *   - the eight-lane YMM accumulators are modelled as explicit arrays and
 *     reduced by the same addition tree as the reference's HADD_YMM macro.
 * Compile with -ffp-contract=off and without -ffast-math (see Makefile).
 *
 * Parity pins (what fixes each function besides this restatement) are listed
 * in the test suite: tests/test_oracle.py.
 */
#include "v7_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "v7_oracle_fpenv.h"

static int g_ref_fp_env = 1;
void orc_set_reference_fp_env(int on) { g_ref_fp_env = on ? 1 : 0; }
int orc_get_reference_fp_env(void) { return g_ref_fp_env; }
unsigned orc_fp_enter(void)
{
    unsigned old = _mm_getcsr();
    if (g_ref_fp_env)
        _mm_setcsr(old | 0x8040u); /* FTZ (bit 15) + DAZ (bit 6) */
    return old;
}

/* ------------------------------------------------------------------------ */
/* HADD_YMM: src/asm/v7_macros.inc:38-45.  v[i] + v[i+4] for i < 4, then
 * (s0 + s1) + (s2 + s3): vmovshdup pairs lanes 0/1 and 2/3, vmovhlps brings
 * lane 2 down to lane 0. */
static float hadd8(const float v[8])
{
    float s0 = v[0] + v[4];
    float s1 = v[1] + v[5];
    float s2 = v[2] + v[6];
    float s3 = v[3] + v[7];
    float t0 = s0 + s1;
    float t2 = s2 + s3;
    return t0 + t2;
}

/* Sum of squares with four YMM accumulators A..D.
 * src/asm/add_rmsnorm_kernel.inc:29-73 (Pass 1 + reduce) and
 * src/asm/v7_macros.inc:263-291 (RMSNORM_ROPE_BODY Pass 1).
 * The row is split into 8-float blocks.  Blocks that do not fill a 4-way group
 * (blocks % 4) are accumulated first, all into A (add_rmsnorm_kernel.inc:37-39,
 * 112-121); then each group of four blocks feeds A, B, C, D in turn
 * (add_rmsnorm_kernel.inc:45-68).  For n % 32 == 0 this is exactly the
 * RMSNORM_ROPE_BODY loop, whose 32-element block feeds elements 0-7 to A, 8-15
 * to B, 16-23 to C and 24-31 to D.  Reduction: (A+B) + (C+D) lane-wise, then
 * HADD_YMM (add_rmsnorm_kernel.inc:70-73, v7_macros.inc:286-289). */
float orc_sumsq_lanes(const float *x, int n)
{
    ORC_REFERENCE_FP_ENV;
    float acc[4][8];
    memset(acc, 0, sizeof(acc));
    int blocks = n / 8;
    int left = blocks & 3;
    int b = 0;
    for (; b < left; ++b)
        for (int j = 0; j < 8; ++j)
            acc[0][j] = fmaf(x[8 * b + j], x[8 * b + j], acc[0][j]);
    for (int g = 0; g < blocks / 4; ++g)
        for (int q = 0; q < 4; ++q, ++b)
            for (int j = 0; j < 8; ++j)
                acc[q][j] = fmaf(x[8 * b + j], x[8 * b + j], acc[q][j]);
    float v[8];
    for (int j = 0; j < 8; ++j) {
        float ab = acc[0][j] + acc[1][j];
        float cd = acc[2][j] + acc[3][j];
        v[j] = ab + cd;
    }
    return hadd8(v);
}

/* COMPUTE_RMS_SCALE: src/asm/v7_macros.inc:348-354.
 * vdivss sumsq/dim; vaddss eps (g_rms_eps); vsqrtss; vdivss 1/x.  dim is
 * converted with vcvtsi2ss (add_rmsnorm_kernel.inc:74-75,
 * rmsnorm_rope_dispatch.inc:20). */
float orc_rms_scale(float sumsq, int n, float eps)
{
    ORC_REFERENCE_FP_ENV;
    float mean = sumsq / (float)n;
    float val = mean + eps;
    float root = sqrtf(val);
    return 1.0f / root;
}

/* v7s_fused_add_rmsnorm(o, residual, add, weight, dim):
 * src/asm/add_rmsnorm_kernel.inc:15-129, typedef src/v7_lib.h:272.
 * Pass 1: residual = residual + add (vaddps, stored in place).
 * Pass 2: o = (scale * residual) * weight, two vmulps (:87-94). */
void orc_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int dim, float eps)
{
    ORC_REFERENCE_FP_ENV;
    for (int i = 0; i < dim; ++i)
        residual[i] = residual[i] + add[i];
    float ss = orc_sumsq_lanes(residual, dim);
    float s = orc_rms_scale(ss, dim, eps);
    for (int i = 0; i < dim; ++i) {
        float t = s * residual[i];
        o[i] = t * weight[i];
    }
}

void orc_fused_add_rmsnorm_rows(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                                float eps)
{
    ORC_REFERENCE_FP_ENV;
    for (int r = 0; r < rows; ++r)
        orc_fused_add_rmsnorm(o + (long long)r * dim, residual + (long long)r * dim, add + (long long)r * dim, weight,
                              dim, eps);
}

/* One head of v7s_rmsnorm_rope_heads: RMSNORM_ROPE_BODY,
 * src/asm/v7_macros.inc:263-340, driven by rmsnorm_rope_kernel.inc:7-23
 * (and identically by qk_fork_kernel.inc:40-62).  cos/sin point at the row of
 * this position already (rmsnorm_rope_dispatch.inc:24-33). */
static void rope_head(float *x, int head_dim, const float *w, const float *c, const float *s, int pos, float eps)
{
    float ss = orc_sumsq_lanes(x, head_dim);
    float scale = orc_rms_scale(ss, head_dim, eps);
    if (pos == 0) {
        /* %%rmsnorm_only, v7_macros.inc:325-339 */
        for (int i = 0; i < head_dim; ++i) {
            float t = x[i] * scale;
            x[i] = t * w[i];
        }
        return;
    }
    /* %%rp_loop, v7_macros.inc:305-323 */
    int half = head_dim / 2;
    for (int j = 0; j < half; ++j) {
        float xe = x[j] * scale;
        float xo = x[j + half] * scale;
        xe = xe * w[j];
        xo = xo * w[j + half];
        float re = xe * c[j];
        float ro = xe * s[j];
        re = fmaf(-xo, s[j], re); /* vfnmadd231ps: re - xo*sin, one rounding */
        ro = fmaf(xo, c[j], ro);  /* vfmadd231ps: ro + xo*cos, one rounding */
        x[j] = re;
        x[j + half] = ro;
    }
}

/* v7s_rmsnorm_rope_heads(buf, n_heads, head_dim, norm_weight, cos, sin, pos,
 * rope_max_dim): src/asm/rmsnorm_rope_dispatch.inc:11-52; typedef
 * src/v7_lib.h:273.  One job per head, heads contiguous in buf; eps is the
 * g_rms_eps global in the reference and an argument here. */
void orc_rmsnorm_rope_heads(float *buf, int n_heads, int head_dim, const float *norm_weight, const float *cos_table,
                            const float *sin_table, int pos, int rope_max_dim, float eps)
{
    ORC_REFERENCE_FP_ENV;
    const float *c = cos_table + (long long)pos * rope_max_dim;
    const float *s = sin_table + (long long)pos * rope_max_dim;
    for (int h = 0; h < n_heads; ++h)
        rope_head(buf + (long long)h * head_dim, head_dim, norm_weight, c, s, pos, eps);
}

void orc_rmsnorm_rope_tokens(float *buf, int n_tokens, long long token_stride, int n_heads, int head_dim,
                             const float *norm_weight, const float *cos_table, const float *sin_table,
                             const int32_t *positions, int rope_max_dim, float eps)
{
    ORC_REFERENCE_FP_ENV;
    for (int t = 0; t < n_tokens; ++t)
        orc_rmsnorm_rope_heads(buf + (long long)t * token_stride, n_heads, head_dim, norm_weight, cos_table, sin_table,
                               positions[t], rope_max_dim, eps);
}

/* The reference builds its RoPE tables with x87 instructions under control
 * word 0x037F (64-bit significand, round to nearest, exceptions masked;
 * src/asm/fused_f32_kernel.inc:109-110,176-177).  The same instructions, one
 * for one, give the same bits: each helper below is one of them. */
static long double x87_fyl2x(long double x, long double y) /* y * log2(x) */
{
    long double r;
    __asm__("fyl2x" : "=t"(r) : "0"(x), "u"(y) : "st(1)");
    return r;
}
static long double x87_frndint(long double x)
{
    long double r;
    __asm__("frndint" : "=t"(r) : "0"(x));
    return r;
}
static long double x87_f2xm1(long double x) /* 2^x - 1, |x| <= 1 */
{
    long double r;
    __asm__("f2xm1" : "=t"(r) : "0"(x));
    return r;
}
static long double x87_fscale(long double x, long double e) /* x * 2^trunc(e) */
{
    long double r;
    __asm__("fscale" : "=t"(r) : "0"(x), "u"(e));
    return r;
}
static void x87_fsincos(long double a, long double *c, long double *s)
{
    long double cc, ss;
    __asm__("fsincos" : "=t"(cc), "=u"(ss) : "0"(a));
    *c = cc;
    *s = ss;
}
static unsigned short x87_enter(void)
{
    unsigned short old, cw = 0x037F;
    __asm__ volatile("fnstcw %0" : "=m"(old));
    __asm__ volatile("fldcw %0" : : "m"(cw));
    return old;
}
static void x87_leave(unsigned short old) { __asm__ volatile("fldcw %0" : : "m"(old)); }

/* RBIT_CALC_INV_FREQ, src/asm/fused_f32_kernel.inc:117-134: t = j/half (fdivp),
 * y = -t * log2(base) (fchs, fyl2x), i = frndint(y), f = y - i, freq =
 * (f2xm1(f) + 1) * 2^i (fld1, faddp, fscale); extended precision throughout. */
static long double ref_inv_freq(float base, int j, int half)
{
    const long double t = (long double)j / (long double)half;
    const long double y = x87_fyl2x((long double)base, -t);
    const long double i = x87_frndint(y);
    return x87_fscale(x87_f2xm1(y - i) + 1.0L, i);
}

/* Plain frequencies (rope type 0, :120-147): freq_j = RBIT_CALC_INV_FREQ
 * stored as a double (fstp qword). */
void orc_rope_freqs(double *freq, int half, float base)
{
    const unsigned short cw = x87_enter();
    for (int j = 0; j < half; ++j) freq[j] = (double)ref_inv_freq(base, j, half);
    x87_leave(cw);
}

/* Tables from precomputed frequencies, the .rbit_outer / .rbit_inner fill
 * (:257-303): angle = freq_j * pos (fld qword freq, fmul qword pos: the
 * product in extended precision), fsincos, each result rounded to float on
 * store (fstp dword). */
static void rope_fill(float *cos_table, float *sin_table, int n_pos, int half, const double *freq)
{
    const unsigned short cw = x87_enter();
    for (int p = 0; p < n_pos; ++p)
        for (int j = 0; j < half; ++j) {
            long double c, s;
            x87_fsincos((long double)freq[j] * (long double)(double)p, &c, &s);
            cos_table[(long long)p * half + j] = (float)c;
            sin_table[(long long)p * half + j] = (float)s;
        }
    x87_leave(cw);
}

/* RoPE tables: src/asm/fused_f32_kernel.inc:69-147,257-303 (plain, type 0). */
void orc_rope_tables(float *cos_table, float *sin_table, int n_pos, int head_dim, float rope_base)
{
    const int half = head_dim / 2;
    double freq[512];
    orc_rope_freqs(freq, half, rope_base);
    rope_fill(cos_table, sin_table, n_pos, half, freq);
}

/* RoPE frequencies with Llama 3 scaling (rope type 1):
 * src/asm/fused_f32_kernel.inc:149-256 (.rbit_llama3_setup, .rbit_prefreq),
 * the HF llama3 formula evaluated in x87 extended precision with the stores to
 * double of the reference:
 *   low_wl = old/low, high_wl = old/high                       (stored double)
 *   inv = base^(-j/half)       (extended; stored double, the extended value
 *                               goes on into the wavelength)
 *   wavelen = 2 pi / inv                                       (stored double)
 *   ifl = wavelen > low_wl ? inv/factor : inv                  (stored double)
 *   smooth = (old/wavelen - low) / (high - low)                (stored double)
 *   smoothed = (1 - smooth) * (ifl/factor) + smooth * ifl      (stored double)
 *   freq = high_wl <= wavelen <= low_wl ? smoothed : ifl. */
void orc_rope_freqs_llama3(double *freq, int half, float base, float factor, float low_freq_factor,
                           float high_freq_factor, int orig_max_pos)
{
    const unsigned short cw = x87_enter();
    const double two_pi = 6.28318530717958647692; /* rbit_two_pi */
    const long double f = (double)factor, lo = (double)low_freq_factor, hi = (double)high_freq_factor;
    const long double old = (double)orig_max_pos;
    const double low_wl = (double)(old / lo);
    const double high_wl = (double)(old / hi);
    for (int j = 0; j < half; ++j) {
        long double inv_x = ref_inv_freq(base, j, half); /* Step A, RBIT_CALC_INV_FREQ */
        double inv = (double)inv_x;
        double wavelen = (double)((long double)two_pi / inv_x);
        double ifl = (wavelen > low_wl) ? (double)((long double)inv / f) : inv;
        double smooth = (double)((old / (long double)wavelen - lo) / (hi - lo));
        double smoothed = (double)((1.0L - (long double)smooth) * ((long double)ifl / f) +
                                   (long double)smooth * (long double)ifl);
        int medium = wavelen >= high_wl && wavelen <= low_wl;
        freq[j] = medium ? smoothed : ifl;
    }
    x87_leave(cw);
}

void orc_rope_tables_llama3(float *cos_table, float *sin_table, int n_pos, int head_dim, float rope_base,
                            float factor, float low_freq_factor, float high_freq_factor, int orig_max_pos)
{
    double freq[512];
    int half = head_dim / 2;
    orc_rope_freqs_llama3(freq, half, rope_base, factor, low_freq_factor, high_freq_factor, orig_max_pos);
    rope_fill(cos_table, sin_table, n_pos, half, freq);
}

/* EVAL_SIGMOID, packed form: src/asm/v7_macros.inc:98-160; constants
 * src/asm/math_data.inc:16-53. */
static float bits_to_float(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float orc_sigmoid(float g)
{
    ORC_REFERENCE_FP_ENV;
    const float log2e = (float)1.4426950408889634; /* scalar_log2e / s_log2e_v */
    const float c5 = bits_to_float(0x3AADD303u);
    const float c4 = bits_to_float(0x3C1E7411u);
    const float c3 = bits_to_float(0x3D635B9Bu);
    const float c2 = bits_to_float(0x3E75FCE0u);
    const float c1 = bits_to_float(0x3F317215u);
    float x = -g;                       /* vxorps sign mask */
    x = (x > -80.0f) ? x : -80.0f;      /* vmaxps x, -80: src1 > src2 ? src1 : src2 */
    x = (x < 80.0f) ? x : 80.0f;        /* vminps x, 80: src1 < src2 ? src1 : src2 */
    float fx = x * log2e;               /* vmulps */
    float ip = nearbyintf(fx);          /* vroundps imm 0: nearest-even */
    float fp = fx - ip;                 /* vsubps */
    int32_t ii = (int32_t)ip;           /* vcvttps2dq, ip is already integral */
    float p2 = bits_to_float((uint32_t)(ii + 127) << 23); /* vpaddd bias, vpslld 23 */
    float p = c5;                       /* vbroadcastss C5 */
    p = fmaf(fp, p, c4);                /* vfmadd213ps: fpart*acc + C4 */
    p = fmaf(fp, p, c3);
    p = fmaf(fp, p, c2);
    p = fmaf(fp, p, c1);
    p = fmaf(fp, p, 1.0f);
    float e = p2 * p;                   /* vmulps ymm0, ymm5, ymm4 */
    float d = e + 1.0f;                 /* vaddps */
    return 1.0f / d;                    /* vdivps */
}

/* Elementwise SwiGLU, the .pq_ffn_silu loop: src/asm/prefill_q8.inc:1159-1166.
 * out = (sigmoid(g) * g) * u, two vmulps. */
void orc_swiglu(float *out, const float *gate, const float *up, long long n)
{
    ORC_REFERENCE_FP_ENV;
    for (long long i = 0; i < n; ++i) {
        float g = gate[i];
        float sg = orc_sigmoid(g) * g;
        out[i] = sg * up[i];
    }
}

/* v7d_quantize / v7s_quantize_chunk: src/asm/utility_dispatch.inc:108-212,
 * src/asm/quantize_kernel.inc:44-159; typedef src/v7_lib.h:123.
 * The reference group size is GS = 64 (src/asm/v7_core.inc:120); gs is a
 * parameter here so the same algorithm also covers 32-element blocks. */
static const float Q_FLOOR = 1.4928778e-36f; /* scalar_epsilon, quantize_kernel.inc:40-41: 127 * 2^-126 */

/* Full-group code: vmulps, vcvtps2dq (nearest-even; NaN and out-of-range give
 * 0x80000000), vpackssdw + vpacksswb (signed saturation), vpmaxsb -127
 * (quantize_kernel.inc:91-105). */
static int8_t code_vec(float v)
{
    int32_t i;
    if (!(v >= -2147483648.0f && v < 2147483648.0f))
        i = INT32_MIN;
    else
        i = (int32_t)nearbyintf(v);
    if (i < -128)
        i = -128;
    if (i > 127)
        i = 127;
    if (i < -127)
        i = -127;
    return (int8_t)i;
}

/* Tail code: vmaxss -127 (NaN gives -127), vminss 127, vcvtss2si
 * (quantize_kernel.inc:143-149). */
static int8_t code_tail(float v)
{
    v = (v > -127.0f) ? v : -127.0f;
    v = (v < 127.0f) ? v : 127.0f;
    return (int8_t)(int32_t)nearbyintf(v);
}

static float absf_bits(float v)
{
    uint32_t u;
    memcpy(&u, &v, 4);
    u &= 0x7FFFFFFFu; /* vandps abs mask */
    return bits_to_float(u);
}

/* vmaxps / vmaxss dst, a, b: a > b ? a : b, so the second operand when either is NaN. */
static float vmax(float a, float b)
{
    return (a > b) ? a : b;
}

/* Absmax of a full group, the vandps + vmaxps tree of quantize_kernel.inc:62-83 with its operand order,
 * which decides where a NaN survives.  Eight-float vectors v_j = |x[8j .. 8j+7]|; for GS = 64:
 * m = max(max(max(v0,v1), max(v2,v3)), max(max(v4,v5), max(v6,v7))) lane-wise, then lanes i and i+4
 * (vextractf128), then 0,2 and 1,3 (vmovhlps), then 0 and 1 (vmovshdup).  GS = 32 takes the same shape over
 * four vectors (the reference has no 32-element kernel); any other group size is scanned in order as the
 * scalar tail scans (vmaxss |x|, wmax). */
static float group_absmax(const float *x, int gs)
{
    if (gs == 64 || gs == 32) {
        float m[8];
        for (int i = 0; i < 8; ++i) {
            float a[8];
            for (int j = 0; j < gs / 8; ++j)
                a[j] = absf_bits(x[8 * j + i]);
            float lo = vmax(vmax(a[0], a[1]), vmax(a[2], a[3]));
            m[i] = (gs == 64) ? vmax(lo, vmax(vmax(a[4], a[5]), vmax(a[6], a[7]))) : lo;
        }
        float p0 = vmax(m[0], m[4]), p1 = vmax(m[1], m[5]), p2 = vmax(m[2], m[6]), p3 = vmax(m[3], m[7]);
        return vmax(vmax(p0, p2), vmax(p1, p3));
    }
    float w = 0.0f;
    for (int i = 0; i < gs; ++i)
        w = vmax(absf_bits(x[i]), w);
    return w;
}

void orc_quantize(int8_t *out_q, const float *in_x, float *out_s, long long n, int gs)
{
    ORC_REFERENCE_FP_ENV;
    long long full = n / gs;
    for (long long g = 0; g < full; ++g) {
        const float *x = in_x + g * gs;
        float wmax = group_absmax(x, gs);
        wmax = (wmax > Q_FLOOR) ? wmax : Q_FLOOR; /* vmaxss wmax, eps (:84) */
        float scale = wmax / 127.0f;              /* vdivss (:86) */
        out_s[g] = scale;
        float recip = 1.0f / scale;               /* vdivss (:88) */
        for (int i = 0; i < gs; ++i)
            out_q[g * gs + i] = code_vec(x[i] * recip);
    }
    long long rem = n - full * gs;
    if (rem > 0) {
        /* scalar tail, quantize_kernel.inc:119-152 */
        const float *x = in_x + full * gs;
        float wmax = 0.0f;
        for (long long i = 0; i < rem; ++i)
            wmax = vmax(absf_bits(x[i]), wmax); /* vmaxss xmm3, |x|, xmm3 */
        wmax = (wmax > Q_FLOOR) ? wmax : Q_FLOOR;
        float scale = wmax / 127.0f;
        out_s[full] = scale;
        float recip = 1.0f / scale;
        for (long long i = 0; i < rem; ++i)
            out_q[full * gs + i] = code_tail(x[i] * recip);
    }
}

void orc_quantize_rows(int8_t *out_q, const float *in_x, float *out_s, int rows, int row_len, int gs)
{
    ORC_REFERENCE_FP_ENV;
    int spr = (row_len + gs - 1) / gs;
    for (int r = 0; r < rows; ++r)
        orc_quantize(out_q + (long long)r * row_len, in_x + (long long)r * row_len, out_s + (long long)r * spr, row_len,
                     gs);
}

/* SwiGLU -> Q8 per row: src/asm/prefill_q8.inc:1154-1183 (.pq_ffn_silu over the
 * row, then v7d_quantize over the same row with n = hidden_dim). */
void orc_swiglu_q8_rows(int8_t *out_q, float *out_s, const float *gate, const float *up, int rows, int hidden, int gs)
{
    ORC_REFERENCE_FP_ENV;
    float *buf = (float *)malloc((size_t)hidden * sizeof(float));
    if (!buf)
        return;
    int spr = (hidden + gs - 1) / gs;
    for (int r = 0; r < rows; ++r) {
        orc_swiglu(buf, gate + (long long)r * hidden, up + (long long)r * hidden, hidden);
        orc_quantize(out_q + (long long)r * hidden, buf, out_s + (long long)r * spr, hidden, gs);
    }
    free(buf);
}

/* v7s_embedding_row(out, token, dim, q_desc): src/asm/forward.inc:13-42.
 * out[i] = (float)q[token*dim + i] * s[(token*dim >> 6) + i/64]: vpmovsxbd +
 * vcvtdq2ps (exact) then one vmulps. */
void orc_embedding_row(float *out, int token, int dim, const int8_t *table_q, const float *table_s)
{
    long long base = (long long)token * dim;
    const int8_t *q = table_q + base;
    const float *s = table_s + (base >> 6);
    for (int i = 0; i < dim; ++i)
        out[i] = (float)q[i] * s[i >> 6];
}

void orc_embedding_gather(float *out, const int32_t *ids, int n_tokens, int dim, const int8_t *table_q,
                          const float *table_s)
{
    for (int t = 0; t < n_tokens; ++t)
        orc_embedding_row(out + (long long)t * dim, ids[t], dim, table_q, table_s);
}

/* v7s_rmsnorm(o, x, weight, size): src/asm/rmsnorm_kernel.inc:12-75, typedef src/v7_lib.h:270.
 * Contract size % 32 == 0 (no leftover blocks).  Phase 1 is the four-accumulator sum of squares
 * (blocks 0,4,8.. into A, 1,5,.. into B, ...), (A+B)+(C+D), HADD_YMM; the scale is
 * COMPUTE_RMS_SCALE with (float)size; phase 2 is o = (scale * x) * weight, two vmulps. */
void orc_rmsnorm(float *o, const float *x, const float *weight, int size, float eps)
{
    ORC_REFERENCE_FP_ENV;
    float ss = orc_sumsq_lanes(x, size);
    float s = orc_rms_scale(ss, size, eps);
    for (int i = 0; i < size; ++i) {
        float t = s * x[i];
        o[i] = t * weight[i];
    }
}

void orc_rmsnorm_rows(float *o, const float *x, const float *weight, int rows, int dim, float eps)
{
    ORC_REFERENCE_FP_ENV;
    for (int r = 0; r < rows; ++r)
        orc_rmsnorm(o + (long long)r * dim, x + (long long)r * dim, weight, dim, eps);
}

/* v7s_rmsnorm_quantize(out_q, in_x, out_s, n, weight): src/asm/rmsnorm_quantize_kernel.inc:62-218,
 * typedef src/v7_lib.h:124.  Phase 1 accumulates 64 floats per iteration, blocks 0..3 then 4..7 into
 * A, B, C, D: the same block-to-accumulator assignment as v7s_rmsnorm for n % 64 == 0; the scale is
 * vdivss by (float)n, + eps, vsqrtss, 1/x (:107-112).  Each 64-group of norm = (scale * x) * weight
 * (:122-137) is quantized exactly as v7s_quantize_chunk does (:138-165).  The reference's validator
 * requires the result to be bit-identical to the two-step chain v7s_rmsnorm -> v7d_quantize
 * (tools/kt_utils.h:850-933), which is what this computes; gs is a parameter (the reference's is 64). */
void orc_rmsnorm_quantize_rows(int8_t *out_q, float *out_s, const float *x, const float *weight, int rows, int dim,
                               int gs, float eps)
{
    ORC_REFERENCE_FP_ENV;
    float *buf = (float *)malloc((size_t)dim * sizeof(float));
    if (!buf)
        return;
    int spr = (dim + gs - 1) / gs;
    for (int r = 0; r < rows; ++r) {
        orc_rmsnorm(buf, x + (long long)r * dim, weight, dim, eps);
        orc_quantize(out_q + (long long)r * dim, buf, out_s + (long long)r * spr, dim, gs);
    }
    free(buf);
}

/* v7s_add_inplace(x, y, n): src/asm/add_kernel.inc:26-49, typedef src/v7_lib.h:271.  x[i] = x[i] + y[i]
 * (vaddps), n % 32 == 0. */
void orc_add_inplace(float *x, const float *y, long long n)
{
    ORC_REFERENCE_FP_ENV;
    for (long long i = 0; i < n; ++i)
        x[i] = x[i] + y[i];
}

/* binary32 -> binary16, round to nearest even, as vcvtps2ph with imm 0 does
 * (src/asm/kv_f16c.inc:5-7: "nearest-even independently of MXCSR"):
 * overflow to +-Inf, binary16 subnormals kept, NaN stays NaN with the top
 * mantissa bits kept and the quiet bit set. */
uint16_t orc_f32_to_f16_bits(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xFFu;
    uint32_t man = u & 0x7FFFFFu;
    if (exp == 0xFFu) /* Inf or NaN */
        return (uint16_t)(sign | 0x7C00u | (man ? (0x0200u | (man >> 13)) : 0u));
    int e = (int)exp - 127 + 15; /* binary16 biased exponent */
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u); /* |f| >= 2^16: overflow (rounding cannot bring it back) */
    if (e <= 0) {
        /* binary16 subnormal or zero: value = m * 2^-24 with m = round(|f| * 2^24) */
        if (e < -10)
            return (uint16_t)sign; /* below half of the smallest subnormal (also f32 zeros/subnormals) */
        uint32_t m = man | 0x800000u; /* implicit bit */
        int shift = 14 - e;           /* 24-bit significand -> (11 + e - 1)-bit result */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u)))
            q += 1u; /* may carry into the smallest normal, which is the right encoding */
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))
        q += 1u; /* a carry into the exponent is the correct result, up to Inf */
    return (uint16_t)(sign | q);
}

/* v7s_kv_pack_f16(dest, src, count): src/asm/kv_f16c.inc:12-52 (internal in v7, called per token for the
 * K and V rows after RoPE, src/asm/forward_q8.inc:345-358, prefill_q8.inc:157-171): dest[i] = f16(src[i]). */
void orc_kv_pack_f16(uint16_t *dst, const float *src, long long n)
{
    for (long long i = 0; i < n; ++i)
        dst[i] = orc_f32_to_f16_bits(src[i]);
}

/* v7s_rope_only_heads(buf, n_heads, head_dim, cos, sin, pos, rope_max_dim): src/asm/rope_only_dispatch.inc:11-47
 * (one job per head) and v7s_rope_only_head, src/asm/rope_only_kernel.inc:11-53 (internal in v7; the RoPE of
 * models without per-head Q/K norm, chosen by PQ_QK_ROPE, src/asm/v7_macros.inc:391-410).  pos == 0 returns
 * the head unchanged; otherwise each pair (j, j + half) of the head:
 *   re = lower*cos; ro = lower*sin; re = fma(-upper, sin, re); ro = fma(upper, cos, ro). */
void orc_rope_only_heads(float *buf, int n_heads, int head_dim, const float *cos_table, const float *sin_table,
                         int pos, int rope_max_dim)
{
    ORC_REFERENCE_FP_ENV;
    if (pos == 0)
        return;
    const float *c = cos_table + (long long)pos * rope_max_dim;
    const float *s = sin_table + (long long)pos * rope_max_dim;
    int half = head_dim / 2;
    for (int h = 0; h < n_heads; ++h) {
        float *x = buf + (long long)h * head_dim;
        for (int j = 0; j < half; ++j) {
            float lo = x[j], up = x[j + half];
            float re = lo * c[j];
            float ro = lo * s[j];
            re = fmaf(-up, s[j], re);
            ro = fmaf(up, c[j], ro);
            x[j] = re;
            x[j + half] = ro;
        }
    }
}

/* PQ_BIAS_ADD (src/asm/v7_macros.inc:366-383): x = x + bias, vaddps, the QKV bias of Stage C
 * (src/asm/prefill_q8.inc:848-879); n is all_heads_dim or kv_dim. */
void orc_bias_add(float *x, const float *bias, long long n)
{
    ORC_REFERENCE_FP_ENV;
    for (long long i = 0; i < n; ++i)
        x[i] = x[i] + bias[i];
}
