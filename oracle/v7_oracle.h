/* v7_oracle.h -- CPU oracle for the fused per-layer kernels (TEST INFRASTRUCTURE).
 *
 * This is the checker, not the product: only the test suite, the smoke check
 * and the CPU-baseline leg of the benchmark load it.  The product path is the
 * HIP library under v7multiplikator_amd/csrc and never calls into this code.
 *
 * Every function restates one reference kernel of cpki-gmbh/v7multiplikator
 * in scalar C, reproducing its operation order, rounding points and FMA
 * placement (see the per-function citations in v7_oracle.c).  Build flags:
 * -O2 -mfma -ffp-contract=off, no fast-math, so every C operator is one
 * binary32 operation rounded to nearest-even and fmaf() is the only fused op,
 * in the reference's MXCSR FTZ+DAZ mode (below).
 */
#ifndef V7_ORACLE_H
#define V7_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Floating-point environment.  The reference computes under MXCSR FTZ+DAZ: init ORs 0x8040 into
 * the init thread's MXCSR (src/asm/v7_init.inc:103-108), every dispatch entry reloads that image on
 * the calling thread (SET_FTZ_DAZ, src/asm/v7_core.inc:301-303) and the direct calls that follow on
 * that thread inherit it.  Each path function below enters that mode (denormal inputs read as zero,
 * results that are still tiny after rounding flushed to zero) and restores the caller's MXCSR on
 * return; the C operators compile to the SSE scalar instructions that obey it, and fmaf() to the
 * hardware FMA (-mfma).  orc_set_reference_fp_env(0) switches the mode off, to show what it changes. */
void orc_set_reference_fp_env(int on);
int orc_get_reference_fp_env(void);

/* a1: v7s_fused_add_rmsnorm, one row; dim % 8 == 0 */
void orc_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int dim, float eps);
/* a1 batched: rows x dim, contiguous rows */
void orc_fused_add_rmsnorm_rows(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                                float eps);
/* a1/a3 building block: the lane-ordered sum of squares of x[0..n), n % 8 == 0 */
float orc_sumsq_lanes(const float *x, int n);
/* a2: COMPUTE_RMS_SCALE */
float orc_rms_scale(float sumsq, int n, float eps);

/* a3: v7s_rmsnorm_rope_heads, one token; tables are the table bases (not pre-offset) */
void orc_rmsnorm_rope_heads(float *buf, int n_heads, int head_dim, const float *norm_weight, const float *cos_table,
                            const float *sin_table, int pos, int rope_max_dim, float eps);
/* a3 batched: tokens x heads; token t at buf + t*token_stride, position positions[t] */
void orc_rmsnorm_rope_tokens(float *buf, int n_tokens, long long token_stride, int n_heads, int head_dim,
                             const float *norm_weight, const float *cos_table, const float *sin_table,
                             const int32_t *positions, int rope_max_dim, float eps);

/* a4: RoPE table builder (host, extended precision); tables are [n_pos, half] */
/* Plain RoPE frequencies base^(-j/half), j < half, by the reference's x87 chain (stored as doubles). */
void orc_rope_freqs(double *freq, int half, float base);
void orc_rope_tables(float *cos_table, float *sin_table, int n_pos, int head_dim, float rope_base);
void orc_rope_freqs_llama3(double *freq, int half, float base, float factor, float low_freq_factor,
                           float high_freq_factor, int orig_max_pos);
void orc_rope_tables_llama3(float *cos_table, float *sin_table, int n_pos, int head_dim, float rope_base,
                            float factor, float low_freq_factor, float high_freq_factor, int orig_max_pos);

/* a5: EVAL_SIGMOID, ps form */
float orc_sigmoid(float g);
/* a6: elementwise SwiGLU (out may alias gate) */
void orc_swiglu(float *out, const float *gate, const float *up, long long n);

/* a7: v7d_quantize with group size gs (the reference fixes gs = 64); n may leave a partial tail group */
void orc_quantize(int8_t *out_q, const float *in_x, float *out_s, long long n, int gs);
/* a7 per row: rows x row_len, scales [rows, ceil(row_len/gs)] */
void orc_quantize_rows(int8_t *out_q, const float *in_x, float *out_s, int rows, int row_len, int gs);
/* a8: SwiGLU -> Q8 chain, rows x hidden */
void orc_swiglu_q8_rows(int8_t *out_q, float *out_s, const float *gate, const float *up, int rows, int hidden, int gs);

/* a9: v7s_embedding_row; scales use 64-element groups over the flat table */
void orc_embedding_row(float *out, int token, int dim, const int8_t *table_q, const float *table_s);
void orc_embedding_gather(float *out, const int32_t *ids, int n_tokens, int dim, const int8_t *table_q,
                          const float *table_s);

/* next rows: v7s_rmsnorm (size % 32 == 0), v7s_rmsnorm_quantize (= quantize(rmsnorm), dim % gs == 0),
 * v7s_add_inplace */
void orc_rmsnorm(float *o, const float *x, const float *weight, int size, float eps);
void orc_rmsnorm_rows(float *o, const float *x, const float *weight, int rows, int dim, float eps);
void orc_rmsnorm_quantize_rows(int8_t *out_q, float *out_s, const float *x, const float *weight, int rows, int dim,
                               int gs, float eps);
void orc_add_inplace(float *x, const float *y, long long n);

/* v7s_kv_pack_f16 (internal in v7): binary32 -> binary16 round-to-nearest-even */
uint16_t orc_f32_to_f16_bits(float f);
void orc_kv_pack_f16(uint16_t *dst, const float *src, long long n);
/* the F16C instruction itself (vcvtps2ph imm 0) and an exhaustive comparison against orc_f32_to_f16_bits */
int orc_f16c_available(void);
void orc_avx2_kv_pack_f16(uint16_t *dst, const float *src, long long n);
unsigned long long orc_check_f16_vs_f16c(uint64_t lo, uint64_t count, int n_threads);

/* v7s_rope_only_heads (internal in v7): RoPE without the per-head norm, one token; PQ_BIAS_ADD */
void orc_rope_only_heads(float *buf, int n_heads, int head_dim, const float *cos_table, const float *sin_table,
                         int pos, int rope_max_dim);
void orc_bias_add(float *x, const float *bias, long long n);

/* AVX2 restatement (v7_oracle_avx2.c): same results bit for bit, used as the CPU baseline */
int orc_avx2_available(void);
void orc_avx2_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int dim, float eps);
void orc_avx2_rmsnorm_rope_heads(float *buf, int n_heads, int head_dim, const float *norm_weight,
                                 const float *cos_table, const float *sin_table, int pos, int rope_max_dim, float eps);
void orc_avx2_swiglu(float *out, const float *gate, const float *up, long long n);
void orc_avx2_rmsnorm(float *o, const float *x, const float *weight, int dim, float eps);
void orc_avx2_add_inplace(float *x, const float *y, long long n);
void orc_avx2_rope_only_heads(float *buf, int n_heads, int head_dim, const float *cos_table,
                              const float *sin_table, int pos, int rope_max_dim);
void orc_avx2_quantize(int8_t *out_q, const float *in_x, float *out_s, long long n, int gs);
void orc_avx2_embedding_row(float *out, int token, int dim, const int8_t *table_q, const float *table_s);

/* Buffers of the per-layer chain (embedding gather, add+RMSNorm, Q/K RMSNorm+RoPE, SwiGLU -> Q8) over
 * n_tokens rows, all host memory, rows contiguous. */
typedef struct orc_chain_args {
    int n_tokens, dim, n_q_heads, n_kv_heads, head_dim, rope_max_dim, hidden, gs;
    float eps;
    const int32_t *ids;
    const int32_t *positions;
    const int8_t *table_q;
    const float *table_s;
    float *emb_out;
    float *residual;
    const float *add;
    const float *w_norm;
    float *normed;
    float *q;
    float *k;
    const float *q_w;
    const float *k_w;
    const float *cos_table;
    const float *sin_table;
    const float *gate;
    const float *up;
    float *act;
    int8_t *codes;
    float *scales;
} orc_chain_args;

/* Runs the chain `reps` times, one call per token row as the reference engine does, rows split over
 * n_threads host threads.  Returns wall seconds. */
double orc_avx2_chain_bench(const orc_chain_args *a, int n_threads, int reps);

/* The widened rows, timed per token row over host threads as the reference engine drives them
 * (v7_oracle_rows.c).  All buffers host memory; the QKV rows are [n_tokens, qkv_stride] with Q, K, V
 * heads in that order; the K/V cache rows are [n_tokens, n_kv_heads * head_dim] binary16. */
enum {
    ORC_ROWS_RMSNORM_Q8 = 0,
    ORC_ROWS_ADD_RMSNORM_Q8 = 1,
    ORC_ROWS_KV_PACK = 2,
    ORC_ROWS_QKV_STAGE = 3,
    ORC_ROWS_QKV_BIAS_ROPE = 4,
    ORC_ROWS_ADD_INPLACE = 5
};
typedef struct orc_rows_args {
    int kind, n_tokens, dim, gs, n_q_heads, n_kv_heads, head_dim, rope_max_dim;
    float eps;
    float *x;
    const float *add;
    const float *weight;
    int8_t *codes;
    float *scales;
    float *qkv;
    long long qkv_stride;
    const float *q_w;
    const float *k_w;
    const float *bias;
    const float *cos_table;
    const float *sin_table;
    const int32_t *positions;
    uint16_t *k_cache;
    uint16_t *v_cache;
} orc_rows_args;

/* Runs `reps` repetitions, repetition r of kind sets[r % n_sets].kind over rows 0..n_tokens-1 of that set's
 * buffers (every set of one kind and shape), rows split over n_threads threads; returns wall seconds. */
double orc_rows_bench(const orc_rows_args *sets, int n_sets, int n_threads, int reps);

/* The reference binary as a baseline (v7_ref_leg.c): loads a libv7_threading.so by path and times its
 * two exported chain kernels, v7s_fused_add_rmsnorm and v7s_rmsnorm_rope_heads, per token row. */
int orc_ref_open(const char *path);
void orc_ref_close(void);
const char *orc_ref_error(void);
double orc_k23_bench(const orc_chain_args *a, int n_threads, int reps, int use_ref);

#ifdef __cplusplus
}
#endif
#endif
