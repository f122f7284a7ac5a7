/* v7_oracle_rows.c -- per-row timing driver for the widened rows (TEST AND BENCHMARK INFRASTRUCTURE ONLY).
 *
 * The benchmark's CPU-baseline leg times the restatement of each widened row of the path the way the
 * reference engine drives those kernels: one call per token row, rows split over host threads, every
 * thread in the reference's MXCSR mode (FTZ+DAZ), repetition r on argument set r % n_sets (copies of the
 * buffers, so that the repetitions together span more than the host caches).  Per row and kind:
 *   RMSNORM_Q8      v7s_rmsnorm_quantize (src/asm/rmsnorm_quantize_kernel.inc:62-218)
 *   ADD_RMSNORM_Q8  v7s_add_inplace then v7s_rmsnorm_quantize (src/asm/forward_q8.inc:386-387)
 *   KV_PACK         v7s_kv_pack_f16 of the K row, then of the V row (src/asm/forward_q8.inc:345-358)
 *   QKV_STAGE       Q and K RMSNorm+RoPE, then the K and V rows packed (src/asm/prefill_q8.inc:848-883)
 *   QKV_BIAS_ROPE   PQ_BIAS_ADD over the QKV row, then RoPE only on Q and K (src/asm/v7_macros.inc:366-410)
 *   ADD_INPLACE     v7s_add_inplace (src/asm/add_kernel.inc:26-49)
 * The AVX2 forms of v7_oracle_avx2.c run (RMSNorm, RMSNorm+RoPE, RoPE without the norm, the Q8 quantizer,
 * vaddps, the F16C pack).  Nothing here is part of the product. */
#define _GNU_SOURCE
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <time.h>

#include "v7_oracle.h"
#include "v7_oracle_fpenv.h"

typedef struct {
    const orc_rows_args *sets;
    int n_sets, t0, t1, reps;
} rows_job;

static void rows_run(const orc_rows_args *a, int t0, int t1, int f16c, float *tmp)
{
    const int dim = a->dim, hd = a->head_dim, nq = a->n_q_heads, nkv = a->n_kv_heads;
    const long long kvd = (long long)nkv * hd;
    for (int t = t0; t < t1; ++t) {
        const long long td = (long long)t * dim;
        float *row = a->qkv ? a->qkv + (long long)t * a->qkv_stride : 0;
        switch (a->kind) {
        case ORC_ROWS_ADD_RMSNORM_Q8:
            orc_avx2_add_inplace(a->x + td, a->add + td, dim);
            __attribute__((fallthrough));
        case ORC_ROWS_RMSNORM_Q8: /* the normalised row, then its groups quantized */
            orc_avx2_rmsnorm(tmp, a->x + td, a->weight, dim, a->eps);
            orc_avx2_quantize(a->codes + td, tmp, a->scales + (long long)t * (dim / a->gs), dim, a->gs);
            break;
        case ORC_ROWS_QKV_STAGE:
            orc_avx2_rmsnorm_rope_heads(row, nq, hd, a->q_w, a->cos_table, a->sin_table, a->positions[t],
                                        a->rope_max_dim, a->eps);
            orc_avx2_rmsnorm_rope_heads(row + (long long)nq * hd, nkv, hd, a->k_w, a->cos_table, a->sin_table,
                                        a->positions[t], a->rope_max_dim, a->eps);
            __attribute__((fallthrough)); /* the K and V rows go to the caches */
        case ORC_ROWS_KV_PACK:
            if (f16c) {
                orc_avx2_kv_pack_f16(a->k_cache + t * kvd, row + (long long)nq * hd, kvd);
                orc_avx2_kv_pack_f16(a->v_cache + t * kvd, row + (long long)nq * hd + kvd, kvd);
            } else {
                orc_kv_pack_f16(a->k_cache + t * kvd, row + (long long)nq * hd, kvd);
                orc_kv_pack_f16(a->v_cache + t * kvd, row + (long long)nq * hd + kvd, kvd);
            }
            break;
        case ORC_ROWS_QKV_BIAS_ROPE:
            orc_avx2_add_inplace(row, a->bias, (long long)(nq + 2 * nkv) * hd);
            orc_avx2_rope_only_heads(row, nq, hd, a->cos_table, a->sin_table, a->positions[t], a->rope_max_dim);
            orc_avx2_rope_only_heads(row + (long long)nq * hd, nkv, hd, a->cos_table, a->sin_table,
                                     a->positions[t], a->rope_max_dim);
            break;
        case ORC_ROWS_ADD_INPLACE:
            orc_avx2_add_inplace(a->x + td, a->add + td, dim);
            break;
        default:
            break;
        }
    }
}

static void *rows_thread(void *p)
{
    ORC_REFERENCE_FP_ENV;
    rows_job *j = (rows_job *)p;
    const int f16c = orc_f16c_available();
    float *tmp = (float *)malloc((size_t)(j->sets[0].dim > 0 ? j->sets[0].dim : 1) * sizeof(float));
    if (!tmp)
        return 0;
    for (int r = 0; r < j->reps; ++r)
        rows_run(&j->sets[r % j->n_sets], j->t0, j->t1, f16c, tmp);
    free(tmp);
    return 0;
}

double orc_rows_bench(const orc_rows_args *sets, int n_sets, int n_threads, int reps)
{
    const orc_rows_args *a = sets;
    if (n_sets < 1)
        n_sets = 1;
    if (n_threads < 1)
        n_threads = 1;
    if (n_threads > 256)
        n_threads = 256;
    pthread_t th[256];
    rows_job jobs[256];
    struct timespec ts0, ts1;
    clock_gettime(CLOCK_MONOTONIC, &ts0);
    for (int i = 0; i < n_threads; ++i) {
        jobs[i].sets = sets;
        jobs[i].n_sets = n_sets;
        jobs[i].t0 = (int)((long long)a->n_tokens * i / n_threads);
        jobs[i].t1 = (int)((long long)a->n_tokens * (i + 1) / n_threads);
        jobs[i].reps = reps;
        if (i > 0)
            pthread_create(&th[i], 0, rows_thread, &jobs[i]);
    }
    rows_thread(&jobs[0]);
    for (int i = 1; i < n_threads; ++i)
        pthread_join(th[i], 0);
    clock_gettime(CLOCK_MONOTONIC, &ts1);
    return (double)(ts1.tv_sec - ts0.tv_sec) + 1e-9 * (double)(ts1.tv_nsec - ts0.tv_nsec);
}
