/* v7_ref_leg.c -- the reference binary as a CPU baseline (TEST AND BENCHMARK INFRASTRUCTURE ONLY).
 *
 * The reference library (libv7_threading.so, built by the reference's own
 * Makefile with nasm, Makefile:36-47) exports two of the per-layer chain's four
 * kernels: v7s_fused_add_rmsnorm and v7s_rmsnorm_rope_heads (src/v7_threading.def;
 * signatures src/v7_lib.h:272-273, called through the ms_abi V7_ABI convention).
 * The Q8 embedding row and the SwiGLU -> Q8 row are internal to it
 * (forward.inc:13-42, prefill_q8.inc:1154-1183).  This file loads such a
 * library by path, as src/v7_lib.h:585-620 does (dlopen, then one dlsym per
 * entry, failing on a missing export), and times those two kernels per token
 * row over the same row-parallel split as the AVX2 restatement; the same
 * timer runs the restatement's two kernels for a like-for-like figure.
 *
 * eps: the reference's norm kernels take none; they read the BSS global
 * g_rms_eps (v7_data.inc:509), which only its database init sets
 * (inf_microdb.inc:49-53).  Loaded on its own, the library runs with the BSS
 * default, 0.  The caller passes the eps the loaded library uses to the
 * restatement's side (orc_chain_args.eps) so that both compute the same thing.
 */
#include "v7_oracle.h"
#include "v7_oracle_fpenv.h"

#include <dlfcn.h>
#include <pthread.h>
#include <stdio.h>
#include <string.h>
#include <time.h>

typedef void(__attribute__((ms_abi)) * ref_fused_add_rmsnorm_fn)(float *o, float *residual, float *add, float *weight,
                                                                   int dim);
typedef void(__attribute__((ms_abi)) * ref_rmsnorm_rope_heads_fn)(float *buf, int n_heads, int head_dim,
                                                                    float *norm_weight, float *cos_table,
                                                                    float *sin_table, int pos, int rope_max_dim);

static struct {
    void *handle;
    ref_fused_add_rmsnorm_fn fused_add_rmsnorm;
    ref_rmsnorm_rope_heads_fn rmsnorm_rope_heads;
} g_ref;

static char g_ref_error[512];

const char *orc_ref_error(void) { return g_ref_error; }

void orc_ref_close(void)
{
    if (g_ref.handle)
        dlclose(g_ref.handle);
    memset(&g_ref, 0, sizeof g_ref);
}

/* 0: loaded; -1: dlopen failed; -2: a required export is missing.  orc_ref_error() says which. */
int orc_ref_open(const char *path)
{
    orc_ref_close();
    g_ref_error[0] = 0;
    void *h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!h) {
        snprintf(g_ref_error, sizeof g_ref_error, "failed to load %s: %s", path, dlerror());
        return -1;
    }
    void *f = dlsym(h, "v7s_fused_add_rmsnorm");
    void *r = dlsym(h, "v7s_rmsnorm_rope_heads");
    if (!f || !r) {
        snprintf(g_ref_error, sizeof g_ref_error, "missing required export '%s' in %s",
                 !f ? "v7s_fused_add_rmsnorm" : "v7s_rmsnorm_rope_heads", path);
        dlclose(h);
        return -2;
    }
    g_ref.handle = h;
    memcpy(&g_ref.fused_add_rmsnorm, &f, sizeof f);
    memcpy(&g_ref.rmsnorm_rope_heads, &r, sizeof r);
    return 0;
}

typedef struct {
    const orc_chain_args *a;
    int t0, t1, reps, use_ref;
} k23_job;

/* add+RMSNorm of the token's residual row, then RMSNorm+RoPE of its Q heads and
 * of its K heads: forward_f32.inc:324-332 and prefill_q8.inc:815-911, one call
 * per token row as the reference engine makes them. */
static void k23_rows(const orc_chain_args *a, int t0, int t1, int use_ref)
{
    const int dim = a->dim, hd = a->head_dim;
    for (int t = t0; t < t1; ++t) {
        const long long td = (long long)t * dim;
        float *q = a->q + (long long)t * a->n_q_heads * hd;
        float *k = a->k + (long long)t * a->n_kv_heads * hd;
        if (use_ref) {
            g_ref.fused_add_rmsnorm(a->normed + td, a->residual + td, (float *)(a->add + td), (float *)a->w_norm, dim);
            g_ref.rmsnorm_rope_heads(q, a->n_q_heads, hd, (float *)a->q_w, (float *)a->cos_table,
                                     (float *)a->sin_table, a->positions[t], a->rope_max_dim);
            g_ref.rmsnorm_rope_heads(k, a->n_kv_heads, hd, (float *)a->k_w, (float *)a->cos_table,
                                     (float *)a->sin_table, a->positions[t], a->rope_max_dim);
        } else {
            orc_avx2_fused_add_rmsnorm(a->normed + td, a->residual + td, a->add + td, a->w_norm, dim, a->eps);
            orc_avx2_rmsnorm_rope_heads(q, a->n_q_heads, hd, a->q_w, a->cos_table, a->sin_table, a->positions[t],
                                        a->rope_max_dim, a->eps);
            orc_avx2_rmsnorm_rope_heads(k, a->n_kv_heads, hd, a->k_w, a->cos_table, a->sin_table, a->positions[t],
                                        a->rope_max_dim, a->eps);
        }
    }
}

static void *k23_thread(void *p)
{
    ORC_REFERENCE_FP_ENV;
    k23_job *j = (k23_job *)p;
    for (int r = 0; r < j->reps; ++r)
        k23_rows(j->a, j->t0, j->t1, j->use_ref);
    return 0;
}

/* Runs the two exported kernels of the chain `reps` times over a->n_tokens rows split over n_threads
 * threads: the loaded reference library's (use_ref = 1, after orc_ref_open) or the AVX2 restatement's
 * (use_ref = 0, with a->eps).  Returns wall seconds, or -1 when use_ref is set and nothing is loaded. */
double orc_k23_bench(const orc_chain_args *a, int n_threads, int reps, int use_ref)
{
    if (use_ref && !g_ref.handle)
        return -1.0;
    if (n_threads < 1)
        n_threads = 1;
    if (n_threads > 256)
        n_threads = 256;
    pthread_t th[256];
    k23_job jobs[256];
    struct timespec ts0, ts1;
    clock_gettime(CLOCK_MONOTONIC, &ts0);
    for (int i = 0; i < n_threads; ++i) {
        jobs[i].a = a;
        jobs[i].t0 = (int)((long long)a->n_tokens * i / n_threads);
        jobs[i].t1 = (int)((long long)a->n_tokens * (i + 1) / n_threads);
        jobs[i].reps = reps;
        jobs[i].use_ref = use_ref;
        if (i > 0)
            pthread_create(&th[i], 0, k23_thread, &jobs[i]);
    }
    k23_thread(&jobs[0]);
    for (int i = 1; i < n_threads; ++i)
        pthread_join(th[i], 0);
    clock_gettime(CLOCK_MONOTONIC, &ts1);
    return (double)(ts1.tv_sec - ts0.tv_sec) + 1e-9 * (double)(ts1.tv_nsec - ts0.tv_nsec);
}
