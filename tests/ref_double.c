/* Test double for the reference-binary baseline leg (oracle/v7_ref_leg.c): a shared library that exports
 * the two entry points the leg binds, under the reference's names and with its ms_abi convention
 * (src/v7_lib.h:272-273), backed by the AVX2 restatement at a fixed eps, as the reference's kernels read
 * theirs from a global.  It lets the CPU suite check the leg's loading, calling convention and argument
 * order without the reference binary; it is not a build of the reference. */
#include "../oracle/v7_oracle.h"

float ref_double_eps = 0.0f;

__attribute__((ms_abi, visibility("default"))) void v7s_fused_add_rmsnorm(float *o, float *residual, float *add,
                                                                          float *weight, int dim)
{
    orc_avx2_fused_add_rmsnorm(o, residual, add, weight, dim, ref_double_eps);
}

__attribute__((ms_abi, visibility("default"))) void v7s_rmsnorm_rope_heads(float *buf, int n_heads, int head_dim,
                                                                           float *norm_weight, float *cos_table,
                                                                           float *sin_table, int pos,
                                                                           int rope_max_dim)
{
    orc_avx2_rmsnorm_rope_heads(buf, n_heads, head_dim, norm_weight, cos_table, sin_table, pos, rope_max_dim,
                                ref_double_eps);
}
