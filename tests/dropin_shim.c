/* dropin_shim.c -- test support: System V wrappers around the ms_abi drop-in
 * entries of libv7g.so, so the Python tests (ctypes, System V only) can call
 * them with their real calling convention.  The compiler emits the ms_abi
 * call from the declarations in include/v7g_lib.h.  Built by
 * __graft_entry__.build() into tests/libdropin_shim.so. */
#include "v7g_lib.h"

void shim_fused_add_rmsnorm(float *o, float *residual, float *add, float *weight, int dim)
{
    v7s_fused_add_rmsnorm(o, residual, add, weight, dim);
}

void shim_rmsnorm_rope_heads(float *buf, int n_heads, int head_dim, float *w, float *cos_table, float *sin_table,
                             int pos, int rope_max_dim)
{
    v7s_rmsnorm_rope_heads(buf, n_heads, head_dim, w, cos_table, sin_table, pos, rope_max_dim);
}

void shim_quantize(char *out_q, float *in_x, float *out_s, int n)
{
    v7d_quantize(out_q, in_x, out_s, n);
}

void shim_embedding_row(float *out, int token, int dim, char *table_q, float *table_s)
{
    v7g_q8_tensor desc;
    desc.q = table_q;
    desc.s = table_s;
    v7s_embedding_row(out, token, dim, &desc);
}

void shim_swiglu_row(float *gate_inout, float *up, int hidden)
{
    v7s_swiglu_row(gate_inout, up, hidden);
}

void shim_swiglu_quantize_row(char *out_q, float *gate, float *up, float *out_s, int hidden)
{
    v7s_swiglu_quantize_row(out_q, gate, up, out_s, hidden);
}

void shim_rope_init(int head_dim, float rope_base)
{
    v7s_rope_init(head_dim, rope_base);
}

void shim_rmsnorm(float *o, float *x, float *weight, int size)
{
    v7s_rmsnorm(o, x, weight, size);
}

void shim_rmsnorm_quantize(char *out_q, float *in_x, float *out_s, int n, float *weight)
{
    v7s_rmsnorm_quantize(out_q, in_x, out_s, n, weight);
}

void shim_add_inplace(float *x, float *y, int n)
{
    v7s_add_inplace(x, y, n);
}

void shim_kv_pack_f16(uint16_t *dest, float *src, int count)
{
    v7s_kv_pack_f16(dest, src, count);
}

void shim_rope_only_heads(float *buf, int n_heads, int head_dim, float *cos_table, float *sin_table, int pos,
                          int rope_max_dim)
{
    v7s_rope_only_heads(buf, n_heads, head_dim, cos_table, sin_table, pos, rope_max_dim);
}

void shim_qk_fork_heads(float *buf, float *weight, float *cos_row, float *sin_row, int head_dim, int heads, int pos)
{
    v7g_qk_fork_args d;
    d.buf = buf;
    d.weight = weight;
    d.cos = cos_row;
    d.sin = sin_row;
    d.head_dim = head_dim;
    d.heads = heads;
    d.pos = pos;
    d.unused = 0;
    v7s_qk_fork_heads(&d);
}
