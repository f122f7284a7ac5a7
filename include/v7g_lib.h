/* v7g_lib.h -- C ABI of libv7g.so, the MI355X (gfx950) implementation of the
 * fused per-layer kernels of the v7 inference engine (cpki-gmbh/v7multiplikator).
 *
 * Two groups of entry points:
 *
 *  1. Drop-in entries with the reference's names, argument order and calling
 *     convention (V7_ABI = ms_abi on Linux, as src/v7_lib.h:40-46 declares for
 *     every export of libv7_threading.so).  They take DEVICE pointers and
 *     enqueue one launch on the library stream; like the reference they return
 *     nothing and read eps from a library global (the reference's g_rms_eps,
 *     set here by v7g_set_rms_eps).  Contract violations do not abort: they set
 *     the sticky error read by v7g_get_last_error().
 *
 *  2. Batched v7g_* entries (plain C calling convention) that process many
 *     rows/tokens per launch -- the performance path.  They return 0 or a
 *     V7G_ERR_* code (also recorded as the sticky error).
 *
 * All data pointers are device pointers (hipMalloc, or torch tensors on
 * cuda:N).  The library never allocates on a kernel call; v7s_rope_init /
 * v7g_rope_init are the only entries that allocate (the library-owned
 * cos/sin tables, as the reference's v7s_rope_init owns its tables).
 * Launches are asynchronous on the calling host thread's stream, set by
 * v7g_set_stream (default: the null stream); v7g_sync() waits for it.  Host
 * threads may drive different streams concurrently; eps (v7g_set_rms_eps) and
 * the sticky error are process-wide, as the reference's g_rms_eps global is.
 *
 * Outputs live in their own memory.  Each kernel reads and writes in one pass
 * with many workgroups in flight, so an output that shares a byte with another
 * output or with an input would be read and written in no fixed order.  Every
 * entry rejects such a call with V7G_ERR_ALIAS before any launch, except the
 * exact in-place forms listed at the entry (an output equal to the input it
 * replaces element by element).  In particular Q8 codes and scales never go
 * over their f32 source: the reference's prefill quantizes the SwiGLU row
 * into the retired up row (src/asm/prefill_q8.inc:1169-1180), which is safe
 * there only because its SwiGLU pass ends before the quantizer starts; the
 * fused SwiGLU -> Q8 kernel reads up while it writes codes.  Strided layouts
 * (Q, K and V heads inside one fused QKV row, cache rows) are compared row
 * against row when the strides are equal, so interleaved but disjoint
 * arguments pass; arguments with different strides are compared by the whole
 * byte range from their first to their last row.
 */
#ifndef V7G_LIB_H
#define V7G_LIB_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__linux__) && defined(__x86_64__)
#define V7_ABI __attribute__((ms_abi))
#else
#define V7_ABI
#endif

#define V7G_LIBRARY_NAME "libv7g.so"

/* Error codes (v7g_get_last_error, return values of the batched entries). */
#define V7G_OK 0
#define V7G_ERR_NULL 1       /* a required pointer is NULL */
#define V7G_ERR_SHAPE 2      /* a size violates the kernel contract */
#define V7G_ERR_ALIGN 3      /* a pointer is not aligned as the kernel needs */
#define V7G_ERR_HIP 4        /* the HIP runtime reported an error */
#define V7G_ERR_NO_TABLES 5  /* RoPE tables requested before v7s_rope_init */
#define V7G_ERR_ADDRESS 6    /* a pointer is not memory the current device can access (pointer checks on) */
#define V7G_ERR_ALIAS 7      /* an output overlaps another argument */

/* Q8 tensor descriptor: int8 codes + per-group f32 scales (GS = 64).
 * Same layout as v7_q8_tensor, src/v7_lib.h:52-56. */
typedef struct v7g_q8_tensor {
    char *q;
    float *s;
} v7g_q8_tensor;

/* ---------------------------------------------------------------------------
 * 1. Drop-in entries (reference signatures, device pointers, ms_abi)
 * ------------------------------------------------------------------------- */

/* Replaces v7s_fused_add_rmsnorm, typedef src/v7_lib.h:272, kernel
 * src/asm/add_rmsnorm_kernel.inc:15-129.  One row: residual += add (in place),
 * o = residual * rms_scale * weight.  Contract dim % 8 == 0, dim <= 16384. */
typedef void(V7_ABI *v7s_fused_add_rmsnorm_fn)(float *o, float *residual, float *add, float *weight, int dim);
V7_ABI void v7s_fused_add_rmsnorm(float *o, float *residual, float *add, float *weight, int dim);

/* Replaces v7s_rmsnorm, typedef src/v7_lib.h:270, kernel src/asm/rmsnorm_kernel.inc:12-75:
 * o = rmsnorm(x) * weight over one row.  Contract size % 32 == 0, size <= 16384. */
typedef void(V7_ABI *v7s_rmsnorm_fn)(float *o, float *x, float *weight, int size);
V7_ABI void v7s_rmsnorm(float *o, float *x, float *weight, int size);

/* Replaces v7s_rmsnorm_quantize, typedef src/v7_lib.h:124, kernel
 * src/asm/rmsnorm_quantize_kernel.inc:62-218: one row normalised and quantized
 * per group of 64 (out_q[n] codes, out_s[n/64] scales), bit-identical to
 * v7s_rmsnorm followed by v7d_quantize.  Contract n % 64 == 0, n <= 16384. */
typedef void(V7_ABI *v7s_rmsnorm_quantize_fn)(char *out_q, float *in_x, float *out_s, int n, float *weight);
V7_ABI void v7s_rmsnorm_quantize(char *out_q, float *in_x, float *out_s, int n, float *weight);

/* Replaces v7s_add_inplace, typedef src/v7_lib.h:271, kernel src/asm/add_kernel.inc:26-49:
 * x[i] += y[i] for n floats. */
typedef void(V7_ABI *v7s_add_inplace_fn)(float *x, float *y, int n);
V7_ABI void v7s_add_inplace(float *x, float *y, int n);

/* Replaces v7s_rmsnorm_rope_heads, typedef src/v7_lib.h:273, dispatcher
 * src/asm/rmsnorm_rope_dispatch.inc:11-52.  n_heads heads of one token,
 * contiguous in buf, normalised and rotated in place at position pos; the
 * tables hold rope_max_dim floats per position and at least pos+1 rows.
 * Contract head_dim % 32 == 0, 64 <= head_dim <= 512, rope_max_dim >= head_dim/2. */
typedef void(V7_ABI *v7s_rmsnorm_rope_heads_fn)(float *buf, int n_heads, int head_dim, float *norm_weight,
                                                float *cos_table, float *sin_table, int pos, int rope_max_dim);
V7_ABI void v7s_rmsnorm_rope_heads(float *buf, int n_heads, int head_dim, float *norm_weight, float *cos_table,
                                   float *sin_table, int pos, int rope_max_dim);

/* The descriptor of v7s_qk_fork_heads (src/asm/qk_fork_kernel.inc:10-28), 48 bytes: buf holds
 * `heads` contiguous heads of head_dim floats, weight the per-head norm weight; cos and sin point at
 * the position's table row already (the caller adds pos * rope_max_dim, src/asm/forward_q8.inc:50-71);
 * pos only decides whether the heads rotate (pos 0: norm only). */
typedef struct v7g_qk_fork_args {
  float *buf;
  float *weight;
  float *cos;
  float *sin;
  int head_dim;
  int heads;
  int pos;
  int unused;
} v7g_qk_fork_args;

/* Replaces v7s_qk_fork_heads (internal in v7, src/asm/qk_fork_kernel.inc:37-62): the reentrant,
 * descriptor-driven RMSNorm+RoPE over one descriptor's heads, the form the Q8 decode step calls for
 * Q and K concurrently (src/asm/forward_q8.inc:322-343).  Same arithmetic and contract as
 * v7s_rmsnorm_rope_heads; eps from v7g_set_rms_eps. */
typedef void(V7_ABI *v7s_qk_fork_heads_fn)(const v7g_qk_fork_args *desc);
V7_ABI void v7s_qk_fork_heads(const v7g_qk_fork_args *desc);

/* Replaces v7d_quantize, typedef src/v7_lib.h:123, src/asm/utility_dispatch.inc:108-212:
 * n floats -> n int8 codes + ceil(n/64) f32 scales, group size 64. */
typedef void(V7_ABI *v7d_quantize_fn)(char *out_q, float *in_x, float *out_s, int n);
V7_ABI void v7d_quantize(char *out_q, float *in_x, float *out_s, int n);

/* Replaces the engine-internal v7s_embedding_row(out, token, dim, q_desc),
 * src/asm/forward.inc:13-42 (no export in src/v7_threading.def; exported here).
 * out[i] = q[token*dim + i] * s[(token*dim)/64 + i/64].  q_desc is a HOST
 * struct holding device pointers.  Contract dim % 64 == 0. */
typedef void(V7_ABI *v7s_embedding_row_fn)(float *out, int token, int dim, v7g_q8_tensor *q_desc);
V7_ABI void v7s_embedding_row(float *out, int token, int dim, v7g_q8_tensor *q_desc);

/* Elementwise SwiGLU over one row, in place over the gate row as
 * .pq_ffn_silu does (src/asm/prefill_q8.inc:1154-1168, no reference export). */
typedef void(V7_ABI *v7s_swiglu_row_fn)(float *gate_inout, float *up, int hidden);
V7_ABI void v7s_swiglu_row(float *gate_inout, float *up, int hidden);

/* SwiGLU -> Q8 over one row, the chain of src/asm/prefill_q8.inc:1154-1183
 * (.pq_ffn_silu then v7d_quantize, group size 64), fused into one launch:
 * out_q[hidden] codes, out_s[ceil(hidden/64)] scales; gate/up are not modified.
 * out_q and out_s must not overlap gate or up (V7G_ERR_ALIAS): the reference's
 * codes-over-the-retired-up-row layout needs its own buffer here. */
typedef void(V7_ABI *v7s_swiglu_quantize_row_fn)(char *out_q, float *gate, float *up, float *out_s, int hidden);
V7_ABI void v7s_swiglu_quantize_row(char *out_q, float *gate, float *up, float *out_s, int hidden);

/* Replaces the engine-internal v7s_rope_only_heads(buf, n_heads, head_dim,
 * cos, sin, pos, rope_max_dim), src/asm/rope_only_dispatch.inc:11-47 and
 * rope_only_kernel.inc:11-53 (no export in src/v7_threading.def; exported
 * here): RoPE without the per-head RMSNorm, for models without Q/K norm
 * (PQ_QK_ROPE, src/asm/v7_macros.inc:391-410).  pos == 0 leaves the heads
 * unchanged.  Contract as v7s_rmsnorm_rope_heads. */
typedef void(V7_ABI *v7s_rope_only_heads_fn)(float *buf, int n_heads, int head_dim, float *cos_table,
                                             float *sin_table, int pos, int rope_max_dim);
V7_ABI void v7s_rope_only_heads(float *buf, int n_heads, int head_dim, float *cos_table, float *sin_table, int pos,
                                int rope_max_dim);

/* Replaces the engine-internal v7s_kv_pack_f16(dest, src, count),
 * src/asm/kv_f16c.inc:12-52 (no export in src/v7_threading.def; exported
 * here): dest[i] = binary16(src[i]), round to nearest even, for one K or V
 * row of count floats.  Contract count > 0, count % 8 == 0; dest 8-byte and
 * src 16-byte aligned. */
typedef void(V7_ABI *v7s_kv_pack_f16_fn)(uint16_t *dest, float *src, int count);
V7_ABI void v7s_kv_pack_f16(uint16_t *dest, float *src, int count);

/* Replaces v7s_rope_init, typedef src/v7_lib.h:275, src/asm/fused_dispatch.inc:58-76:
 * builds the library-owned device cos/sin tables, [131072, head_dim/2] each
 * (positions 0..131071, src/asm/fused_f32_kernel.inc:9), freq_j =
 * base^(-j/(head_dim/2)).  v7g_get_rope_tables returns them.  Like the
 * reference, which keeps only head_dim and reads the base and the rope type
 * from the model DB (src/asm/fused_f32_kernel.inc:97-110), it builds from the
 * configuration set by v7g_set_rope_config when one is set (rope_base is then
 * ignored; type 1 gives the Llama 3 scaled tables), else plain tables from
 * rope_base. */
typedef void(V7_ABI *v7s_rope_init_fn)(int head_dim, float rope_base);
V7_ABI void v7s_rope_init(int head_dim, float rope_base);

/* ---------------------------------------------------------------------------
 * 2. Library control
 * ------------------------------------------------------------------------- */

/* Initialises the HIP runtime on the current device (optional: every entry
 * initialises lazily).  Returns V7G_OK or V7G_ERR_HIP. */
int v7g_init(void);
/* Stream for all subsequent launches from the calling host thread (a
 * hipStream_t; NULL = null stream). */
void v7g_set_stream(void *stream);
void *v7g_get_stream(void);
/* Waits for the library stream; returns V7G_OK or V7G_ERR_HIP. */
int v7g_sync(void);
/* Kernel timing without a profiler (no counterpart in the reference, whose
 * kernels run on the caller thread).  Arms two hipEvent_t events (timing
 * enabled) for the next call from this host thread that launches work: they
 * are handed to hipExtLaunchKernel, `start` with that call's first kernel and
 * `stop` with its last, so no record call sits between the caller's kernels.
 * Create them with hipEventDisableSystemFence: an event's default system-scope
 * fence writes caches back inside the measured interval and slows the next
 * kernel.  Either may be NULL.  A call that launches nothing (a rejected or
 * empty call) leaves the pair armed; a launching call disarms it.  Returns
 * V7G_OK. */
int v7g_time_next_call(void *start_event, void *stop_event);
/* Pointer checks (no counterpart in the reference, whose kernels read host
 * memory).  When on, every entry asks the HIP runtime whether each pointer it
 * was given is device memory of the current device, managed memory or pinned
 * host memory, and rejects any other pointer with V7G_ERR_ADDRESS before
 * launching: a host buffer handed to a drop-in entry by mistake becomes an
 * error code instead of a GPU memory fault.  Off by default (each check costs
 * a runtime query per pointer); the environment variable V7G_CHECK_POINTERS=1
 * turns them on at load.  Process-wide. */
void v7g_set_pointer_checks(int on);
int v7g_get_pointer_checks(void);
/* The same test for one pointer, whatever the switch says: V7G_OK if the
 * current device can access p, else V7G_ERR_ADDRESS (not recorded as the
 * sticky error). */
int v7g_check_pointer(const void *p);
/* eps used by the drop-in norm entries (the reference's g_rms_eps global,
 * src/asm/v7_data.inc:509; default 1e-6). */
void v7g_set_rms_eps(float eps);
float v7g_get_rms_eps(void);
/* First error recorded since the last clear (V7G_OK if none). */
int v7g_get_last_error(void);
void v7g_clear_last_error(void);
const char *v7g_error_string(int code);
/* Library-owned RoPE tables built by v7s_rope_init / v7g_rope_init. */
int v7g_get_rope_tables(float **cos_table, float **sin_table, int *rope_max_dim, int *n_pos);
/* As v7s_rope_init with an explicit position count (1 .. 131072). */
int v7g_rope_init(int head_dim, float rope_base, int n_pos);
/* Fills caller-owned device tables [n_pos, head_dim/2] (host-built in extended
 * precision, then copied; synchronous). */
int v7g_build_rope_tables(float *cos_table, float *sin_table, int n_pos, int head_dim, float rope_base);
/* The same with Llama 3 frequency scaling: rope_build_internal_tables with
 * rope type 1, src/asm/fused_f32_kernel.inc:149-256, whose parameters the
 * reference reads from the model DB keys __sys_rope_factor,
 * __sys_rope_low_freq_factor, __sys_rope_high_freq_factor and
 * __sys_rope_orig_max_pos (:49-64).  factor > 0, 0 < low_freq_factor <
 * high_freq_factor, orig_max_pos > 0. */
int v7g_build_rope_tables_llama3(float *cos_table, float *sin_table, int n_pos, int head_dim, float rope_base,
                                 float factor, float low_freq_factor, float high_freq_factor, int orig_max_pos);
/* Library-owned tables with Llama 3 frequency scaling (v7s_rope_init for a
 * model whose rope type is 1); v7g_get_rope_tables returns them. */
int v7g_rope_init_llama3(int head_dim, float rope_base, int n_pos, float factor, float low_freq_factor,
                         float high_freq_factor, int orig_max_pos);
/* The model's RoPE configuration for v7s_rope_init, standing in for the model
 * DB keys the reference's table builder reads (src/asm/fused_f32_kernel.inc:
 * 49-64,97-110,149-170): rope_type = __sys_rope_type (0 plain, 1 Llama 3),
 * rope_base = __sys_rope_base, and for type 1 factor, low_freq_factor,
 * high_freq_factor and orig_max_pos = __sys_rope_factor,
 * __sys_rope_low_freq_factor, __sys_rope_high_freq_factor and
 * __sys_rope_orig_max_pos (ignored for type 0).  It plays the role
 * v7g_set_rms_eps plays for g_rms_eps.  Returns V7G_OK, or V7G_ERR_SHAPE for
 * another type, a base that is not positive and finite, or Llama 3 parameters
 * outside factor > 0, 0 < low_freq_factor < high_freq_factor, orig_max_pos > 0
 * (the configuration is then left as it was).  Process-wide. */
int v7g_set_rope_config(int rope_type, float rope_base, float factor, float low_freq_factor, float high_freq_factor,
                        int orig_max_pos);
/* 1 and the configuration in the non-NULL outputs if one is set, else 0. */
int v7g_get_rope_config(int *rope_type, float *rope_base, float *factor, float *low_freq_factor,
                        float *high_freq_factor, int *orig_max_pos);
/* Forgets the configuration: v7s_rope_init builds plain tables from its argument again. */
void v7g_clear_rope_config(void);

/* Exhaustive self-check, on the current device, of the arithmetic identities
 * the kernels rely on: mismatches[0] = inputs d in [2^-126, 2^123) where rcp
 * + one Newton step differs from 1.0f/d; mismatches[1] = finite x >=
 * 127*2^-126 where the fma-corrected x*(1/127) differs from x/127.0f;
 * mismatches[2] = non-NaN g where the sigmoid differs from EVAL_SIGMOID with
 * vdivps (src/asm/v7_macros.inc:98-160); mismatches[3] = binary32 patterns
 * where the hardware binary16 conversion differs from round-to-nearest-even
 * (the rounding of vcvtps2ph imm 0, src/asm/kv_f16c.inc), a NaN counting as
 * correct when it gives a binary16 NaN.  mismatches must hold 4 values, all 0
 * on a conforming device.  Synchronous; allocates a 128 KiB device buffer.
 * No reference counterpart. */
int v7g_arith_selfcheck(unsigned long long *mismatches);

/* v7g_arith_selfcheck without allocating: no counterpart in the reference;
 * for callers that cannot allocate device memory (serving loops and harnesses
 * that forbid hipMalloc, e.g. a periodic device health check between
 * batches).  Bit w of `checks` (1..15) selects identity w; mismatches[w] is
 * written for the selected identities only, with the value
 * v7g_arith_selfcheck gives.  The counts live in 32 bytes of static device
 * memory, one copy per device, kept until the process ends; the entry makes
 * no allocation.  Every call on a device shares those counters, so a call
 * holds a per-device lock from clearing them until its counts are read back:
 * calls from several host threads on one device queue up instead of racing.
 * Synchronous.  V7G_ERR_SHAPE for checks outside
 * 1..15 (there are four identities, four counters). */
int v7g_arith_selfcheck_noalloc(unsigned long long *mismatches, int checks);

/* ---------------------------------------------------------------------------
 * 3. Batched entries (performance path)
 * ------------------------------------------------------------------------- */

/* rows x dim fused add+RMSNorm; rows contiguous (row stride = dim).
 * residual is updated in place; o may equal residual or add, and overlaps
 * nothing else.  dim % 8 == 0, dim <= 16384, pointers 16-byte aligned. */
int v7g_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                          float eps);

/* rows x dim RMSNorm (v7s_rmsnorm per row): o = rmsnorm(x) * weight; o may
 * equal x.  dim % 32 == 0, dim <= 16384, pointers 16-byte aligned. */
int v7g_rmsnorm(float *o, const float *x, const float *weight, int rows, int dim, float eps);

/* rows x dim RMSNorm -> Q8 (v7s_rmsnorm_quantize per row) with group size gs
 * (32 or 64; the reference's is 64): out_q [rows*dim] int8, out_s [rows,
 * dim/gs] f32, apart from each other and from x and weight.  dim % gs == 0,
 * dim <= 16384. */
int v7g_rmsnorm_quantize(int8_t *out_q, float *out_s, const float *x, const float *weight, int rows, int dim, int gs,
                         float eps);

/* The Q8 decode step v7s_add_inplace(residual, add) then v7s_rmsnorm_quantize
 * (src/asm/forward_q8.inc:386-387) fused into one pass over rows x dim:
 * residual += add (in place), then RMSNorm -> Q8 of the updated residual.
 * out_q, out_s and residual apart from each other, add and weight.
 * No reference counterpart as one call; the results equal the two calls'. */
int v7g_add_rmsnorm_quantize(int8_t *out_q, float *out_s, float *residual, const float *add, const float *weight,
                             int rows, int dim, int gs, float eps);

/* x[i] += y[i] for n floats (v7s_add_inplace), 0 <= n < 2^40; 16-byte aligned
 * pointers; y equal to x or apart from it. */
int v7g_add_inplace(float *x, const float *y, long long n);

/* RMSNorm+RoPE over n_tokens tokens of n_heads heads each.  Token t's heads
 * start at buf + t*token_stride (floats) and are contiguous.  Position of token
 * t: positions[t] (device int32 array) or, if positions is NULL, pos0 + t.
 * Tables: table_rows rows of rope_max_dim floats (a position outside the tables
 * yields NaN heads).  head_dim % 32 == 0 in [64, 512]; n_tokens times the
 * heads per token (of every side, for the Q/K and Q/K/V forms) < 2^28.  The
 * heads (and binary16 rows) written are apart from each other and from the
 * weights, biases, tables (table_rows rows) and positions. */
int v7g_rmsnorm_rope_heads(float *buf, int n_tokens, long long token_stride, int n_heads, int head_dim,
                           const float *norm_weight, const float *cos_table, const float *sin_table,
                           const int32_t *positions, int pos0, int rope_max_dim, int table_rows, float eps);

/* Q and K heads of n_tokens tokens in one launch (the reentrant two-sided form
 * of v7s_qk_fork_heads, src/asm/qk_fork_kernel.inc:40-62): Q with q_norm_weight,
 * K with k_norm_weight; q/k may live inside one fused QKV row (strides). */
int v7g_qk_rmsnorm_rope(float *q, long long q_token_stride, int n_q_heads, const float *q_norm_weight, float *k,
                        long long k_token_stride, int n_kv_heads, const float *k_norm_weight, int n_tokens,
                        int head_dim, const float *cos_table, const float *sin_table, const int32_t *positions,
                        int pos0, int rope_max_dim, int table_rows, float eps);

/* RoPE only (no per-head norm) over n_tokens tokens, as v7g_rmsnorm_rope_heads. */
int v7g_rope_only_heads(float *buf, int n_tokens, long long token_stride, int n_heads, int head_dim,
                        const float *cos_table, const float *sin_table, const int32_t *positions, int pos0,
                        int rope_max_dim, int table_rows);

/* The per-token Q/K/V stage of the prefill (src/asm/prefill_q8.inc:848-883:
 * QKV bias add, Q and K RMSNorm+RoPE or RoPE only, K and V packed to the
 * binary16 KV cache) for n_tokens tokens in one launch.  Per side: heads of a
 * token contiguous at buf + t*token_stride; norm_weight NULL = RoPE only (Q,
 * K) -- V never has one; bias NULL = no bias add; cache NULL = no binary16
 * rows, else token t's row at cache + t*cache_stride; keep_f32 = 0 (only with
 * a cache) skips writing the f32 result back.  Q has no cache.  V is
 * optional (v.buf NULL).  Results equal the reference's per-token calls bit
 * for bit. */
typedef struct v7g_qkv_side {
    float *buf;
    long long token_stride;
    int n_heads;
    const float *norm_weight;
    const float *bias;
    uint16_t *cache;
    long long cache_stride;
    int keep_f32;
} v7g_qkv_side;

typedef struct v7g_qkv_stage {
    v7g_qkv_side q, k, v;
    int n_tokens;
    int head_dim;
    const float *cos_table;
    const float *sin_table;
    const int32_t *positions; /* device int32 per token, or NULL: pos0 + t */
    int pos0;
    int rope_max_dim;
    int table_rows;
    float eps;
} v7g_qkv_stage;

int v7g_qkv_rope_stage(const v7g_qkv_stage *stage);

/* v7g_qk_rmsnorm_rope that also writes the rotated K heads of token t as
 * binary16 into k_cache + t*k_cache_stride (the v7s_kv_pack_f16 of the K row
 * that follows RoPE, src/asm/forward_q8.inc:345-351, fused into the same
 * pass).  keep_k_f32 = 0 skips writing the f32 K back in place.  k_cache
 * 8-byte aligned, k_cache_stride % 4 == 0. */
int v7g_qk_rmsnorm_rope_kv(float *q, long long q_token_stride, int n_q_heads, const float *q_norm_weight, float *k,
                           long long k_token_stride, int n_kv_heads, const float *k_norm_weight, int n_tokens,
                           int head_dim, const float *cos_table, const float *sin_table, const int32_t *positions,
                           int pos0, int rope_max_dim, int table_rows, float eps, uint16_t *k_cache,
                           long long k_cache_stride, int keep_k_f32);

/* rows x row_len binary32 -> binary16 (v7s_kv_pack_f16 per row): row r from
 * src + r*src_stride to dst + r*dst_stride (strides in elements).  row_len,
 * strides % 4 == 0; dst 8-byte, src 16-byte aligned; dst rows apart from src rows. */
int v7g_kv_pack_f16(uint16_t *dst, long long dst_stride, const float *src, long long src_stride, int rows,
                    int row_len);

/* The K and V rows of a token batch packed to their binary16 cache rows in
 * one launch: the two v7s_kv_pack_f16 calls per token of
 * src/asm/forward_q8.inc:345-358 (src/asm/prefill_q8.inc:157-171).  Token
 * r's K row of row_len floats at k_src + r*src_stride goes to k_dst +
 * r*k_dst_stride, its V row at v_src + r*src_stride to v_dst +
 * r*v_dst_stride (strides in elements: K and V of a fused QKV row share the
 * token stride).  row_len and strides % 4 == 0; destinations 8-byte, sources
 * 16-byte aligned; the two caches apart from each other and from the sources. */
int v7g_kv_pack_f16_kv(uint16_t *k_dst, long long k_dst_stride, uint16_t *v_dst, long long v_dst_stride,
                       const float *k_src, const float *v_src, long long src_stride, int rows, int row_len);

/* out[i] = (sigmoid(gate[i]) * gate[i]) * up[i] for n elements, 0 <= n < 2^40;
 * out may equal gate (the reference's in-place form) or up, and overlaps
 * neither otherwise. */
int v7g_swiglu_f32(float *out, const float *gate, const float *up, long long n);

/* SwiGLU -> Q8: rows x hidden, group size gs (32 or 64, or any 1..4096 on the
 * general path); out_q [rows*hidden] int8, out_s [rows, ceil(hidden/gs)] f32
 * (4-byte aligned).  Groups never cross rows; a row's last group may be
 * partial.  rows * ceil(hidden/gs) < 2^38.  out_q and out_s apart from each
 * other, gate and up. */
int v7g_swiglu_q8(int8_t *out_q, float *out_s, const float *gate, const float *up, int rows, int hidden, int gs);

/* Q8 block quantization of rows x row_len floats (v7d_quantize per row),
 * scales [rows, ceil(row_len/gs)]; the same contract as v7g_swiglu_q8. */
int v7g_quantize_q8(int8_t *out_q, float *out_s, const float *x, int rows, int row_len, int gs);

/* Q8 embedding gather: out[t, :] = dequant(table row ids[t]) for n_tokens ids
 * (device int32).  table_q [vocab, dim] int8 (4-byte aligned), table_s
 * [vocab*dim/64] f32, out 16-byte aligned.  An id outside [0, vocab) yields a
 * zero row.  dim % 64 == 0.  out apart from ids and the table. */
int v7g_embedding_gather_q8(float *out, const int32_t *ids, int n_tokens, const int8_t *table_q,
                            const float *table_s, int dim, int vocab);

#ifdef __cplusplus
}
#endif
#endif /* V7G_LIB_H */
