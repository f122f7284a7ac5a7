// v7g_internal.h -- launchers shared between the kernel files and the C-ABI layer.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace v7g {

// Timing events armed by v7g_time_next_call for the calling host thread.  The
// first kernel of the next launching call takes `start`; every kernel of that
// call takes `stop`, so the last one sets it.  The API layer disarms the pair
// after the call.
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
LaunchEvents &launch_events();

// Every kernel of the library is enqueued through this helper.
template <typename... KArgs, typename... Args>
inline void enqueue(void (*kernel)(KArgs...), dim3 grid, dim3 block, unsigned lds_bytes, hipStream_t stream,
                   Args... args) {
  LaunchEvents &ev = launch_events();
  hipExtLaunchKernelGGL(kernel, grid, block, lds_bytes, stream, ev.start, ev.stop, 0u, args...);
  ev.start = nullptr;
}

// Launchers: shapes and pointers are validated by the caller (v7g_api.hip);
// each launcher only computes the grid and enqueues on `stream`.
void launch_embedding_gather(float *out, const int32_t *ids, int n_tokens, const int8_t *table_q,
                             const float *table_s, int dim, int vocab, hipStream_t stream);

void launch_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                              float eps, hipStream_t stream);

// v7s_rmsnorm over rows x dim (dim % 32 == 0, <= 16384); o may alias x.
void launch_rmsnorm(float *o, const float *x, const float *weight, int rows, int dim, float eps, hipStream_t stream);

// RMSNorm -> Q8 over rows x dim (dim % gs == 0, gs 32 or 64); with add, x is a
// residual updated in place as x + add first (add_inplace fused in front).
void launch_rmsnorm_quantize(int8_t *q, float *q_s, float *x, const float *add, const float *weight, int rows,
                             int dim, int gs, float eps, hipStream_t stream);

// x += y over n floats (n % 4 == 0 on the vector path; any n).
void launch_add_inplace(float *x, const float *y, long long n, hipStream_t stream);

// One side (Q, K or V) of the per-token head stage.
struct RopeSide {
  float *buf;                // first head of token 0 (f32, updated in place)
  long long token_stride;    // floats between consecutive tokens
  int n_heads;
  const float *norm_weight;  // [head_dim], or nullptr: no per-head RMSNorm
  const float *bias = nullptr;       // [n_heads*head_dim] added first, or nullptr
  uint16_t *cache = nullptr;         // binary16 rows (token t at cache + t*cache_stride), or nullptr
  long long cache_stride = 0;        // binary16 elements between consecutive tokens
  bool keep_f32 = true;              // with a cache: also write the f32 result in place
  bool rotate = true;                // false for V: no RoPE
};
// Up to three sides (Q, K, V) of n_tokens tokens in one launch.
void launch_rmsnorm_rope(const RopeSide *sides, int n_sides, int n_tokens, int head_dim, const float *cos_table,
                         const float *sin_table, const int32_t *positions, int pos0, int rope_max_dim, int table_rows,
                         float eps, hipStream_t stream);

// binary32 -> binary16 rows (v7s_kv_pack_f16): rows x row_len (row_len % 4 == 0).
void launch_kv_pack_f16(uint16_t *dst, long long dst_stride, const float *src, long long src_stride, int rows,
                        int row_len, hipStream_t stream);
// The K and V rows of `rows` tokens (sharing src_stride) to two binary16 caches in one launch.
void launch_kv_pack2_f16(uint16_t *k_dst, long long k_dst_stride, uint16_t *v_dst, long long v_dst_stride,
                         const float *k_src, const float *v_src, long long src_stride, int rows, int row_len,
                         hipStream_t stream);

void launch_swiglu_f32(float *out, const float *gate, const float *up, long long n, hipStream_t stream);

// Q8 block quantization of `rows` rows of `row_len` floats, groups of `gs`
// never crossing a row; with gate/up given, the quantized value is the SwiGLU
// of the pair instead of x.
void launch_quantize_q8(int8_t *out_q, float *out_s, const float *x, const float *gate, const float *up, int rows,
                        int row_len, int gs, hipStream_t stream);

// Exhaustive check of rcp_rn, div127_rn and sigmoid_v7 against IEEE division,
// and of f16_bits against a software rounding, on the current device
// (synchronous; allocates a small device buffer).
// mismatches[i] = number of inputs where identity i fails; returns 0 or -1 on
// a HIP error.
int arith_selfcheck(unsigned long long mismatches[4], hipStream_t stream);
// The same identities (bit w of `checks` selects identity w) counted in the
// library's static device counters instead of an allocated buffer; writes
// mismatches[w] for the selected identities only.  Synchronous; returns 0 or
// -1 on a HIP error.
int arith_selfcheck_noalloc(unsigned long long mismatches[4], int checks, hipStream_t stream);

}  // namespace v7g
