// k_embedding.hip -- Q8 embedding-row gather + dequant for gfx950.
//
// Reference: v7s_embedding_row (src/asm/forward.inc:13-42), one token row per
// call: out[i] = (float)q[token*dim + i] * s[(token*dim >> 6) + i/64], an exact
// int8 -> f32 conversion followed by one multiply.  Here one launch gathers all
// tokens of a batch; the result is bit-identical by construction.
//
// Layout: a 256-thread block covers 1024 codes (256 dwords) of one row; lane l
// loads dword l of that stretch (four codes, one coalesced 1 KiB load per
// wave) and its 64-code group's scale, and stores four floats (one coalesced
// 4 KiB dwordx4 store per wave).  Rows of any dim % 64 == 0 take
// ceil(dim/1024) blocks; a partial last block predicates its lanes.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

__global__ __launch_bounds__(256) void embedding_gather_q8_kernel(float *__restrict__ out,
                                                                  const int32_t *__restrict__ ids,
                                                                  unsigned blocks_per_row,
                                                                  const int8_t *__restrict__ table_q,
                                                                  const float *__restrict__ table_s, int dim,
                                                                  int vocab) {
  const unsigned t = blockIdx.x / blocks_per_row;
  const unsigned w = (blockIdx.x - t * blocks_per_row) * 256u + threadIdx.x;  // dword of the row
  const unsigned dw = (unsigned)dim >> 2;
  if (w >= dw) return;
  const int id = ids ? ids[t] : (int)t;  // no id array: row t of the table
  float4 *dst = reinterpret_cast<float4 *>(out + (size_t)t * dim) + w;
  if ((unsigned)id >= (unsigned)vocab) {
    // An id outside the table cannot be read; its row is written as zeros.
    *dst = make_float4(0.f, 0.f, 0.f, 0.f);
    return;
  }
  const size_t base = (size_t)id * (size_t)dim;
  const uint32_t u = reinterpret_cast<const uint32_t *>(table_q + base)[w];
  const float s = table_s[(base >> 6) + (w >> 4)];
  float4 v;
  v.x = (float)((int32_t)(u << 24) >> 24) * s;
  v.y = (float)((int32_t)(u << 16) >> 24) * s;
  v.z = (float)((int32_t)(u << 8) >> 24) * s;
  v.w = (float)((int32_t)u >> 24) * s;
  *dst = v;
}

void launch_embedding_gather(float *out, const int32_t *ids, int n_tokens, const int8_t *table_q,
                             const float *table_s, int dim, int vocab, hipStream_t stream) {
  const unsigned bpr = ((unsigned)dim / 4u + 255u) / 256u;
  const unsigned blocks = (unsigned)n_tokens * bpr;
  hipLaunchKernelGGL(embedding_gather_q8_kernel, dim3(blocks), dim3(256), 0, stream, out, ids, bpr, table_q, table_s,
                     dim, vocab);
}

}  // namespace v7g
